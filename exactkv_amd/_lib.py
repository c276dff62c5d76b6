"""ctypes binding of libexactkv_hip.so (the C-ABI declared in include/exactkv.h).

The library is loaded on first use, after torch (so that it binds to the HIP runtime
torch has loaded). There is no fallback: every compute entry point raises if the
library is missing or a call fails.
"""
import ctypes
import os

# EXACTKV_LIB overrides the path of the library to load (default: the in-tree build)
_PATH = os.environ.get("EXACTKV_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libexactkv_hip.so")
ABI_VERSION = 3

_p, _i32, _i64, _f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float

# name -> argument types (every entry point returns int: 0 ok, 1 bad argument, 2 HIP error)
SIGNATURES = {
    "exkv_encode_pages": [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64,
                          _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p],
    "exkv_encode_pages_paged": [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64,
                                _i32, _p, _i64, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p],
    "exkv_cache_append": [_p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32,
                          _i32, _p],
    "exkv_bf16_append": [_p, _i64, _i64, _p, _p, _i32, _i32, _i32, _i32, _p],
    "exkv_cache_append_paged": [_p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _i64,
                                _i32, _i32, _i32, _i32, _i32, _i32, _p],
    "exkv_bf16_append_paged": [_p, _i64, _i64, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _p],
    "exkv_cache_open_page": [_p, _p, _p, _i64, _i64, _i32, _i32, _i32, _p],
    "exkv_cache_open_pages_paged": [_p, _p, _p, _i32, _p, _p, _i64, _i32, _i32, _i32, _i64, _i64, _i32, _p],
    "exkv_decode_to_bf16": [_p, _p, _p, _p, _p, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _p],
    "exkv_decode_to_bf16_paged": [_p, _p, _p, _p, _p, _p, _i64, _i64, _p, _i64, _p, _i32, _i32, _i32, _i32, _p],
    "exkv_attn_compressed": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p,
                             _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _i32, _i32, _i32, _f32, _p],
    "exkv_attn_bf16": [_p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _i32, _i32,
                       _i32, _f32, _p],
    "exkv_attn_split_compressed": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p,
                                   _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _i32, _i32, _i32, _f32, _p],
    "exkv_attn_split_bf16": [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _i32, _i32,
                             _i32, _f32, _p],
    "exkv_attn_compressed_paged": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p,
                                   _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _i32, _i32,
                                   _i32, _f32, _p],
    "exkv_attn_split_compressed_paged": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _p,
                                         _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _i32,
                                         _i32, _i32, _f32, _p],
    "exkv_attn_bf16_paged": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                             _p, _i64, _i32, _i32, _i32, _f32, _p],
    "exkv_wire_bytes": [_i32, _i32, _i64],
    "exkv_wire_pack": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p, _i64, _p, _p, _p, _p, _i32, _i32, _i32, _p,
                       _i64, _p],
    "exkv_wire_unpack": [_p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _i64, _i32, _p, _i64, _p, _p, _p, _p, _p, _i32,
                         _i32, _i32, _p, _i64, _p],
    "exkv_attn_reduce": [_p, _p, _p, _p, _i64, _i32, _i32, _p],
    "exkv_time_next_split": [_p, _p],
    "exkv_merge_counters": [_i32, _i32, _i32, _i32],
    "exkv_attn_compressed_noalloc": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _i32, _i32,
                                     _i32, _i32, _i32, _i32, _p, _i64, _i32, _i32, _i32, _f32, _p],
    "exkv_noalloc_scratch_bytes": [],
    "exkv_plan_splits": [_i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32)],
    "exkv_plan_splits_hd": [_i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32)],
    "exkv_abi_version": [],
    "exkv_last_error": [],
}

_lib = None


def path():
    return _PATH


def load():
    """Load the library (once). Raises RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_PATH):
        raise RuntimeError(f"exactkv HIP library not found at {_PATH}; build it with "
                           "`python -m exactkv_amd.build` (or __graft_entry__.build())")
    import torch  # noqa: F401  -- torch's HIP runtime must be loaded before the library
    lib = ctypes.CDLL(_PATH)
    for name, args in SIGNATURES.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = {"exkv_last_error": ctypes.c_char_p, "exkv_wire_bytes": ctypes.c_int64,
                     "exkv_noalloc_scratch_bytes": ctypes.c_int64,
                     "exkv_merge_counters": ctypes.c_int64}.get(name, ctypes.c_int)
    v = lib.exkv_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"libexactkv_hip.so ABI version {v}, expected {ABI_VERSION}: rebuild the library")
    runtimes = {ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln}
    if len(runtimes) > 1:
        raise RuntimeError(f"two HIP runtimes loaded in one process: {sorted(runtimes)}")
    _lib = lib
    return lib


def call(name, *args):
    """Call entry point `name`; raise RuntimeError with the library's message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.exkv_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


_raw_stream = None


def stream(index=None):
    """The current HIP stream of device `index` (default: the current device) as an integer,
    through torch's raw-stream query when it has one (a few µs cheaper per call than
    building a torch Stream object)."""
    global _raw_stream
    import torch
    if _raw_stream is None:
        _raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", False)
    if _raw_stream:
        return _raw_stream(torch.cuda.current_device() if index is None else index)
    return torch.cuda.current_stream(index).cuda_stream


def ptr(t, align=16, what="tensor"):
    """Device pointer of a CUDA (HIP) tensor, checked for device and alignment."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError(f"{what} must be on the GPU (got {t.device})")
    p = t.data_ptr()
    if align and p % align:
        raise ValueError(f"{what} is not {align}-byte aligned")
    return p
