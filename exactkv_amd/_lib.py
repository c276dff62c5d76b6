"""ctypes binding of libexactkv_hip.so (the C-ABI declared in include/exactkv.h).

The library is loaded on first use, after torch (so that it binds to the HIP runtime
torch has loaded). There is no fallback: every compute entry point raises if the
library is missing or a call fails.
"""
import ctypes
import os

# EXACTKV_LIB overrides the path of the library to load (default: the in-tree build)
_PATH = os.environ.get("EXACTKV_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libexactkv_hip.so")
# EXACTKV_CHECK_ERRORS=1: after every kernel-launching call, wait for its stream and raise if
# a kernel set a sticky error bit (exkv_error_bits); slow, for debugging
_CHECK = os.environ.get("EXACTKV_CHECK_ERRORS", "") not in ("", "0")
ABI_VERSION = 4

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
    "exkv_error_bits": [_p, _i32, _p],
    "exkv_set_wait_limit": [_i32],
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


# entry points that take no stream (host-only, or hooks)
_NO_STREAM = {"exkv_wire_bytes", "exkv_time_next_split", "exkv_merge_counters", "exkv_noalloc_scratch_bytes",
              "exkv_plan_splits", "exkv_plan_splits_hd", "exkv_abi_version", "exkv_last_error", "exkv_error_bits",
              "exkv_set_wait_limit"}

# error bit -> what a kernel reports with it (include/exactkv.h EXKV_ERR_*)
ERROR_BITS = {
    0x1: "attention: a wait on another wavefront's LDS flag gave up",
    0x2: "attention / decode: a raw row's pool slot lay outside the pool (clamped)",
    0x4: "encoder: the slot scan's look-back gave up on a predecessor",
    0x8: "encoder: inconsistent scan workspace",
    0x10: "wire pack: a raw row's pool slot lay outside the pool (clamped)",
}


def describe_errors(bits):
    """The EXKV_ERR_* bits of `bits` in words."""
    names = [msg for b, msg in ERROR_BITS.items() if bits & b]
    rest = bits & ~sum(ERROR_BITS)
    return "; ".join(names + ([f"unknown bits {rest:#x}"] if rest else [])) or "none"


def call(name, *args):
    """Call entry point `name`; raise RuntimeError with the library's message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.exkv_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")
    if _CHECK and name not in _NO_STREAM:
        bits = stream_error_bits(args[-1], clear=True)
        if bits:
            raise RuntimeError(f"{name}: kernel error bits {bits:#x} ({describe_errors(bits)})")


_hip_rt = None
_ERRBUF = {}


def _stream_device(st):
    """Device index of a raw HIP stream handle (the null stream: the current device)."""
    global _hip_rt
    if _hip_rt is None:
        import torch
        _hip_rt = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
        _hip_rt.hipStreamGetDevice.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    d = ctypes.c_int(-1)
    if _hip_rt.hipStreamGetDevice(st, ctypes.byref(d)) != 0:
        raise RuntimeError("hipStreamGetDevice failed")
    return d.value


def stream_error_bits(st, clear=True):
    """The library's sticky kernel error bits on the GPU of raw stream `st`, once the work
    queued on `st` so far has completed (this waits for it); clear: reset them."""
    import torch
    dev = _stream_device(st)
    buf = _ERRBUF.get(dev)
    if buf is None:
        buf = _ERRBUF[dev] = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", dev))
    lib = load()
    if lib.exkv_error_bits(buf.data_ptr(), int(bool(clear)), st) != 0:
        raise RuntimeError("exkv_error_bits failed: " + lib.exkv_last_error().decode(errors="replace"))
    _hip_rt.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    if _hip_rt.hipStreamSynchronize(st) != 0:
        raise RuntimeError("hipStreamSynchronize failed")
    return int(buf.cpu().item()) & 0xFFFFFFFF


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
