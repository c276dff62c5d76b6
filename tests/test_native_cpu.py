"""CPU-side checks of the native library (no kernel launches): it loads, exports every
entry point include/exactkv.h declares, validates arguments before touching the GPU, the
value-rebuild bit logic is exact on every (sign|mantissa, code, base) combination, and the
split kernels' stage layouts (V^T operands, K and V rows, head-dim-64 pairs) rebuild every
value by the format rule, compiled for the host from the kernels' own header."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

from exactkv_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "exactkv.h")


def _declared():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"\b(exkv_[a-z0-9_]+)\s*\(", txt)))


def test_header_declares_the_bound_entry_points():
    assert _declared() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.exkv_abi_version() == _lib.ABI_VERSION


def test_argument_errors_are_reported_without_launching():
    lib = _lib.load()
    # head dim 96 has no kernels (64, 128 and 256 do): rejected before any HIP call
    rc = lib.exkv_decode_to_bf16(1, 1, 1, 1, 1, 1, 1, 1, 1, 16, 16, 1, 96, None)
    assert rc == 1 and b"head dim" in lib.exkv_last_error()
    for fn, args in (("exkv_attn_reduce", (1, 1, 1, 1, 1, 1, 96, None)),
                     ("exkv_bf16_append", (1, 0, 0, 1, 1, 1, 1, 16, 96, None))):
        assert getattr(lib, fn)(*args) == 1 and b"head dim" in lib.exkv_last_error(), fn
    # head dim 64 passes the head-dim check and fails on the next one (T past TS)
    rc = lib.exkv_decode_to_bf16(1, 1, 1, 1, 1, 1, 1, 1, 1, 17, 16, 1, 64, None)
    assert rc == 1 and b"outside" in lib.exkv_last_error()
    rc = lib.exkv_attn_bf16(1, 1, 1, 1, 1, 1, None, 1, 1, 32, 8, 128, 5000, 4096, None, 0, 1, 4096, 0, 0.1, None)
    assert rc == 1 and b"outside" in lib.exkv_last_error()
    rc = lib.exkv_encode_pages(1, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 1, None, 0, 1, 2, 1, 0, 2, 1, 4, 64, 128, None, 0,
                               None)
    assert rc == 1 and b"outside the cache" in lib.exkv_last_error()
    with pytest.raises(RuntimeError, match="split_len"):
        _lib.call("exkv_attn_bf16", 1, 1, 1, 1, 1, 1, None, 1, 1, 32, 8, 128, 100, 128, None, 0, 4, 30, 0, 0.1, None)
    # grids past 2^32 work-items: 1024 splits x 4096 x 7 workgroups of 256 threads (head dim
    # 64 with an odd KV-head count: the generic kernel's one-dimensional grid), 7M splits of
    # 640-thread workgroups (head dim 128; 64 with an even count takes the same grid)
    rc = lib.exkv_attn_bf16(1, 1, 1, 1, 1, 1, None, 1, 4096, 28, 7, 64, 16384, 16384, None, 0, 1024, 16, 0, 0.1, None)
    assert rc == 1 and b"too many workgroups" in lib.exkv_last_error()
    rc = lib.exkv_attn_bf16(1, 1, 1, 1, 1, 1, None, 1, 1, 32, 8, 64, 112000000, 112000000, None, 0, 7000000, 16, 0,
                            0.1, None)
    assert rc == 1 and b"too many workgroups" in lib.exkv_last_error()
    rc = lib.exkv_attn_bf16(1, 1, 1, 1, 1, 1, None, 1, 1, 32, 8, 128, 112000000, 112000000, None, 0, 7000000, 16, 0,
                            0.1, None)
    assert rc == 1 and b"too many workgroups" in lib.exkv_last_error()
    # paged entry points: a page table narrower than the pages to encode, a raw pool
    # without room for the tail areas, more rows than sequence slots
    rc = lib.exkv_encode_pages_paged(1, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 1, None, 0, 1, 1, 1, 2, 1, 3, 4, 64, 128, None,
                                     0, None)
    assert rc == 1 and b"page table" in lib.exkv_last_error()
    rc = lib.exkv_cache_append_paged(1, 0, 0, 1, 1, 1, 1, 1, 1, 1, 1, 10, 100, None, 1, 1, 8, 2, 4, 2, 8, 16, 128,
                                     None)
    assert rc == 1 and b"tail area" in lib.exkv_last_error()
    rc = lib.exkv_bf16_append_paged(1, 0, 0, 1, None, 1, 1, 8, 3, 4, 2, 8, 16, 128, None)
    assert rc == 1 and b"bad shape" in lib.exkv_last_error()
    # wire form: a scratch row too short for the longest sequence's pages; cap past the raw pool
    rc = lib.exkv_wire_pack(1, 1, 1, 1, 1, 1, 64, 4, 2, 1, 4, 1, 1, 1, 1, 64, 8, 128, 1, 10, None)
    assert rc == 1 and b"ws stride" in lib.exkv_last_error()
    rc = lib.exkv_wire_unpack(1, 1, 1, 1, 1, 1, 64, 80, 1, 1, 4, 2, 1, 4, 1, None, 1, 1, 1, 64, 8, 128, 1, 35, None)
    assert rc == 1 and b"cap" in lib.exkv_last_error()


@pytest.mark.parametrize("B,Hkv,Hq,T,expect", [
    (8, 8, 32, 8192, (16, 512)),       # a workgroup covers 4 of the 8 KV heads: 16 units x 16 splits = 256
    (1, 8, 32, 131072, (128, 1024)),
    (1, 4, 28, 32768, (256, 128)),     # 4 KV heads per workgroup: one unit, 256 splits
    (32, 8, 32, 4096, (4, 1024)),
    (1, 4, 28, 8000, (250, 32)),       # one unit: 256 splits of at least a page, rounded to 32 tokens
    (4, 2, 16, 17, (2, 16)),           # capped by one page per split
    (2, 2, 64, 1000, (63, 16)),        # G = 32: two head groups per KV head, 4 units; one page per split
    (620, 8, 32, 4352, (1, 4352)),     # 1240 units, more than a round: one split gives 4.84 rounds, the last 97% full
    (256, 8, 32, 4096, (1, 4096)),     # 512 units: exactly two rounds
    (300, 8, 32, 4096, (5, 832)),      # 600 units, 11.7 rounds: the first split count whose last round is >= 95% full
    (255, 8, 32, 4096, (2, 2048)),     # 510 units: one split would give 1.99 rounds, two give 3.98
])
def test_plan_splits(B, Hkv, Hq, T, expect):
    from exactkv_amd.kernels import plan_splits
    ns, sl = plan_splits(B, Hkv, Hq, T)
    assert (ns, sl) == expect
    assert (sl % 32 == 0 or sl == 16) and ns * sl >= T and (ns - 1) * sl < T


@pytest.mark.parametrize("B,Hkv,Hq,T,D,expect", [
    (8, 8, 32, 8192, 64, (32, 256)),     # pairs of heads: 4 virtual heads = one block per sequence, 8 units x 32
    (8, 8, 32, 8192, 256, (8, 1024)),    # 64 units x 8 = 512 workgroups (two per CU)
    (32, 2, 14, 4096, 64, (8, 512)),     # Qwen2.5-0.5B shape: one virtual head, 32 units x 8
    (1, 8, 32, 131072, 256, (64, 2048)),
    (2, 2, 64, 1000, 64, (63, 16)),      # G = 32: two query groups, 4 units; one page per split
    (600, 8, 32, 4096, 64, (5, 832)),    # 600 units: the first split count whose last round is >= 95% full
    (8, 7, 28, 8192, 64, (14, 608)),     # odd KV-head count: the generic kernel, 56 units, 768 workgroups
    (8, 8, 32, 8192, 128, (16, 512)),    # head dim 128: exkv_plan_splits
])
def test_plan_splits_hd(B, Hkv, Hq, T, D, expect):
    from exactkv_amd.kernels import plan_splits, plan_splits_hd
    ns, sl = plan_splits_hd(B, Hkv, Hq, T, D)
    assert (ns, sl) == expect
    assert (sl % 32 == 0 or sl == 16) and ns * sl >= T and (ns - 1) * sl < T
    if D == 128:
        assert (ns, sl) == plan_splits(B, Hkv, Hq, T)
    if D == 64 and Hkv % 2 == 0:                     # pairs: the head-dim-128 plan over Hkv / 2 virtual heads
        assert (ns, sl) == plan_splits(B, Hkv // 2, Hq // 2, T)


def test_rebuild_bitmath_exhaustive(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = tmp_path / "rebuild_check"
    subprocess.run([hipcc, "-O2", "-o", str(exe), os.path.join(ROOT, "tests", "native", "rebuild_check.cpp")],
                   check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True)
    assert r.returncode == 0, r.stdout
    assert "0 mismatches" in r.stdout
    assert ctypes is not None


def test_transposed_v_layout(tmp_path):
    """The compressed split kernels' V^T operand (csrc/stage.hpp): page bytes placed as the
    loaders' direct-to-LDS loads place them, ds_read_b64_tr_b8 emulated, rebuilt values
    against the format rule, for head-dim-128 heads and head-dim-64 pairs
    (tests/native/vt_check.cpp)."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = tmp_path / "vt_check"
    subprocess.run([hipcc, "-O2", "-o", str(exe), os.path.join(ROOT, "tests", "native", "vt_check.cpp")],
                   check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True)
    assert r.returncode == 0, r.stdout
    assert ", 0 mismatches" in r.stdout


def test_row_rebuild_layout(tmp_path):
    """The compressed split kernel's K rows (and the V rows of pages with raw V rows), and the
    head-dim-64 pair kernel's K rows, from the same stage placement: row reads and base dwords
    at lds_lane_offsets / pair_lane_offsets, the base dwords taken from the lane's own 16-lane
    row as the DPP row broadcast does, against the format rule (tests/native/krow_check.cpp)."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = tmp_path / "krow_check"
    subprocess.run([hipcc, "-O2", "-o", str(exe), os.path.join(ROOT, "tests", "native", "krow_check.cpp")],
                   check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True)
    assert r.returncode == 0, r.stdout
    assert ", 0 mismatches" in r.stdout


def test_engine_module_imports_without_a_gpu():
    import exactkv_amd as exactkv
    from exactkv_amd import engine
    assert exactkv.Engine is engine.Engine
    assert set(engine.BACKENDS) == {"exactkv", "bf16"}


def test_clamp_detection_of_the_error_bits(tmp_path):
    """The raw-slot clamp behind EXKV_ERR_RAW_SLOT, built for the host: the slot is always
    inside the pool, unchanged when it already was, and flagged exactly for a token whose raw
    row had to be clamped (tests/native/errors_check.cpp)."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    exe = tmp_path / "errors_check"
    subprocess.run([hipcc, "-O2", "-o", str(exe), os.path.join(ROOT, "tests", "native", "errors_check.cpp")],
                   check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True)
    assert r.returncode == 0, r.stdout
    assert " 0 failures" in r.stdout


def test_error_bits_are_declared_and_described():
    """Every EXKV_ERR_* bit of the header has a description on the Python side, and the
    description of a word names each of its bits (and unknown ones)."""
    import re
    from exactkv_amd import _lib
    hdr = open(os.path.join(ROOT, "include", "exactkv.h")).read()
    bits = {int(v, 16) for v in re.findall(r"#define EXKV_ERR_\w+ (0x[0-9a-fA-F]+)u", hdr)}
    assert bits == set(_lib.ERROR_BITS)
    assert _lib.describe_errors(0) == "none"
    d = _lib.describe_errors(0x1 | 0x4 | 0x100)
    assert _lib.ERROR_BITS[0x1] in d and _lib.ERROR_BITS[0x4] in d and "0x100" in d
