"""Decode attention on the GPU (reference kernels.py:142-194, :33-43; reference test
tests/test_exactkv.py:61-78).

Gates:
  * compressed == uncompressed twin, bit for bit (same contents, same split plan);
  * within the north-star tolerance of the oracle's fp32 attention: per element
    |o - r| <= 1e-2 |r| + 2 bf16 ulp of the output row's largest magnitude;
  * within the reference's own bound of 2e-2 absolute vs fp64 softmax attention.
"""
import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import kernels, synthetic
from oracle import attention as oatt
from tests.conftest import same_bits, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[case]", *a, flush=True)


def assert_bf16_tolerance(out, ref):
    """out: bf16 tensor; ref: float array [B, Hq, D] (fp32 oracle). Bound: per element
    |o - r| <= 1e-2 |r| + 2 bf16 ulp of the row's largest |r| (oracle.attention.tolerance_excess)."""
    excess = oatt.tolerance_excess(out.float().cpu().numpy(), ref)
    assert excess <= 0, f"outside the bf16 tolerance by {excess:.3g}"


def _encode(x):
    B, T, H, D = x.shape
    c = exactkv.CompressedKV(B, T, H, D, reserve=1.0)
    st = (x.stride(0), 16 * x.stride(1), x.stride(1), x.stride(2))
    kernels.encode_pages(x, st, c._buf(), 0, 0, B, T // 16)
    return c


def _ref_case(B, T, Hq, Hkv, seed):
    """The reference test's data recipe (tests/test_exactkv.py:64-69), CPU seeded."""
    g = torch.Generator().manual_seed(seed)
    TS = -(-T // 16) * 16
    scale = torch.exp(torch.randn(Hkv, 128, generator=g) * 0.7)
    k = (torch.randn(B, TS, Hkv, 128, generator=g) * scale).to(torch.bfloat16)
    v = torch.randn(B, TS, Hkv, 128, generator=g).to(torch.bfloat16)
    k[:, ::97, :, 3] = 0.0
    q = (torch.randn(B, Hq, 128, generator=g) * 0.3).to(torch.bfloat16)
    return q, k, v


# KV heads per workgroup min(gcd(Hkv, 8), 4) = 4, 4, 4, 2, 2, 1, 1, 2: every page-phase
# count (2, 4, 8), so each loader wavefront serves wavefronts of one phase or of several
SHAPES = [(1, 4096, 28, 4), (3, 1000, 32, 8), (2, 333, 32, 32), (4, 17, 16, 2), (2, 500, 64, 2), (1, 1, 8, 1),
          (2, 700, 8, 1), (2, 777, 12, 6)]


@pytest.mark.parametrize("B,T,Hq,Hkv", SHAPES)
def test_attention_bit_identical_and_accurate(B, T, Hq, Hkv):
    _say("attention", B, T, Hq, Hkv)
    q, k, v = _ref_case(B, T, Hq, Hkv, seed=1 + B + T)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    o_c = kernels.attention_compressed(qd, kc.buffers(), vc.buffers(), T)
    o_r = kernels.attention_reference(qd, kd, vd, T)
    assert same_bits(o_c, o_r)
    for nw in (4, 8):                                  # reference kwargs accepted; same results
        assert same_bits(kernels.attention_compressed(qd, kc, vc, T, num_warps=nw), o_c)
    r32 = oatt.attention(u16(q), u16(k), u16(v), T, np.float32)
    assert_bf16_tolerance(o_c, r32)
    r64 = oatt.attention(u16(q), u16(k), u16(v), T, np.float64)
    assert np.abs(o_c.double().cpu().numpy() - r64).max() < 2e-2       # the reference test's bound


@pytest.mark.parametrize("T,ns_sl", [(1000, (1, None)), (1000, (None, 16)), (1000, (None, 32)), (1000, (None, 64)),
                                     (1000, (None, 96)), (2100, (1, None))])
def test_split_plans(T, ns_sl):
    # 16: 63 splits (multi-wavefront merge); T 2100 in one split: 132 pages per wavefront,
    # past the 64 whose page-table entries a wavefront holds in registers
    B, Hq, Hkv = 2, 32, 8
    q, k, v = _ref_case(B, T, Hq, Hkv, seed=5)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    ns, sl = ns_sl
    if sl is None:
        sl = -(-T // 32) * 32
    ns = -(-T // sl)
    _say("split plan", ns, sl)
    o_c = kernels.attention_compressed(qd, kc, vc, T, nsplit=ns, split_len=sl)
    o_r = kernels.attention_reference(qd, kd, vd, T, nsplit=ns, split_len=sl)
    assert same_bits(o_c, o_r)
    assert_bf16_tolerance(o_c, oatt.attention(u16(q), u16(k), u16(v), T, np.float32))
    # the merge in the split kernel's tail: compressed == twin bit for bit, within the oracle
    # tolerance, the separate merge's bits up to 32 splits (one level), and the arrival
    # counters reset for the next call
    r32 = oatt.attention(u16(q), u16(k), u16(v), T, np.float32)
    for _ in range(2):
        f_c = kernels.attention_compressed(qd, kc, vc, T, nsplit=ns, split_len=sl, fused_merge=True)
        f_r = kernels.attention_reference(qd, kd, vd, T, nsplit=ns, split_len=sl, fused_merge=True)
        assert same_bits(f_c, f_r)
        assert_bf16_tolerance(f_c, r32)
        if ns <= 32:
            assert same_bits(f_c, o_c)


@pytest.mark.parametrize("B,Hq,Hkv,T", [(1, 28, 4, 1000), (2, 8, 1, 777), (4, 32, 8, 500), (1, 32, 8, 8192)])
def test_default_plans_of_small_grids(B, Hq, Hkv, T):
    """Grids smaller than the GPU take splits down to one page (the default plan): with 4 or
    fewer KV heads per workgroup the later page phases of a one-page split have no page."""
    q, k, v = _ref_case(B, T, Hq, Hkv, seed=11)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    ns, sl = kernels.plan_splits(B, Hkv, Hq, T)
    _say("default plan", B, Hq, Hkv, T, ns, sl)
    assert sl <= 64                   # one round of ~256 workgroups over at most 2 units
    o_c = kernels.attention_compressed(qd, kc, vc, T)
    o_r = kernels.attention_reference(qd, kd, vd, T)
    assert same_bits(o_c, o_r)
    assert same_bits(o_c, kernels.attention_compressed(qd, kc, vc, T, nsplit=ns, split_len=sl))
    assert_bf16_tolerance(o_c, oatt.attention(u16(q), u16(k), u16(v), T, np.float32))


def test_synthetic_keys_with_raw_rows_and_zero_groups():
    """Config-0 style K/V (RoPE'd keys, 0.04% zeros, 0.3% raw rows) at 32q/8kv."""
    B, T, Hq, Hkv = 2, 2048 - 7, 32, 8
    TS = 2048
    k = synthetic.make_kv(B, TS, Hkv, kind="k", seed=21, raw_row_rate=0.01)
    v = synthetic.make_kv(B, TS, Hkv, kind="v", seed=22, raw_row_rate=0.01)
    q = synthetic.make_q(B, Hq, seed=23)
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    assert int(kc.cnt.item()) > 0 and int(vc.cnt.item()) > 0
    assert (kc.base >= 128).any()                       # zero-flagged groups present
    _say("synthetic", B, T, Hq, Hkv, "raw rows", int(kc.cnt.item()), int(vc.cnt.item()))
    o_c = kernels.attention_compressed(qd, kc, vc, T)
    assert same_bits(o_c, kernels.attention_reference(qd, kd, vd, T))
    assert_bf16_tolerance(o_c, oatt.attention(u16(q), u16(k), u16(v), T, np.float32))


def test_per_sequence_lengths():
    B, TS, Hq, Hkv = 4, 512, 32, 8
    lens = [512, 333, 17, 480]
    k = synthetic.make_kv(B, TS, Hkv, kind="k", seed=31)
    v = synthetic.make_kv(B, TS, Hkv, kind="v", seed=32)
    q = synthetic.make_q(B, Hq, seed=33)
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    ld = torch.tensor(lens, dtype=torch.int32, device=DEV)
    _say("lens", lens)
    o_c = kernels.attention_compressed(qd, kc, vc, 0, lens=ld)
    assert same_bits(o_c, kernels.attention_reference(qd, kd, vd, 0, lens=ld))
    assert_bf16_tolerance(o_c, oatt.attention(u16(q), u16(k), u16(v), TS, np.float32, lens=lens))


def test_cache_with_open_tail_page():
    """prefill_slot leaves a partial last page in the raw tail area (all rows raw)."""
    B, T, Hq, Hkv, TS = 3, 1000, 32, 8, 1024
    k = synthetic.make_kv(B, T, Hkv, kind="k", seed=41)
    v = synthetic.make_kv(B, T, Hkv, kind="v", seed=42)
    q = synthetic.make_q(B, Hq, seed=43).to(DEV)
    kc = exactkv.CompressedKV(B, TS, Hkv, 128)
    vc = exactkv.CompressedKV(B, TS, Hkv, 128)
    kr, vr = exactkv.BF16KV(B, TS, Hkv, 128), exactkv.BF16KV(B, TS, Hkv, 128)
    for b in range(B):
        for c, x in ((kc, k), (vc, v), (kr, k), (vr, v)):
            c.prefill_slot(b, x[b:b + 1].to(DEV).contiguous())
    _say("open tail", B, T, TS)
    o_c = exactkv.decode_attention(q, kc, vc)
    o_r = exactkv.decode_attention(q, kr, vr)
    assert same_bits(o_c, o_r)
    assert same_bits(kernels.decode_to_bf16(kc.buffers(), T), kr.buf[:, :T])
    assert_bf16_tolerance(o_c, oatt.attention(u16(q), u16(k), u16(v), T, np.float32))


def test_bad_arguments_raise():
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(1, 32, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="outside"):
        kernels.attention_reference(q, k, k, 33)
    with pytest.raises(ValueError):
        kernels.attention_reference(q.float(), k, k, 3)


def _window_oracle(q, k, v, lens, W):
    """fp32 oracle over tokens [len - W, len) of each sequence."""
    outs = []
    for b, n in enumerate(lens):
        lo = max(n - W, 0)
        outs.append(oatt.attention(u16(q[b:b + 1]), u16(k[b:b + 1, lo:n]), u16(v[b:b + 1, lo:n]), n - lo,
                                   np.float32))
    return np.concatenate(outs)


@pytest.mark.parametrize("W", [1, 7, 16, 40, 333, 4096])
def test_sliding_window(W):
    """window > 0: each sequence attends to its last W tokens (no reference counterpart;
    its engine rejects sliding-window models, engine.py:26-28). Compressed == twin bit for
    bit, within the north-star tolerance of the oracle over the window, and equal to the
    full attention of a cache that holds only the window's tokens."""
    B, TS, Hq, Hkv = 3, 1024, 32, 8
    lens = [1000, 517, 33]
    k = synthetic.make_kv(B, TS, Hkv, kind="k", seed=71, raw_row_rate=0.01)
    v = synthetic.make_kv(B, TS, Hkv, kind="v", seed=72, raw_row_rate=0.01)
    q = synthetic.make_q(B, Hq, seed=73)
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    ld = torch.tensor(lens, dtype=torch.int32, device=DEV)
    _say("window", W, lens)
    o_c = kernels.attention_compressed(qd, kc, vc, 0, lens=ld, window=W)
    o_r = kernels.attention_reference(qd, kd, vd, 0, lens=ld, window=W)
    assert same_bits(o_c, o_r)
    assert_bf16_tolerance(o_c, _window_oracle(q, k, v, lens, W))
    if W >= TS:                                       # a window longer than every sequence: no change
        assert same_bits(o_c, kernels.attention_compressed(qd, kc, vc, 0, lens=ld))
    # one length for all (no lens), several split plans
    T = 700
    for ns, sl in ((None, None), (1, -(-min(T, W + 15) // 32) * 32), (None, 64)):
        if sl is not None and ns is None:
            ns = -(-min(T, W + 15) // sl)
        o1 = kernels.attention_compressed(qd, kc, vc, T, window=W, nsplit=ns, split_len=sl)
        assert same_bits(o1, kernels.attention_reference(qd, kd, vd, T, window=W, nsplit=ns, split_len=sl))
        assert_bf16_tolerance(o1, _window_oracle(q, k, v, [T] * B, W))


def test_sliding_window_paged_and_bad_arguments():
    B, Hq, Hkv, npg, W = 2, 32, 8, 20, 100
    pool_pages = 48
    base = synthetic.make_kv(1, pool_pages * 16, Hkv, kind="k", seed=81)
    vbase = synthetic.make_kv(1, pool_pages * 16, Hkv, kind="v", seed=82)
    table = torch.randperm(pool_pages, generator=torch.Generator().manual_seed(4))[:B * npg].view(B, npg)
    table = table.to(torch.int32)
    q = synthetic.make_q(B, Hq, seed=83)
    kd, vd, qd = base.to(DEV), vbase.to(DEV), q.to(DEV)
    kpc, vpc = _encode(kd), _encode(vd)
    idx = (table.long()[:, :, None] * 16 + torch.arange(16)[None, None, :]).reshape(B, npg * 16)
    kg, vg = base[0][idx], vbase[0][idx]
    T = npg * 16 - 9
    bt = table.to(DEV)
    _say("window paged", W, T)
    o_p = kernels.attention_compressed(qd, kpc, vpc, T, block_table=bt, window=W)
    o_g = kernels.attention_reference(qd, kg.to(DEV).contiguous(), vg.to(DEV).contiguous(), T, window=W)
    assert same_bits(o_p, o_g)
    assert_bf16_tolerance(o_p, _window_oracle(q, kg, vg, [T] * B, W))
    q1 = qd[:1].contiguous()
    with pytest.raises(ValueError, match="window"):
        kernels.attention_reference(q1, kd, vd, 16, window=-1)
    with pytest.raises(RuntimeError, match="cover"):
        kernels.attention_reference(q1, kd[:, :512].contiguous(), vd[:, :512].contiguous(), 500, window=200,
                                    nsplit=1, split_len=192)


@pytest.mark.parametrize("ns", [1, 7, 32, 33, 63, 200, 1000])
def test_merge_kernel_against_oracle(ns):
    """exkv_attn_reduce on synthetic partials (some splits empty: m = -inf, l = 0, o = 0):
    the one-wavefront merge up to 32 splits and the (row, channel chunk) merge above, against
    the oracle's LSE merge (reference kernels.py:33-43), within one bf16 rounding step."""
    from exactkv_amd import _lib
    rows, D = 5, 128
    rng = np.random.default_rng(ns)
    m = (rng.standard_normal((rows, ns)) * 4).astype(np.float32)
    l = rng.uniform(1, 5, (rows, ns)).astype(np.float32)
    o = (rng.standard_normal((rows, ns, D)) * l[..., None]).astype(np.float32)
    empty = rng.random((rows, ns)) < 0.2
    empty[:, 0] = False                                 # every row keeps one non-empty split
    m[empty], l[empty], o[empty] = -np.inf, 0.0, 0.0
    _say("merge", ns)
    wo, wm, wl = (torch.from_numpy(x).to(DEV) for x in (o, m, l))
    out = torch.empty(rows, D, dtype=torch.bfloat16, device=DEV)
    _lib.call("exkv_attn_reduce", _lib.ptr(wo), _lib.ptr(wm), _lib.ptr(wl), _lib.ptr(out), rows, ns, D,
              _lib.stream())
    ref = oatt.merge_splits(m, l, o)
    got = out.float().cpu().numpy()
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30), np.abs(got - ref).max()


@pytest.mark.parametrize("B,T,Hq,Hkv,window", [(3, 1000, 32, 8, 0), (2, 777, 28, 4, 0), (4, 300, 16, 2, 100),
                                               (1, 2048, 8, 1, 0)])
def test_one_split_writes_the_merge_bits(B, T, Hq, Hkv, window):
    """With one split the split kernel writes the output itself (no merge launch). Its bits
    must be those of the split kernel's partials merged by the separate merge kernel, in the
    compressed kernel and in the twin, contiguous and paged."""
    from exactkv_amd import _lib
    q, k, v = _ref_case(B, T, Hq, Hkv, seed=930 + T)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    TS = kc.TS
    _say("one split", B, T, Hq, Hkv, window)
    direct = kernels.attention_compressed(qd, kc, vc, T, nsplit=1, split_len=TS, window=window)
    twin = kernels.attention_reference(qd, kd, vd, T, nsplit=1, split_len=TS, window=window)
    assert same_bits(direct, twin)
    # the two-launch form: the split kernel into a workspace, then exkv_attn_reduce
    wo = torch.empty(B * Hq, 1, 128, dtype=torch.float32, device=DEV)
    wm, wl = (torch.empty(B * Hq, 1, dtype=torch.float32, device=DEV) for _ in range(2))
    ka, _, _, _ = kernels._cache_args(kc)
    va, _, _, _ = kernels._cache_args(vc)
    _lib.call("exkv_attn_split_compressed", qd.data_ptr(), *ka, *va, wo.data_ptr(), wm.data_ptr(), wl.data_ptr(),
              B, Hq, Hkv, 128, T, TS, None, 0, 1, TS, window, 128 ** -0.5 * kernels.LOG2E, _lib.stream())
    out = torch.empty_like(qd)
    _lib.call("exkv_attn_reduce", _lib.ptr(wo), _lib.ptr(wm), _lib.ptr(wl), _lib.ptr(out), B * Hq, 1, 128,
              _lib.stream())
    assert same_bits(direct, out)
    lo = T - window if window else 0
    ref = oatt.attention(u16(q), u16(k[:, lo:T]), u16(v[:, lo:T]), T - lo, np.float32)
    assert_bf16_tolerance(direct, ref)
