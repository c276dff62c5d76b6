"""Head dims 64 and 256 on the GPU: the reference's codec encodes any head dim
(codec.py:31-73) while its caches and engine assert 128 (cache.py:21, engine.py:28).

Gates, as at head dim 128:
  * codec and cache bytes equal to the oracle's (pinned by reference-written vectors at
    D = 64 and 256, tests/golden);
  * attention over the compressed cache == the bf16 twin bit for bit, and within the
    north-star tolerance of the oracle's fp32 attention (and 2e-2 of fp64);
  * engines on Llama / Qwen3 models with those head dims give the same tokens and logits
    with either cache.
"""
import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import kernels, synthetic
from oracle import attention as oatt
from oracle import cache as ocache
from oracle import codec as ocodec
from tests.conftest import same_bits, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[case]", *a, flush=True)


def _encode(x):
    B, T, H, D = x.shape
    c = exactkv.CompressedKV(B, T, H, D, reserve=1.0)
    st = (x.stride(0), 16 * x.stride(1), x.stride(1), x.stride(2))
    kernels.encode_pages(x, st, c._buf(), 0, 0, B, T // 16)
    return c


def _case(B, T, Hq, Hkv, D, seed):
    """The reference test's recipe (tests/test_exactkv.py:64-69) at head dim D."""
    g = torch.Generator().manual_seed(seed)
    TS = -(-T // 16) * 16
    scale = torch.exp(torch.randn(Hkv, D, generator=g) * 0.7)
    k = (torch.randn(B, TS, Hkv, D, generator=g) * scale).to(torch.bfloat16)
    v = torch.randn(B, TS, Hkv, D, generator=g).to(torch.bfloat16)
    k[:, ::97, :, 3] = 0.0
    k[:, 5::131, :, D // 2 + 1] = 1e-30                # raw rows
    q = (torch.randn(B, Hq, D, generator=g) * 0.3).to(torch.bfloat16)
    return q, k, v


def _check(o_c, o_r, q, k, v, T, lens=None):
    assert same_bits(o_c, o_r)
    r32 = oatt.attention(u16(q), u16(k), u16(v), T, np.float32, lens=lens)
    excess = oatt.tolerance_excess(o_c.float().cpu().numpy(), r32)
    assert excess <= 0, f"outside the bf16 tolerance by {excess:.3g}"
    r64 = oatt.attention(u16(q), u16(k), u16(v), T, np.float64, lens=lens)
    assert np.abs(o_c.double().cpu().numpy() - r64).max() < 2e-2


# (D, B, T, Hq, Hkv): Qwen2.5-0.5B (14/2) and Llama-3.2-1B (32/8) at 64; one query head per
# KV head; two groups of 16 query heads; a ragged last page; a single token
SHAPES = [(64, 2, 1000, 14, 2), (64, 1, 4096, 32, 8), (64, 3, 333, 8, 8), (64, 2, 517, 64, 2), (64, 1, 1, 4, 1),
          (256, 2, 1000, 16, 4), (256, 1, 2048, 8, 1), (256, 2, 77, 32, 2), (256, 1, 5, 2, 2)]


@pytest.mark.parametrize("D,B,T,Hq,Hkv", SHAPES)
def test_attention_bit_identical_and_accurate(D, B, T, Hq, Hkv):
    _say("attention head dim", D, B, T, Hq, Hkv)
    q, k, v = _case(B, T, Hq, Hkv, D, seed=3 + B + T + D)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    assert int(kc.cnt.item()) > 0 or T < 16
    o_c = kernels.attention_compressed(qd, kc.buffers(), vc.buffers(), T)
    o_r = kernels.attention_reference(qd, kd, vd, T)
    _check(o_c, o_r, q, k, v, T)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("ns_sl", [(1, None), (None, 16), (None, 48)])
def test_split_plans(D, ns_sl):
    """One split over 2100 tokens (132 pages), 16-token splits (132 partials per row) and
    48-token splits; every plan gives the twin's bits and stays within tolerance."""
    B, T, Hq, Hkv = 2, 2100, 8, 2
    _say("split plan head dim", D, ns_sl)
    q, k, v = _case(B, T, Hq, Hkv, D, seed=11 + D)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    ns, sl = ns_sl
    if ns is None:
        ns = -(-T // sl)
    else:
        sl = -(-T // 16) * 16
    o_c = kernels.attention_compressed(qd, kc, vc, T, nsplit=ns, split_len=sl)
    o_r = kernels.attention_reference(qd, kd, vd, T, nsplit=ns, split_len=sl)
    _check(o_c, o_r, q, k, v, T)


@pytest.mark.parametrize("B,TS,Hq,Hkv,rate", [(2, 704, 16, 4, 0.2), (1, 1504, 12, 6, 0.05), (2, 912, 32, 16, 0.1),
                                            (3, 1024, 8, 8, 0.02)])
def test_pairs_of_heads_raw_rows_and_blocks(B, TS, Hq, Hkv, rate):
    """Head dim 64 runs as pairs of KV heads: 2, 1 and 4 pairs per workgroup (Hkv 4, 6, 16;
    4, 8 and 2 page phases), raw rows in K and V of both heads of a pair at rates that put
    1-4 of a page pair's rows through the ring and more of them through the pool, a ragged
    last page, with the default plan, one split and 16-token splits: twin bits and the
    oracle's tolerance."""
    D, T = 64, TS - 3
    _say("pairs of heads", B, TS, Hq, Hkv, rate)
    k = synthetic.make_kv(B, TS, Hkv, D=D, kind="k", seed=Hkv, raw_row_rate=rate)
    v = synthetic.make_kv(B, TS, Hkv, D=D, kind="v", seed=Hkv + 1, raw_row_rate=rate)
    q = synthetic.make_q(B, Hq, D=D, seed=Hkv + 2)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    # raw rows per page pair (K and V of heads 2v, 2v+1): 1-4 (through the ring) at the lower
    # rates, more (from the pool) at the higher ones (all of them at 0.2)
    rows = (_popc16(kc.rowmask) + _popc16(vc.rowmask)).view(B, TS // 16, Hkv // 2, 2).sum(-1)
    if rate <= 0.1:
        assert int(((rows >= 1) & (rows <= 4)).sum()) > 0
    if rate >= 0.05:
        assert int((rows > 4).sum()) > 0
    for ns, sl in ((None, None), (1, TS), (TS // 16, 16)):
        o_c = kernels.attention_compressed(qd, kc, vc, T, nsplit=ns, split_len=sl)
        o_r = kernels.attention_reference(qd, kd, vd, T, nsplit=ns, split_len=sl)
        _check(o_c, o_r, q, k, v, T)


def _popc16(t):
    t = t.to(torch.int32)
    return sum((t >> i) & 1 for i in range(16))


@pytest.mark.parametrize("D", [64, 256])
def test_lengths_window_and_paged(D):
    """Per-sequence lengths, a sliding window and a block table (pages shuffled over a pool):
    the paged call gives the contiguous call's bits, the twin's too, and the oracle's values
    over each sequence's window."""
    B, TS, Hq, Hkv, W = 3, 640, 16, 2, 200
    _say("lens / window / paged head dim", D)
    q, k, v = _case(B, TS, Hq, Hkv, D, seed=21 + D)
    lens = torch.tensor([640, 333, 17], dtype=torch.int32)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    ld = lens.to(DEV)
    o_c = kernels.attention_compressed(qd, kc, vc, TS, lens=ld)
    o_r = kernels.attention_reference(qd, kd, vd, TS, lens=ld)
    _check(o_c, o_r, q, k, v, TS, lens=lens.numpy())
    ow_c = kernels.attention_compressed(qd, kc, vc, TS, lens=ld, window=W)
    ow_r = kernels.attention_reference(qd, kd, vd, TS, lens=ld, window=W)
    assert same_bits(ow_c, ow_r)
    for b in range(B):                                 # the window as a shorter sequence
        n = int(lens[b])
        lo = max(n - W, 0)
        r32 = oatt.attention(u16(q[b:b + 1]), u16(k[b:b + 1, lo:n]), u16(v[b:b + 1, lo:n]), n - lo, np.float32)
        assert oatt.tolerance_excess(ow_c[b:b + 1].float().cpu().numpy(), r32) <= 0
    # the same pages through a block table over one pool
    npg = TS // 16
    perm = torch.randperm(B * npg, generator=torch.Generator().manual_seed(5))
    table = perm.view(B, npg).to(torch.int32)
    pool_k = torch.empty(1, B * TS, Hkv, D, dtype=torch.bfloat16)
    pool_v = torch.empty_like(pool_k)
    for b in range(B):
        for p in range(npg):
            dst = int(table[b, p]) * 16
            pool_k[0, dst:dst + 16] = k[b, p * 16:(p + 1) * 16]
            pool_v[0, dst:dst + 16] = v[b, p * 16:(p + 1) * 16]
    pk, pv = _encode(pool_k.to(DEV)), _encode(pool_v.to(DEV))
    td = table.to(DEV)
    op_c = kernels.attention_compressed(qd, pk, pv, TS, lens=ld, block_table=td)
    op_r = kernels.attention_reference(qd, pool_k.to(DEV), pool_v.to(DEV), TS, lens=ld, block_table=td)
    assert same_bits(op_c, o_c) and same_bits(op_r, o_c)
    dec = kernels.decode_to_bf16(pk, TS, block_table=td)
    assert same_bits(dec, kd)


@pytest.mark.parametrize("D,B,H,T0,TS,rate,reserve", [(64, 2, 3, 300, 400, 0.1, 0.001), (256, 2, 2, 33, 160, 0.05, 0.0)])
def test_cache_append_prefill_and_growth(D, B, H, T0, TS, rate, reserve):
    """CompressedKV at head dim D: prefill, appends across page boundaries and raw-pool
    growth, byte for byte against the CPU model of the protocol (oracle/cache.py); attention
    over it equals attention over the plain bf16 cache after every page."""
    g = torch.Generator().manual_seed(7 + D)
    _say("cache head dim", D, B, H, T0, TS, rate, reserve)

    def make(n):
        x = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16)
        x[torch.rand(B, n, H, generator=g) < rate, D - 2] = 1e-30
        return x

    c, r = exactkv.CompressedKV(B, TS, H, D, reserve=reserve), exactkv.BF16KV(B, TS, H, D)
    m = ocache.CacheModel(B, TS, H, D, reserve=reserve)
    x0 = make(T0)
    for b in range(B):
        c.prefill_slot(b, x0[b:b + 1].to(DEV).contiguous())
        r.prefill_slot(b, x0[b:b + 1].to(DEV).contiguous())
        m.prefill_slot(b, u16(x0[b]))
    q = torch.randn(B, 4 * H, D, generator=g).to(torch.bfloat16).to(DEV)
    xs = make(TS - T0)
    for t in range(TS - T0):
        xt = xs[:, t].to(DEV).contiguous()
        c.append(xt)
        r.append(xt)
        m.append(u16(xs[:, t]))
        exactkv.check_overflow([c])
        m.check_overflow()
        if c.T % 16 == 0 or c.T == TS:
            for k in ("sm", "code", "base", "rowmask", "rowoff"):
                assert np.array_equal(getattr(c, k).cpu().numpy(), getattr(m, k)), (t, k)
            assert np.array_equal(u16(c.raw), m.raw) and int(c.cnt.item()) == m.cnt and c.cap == m.cap, t
            assert same_bits(exactkv.decode_attention(q, c, c), exactkv.decode_attention(q, r, r))
    assert c.grows == m.grows
    assert same_bits(kernels.decode_to_bf16(c, c.T), r.buf[:, :c.T])


@pytest.mark.parametrize("D", [64, 256])
def test_codec_round_trip_and_oracle_bytes(D):
    """encode_reference / decode_reference at head dim D on synthetic model-like keys:
    the oracle's bytes, and every bit back (partial lengths through decode_to_bf16)."""
    x = synthetic.make_kv(2, 512, 4, D=D, kind="k", seed=D, raw_row_rate=0.02)
    _say("codec head dim", D)
    c = exactkv.encode_reference(x.to(DEV))
    want = ocodec.encode(u16(x))
    for k in ("sm", "code", "base", "rowmask", "rowoff"):
        assert np.array_equal(c[k].cpu().numpy(), want[k]), k
    assert np.array_equal(u16(c["raw"]), want["raw"])
    assert same_bits(exactkv.decode_reference(c), x.to(DEV))
    assert same_bits(kernels.decode_to_bf16(c, 500), x[:, :500].to(DEV))


def _model(kind, D, layers=2, seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM
    common = dict(vocab_size=1024, intermediate_size=1024, num_hidden_layers=layers, num_key_value_heads=2,
                  max_position_embeddings=4096)
    if kind == "llama":                                # head dim = hidden / heads
        cfg, cls = LlamaConfig(hidden_size=4 * D, num_attention_heads=4, rope_theta=5e5, **common), LlamaForCausalLM
    else:                                              # Qwen3 states its head dim
        cfg, cls = Qwen3Config(hidden_size=512, num_attention_heads=4, head_dim=D, rope_theta=1e6, **common), \
            Qwen3ForCausalLM
    torch.manual_seed(seed)
    with torch.device("cuda"):
        m = cls(cfg)
    return m.to(torch.bfloat16).eval()


@pytest.mark.parametrize("kind,D", [("llama", 64), ("qwen3", 256), ("qwen3", 64)])
def test_engine_backends_identical(kind, D):
    """Greedy decoding with the compressed and the bf16 cache (graph replay): the same tokens
    and the same logits bit for bit, through page boundaries."""
    B, PROMPT, NEW = 3, 37, 40
    m = _model(kind, D)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 1024, (B, PROMPT), generator=g).cuda()
    out = {}
    for backend in ("bf16", "exactkv"):
        print(f"[engine] {kind} head dim {D}: {backend}", flush=True)
        eng = exactkv.Engine(m, B, PROMPT + NEW, backend=backend)
        assert eng.D == D
        out[backend] = eng.generate(ids, NEW)
        torch.cuda.synchronize()
    (tb, lb), (tc, lc) = out["bf16"], out["exactkv"]
    assert torch.equal(tb, tc)
    assert torch.equal(lb.view(torch.int16), lc.view(torch.int16))
    assert torch.isfinite(lc.float()).all()


def test_paged_engine_matches_the_contiguous_engine():
    """Head dim 64: the paged engine (block tables over a shared pool) gives the contiguous
    engine's logits bit for bit (same pages, same split plan)."""
    B, PROMPT, NEW = 3, 37, 24
    m = _model("llama", 64)
    g = torch.Generator().manual_seed(11)
    ids = torch.randint(0, 1024, (B, PROMPT), generator=g).cuda()
    ref = exactkv.Engine(m, B, PROMPT + NEW, backend="exactkv", graph=False)
    pe = exactkv.PagedEngine(m, B, PROMPT + NEW, backend="exactkv")
    t_r = ref.prefill(ids)
    t_p = torch.stack([pe.add(ids[b])[1] for b in range(B)])
    assert torch.equal(t_r, t_p)
    print("[engine] paged vs contiguous, head dim 64", flush=True)
    for s in range(NEW - 1):
        lr, lp = ref.step(t_r), pe.step(t_p)
        assert torch.equal(lr.view(torch.int16), lp.view(torch.int16)), s
        t_r, t_p = lr.argmax(-1), lp.argmax(-1)
