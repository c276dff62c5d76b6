"""The benchmark configurations at their own sizes, through the C-ABI.

Each attention case checks the two properties the north star fixes for the path:
  * the compressed call is bit-identical to the uncompressed bf16 twin (same contents,
    same split plan: the planner's default for the shape);
  * it is within the bf16 tolerance of the oracle's fp32 attention (per element
    |o - r| <= 1e-2 |r| + 2 bf16 ulp of the row's largest |r|), and within the
    reference test's own 2e-2 absolute bound against fp64 (tests/test_exactkv.py:75-78).

Shapes (the reference's harness runs the same ones, bench/attention.py:68-82):
  c1  Qwen2.5-7B 28q/4kv, B1 x 32768
  c2a Llama-3.1-8B 32q/8kv, B8 x 8192, and B8 x 8185 (the last page partly filled)
  c2b Llama-3.1-8B 32q/8kv, B1 x 131072, and B1 x 131065
  c3  Qwen3-8B 32q/8kv, B32 with lengths U[3500, 4096], 0.6% outlier rows, a raw pool
      that grows from its minimum during prefill, appends across page boundaries
  c4  Llama-3.1-8B layer shapes (hidden 4096, 32/8 heads, FFN 14336, vocab 128256) with
      2 layers: both cache backends give identical tokens and logits
      (reference tests/test_exactkv.py:107-122)
and the long-split paths: one split per sequence, so a wavefront walks more than 64 pages
(its page metadata then comes from scalar loads), contiguous and through a block table.

K/V follow the configuration-0 recipe (exactkv_amd.synthetic): RoPE'd keys with per-channel
scales exp(N(0, 1.5)), values with exp(N(0, 0.5)), 0.04% exact zeros, 0.3% raw rows.
"""
import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import kernels, synthetic
from oracle import attention as oatt
from tests.conftest import same_bits, u16
from tests.test_gpu_attention import _encode, assert_bf16_tolerance

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = 16


def _say(*a):
    print("[case]", *a, flush=True)


def _data(B, TS, Hq, Hkv, seed, raw_row_rate=3e-3):
    k = synthetic.make_kv(B, TS, Hkv, kind="k", seed=seed, raw_row_rate=raw_row_rate)
    v = synthetic.make_kv(B, TS, Hkv, kind="v", seed=seed + 1, raw_row_rate=raw_row_rate)
    q = synthetic.make_q(B, Hq, seed=seed + 2)
    return q, k, v


def _check_call(q, k, v, kc, vc, kd, vd, T, lens=None, fp64=True, **kw):
    """compressed == twin bitwise, with the merge as a second kernel and in the split kernel's
    tail; fp32-oracle tolerance for both; the fp64 bound of the reference test."""
    qd = q.to(DEV)
    ld = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=DEV)
    o_c = kernels.attention_compressed(qd, kc, vc, T, lens=ld, **kw)
    o_r = kernels.attention_reference(qd, kd, vd, T, lens=ld, **kw)
    f_c = kernels.attention_compressed(qd, kc, vc, T, lens=ld, fused_merge=True, **kw)
    f_r = kernels.attention_reference(qd, kd, vd, T, lens=ld, fused_merge=True, **kw)
    torch.cuda.synchronize()
    assert same_bits(o_c, o_r), "compressed and bf16 twin differ"
    assert same_bits(f_c, f_r), "compressed and bf16 twin differ (merge in the split kernel)"
    assert torch.isfinite(o_c.float()).all()
    kq, vq = u16(k), u16(v)
    qq = u16(q)
    r32 = oatt.attention(qq, kq, vq, T, np.float32, lens=lens)
    assert_bf16_tolerance(o_c, r32)
    assert_bf16_tolerance(f_c, r32)
    if fp64:
        r64 = oatt.attention(qq, kq, vq, T, np.float64, lens=lens)
        assert np.abs(o_c.double().cpu().numpy() - r64).max() < 2e-2
    return o_c


@pytest.fixture(scope="module")
def c1_data():
    q, k, v = _data(1, 32768, 28, 4, seed=1100)
    kd, vd = k.to(DEV), v.to(DEV)
    return q, k, v, _encode(kd), _encode(vd), kd, vd


def test_c1_qwen25_b1_32k(c1_data):
    q, k, v, kc, vc, kd, vd = c1_data
    _say("c1", 1, 32768, 28, 4, "plan", kernels.plan_splits(1, 4, 28, 32768))
    assert int(kc.cnt.item()) > 0 and (kc.base >= 128).any()      # raw rows and zero-flag groups present
    _check_call(q, k, v, kc, vc, kd, vd, 32768)


@pytest.fixture(scope="module")
def c2a_data():
    q, k, v = _data(8, 8192, 32, 8, seed=1200)
    kd, vd = k.to(DEV), v.to(DEV)
    return q, k, v, _encode(kd), _encode(vd), kd, vd


@pytest.mark.parametrize("T", [8192, 8185])
def test_c2a_llama31_b8_8k(c2a_data, T):
    q, k, v, kc, vc, kd, vd = c2a_data
    _say("c2a", 8, T, 32, 8, "plan", kernels.plan_splits(8, 8, 32, T))
    _check_call(q, k, v, kc, vc, kd, vd, T)


def test_c2a_graph_replay_and_cache_objects(c2a_data):
    """The headline call through CompressedKV objects (prefill_slot) and a captured HIP
    graph: every replay equals the eager call bit for bit."""
    q, k, v, _, _, kd, vd = c2a_data
    B, T, TS, Hkv = 8, 8185, 8192, 8
    kc, vc = exactkv.CompressedKV(B, TS, Hkv, 128), exactkv.CompressedKV(B, TS, Hkv, 128)
    for b in range(B):
        kc.prefill_slot(b, kd[b:b + 1, :T])
        vc.prefill_slot(b, vd[b:b + 1, :T])
    qd = q.to(DEV)
    _say("c2a cache objects + graph", T)
    o_e = exactkv.decode_attention(qd, kc, vc)
    assert same_bits(o_e, kernels.attention_reference(qd, kd, vd, T))
    out = torch.empty_like(qd)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kernels.attention_compressed(qd, kc, vc, T, out=out)      # workspace allocated outside capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            kernels.attention_compressed(qd, kc, vc, T, out=out)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert same_bits(out, o_e), f"replay {i}"
        assert same_bits(exactkv.decode_attention(qd, kc, vc), o_e)   # eager work between replays


@pytest.fixture(scope="module")
def c2b_data():
    q, k, v = _data(1, 131072, 32, 8, seed=1300)
    kd, vd = k.to(DEV), v.to(DEV)
    return q, k, v, _encode(kd), _encode(vd), kd, vd


@pytest.mark.parametrize("T", [131072, 131065])
def test_c2b_llama31_b1_128k(c2b_data, T):
    q, k, v, kc, vc, kd, vd = c2b_data
    _say("c2b", 1, T, 32, 8, "plan", kernels.plan_splits(1, 8, 32, T))
    _check_call(q, k, v, kc, vc, kd, vd, T, fp64=False)


@pytest.mark.parametrize("paged", [False, True])
def test_long_splits_walk_past_64_pages(paged):
    """nsplit = 1: each wavefront walks every page of its head (T = 2041: 128 pages, the last
    partly filled), past the 64 pages whose metadata it holds in registers."""
    B, TS, Hq, Hkv, T = 2, 2048, 32, 8, 2041
    q, k, v = _data(B, TS, Hq, Hkv, seed=1400, raw_row_rate=0.02)
    kd, vd = k.to(DEV), v.to(DEV)
    npg = TS // P
    _say("long splits", B, T, Hq, Hkv, "paged" if paged else "contiguous")
    if not paged:
        kc, vc = _encode(kd), _encode(vd)
        _check_call(q, k, v, kc, vc, kd, vd, T, nsplit=1, split_len=TS)
        return
    pool_pages = B * npg + 11
    perm = torch.randperm(pool_pages, generator=torch.Generator().manual_seed(14))[:B * npg]
    table = perm.view(B, npg).to(torch.int32)
    kp = torch.zeros(1, pool_pages * P, Hkv, 128, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    rows = (table.long()[:, :, None] * P + torch.arange(P)[None, None, :]).reshape(B, TS)
    for b in range(B):
        kp[0, rows[b]] = k[b]
        vp[0, rows[b]] = v[b]
    kpd, vpd = kp.to(DEV), vp.to(DEV)
    kpc, vpc = _encode(kpd), _encode(vpd)
    qd = q.to(DEV)
    bt = table.to(DEV)
    o_p = kernels.attention_compressed(qd, kpc, vpc, T, block_table=bt, nsplit=1, split_len=TS)
    o_pb = kernels.attention_reference(qd, kpd, vpd, T, block_table=bt, nsplit=1, split_len=TS)
    o_g = kernels.attention_reference(qd, kd, vd, T, nsplit=1, split_len=TS)
    assert same_bits(o_p, o_pb)
    assert same_bits(o_p, o_g)
    assert_bf16_tolerance(o_p, oatt.attention(u16(q), u16(k), u16(v), T, np.float32))
    # the default plan through the block table, merged in the split kernel's tail
    f_p = kernels.attention_compressed(qd, kpc, vpc, T, block_table=bt, fused_merge=True)
    assert same_bits(f_p, kernels.attention_reference(qd, kpd, vpd, T, block_table=bt, fused_merge=True))
    assert same_bits(f_p, kernels.attention_reference(qd, kd, vd, T, fused_merge=True))
    assert_bf16_tolerance(f_p, oatt.attention(u16(q), u16(k), u16(v), T, np.float32))


def test_c3_qwen3_b32_variable_lengths_growth_and_appends():
    """Prefill 4085 tokens of 32 sequences (the last page open) into caches whose raw pools
    start at their minimum (B*H*16 rows) and grow during the prefill; 27 appends cross two
    page boundaries (check_overflow after each); attention with per-sequence lengths
    U[3500, T]."""
    B, Hq, Hkv, T0, NEW = 32, 32, 8, 4085, 27
    TS = T0 + NEW
    q, k, v = _data(B, TS, Hq, Hkv, seed=1500, raw_row_rate=6e-3)
    kc = exactkv.CompressedKV(B, TS, Hkv, 128, reserve=0.0)
    vc = exactkv.CompressedKV(B, TS, Hkv, 128, reserve=0.0)
    cap0 = kc.cap
    kr, vr = exactkv.BF16KV(B, TS, Hkv, 128), exactkv.BF16KV(B, TS, Hkv, 128)
    _say("c3 prefill", B, T0, "cap", cap0)
    kd, vd = k.to(DEV), v.to(DEV)
    for b in range(B):
        for c, r, x in ((kc, kr, kd), (vc, vr, vd)):
            xb = x[b:b + 1, :T0]
            c.prefill_slot(b, xb)
            r.prefill_slot(b, xb)
    assert kc.cap >= 3 * cap0 and vc.cap >= 3 * cap0, (cap0, kc.cap, vc.cap)
    assert kc.grows >= 2 and vc.grows >= 2
    rng = np.random.Generator(np.random.PCG64(1501))
    qd = q.to(DEV)
    checked = 0
    for t in range(T0, TS):
        for c, r, x in ((kc, kr, kd), (vc, vr, vd)):
            xt = x[:, t].contiguous()
            c.append(xt)
            r.append(xt)
        exactkv.check_overflow([kc, vc])
        T = kc.T
        if T % P in (0, 1, 9):
            lens = rng.integers(3500, T + 1, B)
            _say("c3 step", T, "lens", int(lens.min()), int(lens.max()))
            ld = torch.tensor(lens, dtype=torch.int32, device=DEV)
            o_c = kernels.attention_compressed(qd, kc, vc, T, lens=ld)
            assert same_bits(o_c, kernels.attention_reference(qd, kr.buf, vr.buf, T, lens=ld)), T
            f_c = kernels.attention_compressed(qd, kc, vc, T, lens=ld, fused_merge=True)
            assert same_bits(f_c, kernels.attention_reference(qd, kr.buf, vr.buf, T, lens=ld, fused_merge=True)), T
            ref = oatt.attention(u16(q), u16(k[:, :T]), u16(v[:, :T]), T, np.float32, lens=lens)
            assert oatt.tolerance_excess(o_c.float().cpu().numpy(), ref) <= 0, T
            assert oatt.tolerance_excess(f_c.float().cpu().numpy(), ref) <= 0, T
            assert same_bits(exactkv.decode_attention(qd, kc, vc), exactkv.decode_attention(qd, kr, vr)), T
            checked += 1
    assert checked >= 5
    for c, r in ((kc, kr), (vc, vr)):
        assert same_bits(kernels.decode_to_bf16(c.buffers(), c.T), r.buf[:, :c.T])
        assert int(c.cnt.item()) <= c.cap


def test_c4_llama31_layer_shapes_tokens_and_logits():
    """Engine at Llama-3.1-8B layer shapes (2 of its 32 layers, bf16 weights N(0, 0.02)):
    4 prompts of 200 random tokens, 40 greedy tokens (page boundaries at 208, 224, 240,
    inside HIP-graph steps). Both cache backends: identical tokens, bit-identical logits."""
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=2,
                      num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=131072,
                      rope_theta=5e5, rms_norm_eps=1e-5, initializer_range=0.02, tie_word_embeddings=False)
    torch.manual_seed(0)
    with torch.device(DEV):
        m = LlamaForCausalLM(cfg)
    m = m.to(torch.bfloat16).eval()
    B, PROMPT, NEW = 4, 200, 40
    ids = torch.randint(0, cfg.vocab_size, (B, PROMPT), generator=torch.Generator().manual_seed(7)).to(DEV)
    out = {}
    for be in ("bf16", "exactkv"):
        _say("c4 engine", be)
        eng = exactkv.Engine(m, B, PROMPT + NEW, backend=be)
        out[be] = eng.generate(ids, NEW)
        torch.cuda.synchronize()
        assert eng.use_graph and eng.captures >= 1
        del eng
    (tb, lb), (tc, lc) = out["bf16"], out["exactkv"]
    assert torch.equal(tb, tc)
    assert same_bits(lb, lc)
    assert torch.isfinite(lc.float()).all()
