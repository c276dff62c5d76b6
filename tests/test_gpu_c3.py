"""Config-3 style stress at test size (reference tests/test_exactkv.py:81-104 extended with
the per-sequence lengths of the north star's c3): 0.6% outlier rows, a raw pool that
starts at its minimum and grows, appends across page boundaries, and attention with
per-sequence lengths drawn below the cache length.

At every checked step: attention with lens is bit-identical between the compressed and
the bf16 cache and within the bf16 tolerance of the oracle's fp32 attention; the decoded
cache equals the bf16 cache."""
import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import kernels, synthetic
from oracle import attention as oatt
from tests.conftest import same_bits, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_c3_variable_lengths_outliers_and_growth():
    B, Hq, Hkv, T0, NEW = 8, 32, 8, 512, 96
    TS = T0 + NEW
    print("[case] c3-style", B, Hq, Hkv, T0, NEW, flush=True)
    k = synthetic.make_kv(B, TS, Hkv, kind="k", seed=40, raw_row_rate=6e-3)
    v = synthetic.make_kv(B, TS, Hkv, kind="v", seed=41, raw_row_rate=6e-3)
    q = synthetic.make_q(B, Hq, seed=42, device=DEV)
    kc, vc = exactkv.CompressedKV(B, TS, Hkv, 128, reserve=0.0), exactkv.CompressedKV(B, TS, Hkv, 128, reserve=0.0)
    kr, vr = exactkv.BF16KV(B, TS, Hkv, 128), exactkv.BF16KV(B, TS, Hkv, 128)
    for b in range(B):
        for c, r, x in ((kc, kr, k), (vc, vr, v)):
            xb = x[b:b + 1, :T0].to(DEV).contiguous()
            c.prefill_slot(b, xb)
            r.prefill_slot(b, xb)
    rng = np.random.Generator(np.random.PCG64(43))
    checked = 0
    for t in range(T0, TS):
        for c, r, x in ((kc, kr, k), (vc, vr, v)):
            xt = x[:, t].to(DEV).contiguous()
            c.append(xt)
            r.append(xt)
        exactkv.check_overflow([kc, vc])
        T = kc.T
        if t % 16 == 5 or t == TS - 1:
            lens = rng.integers(int(0.85 * T), T + 1, B)
            ld = torch.tensor(lens, dtype=torch.int32, device=DEV)
            o_c = kernels.attention_compressed(q, kc, vc, T, lens=ld)
            o_r = kernels.attention_reference(q, kr.buf, vr.buf, T, lens=ld)
            assert same_bits(o_c, o_r), t
            ref = oatt.attention(u16(q), u16(kr.buf[:, :T]), u16(vr.buf[:, :T]), T, np.float32, lens=lens)
            excess = oatt.tolerance_excess(o_c.float().cpu().numpy(), ref)
            assert excess <= 0, (t, excess)
            assert same_bits(kernels.decode_to_bf16(kc.buffers(), T), kr.buf[:, :T]), t
            assert same_bits(kernels.decode_to_bf16(vc.buffers(), T), vr.buf[:, :T]), t
            checked += 1
    assert checked >= 6
    assert kc.grows + vc.grows >= 2
    assert int(kc.cnt.item()) > 0 and int(vc.cnt.item()) > 0
