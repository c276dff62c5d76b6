"""CompressedKV on the GPU: append, page encode, raw-pool growth (reference cache.py:17-158;
reference test tests/test_exactkv.py:81-104), checked against the plain bf16 cache and,
byte for byte, against the CPU model of the protocol (oracle/cache.py)."""
import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import kernels
from oracle import cache as ocache
from tests.conftest import same_bits, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[case]", *a, flush=True)


def _make(g, B, n, H, D, rate):
    x = torch.randn(B, n, H, D, generator=g).to(torch.bfloat16)
    x[torch.rand(B, n, H, generator=g) < rate, 7] = 1e-30          # forces raw rows
    return x


def _state_equal(c, m, tag):
    for k in ("sm", "code", "base", "rowmask", "rowoff"):
        assert np.array_equal(getattr(c, k).cpu().numpy(), getattr(m, k)), (tag, k)
    assert np.array_equal(u16(c.raw), m.raw), (tag, "raw")
    assert int(c.cnt.item()) == m.cnt and c.cap == m.cap and c.T == m.T and c.grows == m.grows, tag
    assert int(c.state[0].item()) == c.T, tag


@pytest.mark.parametrize("B,H,T0,TS,rate,reserve", [(2, 4, 1000, 1200, 0.1, 0.001), (3, 2, 33, 160, 0.02, 0.01),
                                                    (1, 8, 0, 96, 0.3, 0.0)])
def test_append_and_pool_growth(B, H, T0, TS, rate, reserve):
    g = torch.Generator().manual_seed(2)
    D = 128
    _say("append", B, H, T0, TS, rate, reserve)
    c, r = exactkv.CompressedKV(B, TS, H, D, reserve=reserve), exactkv.BF16KV(B, TS, H, D)
    m = ocache.CacheModel(B, TS, H, D, reserve=reserve)
    x0 = _make(g, B, T0, H, D, rate)
    q = torch.randn(B, 32, D, generator=g).to(torch.bfloat16).to(DEV)
    if T0:
        for b in range(B):
            c.prefill_slot(b, x0[b:b + 1].to(DEV).contiguous())
            r.prefill_slot(b, x0[b:b + 1].to(DEV).contiguous())
            m.prefill_slot(b, u16(x0[b]))
        _state_equal(c, m, "prefill")
    xs = _make(g, B, TS - T0, H, D, rate)
    for t in range(TS - T0):
        xt = xs[:, t].to(DEV).contiguous()
        c.append(xt)
        r.append(xt)
        m.append(u16(xs[:, t]))
        if c.T % 16 == 0:                      # the page encode inside the step never overflows
            assert int(c.cnt.item()) <= c.cap
        exactkv.check_overflow([c])
        m.check_overflow()
        if t % 37 == 0 or t == TS - T0 - 1:
            _state_equal(c, m, t)
            assert same_bits(kernels.decode_to_bf16(c.buffers(), c.T), r.buf[:, :c.T]), t
            assert same_bits(exactkv.decode_attention(q, c, c), exactkv.decode_attention(q, r, r)), t
    assert int(r.state[0].item()) == TS
    assert c.grows > 0 or reserve >= 0.01


def test_prefill_overflow_regrows_and_matches_codec():
    """A prefill whose raw rows exceed the pool: grow, rewind, re-encode (cache.py:77-84)."""
    from oracle import codec as ocodec
    from exactkv_amd import synthetic
    x = synthetic.stress_pages(2, 128, 2, seed=17)
    B, T, H, D = x.shape
    c = exactkv.CompressedKV(B, T, H, D, reserve=0.0)
    for b in range(B):
        c.prefill_slot(b, x[b:b + 1].to(DEV).contiguous())
    ref = ocodec.encode(u16(x))
    n = int(c.cnt.item())
    assert c.grows > 0 and n == ref["raw"].shape[0]
    for k in ("sm", "code", "base", "rowmask", "rowoff"):
        assert np.array_equal(getattr(c, k).cpu().numpy(), ref[k]), k
    assert np.array_equal(u16(c.raw[:n]), ref["raw"])
