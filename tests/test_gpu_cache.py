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


@pytest.mark.parametrize("B,H,T0,TS,rate", [(600, 8, 13, 48, 0.5), (1040, 8, 9, 48, 0.05)])
def test_append_page_ends_with_many_units_and_raw_rows(B, H, T0, TS, rate):
    """The one-launch append's page end with many (sequence, head) units: 4,800 units with
    half the rows raw (the raw rows, several per thread of the last workgroup, found through
    its LDS table of ranks), and 8,320 units, more than that table holds (each thread moves
    its own units' rows). Byte-equal to the CPU model of the protocol at every page end; the
    arrival counter state[1] is zero after every append."""
    g = torch.Generator().manual_seed(5)
    D = 128
    _say("append many units", B, H, T0, TS, rate)
    c = exactkv.CompressedKV(B, TS, H, D, reserve=0.6)
    m = ocache.CacheModel(B, TS, H, D, reserve=0.6)
    x0 = _make(g, B, T0, H, D, rate)
    x0d = x0.to(DEV)
    for b in range(B):
        c.prefill_slot(b, x0d[b:b + 1].contiguous())
        m.prefill_slot(b, u16(x0[b]))
    xs = _make(g, B, TS - T0, H, D, rate)
    xsd = xs.to(DEV)
    ends = 0
    for t in range(TS - T0):
        c.append(xsd[:, t].contiguous())
        m.append(u16(xs[:, t]))
        exactkv.check_overflow([c])
        m.check_overflow()
        assert int(c.state[1].item()) == 0, t
        if c.T % 16 == 0:
            _state_equal(c, m, t)
            ends += 1
    assert ends >= 2
