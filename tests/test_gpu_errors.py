"""The kernels' sticky error bits (exkv_error_bits): a call that gives up a bounded wait or
reads a clamped raw-row slot must say so, where it used to return wrong bits silently.

No counterpart in the reference (its one such condition, raw-pool overflow, is the
counter check_overflow reads, cache.py:149-158; that protocol is unchanged and is not an
error bit). Every condition here is forced from the host so that every kernel still ends
normally: a bound of one poll on the split kernels' flag waits (exkv_set_wait_limit), or a
page's rowoff moved past the pool, which the kernels clamp back into it (no access leaves
the buffers). The conftest fixture checks that every other GPU test leaves the bits clear."""
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import _lib, kernels, synthetic, wire
from tests.conftest import same_bits

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = 16


def _say(*a):
    print("[case]", *a, flush=True)


def _caches(B, T, H, seed, rate=0.02):
    out = []
    for kind, s in (("k", seed), ("v", seed + 1)):
        x = synthetic.make_kv(B, T, H, kind=kind, seed=s, raw_row_rate=rate).to(DEV)
        c = exactkv.CompressedKV(B, T, H, 128)
        for b in range(B):
            c.prefill_slot(b, x[b:b + 1])
        out += [c, x]
    return out


def test_a_wait_that_gives_up_is_reported():
    B, T, Hq, H = 8, 2048, 32, 8
    kc, k, vc, v = _caches(B, T, H, seed=700)
    q = synthetic.make_q(B, Hq, seed=702).to(DEV)
    want = kernels.attention_reference(q, k, v, T)
    assert kernels.error_bits() == 0
    _say("errors: wait limit 1", B, T)
    kernels.set_wait_limit(1)           # every compute wavefront gives up on its first page
    try:
        kernels.attention_compressed(q, kc, vc, T)
        bits = kernels.error_bits()
    finally:
        kernels.set_wait_limit(0)
    assert bits & 0x1, f"bits {bits:#x}"
    _say("errors: default limit again")
    got = kernels.attention_compressed(q, kc, vc, T)
    assert same_bits(got, want)
    assert kernels.error_bits() == 0
    with pytest.raises(RuntimeError, match="LDS flag"):
        kernels.set_wait_limit(1)
        try:
            kernels.attention_compressed(q, kc, vc, T)
            kernels.check_errors()
        finally:
            kernels.set_wait_limit(0)


def _page_with_raw_rows(c):
    """(sequence, page, head) of a full page holding raw rows."""
    m = c.rowmask[:, : c.T // P]
    idx = torch.nonzero(m != 0)
    assert idx.shape[0] > 0
    b, pg, h = (int(x) for x in idx[idx.shape[0] // 2])
    return b, pg, h


def test_a_clamped_raw_slot_is_reported_by_attention_and_decode():
    B, T, Hq, H = 4, 1024, 32, 8
    kc, k, vc, v = _caches(B, T, H, seed=710)
    q = synthetic.make_q(B, Hq, seed=712).to(DEV)
    b, pg, h = _page_with_raw_rows(kc)
    keep = kc.rowoff[b, pg, h].item()
    _say("errors: rowoff past the pool", b, pg, h, keep, kc.raw.shape[0])
    kc.rowoff[b, pg, h] = kc.raw.shape[0] + 1000       # the kernels clamp it back into the pool
    kernels.attention_compressed(q, kc, vc, T)
    assert kernels.error_bits() & 0x2
    kernels.decode_to_bf16(kc.buffers(), T)
    assert kernels.error_bits() & 0x2
    kc.rowoff[b, pg, h] = -5
    kernels.decode_to_bf16(kc.buffers(), T)
    assert kernels.error_bits() & 0x2
    kc.rowoff[b, pg, h] = keep
    got = kernels.attention_compressed(q, kc, vc, T)
    assert same_bits(got, kernels.attention_reference(q, k, v, T))
    assert same_bits(kernels.decode_to_bf16(kc.buffers(), T), k)
    assert kernels.error_bits() == 0


def test_a_clamped_raw_slot_is_reported_by_wire_pack():
    B, T, H = 2, 400, 8
    kc, k, _, _ = _caches(B, T, H, seed=720)
    b, pg, h = _page_with_raw_rows(kc)
    keep = kc.rowoff[b, pg, h].item()
    blob = wire.pack(kc, b)
    assert kernels.error_bits() == 0
    kc.rowoff[b, pg, h] = kc.raw.shape[0] + 7
    _say("errors: wire pack with rowoff past the pool", b, pg, h)
    wire.pack(kc, b)
    assert kernels.error_bits() & 0x10
    kc.rowoff[b, pg, h] = keep
    assert torch.equal(wire.pack(kc, b), blob)
    assert kernels.error_bits() == 0


def test_debug_mode_raises_at_the_call(monkeypatch):
    """EXACTKV_CHECK_ERRORS=1: the call that set a bit raises."""
    B, T, Hq, H = 2, 512, 32, 8
    kc, k, vc, v = _caches(B, T, H, seed=730)
    q = synthetic.make_q(B, Hq, seed=732).to(DEV)
    monkeypatch.setattr(_lib, "_CHECK", True)
    kernels.attention_compressed(q, kc, vc, T)          # sound: no raise
    b, pg, h = _page_with_raw_rows(kc)
    kc.rowoff[b, pg, h] = kc.raw.shape[0] + 3
    with pytest.raises(RuntimeError, match="error bits 0x2"):
        kernels.attention_compressed(q, kc, vc, T)
    assert kernels.error_bits() == 0                    # the raising check cleared them
