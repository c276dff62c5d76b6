"""Wire form on the GPU: pack / unpack of one sequence's compressed cache.

No counterpart in the reference (a byte form of buffers(), cache.py:121-123, is this
build's own). Gates:
  * the GPU blob equals the oracle's blob byte for byte (oracle/wire.py);
  * unpacking into another cache, contiguous or paged, gives the same decoded values and
    bit-identical attention, and decoding can go on from there;
  * a raw pool too small for the blob grows first.
"""
import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import kernels, synthetic, wire
from oracle import wire as owire
from tests.conftest import same_bits, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = 16


def _say(*a):
    print("[case]", *a, flush=True)


def _cache(x, reserve=0.01):
    B, T, H, D = x.shape
    TS = -(-T // P) * P + P
    c = exactkv.CompressedKV(B, TS, H, D, reserve=reserve)
    for b in range(B):
        c.prefill_slot(b, x[b:b + 1].to(DEV).contiguous())
    return c


@pytest.mark.parametrize("T", [37, 1024, 5, 16])
def test_pack_matches_oracle(T):
    H = 8
    x = synthetic.make_kv(2, T, H, kind="k", seed=91 + T, raw_row_rate=0.02)
    c = _cache(x)
    for b in range(2):
        _say("wire pack", T, b)
        blob = wire.pack(c, b)
        want = owire.pack(u16(x[b]))
        assert blob.numel() == want.size
        got = blob.cpu().numpy()
        assert np.array_equal(got, want), f"first difference at byte {int(np.argmax(got != want))}"


def test_unpack_into_contiguous_cache():
    B, T, H, Hq = 3, 200, 8, 32
    k = synthetic.make_kv(B, T, H, kind="k", seed=3, raw_row_rate=0.02)
    v = synthetic.make_kv(B, T, H, kind="v", seed=4, raw_row_rate=0.02)
    ka, va = _cache(k), _cache(v)
    kb = exactkv.CompressedKV(B, ka.TS, H, 128, reserve=1e-4)       # grows on unpack
    vb = exactkv.CompressedKV(B, va.TS, H, 128, reserve=1e-4)
    _say("wire unpack contiguous", B, T)
    for b in reversed(range(B)):                                   # another raw-slot order
        wire.unpack(wire.pack(ka, b), kb, b)
        wire.unpack(wire.pack(va, b), vb, b)
    assert kb.T == T and kb.grows > 0
    assert same_bits(kernels.decode_to_bf16(kb.buffers(), T), k.to(DEV))
    assert same_bits(kernels.decode_to_bf16(vb.buffers(), T), v.to(DEV))
    q = synthetic.make_q(B, Hq, seed=5).to(DEV)
    assert same_bits(exactkv.decode_attention(q, kb, vb), exactkv.decode_attention(q, ka, va))
    xk = synthetic.make_kv(B, 1, H, kind="k", seed=6)[:, 0].to(DEV).contiguous()
    xv = synthetic.make_kv(B, 1, H, kind="v", seed=7)[:, 0].to(DEV).contiguous()
    for c, x in ((ka, xk), (va, xv), (kb, xk), (vb, xv)):
        c.append(x)
    exactkv.check_overflow([ka, va, kb, vb])
    assert same_bits(exactkv.decode_attention(q, kb, vb), exactkv.decode_attention(q, ka, va))


def test_paged_pack_unpack_into_another_pool():
    H, Hq = 4, 16
    lens = [45, 16, 130, 3]
    ta = exactkv.PageTable(num_pages=40, max_seqs=4, max_pages=12)
    tb = exactkv.PageTable(num_pages=50, max_seqs=4, max_pages=12)
    ka, va = exactkv.PagedCompressedKV(ta, H), exactkv.PagedCompressedKV(ta, H)
    kb, vb = exactkv.PagedCompressedKV(tb, H, reserve=1e-4), exactkv.PagedCompressedKV(tb, H, reserve=1e-4)
    kt, vt = exactkv.PagedBF16KV(tb, H), exactkv.PagedBF16KV(tb, H)
    src_k = synthetic.make_kv(4, 192, H, kind="k", seed=21, raw_row_rate=0.03)
    src_v = synthetic.make_kv(4, 192, H, kind="v", seed=22, raw_row_rate=0.03)
    tb.add(20)                                                      # occupy low pages of pool b
    for s, T in enumerate(lens):
        ta.add(T)
        ka.prefill(s, src_k[s:s + 1, :T].to(DEV).contiguous())
        va.prefill(s, src_v[s:s + 1, :T].to(DEV).contiguous())
    for i in range(9):                                              # appends across page boundaries
        ta.begin_step()
        ka.append(torch.stack([src_k[s, ta.length(s) - 1] for s in range(4)]).to(DEV).contiguous())
        va.append(torch.stack([src_v[s, ta.length(s) - 1] for s in range(4)]).to(DEV).contiguous())
        exactkv.check_overflow([ka, va])
    tb.release(0)
    _say("wire paged", [ta.length(s) for s in range(4)])
    order = (2, 0, 3, 1)                                            # slots in another order
    kblobs = wire.pack_many(ka, order)                              # one call for all K
    for s in order:
        tb.add(ta.length(s), slot=s)
    wire.unpack_many(kblobs, kb, order)
    for s in order:
        T = ta.length(s)
        assert same_bits(kblobs[order.index(s)], wire.pack(ka, s))  # batch == one at a time
        wire.unpack(wire.pack(va, s), vb, s)                        # V one call per sequence
        kt.prefill(s, src_k[s:s + 1, :T].to(DEV).contiguous())
        vt.prefill(s, src_v[s:s + 1, :T].to(DEV).contiguous())
    for c in (kb, vb):
        dec = kernels.decode_to_bf16(c.buffers(), c.TS)
        src = src_k if c is kb else src_v
        for s in range(4):
            rows = (torch.tensor(tb.pages(s))[:, None] * P + torch.arange(P)[None, :]).reshape(-1)[:tb.length(s)]
            assert same_bits(dec[0][rows.to(DEV)], src[s, :tb.length(s)].to(DEV)), f"slot {s}"
    for i in range(20):                                             # decoding goes on in pool b
        tb.begin_step()
        xk = torch.stack([src_k[s, tb.length(s) - 1] for s in range(4)]).to(DEV).contiguous()
        xv = torch.stack([src_v[s, tb.length(s) - 1] for s in range(4)]).to(DEV).contiguous()
        for c, x in ((kb, xk), (vb, xv), (kt, xk), (vt, xv)):
            c.append(x)
        q = synthetic.make_q(4, Hq, seed=100 + i).to(DEV)
        assert same_bits(exactkv.decode_attention(q, kb, vb), exactkv.decode_attention(q, kt, vt)), f"step {i}"
        exactkv.check_overflow([kb, vb])


def test_bad_blobs_raise():
    x = synthetic.make_kv(1, 40, 2, kind="k", seed=1)
    c = _cache(x)
    blob = wire.pack(c, 0)
    bad = blob.clone()
    bad[0] = 0
    with pytest.raises(ValueError, match="not an exactkv"):
        wire.unpack(bad, c, 0)
    with pytest.raises(ValueError, match="heads"):
        wire.unpack(blob, exactkv.CompressedKV(1, 64, 4, 128), 0)
    with pytest.raises(ValueError, match="shorter"):
        wire.unpack(blob[:-256].clone() if blob.numel() > 512 else blob[:300].clone(), c, 0)


def test_unpack_skips_a_blob_whose_rowmask_disagrees_with_its_header(monkeypatch):
    """The kernel's own check (behind the host's): a blob whose rowmask marks more raw rows
    than its header declares is skipped on the device -- its sequence is not written and
    the counter advances by the declared rows only -- while the blob before it unpacks."""
    H = 4
    x = synthetic.make_kv(2, 64, H, kind="k", seed=31, raw_row_rate=0.05)
    src = _cache(x)
    good, bad = wire.pack(src, 0), wire.pack(src, 1)
    h = wire.header(bad)
    rm = bad[h["off_rowmask"]: h["off_rowmask"] + 4 * h["full_pages"] * H].view(torch.int32)
    rm[0] |= 0xFFFF                                     # every token of page 0, head 0 raw
    with pytest.raises(ValueError, match="declares"):
        wire.unpack_many([good, bad], exactkv.CompressedKV(2, src.TS, H, 128), [0, 1])
    monkeypatch.setattr(wire, "_check_blob", lambda b, c: wire.header(b))   # past the host check
    dst = exactkv.CompressedKV(2, src.TS, H, 128)
    cnt0 = int(dst.cnt.item())
    _say("wire corrupt blob", wire.header(good)["raw_rows"], h["raw_rows"])
    wire.unpack_many([good, bad], dst, [0, 1])
    torch.cuda.synchronize()
    assert int(dst.cnt.item()) == cnt0 + wire.header(good)["raw_rows"] + h["raw_rows"]
    assert same_bits(kernels.decode_to_bf16(dst.buffers(), 64)[0], x[0].to(DEV))
    assert int(dst.sm[1].sum().item()) == 0 and int(dst.code[1].sum().item()) == 0
