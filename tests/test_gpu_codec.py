"""GPU encoder and decoder vs the CPU oracle (reference codec.py:31-73; reference GPU
test tests/test_exactkv.py:52-58, here with all six tensors byte-identical)."""
import json
import os

import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import synthetic
from exactkv_amd import kernels
from oracle import codec as ocodec
from tests.conftest import same_bits, u16
from tests.golden import cases

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _say(*a):
    print("[case]", *a, flush=True)


def _gpu_encode(x):
    """Encode [B,T,H,D] with the HIP encoder into fresh cache buffers (reference tests:19-26)."""
    B, T, H, D = x.shape
    c = exactkv.CompressedKV(B, T, H, D, reserve=1.0)
    st = (x.stride(0), 16 * x.stride(1), x.stride(1), x.stride(2))
    kernels.encode_pages(x, st, c._buf(), 0, 0, B, T // 16)
    assert int(c.cnt.item()) <= c.cap
    return c


def _compare(c, ref, name):
    for k in ("sm", "code", "base", "rowmask", "rowoff"):
        assert np.array_equal(getattr(c, k).cpu().numpy(), ref[k]), (name, k)
    n = int(c.cnt.item())
    assert n == ref["raw"].shape[0], name
    assert np.array_equal(u16(c.raw[:n]), ref["raw"]), (name, "raw")


@pytest.mark.parametrize("name", list(cases.CASES))
def test_encoder_bytes_equal_oracle_and_decode_exact(name):
    x = cases.CASES[name][0]()
    _say("encoder", name, tuple(x.shape))
    ref = ocodec.encode(u16(x))
    xd = x.to(DEV)
    c = _gpu_encode(xd)
    _compare(c, ref, name)
    assert same_bits(kernels.decode_to_bf16(c.buffers(), x.shape[1]), xd), name


def test_encode_reference_api_matches_golden_bytes():
    z = np.load(os.path.join(GOLD, "codec_vectors.npz"))
    for name, (make, stored) in cases.CASES.items():
        if not stored:
            continue
        _say("encode_reference", name)
        x = make()
        c = exactkv.encode_reference(x)                 # CPU in, CPU out, computed on the GPU
        for k in ("sm", "code", "base", "rowmask", "rowoff", "raw"):
            got = c[k].numpy() if k != "raw" else u16(c[k])
            assert np.array_equal(got, z[f"{name}/{k}"]), (name, k)
        assert same_bits(exactkv.decode_reference(c), x), name
        cg = exactkv.encode_reference(x.to(DEV))        # GPU in, GPU out
        assert cg["sm"].is_cuda and same_bits(exactkv.decode_reference(cg), x.to(DEV))


def test_encode_reference_hashed_cases():
    import hashlib
    h = json.load(open(os.path.join(GOLD, "codec_hashes.json")))["cases"]
    for name, (make, stored) in cases.CASES.items():
        if stored:
            continue
        _say("encode_reference hashed", name)
        c = exactkv.encode_reference(make().to(DEV))
        for k in ("sm", "code", "base", "rowmask", "rowoff", "raw"):
            a = u16(c[k]) if k == "raw" else c[k].cpu().numpy()
            assert hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest() == h[name][k]["sha256"], (name, k)


def test_encoder_strided_source_and_offsets():
    """Encode pages [pg0, pg0+npg) of sequences [b0, b0+nb) from a strided view."""
    big = synthetic.make_kv(3, 96, 8, kind="k", seed=4).to(DEV)
    src = big[:, :, ::2]                                  # heads 0, 2, 4, 6: head stride 256
    B, T, H, D = src.shape
    _say("strided encode", tuple(src.shape), src.stride())
    c = exactkv.CompressedKV(4, 128, H, D, reserve=1.0)
    st = (src.stride(0), 16 * src.stride(1), src.stride(1), src.stride(2))
    kernels.encode_pages(src[1:], st, c._buf(), 2, 1, 2, T // 16)        # sequences 2,3 pages 1..6
    ref = ocodec.encode(u16(src[1:].contiguous()))
    NP = T // 16
    assert np.array_equal(c.sm[2:4, 16:16 + T].cpu().numpy(), ref["sm"])
    assert np.array_equal(c.code[2:4, 16:16 + T].cpu().numpy(), ref["code"])
    assert np.array_equal(c.base[2:4, 1:1 + NP].cpu().numpy(), ref["base"])
    assert np.array_equal(c.rowmask[2:4, 1:1 + NP].cpu().numpy(), ref["rowmask"])
    assert np.array_equal(c.rowoff[2:4, 1:1 + NP].cpu().numpy(), ref["rowoff"])
    assert not c.sm[:2].any() and not c.sm[2:4, :16].any()              # nothing else written


def test_encoder_overflow_skips_rows_past_cap():
    x = synthetic.stress_pages(1, 64, 2, seed=9).to(DEV)       # many raw rows
    ref = ocodec.encode(u16(x))
    n = ref["raw"].shape[0]
    B, T, H, D = x.shape
    c = exactkv.CompressedKV(B, T, H, D, reserve=0.0)                   # cap 64 < n
    assert n > c.cap
    sentinel = torch.full_like(c.raw, 7.0)
    c.raw.copy_(sentinel)
    st = (x.stride(0), 16 * x.stride(1), x.stride(1), x.stride(2))
    kernels.encode_pages(x, st, c._buf(), 0, 0, B, T // 16)
    assert int(c.cnt.item()) == n and int(c._before.item()) == 0
    assert np.array_equal(u16(c.raw[: c.cap]), ref["raw"][: c.cap])
    assert same_bits(c.raw[c.cap:], sentinel[c.cap:])                  # tail area untouched


@pytest.mark.parametrize("T", [1, 15, 16, 17, 100, 128])
def test_decode_partial_lengths(T):
    x = cases.CASES["allpat_perm"][0]().to(DEV)
    c = _gpu_encode(x)
    _say("decode T", T)
    assert same_bits(kernels.decode_to_bf16(c.buffers(), T), x[:, :T])


@pytest.mark.parametrize("width,offset", [(128, 0), (130, 0), (136, 2)])
def test_encoder_row_alignment(width, offset):
    """Source rows inside wider rows: 16-byte aligned rows (width 128) take the wide raw-row
    copy, 4-byte aligned ones (row pitch 130, or a 2-element offset) the narrow one; the
    bytes equal the oracle's either way."""
    x = synthetic.stress_pages(2, 64, 4, seed=21)
    big = torch.zeros(2, 64, 4, width + offset, dtype=torch.bfloat16)
    big[..., offset:offset + 128] = x
    src = big.to(DEV)[..., offset:offset + 128]
    _say("aligned encode", width, offset, src.stride())
    ref = ocodec.encode(u16(x))
    c = exactkv.CompressedKV(2, 64, 4, 128, reserve=1.0)
    st = (src.stride(0), 16 * src.stride(1), src.stride(1), src.stride(2))
    kernels.encode_pages(src, st, c._buf(), 0, 0, 2, 4)
    assert ref["raw"].shape[0] > 0
    _compare(c, ref, f"width {width} offset {offset}")


def _popc16(t):
    t = t.to(torch.int32)
    return sum((t >> i) & 1 for i in range(16))


@pytest.mark.parametrize("chained", [True, False])
@pytest.mark.parametrize("B,T,H", [(8, 8192, 16), (5, 8192, 32)])
def test_encoder_slot_scan_full_size(B, T, H, chained):
    """65,536 and 81,920 units, 5% outlier rows, counter starting at 7, through the
    chained scan (look-back over 64 and 80 blocks) and the three-launch scan:
    every rowoff is 7 + the raw rows of the units before it in (sequence, page, head)
    order, the counter ends at 7 + all of them, and decoding gives back every bit."""
    x = synthetic.make_kv(B, T, H, kind="k", seed=31, raw_row_rate=0.05, device=DEV)
    _say("slot scan", B, T, H, "units", B * (T // 16) * H, "chained", chained)
    c = exactkv.CompressedKV(B, T, H, 128, reserve=0.08)
    c.cnt.fill_(7)
    st = (x.stride(0), 16 * x.stride(1), x.stride(1), x.stride(2))
    kernels.encode_pages(x, st, c._buf(), 0, 0, B, T // 16, chained=chained)
    per = _popc16(c.rowmask).flatten().to(torch.int64)
    n = int(per.sum().item())
    assert n > 0.04 * B * T * H
    assert int(c.cnt.item()) == 7 + n and int(c._before.item()) == 7 and 7 + n <= c.cap
    want = 7 + torch.cumsum(per, 0) - per
    assert torch.equal(c.rowoff.flatten().to(torch.int64), want)
    assert same_bits(kernels.decode_to_bf16(c.buffers(), T), x)


def test_encoder_chained_equals_multi_launch():
    """Encodes of different sizes one after another on one stream (the chained scan's
    workspace is shared: its generation advances between calls), each byte-identical to
    the three-launch scan on the same input and counter, including a raw pool too small for
    every raw row (slots past cap skipped, counter past cap), head dims 64 and 256, a unit
    with every row raw, and source rows 4-byte but not 16-byte aligned (the raw-row copy's
    word path)."""
    cases = [(2, 64, 8, 0.05, 0.5, 128), (4, 4096, 8, 0.02, 0.5, 128), (1, 32, 2, 0.3, 0.5, 128),
             (3, 1024, 16, 0.05, 0.002, 128), (2, 512, 8, 0.05, 0.5, 128), (4, 2048, 8, 0.05, 0.5, 64),
             (2, 1024, 4, 0.05, 0.5, 256), (64, 512, 8, 0.01, 0.5, 128)]
    for i, (B, T, H, rate, reserve, D) in enumerate(cases):
        x = synthetic.make_kv(B, T, H, D=D, kind="k", seed=40 + i, raw_row_rate=rate, device=DEV)
        if i == 2:
            x[0, 16:32, 1] *= 2.0 ** 100                   # a floor >= 128 in every channel: all 16 rows raw
        if i == 4:                                         # rows 4-byte aligned but not 16
            xx = torch.empty(B, T, H, D + 2, dtype=x.dtype, device=DEV)
            xx[..., 2:] = x
            x = xx[..., 2:]
        st = (x.stride(0), 16 * x.stride(1), x.stride(1), x.stride(2))
        out = []
        for chained in (True, False):
            c = exactkv.CompressedKV(B, T, H, D, reserve=reserve)
            c.cnt.fill_(3)
            kernels.encode_pages(x, st, c._buf(), 0, 0, B, T // 16, chained=chained)
            out.append(c)
        a, b = out
        _say("chained vs three-launch scan", B, T, H, D, "counter", int(a.cnt.item()), "cap", a.cap)
        for f in ("sm", "code", "base", "rowmask", "rowoff", "cnt", "_before"):
            assert torch.equal(getattr(a, f), getattr(b, f)), f
        n = min(int(a.cnt.item()), a.cap)
        assert torch.equal(a.raw[:n], b.raw[:n])
        if i == 2:
            assert int(b.rowmask[0, 1, 1].item()) == 0xFFFF
            assert same_bits(kernels.decode_to_bf16(b.buffers(), T), x)
