"""CPU checks that pin the wire-form oracle (oracle/wire.py) and the library's layout.

No counterpart in the reference (a byte form of buffers(), cache.py:121-123, is this
build's own); the fields inside are the reference format's (codec.py:1-25)."""
import numpy as np
import pytest

from exactkv_amd import _lib
from oracle import codec, wire
from tests.conftest import u16
from exactkv_amd import synthetic


def _patterns(T, H):
    x = np.random.default_rng(11).permutation(65536).astype(np.uint16).reshape(-1, H, 128)
    return x[:T]


@pytest.mark.parametrize("T,H", [(512, 1), (509, 1), (256, 2), (250, 2), (5, 2), (0, 4)])
def test_roundtrip_all_patterns(T, H):
    x = _patterns(T, H)
    blob = wire.pack(x)
    assert np.array_equal(wire.unpack(blob), x)


def test_header_closed_forms():
    x = _patterns(37, 2)
    blob = wire.pack(x)
    h = wire.header(blob)
    assert (h["magic"], h["version"], h["heads"], h["head_dim"], h["tokens"]) == (0x564B5845, 1, 2, 128, 37)
    assert (h["full_pages"], h["tail_rows"]) == (2, 5)
    assert bytes(blob[:4]) == b"EXKV"
    # sections in order, each at a multiple of 256, sized by the format
    assert h["off_tail"] == 256
    assert h["off_rowmask"] == 256 + 5 * 2 * 256
    assert h["off_base"] == h["off_rowmask"] + 256                       # 2 pages x 2 heads x 4 B -> 256
    assert h["off_sm"] == h["off_base"] + 512                            # 2 x 2 x 128 B
    assert h["off_code"] == h["off_sm"] + 2 * 16 * 2 * 128
    assert h["off_raw"] == h["off_code"] + 2 * 16 * 2 * 64
    assert h["total"] == h["off_raw"] + h["raw_rows"] * 256 == blob.size
    assert not blob[88:256].any()                                        # header tail zero
    assert not blob[h["off_rowmask"] + 16:h["off_base"]].any()           # alignment gap zero


def test_all_zero_sequence():
    x = np.zeros((40, 4, 128), np.uint16)
    blob = wire.pack(x)
    h = wire.header(blob)
    assert h["raw_rows"] == 0 and h["total"] == wire.layout(4, 40, 0)["total"]
    assert not blob[256:].any()                                          # every field of zeros is zero


def test_raw_rows_are_exactly_the_rows_the_codes_cannot_hold():
    """Independent of the encoder's escape rule: a row is in the raw section iff decoding
    it from its own sm / code / base bytes does not give it back, in (page, head, token)
    order."""
    T, H = 96, 3
    x = u16(synthetic.make_kv(1, T, H, kind="k", seed=5, raw_row_rate=0.05))[0]
    blob = wire.pack(x)
    h = wire.header(blob)
    npf = T // 16

    def sec(off, dt, shape):
        return blob[off:off + int(np.prod(shape)) * np.dtype(dt).itemsize].view(dt).reshape(shape)

    sm = sec(h["off_sm"], np.uint8, (T, H, 128))
    cb = sec(h["off_code"], np.uint8, (T, H, 64)).astype(np.int32)
    base = sec(h["off_base"], np.uint8, (npf, H, 128))
    nib = np.concatenate([cb & 15, cb >> 4], axis=-1)
    dec = codec.decode_values(sm, nib, np.repeat(base, 16, axis=0))
    want = [x[p * 16 + r, hh] for p in range(npf) for hh in range(H) for r in range(16)
            if not np.array_equal(dec[p * 16 + r, hh], x[p * 16 + r, hh])]
    raw = sec(h["off_raw"], "<u2", (h["raw_rows"], 128))
    assert len(want) == h["raw_rows"] > 0
    assert np.array_equal(raw, np.array(want))
    rm = sec(h["off_rowmask"], "<i4", (npf, H))
    assert sum(bin(int(v)).count("1") for v in rm.reshape(-1)) == h["raw_rows"]


def test_library_layout_matches_oracle():
    lib = _lib.load()
    for H in (1, 2, 4, 8, 28, 32):
        for T in (0, 1, 15, 16, 17, 37, 1000, 4096, 131072):
            for N in (0, 1, 77):
                assert lib.exkv_wire_bytes(H, T, N) == wire.layout(H, T, N)["total"], (H, T, N)
    assert lib.exkv_wire_bytes(0, 16, 0) == -1 and lib.exkv_wire_bytes(2, -1, 0) == -1
