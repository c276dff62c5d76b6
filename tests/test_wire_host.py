"""Host side of the wire form (no GPU): the Python header reader and checks agree with the
oracle's layout, and malformed headers are rejected before anything is launched.

No counterpart in the reference (a byte form of buffers(), cache.py:121-123, is this
build's own)."""
import numpy as np
import pytest
import torch

from exactkv_amd import wire
from oracle import wire as owire


class _Cache:
    H, D = 2, 128


def _blob(T=37, H=2, seed=3):
    x = np.random.default_rng(seed).permutation(65536).astype(np.uint16)[:T * H * 128].reshape(T, H, 128)
    return torch.from_numpy(owire.pack(x))


def test_header_reader_matches_the_oracle():
    b = _blob()
    assert wire.header(b) == owire.header(b.numpy())
    assert wire._check_blob(b, _Cache)["tokens"] == 37
    assert wire.nbytes(2, 37, wire.header(b)["raw_rows"]) == b.numel()


def test_malformed_blobs_are_rejected():
    b = _blob()
    with pytest.raises(ValueError, match="1-D uint8"):
        wire.header(b[:100])
    bad = b.clone()
    bad[4] = 2                                          # version 2
    with pytest.raises(ValueError, match="not an exactkv"):
        wire._check_blob(bad, _Cache)
    bad = b.clone()
    bad[16] = 38                                        # tokens no longer match the layout
    with pytest.raises(ValueError, match="inconsistent"):
        wire._check_blob(bad, _Cache)
    with pytest.raises(ValueError, match="shorter"):
        wire._check_blob(b[:-256].clone(), _Cache)

    class Four(_Cache):
        H = 4
    with pytest.raises(ValueError, match="heads"):
        wire._check_blob(b, Four)

    bad = b.clone()
    h = wire.header(b)
    assert h["full_pages"] > 0
    rm = bad[h["off_rowmask"]: h["off_rowmask"] + 4 * h["full_pages"] * 2].view(torch.int32)
    rm[0] ^= 1 << 15                                    # one more (or one less) raw row than declared
    with pytest.raises(ValueError, match="declares"):
        wire._check_blob(bad, _Cache)
