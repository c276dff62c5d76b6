"""CPU restatement of the exactkv wire form of one sequence's cache (test infrastructure
only: the product packs and unpacks on the GPU, exactkv_amd/csrc/wire.hip).

No counterpart in the reference: a byte form of buffers() for KV offload and transfer
is in its future work (cache.py:121-123 holds the buffers; codec.py:10-18 the format).
The sections hold the reference format's own fields for one sequence:

  header   256 B, little-endian: u32 magic 0x564B5845 ("EXKV"), version 1, heads H,
           head_dim 128, tokens T, full_pages T // 16, tail_rows T % 16, raw_rows N;
           then u64 off_tail, off_rowmask, off_base, off_sm, off_code, off_raw, total
  tail     bf16 [T % 16, H, 128]      the open page's tokens
  rowmask  i32  [T // 16, H]
  base     u8   [T // 16, H, 128]
  sm       u8   [16 * (T // 16), H, 128]
  code     u8   [16 * (T // 16), H, 64]
  raw      bf16 [N, 128]              raw rows in (page, head, token) order

Every section starts at a multiple of 256 bytes; the gaps are zero. rowoff is not
stored: it is the exclusive running count of raw rows in (page, head) order.
"""
import numpy as np

from oracle import codec

P = 16
MAGIC = 0x564B5845
VERSION = 1
HEADER = 256
D = 128


def _al(n):
    return (n + 255) // 256 * 256


def layout(H, T, N):
    """Section offsets and total size for H heads, T tokens and N raw rows."""
    npf, tail = T // P, T % P
    off_tail = HEADER
    off_rowmask = off_tail + _al(tail * H * D * 2)
    off_base = off_rowmask + _al(npf * H * 4)
    off_sm = off_base + _al(npf * H * D)
    off_code = off_sm + _al(npf * P * H * D)
    off_raw = off_code + _al(npf * P * H * D // 2)
    total = off_raw + N * D * 2
    return dict(off_tail=off_tail, off_rowmask=off_rowmask, off_base=off_base, off_sm=off_sm, off_code=off_code,
                off_raw=off_raw, total=total)


def header(blob):
    """The header fields of a blob (bytes or uint8 array)."""
    b = np.frombuffer(bytes(np.asarray(blob, dtype=np.uint8)[:HEADER]), dtype=np.uint8)
    u32 = b[:32].view("<u4")
    u64 = b[32:88].view("<u8")
    keys = ("off_tail", "off_rowmask", "off_base", "off_sm", "off_code", "off_raw", "total")
    h = dict(magic=int(u32[0]), version=int(u32[1]), heads=int(u32[2]), head_dim=int(u32[3]), tokens=int(u32[4]),
             full_pages=int(u32[5]), tail_rows=int(u32[6]), raw_rows=int(u32[7]))
    h.update({k: int(v) for k, v in zip(keys, u64)})
    return h


def pack(x):
    """x: uint16 bf16 bits [T, H, 128] of one sequence -> the blob as a uint8 array."""
    T, H, Dx = x.shape
    assert Dx == D and x.dtype == np.uint16
    npf = T // P
    Tf = npf * P
    if npf:
        c = codec.encode(x[None, :Tf])
        raw = c["raw"]
    else:
        c = None
        raw = np.zeros((0, D), np.uint16)
    N = raw.shape[0]
    lay = layout(H, T, N)
    out = np.zeros(lay["total"], np.uint8)
    hdr = np.zeros(HEADER, np.uint8)
    hdr[:32] = np.array([MAGIC, VERSION, H, D, T, npf, T - Tf, N], "<u4").view(np.uint8)
    hdr[32:88] = np.array([lay[k] for k in ("off_tail", "off_rowmask", "off_base", "off_sm", "off_code", "off_raw",
                                            "total")], "<u8").view(np.uint8)
    out[:HEADER] = hdr

    def put(off, a):
        a = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        out[off:off + a.size] = a

    put(lay["off_tail"], x[Tf:].astype("<u2"))
    if npf:
        put(lay["off_rowmask"], c["rowmask"][0].astype("<i4"))
        put(lay["off_base"], c["base"][0])
        put(lay["off_sm"], c["sm"][0])
        put(lay["off_code"], c["code"][0])
        put(lay["off_raw"], raw.astype("<u2"))
    return out


def unpack(blob):
    """The blob -> uint16 bf16 bits [T, H, 128], through the format decoder."""
    blob = np.asarray(blob, dtype=np.uint8)
    h = header(blob)
    assert h["magic"] == MAGIC and h["version"] == VERSION and h["head_dim"] == D
    H, T, npf, tail, N = h["heads"], h["tokens"], h["full_pages"], h["tail_rows"], h["raw_rows"]
    assert h == {**h, **layout(H, T, N)} and npf == T // P and tail == T % P

    def get(off, dtype, shape):
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return blob[off:off + n].view(dtype).reshape(shape)

    out = np.zeros((T, H, D), np.uint16)
    out[npf * P:] = get(h["off_tail"], "<u2", (tail, H, D))
    if npf:
        rowmask = get(h["off_rowmask"], "<i4", (1, npf, H)).astype(np.int32)
        n = np.bitwise_count(rowmask.astype(np.int64)).reshape(-1)
        rowoff = (np.cumsum(n) - n).astype(np.int32).reshape(1, npf, H)
        c = dict(shape=(1, npf * P, H, D), sm=get(h["off_sm"], np.uint8, (1, npf * P, H, D)),
                 code=get(h["off_code"], np.uint8, (1, npf * P, H, D // 2)),
                 base=get(h["off_base"], np.uint8, (1, npf, H, D)), rowmask=rowmask, rowoff=rowoff,
                 raw=get(h["off_raw"], "<u2", (N, D)).astype(np.uint16))
        out[:npf * P] = codec.decode(c)[0]
    return out
