"""CPU restatement of the exactkv byte format (test infrastructure only).

Follows reference exactkv/codec.py: format spec :1-25, P = 16 :28,
encode_reference :31-55, decode_reference :58-73, bits_per_value :76-78.

Values are bf16 bit patterns held as numpy uint16 arrays of shape [B, T, H, D].
For every group (sequence b, page of 16 tokens, head h, channel d) with exponents
e[0..15]:

  floor = max(max(e) - 15, 0)                    the 16-step exponent window
  zflag = any(e == 0) and floor > 0              zeros the window cannot hold
  code  = 0 for (zflag and e == 0), else e - floor
  fits  = floor < 128 and (code >= 1 if zflag and e != 0 else code >= 0)
  nibble = clamp(code, 0, 15)                    also for elements that do not fit
  base  = min(floor + 128 * zflag, 255)

A (token, head) row is stored raw if any element of it does not fit. Raw rows are
numbered in (b, page, head, token) order; rowoff is the exclusive running count.
"""
import numpy as np

P = 16


def split_fields(u):
    """bf16 bits -> (exponent int32, sign|mantissa byte uint8)."""
    u = u.astype(np.int32)
    e = (u >> 7) & 0xFF
    sm = (((u >> 8) & 0x80) | (u & 0x7F)).astype(np.uint8)
    return e, sm


def group_codes(e):
    """Per-group encoder decision. e: int array [..., 16 tokens (axis -2), C channels].

    Returns (floor, zflag, code, fits) where floor/zflag have the token axis removed
    and code/fits have e's shape. The code is the unclamped offset."""
    top = e.max(axis=-2)
    floor = np.maximum(top - 15, 0)
    is_zero = e == 0
    zflag = is_zero.any(axis=-2) & (floor > 0)
    f = floor[..., None, :]
    z = zflag[..., None, :]
    code = np.where(z & is_zero, 0, e - f)
    need = np.where(z & ~is_zero, 1, 0)          # smallest code a non-zero may take
    fits = (code >= need) & (f < 128)
    return floor, zflag, code, fits


def encode(x):
    """x: uint16 [B, T, H, D], T % 16 == 0. Returns the six format tensors as a dict
    (numpy arrays: sm u8, code u8, base u8, rowmask i32, rowoff i32, raw u16 [N, D])."""
    B, T, H, D = x.shape
    assert T % P == 0 and D % 2 == 0 and x.dtype == np.uint16
    NP = T // P
    e, sm = split_fields(x)
    # group axis layout: [B, NP, H, P, D] so the token axis is -2
    eg = e.reshape(B, NP, P, H, D).transpose(0, 1, 3, 2, 4)
    floor, zflag, code, fits = group_codes(eg)
    nib = np.clip(code, 0, 15).transpose(0, 1, 3, 2, 4).reshape(B, T, H, D)
    half = D // 2
    packed = (nib[..., :half] | (nib[..., half:] << 4)).astype(np.uint8)
    base = np.minimum(floor + 128 * zflag, 255).astype(np.uint8)       # [B, NP, H, D]
    raw_row = ~fits.all(axis=-1)                                         # [B, NP, H, P]
    bits = (raw_row.astype(np.int64) << np.arange(P, dtype=np.int64)).sum(-1)
    rowmask = bits.astype(np.int32)
    n = raw_row.sum(-1).reshape(-1).astype(np.int64)
    rowoff = (np.cumsum(n) - n).astype(np.int32).reshape(B, NP, H)
    rows = x.reshape(B, NP, P, H, D).transpose(0, 1, 3, 2, 4)             # [B, NP, H, P, D]
    raw = rows[raw_row].copy()
    return dict(shape=(B, T, H, D), sm=sm, code=packed, base=base, rowmask=rowmask,
                rowoff=rowoff, raw=raw.reshape(-1, D))


def decode_values(sm, nib, base):
    """Rebuild bf16 bits from sign|mantissa bytes, 4-bit codes and the group base byte
    (all broadcastable int arrays). Reference codec.py:65-68."""
    sm = sm.astype(np.int32)
    nib = nib.astype(np.int32)
    base = base.astype(np.int32)
    e = (base & 127) + nib
    e = np.where((base >= 128) & (nib == 0), 0, e)
    return (((sm & 0x80) << 8) | ((e & 0xFF) << 7) | (sm & 0x7F)).astype(np.uint16)


def decode(c, T=None):
    """Inverse of encode (raw rows located through rowmask/rowoff). Returns uint16
    [B, T, H, D]; T defaults to the full buffer length."""
    B, TS, H, D = c["shape"]
    T = TS if T is None else T
    NP = TS // P
    half = D // 2
    cb = c["code"].astype(np.int32)
    nib = np.concatenate([cb & 15, cb >> 4], axis=-1)                      # [B, TS, H, D]
    base = np.repeat(c["base"], P, axis=1)                                 # [B, TS, H, D]
    out = decode_values(c["sm"], nib, base)
    assert half * 2 == D
    slot, is_raw = raw_slots(c["rowmask"], c["rowoff"])                   # [B, NP, H, P]
    rows = out.reshape(B, NP, P, H, D).transpose(0, 1, 3, 2, 4)           # view
    rows[is_raw] = c["raw"][slot[is_raw]]
    return out[:, :T]


def raw_slots(rowmask, rowoff):
    """Slot of every (b, page, head, token) row in the raw pool and whether it is raw:
    rowoff + number of raw rows before it in its page (reference kernels.py:119-123)."""
    rm = rowmask.astype(np.int64)[..., None]
    p = np.arange(P, dtype=np.int64)
    is_raw = ((rm >> p) & 1).astype(bool)
    before = np.bitwise_count(rm & ((1 << p) - 1)).astype(np.int64)
    return rowoff.astype(np.int64)[..., None] + before, is_raw


def bits_per_value(c):
    """Allocated bytes x 8 / number of values (reference codec.py:76-78)."""
    n = c["sm"].size
    tot = sum(np.asarray(c[k]).nbytes for k in ("sm", "code", "base", "rowmask", "rowoff", "raw"))
    return tot * 8 / n
