"""The CPU baseline of the decode path in PyTorch (test and benchmark infrastructure only).

The same restatement of the reference codec as oracle.codec (reference exactkv/codec.py:
encode_reference :31-55, decode_reference :58-73), written with torch tensor ops so that
it runs on all host cores, plus fp32 GQA decode attention with softmax scale 1/sqrt(128)
(the reference test's attention, tests/test_exactkv.py:75-77, in float32). bench.py times
it on the GPU box's host cores as the CPU baseline; tests/ pin it byte for byte against the
reference-written golden vectors and the numpy oracle. Nothing in exactkv_amd imports it.

Tensors are CPU torch tensors: bf16 inputs, and the six format fields with the dtypes of
the reference (sm, code, base uint8; rowmask, rowoff int32; raw bf16 rows).
"""
import torch

P = 16


def _fields(x):
    """bf16 [...] -> (exponent int32, sign|mantissa uint8)."""
    u = x.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    e = (u >> 7) & 0xFF
    sm = (((u >> 8) & 0x80) | (u & 0x7F)).to(torch.uint8)
    return e, sm


def encode(x):
    """x: bf16 [B, T, H, D] (T % 16 == 0) -> dict of the six format tensors + shape."""
    B, T, H, D = x.shape
    assert T % P == 0 and x.dtype == torch.bfloat16
    NP = T // P
    e, sm = _fields(x)
    eg = e.view(B, NP, P, H, D)                                       # token axis 2
    floor = (eg.amax(dim=2) - 15).clamp_min(0)                        # [B, NP, H, D]
    zero = eg == 0
    zflag = zero.any(dim=2) & (floor > 0)
    f, z = floor[:, :, None], zflag[:, :, None]
    code = torch.where(z & zero, torch.zeros_like(eg), eg - f)
    need = (z & ~zero).to(torch.int32)                                # a non-zero in a flagged group needs code >= 1
    fits = (code >= need) & (f < 128)
    nib = code.clamp(0, 15).view(B, T, H, D)
    packed = (nib[..., : D // 2] | (nib[..., D // 2:] << 4)).to(torch.uint8)
    base = (floor + 128 * zflag.to(torch.int32)).clamp_max(255).to(torch.uint8)
    raw_row = ~fits.all(dim=-1)                                       # [B, NP, P, H]
    weights = (1 << torch.arange(P, dtype=torch.int32)).view(1, 1, P, 1)
    rowmask = (raw_row.to(torch.int32) * weights).sum(dim=2, dtype=torch.int32)   # [B, NP, H]
    per_page = raw_row.sum(dim=2).reshape(-1)
    rowoff = (torch.cumsum(per_page, 0) - per_page).to(torch.int32).view(B, NP, H)
    order = raw_row.permute(0, 1, 3, 2)                               # (b, page, head, token) order
    rows = x.view(B, NP, P, H, D).permute(0, 1, 3, 2, 4)
    raw = rows[order].reshape(-1, D).clone()
    return dict(shape=(B, T, H, D), sm=sm, code=packed, base=base, rowmask=rowmask, rowoff=rowoff, raw=raw)


def decode(c, T=None):
    """Inverse of encode: bf16 [B, T, H, D] (T defaults to the buffer length)."""
    B, TS, H, D = c["shape"]
    T = TS if T is None else T
    NP = TS // P
    cb = c["code"].to(torch.int32)
    nib = torch.cat([cb & 15, cb >> 4], dim=-1)
    base = c["base"].to(torch.int32).repeat_interleave(P, dim=1)
    e = (base & 127) + nib
    e = torch.where((base >= 128) & (nib == 0), torch.zeros_like(e), e)
    s = c["sm"].to(torch.int32)
    bits = ((s & 0x80) << 8) | (e << 7) | (s & 0x7F)
    out = bits.to(torch.int16).view(torch.bfloat16)                   # [B, TS, H, D]
    rm = c["rowmask"].to(torch.int32)
    is_raw = ((rm[..., None] >> torch.arange(P, dtype=torch.int32)) & 1).bool()   # [B, NP, H, P]
    if bool(is_raw.any()):
        below = torch.cumsum(is_raw.to(torch.int64), dim=-1) - is_raw.to(torch.int64)
        slot = c["rowoff"].to(torch.int64)[..., None] + below
        rows = out.view(B, NP, P, H, D).permute(0, 1, 3, 2, 4)
        rows[is_raw] = c["raw"][slot[is_raw]]
    return out[:, :T]


def attention(q, k, v, T, lens=None):
    """fp32 GQA decode attention: q bf16 [B, Hq, D], k / v bf16 [B, >=T, Hkv, D] -> float32
    [B, Hq, D] over the first T tokens (or lens[b] of sequence b)."""
    B, Hq, D = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    out = torch.empty(B, Hq, D, dtype=torch.float32)
    for b in range(B):
        n = T if lens is None else int(lens[b])
        qs = q[b].float().view(Hkv, G, D)
        ks = k[b, :n].float().permute(1, 2, 0)                        # [Hkv, D, n]
        vs = v[b, :n].float().transpose(0, 1)                         # [Hkv, n, D]
        w = torch.softmax(torch.bmm(qs, ks) * D ** -0.5, dim=-1)      # [Hkv, G, n]
        out[b] = torch.bmm(w, vs).reshape(Hq, D)
    return out


def decode_attention(q, kc, vc, T, lens=None):
    """The CPU path end to end: decode both caches, then fp32 attention."""
    return attention(q, decode(kc, T), decode(vc, T), T, lens)
