"""The exactkv byte format's whole-tensor codec (drop-in for the reference's
exactkv/codec.py: encode_reference :31-55, decode_reference :58-73, bits_per_value
:76-78, P :28), computed by the HIP encoder and decoder.

Format, per (sequence, 16-token page, KV head, channel) group:

  sm      uint8 [B, T, H, D]      sign and mantissa, unchanged
  code    uint8 [B, T, H, D/2]    4-bit exponent offsets; one byte holds channels j and j + D/2
  base    uint8 [B, T/16, H, D]   < 128: exponent = base + code (a 16-step window)
                                  >= 128: group with zeros: code 0 means exponent 0,
                                  otherwise exponent = base - 128 + code (15 steps)
  rowmask int32 [B, T/16, H]      bit p set: token p of the page is stored raw
  rowoff  int32 [B, T/16, H]      index of the page's first raw row in `raw`
  raw     bf16  [N_raw, D]        rows that contain a value more than 2^15 below the
                                  group maximum (or an exponent window that starts at 128+)

encode_reference returns exactly the reference codec's bytes (raw rows in
(sequence, page, head, token) order). Tensors on the CPU are moved to the current GPU
for the computation and the results are returned on the input's device; there is no
CPU implementation in this package.
"""
import torch

from .kernels import encode_pages, decode_to_bf16, HEAD_DIMS, P


def _gpu(dev):
    if dev.type == "cuda":
        return dev
    if not torch.cuda.is_available():
        raise RuntimeError("exactkv codec runs on the GPU (HIP); no GPU is available")
    return torch.device("cuda", torch.cuda.current_device())


def encode_reference(x):
    """x: [B, T, H, D] bf16, T a multiple of 16, D in HEAD_DIMS. Returns a dict of tensors
    (raw rows in page order)."""
    B, T, H, D = x.shape
    assert T % P == 0 and x.dtype == torch.bfloat16
    if D not in HEAD_DIMS:
        raise ValueError(f"head dim {D}: the GPU codec is built for {HEAD_DIMS}")
    dev = _gpu(x.device)
    xd = x.to(dev).contiguous()
    NP = T // P
    u8 = dict(dtype=torch.uint8, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    buf = dict(sm=torch.empty(B, T, H, D, **u8), code=torch.empty(B, T, H, D // 2, **u8),
               base=torch.empty(B, NP, H, D, **u8), rowmask=torch.empty(B, NP, H, **i32),
               rowoff=torch.empty(B, NP, H, **i32), cnt=torch.zeros(1, **i32), cap=0, TS=T, H=H, D=D,
               raw=torch.empty(1, D, dtype=torch.bfloat16, device=dev))
    st = (xd.stride(0), P * xd.stride(1), xd.stride(1), xd.stride(2))
    encode_pages(xd, st, buf, 0, 0, B, NP)                 # pass 1: layout and raw-row count
    n = int(buf["cnt"].item())
    if n:
        buf["raw"] = torch.empty(n, D, dtype=torch.bfloat16, device=dev)
        buf["cap"] = n
        buf["cnt"].zero_()
        encode_pages(xd, st, buf, 0, 0, B, NP)             # pass 2: same bytes, raw rows stored
    raw = buf["raw"][:n]
    out = dict(shape=(B, T, H, D), sm=buf["sm"], code=buf["code"], base=buf["base"], rowmask=buf["rowmask"],
               rowoff=buf["rowoff"], raw=raw)
    if x.device != dev:
        out = {k: (v.to(x.device) if isinstance(v, torch.Tensor) else v) for k, v in out.items()}
    return out


def decode_reference(c):
    """Inverse of encode_reference (raw rows located through rowmask/rowoff)."""
    B, T, H, D = c["shape"]
    src = c["sm"].device
    dev = _gpu(src)
    g = {k: (v.to(dev).contiguous() if isinstance(v, torch.Tensor) else v) for k, v in c.items()}
    if g["raw"].shape[0] == 0:
        g["raw"] = torch.zeros(1, D, dtype=torch.bfloat16, device=dev)
    out = decode_to_bf16(g, T)
    return out.to(src) if src != dev else out


_STORED = ("sm", "code", "base", "rowmask", "rowoff", "raw")


def bits_per_value(c):
    """Storage cost of an encoded tensor (reference codec.py:76-78): every allocated byte of
    the six arrays, raw pool included, in bits per value of the [B, T, H, D] input. With N
    raw rows that is 8 * (1.5 D + D/16 + 8/16 + 2 D N / (B T H)) / D = 12.5 + 4 / D +
    16 N / (B T H) (12.53125 + 16 N / (B T H) for D = 128)."""
    values = 1
    for n in c["sm"].shape:
        values *= n
    total = 0
    for name in _STORED:
        t = c[name]
        total += t.numel() * t.element_size()
    return 8.0 * total / values
