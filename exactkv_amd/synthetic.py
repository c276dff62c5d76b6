"""Synthetic K/V/q generators for the benchmark configurations (seeded, any device).

Keys follow the recipe of the benchmark configurations: a per-(head, channel) scale
exp(N(0, sigma)), values N(0, 1) * scale, rotary embedding (half-split convention,
theta) applied in fp32 at the token's position, then rounded to bf16 (round to
nearest even). A fraction of entries is forced to exact 0 (zeros that appear after
RoPE in real models) and a fraction of (token, head) rows gets one element scaled by
2^-20, which makes that row not fit its group's 16-step exponent window, so it is
stored raw. Values use the same recipe without rotary embedding.

Nothing here touches the HIP library; it works on CPU tensors as well.
"""
import torch


def rope_fp32(x, pos0, theta):
    """Rotary embedding on fp32 x [B, T, H, D] at positions pos0 + t (half-split form)."""
    B, T, H, D = x.shape
    half = D // 2
    inv = theta ** (-torch.arange(0, half, device=x.device, dtype=torch.float32) * 2.0 / D)
    pos = torch.arange(pos0, pos0 + T, device=x.device, dtype=torch.float32)
    ang = pos[:, None] * inv[None, :]                                     # [T, half]
    cos = torch.cos(ang)[None, :, None, :]
    sin = torch.sin(ang)[None, :, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def make_kv(B, T, H, D=128, kind="k", seed=0, device="cpu", scale_sigma=None, theta=1e6,
            zero_rate=4e-4, raw_row_rate=3e-3, chunk_tokens=4096):
    """Synthetic keys (kind='k', with RoPE) or values (kind='v') as bf16 [B, T, H, D].

    Generated in token chunks so that large caches do not need a full fp32 copy."""
    if scale_sigma is None:
        scale_sigma = 1.5 if kind == "k" else 0.5
    g = torch.Generator(device=device).manual_seed(seed)
    scale = torch.exp(torch.randn(H, D, generator=g, device=device) * scale_sigma)
    out = torch.empty(B, T, H, D, dtype=torch.bfloat16, device=device)
    for b in range(B):
        for t0 in range(0, T, chunk_tokens):
            n = min(chunk_tokens, T - t0)
            x = torch.randn(1, n, H, D, generator=g, device=device) * scale
            if kind == "k":
                x = rope_fp32(x, t0, theta)
            xb = x.to(torch.bfloat16)
            if zero_rate > 0:
                xb[torch.rand(1, n, H, D, generator=g, device=device) < zero_rate] = 0.0
            if raw_row_rate > 0:
                rows = torch.rand(1, n, H, generator=g, device=device) < raw_row_rate
                ch = torch.randint(0, D, (1, n, H), generator=g, device=device)
                sel = torch.zeros(1, n, H, D, dtype=torch.bool, device=device)
                sel.scatter_(3, ch[..., None], rows[..., None])
                xb = torch.where(sel, xb * (2.0 ** -20), xb)
            out[b, t0:t0 + n] = xb[0]
    return out


def make_q(B, Hq, D=128, seed=0, device="cpu"):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(B, Hq, D, generator=g, device=device).to(torch.bfloat16)


def all_bf16_patterns(order="identity", seed=0, shape=(4, 128, 1, 128)):
    """All 65,536 bf16 bit patterns as a bf16 tensor of `shape` (CPU)."""
    v = torch.arange(65536, dtype=torch.int32)
    if order == "perm":
        g = torch.Generator().manual_seed(seed)
        v = v[torch.randperm(65536, generator=g)]
    return v.to(torch.int16).view(torch.bfloat16).reshape(shape)


def stress_pages(B, T, H, D=128, seed=0):
    """bf16 pages whose per-group exponents are drawn to hit every encoder branch:
    tops near 0, near the 127/128 window-floor limit, and inf/nan territory; spreads
    of 0-20 steps below the top; exact zeros, subnormals and -0.0 (CPU)."""
    g = torch.Generator().manual_seed(seed)
    NP = T // 16
    tops = torch.tensor([1, 5, 14, 15, 16, 17, 20, 100, 120, 127, 130, 141, 142, 143, 144, 150, 200, 254, 255])
    top = tops[torch.randint(0, len(tops), (B, NP, H, D), generator=g)]
    spread = torch.randint(0, 21, (B, NP, H, D), generator=g)
    lo = (top - spread).clamp(min=0)
    r = torch.rand(B, NP, 16, H, D, generator=g)
    e = (lo[:, :, None] + (r * (top - lo + 1)[:, :, None]).floor().long()).clamp(max=255)
    # make sure the top is reached inside each group
    e[:, :, 0] = top
    zero = torch.rand(B, NP, 16, H, D, generator=g) < 0.03
    e = torch.where(zero, torch.zeros_like(e), e)
    mant = torch.randint(0, 128, (B, NP, 16, H, D), generator=g)
    # exact zeros keep mantissa 0 half of the time, the rest are subnormals
    mant = torch.where(zero & (torch.rand(B, NP, 16, H, D, generator=g) < 0.5), torch.zeros_like(mant), mant)
    sign = torch.randint(0, 2, (B, NP, 16, H, D), generator=g)
    bits = (sign << 15) | (e << 7) | mant
    return bits.reshape(B, T, H, D).to(torch.int32).to(torch.int16).view(torch.bfloat16)
