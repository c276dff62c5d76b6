"""Synthetic K/V/q generators for the benchmark configurations (seeded, reproducible).

Keys follow the recipe of the benchmark configurations: a per-(head, channel) scale
exp(N(0, sigma)), values N(0, 1) * scale, rotary embedding (half-split convention,
theta) applied in fp32 at the token's position, then rounded to bf16 (round to
nearest even). A fraction of entries is forced to exact 0 (zeros that appear after
RoPE in real models) and a fraction of (token, head) rows gets one element scaled by
2^-20, which makes that row not fit its group's 16-step exponent window, so it is
stored raw. Values use the same recipe without rotary embedding.

Everything is generated on the host with numpy's PCG64 stream, IEEE fp32 arithmetic
and scalar libm calls for the few transcendentals (exp of the scales, the rotary
cos/sin table), so the same seed gives the same bits on any machine; the result is
then moved to the requested device. Nothing here touches the HIP library.
"""
import math

import numpy as np
import torch


def _bf16_bits(f32):
    """float32 array -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f32)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def _to_torch(bits, device):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(device)


def rope_tables(pos0, n, D, theta):
    """fp32 cos/sin [n, D/2] of angle (pos0 + t) * theta^(-2i/D), from scalar libm calls."""
    half = D // 2
    inv = [math.pow(theta, -2.0 * i / D) for i in range(half)]
    ang = [(pos0 + t) * f for t in range(n) for f in inv]
    cos = np.fromiter((math.cos(a) for a in ang), np.float64, len(ang)).astype(np.float32).reshape(n, half)
    sin = np.fromiter((math.sin(a) for a in ang), np.float64, len(ang)).astype(np.float32).reshape(n, half)
    return cos, sin


def make_kv(B, T, H, D=128, kind="k", seed=0, device="cpu", scale_sigma=None, theta=1e6,
            zero_rate=4e-4, raw_row_rate=3e-3, chunk_tokens=4096):
    """Synthetic keys (kind='k', with RoPE) or values (kind='v') as bf16 [B, T, H, D]."""
    if scale_sigma is None:
        scale_sigma = 1.5 if kind == "k" else 0.5
    rng = np.random.Generator(np.random.PCG64(seed))
    z = rng.standard_normal(H * D) * scale_sigma
    scale = np.array([math.exp(s) for s in z.tolist()], np.float32).reshape(H, D)
    out = np.empty((B, T, H, D), np.uint16)
    tables = {}
    for b in range(B):
        for t0 in range(0, T, chunk_tokens):
            n = min(chunk_tokens, T - t0)
            x = rng.standard_normal((n, H, D), dtype=np.float32) * scale
            if kind == "k":
                if t0 not in tables:
                    tables[t0] = rope_tables(t0, n, D, theta)
                cos, sin = tables[t0]
                c, s = cos[:, None, :], sin[:, None, :]
                x1, x2 = x[..., : D // 2], x[..., D // 2:]
                x = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
            bits = _bf16_bits(x)
            if zero_rate > 0:
                bits[rng.random((n, H, D)) < zero_rate] = 0
            if raw_row_rate > 0:
                rows = rng.random((n, H)) < raw_row_rate
                ch = rng.integers(0, D, (n, H))
                ti, hi = np.nonzero(rows)
                ci = ch[ti, hi]
                vals = (bits[ti, hi, ci].astype(np.uint32) << 16).view(np.float32) * np.float32(2.0 ** -20)
                bits[ti, hi, ci] = _bf16_bits(vals)
            out[b, t0:t0 + n] = bits
    return _to_torch(out, device)


def make_q(B, Hq, D=128, seed=0, device="cpu"):
    rng = np.random.Generator(np.random.PCG64(seed))
    return _to_torch(_bf16_bits(rng.standard_normal((B, Hq, D), dtype=np.float32)), device)


def all_bf16_patterns(order="identity", seed=0, shape=(4, 128, 1, 128)):
    """All 65,536 bf16 bit patterns as a bf16 tensor of `shape` (CPU)."""
    v = np.arange(65536, dtype=np.uint16)
    if order == "perm":
        v = np.random.Generator(np.random.PCG64(seed)).permutation(v)
    return _to_torch(v.reshape(shape), "cpu")


def stress_pages(B, T, H, D=128, seed=0):
    """bf16 pages whose per-group exponents are drawn to hit every encoder branch:
    tops near 0, near the 127/128 window-floor limit, and inf/nan territory; spreads
    of 0-20 steps below the top; exact zeros, subnormals and -0.0 (CPU)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    NP = T // 16
    tops = np.array([1, 5, 14, 15, 16, 17, 20, 100, 120, 127, 130, 141, 142, 143, 144, 150, 200, 254, 255])
    top = tops[rng.integers(0, len(tops), (B, NP, H, D))]
    lo = np.maximum(top - rng.integers(0, 21, (B, NP, H, D)), 0)
    r = rng.random((B, NP, 16, H, D))
    e = np.minimum(lo[:, :, None] + np.floor(r * (top - lo + 1)[:, :, None]).astype(np.int64), 255)
    e[:, :, 0] = top                                   # the top is reached in every group
    zero = rng.random((B, NP, 16, H, D)) < 0.03
    e = np.where(zero, 0, e)
    mant = rng.integers(0, 128, (B, NP, 16, H, D))
    # exact zeros keep mantissa 0 half of the time, the rest are subnormals
    mant = np.where(zero & (rng.random((B, NP, 16, H, D)) < 0.5), 0, mant)
    sign = rng.integers(0, 2, (B, NP, 16, H, D))
    bits = ((sign << 15) | (e << 7) | mant).astype(np.uint16)
    return _to_torch(bits.reshape(B, T, H, D), "cpu")
