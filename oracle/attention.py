"""CPU restatement of GQA decode attention and its split-K algebra (test infrastructure only).

Reference: exactkv/kernels.py -- online softmax block :46-59 (base-2 exponent, scores
scaled by D^-1/2 * log2 e, p rounded to bf16 before P.V), split merge :33-43, split
planner :273-277; the fp64 check of tests/test_exactkv.py:75-78.

Arrays: q [B, Hq, D], k/v [B, TS, Hkv, D] as bf16 bit patterns (uint16) or floats.
Query head h uses KV head h // G with G = Hq // Hkv (GQA grouping).
"""
import numpy as np

LOG2E = 1.4426950408889634


def bf16_to_f32(u):
    """bf16 bit patterns (uint16) -> float32."""
    return (np.asarray(u, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    """float32 -> bf16 bit patterns, round to nearest even (NaN stays NaN)."""
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(f, dtype=np.float32))
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def _float(a, dtype):
    a = np.asarray(a)
    if a.dtype == np.uint16:
        a = bf16_to_f32(a)
    return a.astype(dtype)


def lengths(B, T, lens):
    return np.full(B, T, dtype=np.int64) if lens is None else np.asarray(lens, dtype=np.int64)


def attention(q, k, v, T, dtype=np.float64, lens=None):
    """Exact softmax(q k^T / sqrt(D)) v over the first T (or lens[b]) tokens, in `dtype`.
    Returns [B, Hq, D] in dtype."""
    q, k, v = _float(q, dtype), _float(k, dtype), _float(v, dtype)
    B, Hq, D = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, D), dtype=dtype)
    for b, n in enumerate(lengths(B, T, lens)):
        for hk in range(Hkv):
            qs = q[b, hk * G:(hk + 1) * G]                                   # [G, D]
            ks, vs = k[b, :n, hk], v[b, :n, hk]                              # [n, D]
            s = (qs @ ks.T) / dtype(np.sqrt(D))
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            out[b, hk * G:(hk + 1) * G] = (p @ vs) / p.sum(axis=1, keepdims=True)
    return out


def tolerance_excess(out, ref):
    """North-star accuracy bound for a bf16 attention output against a float reference:
    per element |out - ref| <= 1e-2 |ref| + 2 bf16 ulp of the largest |ref| in the output
    row (the row's scale: bf16 rounding alone can cost half an ulp of each element).
    Returns max(|out - ref| - bound); the bound holds when it is <= 0."""
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    rowmax = np.abs(r).max(-1, keepdims=True)
    ulp = np.exp2(np.floor(np.log2(np.maximum(rowmax, 1e-30))) - 7)
    return float((np.abs(o - r) - (1e-2 * np.abs(r) + 2 * ulp)).max())


def choose_split(B, Hkv, T, BLOCK_N, target=512):
    """Reference planner (kernels.py:273-277): about `target` programs in total, split
    lengths a multiple of BLOCK_N. Returns (number of splits, split length)."""
    ns = max(1, min(-(-T // BLOCK_N), target // max(1, B * Hkv)))
    split_len = -(-(-(-T // ns)) // BLOCK_N) * BLOCK_N
    return -(-T // split_len), split_len


def split_partials(q, k, v, T, split_len, block_n=64, lens=None, round_p=True, ns=None):
    """Per-split fp32 partials (m, l, o) of the reference's online softmax, in base 2.

    Returns m [B, Hq, ns], l [B, Hq, ns], o [B, Hq, ns, D]; empty splits give
    m = -inf, l = 0, o = 0."""
    q, k, v = _float(q, np.float32), _float(k, np.float32), _float(v, np.float32)
    B, Hq, D = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    L = lengths(B, T, lens)
    if ns is None:
        ns = int(-(-int(L.max()) // split_len))
    scale = np.float32(D ** -0.5 * LOG2E)
    m = np.full((B, Hq, ns), -np.inf, np.float32)
    l = np.zeros((B, Hq, ns), np.float32)
    o = np.zeros((B, Hq, ns, D), np.float32)
    for b in range(B):
        for hk in range(Hkv):
            qs = q[b, hk * G:(hk + 1) * G]
            for s in range(ns):
                mi = np.full(G, -np.inf, np.float32)
                li = np.zeros(G, np.float32)
                acc = np.zeros((G, D), np.float32)
                end = min((s + 1) * split_len, int(L[b]))
                for n0 in range(s * split_len, end, block_n):
                    n1 = min(n0 + block_n, end)
                    sc = (qs @ k[b, n0:n1, hk].T) * scale                      # [G, n]
                    mn = np.maximum(mi, sc.max(axis=1))
                    alpha = np.exp2(mi - mn)
                    p = np.exp2(sc - mn[:, None])
                    li = li * alpha + p.sum(axis=1)
                    pb = bf16_to_f32(f32_to_bf16(p)) if round_p else p
                    acc = acc * alpha[:, None] + pb @ v[b, n0:n1, hk]
                    mi = mn
                m[b, hk * G:(hk + 1) * G, s] = mi
                l[b, hk * G:(hk + 1) * G, s] = li
                o[b, hk * G:(hk + 1) * G, s] = acc
    return m, l, o


def merge_splits(m, l, o):
    """LSE merge of split partials (kernels.py:33-43): w = 2^(m - max m),
    out = sum(o w) / sum(l w). Returns float32 [..., D]."""
    M = m.max(axis=-1, keepdims=True)
    w = np.exp2(m - M)
    w = np.where(np.isfinite(m), w, 0.0).astype(np.float32)
    num = (o * w[..., None]).sum(axis=-2)
    den = (l * w).sum(axis=-1)
    return (num / den[..., None]).astype(np.float32)


def split_attention(q, k, v, T, split_len, block_n=64, lens=None, round_p=True):
    """The reference's split-K decode attention end to end, in float32 (output not
    rounded to bf16)."""
    return merge_splits(*split_partials(q, k, v, T, split_len, block_n, lens, round_p))
