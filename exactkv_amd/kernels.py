"""Kernel-level API (drop-in for the reference's exactkv/kernels.py), backed by the HIP
library: decode attention over the compressed cache, the bit-identical uncompressed
twin, the compressed -> bf16 decoder and the page encoder.

Reference signatures kept: attention_compressed(q, kc, vc, T, BLOCK_N, num_warps,
num_stages) (kernels.py:310), attention_reference(q, k, v, T, ...) (:321),
decode_to_bf16(c, T) (:331), encode_pages(src, strides, buf, b0, pg0, nb, npg) (:340),
choose_split (:273), P, LOG2E. BLOCK_N / num_warps / num_stages are accepted for
compatibility; the gfx950 kernels use one tiling (16-token pages, 8 wavefronts), so
the compressed and uncompressed results are identical for any value of them.

Additive keywords: lens (int32 [B] device tensor of per-sequence lengths; then T is
ignored and splits are planned over the buffer length), nsplit / split_len (explicit
split plan), out (output tensor).
"""
import ctypes
import math

import torch

from . import _lib

LOG2E = 1.4426950408889634
P = 16
HEAD_DIMS = (64, 128, 256)   # head dims the kernels are built for (128: the tuned attention kernels)


def choose_split(B, Hkv, T, BLOCK_N, target=512):
    """The reference planner (kernels.py:273-277), kept for API compatibility: about
    `target` programs, split length a multiple of BLOCK_N. Returns (nsplit, split_len)."""
    ns = max(1, min(-(-T // BLOCK_N), target // max(1, B * Hkv)))
    split_len = -(-(-(-T // ns)) // BLOCK_N) * BLOCK_N
    return -(-T // split_len), split_len


def plan_splits_hd(B, Hkv, Hq, T, D):
    """Split plan for head dim D (exkv_plan_splits_hd): plan_splits' defaults at 128 and,
    over Hkv / 2 pairs of KV heads, at 64 with an even Hkv; rounds of the generic-head-dim
    kernel's workgroups at 256 and at 64 with an odd Hkv."""
    ns, sl = ctypes.c_int32(), ctypes.c_int32()
    _lib.call("exkv_plan_splits_hd", B, Hkv, Hq, T, D, ctypes.byref(ns), ctypes.byref(sl))
    return ns.value, sl.value


def plan_splits(B, Hkv, Hq, T, target_blocks=256, min_split=16):
    """MI355X split plan (native): about `target_blocks` workgroups (one per CU) when there
    are fewer (sequence, head-block) units than that, else at least two full rounds -- at
    least `min_split` tokens per split, split length a multiple of 32 (or one 16-token page).
    Returns (nsplit, split_len). Short splits cost little: a wavefront's pages follow one
    another at about one round trip each, so few units are best served by many splits
    (measured: B1 x 8K 36 -> 18 -> 14.3 us going from 256- to 64- to 32-token splits)."""
    ns, sl = ctypes.c_int32(), ctypes.c_int32()
    _lib.call("exkv_plan_splits", B, Hkv, Hq, T, target_blocks, min_split, ctypes.byref(ns), ctypes.byref(sl))
    return ns.value, sl.value


def error_bits(device=None, clear=True):
    """The library's sticky kernel error bits on `device` (default: the current one), read
    after the work queued on its current stream has completed: 0 when no kernel has given up
    a bounded wait or clamped an out-of-pool index since the last clear (see
    _lib.ERROR_BITS / include/exactkv.h EXKV_ERR_*). clear: reset them."""
    idx = torch.cuda.current_device() if device is None else torch.device(device).index
    return _lib.stream_error_bits(_lib.stream(idx), clear=clear)


def check_errors(device=None):
    """Raise RuntimeError if a kernel has set an error bit on `device` (and clear them)."""
    bits = error_bits(device, clear=True)
    if bits:
        raise RuntimeError(f"exactkv kernel error bits {bits:#x}: {_lib.describe_errors(bits)}")


def set_wait_limit(polls):
    """Test hook: bound the split kernels' inter-wavefront flag waits of this thread's later
    attention calls to `polls` polls (<= 0: the default, never reached by a correct call)."""
    _lib.call("exkv_set_wait_limit", int(polls))


_WS = {}  # split partials, reused per (device, stream, rows, nsplit): kernels on one stream run in order
_CNT = {}  # merge arrival counters per (device, stream, units): zero between calls


def _workspace(dev, rows, ns, D, st=None):
    key = (dev.index, _lib.stream(dev.index) if st is None else st, rows, ns, D)
    ws = _WS.get(key)
    if ws is None:
        f32 = dict(device=dev, dtype=torch.float32)
        ws = _WS[key] = (torch.empty(rows, ns, D, **f32), torch.empty(rows, ns, **f32),
                         torch.empty(rows, ns, **f32))
    return ws


def merge_units(B, Hkv, Hq):
    """Workgroup units of the split kernel: sequences x KV-head blocks of min(gcd(Hkv, 8), 4)
    x groups of 16 query heads per KV head."""
    return B * (Hkv // min(math.gcd(Hkv, 8), 4)) * (-(-(Hq // Hkv) // 16))


FUSED_MERGE_MAX_SPLITS = 1024   # up to this many splits the split kernel can merge in its tail
# With fused_merge the split kernel's last workgroups merge the partials (one level up to
# 32 splits, with the separate merge's bits; beyond, two levels of about sqrt(nsplit)
# splits each), writing them with device-scope stores so that no L2 write-back is needed.
# It is not the default: measured on MI355X it costs more than the separate merge launch
# (eager calls: c2a 47.7 vs 44.4 us, c1 35.0 vs 19.9): after its last page the last
# workgroup of a unit waits for its stores, an arrival atomic, the partials' loads and the
# output store, device-scope round trips in a row that cost more than a second launch.


def release_workspaces():
    """Drop every cached workspace (split partials, arrival counters, scan workspaces), so
    that torch's allocator can return their memory; later calls allocate new ones (the
    counters and scan workspaces zeroed, as on first use)."""
    _WS.clear()
    _CNT.clear()
    _SCAN.clear()


def _counters(dev, n):
    key = (dev.index, _lib.stream(), n)
    c = _CNT.get(key)
    if c is None:
        c = _CNT[key] = torch.zeros(n, dtype=torch.int32, device=dev)
    return c


def _fused_counters(dev, B, Hkv, Hq, ns, fused_merge):
    """Arrival counters (zero between calls) when the merge runs in the split kernel's tail,
    else None."""
    if not fused_merge or ns > FUSED_MERGE_MAX_SPLITS:
        return None
    n = _lib.load().exkv_merge_counters(B, Hq, Hkv, ns)
    if n < 0:
        raise ValueError(f"no fused merge for B={B} Hq={Hq} Hkv={Hkv} nsplit={ns}")
    return _counters(dev, n)


def _check_q(q):
    if q.dim() != 3 or q.shape[2] not in HEAD_DIMS:
        raise ValueError(f"q must be [B, Hq, D], D in {HEAD_DIMS} (got {tuple(q.shape)})")
    if q.dtype != torch.bfloat16 or not q.is_contiguous() or not q.is_cuda:
        raise ValueError("q must be a contiguous bf16 GPU tensor")


def _cache_args(c):
    """(seven compressed-cache arguments, TS, Hkv, B) from a CompressedKV or its buffers() dict."""
    if isinstance(c, dict):
        B, TS, H, D = c["shape"]
        raw = c["raw"]
        args = (c["sm"], c["code"], c["base"], c["rowmask"], c["rowoff"], raw)
    else:
        args = c.kernel_args()
        memo = getattr(c, "_abi_memo", None)
        if memo is not None and memo[0] is args:      # the same buffers as last call
            return memo[1]
        B, TS, H = c.B, c.TS, c.H
        raw = args[5]
    for t, name in zip(args, ("sm", "code", "base", "rowmask", "rowoff", "raw")):
        if not t.is_contiguous():
            raise ValueError(f"compressed cache tensor {name} must be contiguous")
    if raw.shape[0] < 1:
        raise ValueError("raw pool must have at least one row")
    ptrs = [_lib.ptr(t, what=n) for t, n in zip(args, ("sm", "code", "base", "rowmask", "rowoff", "raw"))]
    res = (*ptrs, raw.shape[0]), TS, H, B
    if not isinstance(c, dict):
        c._abi_memo = (args, res)                      # kernel_args() is rebuilt when the pool grows
    return res


def _cache_dim(c):
    """Head dim of a CompressedKV or its buffers() dict (the sm array's last axis)."""
    return (c["sm"] if isinstance(c, dict) else c.sm).shape[-1]


def _plan(B, Hkv, Hq, T, TS, lens, nsplit, split_len, window=0, D=128):
    if nsplit is not None and split_len is not None:
        return nsplit, split_len
    reach = TS if lens is not None else T
    if window:                                 # the splits start at the window's first page
        reach = min(reach, window + P - 1)
    return plan_splits(B, Hkv, Hq, reach) if D == 128 else plan_splits_hd(B, Hkv, Hq, reach, D)


def _window_arg(window):
    w = int(window or 0)
    if w < 0:
        raise ValueError(f"window must be >= 0 (got {w})")
    return w


def _lens_arg(lens, B):
    if lens is None:
        return None, 0
    if lens.dtype != torch.int32 or not lens.is_cuda or lens.numel() < 1:
        raise ValueError("lens must be an int32 GPU tensor")
    stride = lens.stride(0) if lens.numel() > 1 else 0
    if lens.numel() > 1 and lens.numel() < B:
        raise ValueError(f"lens has {lens.numel()} entries for B={B}")
    return _lib.ptr(lens, align=4, what="lens"), stride


def _block_table_arg(block_table, B):
    """(pointer, stride, capacity in tokens) of a paged call's int32 [B, max_pages] table."""
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or not block_table.is_contiguous():
        raise ValueError("block_table must be a contiguous int32 [B, max_pages] tensor")
    if block_table.shape[0] < B:
        raise ValueError(f"block_table has {block_table.shape[0]} rows for B={B}")
    return _lib.ptr(block_table, what="block_table"), block_table.shape[1], block_table.shape[1] * P


def attention_compressed(q, kc, vc, T, BLOCK_N=64, num_warps=4, num_stages=1, *, lens=None, nsplit=None,
                         split_len=None, out=None, fused_merge=False, block_table=None, window=0):
    """q [B, Hq, D] bf16 contiguous (D = 64, 128 or 256); kc, vc: CompressedKV objects (or
    their .buffers() dicts) of head dim D; T: valid tokens. Returns bf16 [B, Hq, D], bit-identical to
    attention_reference on the same contents and split plan.

    block_table (int32 [B, max_pages], on the GPU): paged caches. kc / vc are then pools
    of pages (any [Bp, TSp] shape, read as Bp * TSp / 16 pages in order) and page p of
    sequence b is pool page block_table[b, p]; T / lens count tokens of the sequences.

    window > 0 (sliding-window attention; not in the reference, engine.py:26-28 rejects
    it): each sequence attends to its last `window` tokens only."""
    _check_q(q)
    ka, TS, Hkv, Bc = _cache_args(kc)
    va, TSv, Hv, Bv = _cache_args(vc)
    B, Hq, D = q.shape
    if (TSv, Hv) != (TS, Hkv) or (Bc < B or Bv < B if block_table is None else Bc != Bv):
        raise ValueError("k and v caches differ in shape or hold fewer sequences than q")
    if _cache_dim(kc) != D or _cache_dim(vc) != D:
        raise ValueError(f"cache head dim {_cache_dim(kc)} / {_cache_dim(vc)} differs from q's {D}")
    if block_table is not None:
        bt, bts, cap = _block_table_arg(block_table, B)
        pool_pages = Bc * TS // P
        TS = cap
    window = _window_arg(window)
    ns, sl = _plan(B, Hkv, Hq, T, TS, lens, nsplit, split_len, window, D)
    lp, lstride = _lens_arg(lens, B)
    st = _lib.stream(q.device.index)
    wo, wm, wl = _workspace(q.device, B * Hq, ns, D, st)
    cnt = _fused_counters(q.device, B, Hkv, Hq, ns, fused_merge)
    out = torch.empty_like(q) if out is None else out
    if block_table is not None:
        _lib.call("exkv_attn_compressed_paged", _lib.ptr(q), *ka, *va, wo.data_ptr(), wm.data_ptr(), wl.data_ptr(),
                  cnt.data_ptr() if cnt is not None else None, _lib.ptr(out), bt, bts, pool_pages, B, Hq, Hkv, D,
                  int(T), TS, lp, lstride, ns, sl, window, D ** -0.5 * LOG2E, st)
        return out
    _lib.call("exkv_attn_compressed", _lib.ptr(q), *ka, *va, wo.data_ptr(), wm.data_ptr(), wl.data_ptr(),
              cnt.data_ptr() if cnt is not None else None, _lib.ptr(out), B, Hq, Hkv, D, int(T), TS, lp, lstride, ns, sl, window, D ** -0.5 * LOG2E,
              st)
    return out


def attention_compressed_noalloc(q, kc, vc, T, *, out, lens=None, nsplit=None, split_len=None, window=0):
    """attention_compressed for callers that cannot allocate device memory (HIP-graph capture,
    serving loops): the caller passes `out`, and the split partials go to the library's fixed
    per-GPU scratch array (exkv_attn_compressed_noalloc) instead of a workspace. Contiguous
    caches only. Calls that overlap on one GPU share that array and race; a plan with more
    than the scratch's B * Hq * nsplit partials raises."""
    _check_q(q)
    if out is None or out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor shaped like q")
    ka, TS, Hkv, Bc = _cache_args(kc)
    va, TSv, Hv, Bv = _cache_args(vc)
    B, Hq, D = q.shape
    if (TSv, Hv) != (TS, Hkv) or Bc < B or Bv < B:
        raise ValueError("k and v caches differ in shape or hold fewer sequences than q")
    if _cache_dim(kc) != D or _cache_dim(vc) != D:
        raise ValueError(f"cache head dim {_cache_dim(kc)} / {_cache_dim(vc)} differs from q's {D}")
    # the library uses the scratch array of the GPU the stream belongs to: q's
    held = [t for c in (kc, vc) for t in ((c["sm"], c["raw"]) if isinstance(c, dict) else (c.sm, c.raw))]
    others = [t for t in (out, lens, *held) if isinstance(t, torch.Tensor)]
    if any(t.device != q.device for t in others):
        raise ValueError(f"q, out, the caches and lens must all be on {q.device}")
    window = _window_arg(window)
    ns, sl = _plan(B, Hkv, Hq, T, TS, lens, nsplit, split_len, window, D)
    lp, lstride = _lens_arg(lens, B)
    _lib.call("exkv_attn_compressed_noalloc", _lib.ptr(q), *ka, *va, _lib.ptr(out), B, Hq, Hkv, D, int(T), TS, lp,
              lstride, ns, sl, window, D ** -0.5 * LOG2E, _lib.stream(q.device.index))
    return out


def attention_reference(q, k, v, T, BLOCK_N=64, num_warps=4, num_stages=1, *, lens=None, nsplit=None,
                        split_len=None, out=None, fused_merge=False, block_table=None, window=0):
    """Same computation on uncompressed bf16 K, V of shape [B, TS, Hkv, D] (contiguous);
    with block_table, k and v are pools of pages as in attention_compressed."""
    _check_q(q)
    if k.shape != v.shape or k.dim() != 4 or k.dtype != torch.bfloat16 or not (k.is_contiguous() and v.is_contiguous()):
        raise ValueError("k and v must be contiguous bf16 [B, TS, Hkv, D] tensors of one shape")
    B, Hq, D = q.shape
    TS, Hkv = k.shape[1], k.shape[2]
    if (block_table is None and k.shape[0] < B) or k.shape[3] != D:
        raise ValueError("k/v hold fewer sequences than q or have the wrong head dim")
    if block_table is not None:
        if TS % P:
            raise ValueError(f"a page pool's token count must be a multiple of {P} (got {TS})")
        bt, bts, cap = _block_table_arg(block_table, B)
        pool_pages = k.shape[0] * TS // P
        TS = cap
    window = _window_arg(window)
    ns, sl = _plan(B, Hkv, Hq, T, TS, lens, nsplit, split_len, window, D)
    lp, lstride = _lens_arg(lens, B)
    st = _lib.stream(q.device.index)
    wo, wm, wl = _workspace(q.device, B * Hq, ns, D, st)
    cnt = _fused_counters(q.device, B, Hkv, Hq, ns, fused_merge)
    out = torch.empty_like(q) if out is None else out
    if block_table is not None:
        _lib.call("exkv_attn_bf16_paged", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), wo.data_ptr(), wm.data_ptr(),
                  wl.data_ptr(), cnt.data_ptr() if cnt is not None else None, _lib.ptr(out), bt, bts, pool_pages, B,
                  Hq, Hkv, D, int(T), TS, lp, lstride, ns, sl, window, D ** -0.5 * LOG2E, st)
        return out
    _lib.call("exkv_attn_bf16", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), wo.data_ptr(), wm.data_ptr(),
              wl.data_ptr(), cnt.data_ptr() if cnt is not None else None, _lib.ptr(out), B, Hq, Hkv, D, int(T), TS, lp, lstride, ns, sl, window,
              D ** -0.5 * LOG2E, st)
    return out


def decode_to_bf16(c, T, block_table=None):
    """Compressed buffers (a buffers() dict or CompressedKV) -> bf16 [B, T, H, D],
    through the same page rebuild attention uses. block_table (int32 [B, max_pages] on the
    GPU): c is a pool of pages and sequence b's page p is pool page block_table[b, p]."""
    ka, TS, H, B = _cache_args(c)
    D = _cache_dim(c)
    dev = (c["sm"] if isinstance(c, dict) else c.sm).device
    if block_table is not None:
        bt, bts, cap = _block_table_arg(block_table, block_table.shape[0])
        Bq = block_table.shape[0]
        out = torch.empty(Bq, T, H, D, dtype=torch.bfloat16, device=dev)
        _lib.call("exkv_decode_to_bf16_paged", *ka, B * TS // P, bt, bts, _lib.ptr(out), Bq, int(T), H, D,
                  _lib.stream(dev.index))
        return out
    out = torch.empty(B, T, H, D, dtype=torch.bfloat16, device=dev)
    _lib.call("exkv_decode_to_bf16", *ka, _lib.ptr(out), B, int(T), TS, H, D, _lib.stream())
    return out


def _check_source(src, strides, nb, npg, H, D):
    if src.dtype != torch.bfloat16 or not src.is_cuda:
        raise ValueError("encode source must be a bf16 GPU tensor")
    if src.stride(-1) != 1:
        raise ValueError("encode source rows (head dim) must be contiguous")
    if any(s < 0 for s in strides):
        raise ValueError("negative source strides")
    s_b, s_pg, s_p, s_h = strides
    last = (nb - 1) * s_b + (npg - 1) * s_pg + (P - 1) * s_p + (H - 1) * s_h + D - 1
    avail = src.untyped_storage().nbytes() // 2 - src.storage_offset()
    if nb > 0 and npg > 0 and last >= avail:
        raise ValueError(f"encode source too small: needs element {last}, has {avail}")


_SCAN = {}  # page-encoder scan workspaces per (device, stream)


def _scan_ws(dev, units):
    """The page encoder's chained-scan workspace for the current stream of `dev`: 2 +
    ceil(units / 1024) int64 words, zero when created (a larger zeroed tensor replaces it
    when a call needs more). Encodes on one stream run in order, so they share it."""
    need = 2 + (units + 1023) // 1024
    key = (dev.index, _lib.stream(dev.index))
    ws = _SCAN.get(key)
    if ws is None or ws.numel() < need:
        ws = _SCAN[key] = torch.zeros(max(need, 1024), dtype=torch.int64, device=dev)
    return ws


def encode_pages(src, strides, buf, b0, pg0, nb, npg, *, chained=True):
    """Page encoder (reference kernels.py:216-268, same arguments). Source page pg0 + p of
    sequence b0 + i sits at src + i*s_b + p*s_pg, its token rows s_p apart and heads s_h
    apart, with (s_b, s_pg, s_p, s_h) = strides in elements; it is written to page pg0 + p
    of cache sequence b0 + i. buf is a cache's encoder view (CompressedKV._buf()): the six
    arrays, the raw-row counter cnt, cap, TS, H, D and optionally 'before', which receives
    the counter's value before the call. Escaped rows take pool slots from the counter on,
    in (sequence, page, head, token) order. Two launches: the page kernel, then one chained
    slot scan (in a per-stream workspace); chained=False: the page kernel, then a
    three-launch scan (same bytes)."""
    H, TS, D = buf["H"], buf["TS"], buf["D"]
    _check_source(src, strides, nb, npg, H, D)
    raw = buf["raw"]
    before = buf.get("before")
    ws = _scan_ws(raw.device, int(nb) * int(npg) * H) if chained else None
    _lib.call("exkv_encode_pages", _lib.ptr(src, align=2, what="src"), *[int(s) for s in strides],
              _lib.ptr(buf["sm"]), _lib.ptr(buf["code"]), _lib.ptr(buf["base"]), _lib.ptr(buf["rowmask"]),
              _lib.ptr(buf["rowoff"]), _lib.ptr(raw), _lib.ptr(buf["cnt"], align=4),
              _lib.ptr(before, align=4) if before is not None else None, int(buf["cap"]), raw.shape[0],
              buf["sm"].shape[0], int(b0), int(pg0), int(nb), int(npg), H, TS, D, _lib.ptr(ws),
              ws.numel() if ws is not None else 0, _lib.stream())


def encode_pages_paged(src, strides, buf, dst_pages, nb, npg, *, chained=True):
    """encode_pages into a paged cache: page pg of source sequence bi (strides as in
    encode_pages) goes to page dst_pages[bi, pg] of the cache's arrays read as a list of
    B * TS / 16 pages. dst_pages: int32 [>= nb, >= npg] on the GPU."""
    H, TS, D = buf["H"], buf["TS"], buf["D"]
    _check_source(src, strides, nb, npg, H, D)
    if (dst_pages.dtype != torch.int32 or dst_pages.dim() != 2 or dst_pages.stride(1) != 1 or dst_pages.shape[0] < nb
            or dst_pages.shape[1] < npg):
        raise ValueError("dst_pages must be an int32 [nb, npg] tensor with unit column stride")
    raw = buf["raw"]
    before = buf.get("before")
    ws = _scan_ws(raw.device, int(nb) * int(npg) * H) if chained else None
    _lib.call("exkv_encode_pages_paged", _lib.ptr(src, align=2, what="src"), *[int(s) for s in strides],
              _lib.ptr(buf["sm"]), _lib.ptr(buf["code"]), _lib.ptr(buf["base"]), _lib.ptr(buf["rowmask"]),
              _lib.ptr(buf["rowoff"]), _lib.ptr(raw), _lib.ptr(buf["cnt"], align=4),
              _lib.ptr(before, align=4) if before is not None else None, int(buf["cap"]), raw.shape[0],
              buf["sm"].shape[0], _lib.ptr(dst_pages, align=4, what="dst_pages"), dst_pages.stride(0), int(nb), int(npg), H,
              TS, D, _lib.ptr(ws), ws.numel() if ws is not None else 0, _lib.stream())


def _paged_append_args(x, table, slots):
    n, H, D = x.shape
    if x.dtype != torch.bfloat16 or x.stride(2) != 1:
        raise ValueError(f"append expects a bf16 [n, H, {D}] tensor with contiguous rows")
    bt, lens = table.block_table, table.lens
    if slots is not None and (slots.dtype != torch.int32 or slots.numel() != n or not slots.is_contiguous()):
        raise ValueError("slots must be a contiguous int32 tensor with one entry per row of x")
    return ((_lib.ptr(slots, align=4, what="slots") if slots is not None else None), _lib.ptr(lens, align=4),
            _lib.ptr(bt, what="block_table"), bt.stride(0), n, H, bt.shape[0], bt.shape[1])


def append_paged(x, buf, table, slots=None):
    """One token per row of x [n, H, D] into a paged compressed cache (buf as for
    encode_pages, arrays of a [1, 16 * pool_pages, H, D] cache) whose slots, lengths and
    block table are those of `table` (lens already counting the new token)."""
    sp, lp, bp, bts, n, H, ms, mp = _paged_append_args(x, table, slots)
    raw = buf["raw"]
    _lib.call("exkv_cache_append_paged", _lib.ptr(x, align=2, what="x"), x.stride(0), x.stride(1),
              _lib.ptr(buf["sm"]), _lib.ptr(buf["code"]), _lib.ptr(buf["base"]), _lib.ptr(buf["rowmask"]),
              _lib.ptr(buf["rowoff"]), _lib.ptr(raw), _lib.ptr(buf["cnt"], align=4), _lib.ptr(buf["before"], align=4),
              int(buf["cap"]), raw.shape[0], sp, lp, bp, bts, n, H, ms, mp, buf["TS"] // P, buf["D"], _lib.stream())


def append_paged_bf16(x, pool, table, slots=None):
    """bf16 twin of append_paged over pool [1, 16 * pool_pages, H, D]."""
    sp, lp, bp, bts, n, H, ms, mp = _paged_append_args(x, table, slots)
    _lib.call("exkv_bf16_append_paged", _lib.ptr(x, align=2, what="x"), x.stride(0), x.stride(1), _lib.ptr(pool),
              sp, lp, bp, bts, n, H, ms, mp, pool.shape[0] * pool.shape[1] // P, x.shape[2], _lib.stream())
