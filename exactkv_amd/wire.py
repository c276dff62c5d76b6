"""Wire form of one sequence's compressed cache: pack it into one contiguous byte blob
(KV offload to host memory or disk, transfer between pools, processes or GPUs) and
unpack it into a contiguous or paged cache, on the GPU.

No counterpart in the reference: its caches hand out their six tensors (buffers(),
cache.py:121-123); a byte form of them is this build's own. The blob keeps the
reference format's fields (codec.py:1-25) for one sequence, about 200 bytes per
(token, head) against 256 for bf16. Layout (little-endian, sections at multiples of
256 bytes, gaps zero):

  header   256 B: u32 magic "EXKV", version 1, heads, head_dim, tokens, full_pages,
           tail_rows, raw_rows; u64 off_tail, off_rowmask, off_base, off_sm, off_code,
           off_raw, total
  tail     bf16 [T % 16, H, 128]       the open page's tokens
  rowmask  i32  [T // 16, H]
  base     u8   [T // 16, H, 128]
  sm       u8   [16 * (T // 16), H, 128]
  code     u8   [16 * (T // 16), H, 64]
  raw      bf16 [N, 128]               raw rows in (page, head, token) order

rowoff is implicit (the running count of raw rows in (page, head) order), so a blob
does not depend on where its rows sat in the source pool.
"""
import struct

import torch

from . import _lib
from .cache import CompressedKV
from .kernels import P
from .paged import PagedCompressedKV, _popc16

HEADER = 256
MAGIC = 0x564B5845
VERSION = 1
_KEYS = ("magic", "version", "heads", "head_dim", "tokens", "full_pages", "tail_rows", "raw_rows",
         "off_tail", "off_rowmask", "off_base", "off_sm", "off_code", "off_raw", "total")


def nbytes(H, T, raw_rows):
    """Blob size for H heads, T tokens and raw_rows raw rows."""
    n = _lib.load().exkv_wire_bytes(int(H), int(T), int(raw_rows))
    if n < 0:
        raise ValueError(f"bad wire size arguments H={H} T={T} raw_rows={raw_rows}")
    return n


def header(blob):
    """The header fields of a blob (a uint8 tensor on any device) as a dict."""
    if blob.dtype != torch.uint8 or blob.dim() != 1 or blob.numel() < HEADER:
        raise ValueError("a wire blob is a 1-D uint8 tensor of at least 256 bytes")
    vals = struct.unpack_from("<8I7Q", bytes(blob[:HEADER].cpu().numpy()))
    return dict(zip(_KEYS, vals))


def _sequence(cache, seq):
    """(T, pool page of each sequence page, first tail row, pool pages, open page exists)."""
    H = cache.H
    if isinstance(cache, PagedCompressedKV):
        t = cache.table
        if t._pages[seq] is None:
            raise ValueError(f"slot {seq} is not in use")
        T = t.length(seq)
        return T, list(t._pages[seq]), cache.cap + seq * H * P, t.num_pages, T // P < t.max_pages
    if isinstance(cache, CompressedKV):
        if not 0 <= seq < cache.B:
            raise ValueError(f"sequence {seq} outside the cache's {cache.B}")
        NP = cache.TS // P
        T = cache.T
        return T, list(range(seq * NP, seq * NP + NP)), cache.cap + seq * H * P, cache.B * NP, T < cache.TS
    raise TypeError(type(cache))


def _pages_arg(pages, n, dev):
    return torch.tensor(pages[:max(n, 1)], dtype=torch.int32).to(dev)


def pack(cache, seq):
    """Sequence `seq` (a CompressedKV slot b, or a PagedCompressedKV slot) -> uint8 blob on
    the cache's GPU. Synchronises once (to size the blob)."""
    if cache._pending is not None:
        raise RuntimeError("call check_overflow() before packing")
    T, pages, tail_row, pool_pages, _ = _sequence(cache, seq)
    H, npf = cache.H, T // P
    dev = cache.sm.device
    pg = _pages_arg(pages, npf, dev)
    N = int(_popc16(cache.rowmask.view(-1, H).index_select(0, pg[:npf].long()) & 0xFFFF).sum().item()) if npf else 0
    size = nbytes(H, T, N)
    blob = torch.empty(size, dtype=torch.uint8, device=dev)
    ws = torch.empty(npf * H + 2, dtype=torch.int32, device=dev)
    raw = cache.raw
    _lib.call("exkv_wire_pack", _lib.ptr(cache.sm), _lib.ptr(cache.code), _lib.ptr(cache.base),
              _lib.ptr(cache.rowmask), _lib.ptr(cache.rowoff), _lib.ptr(raw), raw.shape[0], _lib.ptr(pg, align=4),
              pool_pages, tail_row, H, T, cache.D, _lib.ptr(ws, align=4), _lib.ptr(blob, align=256, what="blob"),
              size, _lib.stream())
    return blob


def unpack(blob, cache, seq):
    """Write a blob into sequence `seq` of `cache`: a CompressedKV slot b (the cache then
    holds the blob's T tokens, as after prefill_slot) or a PagedCompressedKV slot already
    added with table.add(T) for the blob's T. The raw pool grows first if needed."""
    h = header(blob)
    if h["magic"] != MAGIC or h["version"] != VERSION:
        raise ValueError(f"not an exactkv wire blob (magic {h['magic']:#x}, version {h['version']})")
    if h["head_dim"] != cache.D or h["heads"] != cache.H:
        raise ValueError(f"blob holds {h['heads']} heads of dim {h['head_dim']}, the cache {cache.H} of {cache.D}")
    T, N = h["tokens"], h["raw_rows"]
    if h["total"] != nbytes(cache.H, T, N) or h["full_pages"] != T // P or h["tail_rows"] != T % P:
        raise ValueError("inconsistent wire header")
    if blob.numel() < h["total"]:
        raise ValueError(f"blob of {blob.numel()} bytes is shorter than its header's {h['total']}")
    if not blob.is_cuda or blob.device != cache.sm.device:
        blob = blob.to(cache.sm.device)
    if cache._pending is not None:
        raise RuntimeError("call check_overflow() before unpacking")
    if isinstance(cache, CompressedKV):
        if T > cache.TS:
            raise ValueError(f"blob of {T} tokens into a cache of {cache.TS}")
        cache.T = T
        cache.state[0] = T
    elif isinstance(cache, PagedCompressedKV) and cache.table.length(seq) != T:
        raise ValueError(f"blob of {T} tokens into a slot of {cache.table.length(seq)}")
    _, pages, _, pool_pages, open_page = _sequence(cache, seq)
    cnt = int(cache.cnt.item())
    if cnt + N > cache.cap:
        cache._grow(cnt + N)
    tail_row = cache.cap + seq * cache.H * P                # after any growth
    npf = T // P
    dev = cache.sm.device
    pg = _pages_arg(pages, npf + int(open_page), dev)
    ws = torch.empty(npf * cache.H + 2, dtype=torch.int32, device=dev)
    _lib.call("exkv_wire_unpack", _lib.ptr(blob, align=256, what="blob"), blob.numel(), _lib.ptr(cache.sm),
              _lib.ptr(cache.code), _lib.ptr(cache.base), _lib.ptr(cache.rowmask), _lib.ptr(cache.rowoff),
              _lib.ptr(cache.raw), cache.raw.shape[0], cache.cap, _lib.ptr(cache.cnt, align=4),
              _lib.ptr(cache._before, align=4), _lib.ptr(pg, align=4), int(open_page), pool_pages, tail_row,
              cache.H, T, cache.D, _lib.ptr(ws, align=4), _lib.stream())
    cache._ensure_headroom(cnt + N)
