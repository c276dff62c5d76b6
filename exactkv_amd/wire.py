"""Wire form of a sequence's compressed cache: pack it into one contiguous byte blob
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
        if not 0 <= seq < t.max_seqs or t._pages[seq] is None:
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


def _batch_args(cache, seqs, infos, blobs, dev):
    """Device arrays of one pack / unpack call."""
    width = max(max(len(i[1]) for i in infos), 1)
    pages = torch.zeros(len(seqs), width, dtype=torch.int32)
    for r, i in enumerate(infos):
        pages[r, :len(i[1])] = torch.tensor(i[1], dtype=torch.int32)
    max_t = max(i[0] for i in infos)
    ws_stride = (max_t // P) * cache.H + 3
    host = dict(pages=pages, tokens=torch.tensor([i[0] for i in infos], dtype=torch.int32),
                tails=torch.tensor([i[2] for i in infos], dtype=torch.int64),
                blobs=torch.tensor([_lib.ptr(b, align=256, what="blob") for b in blobs], dtype=torch.int64),
                sizes=torch.tensor([b.numel() for b in blobs], dtype=torch.int64),
                open=torch.tensor([int(i[4]) for i in infos], dtype=torch.int32))
    d = {k: v.to(dev) for k, v in host.items()}
    d["ws"] = torch.empty(len(seqs), ws_stride, dtype=torch.int32, device=dev)
    return d, width, max_t, ws_stride


def pack(cache, seq):
    """Sequence `seq` (a CompressedKV slot b, or a PagedCompressedKV slot) -> uint8 blob on
    the cache's GPU. Synchronises once (to size the blob)."""
    return pack_many(cache, [seq])[0]


def pack_many(cache, seqs):
    """Blobs of several sequences of one cache, packed by one call (two launches)."""
    if cache._pending is not None:
        raise RuntimeError("call check_overflow() before packing")
    seqs = list(seqs)
    if not seqs:
        return []
    H, dev = cache.H, cache.sm.device
    infos = [_sequence(cache, s) for s in seqs]
    full = [p for i in infos for p in i[1][:i[0] // P]]
    counts = [0] * len(seqs)
    if full:
        rm = cache.rowmask.view(-1, H).index_select(0, torch.tensor(full, dtype=torch.int64, device=dev))
        per_page = _popc16(rm & 0xFFFF).sum(1).cpu().tolist()
        k = 0
        for r, i in enumerate(infos):
            n = i[0] // P
            counts[r] = int(sum(per_page[k:k + n]))
            k += n
    blobs = [torch.empty(nbytes(H, i[0], n), dtype=torch.uint8, device=dev) for i, n in zip(infos, counts)]
    d, width, max_t, ws_stride = _batch_args(cache, seqs, infos, blobs, dev)
    _lib.call("exkv_wire_pack", _lib.ptr(cache.sm), _lib.ptr(cache.code), _lib.ptr(cache.base),
              _lib.ptr(cache.rowmask), _lib.ptr(cache.rowoff), _lib.ptr(cache.raw), cache.raw.shape[0], infos[0][3],
              len(seqs), d["pages"].data_ptr(), width, d["tokens"].data_ptr(), d["tails"].data_ptr(),
              d["blobs"].data_ptr(), d["sizes"].data_ptr(), max_t, H, cache.D, d["ws"].data_ptr(), ws_stride,
              _lib.stream())
    return blobs


def _check_blob(blob, cache):
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
    npf = h["full_pages"] * cache.H
    if npf:
        rm = blob[h["off_rowmask"]: h["off_rowmask"] + 4 * npf].view(torch.int32)
        rows = int(_popc16(rm & 0xFFFF).sum().item())
        if rows != N:
            raise ValueError(f"blob's rowmask marks {rows} raw rows, its header declares {N}")
    return h


def unpack(blob, cache, seq):
    """Write a blob into sequence `seq` of `cache`: a CompressedKV slot b (the cache then
    holds the blob's T tokens, as after prefill_slot) or a PagedCompressedKV slot already
    added with table.add(T) for the blob's T. The raw pool grows first if needed."""
    unpack_many([blob], cache, [seq])


def unpack_many(blobs, cache, seqs):
    """unpack for several blobs and sequences of one cache in one call (two launches)."""
    seqs = list(seqs)
    if len(blobs) != len(seqs) or len(set(seqs)) != len(seqs):
        raise ValueError("one distinct sequence per blob")
    if not seqs:
        return
    heads = [_check_blob(b, cache) for b in blobs]
    dev = cache.sm.device
    blobs = [b if b.device == dev else b.to(dev) for b in blobs]
    if cache._pending is not None:
        raise RuntimeError("call check_overflow() before unpacking")
    Ts = [h["tokens"] for h in heads]
    if isinstance(cache, CompressedKV):
        if len(set(Ts)) != 1 or Ts[0] > cache.TS:
            raise ValueError(f"blobs of {sorted(set(Ts))} tokens into a cache of {cache.TS} (one length per cache)")
        cache.T = Ts[0]
        cache.state[0] = Ts[0]
    else:
        for s, T in zip(seqs, Ts):
            if cache.table.length(s) != T:
                raise ValueError(f"blob of {T} tokens into a slot of {cache.table.length(s)}")
    N = sum(h["raw_rows"] for h in heads)
    cnt = int(cache.cnt.item())
    if cnt + N > cache.cap:
        cache._grow(cnt + N)
    infos = [_sequence(cache, s) for s in seqs]                 # tail rows after any growth
    d, width, max_t, ws_stride = _batch_args(cache, seqs, infos, blobs, dev)
    _lib.call("exkv_wire_unpack", _lib.ptr(cache.sm), _lib.ptr(cache.code), _lib.ptr(cache.base),
              _lib.ptr(cache.rowmask), _lib.ptr(cache.rowoff), _lib.ptr(cache.raw), cache.raw.shape[0], cache.cap,
              _lib.ptr(cache.cnt, align=4), _lib.ptr(cache._before, align=4), infos[0][3], len(seqs),
              d["pages"].data_ptr(), width, d["tokens"].data_ptr(), d["open"].data_ptr(), d["tails"].data_ptr(),
              d["blobs"].data_ptr(), d["sizes"].data_ptr(), max_t, cache.H, cache.D, d["ws"].data_ptr(), ws_stride,
              _lib.stream())
    cache._keep_headroom(cnt + N)
