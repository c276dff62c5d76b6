"""Decode-time KV caches: CompressedKV (the exactkv byte format) and BF16KV (plain bf16),
with the interface of the reference's exactkv/cache.py:17-158 -- prefill_slot(b, x),
append(x), T, nbytes(), buffers(), check_overflow(caches).

How CompressedKV is organised here:

* Six device arrays per cache in the codec's layout (sm, code, base, rowmask, rowoff, raw)
  plus int32 words on the device: the raw-row counter `cnt`, its value before the latest
  page encode, and `state[0]`, the number of tokens held (`state[1]` is the append
  kernel's arrival counter, zero between calls).
* The raw array is two regions. Rows [0, cap) take escaped rows in the codec's order
  (sequence, page, head, token), which keeps every byte equal to codec.encode's. Behind
  them each (sequence, head) owns 16 rows holding its open page -- the newest, partly
  filled one -- as bf16; that page is marked all-raw, so the attention and decode kernels
  read it through rowmask / rowoff like any escaped row.
* Everything a decode step changes is computed on the device from `state[0]`: the append
  kernel (one launch) writes the token into the open page, encodes the page when it fills,
  places its raw rows, opens the next page and advances the count; exkv_cache_open_page re-derives the open page's rowmask /
  rowoff after a prefill or a pool move. No host value enters a step, so a step can be
  captured once and replayed.
* The host keeps a mirror `T` of the token count for its checks, and runs the overflow
  protocol: the pool always keeps B*H*16 free slots (one page step of every sequence and
  head), so the page encode inside a step cannot overflow; after a page boundary
  check_overflow reads all counters in one transfer, and a pool that did overflow anyway
  (forced in tests) grows and the page is encoded again from its bf16 rows, which are still
  in the open-page region until the next append.
"""
import torch

from . import _lib
from .kernels import encode_pages, HEAD_DIMS, P

_FIELDS = ("sm", "code", "base", "rowmask", "rowoff", "raw")


def _device_words(n, dev):
    return torch.zeros(n, dtype=torch.int32, device=dev)


class CompressedKV:
    def __init__(self, B, TS, H, D, device="cuda", reserve=0.01):
        """B sequences of up to TS tokens (a multiple of 16), H KV heads of dimension D (64,
        128 or 256; the reference stores 128 only, cache.py:21). reserve: escaped-row slots
        to start with, as a fraction of B*TS*H rows (the pool grows on demand; it never
        starts below one page step of every sequence and head)."""
        if TS % P != 0 or D not in HEAD_DIMS:
            raise AssertionError(f"the format needs TS % {P} == 0 and head dim in {HEAD_DIMS} (got TS={TS}, D={D})")
        dev = torch.device(device)
        self.B, self.TS, self.H, self.D, self.dev = B, TS, H, D, dev
        npages = TS // P
        self.sm = torch.zeros((B, TS, H, D), dtype=torch.uint8, device=dev)
        self.code = torch.zeros((B, TS, H, D // 2), dtype=torch.uint8, device=dev)
        self.base = torch.zeros((B, npages, H, D), dtype=torch.uint8, device=dev)
        self.rowmask = torch.zeros((B, npages, H), dtype=torch.int32, device=dev)
        self.rowoff = torch.zeros((B, npages, H), dtype=torch.int32, device=dev)
        self.cnt = _device_words(1, dev)               # escaped rows placed so far
        self._before = _device_words(1, dev)           # cnt before the latest page encode
        self.state = _device_words(4, dev)             # state[0]: tokens held, as the kernels see it
        self._step_rows = B * H * P                    # the open-page region; also the headroom kept
        self.cap = max(64, int(B * TS * H * reserve), self._step_rows)
        self.raw = torch.zeros((self.cap + self._step_rows, D), dtype=torch.bfloat16, device=dev)
        self.T = 0
        self.grows = 0
        self._pending = None                           # page filled by the last append, until checked
        self._abi = None
        self._open_page()                              # appends may start from an empty cache

    # ---------------------------------------------------------------- device-side upkeep
    def _open_page(self):
        """Mark page state[0] // 16 of every (sequence, head) as its open page, rows in the
        open-page region behind the current cap (a kernel: the page index is read on the GPU)."""
        _lib.call("exkv_cache_open_page", _lib.ptr(self.rowmask, 4), _lib.ptr(self.rowoff, 4),
                  _lib.ptr(self.state, 4), self.cap, self.raw.shape[0], self.B, self.H, self.TS, _lib.stream())

    def _open_rows(self):
        """The open-page region as [B, H, 16, D] (a view of raw)."""
        return self.raw[self.cap:].view(self.B, self.H, P, self.D)

    def kernel_args(self):
        """(sm, code, base, rowmask, rowoff, raw) for the attention and decode kernels; the same
        tuple object until the pool moves (kernels.py keys its argument cache on it)."""
        if self._abi is None or self._abi[5] is not self.raw:
            self._abi = (self.sm, self.code, self.base, self.rowmask, self.rowoff, self.raw)
        return self._abi

    def _buf(self):
        """The encoder's view (kernels.encode_pages): arrays, counters and sizes."""
        d = {k: getattr(self, k) for k in _FIELDS}
        d.update(cnt=self.cnt, before=self._before, cap=self.cap, TS=self.TS, H=self.H, D=self.D)
        return d

    # ---------------------------------------------------------------- raw pool
    def _grow(self, need):
        """Give the escaped-row region room for `need` rows: capacity max(2 cap, need + cap/4),
        the growth rule of the reference protocol (cache.py:62-71). Escaped rows keep their
        slots; the open-page region moves behind the new capacity and the open page's rowoff
        is re-derived on the device."""
        old, cap = self.cap, max(2 * self.cap, need + self.cap // 4)
        pool = torch.zeros((cap + self._step_rows, self.D), dtype=torch.bfloat16, device=self.dev)
        pool[:old].copy_(self.raw[:old])
        pool[cap:].copy_(self.raw[old:])
        self.raw, self.cap = pool, cap
        self.grows += 1
        self._open_page()

    def _keep_headroom(self, used):
        """Grow unless one more page step of every (sequence, head) fits behind `used` rows."""
        if self.cap - used >= self._step_rows:
            return False
        self._grow(used + self._step_rows)
        return True

    def _refit(self, source, b0, pg0, nb, npg):
        """Pages just encoded overflowed the pool (counter > cap): grow to the counter, rewind
        it to its value before those pages and encode them again. source() gives (tensor,
        strides) after the move. Returns the counter."""
        self._grow(int(self.cnt.item()))
        self.cnt.copy_(self._before)
        src, strides = source()
        encode_pages(src, strides, self._buf(), b0, pg0, nb, npg)
        used = int(self.cnt.item())
        assert used <= self.cap, "raw pool still overflows after growing"
        return used

    # ---------------------------------------------------------------- interface
    def prefill_slot(self, b, x):
        """x: [1, T, H, D] bf16, the first T tokens of sequence slot b (every slot the same T).
        Full pages are encoded straight from x through its strides; the rest goes to the
        slot's open-page rows."""
        T = x.shape[1]
        if T > self.TS:
            raise AssertionError(f"{T} prompt tokens do not fit a cache of {self.TS}")
        full = T - T % P
        self.T = T
        self.state[0] = T
        used = None
        if full:
            strides = (x.stride(0), P * x.stride(1), x.stride(1), x.stride(2))
            encode_pages(x, strides, self._buf(), b, 0, 1, full // P)
            used = int(self.cnt.item())
            if used > self.cap:
                used = self._refit(lambda: (x, strides), b, 0, 1, full // P)
        self._open_page()
        if T > full:
            self._open_rows()[b, :, : T - full].copy_(x[0, full:].transpose(0, 1))
        self._keep_headroom(int(self.cnt.item()) if used is None else used)

    def append(self, x):
        """x: [B, H, D] bf16, the next token of every sequence."""
        self._check_can_append()
        self._check_token(x)
        self._launch_append(x)
        self._advance()

    # append in parts, so that a captured decode step can replay the kernels alone
    def _check_can_append(self):
        assert self._pending is None, "a page filled: call check_overflow() before the next append"
        assert self.T < self.TS, "cache is full"

    def _check_token(self, x):
        if x.shape != (self.B, self.H, self.D) or x.dtype != torch.bfloat16 or x.stride(2) != 1:
            raise ValueError(f"append expects a bf16 [{self.B}, {self.H}, {self.D}] tensor with contiguous rows")

    def _launch_append(self, x):
        """Tail write (+ at a page end: page encode, slot scan, raw-row copy, next page
        opened): one kernel that reads the token count from state[0] and advances it."""
        _lib.call("exkv_cache_append", _lib.ptr(x, align=2, what="x"), x.stride(0), x.stride(1),
                  _lib.ptr(self.sm), _lib.ptr(self.code), _lib.ptr(self.base), _lib.ptr(self.rowmask),
                  _lib.ptr(self.rowoff), _lib.ptr(self.raw), _lib.ptr(self.cnt, 4), _lib.ptr(self._before, 4),
                  _lib.ptr(self.state, 4), self.cap, self.raw.shape[0], self.B, self.H, self.TS, self.D,
                  _lib.stream())

    def _advance(self):
        """Host mirror of an append whose kernels ran (eagerly or in a graph replay)."""
        self.T += 1
        if self.T % P == 0:
            self._pending = self.T // P - 1

    def finish_page(self, overflowed, cnt=None):
        """check_overflow's step for this cache: if the page filled by the last append did not
        fit, encode it again from its bf16 rows (still in the open-page region) into a grown
        pool; then restore the headroom from the counter `cnt`. True if the pool grew."""
        grew = False
        page, self._pending = self._pending, None
        if page is not None and overflowed:
            def rows():
                t = self._open_rows()
                return t, (t.stride(0), 0, t.stride(2), t.stride(1))
            cnt = self._refit(rows, 0, page, self.B, 1)
            grew = True
        if cnt is not None:
            grew = self._keep_headroom(cnt) or grew
        return grew

    def buffers(self):
        """The six arrays and the shape, as the reference's kernels take them (a dict)."""
        d = {k: getattr(self, k) for k in _FIELDS}
        d["shape"] = (self.B, self.TS, self.H, self.D)
        return d

    def nbytes(self):
        return sum(getattr(self, k).nbytes for k in _FIELDS)


class BF16KV:
    """The uncompressed twin: a plain bf16 [B, TS, H, D] cache (buf) with the same interface;
    its appends are a device-side kernel as well (the position comes from state[0])."""

    def __init__(self, B, TS, H, D, device="cuda"):
        self.B, self.TS, self.H, self.D = B, TS, H, D
        self.buf = torch.zeros((B, TS, H, D), dtype=torch.bfloat16, device=device)
        self.state = _device_words(4, torch.device(device))
        self.T = 0
        self.cnt = None                                # no raw pool: check_overflow passes it by

    def prefill_slot(self, b, x):
        n = x.shape[1]
        self.buf[b].narrow(0, 0, n).copy_(x[0])
        self.T = n
        self.state[0] = n

    def append(self, x):
        self._check_can_append()
        self._check_token(x)
        self._launch_append(x)
        self._advance()

    def _check_can_append(self):
        assert self.T < self.TS, "cache is full"

    def _check_token(self, x):
        if x.shape != (self.B, self.H, self.D) or x.dtype != torch.bfloat16 or x.stride(2) != 1:
            raise ValueError(f"append expects a bf16 [{self.B}, {self.H}, {self.D}] tensor with contiguous rows")

    def _launch_append(self, x):
        _lib.call("exkv_bf16_append", _lib.ptr(x, align=2, what="x"), x.stride(0), x.stride(1),
                  _lib.ptr(self.buf), _lib.ptr(self.state, 4), self.B, self.H, self.TS, self.D, _lib.stream())

    def _advance(self):
        self.T += 1

    def nbytes(self):
        return self.buf.nbytes


def check_overflow(caches):
    """After a step whose token filled a page: one device-to-host transfer of the counters of
    every compressed cache (contiguous or paged) with a page waiting, then each repairs an
    overflow and tops up its headroom. Returns the number of pools that grew."""
    waiting = [c for c in caches if hasattr(c, "finish_page") and c._pending is not None]
    if not waiting:
        return 0
    counts = torch.cat([c.cnt for c in waiting]).tolist()
    return sum(int(c.finish_page(n > c.cap, n)) for c, n in zip(waiting, counts))
