"""Paged KV caches: one pool of 16-token pages shared by many sequences, each addressed
through its row of a block table.

No counterpart in the reference, whose caches are contiguous [B, TS, H, D] arrays
(cache.py:24-32); paged KV is the first item of its future work (README.md:121-123).
The page format is the reference's (codec.py:1-25) and every page holds exactly the
bytes CompressedKV gives the same 16 tokens; only raw-row slot numbers follow the order
in which pages were encoded.

PageTable holds the allocation, shared by every layer's K and V caches:
  * block_table int32 [max_seqs, max_pages] and lens int32 [max_seqs] on the GPU, with
    host mirrors, and a free list of pool pages;
  * add(T) claims a sequence slot with the pages of T tokens and its open page;
    release(slot) gives them back;
  * begin_step(slots) counts one more token for each listed slot, on the host and the
    device, and claims the page that the token will open when it fills one, before any
    cache appends it. Then every cache appends the step's token with append(x), and
    attention reads lens and block table rows in the step's row order.

PagedCompressedKV / PagedBF16KV hold one layer's keys (or values) for the table's pool.
A sequence's newest, partly filled page lives in its tail area at the end of the raw pool
(all rows raw), as in CompressedKV. Raw rows of released sequences stay in the pool until
compact().
"""
import torch

from . import _lib
from .kernels import HEAD_DIMS, P, encode_pages_paged, append_paged, append_paged_bf16


class PageTable:
    def __init__(self, num_pages, max_seqs, max_pages, device="cuda"):
        """num_pages pool pages of 16 tokens; up to max_seqs sequences of up to 16 * max_pages tokens."""
        assert num_pages > 0 and max_seqs > 0 and max_pages > 0
        self.num_pages, self.max_seqs, self.max_pages = num_pages, max_seqs, max_pages
        self.dev = torch.device(device)
        self.block_table = torch.zeros(max_seqs, max_pages, dtype=torch.int32, device=self.dev)
        self.lens = torch.zeros(max_seqs, dtype=torch.int32, device=self.dev)
        self._free = list(range(num_pages - 1, -1, -1))       # pop() hands out low pages first
        self._pages = [None] * max_seqs                         # pool pages of each live slot
        self._len = [0] * max_seqs
        self.step = 0
        self._step_slots = []
        self._rows = None                                       # (slots tensor or None, table, lens) of the step

    @property
    def capacity(self):
        return P * self.max_pages

    def free_pages(self):
        return len(self._free)

    def length(self, slot):
        return self._len[slot]

    def pages(self, slot):
        return list(self._pages[slot])

    def live_slots(self):
        return [s for s in range(self.max_seqs) if self._pages[s] is not None]

    def _claim(self, n):
        if n > len(self._free):
            raise RuntimeError(f"page pool exhausted: need {n} pages, {len(self._free)} free")
        return [self._free.pop() for _ in range(n)]

    def _npages(self, T):
        """Pages a sequence of T tokens holds: its full pages and its open page."""
        return min(T // P + 1, self.max_pages)

    def add(self, T, slot=None):
        """Claim a slot (the lowest free one unless given) for a sequence of T tokens."""
        if not 0 <= T <= self.capacity:
            raise ValueError(f"sequence of {T} tokens does not fit {self.capacity}")
        if slot is None:
            slot = next((s for s in range(self.max_seqs) if self._pages[s] is None), None)
            if slot is None:
                raise RuntimeError("no free sequence slot")
        elif self._pages[slot] is not None:
            raise ValueError(f"slot {slot} is in use")
        pages = self._claim(self._npages(T))
        self._pages[slot] = pages
        self._len[slot] = T
        row = torch.tensor(pages, dtype=torch.int32)
        self.block_table[slot, : len(pages)] = row.to(self.dev)
        self.lens[slot] = T
        self._rows = None
        return slot

    def release(self, slot):
        """Give a slot's pages back to the pool."""
        if self._pages[slot] is None:
            raise ValueError(f"slot {slot} is not in use")
        self._free.extend(reversed(self._pages[slot]))
        self._pages[slot] = None
        self._len[slot] = 0
        self.lens[slot] = 0
        self._rows = None

    def begin_step(self, slots=None):
        """One more token for each slot in `slots` (host ints, all live and distinct; None: every
        live slot, in order). Batch row i of the step's appends and attention is slots[i]."""
        slots = self.live_slots() if slots is None else [int(s) for s in slots]
        if len(set(slots)) != len(slots):
            raise ValueError("a slot appears twice in one step")
        need = 0
        for s in slots:                                         # check everything before changing anything
            if not 0 <= s < self.max_seqs or self._pages[s] is None:
                raise ValueError(f"slot {s} is not in use")
            L = self._len[s] + 1
            if L > self.capacity:
                raise RuntimeError(f"slot {s} is full ({self.capacity} tokens)")
            need += L % P == 0 and L // P < self.max_pages
        if need > len(self._free):
            raise RuntimeError(f"page pool exhausted: need {need} pages, {len(self._free)} free")
        new_cols, new_pages = [], []
        for s in slots:
            L = self._len[s] + 1
            if L % P == 0 and L // P < self.max_pages:          # the token fills a page: open the next
                pg = self._claim(1)[0]
                self._pages[s].append(pg)
                new_cols.append((s, L // P))
                new_pages.append(pg)
            self._len[s] = L
        if new_cols:
            idx = torch.tensor([s * self.max_pages + c for s, c in new_cols], dtype=torch.int64)
            self.block_table.view(-1)[idx.to(self.dev)] = torch.tensor(new_pages, dtype=torch.int32).to(self.dev)
        self.lens.copy_(torch.tensor(self._len, dtype=torch.int32))
        self.step += 1
        self._step_slots = slots
        if slots == list(range(len(slots))):
            self._rows = (None, self.block_table[: len(slots)], self.lens[: len(slots)])
        else:
            sd = torch.tensor(slots, dtype=torch.int32).to(self.dev)
            self._rows = (sd, self.block_table.index_select(0, sd.long()), self.lens.index_select(0, sd.long()))
        return slots

    def step_rows(self):
        """(slots tensor or None, block table rows, lens) in the current step's row order."""
        if self._rows is None:
            raise RuntimeError("no current step: call begin_step() after adding or releasing sequences")
        return self._rows

    def filled_in_step(self):
        """[(row, slot, page index)] of the pages that the current step's tokens filled."""
        out = []
        for i, s in enumerate(self._step_slots):
            L = self._len[s]
            if L % P == 0 and L > 0:
                out.append((i, s, L // P - 1))
        return out


def _popc16(x):
    x = x - ((x >> 1) & 0x5555)
    x = (x & 0x3333) + ((x >> 2) & 0x3333)
    x = (x + (x >> 4)) & 0x0F0F
    return (x + (x >> 8)) & 0x1F


class PagedCompressedKV:
    """One layer's keys (or values) for the pages of a PageTable, in the exactkv byte format."""

    def __init__(self, table, H, D=128, reserve=0.01):
        assert D in HEAD_DIMS, f"head dim must be one of {HEAD_DIMS} (got {D})"
        self.table, self.H, self.D = table, H, D
        dev = self.dev = table.dev
        NPg = table.num_pages
        self.TS = NPg * P                                      # the pool read as one [1, TS] cache
        self.sm = torch.zeros(1, self.TS, H, D, dtype=torch.uint8, device=dev)
        self.code = torch.zeros(1, self.TS, H, D // 2, dtype=torch.uint8, device=dev)
        self.base = torch.zeros(1, NPg, H, D, dtype=torch.uint8, device=dev)
        self.rowmask = torch.zeros(1, NPg, H, dtype=torch.int32, device=dev)
        self.rowoff = torch.zeros(1, NPg, H, dtype=torch.int32, device=dev)
        self.cnt = torch.zeros(1, dtype=torch.int32, device=dev)
        self._before = torch.zeros(1, dtype=torch.int32, device=dev)
        self._step_room = table.max_seqs * H * P                  # rows one step can add at most
        self.cap = max(64, int(self.TS * H * reserve), self._step_room)
        self.raw = torch.zeros(self.cap + self._step_room, D, dtype=torch.bfloat16, device=dev)
        self.grows = 0
        self._pending = None                                   # pages filled by the last append
        self._appended = 0                                     # table step of the last append

    # -- internals
    def _tail(self, slot):
        """bf16 [H, 16, D] view of a slot's open page (its rows behind cap)."""
        first = self.cap + slot * self.H * P
        return self.raw.narrow(0, first, self.H * P).view(self.H, P, self.D)

    def _buf(self):
        """The encoder's view (kernels.encode_pages_paged): arrays, counters and sizes."""
        d = {k: getattr(self, k) for k in ("sm", "code", "base", "rowmask", "rowoff", "raw")}
        d.update(cnt=self.cnt, before=self._before, cap=self.cap, TS=self.TS, H=self.H, D=self.D)
        return d

    def _open(self, slots):
        """Open the page after the last full page of each of `slots` (host ints) -- table entry
        lens[s] // 16, rows behind cap -- on the device, from the table's device lengths."""
        t = self.table
        if not slots:
            return
        sl = torch.tensor(slots, dtype=torch.int32).to(self.dev)
        bt = t.block_table
        _lib.call("exkv_cache_open_pages_paged", _lib.ptr(self.rowmask, 4), _lib.ptr(self.rowoff, 4),
                  _lib.ptr(sl, 4), len(slots), _lib.ptr(t.lens, 4), _lib.ptr(bt, 4), bt.stride(0), t.max_seqs,
                  t.max_pages, t.num_pages, self.cap, self.raw.shape[0], self.H, _lib.stream())

    def _grow(self, need):
        """Room for `need` escaped rows: capacity max(2 cap, need + cap/4) (the contiguous
        cache's rule); the open-page rows move behind the new capacity and every live slot's
        open page is re-pointed on the device."""
        old, cap = self.cap, max(2 * self.cap, need + self.cap // 4)
        pool = torch.zeros((cap + self._step_room, self.D), dtype=torch.bfloat16, device=self.dev)
        pool[:old].copy_(self.raw[:old])
        pool[cap:].copy_(self.raw[old:])
        self.raw, self.cap = pool, cap
        self.grows += 1
        self._open(self.table.live_slots())

    def _keep_headroom(self, cnt):
        """Grow unless one more step of every slot and head fits behind `cnt` rows."""
        if self.cap - cnt >= self._step_room:
            return False
        self._grow(cnt + self._step_room)
        return True

    def _encode_pages(self, src, st, dst, npg):
        encode_pages_paged(src, st, self._buf(), dst, 1, npg)

    # -- interface
    def prefill(self, slot, x):
        """x: [1, T, H, D] bf16, the first T tokens of the slot (T = table.length(slot))."""
        T = x.shape[1]
        if T != self.table.length(slot):
            raise ValueError(f"prefill of {T} tokens into a slot of {self.table.length(slot)}")
        Tf = T // P * P
        dst = self.table.block_table[slot: slot + 1]
        if Tf:
            st = (x.stride(0), P * x.stride(1), x.stride(1), x.stride(2))
            self._encode_pages(x, st, dst, Tf // P)
            n = int(self.cnt.item())
            if n > self.cap:
                self._grow(n)
                self.cnt.copy_(self._before)
                self._encode_pages(x, st, dst, Tf // P)
                n = int(self.cnt.item())
                assert n <= self.cap
        else:
            n = int(self.cnt.item())
        self._open([slot])
        if T > Tf:
            self._tail(slot)[:, : T - Tf] = x[0, Tf:].transpose(0, 1)
        self._keep_headroom(n)

    prefill_slot = prefill                     # the write-through prefill calls this name

    def append(self, x):
        """x: [n, H, D] bf16, row i the new token of the current step's slot i (begin_step)."""
        self._check_append(tuple(x.shape))
        self._launch_append(x)
        self._advance()

    # append in three parts, so that a captured step can replay the kernels alone
    def _check_append(self, shape):
        t = self.table
        if self._appended == t.step:
            raise RuntimeError("append called twice in one table step (call table.begin_step first)")
        if self._pending is not None:
            raise RuntimeError("call check_overflow() after a step that filled pages before appending again")
        t.step_rows()
        if shape != (len(t._step_slots), self.H, self.D):
            raise ValueError(f"append expects [{len(t._step_slots)}, {self.H}, {self.D}] (one row per step slot)")

    def _launch_append(self, x):
        append_paged(x, self._buf(), self.table, self.table.step_rows()[0])

    def _advance(self):
        self._appended = self.table.step
        self._pending = self.table.filled_in_step() or None

    def finish_page(self, overflowed, cnt=None):
        """check_overflow's per-cache step: re-encode the pages of the last append if the raw pool
        overflowed (from the tail areas, in the append's order), then restore the headroom."""
        grew = False
        if self._pending is not None and overflowed:
            self._grow(int(self.cnt.item()))
            self.cnt.copy_(self._before)
            for _, s, pg in self._pending:
                tl = self._tail(s)
                st = (0, 0, tl.stride(1), tl.stride(0))
                self._encode_pages(tl, st, self.table.block_table[s: s + 1, pg: pg + 1], 1)
            cnt = int(self.cnt.item())
            assert cnt <= self.cap
            grew = True
        self._pending = None
        if cnt is not None:
            grew |= self._keep_headroom(cnt)
        return grew

    def compact(self):
        """Repack the raw rows of live full pages (dropping those of released sequences) in
        (page, head) order; returns the rows freed. Host-synchronising; not for a graph."""
        if self._pending is not None:
            raise RuntimeError("call check_overflow() before compact()")
        t = self.table
        live = sorted(p for s in t.live_slots() for p in t._pages[s][: t.length(s) // P])
        old = int(self.cnt.item())
        if not live:
            self.cnt.zero_()
            return old
        pg = torch.tensor(live, dtype=torch.int64, device=self.dev)
        rm = self.rowmask[0].index_select(0, pg)                # [n, H]
        off = self.rowoff[0].index_select(0, pg)
        cnts = _popc16(rm).reshape(-1).long()
        new_off = torch.cumsum(cnts, 0) - cnts
        total = int(cnts.sum().item())
        if total:
            first = torch.repeat_interleave(off.reshape(-1).long(), cnts, output_size=total)
            base = torch.repeat_interleave(new_off, cnts, output_size=total)
            src = first + torch.arange(total, device=self.dev) - base
            self.raw[:total] = self.raw.index_select(0, src)
        self.rowoff[0].index_copy_(0, pg, new_off.view(rm.shape).to(torch.int32))
        self.cnt.fill_(total)
        return old - total

    def buffers(self):
        return dict(shape=(1, self.TS, self.H, self.D), sm=self.sm, code=self.code, base=self.base,
                    rowmask=self.rowmask, rowoff=self.rowoff, raw=self.raw)

    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in (self.sm, self.code, self.base, self.rowmask, self.rowoff, self.raw))


class PagedBF16KV:
    """Plain bf16 pages [1, 16 * num_pages, H, D] for the same table (the reference twin)."""

    def __init__(self, table, H, D=128):
        self.table, self.H, self.D = table, H, D
        self.buf = torch.zeros(1, table.num_pages * P, H, D, dtype=torch.bfloat16, device=table.dev)
        self._appended = 0
        self.cnt = None

    def prefill(self, slot, x):
        T = x.shape[1]
        if T != self.table.length(slot):
            raise ValueError(f"prefill of {T} tokens into a slot of {self.table.length(slot)}")
        if T:
            pages = torch.tensor(self.table._pages[slot], dtype=torch.int64)
            rows = (pages[:, None] * P + torch.arange(P)[None, :]).reshape(-1)[:T]
            self.buf[0].index_copy_(0, rows.to(self.buf.device), x[0])

    def prefill_slot(self, slot, x):
        self.prefill(slot, x)

    def append(self, x):
        self._check_append(tuple(x.shape))
        self._launch_append(x)
        self._advance()

    def _check_append(self, shape):
        t = self.table
        if self._appended == t.step:
            raise RuntimeError("append called twice in one table step (call table.begin_step first)")
        t.step_rows()
        if shape != (len(t._step_slots), self.H, self.D):
            raise ValueError(f"append expects [{len(t._step_slots)}, {self.H}, {self.D}] (one row per step slot)")

    def _launch_append(self, x):
        append_paged_bf16(x, self.buf, self.table, self.table.step_rows()[0])

    def _advance(self):
        self._appended = self.table.step

    def nbytes(self):
        return self.buf.numel() * 2
