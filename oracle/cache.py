"""CPU model of the CompressedKV bookkeeping protocol (test infrastructure only).

Restates reference exactkv/cache.py:17-158 with the two deliberate differences of
this build, so that the GPU cache's buffers can be compared byte for byte:

  * raw-row slots are assigned deterministically: within one encode call, pages are
    visited in (sequence, page, head) order and rows in token order, starting at the
    pool counter -- the order of codec.encode (the reference GPU encoder used an
    atomic counter, kernels.py:262, so its order was not fixed);
  * headroom: the pool starts with at least B*H*16 slots and, after every page-boundary
    check (and after a prefill), keeps at least B*H*16 free slots -- the most one page
    step can add -- growing when needed, so an encode inside a decode step never
    overflows the pool;
  * page 0 is opened at construction, so appends alone can fill a cache.

Layout (as the reference): raw pool = [cap rows for rows that do not fit | B*H*16
tail rows holding the open page of every (sequence, head)]; the open page is marked
all-raw (rowmask 0xFFFF) with rowoff pointing into the tail area.
"""
import numpy as np

from . import codec

P = codec.P


class CacheModel:
    def __init__(self, B, TS, H, D=128, reserve=0.01):
        assert TS % P == 0
        self.B, self.TS, self.H, self.D = B, TS, H, D
        NP = TS // P
        self.sm = np.zeros((B, TS, H, D), np.uint8)
        self.code = np.zeros((B, TS, H, D // 2), np.uint8)
        self.base = np.zeros((B, NP, H, D), np.uint8)
        self.rowmask = np.zeros((B, NP, H), np.int32)
        self.rowoff = np.zeros((B, NP, H), np.int32)
        self.cnt = 0
        self.before = 0
        self.cap = max(64, int(B * TS * H * reserve), B * H * P)
        self.raw = np.zeros((self.cap + B * H * P, D), np.uint16)
        self.T = 0
        self.grows = 0
        self.pending = None
        self.open_tail(0)

    # -- helpers
    def toff(self, b, h):
        return self.cap + (b * self.H + h) * P

    def tail(self, b, h):
        o = self.toff(b, h)
        return self.raw[o:o + P]

    def open_tail(self, pg):
        for b in range(self.B):
            for h in range(self.H):
                self.rowmask[b, pg, h] = -1 & 0xFFFF
                self.rowoff[b, pg, h] = self.toff(b, h)

    def encode_units(self, units):
        """units: list of (b, pg, h, rows uint16 [16, D]) in slot order."""
        self.before = self.cnt
        for b, pg, h, rows in units:
            c = codec.encode(rows.reshape(1, P, 1, self.D))
            t0 = pg * P
            self.sm[b, t0:t0 + P, h] = c["sm"][0, :, 0]
            self.code[b, t0:t0 + P, h] = c["code"][0, :, 0]
            self.base[b, pg, h] = c["base"][0, 0, 0]
            self.rowmask[b, pg, h] = c["rowmask"][0, 0, 0]
            self.rowoff[b, pg, h] = self.cnt
            for k in range(c["raw"].shape[0]):
                if self.cnt + k < self.cap:
                    self.raw[self.cnt + k] = c["raw"][k]
            self.cnt += c["raw"].shape[0]

    def grow(self, need):
        new_cap = max(2 * self.cap, need + self.cap // 4)
        raw = np.zeros((new_cap + self.B * self.H * P, self.D), np.uint16)
        raw[:self.cap] = self.raw[:self.cap]
        raw[new_cap:] = self.raw[self.cap:]
        self.raw, self.cap = raw, new_cap
        self.grows += 1
        if self.T < self.TS:
            pg = self.T // P
            for b in range(self.B):
                for h in range(self.H):
                    self.rowoff[b, pg, h] = self.toff(b, h)

    def redo(self, units_fn):
        if self.cnt <= self.cap:
            return
        self.grow(self.cnt)
        self.cnt = self.before
        self.encode_units(units_fn())
        assert self.cnt <= self.cap

    def ensure_headroom(self):
        need = self.B * self.H * P
        if self.cap - self.cnt < need:
            self.grow(self.cnt + need)

    # -- interface (reference cache.py:87-119, 149-158)
    def prefill_slot(self, b, x):
        """x: uint16 [T, H, D] for sequence slot b."""
        T = x.shape[0]
        Tf = T // P * P

        def units():
            return [(b, pg, h, x[pg * P:(pg + 1) * P, h]) for pg in range(Tf // P) for h in range(self.H)]
        if Tf:
            self.encode_units(units())
            self.redo(units)
        if Tf < self.TS and b == 0:
            self.open_tail(Tf // P)
        for h in range(self.H):
            self.tail(b, h)[:T - Tf] = x[Tf:, h]
        self.T = T
        self.ensure_headroom()

    def append(self, x):
        """x: uint16 [B, H, D]."""
        assert self.pending is None
        p = self.T % P
        for b in range(self.B):
            for h in range(self.H):
                self.tail(b, h)[p] = x[b, h]
        self.T += 1
        if self.T % P == 0:
            pg = self.T // P - 1
            self.encode_units(self._tail_units(pg))
            self.pending = pg
            if self.T < self.TS:
                self.open_tail(pg + 1)

    def _tail_units(self, pg):
        return [(b, pg, h, self.tail(b, h).copy()) for b in range(self.B) for h in range(self.H)]

    def check_overflow(self):
        """One cache's share of check_overflow: re-encode the pending page if the pool
        overflowed, then restore the headroom. Returns 1 if the pool grew."""
        if self.pending is None:
            return 0
        g0 = self.grows
        pg = self.pending
        if self.cnt > self.cap:
            self.grow(self.cnt)
            self.cnt = self.before
            self.encode_units(self._tail_units(pg))
            assert self.cnt <= self.cap
        self.pending = None
        self.ensure_headroom()
        return int(self.grows > g0)

    def buffers(self):
        return dict(shape=(self.B, self.TS, self.H, self.D), sm=self.sm, code=self.code, base=self.base,
                    rowmask=self.rowmask, rowoff=self.rowoff, raw=self.raw)
