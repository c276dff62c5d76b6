"""KV caches with one interface: prefill_slot(b, x), append(x), T, nbytes() (drop-in for
the reference's exactkv/cache.py:17-158).

CompressedKV holds one layer's keys (or values) in the exactkv byte format. Full pages
are encoded on the GPU as they fill. The newest, partly filled page is held as bf16 in
a fixed tail area at the end of the raw pool, with all its rows marked raw, so
attention reads it like any other page. Raw pool layout: [rows that did not fit | tail].

Differences from the reference, all internal:
  * the token count lives on the device too (state[0]); append is three HIP launches
    that read it there (tail write + page encode when a page fills, slot scan, raw-row
    copy), so a decode step can be captured in a HIP graph and replayed;
  * raw-row slots are assigned in (sequence, page, head, token) order -- the codec's
    order -- so the buffers are byte-identical to the reference codec's output;
  * the pool starts with at least B*H*16 slots and, after each page-boundary check and
    after a prefill, is grown so that at least B*H*16 slots are free: the next page
    encode (inside a decode step, before attention reads the page) can then never
    overflow. Overflow is still detected and repaired exactly as in the reference
    (grow, rewind the counter, re-encode);
  * page 0 is opened (all raw, in the tail area) at construction, so a cache can also
    be filled by appends alone.
"""
import torch

from . import _lib
from .kernels import encode_pages, P


class CompressedKV:
    def __init__(self, B, TS, H, D, device="cuda", reserve=0.01):
        """B sequences of up to TS tokens (multiple of 16), H KV heads, head dim D.
        reserve: initial raw-row capacity as a fraction of all rows (grows on demand)."""
        assert TS % P == 0 and D == 128, "D = 128 only (Qwen2/2.5/3, Llama-3 family)"
        NP = TS // P
        self.B, self.TS, self.H, self.D, self.dev = B, TS, H, D, torch.device(device)
        dev = self.dev
        self.sm = torch.zeros(B, TS, H, D, dtype=torch.uint8, device=dev)
        self.code = torch.zeros(B, TS, H, D // 2, dtype=torch.uint8, device=dev)
        self.base = torch.zeros(B, NP, H, D, dtype=torch.uint8, device=dev)
        self.rowmask = torch.zeros(B, NP, H, dtype=torch.int32, device=dev)
        self.rowoff = torch.zeros(B, NP, H, dtype=torch.int32, device=dev)
        self.cnt = torch.zeros(1, dtype=torch.int32, device=dev)
        self._before = torch.zeros(1, dtype=torch.int32, device=dev)        # counter before the last encode
        self.state = torch.zeros(4, dtype=torch.int32, device=dev)          # [T, -, -, -] on the device
        # at least one page step of every (sequence, head) fits from the start
        self.cap = max(64, int(B * TS * H * reserve), B * H * P)
        self.raw = torch.zeros(self.cap + B * H * P, D, dtype=torch.bfloat16, device=dev)
        self.T = 0
        self.grows = 0
        self._pending = None                                                # page waiting for check_overflow
        self._refresh()
        self._open_tail(0)                                                  # appends may start from empty

    # -- internals
    def _refresh(self):
        """Views and kernel arguments that depend on the raw pool; rebuilt when it grows."""
        self._tailv = self.raw[self.cap:].view(self.B, self.H, P, self.D)
        self._toff = (self.cap + torch.arange(self.B * self.H, device=self.dev, dtype=torch.int32) * P).view(
            self.B, self.H)
        self._kargs = (self.sm, self.code, self.base, self.rowmask, self.rowoff, self.raw)

    def kernel_args(self):
        return self._kargs

    def _tail_off(self):
        return self._toff

    def _tail(self):
        return self._tailv

    def _open_tail(self, pg):
        self.rowmask[:, pg] = (1 << P) - 1
        self.rowoff[:, pg] = self._toff

    def _buf(self):
        return dict(sm=self.sm, code=self.code, base=self.base, rowmask=self.rowmask, rowoff=self.rowoff,
                    raw=self.raw, cnt=self.cnt, before=self._before, cap=self.cap, TS=self.TS, H=self.H, D=self.D)

    def _grow(self, need):
        new_cap = max(2 * self.cap, need + self.cap // 4)
        raw = torch.zeros(new_cap + self.B * self.H * P, self.D, dtype=torch.bfloat16, device=self.dev)
        raw[: self.cap] = self.raw[: self.cap]
        raw[new_cap:] = self.raw[self.cap:]
        self.raw, self.cap = raw, new_cap
        self.grows += 1
        self._refresh()
        if self.T < self.TS:
            self.rowoff[:, self.T // P] = self._tail_off()                   # the open tail page moved

    def _encode(self, src, strides, b0, pg0, nb, npg):
        encode_pages(src, strides, self._buf(), b0, pg0, nb, npg)          # also records the counter before

    def _redo(self, src, strides, b0, pg0, nb, npg):
        need = int(self.cnt.item())
        if need <= self.cap:
            return need
        self._grow(need)
        self.cnt.copy_(self._before)
        encode_pages(src, strides, self._buf(), b0, pg0, nb, npg)
        n = int(self.cnt.item())
        assert n <= self.cap
        return n

    def _ensure_headroom(self, cnt):
        """Keep room for one more page step of every (sequence, head): B*H*16 rows."""
        need = self.B * self.H * P
        if self.cap - cnt < need:
            self._grow(cnt + need)
            return True
        return False

    # -- interface
    def prefill_slot(self, b, x):
        """x: [1, T, H, D] bf16 for sequence slot b. All slots must have the same T."""
        T = x.shape[1]
        assert T <= self.TS, f"prefill of {T} tokens into a cache of {self.TS}"
        Tf = T // P * P
        if Tf:
            st = (x.stride(0), P * x.stride(1), x.stride(1), x.stride(2))
            self._encode(x, st, b, 0, 1, Tf // P)
            n = self._redo(x, st, b, 0, 1, Tf // P)                          # prefill may sync
        else:
            n = int(self.cnt.item())
        if Tf < self.TS and b == 0:
            self._open_tail(Tf // P)
        self._tail()[b, :, : T - Tf] = x[0, Tf:].transpose(0, 1)
        self.T = T
        self.state[0] = T
        self._ensure_headroom(n)

    def append(self, x):
        """x: [B, H, D] bf16, one new token per sequence."""
        self._check_can_append()
        self._check_token(x)
        self._launch_append(x)
        self._advance()

    def _check_can_append(self):
        assert self._pending is None, "call check_overflow() after a page boundary before appending again"
        assert self.T < self.TS, "cache is full"

    def _check_token(self, x):
        if x.shape != (self.B, self.H, self.D) or x.dtype != torch.bfloat16 or x.stride(2) != 1:
            raise ValueError(f"append expects a bf16 [{self.B}, {self.H}, {self.D}] tensor with contiguous rows")

    def _advance(self):
        """Host side of an append whose kernels already ran (directly or in a graph replay)."""
        self.T += 1
        if self.T % P == 0:
            self._pending = self.T // P - 1

    def _launch_append(self, x):
        _lib.call("exkv_cache_append", _lib.ptr(x, align=2, what="x"), x.stride(0), x.stride(1),
                  _lib.ptr(self.sm), _lib.ptr(self.code), _lib.ptr(self.base), _lib.ptr(self.rowmask),
                  _lib.ptr(self.rowoff), _lib.ptr(self.raw), _lib.ptr(self.cnt, 4), _lib.ptr(self._before, 4),
                  _lib.ptr(self.state, 4), self.cap, self.raw.shape[0], self.B, self.H, self.TS, self.D,
                  _lib.stream())

    def finish_page(self, overflowed, cnt=None):
        """Called by check_overflow with this cache's result; returns True if the pool grew."""
        grew = False
        if self._pending is not None and overflowed:
            pg = self._pending
            t = self._tail()
            st = (t.stride(0), 0, t.stride(2), t.stride(1))
            cnt = self._redo(t, st, 0, pg, self.B, 1)
            grew = True
        self._pending = None
        if cnt is not None:
            grew |= self._ensure_headroom(cnt)
        return grew

    def buffers(self):
        return dict(shape=(self.B, self.TS, self.H, self.D), sm=self.sm, code=self.code, base=self.base,
                    rowmask=self.rowmask, rowoff=self.rowoff, raw=self.raw)

    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in (self.sm, self.code, self.base, self.rowmask, self.rowoff, self.raw))


class BF16KV:
    """Plain bf16 cache [B, TS, H, D] with the same interface (the reference)."""

    def __init__(self, B, TS, H, D, device="cuda"):
        self.B, self.TS, self.H, self.D = B, TS, H, D
        self.buf = torch.zeros(B, TS, H, D, dtype=torch.bfloat16, device=device)
        self.state = torch.zeros(4, dtype=torch.int32, device=device)
        self.T = 0
        self.cnt = None

    def prefill_slot(self, b, x):
        self.buf[b, : x.shape[1]] = x[0]
        self.T = x.shape[1]
        self.state[0] = self.T

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

    def _advance(self):
        self.T += 1

    def _launch_append(self, x):
        _lib.call("exkv_bf16_append", _lib.ptr(x, align=2, what="x"), x.stride(0), x.stride(1),
                  _lib.ptr(self.buf), _lib.ptr(self.state, 4), self.B, self.H, self.TS, self.D, _lib.stream())

    def nbytes(self):
        return self.buf.numel() * 2


def check_overflow(caches):
    """After a page boundary: one host sync for all compressed caches, then re-encode any
    page that overflowed its raw pool and restore every pool's headroom. Returns the
    number of caches whose pool grew."""
    cs = [c for c in caches if hasattr(c, "finish_page") and c._pending is not None]   # compressed, flat or paged
    if not cs:
        return 0
    cnts = torch.cat([c.cnt for c in cs]).cpu().tolist()
    grown = 0
    for c, n in zip(cs, cnts):
        grown += int(c.finish_page(n > c.cap, n))
    return grown
