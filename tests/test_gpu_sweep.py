"""A seeded sweep over the decode-attention configuration space on the GPU: head dims 64,
128 and 256; GQA ratios from 1 to 32; odd and even KV-head counts (every heads-per-workgroup
and page-phase count, and the generic kernel for odd counts at head dim 64); one length for
the batch or one per sequence; sliding windows; the default split plan, one split, and
explicit split lengths of 1 to 8 pages; paged pools whose unused pages hold NaN and inf;
raw-row rates from none to every tenth row; the merge in the split kernel's tail at head
dim 128 (reference kernels.py:142-194 for the split kernels, :33-43 for the merge).

Every case checks:
  * the compressed call == the bf16 twin bit for bit (same contents, same plan);
  * the same call through a block table over a shuffled page pool == the contiguous call,
    for both caches;
  * each sequence's output within the north-star tolerance (1e-2 relative + 2 bf16 ulp of
    the row) of the oracle's fp32 and fp64 softmax attention over its window. The
    reference's absolute 2e-2 bound against fp64 (tests/test_exactkv.py:75-78) is for its
    unit-scale V; the sweep's V carries per-channel scales, so outputs of a few units (2
    bf16 ulp above 2e-2) are expected and the relative bound is the one that applies;
  * the fused merge == the separate merge bit for bit up to 32 splits (within the oracle's
    tolerance beyond);
  * decode_to_bf16 of the encoded cache == its source.
"""
import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import kernels
from oracle import attention as oatt
from tests.conftest import same_bits, u16

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = 16
N_CASES = 256


def _cases(seed=20261202):
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(N_CASES):
        D = int(rng.choice([64, 128, 256], p=[0.3, 0.45, 0.25]))
        Hkv = int(rng.choice([1, 2, 3, 4, 6, 8, 16]))
        G = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 16, 32]))
        B = int(rng.integers(1, 5))
        TS = P * int(rng.integers(1, 65))
        per_seq = bool(rng.random() < 0.5)
        lens = [int(x) for x in rng.integers(1, TS + 1, size=B)] if per_seq else None
        T = TS if per_seq else int(rng.integers(1, TS + 1))
        window = int(rng.integers(1, TS + 1)) if rng.random() < 0.35 else 0
        reach = TS if per_seq else T
        if window:
            reach = min(reach, window + P - 1)
        u = rng.random()
        if u < 0.5:
            plan = (None, None)
        elif u < 0.65:
            plan = (1, -(-reach // P) * P)
        else:
            sl = P * int(rng.integers(1, 9))
            plan = (-(-reach // sl), sl)
        rate = float(rng.choice([0.0, 0.003, 0.03, 0.1]))
        fused = D == 128 and bool(rng.random() < 0.4)
        spare = int(rng.integers(0, 9))
        out.append(dict(i=i, D=D, Hkv=Hkv, Hq=Hkv * G, B=B, TS=TS, T=T, lens=lens, window=window, plan=plan,
                        rate=rate, fused=fused, spare=spare, seed=int(rng.integers(1, 2**31))))
    return out


CASES = _cases()


def _data(c):
    """K (per-channel scales, exact zeros, rows forced raw at the case's rate), V, q: CPU seeded."""
    g = torch.Generator().manual_seed(c["seed"])
    B, TS, Hkv, D, Hq = c["B"], c["TS"], c["Hkv"], c["D"], c["Hq"]
    sk = 0.3 + 1.2 * float(torch.rand(1, generator=g))
    k = torch.randn(B, TS, Hkv, D, generator=g) * torch.exp(torch.randn(Hkv, D, generator=g) * sk)
    v = torch.randn(B, TS, Hkv, D, generator=g) * torch.exp(torch.randn(Hkv, D, generator=g) * 0.5)
    k[:, ::97, :, 3] = 0.0
    v[:, 7::89, :, D - 2] = 0.0
    for x in (k, v):
        raw = torch.rand(B, TS, Hkv, generator=g) < c["rate"]
        ch = torch.randint(0, D, (B, TS, Hkv), generator=g)
        sel = x.gather(3, ch.unsqueeze(-1)) * 2.0 ** -20
        x.scatter_(3, ch.unsqueeze(-1), torch.where(raw.unsqueeze(-1), sel, x.gather(3, ch.unsqueeze(-1))))
    q = torch.randn(B, Hq, D, generator=g) * (0.1 + 0.4 * float(torch.rand(1, generator=g)))
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def _encode(x):
    B, T, H, D = x.shape
    c = exactkv.CompressedKV(B, T, H, D, reserve=1.0)
    st = (x.stride(0), P * x.stride(1), x.stride(1), x.stride(2))
    kernels.encode_pages(x, st, c._buf(), 0, 0, B, T // P)
    return c


def _pool(x, table, pool_pages, seed):
    """x's pages placed at table's pool pages; the unused pages hold random values with NaN and
    inf (attention must never read them)."""
    B, TS, H, D = x.shape
    g = torch.Generator().manual_seed(seed)
    pool = torch.randn(1, pool_pages * P, H, D, generator=g) * 1e4
    pool[0, ::5, :, 1] = float("nan")
    pool[0, 3::7, :, 2] = float("inf")
    pool = pool.to(torch.bfloat16)
    for b in range(B):
        for p in range(TS // P):
            dst = int(table[b, p]) * P
            pool[0, dst:dst + P] = x[b, p * P:(p + 1) * P]
    return pool


def _label(c):
    return (f"case {c['i']}: D={c['D']} B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} TS={c['TS']} T={c['T']} "
            f"lens={c['lens']} window={c['window']} plan={c['plan']} rate={c['rate']} fused={c['fused']}")


@pytest.mark.parametrize("c", CASES, ids=[f"case{c['i']}" for c in CASES])
def test_attention_sweep(c):
    print("[case]", _label(c), flush=True)
    B, TS, T, W, D = c["B"], c["TS"], c["T"], c["window"], c["D"]
    ns, sl = c["plan"]
    q, k, v = _data(c)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kc, vc = _encode(kd), _encode(vd)
    ld = torch.tensor(c["lens"], dtype=torch.int32, device=DEV) if c["lens"] else None
    kw = dict(lens=ld, nsplit=ns, split_len=sl, window=W)

    o_c = kernels.attention_compressed(qd, kc, vc, T, **kw)
    o_r = kernels.attention_reference(qd, kd, vd, T, **kw)
    assert same_bits(o_c, o_r), "compressed != bf16 twin"

    # the oracle over each sequence's window
    qn, kn, vn = u16(q), u16(k), u16(v)
    oc = o_c.float().cpu().numpy()
    for b in range(B):
        n = c["lens"][b] if c["lens"] else T
        lo = max(n - W, 0) if W else 0
        ks, vs = kn[b:b + 1, lo:n], vn[b:b + 1, lo:n]
        r32 = oatt.attention(qn[b:b + 1], ks, vs, n - lo, np.float32)
        excess = oatt.tolerance_excess(oc[b:b + 1], r32)
        assert excess <= 0, f"sequence {b}: outside the bf16 tolerance by {excess:.3g}"
        r64 = oatt.attention(qn[b:b + 1], ks, vs, n - lo, np.float64)
        excess = oatt.tolerance_excess(oc[b:b + 1], r64)
        assert excess <= 0, f"sequence {b}: outside the bf16 tolerance of fp64 by {excess:.3g}"

    # the same pages through a block table over a shuffled pool with garbage pages
    npg = TS // P
    pool_pages = B * npg + c["spare"]
    perm = torch.randperm(pool_pages, generator=torch.Generator().manual_seed(c["seed"] + 1))
    table = perm[: B * npg].view(B, npg).to(torch.int32)
    pk_cpu, pv_cpu = _pool(k, table, pool_pages, c["seed"] + 2), _pool(v, table, pool_pages, c["seed"] + 3)
    pk, pv = pk_cpu.to(DEV), pv_cpu.to(DEV)
    pkc, pvc = _encode(pk), _encode(pv)
    td = table.to(DEV)
    op_c = kernels.attention_compressed(qd, pkc, pvc, T, block_table=td, **kw)
    op_r = kernels.attention_reference(qd, pk, pv, T, block_table=td, **kw)
    assert same_bits(op_c, o_c), "paged compressed != contiguous compressed"
    assert same_bits(op_r, o_c), "paged twin != contiguous compressed"

    if c["fused"]:
        o_f = kernels.attention_compressed(qd, kc, vc, T, fused_merge=True, **kw)
        nsplit = ns if ns is not None else kernels._plan(B, c["Hkv"], c["Hq"], T, TS, ld, None, None, W, D)[0]
        if nsplit <= 32:
            assert same_bits(o_f, o_c), "fused merge != separate merge"
        else:
            for b in range(B):
                n = c["lens"][b] if c["lens"] else T
                lo = max(n - W, 0) if W else 0
                r32 = oatt.attention(qn[b:b + 1], kn[b:b + 1, lo:n], vn[b:b + 1, lo:n], n - lo, np.float32)
                assert oatt.tolerance_excess(o_f[b:b + 1].float().cpu().numpy(), r32) <= 0

    assert same_bits(kernels.decode_to_bf16(kc, TS), kd)


def _cache_cases(seed=7021):
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(32):
        D = int(rng.choice([64, 128, 256]))
        B = int(rng.integers(1, 7))
        H = int(rng.choice([1, 2, 3, 4, 8]))
        TS = P * int(rng.integers(2, 13))
        T0 = int(rng.integers(0, TS))
        n = min(TS - T0, int(rng.integers(1, 81)))
        rate = float(rng.choice([0.0, 0.05, 0.3]))
        reserve = float(rng.choice([0.0, 0.001, 0.01, 0.5]))
        out.append(dict(i=i, D=D, B=B, H=H, TS=TS, T0=T0, n=n, rate=rate, reserve=reserve,
                        seed=int(rng.integers(1, 2**31))))
    return out


CACHE_CASES = _cache_cases()


@pytest.mark.parametrize("c", CACHE_CASES, ids=[f"cache{c['i']}" for c in CACHE_CASES])
def test_cache_sweep(c):
    """Prefill, then appends across page ends with check_overflow after each (pools started
    small enough to grow): byte-equal to the CPU model of the protocol (oracle/cache.py;
    reference cache.py:17-158) at every page end and at the end; the decoded cache and
    attention over it equal the bf16 cache's (reference tests/test_exactkv.py:81-104)."""
    from oracle import cache as ocache
    print("[case]", c, flush=True)
    B, H, D, TS, T0 = c["B"], c["H"], c["D"], c["TS"], c["T0"]
    g = torch.Generator().manual_seed(c["seed"])

    def make(n):
        x = torch.randn(B, n, H, D, generator=g) * torch.exp(torch.randn(H, D, generator=g))
        x[torch.rand(B, n, H, generator=g) < c["rate"], D // 3] = 1e-30       # forces raw rows
        return x.to(torch.bfloat16)

    kc = exactkv.CompressedKV(B, TS, H, D, reserve=c["reserve"])
    tw = exactkv.BF16KV(B, TS, H, D)
    m = ocache.CacheModel(B, TS, H, D, reserve=c["reserve"])

    def same_state(tag):
        for k in ("sm", "code", "base", "rowmask", "rowoff"):
            assert np.array_equal(getattr(kc, k).cpu().numpy(), getattr(m, k)), (tag, k)
        assert np.array_equal(u16(kc.raw), m.raw), (tag, "raw")
        assert int(kc.cnt.item()) == m.cnt and kc.cap == m.cap and kc.T == m.T and kc.grows == m.grows, tag

    if T0:
        x0 = make(T0)
        x0d = x0.to(DEV)
        for b in range(B):
            kc.prefill_slot(b, x0d[b:b + 1].contiguous())
            tw.prefill_slot(b, x0d[b:b + 1].contiguous())
            m.prefill_slot(b, u16(x0[b]))
        same_state("prefill")
    xs = make(c["n"])
    xsd = xs.to(DEV)
    for t in range(c["n"]):
        kc.append(xsd[:, t].contiguous())
        tw.append(xsd[:, t].contiguous())
        m.append(u16(xs[:, t]))
        exactkv.check_overflow([kc])
        m.check_overflow()
        if kc.T % P == 0:
            same_state(t)
    same_state("end")
    assert same_bits(kernels.decode_to_bf16(kc.buffers(), kc.T), tw.buf[:, :kc.T])
    q = (torch.randn(B, 4 * H, D, generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    assert same_bits(exactkv.decode_attention(q, kc, kc), exactkv.decode_attention(q, tw, tw))


def _paged_cases(seed=9103):
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(16):
        max_seqs, max_pages = int(rng.integers(2, 7)), int(rng.integers(2, 9))
        out.append(dict(i=i, D=int(rng.choice([64, 128, 256])), H=int(rng.choice([1, 2, 3, 4, 8])),
                        G=int(rng.choice([1, 4, 7])), max_seqs=max_seqs, max_pages=max_pages,
                        num_pages=int(rng.integers(max_pages, max_seqs * max_pages + 5)),
                        reserve=float(rng.choice([1e-4, 0.01, 0.5])), ops=150, seed=int(rng.integers(1, 2**31))))
    return out


PAGED_CASES = _paged_cases()


@pytest.mark.parametrize("c", PAGED_CASES, ids=[f"paged{c['i']}" for c in PAGED_CASES])
def test_paged_protocol_sweep(c):
    """Random operations on one PageTable shared by paged K/V caches and their bf16 twins:
    prefills of random lengths (0 to the slot capacity), releases, decode steps over random
    subsets of the live slots in random order (pages opened as tokens fill them), raw-pool
    growth (small reserves, 5% raw rows) and compact(). After every step the compressed and
    bf16 paged attention agree bit for bit; every few operations, and at the end, each live
    slot's tokens decoded through the block table equal the tokens written."""
    print("[case]", c, flush=True)
    rng = np.random.Generator(np.random.PCG64(c["seed"]))
    g = torch.Generator().manual_seed(c["seed"])
    D, H, Hq = c["D"], c["H"], c["H"] * c["G"]
    table = exactkv.PageTable(num_pages=c["num_pages"], max_seqs=c["max_seqs"], max_pages=c["max_pages"])
    kc = exactkv.PagedCompressedKV(table, H, D=D, reserve=c["reserve"])
    vc = exactkv.PagedCompressedKV(table, H, D=D, reserve=c["reserve"])
    kb, vb = exactkv.PagedBF16KV(table, H, D=D), exactkv.PagedBF16KV(table, H, D=D)
    scale = torch.exp(torch.randn(H, D, generator=g))
    truth = {}

    def tokens(n, k):
        x = torch.randn(n, H, D, generator=g) * (scale if k else 1.0)
        x[torch.rand(n, H, generator=g) < 0.05, D // 3] = 1e-30            # raw rows
        return x.to(torch.bfloat16)

    def check_contents(tag):
        live = [s for s in table.live_slots() if table.length(s)]
        if not live:
            return
        Tm = max(table.length(s) for s in live)
        bt = table.block_table.index_select(0, torch.tensor(live, device=DEV))
        for cache, j in ((kc, 0), (vc, 1)):
            dec = kernels.decode_to_bf16(cache.buffers(), Tm, block_table=bt)
            for i, s in enumerate(live):
                T = table.length(s)
                assert same_bits(dec[i, :T], torch.stack(truth[s][j]).to(DEV)), (tag, s, j)

    cap = P * c["max_pages"]
    for op in range(c["ops"]):
        r = rng.random()
        free_slots = [s for s in range(c["max_seqs"]) if s not in truth]
        if r < 0.2 and free_slots:
            T = int(rng.integers(0, cap + 1))
            if min(T // P + 1, c["max_pages"]) > table.free_pages():
                continue
            s = table.add(T, slot=int(rng.choice(free_slots)))
            xk, xv = tokens(T, True), tokens(T, False)
            for cache, x in ((kc, xk), (vc, xv), (kb, xk), (vb, xv)):
                cache.prefill(s, x.unsqueeze(0).to(DEV).contiguous())
            truth[s] = [list(xk), list(xv)]
        elif r < 0.3 and truth:
            s = int(rng.choice(sorted(truth)))
            table.release(s)
            del truth[s]
        elif r < 0.34 and truth:
            kc.compact()
            vc.compact()
            check_contents(f"compact {op}")
        else:
            cand = [s for s in sorted(truth) if table.length(s) < cap]
            if not cand:
                continue
            rows = [int(s) for s in rng.permutation(cand)[: int(rng.integers(1, len(cand) + 1))]]
            need = sum((table.length(s) + 1) % P == 0 and (table.length(s) + 1) // P < c["max_pages"] for s in rows)
            if need > table.free_pages():
                continue
            table.begin_step(rows)
            xk, xv = tokens(len(rows), True), tokens(len(rows), False)
            for i, s in enumerate(rows):
                truth[s][0].append(xk[i])
                truth[s][1].append(xv[i])
            for cache, x in ((kc, xk), (vc, xv), (kb, xk), (vb, xv)):
                cache.append(x.to(DEV).contiguous())
            q = (torch.randn(len(rows), Hq, D, generator=g) * 0.3).to(torch.bfloat16).to(DEV)
            o_c = exactkv.decode_attention(q, kc, vc)
            o_b = exactkv.decode_attention(q, kb, vb)
            assert same_bits(o_c, o_b), f"op {op}: compressed != bf16 paged attention"
            exactkv.check_overflow([kc, vc])
        if op % 10 == 9:
            check_contents(op)
    check_contents("end")


def _wire_cases(seed=4417):
    rng = np.random.Generator(np.random.PCG64(seed))
    return [dict(i=i, B=int(rng.integers(1, 5)), H=int(rng.choice([1, 2, 3, 4, 8])), T=int(rng.integers(1, 701)),
                 rate=float(rng.choice([0.0, 0.01, 0.1])), seed=int(rng.integers(1, 2**31))) for i in range(24)]


WIRE_CASES = _wire_cases()


@pytest.mark.parametrize("c", WIRE_CASES, ids=[f"wire{c['i']}" for c in WIRE_CASES])
def test_wire_sweep(c):
    """Pack every sequence of a cache in one call (sequences in a random order): each blob
    equals the oracle's (oracle/wire.py) byte for byte; unpacked in another order into a
    cache whose raw pool must grow, the decoded tokens and the attention bits equal the
    source cache's."""
    from exactkv_amd import wire
    from oracle import wire as owire
    print("[case]", c, flush=True)
    B, H, T = c["B"], c["H"], c["T"]
    g = torch.Generator().manual_seed(c["seed"])
    x = torch.randn(B, T, H, 128, generator=g) * torch.exp(torch.randn(H, 128, generator=g))
    x[torch.rand(B, T, H, generator=g) < c["rate"], 11] = 1e-30
    x = x.to(torch.bfloat16)
    TS = -(-T // P) * P + P
    src = exactkv.CompressedKV(B, TS, H, 128, reserve=0.5)
    for b in range(B):
        src.prefill_slot(b, x[b:b + 1].to(DEV).contiguous())
    order = [int(b) for b in np.random.Generator(np.random.PCG64(c["seed"])).permutation(B)]
    blobs = wire.pack_many(src, order)
    for b, blob in zip(order, blobs):
        want = owire.pack(u16(x[b]))
        got = blob.cpu().numpy()
        assert got.size == want.size and np.array_equal(got, want), f"sequence {b}"
    dst = exactkv.CompressedKV(B, TS, H, 128, reserve=1e-5)
    wire.unpack_many(blobs[::-1], dst, order[::-1])
    assert dst.T == T
    assert same_bits(kernels.decode_to_bf16(dst.buffers(), T), x.to(DEV))
    q = (torch.randn(B, 4 * H, 128, generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    assert same_bits(exactkv.decode_attention(q, dst, dst), exactkv.decode_attention(q, src, src))


def _enc_cases(seed=5519):
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(40):
        nb, npg = int(rng.integers(1, 5)), int(rng.integers(1, 13))
        out.append(dict(i=i, D=int(rng.choice([64, 128, 256])), H=int(rng.integers(1, 9)), nb=nb, npg=npg,
                        b0=int(rng.integers(0, 3)), pg0=int(rng.integers(0, 4)),
                        layout=str(rng.choice(["bthd", "bhtd", "heads2"])), cnt0=int(rng.choice([0, 0, 37, 1000])),
                        small_cap=bool(rng.random() < 0.3), chained=bool(rng.random() < 0.6),
                        rate=float(rng.choice([0.0, 0.02, 0.2])), nan_page=bool(rng.random() < 0.2),
                        seed=int(rng.integers(1, 2**31))))
    return out


ENC_CASES = _enc_cases()


@pytest.mark.parametrize("c", ENC_CASES, ids=[f"enc{c['i']}" for c in ENC_CASES])
def test_encoder_sweep(c):
    """encode_pages (reference kernels.py:216-268, 340-346) of pages [pg0, pg0 + npg) of
    sequences [b0, b0 + nb) from token-major, head-major and every-other-head strided
    sources, the counter starting at 0 or not, a pool large enough or not (rows past cap are
    dropped while the counter advances), chained or three-launch slot scan, head dims 64 /
    128 / 256, pages of NaN and inf: every written byte equals the oracle's encode of the same
    pages (rowoff shifted by the counter's start), nothing outside the pages is written, and
    the counter and 'before' are the oracle's."""
    from oracle import codec as ocodec
    print("[case]", c, flush=True)
    D, H, nb, npg, b0, pg0 = c["D"], c["H"], c["nb"], c["npg"], c["b0"], c["pg0"]
    T = P * npg
    g = torch.Generator().manual_seed(c["seed"])
    Hs = 2 * H if c["layout"] == "heads2" else H
    x = torch.randn(nb, T, Hs, D, generator=g) * torch.exp(torch.randn(Hs, D, generator=g))
    x[torch.rand(nb, T, Hs, generator=g) < c["rate"], D // 5] = 1e-30
    if c["nan_page"]:
        x[0, :P, 0, 1] = float("nan")
        x[-1, T - P:, -1, 2] = float("inf")
    x = x.to(torch.bfloat16)
    if c["layout"] == "bhtd":
        src = x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)   # [nb, T, H, D] view, head-major memory
    elif c["layout"] == "heads2":
        src = x.to(DEV)[:, :, ::2]
    else:
        src = x.to(DEV)
    want = ocodec.encode(u16(src.contiguous()))
    n = want["raw"].shape[0]
    Bc, TS = b0 + nb + 1, P * (pg0 + npg + 1)
    kc = exactkv.CompressedKV(Bc, TS, H, D, reserve=0.0 if c["small_cap"] else 1.0)
    kc.cnt.fill_(c["cnt0"])
    sentinel = torch.full_like(kc.raw, 3.0)
    kc.raw.copy_(sentinel)
    st = (src.stride(0), P * src.stride(1), src.stride(1), src.stride(2))
    fields = ("sm", "code", "base", "rowmask", "rowoff")
    old = {k: getattr(kc, k).clone() for k in fields}     # the open page 0 is marked already
    kernels.encode_pages(src, st, kc._buf(), b0, pg0, nb, npg, chained=c["chained"])
    t0, t1, p0, p1 = P * pg0, P * (pg0 + npg), pg0, pg0 + npg
    tok, pag = (slice(b0, b0 + nb), slice(t0, t1)), (slice(b0, b0 + nb), slice(p0, p1))
    wants = dict(want, rowoff=want["rowoff"] + c["cnt0"])
    for k, sl in (("sm", tok), ("code", tok), ("base", pag), ("rowmask", pag), ("rowoff", pag)):
        got = getattr(kc, k)
        assert np.array_equal(got[sl].cpu().numpy(), wants[k]), k
        rest, prev = got.clone(), old[k].clone()
        rest[sl] = 0
        prev[sl] = 0
        assert torch.equal(rest, prev), f"{k} written outside the encoded pages"
    assert int(kc.cnt.item()) == c["cnt0"] + n and int(kc._before.item()) == c["cnt0"]
    lo, hi = min(c["cnt0"], kc.cap), min(c["cnt0"] + n, kc.cap)
    assert np.array_equal(u16(kc.raw[lo:hi]), want["raw"][: hi - lo])
    assert same_bits(kc.raw[:lo], sentinel[:lo]) and same_bits(kc.raw[hi:], sentinel[hi:])
