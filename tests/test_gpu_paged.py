"""Paged caches (block tables) on the GPU: the same attention over a pool of pages.

No counterpart in the reference, which stores contiguous [B, TS, ...] caches only (paged KV
is the first item of its future work, README.md:121-123). Gates:
  * over a pool whose pages are the contiguous cache's pages in shuffled order, the paged
    call returns the contiguous call's bits (same page contents, same split plan);
  * the compressed and bf16 paged calls are bit-identical;
  * within the north-star tolerance of the oracle's fp32 attention.
"""
import numpy as np
import pytest
import torch

import exactkv_amd as exactkv
from exactkv_amd import kernels, synthetic
from oracle import attention as oatt
from tests.conftest import same_bits, u16
from tests.test_gpu_attention import _encode, assert_bf16_tolerance

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = 16


def _say(*a):
    print("[case]", *a, flush=True)


def _pool(x, table, pool_pages):
    """bf16 [1, 16 * pool_pages, H, D] holding page p of sequence b of x at page table[b, p];
    the unused pool pages hold unrelated values."""
    B, TS, H, D = x.shape
    g = torch.Generator(device="cpu").manual_seed(99)
    pool = (torch.randn(1, pool_pages * P, H, D, generator=g) * 3).to(torch.bfloat16).to(x.device)
    for b in range(B):
        for p in range(TS // P):
            s = int(table[b, p])
            pool[0, s * P:(s + 1) * P] = x[b, p * P:(p + 1) * P]
    return pool


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (28, 4)])
def test_paged_matches_contiguous(Hq, Hkv):
    B, TS = 3, 1024
    lens = [1000, 517, 33]
    k = synthetic.make_kv(B, TS, Hkv, kind="k", seed=51, raw_row_rate=0.01)
    v = synthetic.make_kv(B, TS, Hkv, kind="v", seed=52, raw_row_rate=0.01)
    q = synthetic.make_q(B, Hq, seed=53)
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    npg = TS // P
    pool_pages = B * npg + 17
    perm = torch.randperm(pool_pages, generator=torch.Generator().manual_seed(7))[:B * npg]
    table = perm.view(B, npg).to(torch.int32)
    kp, vp = _pool(kd, table, pool_pages), _pool(vd, table, pool_pages)
    kc, vc = _encode(kd), _encode(vd)
    kpc, vpc = _encode(kp), _encode(vp)
    bt = table.to(DEV)
    ld = torch.tensor(lens, dtype=torch.int32, device=DEV)
    _say("paged", B, TS, Hq, Hkv, "pool pages", pool_pages)
    o_ref = kernels.attention_compressed(qd, kc, vc, 0, lens=ld)
    o_pc = kernels.attention_compressed(qd, kpc, vpc, 0, lens=ld, block_table=bt)
    o_pb = kernels.attention_reference(qd, kp, vp, 0, lens=ld, block_table=bt)
    assert same_bits(o_pc, o_ref)
    assert same_bits(o_pb, o_pc)
    assert_bf16_tolerance(o_pc, oatt.attention(u16(q), u16(k), u16(v), TS, np.float32, lens=lens))


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (28, 4)])
def test_paged_long_split(Hq, Hkv):
    """One split over 2048 tokens: a wavefront's pages past the 64 whose block-table entries
    it (and its loader) holds in registers come through scalar loads of the table."""
    B, TS = 2, 2048
    k = synthetic.make_kv(B, TS, Hkv, kind="k", seed=54, raw_row_rate=0.01)
    v = synthetic.make_kv(B, TS, Hkv, kind="v", seed=55, raw_row_rate=0.01)
    q = synthetic.make_q(B, Hq, seed=56)
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    npg = TS // P
    pool_pages = B * npg + 5
    perm = torch.randperm(pool_pages, generator=torch.Generator().manual_seed(8))[:B * npg]
    table = perm.view(B, npg).to(torch.int32)
    kp, vp = _pool(kd, table, pool_pages), _pool(vd, table, pool_pages)
    kc, vc = _encode(kd), _encode(vd)
    kpc, vpc = _encode(kp), _encode(vp)
    bt = table.to(DEV)
    _say("paged long split", B, TS, Hq, Hkv)
    o_ref = kernels.attention_compressed(qd, kc, vc, TS, nsplit=1, split_len=TS)
    o_pc = kernels.attention_compressed(qd, kpc, vpc, TS, nsplit=1, split_len=TS, block_table=bt)
    o_pb = kernels.attention_reference(qd, kp, vp, TS, nsplit=1, split_len=TS, block_table=bt)
    assert same_bits(o_pc, o_ref)
    assert same_bits(o_pb, o_pc)
    assert_bf16_tolerance(o_pc, oatt.attention(u16(q), u16(k), u16(v), TS, np.float32))


def test_paged_shared_prefix_pages():
    """Two sequences whose first pages are the same pool pages (a shared prefix) and a
    third whose table repeats one page: the result is that of the gathered contents."""
    B, Hq, Hkv, npg = 3, 32, 8, 20
    pool_pages = 40
    g = torch.Generator().manual_seed(3)
    base = synthetic.make_kv(1, pool_pages * P, Hkv, kind="k", seed=61)
    vbase = synthetic.make_kv(1, pool_pages * P, Hkv, kind="v", seed=62)
    table = torch.randint(0, pool_pages, (B, npg), generator=g, dtype=torch.int32)
    table[1, :8] = table[0, :8]                        # shared prefix
    table[2, :] = table[2, 5]                          # one page again and again
    q = synthetic.make_q(B, Hq, seed=63)
    kd, vd, qd = base.to(DEV), vbase.to(DEV), q.to(DEV)
    kpc, vpc = _encode(kd), _encode(vd)
    # the gathered contiguous caches
    idx = (table.long()[:, :, None] * P + torch.arange(P)[None, None, :]).reshape(B, npg * P)
    kg, vg = base[0][idx], vbase[0][idx]               # [B, T, H, D]
    T = npg * P - 5
    _say("paged shared", B, T, table[2, 0].item())
    bt = table.to(DEV)
    o_pc = kernels.attention_compressed(qd, kpc, vpc, T, block_table=bt)
    o_pb = kernels.attention_reference(qd, kd, vd, T, block_table=bt)
    o_g = kernels.attention_reference(qd, kg.to(DEV).contiguous(), vg.to(DEV).contiguous(), T)
    assert same_bits(o_pc, o_pb)
    assert same_bits(o_pb, o_g)
    assert_bf16_tolerance(o_pc, oatt.attention(u16(q), u16(kg), u16(vg), T, np.float32))


def test_paged_bad_arguments_raise():
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(1, 64, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        kernels.attention_reference(q, k, k, 16, block_table=torch.zeros(1, 2, dtype=torch.int64, device=DEV))
    with pytest.raises(RuntimeError, match="exceeds|outside"):
        kernels.attention_reference(q, k, k, 48, block_table=torch.zeros(1, 2, dtype=torch.int32, device=DEV))


@pytest.mark.parametrize("chained", [True, False])
def test_paged_encoder_bytes_match_contiguous(chained):
    """encode_pages_paged writes, at each mapped pool page, the bytes encode_pages writes
    at the contiguous page (same raw-slot order, so rowoff and raw agree too); through the
    chained scan and through the three-launch scan."""
    B, TS, H = 3, 512, 8
    npg = TS // P
    x = synthetic.make_kv(B, TS, H, kind="k", seed=71, raw_row_rate=0.02).to(DEV)
    pool_pages = B * npg + 9
    table = torch.randperm(pool_pages, generator=torch.Generator().manual_seed(8))[:B * npg].view(B, npg)
    c = _encode(x)
    pool = exactkv.CompressedKV(1, pool_pages * P, H, 128, reserve=1.0)
    st = (x.stride(0), P * x.stride(1), x.stride(1), x.stride(2))
    _say("paged encode", B, TS, H, pool_pages)
    kernels.encode_pages_paged(x, st, pool._buf(), table.to(torch.int32).to(DEV), B, npg, chained=chained)
    n = int(c.cnt.item())
    assert n > 0 and int(pool.cnt.item()) == n
    tl = table.reshape(-1).to(DEV)
    rows = (tl[:, None] * P + torch.arange(P, device=DEV)[None, :]).reshape(-1)
    assert torch.equal(pool.sm[0][rows], c.sm.reshape(-1, H, 128))
    assert torch.equal(pool.code[0][rows], c.code.reshape(-1, H, 64))
    assert torch.equal(pool.base[0][tl], c.base.reshape(-1, H, 128))
    assert torch.equal(pool.rowmask[0][tl], c.rowmask.reshape(-1, H))
    assert torch.equal(pool.rowoff[0][tl], c.rowoff.reshape(-1, H))
    assert torch.equal(pool.raw[:n], c.raw[:n])


def _gather(pool_bf16, pages, T):
    rows = (torch.tensor(pages)[:, None] * P + torch.arange(P)[None, :]).reshape(-1)[:T]
    return pool_bf16[0][rows.to(pool_bf16.device)]


@pytest.mark.parametrize("D", [128, 64, 256])
def test_paged_cache_prefill_append_release_compact(D):
    """A PageTable shared by paged K/V caches and their bf16 twins: prefills of ragged
    lengths, decode steps over dense and permuted slot subsets, a forced raw-pool overflow,
    release + reuse of pages and compact(). After every step the compressed and bf16 paged
    attention agree bit for bit; the decoded pool equals the tokens written. At head dims
    128, 64 and 256 (the paged encoder and appends are templates on the head dim)."""
    H, Hq = 4, 16
    table = exactkv.PageTable(num_pages=64, max_seqs=4, max_pages=16)
    kc, vc = (exactkv.PagedCompressedKV(table, H, D=D, reserve=1e-4),
              exactkv.PagedCompressedKV(table, H, D=D, reserve=1e-4))
    kb, vb = exactkv.PagedBF16KV(table, H, D=D), exactkv.PagedBF16KV(table, H, D=D)
    src_k = synthetic.make_kv(6, 256, H, D=D, kind="k", seed=81, raw_row_rate=0.05)
    src_v = synthetic.make_kv(6, 256, H, D=D, kind="v", seed=82, raw_row_rate=0.05)
    truth = {}                                          # slot -> (k rows, v rows) on the CPU

    def prefill(seq, T):
        s = table.add(T)
        k, v = src_k[seq:seq + 1, :T], src_v[seq:seq + 1, :T]
        for c, x in ((kc, k), (vc, v), (kb, k), (vb, v)):
            c.prefill(s, x.to(DEV).contiguous())
        truth[s] = [list(k[0]), list(v[0]), seq]
        return s

    def step(slots, check=True):
        table.begin_step(slots)
        rows = table._step_slots
        xk = torch.stack([src_k[truth[s][2], len(truth[s][0])] for s in rows])
        xv = torch.stack([src_v[truth[s][2], len(truth[s][1])] for s in rows])
        for s, a, b in zip(rows, xk, xv):
            truth[s][0].append(a)
            truth[s][1].append(b)
        for c, x in ((kc, xk), (vc, xv), (kb, xk), (vb, xv)):
            c.append(x.to(DEV).contiguous())
        if check:
            q = synthetic.make_q(len(rows), Hq, D=D, seed=table.step).to(DEV)
            o_c = exactkv.decode_attention(q, kc, vc)
            o_b = exactkv.decode_attention(q, kb, vb)
            assert same_bits(o_c, o_b), f"step {table.step}"
        exactkv.check_overflow([kc, vc])

    def check_contents():
        live = table.live_slots()
        for c, b in ((kc, kb), (vc, vb)):
            # through the block table: each live slot's tokens in order
            Tm = max(table.length(s) for s in live)
            if Tm:
                bt = table.block_table.index_select(0, torch.tensor(live, device=DEV))
                dec_bt = kernels.decode_to_bf16(c.buffers(), Tm, block_table=bt)
                for i, s in enumerate(live):
                    T = table.length(s)
                    if T:
                        want = torch.stack(truth[s][0 if c is kc else 1]).to(DEV)
                        assert same_bits(dec_bt[i, :T], want), f"slot {s} (block table)"
            dec = kernels.decode_to_bf16(c.buffers(), c.TS)
            for s in table.live_slots():
                pages, T = table.pages(s), table.length(s)
                want = torch.stack(truth[s][0 if c is kc else 1]).to(DEV) if T else None
                if T:
                    assert same_bits(_gather(dec, pages, T), want), f"slot {s}"
                    assert same_bits(_gather(b.buf, pages, T), want)

    _say("paged cache: prefill 37, 16, 100, 0")
    for seq, T in enumerate((37, 16, 100, 0)):
        prefill(seq, T)
    check_contents()
    for i in range(20):
        step(None)
    _say("paged cache: permuted subsets")
    for i in range(12):
        step([3, 1] if i % 2 else [2, 0, 3])
    check_contents()
    _say("paged cache: forced overflow")
    grows = kc.grows
    kc.cnt.fill_(kc.cap + 1)                            # the next filled pages overflow the pool
    for i in range(40):                                 # attention would read dropped rows until repaired
        step(None, check=False)
        if kc.grows > grows:
            break
    assert kc.grows > grows and int(kc.cnt.item()) >= int(kc._before.item()) > 0
    check_contents()
    step(None)
    _say("paged cache: release, reuse, compact")
    table.release(1)
    del truth[1]
    assert prefill(4, 61) == 1                          # the lowest free slot, reusing freed pages
    for i in range(18):
        step(None)
    assert kc.compact() > 0                             # the overflow left a gap; slot 1's old rows
    vc.compact()
    check_contents()
    step(None)
    check_contents()
    rows = table._step_slots
    lens = [table.length(s) for s in rows]
    Tm = max(lens)
    kk = torch.zeros(len(rows), Tm, H, D, dtype=torch.bfloat16)
    vv = torch.zeros_like(kk)
    for i, s in enumerate(rows):
        kk[i, :lens[i]] = torch.stack(truth[s][0])
        vv[i, :lens[i]] = torch.stack(truth[s][1])
    q = synthetic.make_q(len(rows), Hq, D=D, seed=table.step)
    _say("paged cache: oracle", D, lens)
    o_c = exactkv.decode_attention(q.to(DEV), kc, vc)
    assert_bf16_tolerance(o_c, oatt.attention(u16(q), u16(kk), u16(vv), Tm, np.float32, lens=lens))


def test_paged_table_errors():
    table = exactkv.PageTable(num_pages=4, max_seqs=2, max_pages=4)
    kc = exactkv.PagedCompressedKV(table, 2)
    with pytest.raises(ValueError):
        table.add(65)                                   # beyond 4 pages of 16
    s = table.add(30)
    with pytest.raises(RuntimeError, match="begin_step"):
        kc.append(torch.zeros(1, 2, 128, dtype=torch.bfloat16, device=DEV))
    table.begin_step([s])
    with pytest.raises(ValueError):
        kc.append(torch.zeros(2, 2, 128, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        table.begin_step([s, s])
    with pytest.raises(RuntimeError, match="exhausted"):
        table.add(40)                                   # 3 pages, 2 free
