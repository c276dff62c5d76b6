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
