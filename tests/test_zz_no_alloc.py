"""exkv_attn_compressed_noalloc: decode attention with the split partials in the library's
fixed per-GPU scratch array instead of a caller workspace, for callers that cannot allocate.
No counterpart in the reference. Checked against exkv_attn_compressed (same caches, same
split plan) bit for bit, on two calls in a row -- the second smaller, so it runs over the
first call's leftovers in the scratch -- and on a plan too large for the scratch, which
must be rejected without a launch."""
import pytest
import torch

from exactkv_amd import _lib, kernels, synthetic
from tests.conftest import same_bits
from tests.test_gpu_attention import _encode

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(B, T, Hq, Hkv, seed, D=128):
    TS = -(-T // 16) * 16
    k = synthetic.make_kv(B, TS, Hkv, D=D, kind="k", seed=seed, raw_row_rate=0.01).to(DEV)
    v = synthetic.make_kv(B, TS, Hkv, D=D, kind="v", seed=seed + 1, raw_row_rate=0.01).to(DEV)
    q = synthetic.make_q(B, Hq, D=D, seed=seed + 2).to(DEV)
    return q, _encode(k), _encode(v)


# head dims 64 and 256: the partials take (D + 2) floats each in the same scratch
@pytest.mark.parametrize("B,T,Hq,Hkv,ns,D", [(8, 8192, 32, 8, None, 128), (3, 1000, 28, 4, 7, 128),
                                             (4, 2000, 14, 2, None, 64), (2, 1500, 16, 4, 5, 256)])
def test_noalloc_equals_the_workspace_call(B, T, Hq, Hkv, ns, D):
    print("[case] noalloc", B, T, Hq, Hkv, ns, D, flush=True)
    big = _case(B, T, Hq, Hkv, seed=301, D=D)
    small = _case(max(1, B // 2), T // 3 + 5, Hq, Hkv, seed=311, D=D)
    for q, kc, vc in (big, small):                  # two calls in a row, the second smaller
        Tq = kc.TS if kc.TS < T else T
        nsplit = sl = None
        if ns is not None:                          # an explicit plan of about ns splits
            per = -(-Tq // ns)
            sl = -(-per // 32) * 32
            nsplit = -(-Tq // sl)
        want = kernels.attention_compressed(q, kc, vc, Tq, nsplit=nsplit, split_len=sl)
        out = torch.empty_like(q)
        got = kernels.attention_compressed_noalloc(q, kc, vc, Tq, out=out, nsplit=nsplit, split_len=sl)
        torch.cuda.synchronize()
        assert got is out
        assert same_bits(out, want)


def test_noalloc_rejects_plans_beyond_the_scratch():
    q, kc, vc = _case(4, 512, 32, 8, seed=321)
    cap = _lib.load().exkv_noalloc_scratch_bytes()
    assert cap == 32 << 20
    # 4 x 32 rows x 32 splits x 520 bytes fits; 4 x 32 x 512 splits of 16 tokens does not
    out = torch.empty_like(q)
    kernels.attention_compressed_noalloc(q, kc, vc, 512, out=out, nsplit=32, split_len=16)
    assert 4 * 32 * 512 * 520 > cap
    with pytest.raises(RuntimeError, match="scratch"):
        kernels.attention_compressed_noalloc(q, kc, vc, 8192, out=out, nsplit=512, split_len=16)
    with pytest.raises(ValueError, match="out"):
        kernels.attention_compressed_noalloc(q, kc, vc, 512, out=None)


def test_noalloc_replays_from_a_hip_graph():
    """The call's use case: captured in a HIP graph (no allocation inside the capture) and
    replayed. The first call on the GPU (which looks the scratch address up) runs eagerly,
    then three replays with new queries written in place between them, each checked against
    the workspace call run eagerly after it."""
    print("[case] noalloc graph replay", flush=True)
    B, T, Hq, Hkv = 8, 4096, 32, 8
    q, kc, vc = _case(B, T, Hq, Hkv, seed=331)
    out = torch.empty_like(q)
    kernels.attention_compressed_noalloc(q, kc, vc, T, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kernels.attention_compressed_noalloc(q, kc, vc, T, out=out)
    for i in range(3):
        q.copy_(synthetic.make_q(B, Hq, seed=340 + i).to(DEV))
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        want = kernels.attention_compressed(q, kc, vc, T)
        torch.cuda.synchronize()
        assert same_bits(out, want), i
