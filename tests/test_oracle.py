"""CPU checks that pin the oracle (oracle/) before it is trusted as the GPU's checker.

Reference anchors: codec.py:31-78 (format), kernels.py:33-59 and :273-277 (attention
algebra, planner), cache.py:17-158 (cache protocol), tests/test_exactkv.py:29-49 (inputs).
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import cache as ocache
from oracle import codec
from tests.conftest import u16
from tests.golden import cases

GOLD = os.path.join(os.path.dirname(__file__), "golden")
FIELDS = ("sm", "code", "base", "rowmask", "rowoff", "raw")


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLD, "codec_vectors.npz")), json.load(open(os.path.join(GOLD, "codec_hashes.json")))


# ---------------------------------------------------------------- codec vs reference vectors

@pytest.mark.parametrize("name", list(cases.CASES))
def test_codec_matches_reference_vectors(golden, name):
    """Every byte of the six tensors equals what the reference codec wrote."""
    z, h = golden
    make, stored = cases.CASES[name]
    x = u16(make())
    c = codec.encode(x)
    for k in FIELDS:
        if stored:
            assert np.array_equal(c[k], z[f"{name}/{k}"]), (name, k)
        else:
            assert _sha(c[k]) == h["cases"][name][k]["sha256"], (name, k)
    if stored:
        assert np.array_equal(x, z[f"{name}/input"])
    else:
        assert _sha(x) == h["cases"][name]["input"]["sha256"], f"{name}: input generator drifted"
        for k in ("rowmask", "rowoff"):
            assert np.array_equal(c[k], z[f"{name}/{k}"])


@pytest.mark.parametrize("name", list(cases.CASES))
def test_codec_roundtrip(name):
    x = u16(cases.CASES[name][0]())
    assert np.array_equal(codec.decode(codec.encode(x)), x)


def test_all_patterns_roundtrip_many_orders():
    rng = np.random.default_rng(7)
    for _ in range(4):
        x = rng.permutation(65536).astype(np.uint16).reshape(8, 64, 1, 128)
        assert np.array_equal(codec.decode(codec.encode(x)), x)


# ---------------------------------------------------------------- closed forms

def test_all_zero_page():
    c = codec.encode(np.zeros((1, 32, 2, 128), np.uint16))
    for k in ("sm", "code", "base", "rowmask", "rowoff"):
        assert not c[k].any(), k
    assert c["raw"].shape == (0, 128)


def test_constant_page():
    # 1.5 = 0x3FC0: exponent 127, sign|mantissa byte 0x40; window floor 112, code 15
    c = codec.encode(np.full((1, 16, 1, 128), 0x3FC0, np.uint16))
    assert (c["sm"] == 0x40).all() and (c["code"] == 0xFF).all() and (c["base"] == 112).all()
    assert c["rowmask"].item() == 0 and c["raw"].shape[0] == 0


def test_inf_nan_make_every_row_raw():
    x = np.full((1, 16, 1, 128), 0x3F80, np.uint16)          # 1.0
    x[0, 5, 0, 9] = 0x7F80                                     # +inf: exponent 255 -> floor 240 >= 128
    c = codec.encode(x)
    assert c["rowmask"].item() == 0xFFFF and c["raw"].shape[0] == 16
    assert c["base"][0, 0, 0, 9] == 240
    x[0, 6, 0, 9] = 0                                          # + a zero in the same group: 240 + 128 -> 255
    assert codec.encode(x)["base"][0, 0, 0, 9] == 255


def test_lone_zero_sets_flag_and_equal_floor_escapes():
    x = np.full((1, 16, 1, 128), 0x3F80, np.uint16)           # exponent 127
    x[0, 3, 0, 0] = 0x0000                                     # zero in a group with floor 112
    c = codec.encode(x)
    assert c["base"][0, 0, 0, 0] == 112 + 128 and c["rowmask"].item() == 0
    assert c["code"][0, 3, 0, 0] & 15 == 0
    x[0, 4, 0, 0] = 112 << 7                                   # exponent == floor in a zero group: code 0 taken
    c = codec.encode(x)
    assert c["rowmask"].item() == 1 << 4


def test_small_exponents_no_zero_flag():
    # all exponents <= 15: floor 0, zeros are ordinary code 0 values, no flag
    x = (np.arange(16, dtype=np.uint16)[None, :, None, None] << 7).repeat(128, 3)
    c = codec.encode(x)
    assert (c["base"] == 0).all() and c["rowmask"].item() == 0


# ---------------------------------------------------------------- brute force per group

def test_escape_iff_no_code_decodes():
    """An element is escaped exactly when no 4-bit code decodes to its exponent under the
    chosen base byte; a non-escaped element's stored code decodes to it."""
    rng = np.random.default_rng(11)
    x = u16(cases.CASES["stress"][0]())
    B, T, H, D = x.shape
    c = codec.encode(x)
    e, sm = codec.split_fields(x)
    base = np.repeat(c["base"], 16, axis=1).astype(np.int32)
    cb = c["code"].astype(np.int32)
    nib = np.concatenate([cb & 15, cb >> 4], axis=-1)
    allc = np.arange(16)
    dec_e = (base[..., None] & 127) + allc                                      # [..., 16 codes]
    dec_e = np.where((base[..., None] >= 128) & (allc == 0), 0, dec_e)
    representable = (dec_e == e[..., None]).any(-1)
    floor, _, _, fits = codec.group_codes(e.reshape(B, T // 16, 16, H, D).transpose(0, 1, 3, 2, 4))
    fits = fits.transpose(0, 1, 3, 2, 4).reshape(B, T, H, D)
    high = np.repeat(floor, 16, axis=1) >= 128          # window floor >= 128: the whole group escapes
    assert high.any() and (~high).any()
    assert not fits[high].any()
    assert np.array_equal(fits[~high], representable[~high])
    stored = (base & 127) + nib
    stored = np.where((base >= 128) & (nib == 0), 0, stored)
    assert np.array_equal(stored[fits], e[fits])
    # rows: raw iff any element of the row does not fit
    rm = c["rowmask"]
    row_raw = ~fits.all(-1)
    got = ((rm[:, :, :, None] >> np.arange(16)) & 1).astype(bool).transpose(0, 1, 3, 2).reshape(B, T, H)
    assert np.array_equal(got, row_raw)
    assert rng is not None


def test_window_floor_bruteforce():
    """base byte and codes against a brute-force search of the format rule on random groups."""
    rng = np.random.default_rng(5)
    for _ in range(300):
        top = int(rng.choice([0, 3, 15, 16, 40, 127, 128, 142, 143, 200, 255]))
        e = rng.integers(max(0, top - 20), top + 1, size=16)
        e[0] = top
        if rng.random() < 0.4:
            e[rng.integers(0, 16)] = 0
        floor, zflag, code, fits = codec.group_codes(e.reshape(16, 1))
        f = max(int(e.max()) - 15, 0)
        zf = bool((e == 0).any()) and f > 0
        assert floor[0] == f and zflag[0] == zf
        for i, ei in enumerate(e):
            if zf and ei == 0:
                ok = f < 128
            else:
                ok = f < 128 and (ei - f) >= (1 if zf else 0)
            assert fits[i, 0] == ok


# ---------------------------------------------------------------- attention oracle

def _rand_case(B, T, Hq, Hkv, seed):
    g = torch.Generator().manual_seed(seed)
    TS = -(-T // 16) * 16
    scale = torch.exp(torch.randn(Hkv, 128, generator=g) * 0.7)
    k = (torch.randn(B, TS, Hkv, 128, generator=g) * scale).to(torch.bfloat16)
    v = torch.randn(B, TS, Hkv, 128, generator=g).to(torch.bfloat16)
    q = (torch.randn(B, Hq, 128, generator=g) * 0.3).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("B,T,Hq,Hkv", [(1, 300, 28, 4), (2, 77, 32, 8), (2, 33, 8, 8), (1, 17, 16, 2)])
def test_attention_oracle_vs_torch_sdpa(B, T, Hq, Hkv):
    q, k, v = _rand_case(B, T, Hq, Hkv, seed=B * 1000 + T)
    G = Hq // Hkv
    kf = k[:, :T].double().repeat_interleave(G, 2).permute(0, 2, 1, 3)
    vf = v[:, :T].double().repeat_interleave(G, 2).permute(0, 2, 1, 3)
    ref = torch.nn.functional.scaled_dot_product_attention(q.double()[:, :, None], kf, vf)[:, :, 0]
    got = oatt.attention(u16(q), u16(k), u16(v), T, np.float64)
    assert np.abs(got - ref.numpy()).max() < 1e-12


def test_attention_closed_forms():
    B, T, Hq, Hkv = 1, 40, 4, 2
    q, k, v = _rand_case(B, T, Hq, Hkv, 3)
    kc = torch.zeros_like(k)                                   # equal keys: output = mean of values
    out = oatt.attention(u16(q), u16(kc), u16(v), T, np.float64)
    mean = v[:, :T].double().mean(1).repeat_interleave(Hq // Hkv, 1)
    assert np.abs(out - mean.numpy()).max() < 1e-12
    kh = torch.zeros_like(k)                                   # one key aligned with q, far above the rest
    kh[0, 7, 0] = (q[0, 0].float() * 1000).to(torch.bfloat16)
    out = oatt.attention(u16(q), u16(kh), u16(v), T, np.float64)
    assert np.abs(out[0, 0] - v[0, 7, 0].double().numpy()).max() < 1e-6


@pytest.mark.parametrize("split_len", [32, 64, 96, 1024])
def test_split_merge_invariance(split_len):
    """Any split of the tokens merges to the unsplit result (exact p, fp32)."""
    B, T, Hq, Hkv = 2, 200, 8, 2
    q, k, v = _rand_case(B, T, Hq, Hkv, 9)
    one = oatt.split_attention(u16(q), u16(k), u16(v), T, split_len=1 << 20, round_p=False)
    many = oatt.split_attention(u16(q), u16(k), u16(v), T, split_len=split_len, round_p=False)
    assert np.abs(one - many).max() < 1e-5
    exact = oatt.attention(u16(q), u16(k), u16(v), T, np.float64)
    assert np.abs(many - exact).max() < 1e-5


def test_split_model_within_reference_bound():
    """With p rounded to bf16 (the reference algorithm) the result stays within the
    reference's 2e-2 absolute fp64 bound (tests/test_exactkv.py:75-78)."""
    B, T, Hq, Hkv = 2, 500, 32, 8
    q, k, v = _rand_case(B, T, Hq, Hkv, 13)
    got = oatt.split_attention(u16(q), u16(k), u16(v), T, split_len=128)
    exact = oatt.attention(u16(q), u16(k), u16(v), T, np.float64)
    assert np.abs(got - exact).max() < 2e-2


def test_choose_split_closed_forms():
    # reference launch math (kernels.py:273-277) at the benchmark shapes
    assert oatt.choose_split(8, 8, 8192, 64) == (8, 1024)
    assert oatt.choose_split(1, 8, 131072, 64) == (64, 2048)
    assert oatt.choose_split(1, 4, 32768, 64) == (128, 256)
    assert oatt.choose_split(32, 8, 4096, 64) == (2, 2048)
    assert oatt.choose_split(4, 2, 17, 64) == (1, 64)


def test_bf16_rounding_helpers():
    f = np.array([1.0, 1.00390625, 1.01171875, -2.5, 0.0, np.inf], np.float32)
    b = oatt.f32_to_bf16(f)
    assert list(b) == [0x3F80, 0x3F80, 0x3F82, 0xC020, 0, 0x7F80]   # ties to even
    assert np.array_equal(oatt.bf16_to_f32(b)[[0, 3]], np.array([1.0, -2.5], np.float32))


# ---------------------------------------------------------------- cache protocol model

def test_cache_model_prefill_equals_codec():
    x = u16(cases.CASES["mixed"][0]())[:, :256]                       # [2, 256, 4, 128]
    m = ocache.CacheModel(2, 256, 4, reserve=1.0)
    for b in range(2):
        m.prefill_slot(b, x[b])
    c = codec.encode(x)
    for k in ("sm", "code", "base", "rowmask", "rowoff"):
        assert np.array_equal(getattr(m, k), c[k]), k
    assert np.array_equal(m.raw[: m.cnt], c["raw"])


def test_cache_model_append_growth_stays_exact():
    rng = np.random.default_rng(2)
    B, H, T0, TS = 2, 4, 100, 208

    def make(n):
        x = torch.from_numpy(rng.standard_normal((B, n, H, 128)).astype(np.float32)).to(torch.bfloat16)
        sel = torch.from_numpy(rng.random((B, n, H)) < 0.1)
        x[sel, 7] = 1e-30
        return u16(x)
    m = ocache.CacheModel(B, TS, H, reserve=0.001)
    ref = np.zeros((B, TS, H, 128), np.uint16)
    x0 = make(T0)
    for b in range(B):
        m.prefill_slot(b, x0[b])
        ref[b, :T0] = x0[b]
    xs = make(TS - T0)
    for t in range(TS - T0):
        m.append(xs[:, t])
        ref[:, T0 + t] = xs[:, t]
        m.check_overflow()
        assert m.cap - m.cnt >= B * H * 16 or m.T == TS
        if t % 13 == 0 or t == TS - T0 - 1:
            assert np.array_equal(codec.decode(m.buffers(), m.T), ref[:, : m.T]), t
    assert m.grows > 0


def test_tolerance_bound_rejects_plausible_mistakes():
    """The accuracy gate used on the GPU output must fail for a dropped token, a wrong head
    and a missing bf16 rounding of p is within it."""
    B, T, Hq, Hkv = 1, 300, 8, 2
    q, k, v = _rand_case(B, T, Hq, Hkv, 17)
    ref = oatt.attention(u16(q), u16(k), u16(v), T, np.float32)
    model = oatt.split_attention(u16(q), u16(k), u16(v), T, split_len=64)
    out = oatt.bf16_to_f32(oatt.f32_to_bf16(model))
    assert oatt.tolerance_excess(out, ref) <= 0
    dropped = oatt.attention(u16(q), u16(k)[:, 1:], u16(v)[:, 1:], T - 1, np.float32)
    assert oatt.tolerance_excess(dropped, ref) > 0
    swapped = ref[:, ::-1]
    assert oatt.tolerance_excess(swapped, ref) > 0


# ---------------------------------------------------------------- bits_per_value

@pytest.mark.parametrize("name", [n for n, (_, stored) in cases.CASES.items() if stored])
def test_bits_per_value_closed_form(golden, name):
    """bits_per_value (reference codec.py:76-78) on the reference-written buffers: with N raw
    rows over B*T*H rows of D values it is 8 * (D + D/2 + D/16 + 0.5 + 2 D N / (B T H)) / D
    = 12.5 + 4 / D + 16 N / (B T H) (12.53125 + ... at D = 128): a page's 16 sm rows, 16
    code rows, one base row and two int32 per head, plus 2 D bytes per raw row."""
    from exactkv_amd.codec import bits_per_value
    z, _ = golden
    c = {k: torch.from_numpy(np.ascontiguousarray(z[f"{name}/{k}"])) for k in FIELDS}
    B, T, H, D = c["sm"].shape
    N = c["raw"].shape[0]
    assert D in (64, 128, 256)
    want = 12.5 + 4.0 / D + 16.0 * N / (B * T * H)
    assert bits_per_value(c) == pytest.approx(want, rel=1e-12)
    if name in ("zeros", "constant"):
        assert N == 0 and bits_per_value(c) == 12.53125
    if name == "allpat_identity":
        assert N > 0 and bits_per_value(c) > 12.53125


# ---------------------------------------------------------------- the torch CPU baseline

@pytest.mark.parametrize("name", list(cases.CASES))
def test_torch_codec_matches_reference_vectors(golden, name):
    """oracle.torch_codec (the timed CPU baseline) writes the reference codec's bytes and
    decodes them back exactly."""
    from oracle import torch_codec
    z, h = golden
    make, stored = cases.CASES[name]
    x = make()
    c = torch_codec.encode(x)
    for k in FIELDS:
        a = c[k].contiguous().view(torch.int16).numpy().view(np.uint16) if k == "raw" else c[k].numpy()
        if stored:
            assert np.array_equal(a, z[f"{name}/{k}"]), (name, k)
        else:
            assert _sha(a) == h["cases"][name][k]["sha256"], (name, k)
    assert torch.equal(torch_codec.decode(c).view(torch.int16), x.view(torch.int16)), name


def test_torch_attention_matches_the_oracle():
    from oracle import torch_codec
    g = torch.Generator().manual_seed(11)
    B, T, Hq, Hkv = 2, 77, 12, 3
    q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(B, 80, Hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(B, 80, Hkv, 128, generator=g).to(torch.bfloat16)
    lens = [77, 40]
    got = torch_codec.attention(q, k, v, T, lens=lens).numpy()
    want = oatt.attention(u16(q), u16(k), u16(v), T, np.float64, lens=lens)
    assert np.abs(got - want).max() < 1e-5
