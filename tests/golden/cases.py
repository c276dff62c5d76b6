"""Deterministic codec inputs shared by the golden-vector writer and the tests.

Each case maps to (make() -> bf16 CPU tensor [B, T, H, D], store_bytes). Small cases
store their bytes in codec_vectors.npz; large ones store sha256 digests and are
regenerated here from fixed seeds (torch CPU generator / explicit construction).
"""
import math

import numpy as np
import torch

from exactkv_amd.synthetic import _bf16_bits, all_bf16_patterns, make_kv, stress_pages


def _mixed():
    # the reference test's mixed recipe (tests/test_exactkv.py:33-41) on a numpy stream
    rng = np.random.Generator(np.random.PCG64(0))
    scale = np.array([math.exp(z) for z in rng.standard_normal(4 * 128).tolist()], np.float32).reshape(4, 128)
    scale[0, 5] = 300.0
    xf = rng.standard_normal((2, 512, 4, 128), dtype=np.float32) * scale
    x = torch.from_numpy(_bf16_bits(xf).astype(np.int16)).view(torch.bfloat16)
    x[0, 7, 1, 3] = 0.0
    x[1, 9, 2, 5] = -0.0
    x[1, 100, 2, :] = 1e-30
    x[0, 200, 3, 64] = float("inf")
    x[1, 300, 0, 1] = float("nan")
    return x


def _mixed_small():
    x = _mixed()[:, :32].contiguous()
    x[0, 17, 2, 70] = float("-inf")
    x[1, 20, 1, 0] = 0.0
    return x


def _mixed_dim(D, seed):
    # lognormal channel scales with one huge channel, signed zeros, a tiny row, inf and nan,
    # at head dim D: channels on both sides of D/2 carry the specials
    rng = np.random.Generator(np.random.PCG64(seed))
    scale = np.array([math.exp(z) for z in rng.standard_normal(2 * D).tolist()], np.float32).reshape(2, D)
    scale[1, D // 2 + 3] = 500.0
    xf = rng.standard_normal((1, 48, 2, D), dtype=np.float32) * scale
    x = torch.from_numpy(_bf16_bits(xf).astype(np.int16)).view(torch.bfloat16)
    x[0, 3, 0, 1] = 0.0
    x[0, 5, 1, D // 2] = -0.0
    x[0, 20, 1, :] = 1e-30
    x[0, 33, 0, D - 1] = float("inf")
    x[0, 40, 1, D // 2 - 1] = float("nan")
    return x


CASES = {
    "allpat_identity": (lambda: all_bf16_patterns("identity"), True),
    "allpat_perm": (lambda: all_bf16_patterns("perm", seed=0), False),
    "constant": (lambda: torch.full((1, 64, 2, 128), 1.5, dtype=torch.bfloat16), True),
    "zeros": (lambda: torch.zeros(1, 64, 2, 128, dtype=torch.bfloat16), True),
    "stress": (lambda: stress_pages(2, 64, 2, seed=3), True),
    "mixed_small": (_mixed_small, True),
    "mixed": (_mixed, False),
    "c0_keys": (lambda: make_kv(1, 4096, 4, kind="k", seed=0), False),
    "c0_values": (lambda: make_kv(1, 1024, 4, kind="v", seed=1), False),
    # other head dims (the code byte pairs channel j with j + D/2)
    "d64_stress": (lambda: stress_pages(2, 64, 3, D=64, seed=5), True),
    "d256_stress": (lambda: stress_pages(1, 64, 2, D=256, seed=6), True),
    "d64_mixed": (lambda: _mixed_dim(64, seed=9), True),
    "d256_mixed": (lambda: _mixed_dim(256, seed=10), True),
    "d64_keys": (lambda: make_kv(2, 1024, 2, D=64, kind="k", seed=7, raw_row_rate=0.01), False),
    "d256_values": (lambda: make_kv(1, 512, 4, D=256, kind="v", seed=8, raw_row_rate=0.01), False),
}
