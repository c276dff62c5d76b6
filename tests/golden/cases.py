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
}
