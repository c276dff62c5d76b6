"""Write the codec golden vectors by running the reference codec on the CPU.

The reference's encoder output for rows that are stored raw (their clamped codes),
the base-byte saturation and the zero-flag condition are not fixed by the round-trip
property, so they are pinned by vectors that the reference codec itself produced:
exactkv/codec.py (encode_reference, codec.py:31-55) is imported by file path from the
reference checkout -- only that file, on the CPU; it needs nothing but torch.

Outputs (committed, data only):
  codec_vectors.npz   inputs and all six encoded tensors for the small cases
  codec_hashes.json   sha256 of inputs and encoded tensors for the larger cases,
                      whose inputs are regenerated from seeds by the tests

Run from the repo root:  python tests/golden/make_codec_vectors.py
"""
import hashlib
import importlib.util
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", ".."))
from tests.golden import cases  # noqa: E402

REF_CODEC = "/root/reference/exactkv/codec.py"
FIELDS = ("sm", "code", "base", "rowmask", "rowoff", "raw")


def load_reference_codec():
    spec = importlib.util.spec_from_file_location("reference_codec", REF_CODEC)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def as_np(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.contiguous().numpy()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    ref = load_reference_codec()
    arrays, hashes = {}, {}
    for name, (make, store_bytes) in cases.CASES.items():
        x = make()
        c = ref.encode_reference(x)
        out = {k: as_np(c[k]) for k in FIELDS}
        out["input"] = as_np(x)
        if store_bytes:
            for k, v in out.items():
                arrays[f"{name}/{k}"] = v
        else:
            hashes[name] = {k: dict(sha256=sha(v), shape=list(v.shape), dtype=str(v.dtype)) for k, v in out.items()}
            # page metadata is small: keep it as bytes too
            for k in ("rowmask", "rowoff"):
                arrays[f"{name}/{k}"] = out[k]
        print(name, tuple(x.shape), "raw rows:", out["raw"].shape[0], flush=True)
    np.savez_compressed(os.path.join(HERE, "codec_vectors.npz"), **arrays)
    with open(os.path.join(HERE, "codec_hashes.json"), "w") as f:
        json.dump(dict(source="reference exactkv/codec.py encode_reference, CPU", torch=torch.__version__,
                       cases=hashes), f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
