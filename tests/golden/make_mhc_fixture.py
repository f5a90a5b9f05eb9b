"""Writes tests/golden/mhc_fixture.npz from go-whistle's own mHC fixture,
testdata/needle/mhc.safetensors (upstream's Flax mHC of Whistle's layers 0
and 1 at float32, seed 20261014, 20 Sinkhorn iterations; see the fixture
directory's README). Only data is copied: the tensors around the φ
products, which need the model's weights and so are not part of it. Read
with the safetensors loader (no code in the file runs).

Run from the repository root: python tests/golden/make_mhc_fixture.py
"""

import os

import numpy as np
from safetensors import safe_open

SRC = "/root/reference/testdata/needle/mhc.safetensors"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mhc_fixture.npz")
KEYS = ["x"] + [f"layer{l}.{k}" for l in (0, 1) for k in (
    "nx", "h_pre_logits", "h_pre", "h_post_logits", "h_post", "h_res_logits", "h_res", "u", "block_out", "y",
    "stream_out")] + ["layer1.stream_in"]


def main():
    out = {}
    with safe_open(SRC, framework="numpy") as f:
        meta = f.metadata()
        assert meta["lanes"] == "4" and meta["sinkhorn_iters"] == "20", meta
        for k in KEYS:
            out[k.replace(".", "__")] = f.get_tensor(k).astype(np.float32)
    np.savez_compressed(OUT, **out)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
