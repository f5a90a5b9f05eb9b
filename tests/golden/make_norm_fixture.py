"""Writes tests/golden/zcrmsnorm_fixture.npz from go-whistle's own fixture
testdata/needle/zcrmsnorm.safetensors (upstream's ZCRMSNorm(eps=1e-6) and
_rms_unit at float32, Whistle's layer 0): the input x, the row divisors rms
and rms_unit, the tensors that need no weight (y needs the norm's scale,
which the fixture does not hold). Read with the safetensors loader.

Run from the repository root: python tests/golden/make_norm_fixture.py
"""

import os

import numpy as np
from safetensors import safe_open

SRC = "/root/reference/testdata/needle/zcrmsnorm.safetensors"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "zcrmsnorm_fixture.npz")


def main():
    with safe_open(SRC, framework="numpy") as f:
        assert f.metadata()["eps"] == "1e-6"
        out = {k: f.get_tensor(k).astype(np.float32) for k in ("x", "rms", "rms_unit")}
    np.savez_compressed(OUT, **out)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
