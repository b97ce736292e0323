"""Write golden vectors for the weight encoders by running the reference encoder itself.

The exact bytes of ggml Q8_0 / Q4_K blocks depend on numpy's rounding (np.rint /
np.round are half-to-even) and on its float32 -> float16 cast, which no closed form
in the reference pins. This script imports ``quant_q8_0`` and ``quant_q4_k`` from the
reference's ``tools/convert_to_gguf.py`` (lines 68-124) — in the build container only,
where the reference tree exists — and stores seeded inputs with the bytes it produces.
The GPU box never runs this; tests read the committed ``quant_golden.npz``.

Usage: python tests/golden/make_golden.py [/path/to/reference]
"""
from __future__ import annotations

import os
import sys

import numpy as np


def inputs():
    rng = np.random.default_rng(20261201)
    # ---- Q8_0: [N=8, K=256] ----
    q8 = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
    q8[1, 0:32] = 0.0                                    # all-zero block -> d = 0
    q8[1, 32:64] = np.arange(32, dtype=np.float32) - 15.5     # amax 16.5; x/d ties? (generic)
    blk = np.zeros(32, np.float32)
    blk[0] = 127.0                                        # d = 1 exactly
    blk[1:12] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5, 126.5, -126.5, 63.5],
                         np.float32)                      # exact .5 ties -> half-to-even
    q8[1, 64:96] = blk
    q8[2, 0:32] = 1e-6 * rng.standard_normal(32).astype(np.float32)   # fp16(d) underflows
    q8[2, 32:64] = -5.0                                   # constant negative block
    q8[2, 64:96] = 0.0
    q8[2, 64] = -3.0                                       # single spike
    q8[3, :] = (rng.standard_normal(256) * 40.0).astype(np.float32)  # large magnitudes
    # ---- Q4_K: [N=4, K=512] ----
    q4 = (rng.standard_normal((4, 512)) * 0.02).astype(np.float32)
    q4[1, 0:256] = 0.0                                   # all-zero super-block
    q4[1, 256:512] = np.abs(q4[1, 256:512]) + 0.01        # all positive: dmin = 0
    q4[2, 0:256] = -np.abs(q4[2, 0:256]) - 0.01           # all negative
    q4[2, 256:288] = np.linspace(-1.0, 1.0, 32, dtype=np.float32)
    q4[3, :] = (rng.standard_normal(512) * 3.0).astype(np.float32)
    return q8, q4


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, os.path.join(ref, "tools"))
    from convert_to_gguf import quant_q4_k, quant_q8_0  # noqa: E402  (reference encoder)

    q8, q4 = inputs()
    q8_out = np.frombuffer(quant_q8_0(q8), np.uint8).reshape(q8.shape[0], -1)
    q4_out = np.frombuffer(quant_q4_k(q4), np.uint8).reshape(q4.shape[0], -1)
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_golden.npz")
    np.savez_compressed(dst, q8_in=q8, q8_out=q8_out, q4_in=q4, q4_out=q4_out,
                        numpy_version=np.array(np.__version__))
    print(f"wrote {dst}: q8 {q8_out.shape} q4 {q4_out.shape} (numpy {np.__version__})")


if __name__ == "__main__":
    main()
