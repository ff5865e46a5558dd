"""Writes the committed golden fixtures of tests/golden/ (run from the repo root:
`python -m tests.golden.make_golden`). Expected outputs come from the independent numpy restatements in
the tests (not from the C oracle), so the fixtures check the oracle and the GPU path alike."""
import os

import numpy as np

from kern_amd import workload as wl
from tests.test_oracle_quant import numpy_quant

HERE = os.path.dirname(os.path.abspath(__file__))


def quant_fixture():
    x = wl.activations_bf16(2024, 16, 256, outlier_frac=0.02)
    f = wl.bf16_bits_to_f32(x).astype(np.float64)
    f *= np.exp2(np.linspace(-130, 100, 16))[:, None]
    f[3, 5] = 1.875 * 2.0**4      # saturating block
    f[4, 32:64] = 0.0             # zero block
    f[5, 64] = 1.75               # exactly 448 after scaling
    x = wl.f32_to_bf16_bits(f.astype(np.float32))
    q, sf = numpy_quant(x)
    np.savez_compressed(os.path.join(HERE, "mxfp8_quant.npz"), x_bf16=x, q=q, sf=sf)


if __name__ == "__main__":
    quant_fixture()
    print("wrote", os.listdir(HERE))
