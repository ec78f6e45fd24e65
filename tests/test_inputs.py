"""The product's seeded input generator (example_matmul_metal4_amd.inputs, used by bench.py)
follows the same SplitMix64 recipe as the test oracle's generator."""
import numpy as np

import oracle
from example_matmul_metal4_amd import inputs


def test_uniform_streams_identical():
    for dtype in ("f16", "bf16"):
        a = inputs.uniform(17, (3, 1000), -1.0, 1.0, dtype)
        b = oracle.uniform(17, (3, 1000), -1.0, 1.0, dtype)
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_normal_streams_agree():
    for dtype in ("f16", "bf16"):
        a = inputs.normal(5, (4097,), 0.0, 0.02, dtype).view(np.uint16)
        b = oracle.normal(5, (4097,), 0.0, 0.02, dtype).view(np.uint16)
        # vectorised vs scalar libm may differ in the last bit of log/cos/sin for rare inputs
        assert np.mean(a == b) > 0.999
