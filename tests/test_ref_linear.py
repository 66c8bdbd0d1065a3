"""CPU: the reference's fp32 dense_linear binding (oracle/_ref) against the
float64 product, so the GPU tests' second check is pinned."""

import numpy as np
import pytest

from helpers import load_synth, oracle


@pytest.mark.parametrize("M,K,N", [(1, 14, 512), (50, 1440, 720), (17, 33, 20)])
def test_ref_dense_linear_matches_float64(M, K, N):
    ob = oracle()
    if not ob.ref_available():
        pytest.skip("oracle/_ref not built")
    s = load_synth()
    x = s.normal("rl.x", (M, K))
    W = s.normal("rl.w", (N, K), 1.0 / np.sqrt(K))
    b = s.normal("rl.b", (N,), 0.02)
    got = ob.ref_dense_linear(x, W, b)
    exact = x.astype(np.float64) @ W.astype(np.float64).T + b
    assert np.max(np.abs(got - exact)) / np.max(np.abs(exact)) <= 1e-5
    # a dropped bias or a transposed operand fails the same check
    assert np.max(np.abs(ob.ref_dense_linear(x, W, None) - exact)) > 1e-3
