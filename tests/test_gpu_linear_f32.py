"""GPU parity of the fp32 linear (dense_linear, src/ops/lm_ops.h:81-84): the
layers a graph's int8 mask leaves in fp32 (ACT's state projection and action
head, SmolVLA's flow-matching projections, Octo's token projections).

fp32 sums in another order than the reference, so the bar is a tolerance:
1e-5 of max(|ref|) against the float64 product and against the reference's
own dense_linear (oracle/_ref). Shapes cover the split-K kernel (M <= 128),
the double-buffered tiled one (M > 128, 16-byte aligned rows) and the scalar
tiled one (rows not a multiple of 4 floats), and the BASELINE layers.
"""

import numpy as np
import pytest

from helpers import load_synth

pytestmark = pytest.mark.gpu

SHAPES = [  # (M, K, N)
    (1, 14, 512), (100, 512, 14), (50, 32, 720), (50, 1440, 720), (50, 720, 32), (1, 960, 960),
    (16, 17, 33), (17, 64, 16), (63, 100, 70), (64, 256, 48), (65, 96, 80), (128, 512, 64),
    (129, 512, 64), (300, 512, 768), (256, 768, 768),
    # the double-buffered tiled kernel (M > 128, aligned rows): ResNet conv
    # GEMMs, a ragged K slab (K % 32 != 0), N and M edges, 128-row tiles
    (19200, 576, 64), (1200, 2304, 256), (513, 100, 130), (4800, 64, 128),
    # few tiles over a long K: row tiles of the split-K kernel
    (300, 4608, 512), (300, 2304, 200), (150, 1152, 64),
]


def _case(M, K, N):
    s = load_synth()
    x = s.normal(f"lf.x.{M}.{K}", (M, K))
    W = s.uniform(f"lf.w.{K}.{N}", (N, K), -1.0 / np.sqrt(K), 1.0 / np.sqrt(K))
    b = s.normal(f"lf.b.{N}", (N,), 0.02)
    return x, W, b


def _rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got))
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_dense_linear(vla, M, K, N):
    from helpers import oracle
    x, W, b = _case(M, K, N)
    got = vla.dense_linear(x, W, b)
    exact = x.astype(np.float64) @ W.astype(np.float64).T + b
    assert _rel(got, exact) <= 1e-5
    ob = oracle()
    if ob.ref_available():
        assert _rel(got, ob.ref_dense_linear(x, W, b)) <= 1e-5
    nob = vla.dense_linear(x, W, None)
    assert _rel(nob, x.astype(np.float64) @ W.astype(np.float64).T) <= 1e-5


@pytest.mark.parametrize("M,K,N", [(50, 720, 32), (50, 1440, 720), (300, 512, 768)])
def test_dense_linear_dev_epilogues(vla, torch_cuda, M, K, N):
    torch = torch_cuda
    x, W, b = _case(M, K, N)
    dx, dW, db = (torch.from_numpy(a).cuda() for a in (x, W, b))
    exact = x.astype(np.float64) @ W.astype(np.float64).T + b
    # silu epilogue (action_time_mlp_in)
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    vla.dense_linear_dev(out, dx, dW, db, act=4)
    torch.cuda.synchronize()
    assert _rel(out.cpu().numpy(), exact / (1.0 + np.exp(-exact))) <= 1e-5
    # Euler step: out = fmaf(alpha, result, out)
    base = load_synth().normal(f"lf.base.{M}.{N}", (M, N))
    out = torch.from_numpy(base.copy()).cuda()
    vla.dense_linear_dev(out, dx, dW, db, accumulate=1, alpha=-0.1)
    torch.cuda.synchronize()
    assert _rel(out.cpu().numpy(), base + (-0.1) * exact) <= 1e-5


@pytest.mark.parametrize("groups", ["1", "2", "3", "8"])
@pytest.mark.parametrize("M,K,N", [(50, 1440, 720), (100, 512, 14), (128, 512, 64), (17, 64, 16)])
def test_skinny_row_groups_identical(vla, groups, M, K, N):
    """Row groups of the M <= 128 kernel (16 x FM rows per block) leave every
    output's sum unchanged: identical to one group, and within the bar."""
    import os
    x, W, b = _case(M, K, N)
    os.environ["VLA_HIP_SKINNY_R"] = "1"
    try:
        one = vla.dense_linear(x, W, b)
        os.environ["VLA_HIP_SKINNY_R"] = groups
        got = vla.dense_linear(x, W, b)
    finally:
        del os.environ["VLA_HIP_SKINNY_R"]
    assert np.array_equal(got.view(np.uint32), one.view(np.uint32))
    assert _rel(got, x.astype(np.float64) @ W.astype(np.float64).T + b) <= 1e-5
