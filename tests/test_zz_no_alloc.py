"""The allocation-free int8 linear (vla_dense_linear_i8_noalloc_dev) against
the entry point it varies, vla_dense_linear_i8_dev with caller scratch.

Both run the same quantizer and GEMM kernels; the allocation-free form keeps
its activations (panel layout up to 128 rows), scales and split-K partial sums
in the library's fixed device array. Bar: bit-identical outputs (integer
accumulators and one fp32 epilogue expression). Each case is two calls in a
row on the same shared scratch, the second with a smaller input, so stale
bytes of the first call must not leak into the second.
"""

import numpy as np
import pytest

from helpers import same_bits

pytestmark = pytest.mark.gpu

# (first call, second smaller call): (seq, N, K, act, accumulate)
SEQUENCES = [
    ((2048, 960, 2560, 0, 0), (100, 3200, 512, 0, 0)),   # split-K row-major, then panel
    ((100, 4096, 4096, 1, 0), (50, 2560, 960, 2, 1)),    # panel split-K, then panel
    ((302, 3200, 512, 0, 1), (7, 48, 1027, 0, 0)),       # row-major, then unaligned K
    ((128, 1024, 2048, 0, 0), (1, 3200, 512, 1, 1)),     # the largest panel, then one row
]


def _case(rng, seq, N, K):
    x = rng.standard_normal((seq, K)).astype(np.float32)
    Wq = rng.integers(-127, 128, size=(N, (K + 3) & ~3), dtype=np.int8)
    Wq[:, K:] = 0
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    b = (0.02 * rng.standard_normal(N)).astype(np.float32)
    return x, Wq, ws, b


def _run_pair(vla, torch, shape, seed):
    seq, N, K, act, accumulate = shape
    print(f"no-alloc case seq={seq} N={N} K={K} act={act} acc={accumulate}", flush=True)
    rng = np.random.default_rng(seed)
    x, Wq, ws, b = _case(rng, seq, N, K)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    Wd = torch.from_numpy(Wq).to(dev)
    wsd, bd = torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    base = rng.standard_normal((seq, N)).astype(np.float32)
    want = torch.from_numpy(base).to(dev)
    xq = torch.empty((seq, Wq.shape[1]), dtype=torch.int8, device=dev)
    sa = torch.empty(seq, dtype=torch.float32, device=dev)
    vla.dense_linear_i8_dev(want, xd, Wd, wsd, bd, K, xq, sa, act=act, accumulate=accumulate)
    got = torch.from_numpy(base).to(dev)
    vla.dense_linear_i8_noalloc_dev(got, xd, Wd, wsd, bd, K, act=act, accumulate=accumulate)
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


@pytest.mark.parametrize("first,second", SEQUENCES)
def test_noalloc_matches_caller_scratch(vla, torch_cuda, first, second):
    for i, shape in enumerate((first, second)):
        got, want = _run_pair(vla, torch_cuda, shape, seed=1000 * i + shape[0])
        assert same_bits(got, want), f"allocation-free output differs on call {i + 1} {shape}"


def test_noalloc_rejects_oversize(vla, torch_cuda):
    """seq x K beyond the fixed scratch comes back as VLA_ERR_ARG before any launch."""
    torch = torch_cuda
    cap = int(vla.lib().vla_dense_linear_i8_noalloc_max_bytes())
    assert cap == 32 << 20
    seq, K, N = 8193, 4096, 16
    dev = torch.device("cuda")
    x = torch.zeros((seq, K), dtype=torch.float32, device=dev)
    out = torch.zeros((seq, N), dtype=torch.float32, device=dev)
    W = torch.zeros((N, K), dtype=torch.int8, device=dev)
    ws = torch.ones(N, dtype=torch.float32, device=dev)
    st = vla.lib().vla_dense_linear_i8_noalloc_dev(
        vla._dp(out), N, vla._dp(x), K, vla._dp(W), K, vla._dp(ws), None, seq, N, K, 0, 0, vla._stream(None))
    assert st == vla.VLA_ERR_ARG
    assert b"allocation-free scratch" in vla.lib().vla_last_error()
