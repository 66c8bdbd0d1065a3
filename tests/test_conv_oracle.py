"""Pins the oracle's W8A8 convolution (orc_conv2d_i8) before it checks the GPU.

  * bit-exact against the reference's own conv2d_i8 (src/hal/common/conv.cpp
    :424-526, compiled from its sources into oracle/_ref, weights packed by its
    pack_weights_i8), at a ResNet stem (7x7 stride 2 over 3 channels), a 3x3
    block, a 1x1 stride-2 downsample and ragged shapes, and with
    TCPU_I8_CLIP < 1 (the reference reads it once per process, so that case
    runs in a child process);
  * the im2col layout against what the mathematics fixes: a direct per-tap
    convolution of the quantized input in int64 equals the int32 GEMM over the
    im2col rows;
  * the per-tensor scale closed form: s = max|x| * clip / 127, zero input ->
    s = 1 and all-zero bytes, and a planted mistake (a transposed tap order)
    is caught.
"""

import os
import subprocess
import sys

import numpy as np
import pytest

from helpers import oracle, same_bits

ob = oracle()

# (H, Wd, Cin, Cout, k, stride, pad)
SHAPES = [(32, 40, 3, 64, 7, 2, 3), (16, 16, 64, 64, 3, 1, 1), (16, 12, 64, 128, 1, 2, 0),
          (9, 13, 5, 16, 3, 2, 1), (2, 2, 4, 16, 3, 1, 1), (20, 20, 32, 32, 5, 3, 2)]


def _case(shape, seed=3):
    H, Wd, Cin, Cout, k, s, p = shape
    r = np.random.default_rng(seed + H * 131 + Cin)
    x = r.normal(0.0, 1.0, (H, Wd, Cin)).astype(np.float32)
    W = r.uniform(-0.2, 0.2, (Cout, k, k, Cin)).astype(np.float32)
    b = r.normal(0.0, 0.02, Cout).astype(np.float32)
    return x, W, b


@pytest.mark.skipif(not ob.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("shape", SHAPES)
def test_conv2d_i8_matches_reference_build(shape):
    H, Wd, Cin, Cout, k, s, p = shape
    x, W, b = _case(shape)
    Wq, ws = ob.quantize_weights_i8(W.reshape(Cout, -1))
    got = ob.conv2d_i8(x, Wq, ws, b, k, s, p)
    want = ob.ref_conv2d_i8(x, W, b, k, s, p)
    assert got.shape == want.shape
    assert same_bits(got, want), "oracle conv2d_i8 differs from the reference build"


@pytest.mark.parametrize("shape", SHAPES)
def test_im2col_equals_direct_convolution(shape):
    H, Wd, Cin, Cout, k, s, p = shape
    x, W, b = _case(shape)
    xq, sa = ob.quantize_tensor_i8(x)
    Wq, _ = ob.quantize_weights_i8(W.reshape(Cout, -1))
    K = k * k * Cin
    col = ob.im2col_i8(xq, k, s, p)
    acc = ob.gemm_i8_acc(col, Wq, K)
    Ho, Wo = ob.conv_out(H, Wd, k, s, p)
    xp = np.zeros((H + 2 * p + k, Wd + 2 * p + k, Cin), np.int64)
    xp[p:p + H, p:p + Wd] = xq
    w4 = Wq[:, :K].reshape(Cout, k, k, Cin).astype(np.int64)
    direct = np.zeros((Ho, Wo, Cout), np.int64)
    for ky in range(k):
        for kx in range(k):
            tap = xp[ky:ky + s * Ho:s, kx:kx + s * Wo:s][:Ho, :Wo]     # [Ho, Wo, Cin]
            direct += np.einsum("hwc,oc->hwo", tap, w4[:, ky, kx, :])
    assert np.array_equal(acc.reshape(Ho, Wo, Cout).astype(np.int64), direct)


def test_tensor_scale_closed_form_and_zero_input():
    r = np.random.default_rng(7)
    x = r.normal(0, 3, (5, 6, 7)).astype(np.float32)
    for clip in (1.0, 0.5, 0.25):
        q, s = ob.quantize_tensor_i8(x, clip)
        amax = np.float32(np.abs(x).max())
        assert s == np.float32(np.float32(amax * np.float32(clip)) / np.float32(127.0))
        inv = np.float32(1.0) / s
        want = np.clip(np.rint(x * inv), -127, 127).astype(np.int8)
        assert np.array_equal(q, want)
    q, s = ob.quantize_tensor_i8(np.zeros((3, 3, 2), np.float32))
    assert s == np.float32(1.0) and not q.any()


def test_planted_tap_order_mistake_is_caught():
    """The check above fails for an im2col with kx and ky swapped."""
    shape = (9, 13, 5, 16, 3, 2, 1)
    H, Wd, Cin, Cout, k, s, p = shape
    x, W, _ = _case(shape)
    xq, _ = ob.quantize_tensor_i8(x)
    col = ob.im2col_i8(xq, k, s, p)
    K = k * k * Cin
    swapped = col[:, :K].reshape(-1, k, k, Cin).transpose(0, 2, 1, 3).reshape(-1, K)
    Wq, _ = ob.quantize_weights_i8(W.reshape(Cout, -1))
    assert not np.array_equal(ob.gemm_i8_acc(swapped, Wq, K), ob.gemm_i8_acc(col, Wq, K))


@pytest.mark.skipif(not ob.ref_available(), reason="oracle/_ref not built")
def test_conv2d_i8_clip_matches_reference_build():
    code = (
        "import sys, numpy as np\n"
        "sys.path.insert(0, %r)\n"
        "from helpers import oracle, same_bits\n"
        "from test_conv_oracle import _case, SHAPES\n"
        "ob = oracle()\n"
        "for shape in SHAPES[:4]:\n"
        "    H, Wd, Cin, Cout, k, s, p = shape\n"
        "    x, W, b = _case(shape)\n"
        "    Wq, ws = ob.quantize_weights_i8(W.reshape(Cout, -1))\n"
        "    got = ob.conv2d_i8(x, Wq, ws, b, k, s, p, clip=0.6)\n"
        "    assert same_bits(got, ob.ref_conv2d_i8(x, W, b, k, s, p)), shape\n"
        "print('ok')\n" % os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, TCPU_I8_CLIP="0.6")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]
