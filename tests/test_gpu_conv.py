"""GPU parity of the W8A8 convolution (vla_conv2d_i8 / _dev).

Bar: bit-exact with the oracle's orc_conv2d_i8 (int8 bytes, int32 sums and the
fp32 epilogue are all exact), which tests/test_conv_oracle.py pins to the
reference's own conv2d_i8 (src/hal/common/conv.cpp:424-526). Shapes: a ResNet
stem (7x7 stride 2 over RGB, the per-byte im2col path), 3x3 blocks and 1x1
stride-2 downsamples (the implicit GEMM over 64-channel multiples, and the
float4 im2col path), ragged sizes, a Cout that is not a
multiple of 16 (the reference requires one; the GPU does not), an all-zero
input (scale 1, output = bias) and repeated calls on one workspace.
"""

import numpy as np
import pytest

from helpers import same_bits

pytestmark = pytest.mark.gpu

# (H, Wd, Cin, Cout, k, stride, pad)
SHAPES = [(224, 224, 3, 64, 7, 2, 3), (56, 56, 64, 64, 3, 1, 1), (56, 56, 64, 128, 1, 2, 0),
          (28, 28, 128, 128, 3, 1, 1), (9, 13, 5, 24, 3, 2, 1), (2, 2, 4, 16, 3, 1, 1),
          (20, 20, 32, 40, 5, 3, 2), (64, 48, 3, 32, 3, 2, 1),
          # ResNet-18's deeper layers (split K over long K, 1x1 stride 2), 16 and
          # 48 channels, N not a multiple of 64, ragged pixel counts
          (15, 20, 512, 512, 3, 1, 1), (30, 40, 256, 512, 1, 2, 0), (17, 23, 16, 48, 3, 1, 1),
          (9, 9, 48, 32, 5, 2, 2), (60, 80, 128, 256, 3, 2, 1), (120, 160, 64, 128, 3, 1, 1)]


def _case(shape, seed=5):
    H, Wd, Cin, Cout, k, s, p = shape
    r = np.random.default_rng(seed + 7 * H + Cin)
    x = r.normal(0.0, 1.0, (H, Wd, Cin)).astype(np.float32)
    W = r.uniform(-0.2, 0.2, (Cout, k, k, Cin)).astype(np.float32)
    b = r.normal(0.0, 0.02, Cout).astype(np.float32)
    return x, W, b


@pytest.mark.parametrize("shape", SHAPES)
def test_conv2d_i8_host_form(vla, orc, shape):
    H, Wd, Cin, Cout, k, s, p = shape
    x, W, b = _case(shape)
    Wq, ws = orc.quantize_weights_i8(W.reshape(Cout, -1))
    print(f"conv host {shape}", flush=True)
    got = vla.conv2d_i8(x, Wq, ws, b, k, s, p)
    want = orc.conv2d_i8(x, Wq, ws, b, k, s, p)
    assert same_bits(got, want), "conv2d_i8 differs from the oracle"


@pytest.mark.parametrize("shape", SHAPES[:5])
def test_conv2d_i8_dev_form(vla, orc, torch_cuda, shape):
    torch = torch_cuda
    H, Wd, Cin, Cout, k, s, p = shape
    x, W, b = _case(shape)
    lin = vla.LinearI8.from_f32(W.reshape(Cout, -1), b)
    Ho, Wo = (H + 2 * p - k) // s + 1, (Wd + 2 * p - k) // s + 1
    n = vla.conv2d_i8_workspace_bytes(H, Wd, Cin, Cout, k, s, p)
    work = torch.empty(n, dtype=torch.uint8, device="cuda")
    xd = torch.from_numpy(x).cuda()
    out = torch.full((Ho, Wo, Cout), 7.0, device="cuda")
    print(f"conv dev {shape}", flush=True)
    vla.conv2d_i8_dev(lin, out, xd, k, s, p, work)
    torch.cuda.synchronize()
    Wq, ws = orc.quantize_weights_i8(W.reshape(Cout, -1))
    assert same_bits(out.cpu().numpy(), orc.conv2d_i8(x, Wq, ws, b, k, s, p))


# the implicit forms (the LDS GEMM tile above 320 pixels, conv_i8_implicit
# for smaller 1x1 maps and, with the LDS form off, for >= 256 output tiles
# of 64 x 64 or 1x1) and the im2col rows: ragged rows and channels, 18 K
# steps; then inputs
# of 1-4 channels, which take the word-per-pixel form (kernels up to 8 x 8,
# strides 1-4, channel counts off the 64-wide block; 30 channels, not a
# multiple of 4, keep the im2col rows)
IMPLICIT_SHAPES = [(128, 128, 64, 64, 3, 1, 1), (30, 40, 256, 512, 1, 2, 0), (161, 203, 64, 48, 5, 3, 2),
                   (131, 121, 128, 100, 3, 1, 1), (33, 29, 64, 36, 1, 1, 0), (15, 20, 512, 512, 3, 1, 1),
                   (20, 20, 128, 100, 3, 2, 1), (56, 56, 64, 64, 3, 1, 1),
                   (224, 224, 3, 64, 7, 2, 3), (97, 131, 1, 20, 5, 1, 2), (33, 47, 2, 36, 3, 2, 1),
                   (40, 30, 4, 72, 7, 3, 3), (50, 50, 3, 16, 8, 4, 2), (64, 48, 3, 30, 3, 2, 1)]


@pytest.mark.parametrize("shape", IMPLICIT_SHAPES)
def test_conv2d_i8_implicit_and_im2col_forms(vla, orc, shape, monkeypatch):
    """Input channels a multiple of 64 take an implicit GEMM (the int8 map
    gathered per tap): over more than 320 pixels the LDS GEMM tile, smaller
    1x1 maps conv_i8_implicit (with VLA_HIP_CONV_LDS_IMPLICIT=0, 1x1 maps and
    those over >= 256 output tiles conv_i8_implicit); 1-4 input channels the
    word-per-pixel form (zero bytes past the channels and past the last tap
    add nothing to the int32 sums); VLA_HIP_CONV_IMPLICIT=0 (read per call)
    forces the im2col rows. All bit-exact with the oracle: ragged output
    tiles (48, 100, 36, 20, 72 channels), pixel counts off the 64-row tile,
    strides 2-4, padding 2-3."""
    H, Wd, Cin, Cout, k, s, p = shape
    x, W, b = _case(shape, seed=11)
    Wq, ws = orc.quantize_weights_i8(W.reshape(Cout, -1))
    want = orc.conv2d_i8(x, Wq, ws, b, k, s, p)
    print(f"conv implicit {shape}", flush=True)
    got = vla.conv2d_i8(x, Wq, ws, b, k, s, p)
    monkeypatch.setenv("VLA_HIP_CONV_LDS_IMPLICIT", "0")
    got_64 = vla.conv2d_i8(x, Wq, ws, b, k, s, p)
    monkeypatch.setenv("VLA_HIP_CONV_IMPLICIT", "0")
    got_im2col = vla.conv2d_i8(x, Wq, ws, b, k, s, p)
    assert same_bits(got, want), "implicit form differs from the oracle"
    assert same_bits(got_64, want), "64 x 64 implicit form differs from the oracle"
    assert same_bits(got_im2col, want), "im2col form differs from the oracle"


# fewer than 256 output tiles over 64-channel multiples: the LDS GEMM tile
# gathering A from the int8 map (above 320 pixels, or at every count with
# VLA_HIP_CONV_LDS_IMPLICIT=all): 192 channels (a 128-byte K slab spanning
# two taps mid-tap), 64 channels (two taps per slab), a ragged last slab
# (K = 4800, 576), pixel counts off the 32-row tile, Cout off the 64-column
# tile, strides 1-3, padding 1-2, and 300- / 81-pixel maps under "all";
# 129-320 pixels take the skinny kernel loading A from the map by default
# (306, 182 and 300 pixels: Cout 48 / 36 off the 16-column block, K steps
# for 8 and 16 waves, a 1x1 stride-2 downsample)
LDS_IMPLICIT_SHAPES = [(41, 37, 192, 100, 5, 2, 2), (60, 70, 64, 36, 3, 3, 2), (56, 56, 64, 64, 3, 1, 1),
                       (60, 80, 128, 256, 3, 2, 1), (30, 40, 256, 256, 3, 1, 1), (15, 20, 512, 512, 3, 1, 1),
                       (9, 9, 64, 32, 3, 1, 1), (33, 35, 64, 48, 5, 2, 2), (25, 27, 192, 36, 3, 2, 1),
                       (30, 40, 256, 512, 1, 2, 0)]


@pytest.mark.parametrize("shape", LDS_IMPLICIT_SHAPES)
def test_conv2d_i8_lds_implicit_form(vla, orc, shape, monkeypatch):
    """The 32 x 64 LDS GEMM tile with A gathered per tap from the int8 map:
    bit-exact with the oracle, with the im2col rows and with
    conv_i8_implicit (VLA_HIP_CONV_LDS_IMPLICIT=0, then with
    VLA_HIP_CONV_IMPLICIT_TILES=0); "all" puts the small maps on it too."""
    H, Wd, Cin, Cout, k, s, p = shape
    x, W, b = _case(shape, seed=13)
    Wq, ws = orc.quantize_weights_i8(W.reshape(Cout, -1))
    want = orc.conv2d_i8(x, Wq, ws, b, k, s, p)
    print(f"conv lds implicit {shape}", flush=True)
    outs = {}
    monkeypatch.setenv("VLA_HIP_CONV_SKINNY_IMPLICIT", "0")
    outs["1, no skinny"] = vla.conv2d_i8(x, Wq, ws, b, k, s, p)
    monkeypatch.delenv("VLA_HIP_CONV_SKINNY_IMPLICIT")
    for mode in ("1", "all", "0"):
        monkeypatch.setenv("VLA_HIP_CONV_LDS_IMPLICIT", mode)
        outs[mode] = vla.conv2d_i8(x, Wq, ws, b, k, s, p)
    monkeypatch.setenv("VLA_HIP_CONV_IMPLICIT_TILES", "0")
    outs["0, 64 x 64 implicit"] = vla.conv2d_i8(x, Wq, ws, b, k, s, p)
    for mode, got in outs.items():
        assert same_bits(got, want), f"VLA_HIP_CONV_LDS_IMPLICIT={mode} differs from the oracle"


def test_conv2d_i8_repeat_and_zero_input(vla, orc, torch_cuda):
    """One workspace, two calls in a row (the second on an all-zero input:
    scale 1, every byte 0, every output the bias), then the first again."""
    torch = torch_cuda
    shape = (56, 56, 64, 64, 3, 1, 1)
    H, Wd, Cin, Cout, k, s, p = shape
    x, W, b = _case(shape)
    lin = vla.LinearI8.from_f32(W.reshape(Cout, -1), b)
    work = torch.empty(vla.conv2d_i8_workspace_bytes(H, Wd, Cin, Cout, k, s, p), dtype=torch.uint8, device="cuda")
    out = torch.empty((H, Wd, Cout), device="cuda")
    Wq, ws = orc.quantize_weights_i8(W.reshape(Cout, -1))
    want = orc.conv2d_i8(x, Wq, ws, b, k, s, p)
    vla.conv2d_i8_dev(lin, out, torch.from_numpy(x).cuda(), k, s, p, work)
    torch.cuda.synchronize()
    assert same_bits(out.cpu().numpy(), want)
    vla.conv2d_i8_dev(lin, out, torch.zeros((H, Wd, Cin), device="cuda"), k, s, p, work)
    torch.cuda.synchronize()
    assert same_bits(out.cpu().numpy(), np.broadcast_to(b, (H, Wd, Cout)))
    vla.conv2d_i8_dev(lin, out, torch.from_numpy(x).cuda(), k, s, p, work)
    torch.cuda.synchronize()
    assert same_bits(out.cpu().numpy(), want)


def test_conv2d_i8_rejects_bad_calls(vla, torch_cuda):
    torch = torch_cuda
    assert vla.conv2d_i8_workspace_bytes(2, 2, 3, 16, 7, 1, 0) == -1      # kernel larger than the input
    assert vla.conv2d_i8_workspace_bytes(8, 8, 3, 16, 3, 0, 1) == -1      # stride 0
    lin = vla.LinearI8.from_f32(np.ones((16, 27), np.float32))
    x = torch.zeros((8, 8, 3), device="cuda")
    out = torch.zeros((8, 8, 16), device="cuda")
    small = torch.empty(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(vla.VlaError) as e:                             # workspace too small
        vla.conv2d_i8_dev(lin, out, x, 3, 1, 1, small)
    assert e.value.status == vla.VLA_ERR_ARG
    with pytest.raises(vla.VlaError) as e:                             # K != k*k*Cin
        vla.conv2d_i8_dev(lin, out, x, 5, 1, 2, small)
    assert e.value.status == vla.VLA_ERR_ARG

