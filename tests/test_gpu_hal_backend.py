"""The reference's own nn layer on the HIP op backend.

vla.simd_amd/hal/ops_hip.cpp implements the reference's op layer
(src/ops/quant_ops.h, lm_ops.h, conv_ops.h) over libvla_simd_hip.so;
oracle/Makefile's ref_hip target compiles it against the reference's headers
and links it with the reference's own nn::Linear, nn::MhaQKV, nn::EncoderLayer
and fp32 GEMM objects into oracle/_ref/libvla_ref_hip.so, exactly as a
maintainer would build the TCPU_HAL_HIP backend. These tests drive that build
(through oracle/ref_nn_shim.cpp) next to the reference's CPU build.

Bars: the reference's own assertions hold on the HIP backend bit for bit
(test_ops.cpp:138-157 dense_linear_i8_pre == dense_linear_i8_ref;
test_ops.cpp:188-220 shared quantization == separate quantization); int8
linears and the q/k/v projections equal the CPU build bit for bit; the
attention output (fp32 softmax, ulp differences between backends) is within
1e-5 of the output scale when wo is fp32, and within a few int8 steps of
the output scale (2e-2) when wo re-quantizes it.
"""

import numpy as np
import pytest

from helpers import same_bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nn(vla):
    from helpers import oracle
    ob = oracle()
    if not ob.ref_hip_available():
        pytest.fail("oracle/_ref/libvla_ref_hip.so is not built (make -C oracle ref_hip)")
    ob.ref_nn("hip")
    return ob


def _rv(fr, n, lo=-1.0, hi=1.0):
    return fr.rv(n, lo, hi)


@pytest.mark.parametrize("seq,N,K", [(1, 16, 3), (7, 48, 64), (50, 768, 1027), (13, 64, 17), (257, 96, 48),
                                     (100, 3200, 512)])
def test_pre_equals_ref_on_hip_backend(nn, seq, N, K):
    """test_ops.cpp:138-157 on the HIP backend: pack_weights_i8 +
    quantize_act_i8, then the device dense_linear_i8_pre against the
    backend's scalar dense_linear_i8_ref, bit for bit."""
    fr = nn.Frand()
    x = _rv(fr, seq * K).reshape(seq, K)
    W = _rv(fr, N * K, -0.2, 0.2).reshape(N, K)
    b = _rv(fr, N)
    pre, ref = nn.nn_pre_vs_ref("hip", W, x, b)
    assert same_bits(pre, ref)
    # and the CPU build computes the same values (its panels, its VNNI kernel)
    pre_cpu, _ = nn.nn_pre_vs_ref("cpu", W, x, b)
    assert same_bits(pre, pre_cpu)


@pytest.mark.parametrize("seq,N,K", [(100, 3200, 512), (50, 2560, 960), (302, 512, 512), (1, 768, 3072)])
def test_linear_int8_forward_matches_cpu_build(nn, seq, N, K):
    """nn::Linear::init_int8 + forward (linear.cpp:66-133) on both backends."""
    fr = nn.Frand()
    x = _rv(fr, seq * K).reshape(seq, K)
    W = _rv(fr, N * K, -0.05, 0.05).reshape(N, K)
    b = _rv(fr, N, -0.02, 0.02)
    got, q1 = nn.nn_linear_forward("hip", W, b, x)
    want, q2 = nn.nn_linear_forward("cpu", W, b, x)
    assert q1 and q2
    assert same_bits(got, want)


@pytest.mark.parametrize("rows", [7, 1])
def test_shared_quantization_on_hip_backend(nn, rows):
    """test_ops.cpp:188-220 on the HIP backend: MhaQKV with aliasing inputs
    (one quantize_act_i8 shared by q|k and k|v, attention.cpp:40-59) equals the
    same layer on separate copies of the inputs, bit for bit, for every
    sharing pattern; and both equal the CPU build's projections."""
    dim, seq = 32, 7
    fr = nn.Frand()
    W = _rv(fr, dim * dim)
    b = _rv(fr, dim)
    source = _rv(fr, seq * dim).reshape(seq, dim)
    qcopy, kcopy, vcopy = source.copy(), source.copy(), source.copy()
    for sharing in range(4):
        q_in = source if sharing & 1 else qcopy
        v_in = source if sharing & 2 else vcopy
        actual = nn.nn_mha_forward("hip", dim, 4, W, b, q_in, source, v_in, rows, seq)
        expected = nn.nn_mha_forward("hip", dim, 4, W, b, qcopy, kcopy, vcopy, rows, seq)
        for a, e, what in zip(actual, expected, ("out", "q", "k", "v")):
            assert same_bits(a, e), f"shared quantization changed {what} (sharing {sharing}, rows {rows})"
        cpu = nn.nn_mha_forward("cpu", dim, 4, W, b, q_in, source, v_in, rows, seq)
        for a, c, what in zip(actual[1:], cpu[1:], ("q", "k", "v")):
            assert same_bits(a, c), f"{what} projection differs from the CPU build"
        scale = float(np.max(np.abs(cpu[0])))
        assert float(np.max(np.abs(actual[0] - cpu[0]))) <= 2e-2 * scale


def test_mha_fp32_layers_match_cpu_build(nn):
    """The same layer with fp32 projections: the projections are the
    reference's own CPU GEMM in both builds (bit-identical); only the
    attention runs on the device, so the output agrees to 1e-5."""
    dim, seq, rows = 64, 33, 33
    fr = nn.Frand()
    W = _rv(fr, dim * dim, -0.2, 0.2)
    b = _rv(fr, dim)
    x = _rv(fr, seq * dim).reshape(seq, dim)
    hip = nn.nn_mha_forward("hip", dim, 4, W, b, x, x, x, rows, seq, int8=0)
    cpu = nn.nn_mha_forward("cpu", dim, 4, W, b, x, x, x, rows, seq, int8=0)
    assert same_bits(hip[1], cpu[1]) and same_bits(hip[3], cpu[3])
    scale = float(np.max(np.abs(cpu[0])))
    assert float(np.max(np.abs(hip[0] - cpu[0]))) <= 1e-5 * scale


@pytest.mark.parametrize("full", [False, True])
def test_diffusion_unet_int8_linears_on_device(nn, tmp_path, full):
    """Diffusion Policy's noise-prediction UNet (src/models/diffusion/unet1d.cpp)
    with DIFFUSION_INT8 bit 1 (diffusion_model.cpp:113-114): the reference's own
    DPUNet1d on the HIP backend runs its Gemm-role conv, residual and
    downsample linears (unet1d.cpp:70-80) as dense_linear_i8 on the device;
    group norm, mish, the 1-D im2col, the transposed convs and the fp32 step /
    FiLM / output linears are the reference's CPU code in both builds. The int8
    GEMMs are exact, so the noise prediction equals the CPU build bit for bit,
    at every timestep. full: lerobot's stock widths (512, 1024, 2048), horizon 64."""
    from helpers import load_pkg
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    import vla_simd_amd.synth as synth
    c = dict(ck.DP_UNET_BASE) if full else dict(ck.DP_UNET_BASE, horizon=16, down_dims=(64, 128, 256),
                                                 step_embed_dim=32, num_keypoints=8)
    d = ck.write_dp_unet(str(tmp_path / "unet"), c)
    hip = nn.NnUnet("hip", d, c, 1)
    cpu = nn.NnUnet("cpu", d, c, 1)
    assert hip.n_int8 == cpu.n_int8 > 0
    sample = synth.normal("dp.sample", (c["horizon"], c["action_dim"]))
    gc = synth.normal("dp.gc", (ck.dp_cond_dim(c) - c["step_embed_dim"],))
    for t in (0, 37, 99):
        a, b = hip.forward(sample, gc, t), cpu.forward(sample, gc, t)
        assert same_bits(a, b), f"UNet noise prediction differs at t={t}"


def _weight_bytes(vla):
    return int(vla.lib().vla_h2d_bytes(1))


def test_int8_layers_stay_resident_on_device(nn, vla, tmp_path, monkeypatch):
    """Weight residency of the reference's own layers on the HIP backend: an
    nn::Linear, an nn::MhaQKV (four int8 projections, shared quantization),
    an nn::Conv2d and Diffusion Policy's UNet upload their int8 weights once,
    at init_int8's pack_weights_i8 (linear.cpp:97-99, conv.cpp:46); each
    forward after that moves no weight bytes to the device (the library's own
    H2D byte counter), and its outputs equal, bit for bit, both the same
    layers on the upload-per-call path (VLA_HIP_RESIDENT_MB=0) and the CPU
    build."""
    from helpers import load_pkg
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    import vla_simd_amd.synth as synth
    fr = nn.Frand()
    W = _rv(fr, 3200 * 512, -0.05, 0.05).reshape(3200, 512)
    b = _rv(fr, 3200, -0.02, 0.02)
    x = _rv(fr, 100 * 512).reshape(100, 512)
    Wc = _rv(fr, 64 * 3 * 3 * 32, -0.1, 0.1).reshape(64, 3, 3, 32)
    bc = _rv(fr, 64)
    img = _rv(fr, 20 * 24 * 32).reshape(20, 24, 32)
    dim = 64
    Wm = _rv(fr, dim * dim, -0.2, 0.2)
    bm = _rv(fr, dim)
    xm = _rv(fr, 33 * dim).reshape(33, dim)
    c = dict(ck.DP_UNET_BASE, horizon=16, down_dims=(64, 128, 256), step_embed_dim=32, num_keypoints=8)
    d = ck.write_dp_unet(str(tmp_path / "unet"), c)
    sample = synth.normal("dp.sample", (c["horizon"], c["action_dim"]))
    gc = synth.normal("dp.gc", (ck.dp_cond_dim(c) - c["step_embed_dim"],))

    def layers():
        return (nn.NnLinear("hip", W, b), nn.NnMha("hip", dim, 4, Wm, bm), nn.NnConv("hip", Wc, bc),
                nn.NnUnet("hip", d, c, 1))

    def run(lin, mha, conv, unet):
        xq, sa = nn.quantize_act_i8(x)
        return [lin.forward(x), lin.forward_quantized(xq, sa), mha.forward(xm, xm, xm, 33, 33),
                conv.forward(img, 1, 1), conv.forward(img, 2, 1)] + [unet.forward(sample, gc, t) for t in (0, 37)]

    monkeypatch.setenv("VLA_HIP_RESIDENT_MB", "0")
    per_call = layers()
    assert per_call[0].int8 and per_call[2].int8
    before = _weight_bytes(vla)
    want = run(*per_call)
    uploaded = _weight_bytes(vla) - before
    monkeypatch.delenv("VLA_HIP_RESIDENT_MB")
    resident = layers()
    run(*resident)  # first calls: biases move once
    for rep in range(3):
        before = _weight_bytes(vla)
        got = run(*resident)
        moved = _weight_bytes(vla) - before
        print(f"residency: forward weight bytes {moved} (upload-per-call path: {uploaded})", flush=True)
        assert moved == 0, f"repeat {rep}: {moved} weight bytes uploaded"
        for i, (g, w) in enumerate(zip(got, want)):
            assert same_bits(g, w), f"output {i} differs from the upload-per-call path"
    assert uploaded > 3200 * 512
    # the CPU build agrees (its own panels and VNNI kernel)
    assert same_bits(got[0], nn.NnLinear("cpu", W, b).forward(x))
    cpu_conv = nn.NnConv("cpu", Wc, bc)
    assert same_bits(got[3], cpu_conv.forward(img, 1, 1)) and same_bits(got[4], cpu_conv.forward(img, 2, 1))
    cpu_unet = nn.NnUnet("cpu", d, c, 1)
    assert same_bits(got[5], cpu_unet.forward(sample, gc, 0)) and same_bits(got[6], cpu_unet.forward(sample, gc, 37))


def test_residency_follows_repacked_buffers(nn, vla):
    """A buffer packed again (the same nn::Linear address with new weights, as
    when a layer object is re-initialised) replaces its resident copy: the
    forward uses the new weights. Many layers packed and dropped in turn stay
    correct (each new layer's pack replaces any stale entry at its address)."""
    fr = nn.Frand()
    x = _rv(fr, 17 * 96).reshape(17, 96)
    for i in range(6):
        W = _rv(fr, 48 * 96, -0.3, 0.3).reshape(48, 96)
        b = _rv(fr, 48) if i % 2 else None
        got = nn.NnLinear("hip", W, b).forward(x)
        want = nn.NnLinear("cpu", W, b).forward(x)
        assert same_bits(got, want), f"layer {i}"
