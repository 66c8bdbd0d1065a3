"""GPU parity of the int8 path: quantizer, int32 accumulators, fused epilogue.

Bar: quantized activations, scales and int32
accumulators bit-exact; the fp32 epilogue is the reference's single
expression fma((float)acc*ws, sa, b) (src/hal/common/gemm_i8.cpp:278), so the
fp32 outputs are required bit-exact too. The checker is the CPU oracle
(oracle/oracle.c) on the same seeded inputs, itself pinned to the real
reference build in tests/test_oracle.py.
"""

import os

import numpy as np
import pytest

from helpers import load_synth, max_rel, same_bits

pytestmark = pytest.mark.gpu

# tests/test_ops.cpp:138 shapes (seq, N, K), plus tails and BASELINE-like ones
TESTOPS_SHAPES = [(1, 16, 3), (7, 48, 64), (50, 768, 1027), (13, 64, 17), (257, 96, 48)]
EXTRA_SHAPES = [(1, 3200, 512), (100, 3200, 512), (129, 100, 70), (300, 512, 512),
                (302, 3200, 512), (64, 2560, 960), (100, 960, 2560), (16, 4096, 4096),
                (600, 200, 36), (2, 40, 1)]


def _case(orc, seq, N, K):
    fr = orc.Frand()
    x = fr.rv(seq * K).reshape(seq, K)
    W = fr.rv(N * K, -0.2, 0.2).reshape(N, K)
    b = fr.rv(N)
    return x, W, b


@pytest.mark.parametrize("magnitude", [0.0, np.finfo(np.float32).smallest_subnormal, 1e-37, 1.0])
@pytest.mark.parametrize("width", [3, 16, 33])
def test_quantize_edge_cases(vla, orc, magnitude, width):
    """test_ops.cpp:93-112: zero, denormal, tiny and unit rows."""
    x = np.array([(1 if i % 2 == 0 else -1) * magnitude for i in range(width)], np.float32)[None]
    q, s = vla.quantize_act_i8(x)
    qo, so = orc.quantize_act_i8(x)
    assert same_bits(q, qo) and same_bits(s, so)
    assert np.isfinite(s[0]) and s[0] > 0
    assert q.min() >= -127
    assert np.all(np.abs(q[0, :width].astype(np.float64) * s[0] - x[0]) <= s[0] * 0.51)
    assert np.all(q[0, width:] == 0)


@pytest.mark.parametrize("seq,K", [(1, 3), (5, 17), (100, 512), (302, 512), (177, 960), (50, 720),
                                   (64, 4096), (1000, 2560), (3, 1027)])
def test_quantize_rows(vla, orc, seq, K):
    synth = load_synth()
    x = synth.normal(f"q.{seq}x{K}", (seq, K))
    x[0, :] *= 1e-3
    if seq > 2:
        x[2, :] = 0.0
    q, s = vla.quantize_act_i8(x)
    qo, so = orc.quantize_act_i8(x)
    assert same_bits(q, qo), "int8 activations differ from the oracle"
    assert same_bits(s, so), "activation scales differ from the oracle"


@pytest.mark.parametrize("seq,N,K", TESTOPS_SHAPES + EXTRA_SHAPES)
def test_gemm_int32_and_epilogue(vla, orc, seq, N, K):
    x, W, b = _case(orc, seq, N, K)
    Wq, ws = orc.quantize_weights_i8(W)
    xq, sa = orc.quantize_act_i8(x)
    acc = vla.gemm_i8_i32(xq, Wq, K)
    acc_o = orc.gemm_i8_acc(xq, Wq, K)
    assert same_bits(acc, acc_o), "int32 accumulators differ"
    out = vla.dense_linear_i8_pre(xq, sa, Wq, ws, b, K)
    out_o = orc.dense_linear_i8_pre(xq, sa, Wq, ws, b, K)
    assert same_bits(out, out_o), "fp32 epilogue differs"
    out_nb = vla.dense_linear_i8_pre(xq, sa, Wq, ws, None, K)
    assert same_bits(out_nb, orc.dense_linear_i8_pre(xq, sa, Wq, ws, None, K))
    full = vla.dense_linear_i8(x, Wq, ws, b)
    assert same_bits(full, out_o), "quantize + GEMM differs from the two-step oracle"


def test_int8_accuracy_vs_double(vla, orc):
    """test_ops.cpp:153: the int8 linear within 2e-2 of the double product, scaled
    by the magnitude sum."""
    for seq, N, K in TESTOPS_SHAPES:
        x, W, b = _case(orc, seq, N, K)
        Wq, ws = vla.pack_weights_i8(W)
        out = vla.dense_linear_i8(x, Wq, ws, b)
        ref = x.astype(np.float64) @ W.T.astype(np.float64) + b
        mag = np.abs(x.astype(np.float64)) @ np.abs(W.T.astype(np.float64)) + np.abs(b)
        assert np.max(np.abs(out - ref) / (mag + 1e-30)) <= 2e-2


@pytest.mark.parametrize("M,K,N", [(100, 512, 3200), (1, 4096, 4096), (50, 960, 2560),
                                   (100, 2560, 960), (100, 768, 3072), (512, 512, 3200),
                                   (512, 960, 2560)])
def test_baseline_shapes(vla, orc, M, K, N):
    """BASELINE.json distributions: x ~ N(0,1), int8 W uniform, scales U(1e-3,1e-2), bias N(0,.02)."""
    synth = load_synth()
    x, Wq, ws, b = synth.linear_case(M, K, N)
    xq, sa = vla.quantize_act_i8(x)
    xqo, sao = orc.quantize_act_i8(x)
    assert same_bits(xq, xqo) and same_bits(sa, sao)
    Wp = np.zeros((N, (K + 3) & ~3), np.int8)
    Wp[:, :K] = Wq
    out = vla.dense_linear_i8(x, Wp, ws, b)
    out_o = orc.dense_linear_i8_pre(xqo, sao, Wp, ws, b, K)
    assert same_bits(out, out_o)


@pytest.mark.parametrize("act", [1, 2, 3])
def test_fused_activation_and_accumulate(vla, orc, torch_cuda, act):
    torch = torch_cuda
    seq, N, K = 302, 3200, 512
    x, W, b = _case(orc, seq, N, K)
    lin = vla.LinearI8.from_f32(W, b)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    xq = torch.zeros((seq, lin.ldw), dtype=torch.int8, device=dev)
    sa = torch.zeros(seq, dtype=torch.float32, device=dev)
    out = torch.zeros((seq, N), dtype=torch.float32, device=dev)
    lin.forward_dev(out, xd, xq, sa, act=act)
    torch.cuda.synchronize()
    Wq, ws = orc.quantize_weights_i8(W)
    xqo, sao = orc.quantize_act_i8(x)
    lin_o = orc.dense_linear_i8_pre(xqo, sao, Wq, ws, b, K)
    got = out.cpu().numpy()
    want = orc.apply_act(lin_o, act)
    if act == 1:
        assert same_bits(got, want), "relu epilogue must be exact"
    else:
        assert max_rel(got, want) <= 2e-6
    # accumulate: out += linear(x) on top of a residual
    res = torch.from_numpy(np.full((seq, N), 0.5, np.float32)).to(dev)
    lin.forward_dev(res, xd, xq, sa, act=0, accumulate=1)
    torch.cuda.synchronize()
    assert same_bits(res.cpu().numpy(), (np.float32(0.5) + lin_o).astype(np.float32))
    lin.close()


def test_resident_linear_from_int8(vla, orc, torch_cuda):
    torch = torch_cuda
    synth = load_synth()
    M, K, N = 100, 512, 3200
    x, Wq, ws, b = synth.linear_case(M, K, N)
    lin = vla.LinearI8.from_i8(Wq, ws, b)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    xq = torch.zeros((M, lin.ldw), dtype=torch.int8, device=dev)
    sa = torch.zeros(M, dtype=torch.float32, device=dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    lin.forward_dev(out, xd, xq, sa)
    torch.cuda.synchronize()
    xqo, sao = orc.quantize_act_i8(x)
    assert same_bits(out.cpu().numpy(), orc.dense_linear_i8_pre(xqo, sao, Wq, ws, b, K))
    # quantized-input entry (Linear::forward_quantized)
    out2 = torch.empty_like(out)
    lin.forward_quantized_dev(out2, xq, sa)
    torch.cuda.synchronize()
    assert same_bits(out2.cpu().numpy(), out.cpu().numpy())
    lin.close()


def test_k_bound_rejected(vla):
    """test_ops.cpp:79-92: K > INT_MAX/(255*127) is refused, not computed."""
    K = 2147483647 // (255 * 127) + 1
    with pytest.raises(vla.VlaError) as e:
        vla.LinearI8.from_f32(np.ones((16, K), np.float32))
    assert e.value.status == vla.VLA_ERR_ARG


TILES = ["128x128x64", "64x128x64", "64x64x64", "128x128x64s4", "64x128x64s4", "256x128x128s3w8",
         "256x256x128s2w8", "256x128x128s3w8p", "256x256x128s2w8p", "128x128x128s2", "64x64x128s3", "64x64x128s4", "32x64x128s3", "32x64x128s4"]


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("M,N,K", [(300, 200, 200), (257, 130, 48), (520, 272, 1024), (129, 17, 64), (257, 17, 64)])
def test_every_tile_config(vla, orc, torch_cuda, tile, M, N, K):
    """Each aligned-kernel tile, forced, on shapes off the tile grid: M and N
    edges, a K tail, K below one slab (device rows padded to 16 bytes)."""
    torch = torch_cuda
    ld = (K + 15) // 16 * 16
    x, W, b = _case(orc, M, N, K)
    Wq, ws = orc.quantize_weights_i8(W, ldq=ld)
    xq, sa = orc.quantize_act_i8(x, ldq=ld)
    dev = torch.device("cuda")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    acc = torch.zeros((M, N), dtype=torch.int32, device=dev)
    out = torch.zeros((M, N), dtype=torch.float32, device=dev)
    os.environ["VLA_HIP_GEMM_TILE"] = tile
    try:
        vla.gemm_i8_i32_dev(acc, d(xq), d(Wq), K)
        vla.dense_linear_i8_pre_dev(out, d(xq), d(sa), d(Wq), d(ws), d(b), K)
        torch.cuda.synchronize()
    finally:
        del os.environ["VLA_HIP_GEMM_TILE"]
    assert same_bits(acc.cpu().numpy(), orc.gemm_i8_acc(xq, Wq, K)), f"int32 differs with tile {tile}"
    assert same_bits(out.cpu().numpy(), orc.dense_linear_i8_pre(xq, sa, Wq, ws, b, K))


@pytest.mark.parametrize("tile", TILES)
def test_tile_epilogue_options(vla, orc, torch_cuda, tile):
    """act + accumulate through each tile's LDS-staged epilogue, with an output
    row stride wider than N."""
    torch = torch_cuda
    M, N, K = 300, 200, 192
    x, W, b = _case(orc, M, N, K)
    Wq, ws = orc.quantize_weights_i8(W, ldq=192)
    xq, sa = orc.quantize_act_i8(x, ldq=192)
    dev = torch.device("cuda")
    out = torch.full((M, 260), 0.25, dtype=torch.float32, device=dev)
    os.environ["VLA_HIP_GEMM_TILE"] = tile
    try:
        vla.dense_linear_i8_pre_dev(out[:, :N], torch.from_numpy(xq).to(dev), torch.from_numpy(sa).to(dev),
                                    torch.from_numpy(Wq).to(dev), torch.from_numpy(ws).to(dev),
                                    torch.from_numpy(b).to(dev), K, act=1, accumulate=1)
        torch.cuda.synchronize()
    finally:
        del os.environ["VLA_HIP_GEMM_TILE"]
    got = out.cpu().numpy()
    want = np.float32(0.25) + orc.apply_act(orc.dense_linear_i8_pre(xq, sa, Wq, ws, b, K), 1)
    assert same_bits(got[:, :N], want.astype(np.float32))
    assert np.all(got[:, N:] == np.float32(0.25)), "wrote past N"


def _from_panel(buf, seq, K):
    """Row-major [seq, K] view of panel-layout bytes (the layout vla_simd_hip.h
    documents: byte (k/64)*round16(seq)*64 + t*64 + k%64), plus each row's
    bytes [K, round64(K))."""
    mp, k64 = (seq + 15) // 16 * 16, (K + 63) // 64 * 64
    p = np.asarray(buf, np.int8)[: mp * k64].reshape(k64 // 64, mp, 64)
    rows = p.transpose(1, 0, 2).reshape(mp, k64)[:seq]
    return rows[:, :K], rows[:, K:]


@pytest.mark.parametrize("seq,K", [(1, 3), (5, 17), (16, 64), (50, 720), (100, 512), (128, 960),
                                   (3, 1027), (77, 4100), (128, 2048), (9, 2052), (64, 12288),
                                   (3, 16384), (4, 16388)])
def test_quantize_panel_layout(vla, orc, torch_cuda, seq, K):
    """Panel-layout quantization: the same bytes and scales as the oracle's
    row-major quantize_act_i8, at the documented panel offsets, pads zero."""
    torch = torch_cuda
    synth = load_synth()
    x = synth.normal(f"qp.{seq}x{K}", (seq, K))
    if seq > 2:
        x[1, :] = 0.0
    n = vla.i8_panel_bytes(seq, K)
    assert n == (seq + 15) // 16 * 16 * ((K + 63) // 64 * 64)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    xq = torch.full((n,), 99, dtype=torch.int8, device=dev)  # pads must be overwritten
    sa = torch.zeros(seq, dtype=torch.float32, device=dev)
    vla.quantize_act_i8_panel_dev(xd, xq, sa)
    torch.cuda.synchronize()
    got, pad = _from_panel(xq.cpu().numpy(), seq, K)
    qo, so = orc.quantize_act_i8(x)
    assert same_bits(got, qo[:, :K]), "panel bytes differ from the oracle's row-major quantization"
    assert same_bits(sa.cpu().numpy(), so)
    assert np.all(pad == 0), "bytes past K in a row's last panel must be zero"


@pytest.mark.parametrize("seq,N,K", [(1, 16, 3), (7, 48, 64), (50, 768, 1027), (13, 64, 17),
                                     (100, 3200, 512), (64, 2560, 960), (100, 960, 2560),
                                     (50, 4096, 4096), (128, 720, 2048), (2, 40, 1)])
@pytest.mark.parametrize("act,accumulate", [(0, 0), (1, 1), (2, 0)])
def test_panel_gemm_bitexact(vla, orc, torch_cuda, seq, N, K, act, accumulate):
    """The skinny GEMM over panel-layout activations: bit-exact with the
    oracle's dense_linear_i8_pre (ReLU exact; GELU within device libm)."""
    torch = torch_cuda
    x, W, b = _case(orc, seq, N, K)
    Wq, ws = orc.quantize_weights_i8(W)
    ld = (K + 63) // 64 * 64
    Wp = np.zeros((N, ld), np.int8)
    Wp[:, :Wq.shape[1]] = Wq
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    xq = torch.empty((vla.i8_panel_bytes(seq, K),), dtype=torch.int8, device=dev)
    sa = torch.empty(seq, dtype=torch.float32, device=dev)
    vla.quantize_act_i8_panel_dev(xd, xq, sa)
    Wd = torch.from_numpy(Wp).to(dev)
    wsd = torch.from_numpy(ws).to(dev)
    bd = torch.from_numpy(b).to(dev)
    base = np.full((seq, N), 0.25, np.float32)
    out = torch.from_numpy(base.copy()).to(dev)
    vla.dense_linear_i8_panel_dev(out, xq, sa, Wd, wsd, bd, K, act=act, accumulate=accumulate)
    torch.cuda.synchronize()
    xqo, sao = orc.quantize_act_i8(x)
    want = orc.apply_act(orc.dense_linear_i8_pre(xqo, sao, Wq, ws, b, K), act)
    if accumulate:
        want = (base + want).astype(np.float32)
    got = out.cpu().numpy()
    if act == 2:
        assert max_rel(got, want) <= 2e-6
    else:
        assert same_bits(got, want), "panel-layout GEMM differs from the oracle"


def test_panel_rejects_large_m(vla, torch_cuda):
    torch = torch_cuda
    assert vla.i8_panel_bytes(129, 64) == -1
    dev = torch.device("cuda")
    x = torch.zeros((129, 64), dtype=torch.float32, device=dev)
    xq = torch.zeros((144 * 64,), dtype=torch.int8, device=dev)
    sa = torch.zeros(129, dtype=torch.float32, device=dev)
    with pytest.raises(vla.VlaError) as e:
        vla.quantize_act_i8_panel_dev(x, xq, sa)
    assert e.value.status == vla.VLA_ERR_ARG


# ---------------------------------------------------------------- split K --

# very long K over at most 64 tiles of 64 x 64 (M > 128 splits only there),
# more than 320 rows (129..320 rows over N <= 2048 take the unsplit skinny
# kernel): a w2-like 340 x 512 x 3200, a ResNet-like 3x3/512 conv
# (330 x 512 x 4608), K tails (4100, 3100), one row past the skinny bound, an
# N edge (48) and a 60-tile output
SPLIT_SHAPES = [(340, 512, 3200), (330, 512, 4608), (321, 100, 4100), (330, 48, 3100), (330, 640, 4096),
                (330, 512, 4100),
                # at most 128 rows (the skinny kernel splits from K = 8192):
                # SigLIP's projection (64 x 960 x 12288), a K tail, one row,
                # 16 columns, a UNet-like 4 x 1024 x 20480
                (64, 960, 12288), (100, 1000, 8200), (1, 16, 8192), (16, 200, 8192), (4, 1024, 20480)]


@pytest.mark.parametrize("seq,N,K", SPLIT_SHAPES)
@pytest.mark.parametrize("act,accumulate", [(0, 0), (1, 1), (2, 0)])
def test_split_k_bitexact(vla, orc, torch_cuda, seq, N, K, act, accumulate):
    """Split-K (int32 partial sums over K chunks, then one reduce + epilogue)
    equals the unsplit launch and the oracle bit for bit."""
    torch = torch_cuda
    n = vla.gemm_i8_split_bytes(seq, N, K)
    assert n > 0, "shape expected to split"
    x, W, b = _case(orc, seq, N, K)
    xq, sa = orc.quantize_act_i8(x)
    Wq, ws = orc.quantize_weights_i8(W)
    ld = (K + 63) // 64 * 64
    Xp = np.zeros((seq, ld), np.int8)
    Xp[:, :xq.shape[1]] = xq
    Wp = np.zeros((N, ld), np.int8)
    Wp[:, :Wq.shape[1]] = Wq
    dev = torch.device("cuda")
    Xd, Wd = torch.from_numpy(Xp).to(dev), torch.from_numpy(Wp).to(dev)
    sad, wsd, bd = torch.from_numpy(sa).to(dev), torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    base = np.full((seq, N), 0.25, np.float32)
    work = torch.empty(n, dtype=torch.uint8, device=dev)
    split = torch.from_numpy(base.copy()).to(dev)
    vla.dense_linear_i8_pre_split_dev(split, Xd, sad, Wd, wsd, bd, K, work, act=act, accumulate=accumulate)
    plain = torch.from_numpy(base.copy()).to(dev)
    vla.dense_linear_i8_pre_dev(plain, Xd, sad, Wd, wsd, bd, K, act=act, accumulate=accumulate)
    small = torch.from_numpy(base.copy()).to(dev)  # a workspace one byte short runs unsplit
    vla.dense_linear_i8_pre_split_dev(small, Xd, sad, Wd, wsd, bd, K, work[: n - 1], act=act,
                                      accumulate=accumulate)
    torch.cuda.synchronize()
    got = split.cpu().numpy()
    assert same_bits(got, plain.cpu().numpy()) and same_bits(small.cpu().numpy(), got)
    want = orc.apply_act(orc.dense_linear_i8_pre(xq, sa, Wq, ws, b, K), act)
    if accumulate:
        want = (base + want).astype(np.float32)
    if act == 2:
        assert max_rel(got, want) <= 2e-6
    else:
        assert same_bits(got, want)


@pytest.mark.parametrize("seq,N,K", [(64, 960, 12288), (100, 1000, 8200), (5, 48, 8200), (8, 512, 10240)])
def test_split_k_panel_bitexact(vla, orc, torch_cuda, seq, N, K):
    """Split-K over panel-layout activations (the chunks start at whole
    64-byte panels): equal to the unsplit panel GEMM and the oracle."""
    torch = torch_cuda
    n = vla.gemm_i8_split_bytes(seq, N, K)
    assert n > 0, "shape expected to split"
    x, W, b = _case(orc, seq, N, K)
    Wq, ws = orc.quantize_weights_i8(W)
    ld = (K + 63) // 64 * 64
    Wp = np.zeros((N, ld), np.int8)
    Wp[:, :Wq.shape[1]] = Wq
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    xq = torch.empty((vla.i8_panel_bytes(seq, K),), dtype=torch.int8, device=dev)
    sa = torch.empty(seq, dtype=torch.float32, device=dev)
    vla.quantize_act_i8_panel_dev(xd, xq, sa)
    Wd, wsd, bd = torch.from_numpy(Wp).to(dev), torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    work = torch.empty(n, dtype=torch.uint8, device=dev)
    split = torch.full((seq, N), 0.5, device=dev)
    vla.dense_linear_i8_panel_split_dev(split, xq, sa, Wd, wsd, bd, K, work, act=1, accumulate=1)
    plain = torch.full((seq, N), 0.5, device=dev)
    vla.dense_linear_i8_panel_dev(plain, xq, sa, Wd, wsd, bd, K, act=1, accumulate=1)
    torch.cuda.synchronize()
    got = split.cpu().numpy()
    assert same_bits(got, plain.cpu().numpy())
    xo, so = orc.quantize_act_i8(x)
    want = (np.float32(0.5) + orc.apply_act(orc.dense_linear_i8_pre(xo, so, Wq, ws, b, K), 1)).astype(np.float32)
    assert same_bits(got, want)


def test_split_k_plan_bounds(vla):
    """Short K, skinny M and tile-rich shapes are not split; the workspace a
    split asks for stays within 8 MiB."""
    assert vla.gemm_i8_split_bytes(100, 4096, 4096) == 0      # skinny kernel
    assert vla.gemm_i8_split_bytes(8, 1024, 5120) == 0        # skinny, K < 8192: measured slower split
    assert vla.gemm_i8_split_bytes(658, 768, 768) == 0        # K < 1024
    assert vla.gemm_i8_split_bytes(8192, 4096, 4096) == 0     # fills the chip
    assert vla.gemm_i8_split_bytes(512, 4096, 4096) == 0      # one LDS-DMA tile per CU: measured slower split
    for seq, N, K in [(129, 100, 4100), (200, 48, 3100), (256, 1024, 4096), (302, 512, 3200), (320, 100, 4100)]:
        assert vla.gemm_i8_split_bytes(seq, N, K) == 0        # 129..320 rows, N <= 2048: unsplit skinny kernel
    for seq, N, K in SPLIT_SHAPES:
        assert 0 < vla.gemm_i8_split_bytes(seq, N, K) <= 8 << 20


@pytest.mark.parametrize("seq,N,K,act,accumulate", [(100, 3200, 512, 0, 0), (7, 48, 1027, 1, 1),
                                                    (302, 512, 512, 2, 0), (1, 16, 3, 0, 1),
                                                    (2048, 960, 2560, 0, 0),
                                                    # <= 16 rows: quantized inside the GEMM
                                                    (1, 3200, 512, 0, 0), (16, 2560, 960, 1, 1),
                                                    (5, 100, 2048, 2, 0), (9, 200, 64, 1, 0)])
def test_dense_linear_i8_dev_caller_scratch(vla, orc, torch_cuda, seq, N, K, act, accumulate):
    """tcpu::dense_linear_i8 with caller-owned scratch (quant_ops.h:66-72) on
    device pointers: the scratch holds exactly seq x i8_kpad(K) bytes and seq
    scales, as the reference's contract sizes it; the quantized bytes it leaves
    there and the output equal the oracle's quantize + dense_linear_i8_pre."""
    torch = torch_cuda
    x, W, b = _case(orc, seq, N, K)
    Kp = (K + 3) & ~3
    Wq, ws = orc.quantize_weights_i8(W, Kp)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    Wd = torch.from_numpy(np.ascontiguousarray(Wq)).to(dev)
    wsd, bd = torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    xq = torch.full((seq, Kp), 99, dtype=torch.int8, device=dev)
    sa = torch.zeros(seq, dtype=torch.float32, device=dev)
    base = np.full((seq, N), 0.25, np.float32)
    out = torch.from_numpy(base).to(dev)
    vla.dense_linear_i8_dev(out, xd, Wd, wsd, bd, K, xq, sa, act=act, accumulate=accumulate)
    torch.cuda.synchronize()
    xqo, sao = orc.quantize_act_i8(x)
    assert same_bits(xq.cpu().numpy(), xqo) and same_bits(sa.cpu().numpy(), sao)
    want = orc.apply_act(orc.dense_linear_i8_pre(xqo, sao, Wq, ws, b, K), act)
    if accumulate:
        want = (base + want).astype(np.float32)
    got = out.cpu().numpy()
    if act in (0, 1):
        assert same_bits(got, want)
    else:
        assert max_rel(got, want) <= 2e-6


@pytest.mark.parametrize("seq,N,K", [(1, 3200, 512), (16, 2560, 960), (7, 33, 2048), (12, 64, 4)])
def test_op_fusion_matches_two_launches(vla, orc, torch_cuda, seq, N, K):
    """The op API's few-row path (quantize inside the GEMM, the scratch written
    by the same kernel) leaves the same scratch bytes, scales and outputs as
    the separate quantize + GEMM launches (VLA_HIP_OP_FUSE=0), twice in a row."""
    torch = torch_cuda
    x, W, b = _case(orc, seq, N, K)
    Kp = (K + 3) & ~3
    ld = (Kp + 15) // 16 * 16
    Wq, ws = orc.quantize_weights_i8(W, ld)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    Wd = torch.from_numpy(np.ascontiguousarray(Wq)).to(dev)
    wsd, bd = torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    res = {}
    for fuse in ("1", "0"):
        os.environ["VLA_HIP_OP_FUSE"] = fuse
        try:
            for rep in range(2):
                xq = torch.full((seq, ld), 99, dtype=torch.int8, device=dev)
                sa = torch.full((seq,), 7.0, dtype=torch.float32, device=dev)
                out = torch.full((seq, N), 0.5, dtype=torch.float32, device=dev)
                vla.dense_linear_i8_dev(out, xd, Wd, wsd, bd, K, xq, sa, act=1, accumulate=1)
                torch.cuda.synchronize()
                res[(fuse, rep)] = (xq.cpu().numpy(), sa.cpu().numpy(), out.cpu().numpy())
        finally:
            os.environ.pop("VLA_HIP_OP_FUSE", None)
    ref = res[("0", 0)]
    for k, v in res.items():
        for a, b_ in zip(v, ref):
            assert same_bits(a, b_), f"{k} differs from the two-launch path"
    xqo, sao = orc.quantize_act_i8(x, ldq=ld)
    assert same_bits(ref[0], xqo) and same_bits(ref[1], sao)


# ------------------------------------------------------------- row groups --

@pytest.mark.parametrize("fn", ["1", "2"])
@pytest.mark.parametrize("groups", ["1", "2", "3", "4", "8"])
@pytest.mark.parametrize("seq,N,K", [(100, 960, 2560), (50, 720, 960), (128, 48, 1027), (37, 200, 4100),
                                     (17, 64, 64), (1, 16, 3), (100, 4096, 4096), (33, 40, 200)])
def test_skinny_row_groups_bitexact(vla, orc, torch_cuda, fn, groups, seq, N, K):
    """The skinny kernel split into row groups (each block: 16 x FN columns x
    its 16-row fragments; fragments past M repeat the last and are never
    stored) gives the oracle's outputs bit for bit, row-major, panel and
    split-K."""
    torch = torch_cuda
    x, W, b = _case(orc, seq, N, K)
    xq, sa = orc.quantize_act_i8(x)
    Wq, ws = orc.quantize_weights_i8(W)
    ld = (K + 63) // 64 * 64
    Xp = np.zeros((seq, ld), np.int8)
    Xp[:, :xq.shape[1]] = xq
    Wp = np.zeros((N, ld), np.int8)
    Wp[:, :Wq.shape[1]] = Wq
    dev = torch.device("cuda")
    Xd, Wd = torch.from_numpy(Xp).to(dev), torch.from_numpy(Wp).to(dev)
    sad, wsd, bd = torch.from_numpy(sa).to(dev), torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    xd = torch.from_numpy(x).to(dev)
    xpan = torch.empty((vla.i8_panel_bytes(seq, K),), dtype=torch.int8, device=dev)
    span = torch.empty(seq, dtype=torch.float32, device=dev)
    nsplit = vla.gemm_i8_split_bytes(seq, N, K)
    work = torch.empty(max(nsplit, 16), dtype=torch.uint8, device=dev)
    base = np.full((seq, N), 0.25, np.float32)
    outs = [torch.from_numpy(base.copy()).to(dev) for _ in range(3)]
    os.environ["VLA_HIP_SKINNY_R"] = groups
    os.environ["VLA_HIP_SKINNY_FN"] = fn
    try:
        vla.dense_linear_i8_pre_dev(outs[0], Xd, sad, Wd, wsd, bd, K, act=1, accumulate=1)
        vla.quantize_act_i8_panel_dev(xd, xpan, span)
        vla.dense_linear_i8_panel_dev(outs[1], xpan, span, Wd, wsd, bd, K, act=1, accumulate=1)
        vla.dense_linear_i8_pre_split_dev(outs[2], Xd, sad, Wd, wsd, bd, K, work, act=1, accumulate=1)
        torch.cuda.synchronize()
    finally:
        del os.environ["VLA_HIP_SKINNY_R"], os.environ["VLA_HIP_SKINNY_FN"]
    want = (base + orc.apply_act(orc.dense_linear_i8_pre(xq, sa, Wq, ws, b, K), 1)).astype(np.float32)
    for i, o in enumerate(outs):
        assert same_bits(o.cpu().numpy(), want), f"form {i} with {groups} row groups differs from the oracle"


# -------------------------------------------------------------------- gemv --

@pytest.mark.parametrize("seq,N,K", [(1, 720, 2048), (2, 17, 2050), (1, 1, 4100), (2, 4096, 4096),
                                     (1, 33, 8196), (2, 960, 2560)])
@pytest.mark.parametrize("act,accumulate", [(0, 0), (1, 1), (2, 0)])
def test_gemv_rows_bitexact(vla, orc, torch_cuda, seq, N, K, act, accumulate):
    """One or two rows over K >= 2048 (the dot-product kernel, weight bytes
    past K masked): the oracle's outputs, row-major and panel activations."""
    torch = torch_cuda
    x, W, b = _case(orc, seq, N, K)
    xq, sa = orc.quantize_act_i8(x)
    Wq, ws = orc.quantize_weights_i8(W)
    ld = (K + 63) // 64 * 64
    Xp = np.zeros((seq, ld), np.int8)
    Xp[:, :xq.shape[1]] = xq
    Wp = np.full((N, ld), 77, np.int8)  # bytes past K are not zero: the kernel must mask them
    Wp[:, :K] = Wq[:, :K]
    dev = torch.device("cuda")
    Xd, Wd = torch.from_numpy(Xp).to(dev), torch.from_numpy(Wp).to(dev)
    sad, wsd, bd = torch.from_numpy(sa).to(dev), torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    xd = torch.from_numpy(x).to(dev)
    xpan = torch.empty((vla.i8_panel_bytes(seq, K),), dtype=torch.int8, device=dev)
    span = torch.empty(seq, dtype=torch.float32, device=dev)
    base = np.full((seq, N), 0.25, np.float32)
    row = torch.from_numpy(base.copy()).to(dev)
    pan = torch.from_numpy(base.copy()).to(dev)
    vla.dense_linear_i8_pre_dev(row, Xd, sad, Wd, wsd, bd, K, act=act, accumulate=accumulate)
    vla.quantize_act_i8_panel_dev(xd, xpan, span)
    vla.dense_linear_i8_panel_dev(pan, xpan, span, Wd, wsd, bd, K, act=act, accumulate=accumulate)
    torch.cuda.synchronize()
    want = orc.apply_act(orc.dense_linear_i8_pre(xq, sa, Wq, ws, b, K), act)
    if accumulate:
        want = (base + want).astype(np.float32)
    for got in (row.cpu().numpy(), pan.cpu().numpy()):
        if act == 2:
            assert max_rel(got, want) <= 2e-6
        else:
            assert same_bits(got, want), "gemv rows differ from the oracle"


@pytest.mark.parametrize("groups", ["", "1", "3"])
@pytest.mark.parametrize("seq,N,K", [(177, 960, 960), (256, 100, 300), (129, 17, 64), (200, 1024, 4100),
                                     (177, 2048, 2560), (240, 33, 1027), (302, 512, 512), (302, 512, 3200),
                                     (320, 48, 1027)])
def test_skinny_129_to_320_rows_bitexact(vla, orc, torch_cuda, groups, seq, N, K):
    """129..320 rows over N <= 2048 take the skinny kernel in row groups of at
    most 8 fragments (a forced count below that is raised): the oracle's
    outputs bit for bit, also through the split-K entry point, and with the
    route switched off per call (VLA_HIP_SKINNY_MAXM=128: the tiles, split
    over K where the plan says so)."""
    torch = torch_cuda
    x, W, b = _case(orc, seq, N, K)
    xq, sa = orc.quantize_act_i8(x)
    Wq, ws = orc.quantize_weights_i8(W)
    ld = (K + 63) // 64 * 64
    Xp = np.zeros((seq, ld), np.int8)
    Xp[:, :xq.shape[1]] = xq
    Wp = np.zeros((N, ld), np.int8)
    Wp[:, :Wq.shape[1]] = Wq
    dev = torch.device("cuda")
    Xd, Wd = torch.from_numpy(Xp).to(dev), torch.from_numpy(Wp).to(dev)
    sad, wsd, bd = torch.from_numpy(sa).to(dev), torch.from_numpy(ws).to(dev), torch.from_numpy(b).to(dev)
    assert vla.gemm_i8_split_bytes(seq, N, K) == 0
    base = np.full((seq, N), 0.25, np.float32)
    outs = [torch.from_numpy(base.copy()).to(dev) for _ in range(3)]
    if groups:
        os.environ["VLA_HIP_SKINNY_R"] = groups
    try:
        vla.dense_linear_i8_pre_dev(outs[0], Xd, sad, Wd, wsd, bd, K, act=1, accumulate=1)
        work = torch.empty(16, dtype=torch.uint8, device=dev)
        vla.dense_linear_i8_pre_split_dev(outs[1], Xd, sad, Wd, wsd, bd, K, work, act=1, accumulate=1)
        os.environ["VLA_HIP_SKINNY_MAXM"] = "128"
        work = torch.empty(max(vla.gemm_i8_split_bytes(seq, N, K), 16), dtype=torch.uint8, device=dev)
        vla.dense_linear_i8_pre_split_dev(outs[2], Xd, sad, Wd, wsd, bd, K, work, act=1, accumulate=1)
        torch.cuda.synchronize()
    finally:
        os.environ.pop("VLA_HIP_SKINNY_R", None)
        os.environ.pop("VLA_HIP_SKINNY_MAXM", None)
    want = (base + orc.apply_act(orc.dense_linear_i8_pre(xq, sa, Wq, ws, b, K), 1)).astype(np.float32)
    for o in outs:
        assert same_bits(o.cpu().numpy(), want)


@pytest.mark.parametrize("seq,N,K", [(100, 3200, 512), (7, 48, 1027), (302, 96, 17), (1, 16, 4096)])
def test_resident_linear_host_forms(vla, orc, seq, N, K):
    """The host-pointer forms over resident weights (what the reference's op
    layer calls for a packed nn::Linear): the quantized rows and scales the
    caller's scratch receives and the output equal the oracle's bit for bit;
    the quantized-input form gives the same output; the downloaded rows and
    scales are the packer's; a bias set, changed and dropped after creation
    takes effect; and no call moves weight bytes once the layer exists."""
    x, W, b = _case(orc, seq, N, K)
    Wq, ws = orc.quantize_weights_i8(W)
    lin = vla.LinearI8.from_f32(W)
    Wd, wsd = lin.download()
    assert same_bits(Wd, Wq) and same_bits(wsd, ws)
    xqo, sao = orc.quantize_act_i8(x)
    before = int(vla.lib().vla_h2d_bytes(1))
    out, xq, sa = lin.forward(x)
    assert int(vla.lib().vla_h2d_bytes(1)) == before, "a forward uploaded weight bytes"
    assert same_bits(xq, xqo) and same_bits(sa, sao)
    assert same_bits(out, orc.dense_linear_i8_pre(xqo, sao, Wq, ws, None, K))
    assert same_bits(lin.forward_quantized(xqo, sao), out)
    lin.set_bias(b)
    assert same_bits(lin.forward(x)[0], orc.dense_linear_i8_pre(xqo, sao, Wq, ws, b, K))
    b2 = (b * -3.0).astype(np.float32)
    lin.set_bias(b2)
    assert same_bits(lin.forward_quantized(xqo, sao), orc.dense_linear_i8_pre(xqo, sao, Wq, ws, b2, K))
    lin.set_bias(None)
    assert same_bits(lin.forward(x)[0], out)
    lin.close()


def test_resident_conv_host_form(vla, orc):
    """vla_conv2d_i8_resident (nn::Conv2d's forward over resident weights)
    equals vla_conv2d_i8 with the same weights uploaded per call, bit for bit,
    at a 3x3 and a strided 1x1 layer."""
    r = np.random.default_rng(4)
    for (H, Wd, Cin, Cout, k, s, p) in [(20, 24, 32, 64, 3, 1, 1), (16, 16, 64, 32, 1, 2, 0)]:
        x = r.normal(0, 1, (H, Wd, Cin)).astype(np.float32)
        W = r.uniform(-0.2, 0.2, (Cout, k * k * Cin)).astype(np.float32)
        b = r.normal(0, 0.02, Cout).astype(np.float32)
        lin = vla.LinearI8.from_f32(W, b)
        Wq, ws = lin.download()
        got = lin.conv2d(x, k, s, p)
        want = vla.conv2d_i8(x, Wq, ws, b, k, s, p)
        assert same_bits(got, want), (H, Wd, Cin, Cout, k, s, p)
        lin.close()
