"""GPU parity of the row op fused into the int8 linear (gemm_i8_rowop).

The fused kernel must give exactly what the two-kernel path gives: the row op
and its int8 quantization (vla_rowop_quantize_i8_panel_dev), then the panel
GEMM (vla_dense_linear_i8_panel_dev) -- bit for bit, fp32 outputs included.
The two-kernel path is pinned to the oracle: its GEMM bit-exact from its own
bytes and scales (oracle dense_linear_i8_pre, src/hal/common/gemm_i8.cpp:278),
its bytes against the oracle's rmsnorm / silu_gate (src/hal/common/norms.cpp:19-35,
src/ops/eltwise.cpp:29-64) followed by quantize_act_i8 (src/ops/quant_ops.h:17-21):
the device's double sums run in another order and its expf is the device libm,
so a byte may sit one step away where the fp32 value lies within rounding of a
half-step boundary, and the scales agree within 2e-6.
"""

import numpy as np
import pytest

from helpers import max_rel, same_bits

pytestmark = pytest.mark.gpu

OPS = {"identity": 0, "rmsnorm": 2, "silu_gate": 3}
# (seq, N, K): SmolVLA's expert (50 rows; 720 wide, 960 attention, 2048 MLP),
# ACT's decoder (100 rows), single rows, ragged N and K, the 128-row bound
SHAPES = [(50, 960, 720), (50, 4096, 720), (50, 720, 960), (50, 720, 2048), (1, 768, 768),
          (100, 512, 512), (7, 40, 68), (16, 16, 64), (33, 100, 260), (64, 2560, 960),
          (128, 96, 1024), (3, 17, 4)]


def _inputs(orc, seq, N, K, op):
    fr = orc.Frand()
    if op == 3:
        gu = fr.rv(seq * 2 * K, -4.0, 4.0).reshape(seq, 2 * K)
        x, u = gu[:, :K], gu[:, K:]
    else:
        x, u = fr.rv(seq * K, -3.0, 5.0).reshape(seq, K), None
    w = fr.rv(K, 0.5, 1.5)
    W = fr.rv(N * K, -0.2, 0.2).reshape(N, K)
    b = fr.rv(N)
    if seq > 2 and op != 3:
        x[1, :] = 0.0  # an all-zero row: scale 1, bytes 0
    return x, u, w, W, b


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run_both(vla, orc, torch, seq, N, K, op, act, accumulate, eps=1e-6):
    x, u, w, W, b = _inputs(orc, seq, N, K, op)
    Wq, ws = orc.quantize_weights_i8(W)
    ld = (K + 63) // 64 * 64
    Wp = np.zeros((N, ld), np.int8)
    Wp[:, :Wq.shape[1]] = Wq
    if op == 3:  # x and u are the two halves of one [seq, 2K] buffer, as after a gate|up GEMM
        gud = _dev(torch, np.concatenate([x, u], axis=1))
        xd, ud = gud[:, :K], gud[:, K:]
    else:
        xd, ud = _dev(torch, x), None
    wd = _dev(torch, w) if op == 2 else None
    Wd, wsd, bd = _dev(torch, Wp), _dev(torch, ws), _dev(torch, b)
    base = np.full((seq, N), 0.25, np.float32)

    xq = torch.full((vla.i8_panel_bytes(seq, K),), 0, dtype=torch.int8, device="cuda")
    sa = torch.empty(seq, dtype=torch.float32, device="cuda")
    vla.rowop_quantize_i8_panel_dev(op, xd, xq, sa, u=ud, w=wd, eps=eps)
    two = _dev(torch, base)
    vla.dense_linear_i8_panel_dev(two, xq, sa, Wd, wsd, bd, K, act=act, accumulate=accumulate)
    fused = _dev(torch, base)
    vla.rowop_linear_i8_dev(fused, op, xd, Wd, wsd, bd, u=ud, w=wd, eps=eps, act=act, accumulate=accumulate)
    torch.cuda.synchronize()
    return dict(x=x, u=u, w=w, Wq=Wq, ws=ws, b=b, base=base, xq=xq.cpu().numpy(), sa=sa.cpu().numpy(),
                two=two.cpu().numpy(), fused=fused.cpu().numpy())


def _rows_from_panel(buf, seq, K):
    mp, k64 = (seq + 15) // 16 * 16, (K + 63) // 64 * 64
    p = np.asarray(buf, np.int8)[: mp * k64].reshape(k64 // 64, mp, 64)
    return p.transpose(1, 0, 2).reshape(mp, k64)[:seq, :K]


@pytest.mark.parametrize("seq,N,K", SHAPES)
@pytest.mark.parametrize("opname", list(OPS))
def test_fused_equals_two_kernel_path(vla, orc, torch_cuda, seq, N, K, opname):
    op = OPS[opname]
    assert vla.rowop_linear_i8_fits(op, seq, K)
    r = _run_both(vla, orc, torch_cuda, seq, N, K, op, act=0, accumulate=0)
    assert same_bits(r["fused"], r["two"]), "fused row-op GEMM differs from row op + panel GEMM"

    # the two-kernel path against the oracle: GEMM bit-exact from its own bytes
    q = _rows_from_panel(r["xq"], seq, K)
    kp = (K + 3) // 4 * 4
    qpad = np.zeros((seq, kp), np.int8)
    qpad[:, :K] = q
    want = orc.dense_linear_i8_pre(qpad, r["sa"], r["Wq"], r["ws"], r["b"], K)
    assert same_bits(r["two"], want)

    # ... and its bytes / scales from the oracle's row op + quantizer
    if op == 0:
        y = r["x"]
    elif op == 2:
        y = orc.rmsnorm(np.ascontiguousarray(r["x"]), r["w"], 1e-6)
    else:
        y = orc.silu_gate(np.ascontiguousarray(r["x"]), np.ascontiguousarray(r["u"]))
    qo, so = orc.quantize_act_i8(y)
    d = np.abs(q.astype(np.int32) - qo[:, :K].astype(np.int32))
    if op == 0:
        assert d.max() == 0 and same_bits(r["sa"], so)
    else:
        assert d.max() <= 1 and np.mean(d) < 1e-3
        assert max_rel(r["sa"], so) <= 2e-6


@pytest.mark.parametrize("op", [0, 2, 3])
@pytest.mark.parametrize("act,accumulate", [(1, 1), (2, 0), (3, 1)])
def test_fused_epilogue_options(vla, orc, torch_cuda, op, act, accumulate):
    r = _run_both(vla, orc, torch_cuda, 50, 720, 960, op, act=act, accumulate=accumulate)
    assert same_bits(r["fused"], r["two"])


def test_fused_repeat_calls(vla, orc, torch_cuda):
    """The LDS panel starts unwritten in every block: a second call with other
    rows (fewer, narrower) gives its own two-kernel result, nothing left over."""
    a = _run_both(vla, orc, torch_cuda, 64, 300, 2048, 3, act=0, accumulate=0)
    b = _run_both(vla, orc, torch_cuda, 9, 300, 196, 2, act=0, accumulate=0)
    assert same_bits(a["fused"], a["two"]) and same_bits(b["fused"], b["two"])


def test_fits_and_rejects(vla, torch_cuda):
    torch = torch_cuda
    assert vla.rowop_linear_i8_fits(2, 128, 1024)
    assert not vla.rowop_linear_i8_fits(2, 129, 1024)     # more rows than a panel holds
    assert not vla.rowop_linear_i8_fits(2, 50, 2052)      # K past 2048
    assert not vla.rowop_linear_i8_fits(2, 50, 718)       # K not a multiple of 4
    assert not vla.rowop_linear_i8_fits(1, 50, 512)       # LayerNorm is not fused
    assert not vla.rowop_linear_i8_fits(2, 128, 2048)     # 128 x 2048 panel exceeds LDS
    x = torch.zeros((50, 720), dtype=torch.float32, device="cuda")
    Wq = torch.zeros((64, 768), dtype=torch.int8, device="cuda")
    ws = torch.ones(64, dtype=torch.float32, device="cuda")
    out = torch.zeros((50, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(vla.VlaError) as e:  # out overlapping the rows read
        vla.rowop_linear_i8_dev(x[:, :64], 0, x, Wq, ws, None)
    assert e.value.status == vla.VLA_ERR_ARG
    with pytest.raises(vla.VlaError) as e:
        vla.rowop_linear_i8_dev(out, 1, x, Wq, ws, None, w=ws)
    assert e.value.status == vla.VLA_ERR_ARG


@pytest.mark.parametrize("groups", ["1", "2", "3", "8"])
@pytest.mark.parametrize("seq,N,K,op", [(50, 720, 960, 0), (100, 512, 512, 2), (128, 96, 1024, 3),
                                        (33, 100, 260, 2), (50, 720, 2048, 3)])
def test_fused_row_groups(vla, orc, torch_cuda, groups, seq, N, K, op):
    """Row groups (each block applies the row op to its own 16 x FM rows and
    multiplies them by its 16 columns) give the two-kernel path's outputs bit
    for bit, whatever the forced group count."""
    import os
    os.environ["VLA_HIP_SKINNY_R"] = os.environ["VLA_HIP_ROWOP_R"] = groups
    try:
        r = _run_both(vla, orc, torch_cuda, seq, N, K, op, act=1, accumulate=1)
    finally:
        del os.environ["VLA_HIP_SKINNY_R"], os.environ["VLA_HIP_ROWOP_R"]
    assert same_bits(r["fused"], r["two"]), f"{groups} row groups differ from the two-kernel path"
