"""GPU parity of LayerNorm / RMSNorm / RoPE / activations.

Norms: 1e-5 absolute of the double formula (test_ops.cpp:296-321) and close
to the oracle (same double accumulation). Activations: 2e-6 of max(|ref|,1)
against the libm double formula over [-30, 30] (test_ops.cpp:272-294), NaN in
gives NaN out.
"""

import math

import numpy as np
import pytest

from helpers import load_synth, max_rel, same_bits

pytestmark = pytest.mark.gpu

NORM_SHAPES = [(1, 768), (50, 960), (7, 6), (302, 512), (658, 768), (177, 960), (50, 720), (3, 4097)]


def _norm_case(orc, seq, H):
    fr = orc.Frand()
    return fr.rv(seq * H, -3.0, 5.0).reshape(seq, H), fr.rv(H), fr.rv(H)


@pytest.mark.parametrize("seq,H", NORM_SHAPES)
def test_layernorm(vla, orc, seq, H):
    x, w, b = _norm_case(orc, seq, H)
    got = vla.layernorm(x, w, b, 1e-5)
    xd = x.astype(np.float64)
    mu = xd.mean(axis=1, keepdims=True)
    var = ((xd - mu) ** 2).mean(axis=1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-5) * w + b
    assert np.max(np.abs(got - ref)) <= 1e-5
    assert np.max(np.abs(got - orc.layernorm(x, w, b, 1e-5))) <= 2e-6
    nob = vla.layernorm(x, w, None, 1e-6)
    assert np.max(np.abs(nob - orc.layernorm(x, w, None, 1e-6))) <= 2e-6


@pytest.mark.parametrize("seq,H", NORM_SHAPES)
def test_rmsnorm(vla, orc, seq, H):
    x, w, _ = _norm_case(orc, seq, H)
    got = vla.rmsnorm(x, w, 1e-6)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(got - ref)) <= 1e-5
    # same double sum, same float rounding steps: equal up to the last-bit effect
    # of a different summation order inside the double
    assert np.max(np.abs(got - orc.rmsnorm(x, w, 1e-6))) <= 1e-6


def test_layernorm_in_place(vla, orc, torch_cuda):
    torch = torch_cuda
    x, w, b = _norm_case(orc, 302, 512)
    xd = torch.from_numpy(x).cuda()
    wd, bd = torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda()
    import ctypes
    vla.check("vla_layernorm_dev", vla.lib().vla_layernorm_dev(
        ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(wd.data_ptr()),
        ctypes.c_void_p(bd.data_ptr()), 302, 512, ctypes.c_float(1e-5),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    assert same_bits(xd.cpu().numpy(), vla.layernorm(x, w, b, 1e-5))


def _eltwise_input(orc):
    return orc.Frand().rv(20011, -30.0, 30.0)


@pytest.mark.parametrize("name,fn", [
    ("gelu_tanh", lambda v: 0.5 * v * (1.0 + math.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))),
    ("gelu_erf", lambda v: 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0)))),
    ("relu", lambda v: max(v, 0.0)),
])
def test_activations(vla, orc, name, fn):
    x = _eltwise_input(orc)
    got = getattr(vla, name)(x)
    ref = np.array([fn(float(v)) for v in x])
    assert np.all(np.isfinite(got))
    assert max_rel(got, ref) <= 2e-6
    assert max_rel(got, getattr(orc, name)(x)) <= 2e-6
    nan = getattr(vla, name)(np.array([np.nan], np.float32))
    assert np.isnan(nan[0]) or name == "relu"


def test_silu_gate(vla, orc):
    x = _eltwise_input(orc)
    u = orc.Frand(12345).rv(x.size, -2.0, 2.0)
    got = vla.silu_gate(x, u)
    ref = np.array([float(g) / (1.0 + math.exp(-float(g))) * float(uu) for g, uu in zip(x, u)])
    assert max_rel(got, ref) <= 2e-6
    assert max_rel(got, orc.silu_gate(x, u)) <= 2e-6


def test_rope_neox(vla, orc):
    s = load_synth()
    for seq, nh, hd in ((177, 15, 64), (50, 5, 64), (7, 3, 16)):
        x = s.normal(f"rope.{seq}", (seq, nh * hd))
        pos = np.arange(seq, dtype=np.int32) + 3
        got = vla.rope_neox(x, pos, nh, hd, 10000.0)
        want = orc.rope_neox(x, pos, nh, hd, 10000.0)
        assert np.max(np.abs(got - want)) <= 1e-6 * max(1.0, float(np.max(np.abs(want))))
