"""Octo end to end through the reference's own entry points (vla_octo_load /
vla_octo_predict / vla_octo_predict_ex, include/vla_simd.h:126-153):
pre-resized uint8 frames -> SmallStems -> block transformer with the T5
embedding of the instruction -> readout -> DDPM head -> actions, on the
device, against the reference's OctoModel and octo_capi.cpp compiled into
oracle/_ref.

Bars:
  * dims and status codes: identical;
  * the T5 embedding: within 1e-4 of its scale (fp32, summation order);
  * actions, fp32 (OCTO_INT8 unset): within 1e-3 of the output scale; the
    default noise drawn from mt19937_64(seed) meets the same bar;
  * actions, int8 groups: twice the reference's own spread under two seeded
    1-ulp perturbations of its stem tokens (the class of difference fp32
    stem convolutions leave), floor 1e-3.
The reference latches OCTO_INT8 once per process, so every reference load
runs with the variable unset; int8 references come from ref_octo_model_load,
tied to the library's own vla_octo_predict_ex bit for bit at mask 0.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from helpers import load_pkg, oracle

pytestmark = pytest.mark.gpu

ENV = "OCTO_INT8"
TEXT = "pick up the red block"


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


def _small(ck):
    t5 = dict(ck.T5_BASE, d_model=128, n_layers=2, n_heads=2, d_kv=64, d_ff=256, vocab=1024)
    stem = dict(ck.OCTO_STEM_BASE, features=(16, 32, 32, 64), embed_dim=64, gn_groups=8)
    tf = dict(ck.OCTO_BASE, d=128, n_layers=2, heads=2, head_dim=64, mlp=256, max_horizon=2, stem_dim=64,
              t5_dim=128, repeat_task=1)
    head = dict(ck.OCTO_HEAD_BASE, hidden=64, num_blocks=2, steps=5)
    return dict(t5=t5, stem=stem, tf=tf, head=head)


@pytest.fixture
def env():
    saved = os.environ.get(ENV)

    def set_(v):
        if v is None:
            os.environ.pop(ENV, None)
        else:
            os.environ[ENV] = str(v)
    yield set_
    set_(saved)


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    ck = _ck()
    c = _small(ck)
    return ck.write_octo_model(str(tmp_path_factory.mktemp("octom") / "small"), c), c


def _rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got))
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _ref(ob, d, env, mask=None):
    env(None)  # the reference reads OCTO_INT8 once per process: keep it at 0
    return ob.RefOctoModel(d, int8_mask=mask)


def test_dims_and_status_codes(vla, small, env):
    d, c = small
    ck = _ck()
    ob = oracle()
    r = _ref(ob, d, env)
    m = vla.OctoModel(d)
    assert (m.horizon, m.action_dim, m.max_window) == (r.horizon, r.action_dim, r.max_window) == (4, 7, 2)
    p, w, tm, n, z = ck.octo_model_inputs(c)
    L, RL = vla.lib(), ob._ref_models()
    out = np.zeros((m.horizon, m.action_dim), np.float32)
    P = lambda a: None if a is None else a.ctypes.data_as(__import__("ctypes").c_void_p)  # noqa: E731
    cases = [("wnd 0", dict(wnd=0)), ("wnd beyond max_window", dict(wnd=3)), ("noise without z", dict(z=None)),
             ("z without noise", dict(noise=None)), ("null primary", dict(p=None)), ("null mask", dict(tm=None))]
    for name, kw in cases:
        a = dict(p=p, w=w, wnd=2, tm=tm, noise=n, z=z)
        a.update(kw)
        args = (P(a["p"]), P(a["w"]), a["wnd"], P(a["tm"]), TEXT.encode(), P(a["noise"]), P(a["z"]), 0, 1, P(out))
        ours, theirs = L.vla_octo_predict_ex(m.h, *args), RL.vla_octo_predict_ex(r.h, *args)
        print(f"{name}: ours {ours}, reference {theirs}", flush=True)
        assert ours == theirs and ours != 0, name
    assert L.vla_octo_horizon(None) == 0


def test_t5_embedding(vla, small, env):
    d, c = small
    ob = oracle()
    shim = _ref(ob, d, env, 0)
    m = vla.OctoModel(d)
    for text in (TEXT, "place the cup on the plate, then open the drawer and push the green button twice",
                 "unknown ЖЖЖ 🤖", ""):
        ref = shim.lang(text)
        got = m.lang(text, shim.n_task, shim.t5_dim)
        err = _rel(got, ref)
        print(f"t5 {text[:20]!r}: rel err {err:.3e}", flush=True)
        assert err <= 1e-4


def test_predict_fp32(vla, small, env):
    d, c = small
    ck = _ck()
    ob = oracle()
    r = _ref(ob, d, env)
    shim = _ref(ob, d, env, 0)
    m = vla.OctoModel(d)
    assert m.int8_layers == 0
    p, w, tm, n, z = ck.octo_model_inputs(c)
    for unnorm in (True, False):
        st, ref = r.predict(p, w, tm, TEXT, noise=n, z=z, unnormalize=unnorm)
        assert st == 0
        _, ref2 = shim.predict(p, w, tm, TEXT, noise=n, z=z, unnormalize=unnorm)
        assert ref2.tobytes() == ref.tobytes(), "shim path differs from vla_octo_predict_ex"
        got = m.predict(p, w, tm, TEXT, noise=n, z=z, unnormalize=unnorm)
        err = _rel(got, ref)
        print(f"octo model fp32 unnormalize={unnorm}: rel err {err:.3e}", flush=True)
        assert err <= 1e-3
    # the default noise from mt19937_64(seed), on both sides
    st, ref = r.predict(p, w, tm, TEXT, seed=77)
    got = m.predict(p, w, tm, TEXT, seed=77)
    assert st == 0 and _rel(got, ref) <= 1e-3
    # without the wrist camera, with a padded history step
    tm0 = np.array([0, 1], np.uint8)
    st, ref = r.predict(p, None, tm0, TEXT, noise=n, z=z)
    got = m.predict(p, None, tm0, TEXT, noise=n, z=z)
    assert st == 0 and _rel(got, ref) <= 1e-3


def test_window_reuse(vla, small, env):
    """Frames repeated inside a window and shifted across calls reuse their
    stem tokens; the actions are the same as a fresh model's."""
    d, c = small
    ck = _ck()
    m = vla.OctoModel(d)
    p, w, tm, n, z = ck.octo_model_inputs(c)
    p2, w2 = p.copy(), w.copy()
    p2[1], w2[1] = p[0], w[0]  # a repeated frame within the window
    first = m.predict(p2, w2, tm, TEXT, noise=n, z=z)
    shifted_p = np.stack([p[1], p[0]])
    shifted_w = np.stack([w[1], w[0]])
    second = m.predict(shifted_p, shifted_w, tm, TEXT, noise=n, z=z)  # both frames seen last call
    fresh = vla.OctoModel(d)
    assert fresh.predict(p2, w2, tm, TEXT, noise=n, z=z).tobytes() == first.tobytes()
    fresh2 = vla.OctoModel(d)
    assert fresh2.predict(shifted_p, shifted_w, tm, TEXT, noise=n, z=z).tobytes() == second.tobytes()


@pytest.mark.parametrize("mask", [7, 24, 32, 63])
def test_predict_int8(vla, small, env, mask):
    d, c = small
    ck = _ck()
    ob = oracle()
    shim = _ref(ob, d, env, mask)
    env(mask)
    m = vla.OctoModel(d)
    assert m.int8_layers > 0
    p, w, tm, n, z = ck.octo_model_inputs(c)
    _, ref = shim.predict(p, w, tm, TEXT, noise=n, z=z)
    spread = max(_rel(shim.predict(p, w, tm, TEXT, noise=n, z=z, perturb=k)[1], ref) for k in (1, 2))
    bar = max(2.0 * spread, 1e-3)
    got = m.predict(p, w, tm, TEXT, noise=n, z=z)
    err = _rel(got, ref)
    print(f"octo model OCTO_INT8={mask}: rel err {err:.3e} (bar {bar:.3e}), int8 layers {m.int8_layers}",
          flush=True)
    assert err <= bar


def test_octo_model_full_size(vla, env, tmp_path):
    """BASELINE's Octo-base transformer (12 x 768) with the T5-base encoder,
    the SmallStem16 towers at 256 x 256 / 128 x 128, two timesteps (the
    reference's 690-token layout) and the 20-step DDPM head; OCTO_INT8=7."""
    ck = _ck()
    ob = oracle()
    c = ck.OCTO_MODEL_BASE
    d = ck.write_octo_model(str(tmp_path / "octo_full"), c)
    shim = _ref(ob, d, env, 7)
    env(7)
    m = vla.OctoModel(d)
    p, w, tm, n, z = ck.octo_model_inputs(c)
    _, ref = shim.predict(p, w, tm, TEXT, noise=n, z=z)
    spread = max(_rel(shim.predict(p, w, tm, TEXT, noise=n, z=z, perturb=k)[1], ref) for k in (1, 2))
    bar = max(2.0 * spread, 1e-3)
    got = m.predict(p, w, tm, TEXT, noise=n, z=z)
    err = _rel(got, ref)
    print(f"octo model full size: rel err {err:.3e} (bar {bar:.3e})", flush=True)
    assert err <= bar


@pytest.mark.parametrize("mask", [0, 32, 63])
def test_fused_head_matches_layer_kernels(vla, small, env, mask):
    """The DDPM head as one workgroup against the same head as separate
    kernels (VLA_OCTO_HEAD_FUSED=0). Its int8 layers (OCTO_INT8 bit 32) repeat
    the separate kernels' arithmetic (quantized rows, exact integer sums, the
    epilogue, LayerNorm, the update); its fp32 layers - all of them at mask 0,
    and the 28-wide output projection, which int8_fits leaves fp32, at every
    mask - sum their dot products in another order (measured at masks 0,
    32, 63: 3.8e-8, 9.5e-9, 3.8e-8 of the output scale); bar 1e-6."""
    d, c = small
    ck = _ck()
    env(mask)
    p, w, tm, n, z = ck.octo_model_inputs(c)
    os.environ["VLA_OCTO_HEAD_FUSED"] = "0"
    try:
        ref = vla.OctoModel(d).predict(p, w, tm, TEXT, noise=n, z=z)
    finally:
        del os.environ["VLA_OCTO_HEAD_FUSED"]
    got = vla.OctoModel(d).predict(p, w, tm, TEXT, noise=n, z=z)
    print(f"fused head OCTO_INT8={mask}: rel diff {_rel(got, ref):.3e}", flush=True)
    assert _rel(got, ref) <= 1e-6
