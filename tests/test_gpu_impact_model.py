"""IMPACT end to end through the reference's own entry points (vla_impact_load
/ _set_instruction / _predict / _tokens / _film, include/vla_simd.h:206-243):
uint8 frames + raw state + an instruction -> actions on the device, against the
reference's ImpactModel (src/models/impact/impact_model.cpp, t5_text.cpp,
impact_capi.cpp) built into oracle/_ref from its own sources, on a synthetic
checkpoint in the reference's file layout (checkpoints.write_impact_model).

Bars:
  * tokens (ids, compacted ids, mask): equal, including words outside the
    pruned vocabulary (substituted with <unk>) and instructions longer than
    n_text;
  * FiLM gamma / beta: T5-small, the mean pool and the FiLM head in fp32 on
    the matrix cores against the reference's fp32 GEMMs (summation order
    only): within 1e-4 of their scale;
  * actions, fp32 trunk and transformer (IMPACT_INT8 0): within 1e-3 of the
    output scale, as ACT's;
  * actions with every group int8 (IMPACT_INT8 63): the int8 trunk reads
    FiLM-modulated maps whose gamma / beta carry the fp32 text tower's
    summation-order differences, so a quantized byte may flip; within 2e-2.
IMPACT_INT8 is read at load by both sides, as the reference reads it.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from helpers import load_pkg

pytestmark = pytest.mark.gpu

ENV = ("IMPACT_INT8", "IMPACT_I8_CONV_FROM", "IMPACT_I8_CONV_TO")
INSTR = ["pick up the red block", "put the cube in the bowl and then close the drawer slowly please",
         "zzqx blorp the red block", ""]


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


def _small(ck):
    return dict(ck.IMPACT_MODEL_BASE, img_h=96, img_w=128, n_cams=2, width=16, dim=128, heads=4, head_dim=32,
                ff=256, n_enc=2, n_text=8,
                t5=dict(ck.IMPACT_T5, d_model=64, n_layers=2, n_heads=4, d_kv=16, d_ff=128))


@pytest.fixture
def env():
    saved = {k: os.environ.get(k) for k in ENV}

    def set_(**kv):
        for k in ENV:
            os.environ.pop(k, None)
        for k, v in kv.items():
            os.environ[k] = str(v)
    yield set_
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


@pytest.fixture(scope="module")
def small_dir(tmp_path_factory):
    ck = _ck()
    return ck.write_impact_model(str(tmp_path_factory.mktemp("impact") / "small"), _small(ck))


def _rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got))
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _inputs(ck, c):
    return ck.act_model_inputs(c)


def test_server_binding_dims_and_errors(vla, small_dir, env):
    """The library binds the way vla_simd/policy_server.py:309-345 binds
    IMPACT: ctypes symbols vla_impact_load/free/<ints>/predict with the
    server's argtypes; dims agree with the reference; the status codes of
    impact_capi.cpp for null arguments, a missing instruction and a bad
    directory."""
    from helpers import oracle
    ob = oracle()
    env()
    lib = ctypes.CDLL(vla.LIB_PATH)
    vp, f32p, u8p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint8)
    lib.vla_impact_load.argtypes, lib.vla_impact_load.restype = [ctypes.c_char_p], vp
    lib.vla_impact_free.argtypes, lib.vla_impact_free.restype = [vp], None
    ints = ("chunk", "action_dim", "state_dim", "n_cams", "img_h", "img_w", "n_text")
    for i in ints:
        f = getattr(lib, f"vla_impact_{i}")
        f.argtypes, f.restype = [vp], ctypes.c_int32
    lib.vla_impact_predict.argtypes = [vp, u8p, f32p, ctypes.c_char_p, ctypes.c_int32, f32p]
    lib.vla_impact_predict.restype = ctypes.c_int32
    lib.vla_impact_tokens.argtypes = [vp, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32]
    lib.vla_impact_tokens.restype = ctypes.c_int32
    lib.vla_impact_film.argtypes = [vp, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32]
    lib.vla_impact_film.restype = ctypes.c_int32
    h = lib.vla_impact_load(small_dir.encode())
    assert h
    try:
        got = {i: getattr(lib, f"vla_impact_{i}")(h) for i in ints}
        r = ob.RefImpactModel(small_dir)
        assert got == dict(chunk=r.chunk, action_dim=r.action_dim, state_dim=r.state_dim, n_cams=r.n_cams,
                           img_h=r.img_h, img_w=r.img_w, n_text=r.n_text)
        # before any instruction: tokens and film are VLA_ERR_ARG, as the reference's
        assert lib.vla_impact_tokens(h, None, None, None, 64) == -1 == r.tokens()[0]
        assert lib.vla_impact_film(h, None, None, 1 << 20) == -1 == r.film()[0]
        ck = _ck()
        images, state = _inputs(ck, _small(ck))
        out = np.empty((got["chunk"], got["action_dim"]), np.float32)
        rc = lib.vla_impact_predict(h, images.ctypes.data_as(u8p), state.ctypes.data_as(f32p), INSTR[0].encode(),
                                    1, out.ctypes.data_as(f32p))
        assert rc == 0 and np.all(np.isfinite(out))
        assert lib.vla_impact_predict(h, None, state.ctypes.data_as(f32p), b"x", 1, out.ctypes.data_as(f32p)) == -1
        assert lib.vla_impact_predict(h, images.ctypes.data_as(u8p), state.ctypes.data_as(f32p), None, 1,
                                      out.ctypes.data_as(f32p)) == -1
        n = got["n_text"]
        assert lib.vla_impact_tokens(h, None, None, None, n - 1) == -1  # short buffer
        assert lib.vla_impact_tokens(h, None, None, None, n) == n
        assert lib.vla_impact_chunk(None) == 0
    finally:
        lib.vla_impact_free(h)
    assert lib.vla_impact_load(b"/nonexistent/impact") is None


def test_tokens_and_film_match_reference(vla, small_dir, env):
    """The language pathway: ids, the pruned-vocabulary remap (<unk> for the
    words the table lacks) and the mask equal the reference's; FiLM gamma /
    beta within 1e-4 of their scale; re-setting the same instruction is a
    no-op and a new one changes them."""
    from helpers import oracle
    ob = oracle()
    env()
    r = ob.RefImpactModel(small_dir)
    m = vla.ImpactModel(small_dir)
    prev = None
    for s in INSTR:
        assert r.set_instruction(s) == 0
        m.set_instruction(s)
        n, rid, rcomp, rmask = r.tokens()
        ids, comp, mask = m.tokens()
        assert n == m.n_text
        assert ids.tolist() == rid.tolist() and comp.tolist() == rcomp.tolist() and mask.tolist() == rmask.tolist()
        nf, rg, rb = r.film()
        g, b = m.film()
        assert nf == g.size == b.size == 240
        eg, eb = _rel(g, rg), _rel(b, rb)
        print(f"impact film '{s[:20]}': gamma rel {eg:.2e}, beta rel {eb:.2e}", flush=True)
        assert eg <= 1e-4 and eb <= 1e-4
        m.set_instruction(s)  # cached
        assert m.film()[0].tobytes() == g.tobytes()
        if prev is not None:
            assert not np.array_equal(prev, g)
        prev = g
    # the OOV instruction maps unknown pieces to <unk>'s row
    m.set_instruction(INSTR[2])
    ids, comp, mask = m.tokens()
    vmap = np.fromfile(os.path.join(small_dir, "vocab_map.bin"), np.int32)
    unk = vmap[2]
    assert all((vmap[i] if vmap[i] >= 0 else unk) == c for i, c in zip(ids.tolist(), comp.tolist()))
    assert any(vmap[i] < 0 for i in ids[mask.astype(bool)].tolist())


@pytest.mark.parametrize("mask", [0, 31, 63])
def test_actions_match_reference(vla, small_dir, env, mask):
    """Actions against the reference's ImpactModel for several instructions:
    fp32 (0), int8 transformer (31), and int8 trunk + transformer (63)."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    env(IMPACT_INT8=mask)
    c = _small(ck)
    images, state = _inputs(ck, c)
    r = ob.RefImpactModel(small_dir)
    m = vla.ImpactModel(small_dir)
    assert (m.int8_layers > 0) == bool(mask & 31) and (m.int8_convs > 0) == bool(mask & 32)
    bar = {0: 1e-3, 31: 5e-3, 63: 2e-2}[mask]
    for s in INSTR[:3]:
        st, ref = r.predict(images, state, s, unnormalize=False)
        assert st == 0
        got = m.predict(images, state, s, unnormalize=False)
        err = _rel(got, ref)
        print(f"impact mask {mask} '{s[:20]}': action rel err {err:.3e} (bar {bar:.0e})", flush=True)
        assert err <= bar
        # graph replays reproduce the pass, and un-normalization is v * std + mean
        assert m.predict(images, state, s, unnormalize=False).tobytes() == got.tobytes()
    st = np.fromfile(os.path.join(small_dir, "stats.bin"), np.float32)
    sd, ad = m.state_dim, m.action_dim
    un = m.predict(images, state, INSTR[0], unnormalize=True)
    base = m.predict(images, state, INSTR[0], unnormalize=False)
    want = base.astype(np.float64) * st[2 * sd + ad:2 * sd + 2 * ad] + st[2 * sd:2 * sd + ad]
    assert _rel(un, want) <= 1e-6


def test_film_modulates_the_trunk(vla, small_dir, env, tmp_path):
    """The FiLM points matter: a checkpoint whose FiLM head is zero (gamma =
    beta = 0, the identity modulation) gives the same actions as the
    reference's, and different actions from the trained head; a checkpoint
    whose film_after points disagree with the head's width does not load."""
    import shutil
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    env()
    c = _small(ck)
    d = str(tmp_path / "zero")
    shutil.copytree(small_dir, d)
    meta = dict(l.split() for l in open(os.path.join(d, "text.meta")) if l.strip())
    F, D = int(meta["film_total"]), int(meta["d_model"])
    tb = np.fromfile(os.path.join(d, "text.bin"), np.float32)
    tb[tb.size - (2 * F * D + 2 * F):] = 0.0
    tb.tofile(os.path.join(d, "text.bin"))
    images, state = _inputs(ck, c)
    mz = vla.ImpactModel(d)
    mz.set_instruction(INSTR[0])
    g, b = mz.film()
    assert not g.any() and not b.any()
    got = mz.predict(images, state, INSTR[0], unnormalize=False)
    st, ref = ob.RefImpactModel(d).predict(images, state, INSTR[0], unnormalize=False)
    assert st == 0 and _rel(got, ref) <= 1e-3
    trained = vla.ImpactModel(small_dir).predict(images, state, INSTR[0], unnormalize=False)
    assert _rel(trained, got) > 1e-3
    # film_after without the last point: the head emits more channels than the trunk takes
    bad = str(tmp_path / "bad")
    shutil.copytree(small_dir, bad)
    lines = [l for l in open(os.path.join(bad, "vision.meta")) if l.strip() != "film_after 7"]
    open(os.path.join(bad, "vision.meta"), "w").writelines(lines)
    with pytest.raises(vla.VlaError):
        vla.ImpactModel(bad)
    with pytest.raises(RuntimeError):
        ob.RefImpactModel(bad)


def test_loads_from_gguf(vla, small_dir, env, tmp_path):
    """The same checkpoint packed into one vla.simd GGUF (the format
    tools/_gguf.py writes, which the reference mounts through io::Mount):
    our actions from the GGUF are byte-identical to the directory's, and the
    reference loads the GGUF too."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    env(IMPACT_INT8=31)
    g = ck.write_gguf(small_dir, str(tmp_path / "impact.gguf"), "impact")
    images, state = _inputs(ck, _small(ck))
    a = vla.ImpactModel(small_dir).predict(images, state, INSTR[0], unnormalize=True)
    b = vla.ImpactModel(g).predict(images, state, INSTR[0], unnormalize=True)
    assert a.tobytes() == b.tobytes()
    st, ref = ob.RefImpactModel(g).predict(images, state, INSTR[0], unnormalize=True)
    assert st == 0 and _rel(b, ref) <= 5e-3
