"""SmolVLA end to end through the reference's own entry points
(vla_smolvla_load / _tokenize / _predict / _predict_rtc, include/vla_simd.h:
83-124): native-size uint8 frames -> resize_with_pad -> SigLIP per view,
language embeddings, projected state -> prefix tower -> flow-matching denoise
(optionally guided) -> un-normalized actions, on the device, against the
reference's SmolvlaModel and smolvla_capi.cpp compiled into oracle/_ref.

Bars:
  * dims, tokenize (ids, mask, count) and the status codes: identical;
  * resize_with_pad: bit-exact (the same double arithmetic, rounded to float);
  * actions, fp32 graph (SMOLVLA_INT8 unset): within 1e-3 of the output scale
    (summation order only); the default noise drawn from mt19937_64(seed)
    meets the same bar, so both draw the same numbers;
  * actions, int8 groups: twice the reference's own spread under two seeded
    1-ulp perturbations of its preprocessed pixels (the class of difference
    the fp32 parts upstream of the int8 layers leave), as the graph tests do
    with their inputs.
The reference latches SMOLVLA_INT8 once per process, so every reference load
here runs with the variable unset; int8 references come from
ref_smolvla_model_load, which applies a given mask's groups, and that path is
tied to the library's own vla_smolvla_predict_rtc bit for bit at mask 0.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from helpers import load_pkg, oracle

pytestmark = pytest.mark.gpu

ENV = "SMOLVLA_INT8"


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


def _small(ck):
    vit = dict(hidden=192, n_heads=3, head_dim=64, inter=768, n_layers=2, patch=16, img=128, n_patches=64,
               ln_eps=1e-6, scale_factor=2, mm_out=256, n_img_tok=16)
    tf = dict(ck.SMOLVLA_BASE, hidden=256, n_q=4, n_kv=2, head_dim=64, ffn=512, n_layers=4, expert_h=192,
              expert_ffn=384, expert_layers=4, chunk=12, num_steps=4)
    return dict(ck.SMOLVLA_MODEL_BASE, vit=vit, tf=tf, vocab=512, tok_maxlen=16)


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
    return ck.write_smolvla_model(str(tmp_path_factory.mktemp("smolm") / "small"), c), c


def _rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got))
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _ref(ob, d, env, mask=None):
    env(None)  # the reference reads SMOLVLA_INT8 once per process: keep it at 0
    return ob.RefSmolvlaModel(d, int8_mask=mask)


TEXTS = ["pick up the red block", "don't drop the sponge!\n\n", "move 10 cm to the left",
         "place the cup on the plate, then open the drawer and push the green button twice",
         "café 🤖 Привет", ""]


def test_dims_and_tokenize(vla, small, env):
    d, c = small
    ob = oracle()
    r = _ref(ob, d, env)
    m = vla.SmolvlaModel(d)
    rd = r.dims()
    assert rd == dict(chunk=m.chunk, action_dim=m.action_dim, state_dim=m.state_dim, n_views=m.n_views,
                      img_size=m.img_size, tok_maxlen=m.tok_maxlen)
    assert m.tok_maxlen == 16 and m.img_size == 128 and m.chunk == 12
    for t in TEXTS:
        ids, mask, n = m.tokenize(t)
        rids, rmask, rn = r.tokenize(t, m.tok_maxlen)
        assert n == rn and ids.tolist() == rids.tolist() and mask.tolist() == rmask.tolist(), repr(t)
    # the long instruction keeps its last tok_maxlen tokens
    assert m.tokenize(TEXTS[3])[2] == m.tok_maxlen
    L = vla.lib()
    assert L.vla_smolvla_tokenize(m.h, None, None, None) == -1
    assert L.vla_smolvla_chunk(None) == 0


@pytest.mark.parametrize("hw", [(480, 640), (640, 480), (128, 128), (100, 37), (7, 300)])
def test_resize_with_pad_bit_exact(vla, small, hw):
    d, c = small
    ob = oracle()
    m = vla.SmolvlaModel(d)
    r = np.random.default_rng(hw[0] * 1000 + hw[1])
    frames = r.integers(0, 256, size=(2, hw[0], hw[1], 3), dtype=np.uint8)
    got = m.preprocess(frames)
    for v in range(2):
        want = ob.ref_resize_with_pad(frames[v], m.img_size)
        assert got[v].tobytes() == want.tobytes(), f"view {v} of {hw}"


def _inputs(ck, c, m, text="pick up the red block"):
    frames, state, noise = ck.smolvla_model_inputs(c, height=96, width=160)
    ids, mask, _ = m.tokenize(text)
    return frames, ids, mask, state, noise


def test_predict_fp32(vla, small, env):
    d, c = small
    ck = _ck()
    ob = oracle()
    r = _ref(ob, d, env)
    shim = _ref(ob, d, env, 0)
    m = vla.SmolvlaModel(d)
    assert m.int8_layers == 0
    frames, ids, mask, state, noise = _inputs(ck, c, m)
    st, ref = r.predict(frames, ids, mask, state, m.chunk, m.action_dim, noise=noise)
    assert st == 0
    st2, ref2 = shim.predict(frames, ids, mask, state, m.chunk, m.action_dim, noise=noise)
    assert st2 == 0 and ref2.tobytes() == ref.tobytes(), "shim path differs from vla_smolvla_predict_rtc"
    got = m.predict(frames, ids, mask, state, noise=noise)
    err = _rel(got, ref)
    print(f"smolvla model fp32: rel err {err:.3e}, graph nodes {m.graph_nodes}", flush=True)
    assert err <= 1e-3
    for _ in range(2):  # graph replays reproduce the first call
        assert m.predict(frames, ids, mask, state, noise=noise).tobytes() == got.tobytes()
    # the default noise: N(0, 1) from mt19937_64(seed) on both sides
    st, ref_s = r.predict(frames, ids, mask, state, m.chunk, m.action_dim, noise=None, seed=1234)
    got_s = m.predict(frames, ids, mask, state, noise=None, seed=1234)
    assert st == 0 and _rel(got_s, ref_s) <= 1e-3
    assert _rel(got_s, got) > 1e-2  # a different draw than the given noise


def test_predict_rtc(vla, small, env):
    d, c = small
    ck = _ck()
    ob = oracle()
    r = _ref(ob, d, env)
    m = vla.SmolvlaModel(d)
    frames, ids, mask, state, noise = _inputs(ck, c, m, "move 10 cm to the left")
    rng = np.random.default_rng(3)
    prev = rng.normal(0, 1.5, size=(5, m.action_dim)).astype(np.float32)
    weights = np.linspace(1.0, 0.0, m.chunk).astype(np.float32)
    plain = m.predict(frames, ids, mask, state, noise=noise)
    for mg in (1.5, 0.25):
        st, ref = r.predict(frames, ids, mask, state, m.chunk, m.action_dim, noise=noise, prev=prev,
                            weights=weights, max_guidance=mg)
        assert st == 0
        got = m.predict(frames, ids, mask, state, noise=noise, prev=prev, weights=weights, max_guidance=mg)
        err = _rel(got, ref)
        print(f"smolvla model rtc max_guidance {mg}: rel err {err:.3e}, "
              f"guided vs plain {_rel(got, plain):.3e}", flush=True)
        assert err <= 1e-3
        assert _rel(got, plain) > 1e-3  # the guidance changed the chunk
    # back to the unguided graph
    assert m.predict(frames, ids, mask, state, noise=noise).tobytes() == plain.tobytes()


def test_alternating_guided_and_plain_chunks_replay(vla, small, env):
    """A caller that alternates guided (RTC) and plain chunks keeps a captured
    graph per mode: after the first two calls of each mode every call replays
    (graph nodes as when one mode runs alone), and each mode's outputs stay
    bit-identical from call to call."""
    d, c = small
    ck = _ck()
    env(None)
    m = vla.SmolvlaModel(d)
    frames, ids, mask, state, noise = _inputs(ck, c, m, "move 10 cm to the left")
    rng = np.random.default_rng(5)
    prev = rng.normal(0, 1.5, size=(4, m.action_dim)).astype(np.float32)
    weights = np.linspace(1.0, 0.0, m.chunk).astype(np.float32)
    plain = lambda: m.predict(frames, ids, mask, state, noise=noise)
    guided = lambda: m.predict(frames, ids, mask, state, noise=noise, prev=prev, weights=weights,
                               max_guidance=1.5)
    outs, nodes = {"p": [], "g": []}, {"p": [], "g": []}
    for _ in range(4):
        for k, f in (("p", plain), ("g", guided)):
            outs[k].append(f().tobytes())
            nodes[k].append(m.graph_nodes)
    solo = vla.SmolvlaModel(d)
    solo_nodes = {}
    for k, f in (("p", lambda: solo.predict(frames, ids, mask, state, noise=noise)),
                 ("g", lambda: solo.predict(frames, ids, mask, state, noise=noise, prev=prev, weights=weights,
                                            max_guidance=1.5))):
        for _ in range(3):
            f()
        solo_nodes[k] = solo.graph_nodes
    print(f"alternating modes: graph nodes {nodes}, alone {solo_nodes}", flush=True)
    for k in ("p", "g"):
        assert len(set(outs[k])) == 1, f"mode {k} changed between calls"
        assert nodes[k][2:] == [solo_nodes[k]] * 2 and solo_nodes[k] > 0
    assert outs["p"][0] != outs["g"][0]


@pytest.mark.parametrize("mask", [15, 48, 63])
def test_predict_int8(vla, small, env, mask):
    d, c = small
    ck = _ck()
    ob = oracle()
    shim = _ref(ob, d, env, mask)
    env(mask)
    m = vla.SmolvlaModel(d)
    assert m.int8_layers > 0
    frames, ids, lmask, state, noise = _inputs(ck, c, m)
    st, ref = shim.predict(frames, ids, lmask, state, m.chunk, m.action_dim, noise=noise)
    assert st == 0
    spread = max(_rel(shim.predict(frames, ids, lmask, state, m.chunk, m.action_dim, noise=noise, perturb=k)[1],
                      ref) for k in (1, 2))
    bar = max(2.0 * spread, 1e-3)
    got = m.predict(frames, ids, lmask, state, noise=noise)
    err = _rel(got, ref)
    print(f"smolvla model SMOLVLA_INT8={mask}: rel err {err:.3e} (bar {bar:.3e}), int8 layers {m.int8_layers}",
          flush=True)
    assert err <= bar


def test_status_codes(vla, small, env):
    """The argument checks of smolvla_capi.cpp:123-139 and the token range
    check of smolvla_model.cpp:197-206: the same status on both sides."""
    d, c = small
    ck = _ck()
    ob = oracle()
    r = _ref(ob, d, env)
    m = vla.SmolvlaModel(d)
    frames, ids, mask, state, noise = _inputs(ck, c, m)
    L = vla.lib()
    RL = ob._ref_models()
    out = np.zeros((m.chunk, m.action_dim), np.float32)
    P = lambda a: None if a is None else a.ctypes.data_as(__import__("ctypes").c_void_p)  # noqa: E731
    weights = np.ones(m.chunk, np.float32)
    prev = np.zeros((2, m.action_dim), np.float32)
    bad_ids = ids.copy()
    bad_ids[0] = 512  # the checkpoint's vocab is 512
    nan_w = weights.copy()
    nan_w[3] = np.nan
    cases = [
        ("wrong view count", dict(nv=1)),
        ("token out of range", dict(ids=bad_ids)),
        ("negative token", dict(ids=np.where(np.arange(ids.size) == 1, -1, ids).astype(np.int32))),
        ("zero height", dict(h=0)),
        ("negative n_lang", dict(n_lang=-1)),
        ("null frames", dict(frames=None)),
        ("null state", dict(state=None)),
        ("prev without weights", dict(prev=prev, n_prev=2, weights=None, mg=1.0)),
        ("prev with max_guidance 0", dict(prev=prev, n_prev=2, weights=weights, mg=0.0)),
        ("prev with a NaN weight", dict(prev=prev, n_prev=2, weights=nan_w, mg=1.0)),
        ("n_prev beyond the chunk", dict(prev=np.zeros((m.chunk + 1, m.action_dim), np.float32),
                                         n_prev=m.chunk + 1, weights=weights, mg=1.0)),
    ]
    for name, kw in cases:
        a = dict(frames=frames, nv=2, h=frames.shape[1], w=frames.shape[2], ids=ids, mask=mask, n_lang=ids.size,
                 state=state, prev=None, n_prev=0, weights=None, mg=0.0)
        a.update(kw)
        args = (P(a["frames"]), a["nv"], a["h"], a["w"], P(a["ids"]), P(a["mask"]), a["n_lang"], P(a["state"]),
                P(noise), 0, P(out), P(a["prev"]), a["n_prev"], P(a["weights"]), a["mg"])
        ours = L.vla_smolvla_predict_rtc(m.h, *args)
        theirs = RL.vla_smolvla_predict_rtc(r.h, *args)
        print(f"{name}: ours {ours}, reference {theirs}", flush=True)
        assert ours == theirs and ours != 0, name


def test_smolvla_model_full_size(vla, env, tmp_path):
    """BASELINE's SmolVLA shape end to end: two 480 x 640 cameras resized to
    512 x 512 for the 12-layer SigLIP tower (64 tokens each), a 48-token
    instruction, the state token (177 prefix tokens), 16 text layers, the
    16-layer expert over 10 Euler steps; SMOLVLA_INT8=48 against the
    reference with the same groups."""
    ck = _ck()
    ob = oracle()
    c = ck.SMOLVLA_MODEL_BASE
    d = ck.write_smolvla_model(str(tmp_path / "smol_full"), c)
    shim = _ref(ob, d, env, 48)
    env(48)
    m = vla.SmolvlaModel(d)
    frames, state, noise = ck.smolvla_model_inputs(c)
    ids, lmask, n = m.tokenize("pick up the red block and put it in the box, then " * 6)
    assert n == 48 and m.img_size == 512
    st, ref = shim.predict(frames, ids, lmask, state, m.chunk, m.action_dim, noise=noise)
    assert st == 0
    spread = max(_rel(shim.predict(frames, ids, lmask, state, m.chunk, m.action_dim, noise=noise, perturb=k)[1],
                      ref) for k in (1, 2))
    bar = max(2.0 * spread, 1e-3)
    got = m.predict(frames, ids, lmask, state, noise=noise)
    err = _rel(got, ref)
    print(f"smolvla model full size: rel err {err:.3e} (bar {bar:.3e}), graph nodes {m.graph_nodes}", flush=True)
    assert err <= bar
