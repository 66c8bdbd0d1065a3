"""Diffusion Policy end to end through the reference's own entry points
(vla_diffusion_load / _predict and the getters, include/vla_simd.h:245-280):
an observation history of uint8 frames and raw states plus the sampler's noise
-> actions on the device, against the reference's DiffusionModel
(src/models/diffusion/*.cpp) built into oracle/_ref from its own sources, on
synthetic checkpoints in the reference's file layout
(checkpoints.write_diffusion_model).

Bars (relative to the output scale):
  * fp32 (DIFFUSION_INT8 0): the convolutions, GroupNorms and linears differ
    from the reference's only by summation order, carried through every
    sampler step: 1e-3, as ACT's fp32 bar;
  * int8 (bit 1 the UNet's GEMM layers, bit 2 the encoders' convs): every int8
    GEMM is bit-exact on its own inputs (test_gpu_int8_steps.py), but those
    inputs carry the fp32 differences, so a quantized byte may flip and the
    sampler carries the flip on. The bar is the reference's own spread: on
    the small checkpoint, one state value moved by 1 ulp moves the
    reference's actions by up to 6.9e-2 with the UNet int8 (DDIM 10) and
    2.4e-2 with every group int8 (DDPM 10), against 5.5e-6 with only the
    encoders' convs int8 (measured on its CPU build). So 1e-1 where the UNet
    is int8, 1e-2 for the encoders alone;
  * the sampler's arithmetic (the DDPM / DDIM update in double, the MIN_MAX
    maps) is checked exactly where it is the only computation: un-normalized
    actions equal (a + 1) / 2 * (max - min) + min of the normalized ones.
DIFFUSION_INT8, DP_STEPS and DP_SCHEDULER are read at load by both sides.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from helpers import load_pkg

pytestmark = pytest.mark.gpu

ENV = ("DIFFUSION_INT8", "DP_STEPS", "DP_SCHEDULER")


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


def _small(ck, **kw):
    c = dict(ck.DP_MODEL_BASE, down_dims=(64, 128, 256), step_embed_dim=32, num_keypoints=8, width=16,
             num_inference_steps=10, num_train_timesteps=100)
    c.update(kw)
    return c


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
    return ck.write_diffusion_model(str(tmp_path_factory.mktemp("dp") / "small"), _small(ck))


def _rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got))
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _queries(ck, c):
    """Two consecutive queries of a rollout: the second's oldest frames and
    state are the first's newest (the frame cache's case), new noise."""
    f0, s0, z0 = ck.diffusion_model_inputs(c, tag="q0")
    f1, s1, z1 = ck.diffusion_model_inputs(c, tag="q1")
    f1 = f1.copy()
    s1 = s1.copy()
    f1[:-1] = f0[1:]
    s1[:-1] = s0[1:]
    return [(f0, s0, z0), (f1, s1, z1)]


def test_server_binding_dims_and_errors(vla, small_dir, env):
    """The library binds the way vla_simd/policy_server.py:544-587 binds
    Diffusion Policy: ctypes symbols vla_diffusion_<getters> and _predict with
    the server's argtypes; dims agree with the reference; null handles and
    buffers and a bad directory fail as diffusion_capi.cpp's do."""
    from helpers import oracle
    ob = oracle()
    env()
    lib = ctypes.CDLL(vla.LIB_PATH)
    vp, f32p, u8p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint8)
    lib.vla_diffusion_load.argtypes, lib.vla_diffusion_load.restype = [ctypes.c_char_p], vp
    lib.vla_diffusion_free.argtypes, lib.vla_diffusion_free.restype = [vp], None
    dims = ("chunk", "horizon", "action_dim", "state_dim", "n_cams", "n_obs_steps", "img_h", "img_w", "num_steps",
            "is_ddim")
    for k in dims:
        f = getattr(lib, f"vla_diffusion_{k}")
        f.argtypes, f.restype = [vp], ctypes.c_int32
    lib.vla_diffusion_predict.argtypes = [vp, u8p, f32p, ctypes.c_int32, f32p, f32p]
    lib.vla_diffusion_predict.restype = ctypes.c_int32
    h = lib.vla_diffusion_load(small_dir.encode())
    assert h
    try:
        got = {k: getattr(lib, f"vla_diffusion_{k}")(h) for k in dims}
        r = ob.RefDiffusionModel(small_dir)
        assert got == {k: getattr(r, k) for k in dims}
        ck = _ck()
        frames, state, noise = ck.diffusion_model_inputs(_small(ck))
        out = np.empty((got["chunk"], got["action_dim"]), np.float32)
        rc = lib.vla_diffusion_predict(h, frames.ctypes.data_as(u8p), state.ctypes.data_as(f32p), 1,
                                       out.ctypes.data_as(f32p), noise.ctypes.data_as(f32p))
        assert rc == 0 and np.all(np.isfinite(out))
        assert lib.vla_diffusion_predict(h, None, state.ctypes.data_as(f32p), 1, out.ctypes.data_as(f32p),
                                         None) == -1
        assert lib.vla_diffusion_predict(h, frames.ctypes.data_as(u8p), None, 1, out.ctypes.data_as(f32p),
                                         None) == -1
        assert lib.vla_diffusion_predict(None, frames.ctypes.data_as(u8p), state.ctypes.data_as(f32p), 1,
                                         out.ctypes.data_as(f32p), None) == -1
        for k in dims:  # DP_GET: VLA_ERR_ARG for a null handle
            assert getattr(lib, f"vla_diffusion_{k}")(None) == -1
    finally:
        lib.vla_diffusion_free(h)
    assert lib.vla_diffusion_load(b"/nonexistent/diffusion") is None


CASES = [
    # (id, DIFFUSION_INT8, scheduler, steps, meta overrides, bar)
    ("ddpm10_fp32", 0, "DDPM", 10, {}, 1e-3),
    ("ddim10_fp32", 0, "DDIM", 10, {}, 1e-3),
    ("ddim10_noclip_fp32", 0, "DDIM", 10, {"clip_sample": 0}, 1e-3),
    ("ddpm10_shared_noscale_fp32", 0, "DDPM", 10, {"separate_encoders": 0, "film_scale": 0, "kernel_size": 3}, 1e-3),
    ("ddim10_unet_int8", 1, "DDIM", 10, {}, 1e-1),
    ("ddim10_conv_int8", 2, "DDIM", 10, {}, 1e-2),
    ("ddpm10_all_int8", 3, "DDPM", 10, {}, 1e-1),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_actions_match_reference(vla, env, tmp_path, case):
    """Two consecutive queries of a rollout against the reference's
    DiffusionModel, normalized and un-normalized, and the zero-noise query."""
    name, mask, sched, steps, over, bar = case
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = _small(ck, **over)
    d = ck.write_diffusion_model(str(tmp_path / name), c)
    env(DIFFUSION_INT8=mask, DP_SCHEDULER=sched, DP_STEPS=steps)
    r = ob.RefDiffusionModel(d)
    m = vla.DiffusionModel(d)
    assert m.num_steps == r.num_steps == steps and m.is_ddim == bool(r.is_ddim) == (sched == "DDIM")
    assert (m.int8_layers > 0) == bool(mask & 1) and (m.int8_convs > 0) == bool(mask & 2)
    for qi, (frames, state, noise) in enumerate(_queries(ck, c)):
        st, ref = r.predict(frames, state, noise, unnormalize=False)
        assert st == 0
        got = m.predict(frames, state, noise, unnormalize=False)
        err = _rel(got, ref)
        print(f"diffusion {name} query {qi}: action rel err {err:.3e} (bar {bar:.0e})", flush=True)
        assert err <= bar
    # the same query again replays the captured graphs and hits the frame cache
    again = m.predict(frames, state, noise, unnormalize=False)
    assert again.tobytes() == got.tobytes()
    # un-normalization: (a + 1) / 2 * (max - min) + min per action dim
    stats = np.fromfile(os.path.join(d, "stats.bin"), np.float32)
    sd, ad = c["state_dim"], c["action_dim"]
    amin, amax = stats[2 * sd:2 * sd + ad], stats[2 * sd + ad:2 * sd + 2 * ad]
    un = m.predict(frames, state, noise, unnormalize=True)
    want = (got + np.float32(1)) / np.float32(2) * (amax - amin) + amin
    assert _rel(un, want) <= 1e-6
    # no noise: the sampler starts from zeros and DDPM adds none (diffusion_model.cpp:249-262)
    st, ref = r.predict(frames, state, None, unnormalize=False)
    got = m.predict(frames, state, None, unnormalize=False)
    err = _rel(got, ref)
    print(f"diffusion {name} zero noise: action rel err {err:.3e}", flush=True)
    assert st == 0 and err <= bar


def test_frame_cache_keeps_results(vla, small_dir, env):
    """Features cached across queries (a frame equal to one a slot of the
    same camera holds) give the same actions as a fresh model that encodes
    every frame."""
    ck = _ck()
    env(DP_SCHEDULER="DDIM", DP_STEPS=5)
    c = _small(ck)
    q = [(f, st, z[:6]) for f, st, z in _queries(ck, c)]  # the prior + 5 steps
    m = vla.DiffusionModel(small_dir)
    m.predict(*q[0], unnormalize=False)
    cached = m.predict(*q[1], unnormalize=False)
    fresh = vla.DiffusionModel(small_dir).predict(*q[1], unnormalize=False)
    assert cached.tobytes() == fresh.tobytes()


def test_bad_checkpoints_fail_like_the_reference(vla, small_dir, env, tmp_path):
    """Loader checks the reference makes: an unknown scheduler, a UNet file of
    the wrong size, identity action statistics, more inference than training
    steps."""
    import shutil
    from helpers import oracle
    ob = oracle()
    env()

    def variant(name, edit):
        d = str(tmp_path / name)
        shutil.copytree(small_dir, d)
        edit(d)
        return d

    def meta_set(d, key, val):
        p = os.path.join(d, "diffusion.meta")
        lines = [l for l in open(p) if l.split()[:1] != [key]]
        open(p, "w").writelines(lines + [f"{key} {val}\n"])

    bad = [
        variant("sched", lambda d: meta_set(d, "scheduler", "PNDM")),
        variant("unet", lambda d: open(os.path.join(d, "unet.bin"), "ab").write(b"\0\0\0\0")),
        variant("steps", lambda d: meta_set(d, "num_inference_steps", 101)),
    ]

    def flat_stats(d):
        p = os.path.join(d, "stats.bin")
        s = np.fromfile(p, np.float32)
        c = _small(_ck())
        sd, ad = c["state_dim"], c["action_dim"]
        s[2 * sd + ad:2 * sd + 2 * ad] = s[2 * sd:2 * sd + ad]
        s.tofile(p)
    bad.append(variant("stats", flat_stats))
    for d in bad:
        with pytest.raises(RuntimeError):
            ob.RefDiffusionModel(d)
        with pytest.raises(vla.VlaError):
            vla.DiffusionModel(d)
    env(DP_SCHEDULER="EULER")
    with pytest.raises(RuntimeError):
        ob.RefDiffusionModel(small_dir)
    with pytest.raises(vla.VlaError):
        vla.DiffusionModel(small_dir)


def test_full_size_ddim10(vla, env, tmp_path):
    """lerobot's stock pusht-shaped policy (two 96 x 96 cameras cropped to
    84 x 84, 512/1024/2048 UNet, horizon 16) at DDIM 10, fp32 and with every
    int8 group, against the reference."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = ck.DP_MODEL_BASE
    d = ck.write_diffusion_model(str(tmp_path / "full"), c)
    frames, state, _ = ck.diffusion_model_inputs(c)
    noise = ck.diffusion_model_inputs(dict(c, num_inference_steps=10))[2]
    for mask, bar in ((0, 1e-3), (3, 1e-1)):
        env(DIFFUSION_INT8=mask, DP_SCHEDULER="DDIM", DP_STEPS=10)
        st, ref = ob.RefDiffusionModel(d).predict(frames, state, noise, unnormalize=False)
        m = vla.DiffusionModel(d)
        got = m.predict(frames, state, noise, unnormalize=False)
        err = _rel(got, ref)
        print(f"diffusion full DDIM10 mask {mask}: action rel err {err:.3e} (bar {bar:.0e}), "
              f"{m.int8_layers} int8 GEMMs, {m.int8_convs} int8 convs, {m.graph_nodes} graph nodes", flush=True)
        assert st == 0 and err <= bar


def test_loads_from_gguf(vla, small_dir, env, tmp_path):
    """The same checkpoint packed into one vla.simd GGUF: our actions from the
    GGUF are byte-identical to the directory's, and the reference loads the
    GGUF too (io::Mount)."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    env(DP_SCHEDULER="DDIM", DP_STEPS=5)
    g = ck.write_gguf(small_dir, str(tmp_path / "diffusion.gguf"), "diffusion")
    frames, state, noise = ck.diffusion_model_inputs(_small(ck))
    noise = noise[:6]
    a = vla.DiffusionModel(small_dir).predict(frames, state, noise)
    b = vla.DiffusionModel(g).predict(frames, state, noise)
    assert a.tobytes() == b.tobytes()
    st, ref = ob.RefDiffusionModel(g).predict(frames, state, noise)
    assert st == 0 and _rel(b, ref) <= 1e-3
