"""ACT end to end through the reference's own entry points (vla_act_load /
vla_act_predict, include/vla_simd.h:66-81): uint8 frames -> per-camera
normalization -> ResNet-18 -> ACT transformer -> un-normalized actions, on the
device, against the reference's ActModel (src/models/act/act_model.cpp,
resnet_backbone.cpp) built into oracle/_ref from its own sources.

Bars:
  * backbone, fp32 convs: the device convs are im2col + an fp32 matrix-core
    GEMM, the reference's are its packed-panel GEMM; they differ by summation
    order only: features within 1e-4 of their scale.
  * backbone, every conv int8 (ACT_INT8 bit 32): normalization, conv2d_i8,
    max pool and the residual adds are each exact, so the features are the
    reference's bit for bit.
  * actions: fp32 transformer (ACT_INT8 0) within 1e-3 of the output scale;
    int8 transformer within twice the reference transformer's own spread under
    1-ulp perturbations of its input features (the class of difference the
    fp32 backbone leaves), as in test_gpu_graphs.py.
ACT_INT8 / ACT_I8_CONV_FROM / ACT_I8_CONV_TO are read at load by both sides,
as the reference reads them.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from helpers import load_pkg

pytestmark = pytest.mark.gpu

ENV = ("ACT_INT8", "ACT_I8_CONV_FROM", "ACT_I8_CONV_TO")


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


def _small(ck):
    return dict(ck.ACT_MODEL_BASE, img_h=96, img_w=128, n_cams=2, width=16, dim=128, heads=4, head_dim=32,
                ff=256, n_enc=2)


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
    return ck.write_act_model(str(tmp_path_factory.mktemp("actm") / "small"), _small(ck))


def _rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got))
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _ulp(x, k):
    r = np.random.default_rng(500 + k)
    s = r.integers(0, 3, size=x.shape) - 1
    y = np.array(x, np.float32, copy=True)
    y[s > 0] = np.nextafter(y[s > 0], np.float32(np.inf))
    y[s < 0] = np.nextafter(y[s < 0], np.float32(-np.inf))
    return y


def _norm_state(d, state, sd, ad, eps):
    st = np.fromfile(os.path.join(d, "stats.bin"), np.float32)
    return ((np.float32(state) - st[:sd]) / (st[sd:2 * sd] + np.float32(eps))).astype(np.float32)


def _spread(ob, d, ref_model, mask, images, state, eps):
    """The reference transformer's own output change under two 1-ulp
    perturbations of the reference backbone's features (unnormalized actions)."""
    feats = ref_model.encode(images)
    sn = _norm_state(d, state, ref_model.state_dim, ref_model.action_dim, eps)
    tf = ob.RefAct(d, ref_model.feat_ch, mask, ref_model.chunk, ref_model.action_dim)
    base = tf.forward(feats, ref_model.n_cams, ref_model.feat_h, ref_model.feat_w, sn)
    return max(_rel(tf.forward(_ulp(feats, k), ref_model.n_cams, ref_model.feat_h, ref_model.feat_w, sn), base)
               for k in range(2))


def test_server_binding_and_dims(vla, small_dir, env):
    """The library binds the way vla_simd/policy_server.py:203-235 binds a
    model library: ctypes symbols vla_act_load/free/<ints>/predict with the
    server's argtypes; dims agree with the reference; null buffers give
    VLA_ERR_ARG."""
    from helpers import oracle
    ob = oracle()
    env(ACT_INT8=31)
    lib = ctypes.CDLL(vla.LIB_PATH)
    lib.vla_act_load.argtypes, lib.vla_act_load.restype = [ctypes.c_char_p], ctypes.c_void_p
    lib.vla_act_free.argtypes, lib.vla_act_free.restype = [ctypes.c_void_p], None
    ints = ("chunk", "action_dim", "state_dim", "n_cams", "img_h", "img_w")
    for i in ints:
        f = getattr(lib, f"vla_act_{i}")
        f.argtypes, f.restype = [ctypes.c_void_p], ctypes.c_int32
    f32p = ctypes.POINTER(ctypes.c_float)
    lib.vla_act_predict.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint8), f32p, ctypes.c_int32, f32p]
    lib.vla_act_predict.restype = ctypes.c_int32
    h = lib.vla_act_load(small_dir.encode())
    assert h
    try:
        got = {i: getattr(lib, f"vla_act_{i}")(h) for i in ints}
        r = ob.RefActModel(small_dir)
        assert got == dict(chunk=r.chunk, action_dim=r.action_dim, state_dim=r.state_dim, n_cams=r.n_cams,
                           img_h=r.img_h, img_w=r.img_w)
        ck = _ck()
        images, state = ck.act_model_inputs(_small(ck))
        out = np.empty((got["chunk"], got["action_dim"]), np.float32)
        rc = lib.vla_act_predict(h, images.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                                 state.ctypes.data_as(f32p), 1, out.ctypes.data_as(f32p))
        assert rc == 0 and np.all(np.isfinite(out))
        assert lib.vla_act_predict(h, None, state.ctypes.data_as(f32p), 1, out.ctypes.data_as(f32p)) == -1
        assert lib.vla_act_chunk(None) == 0
    finally:
        lib.vla_act_free(h)
    env(ACT_INT8=31)
    assert lib.vla_act_load(b"/nonexistent/act") is None


@pytest.mark.parametrize("mask", [0, 31])
def test_fp32_backbone_and_actions(vla, small_dir, env, mask):
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = _small(ck)
    env(ACT_INT8=mask)
    images, state = ck.act_model_inputs(c)
    r = ob.RefActModel(small_dir)
    m = vla.ActModel(small_dir)
    assert m.int8_convs == 0 and (m.int8_layers > 0) == (mask != 0)
    assert (m.feat_h, m.feat_w, m.feat_ch) == (r.feat_h, r.feat_w, r.feat_ch) == (3, 4, 128)
    f_err = _rel(m.encode(images), r.encode(images))
    print(f"act model mask {mask}: feature rel err {f_err:.3e}", flush=True)
    assert f_err <= 1e-4
    ref = r.predict(images, state, unnormalize=False)
    got = m.predict(images, state, unnormalize=False)
    bar = 1e-3 if mask == 0 else max(2.0 * _spread(ob, small_dir, r, mask, images, state, c["norm_eps"]), 1e-3)
    err = _rel(got, ref)
    print(f"act model mask {mask}: action rel err {err:.3e} (bar {bar:.3e})", flush=True)
    assert err <= bar
    # un-normalization: v * std + mean per action dimension (act_model.cpp:152-157)
    st = np.fromfile(os.path.join(small_dir, "stats.bin"), np.float32)
    sd, ad = m.state_dim, m.action_dim
    un = m.predict(images, state, unnormalize=True)
    want = got.astype(np.float64) * st[2 * sd + ad:2 * sd + 2 * ad] + st[2 * sd:2 * sd + ad]
    assert _rel(un, want) <= 1e-6
    assert _rel(un, r.predict(images, state, unnormalize=True)) <= bar
    # graph replays reproduce the eager pass
    for _ in range(2):
        assert m.predict(images, state, unnormalize=False).tobytes() == got.tobytes()


@pytest.mark.parametrize("frm,to", [(0, -1), (0, 3), (2, -1)])
def test_int8_backbone(vla, small_dir, env, frm, to):
    """ACT_INT8 bit 32: every conv (0, -1) is conv2d_i8 and the features are
    the reference's bit for bit; with ACT_I8_CONV_TO=3 the stem and the first
    two blocks are int8 (exact) and the rest fp32 (summation order); with
    ACT_I8_CONV_FROM=2 the stem and the first block are fp32 and the int8
    convs after them take the block maxima their producers (max pool, residual
    add, relu) wrote, as the all-int8 trunk does."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    env(ACT_INT8=32 | 31, ACT_I8_CONV_FROM=frm, ACT_I8_CONV_TO=to)
    images, state = ck.act_model_inputs(_small(ck))
    r = ob.RefActModel(small_dir)
    m = vla.ActModel(small_dir)
    assert m.int8_convs == {(0, -1): 20, (0, 3): 1 + 2 * 2, (2, -1): 17}[(frm, to)]
    got, ref = m.encode(images), r.encode(images)
    if (frm, to) == (0, -1):
        assert got.tobytes() == ref.tobytes(), f"int8 backbone differs (rel {_rel(got, ref):.3e})"
    else:
        assert _rel(got, ref) <= 1e-4
    a = m.predict(images, state)
    assert np.all(np.isfinite(a))


def test_int8_backbone_fused_epilogues_full_size(vla, env, tmp_path, torch_cuda):
    """ResNet-18 at 480 x 640, every conv int8 (ACT_INT8=63): each block's
    ReLU after conv1 and residual add + ReLU after conv2 run in the conv's
    epilogue - the 32 x 64 LDS GEMM tile gathering from the int8 map (19200,
    4800 and 1200 pixels), the skinny kernel doing the same (300 pixels) -
    which also writes the block maxima the next conv folds into its scale;
    the first conv after a downsample reuses its int8 map, and the max pool
    writes the first conv's map from the stem's ReLU maxima. The features are
    the reference's bit for bit, and the same bits with VLA_HIP_CONV_FUSE=0,
    VLA_HIP_CONV_SHARE=0 and VLA_HIP_CONV_POOL_FUSE=0 (separate passes), on
    the eager, the captured and a replayed call of vla_act_encode_dev (the
    graph reading the frames and writing the features in place) and of the
    host form."""
    torch = torch_cuda
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = ck.ACT_MODEL_BASE
    d = ck.write_act_model(str(tmp_path / "act_full"), c)
    env(ACT_INT8=63)
    images, state = ck.act_model_inputs(c)
    ref = ob.RefActModel(d).encode(images)
    ti, ts = torch.from_numpy(images).cuda(), torch.from_numpy(state).cuda()

    def run(m):
        assert m.int8_convs == 20
        tf = torch.empty((m.n_cams * m.feat_h * m.feat_w, m.feat_ch), dtype=torch.float32, device="cuda")
        ta = torch.empty((m.chunk, m.action_dim), dtype=torch.float32, device="cuda")
        feats = []
        for _ in range(3):
            m.encode_dev(ti, tf)
            torch.cuda.synchronize()
            feats.append(tf.cpu().numpy())
            m.predict_dev(ti, ts, ta)
        torch.cuda.synchronize()
        return feats + [m.encode(images)], m.graph_nodes

    knobs = ("VLA_HIP_CONV_FUSE", "VLA_HIP_CONV_SHARE", "VLA_HIP_CONV_POOL_FUSE")
    for k in knobs:
        os.environ[k] = "0"
    try:
        passes, n0 = run(vla.ActModel(d))
    finally:
        for k in knobs:
            del os.environ[k]
    fused, n1 = run(vla.ActModel(d))
    print(f"int8 trunk 480x640: graph nodes {n0} with passes, {n1} fused", flush=True)
    for i, f in enumerate(passes + fused):
        assert f.tobytes() == ref.tobytes(), f"call {i}: features differ (rel {_rel(f, ref):.3e})"
    assert n1 < n0


def test_act_model_full_size(vla, env, tmp_path):
    """BASELINE's ACT shape end to end: one 480 x 640 camera through ResNet-18
    (15 x 20 x 512 features) into the 4-layer d=512 transformer, ACT_INT8=31."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = ck.ACT_MODEL_BASE
    d = ck.write_act_model(str(tmp_path / "act_full"), c)
    env(ACT_INT8=31)
    images, state = ck.act_model_inputs(c)
    r = ob.RefActModel(d)
    m = vla.ActModel(d)
    assert (m.feat_h, m.feat_w, m.feat_ch) == (15, 20, 512)
    ref = r.predict(images, state, unnormalize=False)
    got = m.predict(images, state, unnormalize=False)
    bar = max(2.0 * _spread(ob, d, r, 31, images, state, c["norm_eps"]), 1e-3)
    err = _rel(got, ref)
    print(f"act model 480x640: action rel err {err:.3e} (bar {bar:.3e}), graph nodes {m.graph_nodes}", flush=True)
    assert err <= bar


def test_implicit_conv_gemm_bit_exact(vla, env, tmp_path):
    """The fp32 convolutions as implicit GEMMs (each patch gathered by the
    GEMM's own A loads from the NHWC map) give the im2col + GEMM features and
    actions bit for bit: the same products in the same order. BASELINE's
    480 x 640 ResNet-18, whose layers with Cin % 32 == 0 and a tiled GEMM take
    the implicit form; VLA_CONV_F32_IMPLICIT=0 keeps im2col."""
    ck = _ck()
    c = ck.ACT_MODEL_BASE
    d = ck.write_act_model(str(tmp_path / "act_full"), c)
    env(ACT_INT8=31)
    images, state = ck.act_model_inputs(c)
    os.environ["VLA_CONV_F32_IMPLICIT"] = "0"
    try:
        m0 = vla.ActModel(d)
        f0, a0 = m0.encode(images), m0.predict(images, state)
    finally:
        del os.environ["VLA_CONV_F32_IMPLICIT"]
    m1 = vla.ActModel(d)
    f1, a1 = m1.encode(images), m1.predict(images, state)
    assert f1.tobytes() == f0.tobytes(), f"features differ (rel {_rel(f1, f0):.3e})"
    assert a1.tobytes() == a0.tobytes()
