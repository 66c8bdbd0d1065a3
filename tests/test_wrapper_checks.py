"""CPU checks of the Python model wrappers' input validation: the C ABI reads
host buffers whose sizes it cannot see, so each wrapper checks them against the
loaded model's shapes and raises ValueError before any library call. The
wrappers are built without a loaded model here (no device); h = None, so a
check that let a bad call through would fail on the null handle instead."""

import numpy as np
import pytest

from helpers import load_pkg


def _bare(cls, **attrs):
    obj = object.__new__(cls)
    obj.h = None
    for k, v in attrs.items():
        setattr(obj, k, v)
    return obj


def test_act_transformer_checks_feats_and_state():
    vla = load_pkg()
    m = _bare(vla.ActTransformer, chunk=100, action_dim=14, state_dim=14, img_ch=512)
    feats = np.zeros((300, 512), np.float32)
    with pytest.raises(ValueError, match="feats"):
        m.forward(feats[:-1], 1, 15, 20, np.zeros(14, np.float32))
    with pytest.raises(ValueError, match="state"):
        m.forward(feats, 1, 15, 20, np.zeros(13, np.float32))
    with pytest.raises(ValueError, match="n_cams"):
        m.forward(feats, 0, 15, 20, np.zeros(14, np.float32))


def test_octo_transformer_checks_window_and_stems():
    vla = load_pkg()
    m = _bare(vla.OctoTransformer, d=768, n_task=16, t5_dim=768, stem_dim=512, tok_primary=256,
              tok_wrist=64, max_horizon=10)
    t5 = np.zeros((16, 768), np.float32)
    sp = np.zeros((2, 256, 512), np.float32)
    sw = np.zeros((2, 64, 512), np.float32)
    with pytest.raises(ValueError, match="timestep_mask"):
        m.forward(t5, sp, sw, 2, np.ones(1, np.uint8))
    with pytest.raises(ValueError, match="wnd"):
        m.forward(t5, sp, sw, 11, np.ones(11, np.uint8))
    with pytest.raises(ValueError, match="t5"):
        m.forward(t5[:15], sp, sw, 2, np.ones(2, np.uint8))
    with pytest.raises(ValueError, match="stem_p"):
        m.forward(t5, sp[:1], sw, 2, np.ones(2, np.uint8))
    with pytest.raises(ValueError, match="stem_w"):
        m.forward(t5, sp, sw[:, :63], 2, np.ones(2, np.uint8))


def test_smolvla_chunk_checks_pad_and_noise():
    vla = load_pkg()
    m = _bare(vla.SmolvlaChunk, chunk=50, max_action_dim=32, hidden=960)
    prefix = np.zeros((177, 960), np.float32)
    pad = np.ones(177, np.int32)
    noise = np.zeros((50, 32), np.float32)
    with pytest.raises(ValueError, match="pad"):
        m.run(prefix, pad[:-1], noise)
    with pytest.raises(ValueError, match="noise"):
        m.run(prefix, pad, noise[:49])
    with pytest.raises(ValueError, match="prefix"):
        m.run(prefix[:, :959], pad, noise)
