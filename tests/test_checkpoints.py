"""Synthetic checkpoints (vla_simd_amd.checkpoints) against the reference's
own loaders, on the CPU: the files the device graphs read must be exactly the
layout ActTransformer::load, OctoTransformer::load, SmollmVlm::load and
ActionExpert::load accept (each checks the .bin size against its .meta), and
the reference graphs must run on them deterministically. Small configurations
keep this in seconds; the GPU tests use the BASELINE sizes."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import load_pkg, oracle


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


@pytest.fixture(scope="module")
def ob():
    o = oracle()
    if not o.ref_available():
        pytest.skip("oracle/_ref/libvla_ref.so not built")
    return o


ACT_SMALL = dict(dim=64, heads=4, head_dim=16, ff=128, n_enc=2, n_dec=1, chunk=10, state_dim=6,
                 action_dim=6, n_1d=2, n_text=0, ln_eps=1e-5, img_ch=32, n_cams=1, fh=3, fw=4)
OCTO_SMALL = dict(d=64, n_layers=2, heads=4, head_dim=16, mlp=128, max_horizon=3, n_task=4,
                  tok_primary=8, tok_wrist=4, n_readout=1, t5_dim=32, stem_dim=32, ln_eps=1e-6,
                  gelu_erf=0, repeat_task=1, wnd=2)
SMOL_SMALL = dict(hidden=128, n_q=2, n_kv=1, head_dim=64, ffn=256, eps=1e-5, rope_base=10000.0,
                  n_layers=3, expert_h=96, expert_ffn=192, expert_layers=3, self_attn_every_n=2,
                  chunk=8, num_steps=3, max_action_dim=16, min_period=4e-3, max_period=4.0,
                  n_prefix=12)


@pytest.mark.parametrize("mask", [0, 31])
def test_act_checkpoint_loads_in_reference(ob, tmp_path, mask):
    ck = _ck()
    c = ACT_SMALL
    ck.write_act(str(tmp_path), c)
    r = ob.RefAct(str(tmp_path), c["img_ch"], mask, c["chunk"], c["action_dim"])
    f, s = ck.act_inputs(c)
    a = r.forward(f, 1, c["fh"], c["fw"], s)
    b = r.forward(f, 1, c["fh"], c["fw"], s)
    assert a.shape == (c["chunk"], c["action_dim"]) and np.all(np.isfinite(a))
    assert a.tobytes() == b.tobytes()


def test_act_checkpoint_truncated_is_refused(ob, tmp_path):
    ck = _ck()
    ck.write_act(str(tmp_path), ACT_SMALL)
    p = tmp_path / "act.bin"
    p.write_bytes(p.read_bytes()[:-4])
    with pytest.raises(RuntimeError):
        ob.RefAct(str(tmp_path), ACT_SMALL["img_ch"], 0, ACT_SMALL["chunk"], ACT_SMALL["action_dim"])


@pytest.mark.parametrize("mask", [0, 15])
def test_octo_checkpoint_loads_in_reference(ob, tmp_path, mask):
    ck = _ck()
    c = OCTO_SMALL
    ck.write_octo(str(tmp_path), c)
    r = ob.RefOcto(str(tmp_path), mask, c["d"])
    t5, sp, sw, tm = ck.octo_inputs(c)
    a = r.forward(t5, sp, sw, 2, tm)
    assert a.shape == (c["d"],) and np.all(np.isfinite(a)) and np.any(a != 0)
    assert a.tobytes() == r.forward(t5, sp, sw, 2, tm).tobytes()


@pytest.mark.parametrize("mask", [0, 48])
def test_smolvla_checkpoint_loads_in_reference(ob, tmp_path, mask):
    ck = _ck()
    c = SMOL_SMALL
    ck.write_smolvla(str(tmp_path), c)
    r = ob.RefSmolvla(str(tmp_path), mask)
    assert (r.chunk, r.mad) == (c["chunk"], c["max_action_dim"])
    p, pad, n = ck.smolvla_inputs(c, n_pad=2)
    a = r.run(p, pad, n)
    assert np.all(np.isfinite(a)) and a.tobytes() == r.run(p, pad, n).tobytes()


def test_bf16_rounding_is_nearest_even():
    ck = _ck()
    x = np.array([1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -2.5, 1.0 + 2.0 ** -9, 1.0 + 2.0 ** -7 + 2.0 ** -12],
                 np.float32)
    got = (ck._bf16(x).astype(np.uint32) << 16).view(np.float32)
    # halfway cases go to the even mantissa (1 + 2^-8 -> 1, 1 + 3 * 2^-8 -> 1 + 2^-6),
    # anything above halfway rounds up
    assert got.tolist() == [1.0, 1.0, 1.0 + 2.0 ** -6, -2.5, 1.0, 1.0 + 2.0 ** -7]
