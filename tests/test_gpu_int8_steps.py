"""Every int8 step inside the device policy graphs, checked on its own.

The graph parity tests (test_gpu_graphs.py) compare whole passes against the
reference. At the int8 masks their bar is the reference's own spread under
1-ulp input perturbations (a few percent of the output scale), because fp32
differences of a few ulp move values across int8 rounding boundaries. A mistake
confined to the int8 steps (a scale from the wrong quantization slot, a slot
read after a later layer overwrote it, the wrong weight rows) could hide under
that bar. So here one pass of each graph runs with the int8-step probe on
(vla_probe_*): each int8 GEMM of the pass is recorded with the fp32 rows its
activations were quantized from, the int8 activations and scales it actually
read, its weights, and its output before and after. Each step must then be
bit-exact against the oracle on the recorded inputs (oracle/oracle.c, pinned
to the reference build in tests/test_oracle.py):
  * xq, ascale == orc_quantize_act_i8(fp32 rows)             (gemm_i8.cpp:209-244)
  * after == [before +] act(orc_dense_linear_i8_pre(xq, ...)) (gemm_i8.cpp:262-281)
bit for bit where the epilogue has no transcendental (no activation, ReLU);
GELU epilogues within 2e-6 of the output scale (the activation class of
test_ops.cpp:272-294). Weight rows must be those of the per-row absmax
quantizer (every non-zero row reaches +-127).
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from helpers import load_pkg, max_rel, same_bits

pytestmark = pytest.mark.gpu


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


@pytest.fixture(scope="module")
def ckdir(tmp_path_factory):
    return tmp_path_factory.mktemp("ck_steps")


def _check_steps(vla, orc, run, expect_min, max_records=512, what=""):
    recs = vla.probe_records(run, max_records)
    print(f"{what}: {len(recs)} int8 GEMM steps recorded", flush=True)
    assert len(recs) >= expect_min
    for i, r in enumerate(recs):
        M, K, N, act, acc = r["M"], r["K"], r["N"], r["act"], r["acc"]
        tag = f"{what} step {i} (M={M} K={K} N={N} act={act} acc={acc})"
        assert r["src"] is not None, f"{tag}: no fp32 source recorded for its quantization slot"
        Kp = (K + 3) & ~3
        xqo, sao = orc.quantize_act_i8(r["src"])
        assert same_bits(r["ascale"], sao), f"{tag}: activation scales differ from the oracle's"
        assert same_bits(r["xq"], np.ascontiguousarray(xqo[:, :K])), f"{tag}: int8 activations differ"
        W = r["W"]
        amax = np.abs(W.astype(np.int32)).max(axis=1)
        assert np.all((amax == 127) | (amax == 0)), f"{tag}: weight rows are not absmax-quantized"
        xq = np.zeros((M, Kp), np.int8)
        xq[:, :K] = r["xq"]
        Wp = np.zeros((N, Kp), np.int8)
        Wp[:, :K] = W
        v = orc.apply_act(orc.dense_linear_i8_pre(xq, r["ascale"], Wp, r["wscale"], r["bias"], K), act)
        want = (r["before"] + v).astype(np.float32) if acc else v
        if act in (0, 1):
            assert same_bits(r["after"], want), f"{tag}: output differs from the oracle's"
        else:
            assert max_rel(r["after"], want, float(np.max(np.abs(want)))) <= 2e-6, f"{tag}: GELU epilogue"
    return recs


def test_act_int8_steps(vla, orc, ckdir):
    ck = _ck()
    c = ck.ACT_BASE
    d = str(ckdir / "act")
    ck.write_act(d, c)
    feats, state = ck.act_inputs(c)
    m = vla.ActTransformer(d, c["img_ch"], 31)
    m.forward(feats, c["n_cams"], c["fh"], c["fw"], state)  # eager first call, then a graph
    m.forward(feats, c["n_cams"], c["fh"], c["fw"], state)
    recs = _check_steps(vla, orc, lambda: m.forward(feats, c["n_cams"], c["fh"], c["fw"], state),
                        expect_min=4 * 4 + 4 + 4, what="act mask 31")
    # the probe runs eagerly; the captured graph still reproduces the pass
    again = m.forward(feats, c["n_cams"], c["fh"], c["fw"], state)
    assert np.all(np.isfinite(again)) and len(recs) > 0


@pytest.mark.parametrize("repeat_task", [0, 1])
def test_octo_int8_steps(vla, orc, ckdir, repeat_task):
    ck = _ck()
    c = dict(ck.OCTO_BASE, repeat_task=repeat_task)
    d = str(ckdir / f"octo{repeat_task}")
    ck.write_octo(d, c)
    t5, sp, sw, tm = ck.octo_inputs(c)
    m = vla.OctoTransformer(d, 15)
    ref = m.forward(t5, sp, sw, 2, tm)
    _check_steps(vla, orc, lambda: m.forward(t5, sp, sw, 2, tm), expect_min=12 * 3 + 3,
                 what=f"octo mask 15 ({m.total_tokens(2)} tokens)")
    # a probed pass computes what the graph computes
    assert m.forward(t5, sp, sw, 2, tm).tobytes() == ref.tobytes()


@pytest.mark.parametrize("chunk,layers,n_prefix", [(50, 16, 177), (12, 4, 60)])
def test_smolvla_int8_steps(vla, orc, ckdir, chunk, layers, n_prefix):
    """The prefix tower and the first denoise steps (the probe keeps the first
    300 steps of the pass; later Euler steps repeat the same layer calls)."""
    ck = _ck()
    c = dict(ck.SMOLVLA_BASE, chunk=chunk, n_layers=layers, expert_layers=layers, n_prefix=n_prefix)
    d = str(ckdir / f"smol{chunk}")
    ck.write_smolvla(d, c)
    prefix, pad, noise = ck.smolvla_inputs(c, n_pad=3)
    m = vla.SmolvlaChunk(d, 48)
    ref = m.run(prefix, pad, noise)
    _check_steps(vla, orc, lambda: m.run(prefix, pad, noise), expect_min=layers * 3, max_records=300,
                 what=f"smolvla mask 48 chunk {chunk}")
    assert m.run(prefix, pad, noise).tobytes() == ref.tobytes()


DP_STEP_CASES = {
    "k5": dict(down_dims=(64, 128, 256), kernel_size=5),
    "k3": dict(down_dims=(64, 128, 256), kernel_size=3),
    # two levels, groups of 64 / 128 channels
    "g4": dict(down_dims=(256, 512), n_groups=4, kernel_size=5),
}


@pytest.mark.parametrize("case", list(DP_STEP_CASES))
def test_diffusion_int8_steps(vla, orc, ckdir, case):
    """Diffusion Policy's UNet at DIFFUSION_INT8=1: the 1-D convolutions read
    their taps as overlapping rows of the padded sequence (the quantizer
    included), the strided downsample reads every second row, the 1x1 convs
    feed the block's second norm. Two sampler steps, DDIM. The probed pass
    runs eagerly and without row-op fusion; the captured graph's actions must
    be bit-identical to it."""
    ck = _ck()
    c = dict(ck.DP_MODEL_BASE, step_embed_dim=32, num_keypoints=8, width=16, **DP_STEP_CASES[case])
    d = str(ckdir / f"dp_{case}")
    ck.write_diffusion_model(d, c)
    frames, state, noise = ck.diffusion_model_inputs(dict(c, num_inference_steps=2))
    saved = {k: os.environ.get(k) for k in ("DIFFUSION_INT8", "DP_STEPS", "DP_SCHEDULER")}
    os.environ.update(DIFFUSION_INT8="1", DP_STEPS="2", DP_SCHEDULER="DDIM")
    try:
        m = vla.DiffusionModel(d)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    ref = m.predict(frames, state, noise, unnormalize=False)
    # per step: 2 convs per res block + the width-changing 1x1 convs + the
    # downsamples + the final conv
    nd = len(c["down_dims"])
    per_step = 2 * (4 * nd) + (2 * nd - 1) + (nd - 1) + 1  # 4 nd res blocks
    probed = []
    _check_steps(vla, orc, lambda: probed.append(m.predict(frames, state, noise, unnormalize=False)),
                 expect_min=2 * per_step, what=f"diffusion mask 1 {case}")
    assert probed[0].tobytes() == ref.tobytes()
    assert m.predict(frames, state, noise, unnormalize=False).tobytes() == ref.tobytes()
