"""Device policy graphs (ACT, Octo, SmolVLA) against the reference's own graphs.

Both sides load the same synthetic checkpoint files (vla_simd_amd.checkpoints,
written in the reference's .meta/.bin layouts) and run on the same seeded
inputs: the device graph through libvla_simd_hip.so's C ABI, the reference
through oracle/_ref/libvla_ref.so (ActTransformer, OctoTransformer,
SmollmVlm + ActionExpert compiled from the reference sources).

Two bars:
  * int8 mask 0 (every layer fp32): the graphs differ from the reference only
    by fp32 summation order, so outputs agree to 1e-3 of the output scale (the
    north-star tolerance for fp32 outputs; measured ~1e-6).
  * the BASELINE int8 masks: every int8 linear is bit-exact given identical
    inputs (tests/test_gpu_gemm.py, test_gpu_golden.py), but the fp32 ops
    between them (attention, norms, activations) differ by a few ulp, and a
    value within that distance of a quantization rounding boundary moves one
    int8 step; the flips compound through every later re-quantization. The
    reference itself is that sensitive: nudging each input element by -1, 0 or
    +1 ulp moves its own int8 output by ~3e-3 (ACT), ~2.5e-2 (Octo) and ~1.5e-2
    (SmolVLA) of the output scale. So the bar is computed here, on the same
    checkpoint and inputs: the device graph must sit within twice the largest
    of two such reference-vs-reference ulp perturbations.
Replays of the captured HIP graph must reproduce the first (eager) call bit
for bit.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from helpers import load_pkg

pytestmark = pytest.mark.gpu


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


def _rel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape and np.all(np.isfinite(got))
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.fixture(scope="module")
def ckdir(tmp_path_factory):
    return tmp_path_factory.mktemp("ck")


def _ulp(x, k):
    """x with each element moved by -1, 0 or +1 ulp (seeded)."""
    r = np.random.default_rng(1000 + k)
    s = r.integers(0, 3, size=x.shape) - 1
    y = np.array(x, np.float32, copy=True)
    y[s > 0] = np.nextafter(y[s > 0], np.float32(np.inf))
    y[s < 0] = np.nextafter(y[s < 0], np.float32(-np.inf))
    return y


def _bar(mask, run_ref, x, ref):
    """fp32 graphs: 1e-3. int8 graphs: twice the reference's own spread under
    two 1-ulp perturbations of input x (run_ref(x') -> output)."""
    if mask == 0:
        return 1e-3, 0.0
    sens = max(_rel(run_ref(_ulp(x, k)), ref) for k in range(2))
    return max(2.0 * sens, 1e-3), sens


def _check_replay(run, first):
    for _ in range(3):
        again = run()
        assert again.tobytes() == first.tobytes(), "graph replay differs from the eager call"


# ----------------------------------------------------------------- ACT ----

@pytest.mark.parametrize("mask", [0, 31])
def test_act_transformer(vla, ckdir, mask):
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = ck.ACT_BASE
    d = str(ckdir / "act")
    if not os.path.exists(os.path.join(d, "act.bin")):
        ck.write_act(d, c)
    feats, state = ck.act_inputs(c)
    print(f"act mask {mask}: T = {1 * 15 * 20 + 2}", flush=True)
    r = ob.RefAct(d, c["img_ch"], mask, c["chunk"], c["action_dim"])
    ref = r.forward(feats, c["n_cams"], c["fh"], c["fw"], state)
    bar, sens = _bar(mask, lambda f: r.forward(f, c["n_cams"], c["fh"], c["fw"], state), feats, ref)
    m = vla.ActTransformer(d, c["img_ch"], mask)
    assert m.int8_layers == (0 if mask == 0 else 4 * 4 + 4 * 2 + 1 + 10)
    got = m.forward(feats, c["n_cams"], c["fh"], c["fw"], state)
    err = _rel(got, ref)
    print(f"act mask {mask}: rel err {err:.3e} (reference ulp spread {sens:.3e}, bar {bar:.3e})", flush=True)
    assert err <= bar
    _check_replay(lambda: m.forward(feats, c["n_cams"], c["fh"], c["fw"], state), got)
    assert m.graph_nodes > 0


def test_act_two_cameras(vla, ckdir):
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = dict(ck.ACT_BASE, n_cams=2, fh=6, fw=8, n_enc=2)
    d = str(ckdir / "act2")
    ck.write_act(d, c)
    feats, state = ck.act_inputs(c)
    r = ob.RefAct(d, c["img_ch"], 31, c["chunk"], c["action_dim"])
    ref = r.forward(feats, 2, 6, 8, state)
    bar, sens = _bar(31, lambda f: r.forward(f, 2, 6, 8, state), feats, ref)
    got = vla.ActTransformer(d, c["img_ch"], 31).forward(feats, 2, 6, 8, state)
    err = _rel(got, ref)
    print(f"act 2 cams: rel err {err:.3e} (reference ulp spread {sens:.3e})", flush=True)
    assert err <= bar


@pytest.mark.parametrize("small", [False, True])
def test_act_paired_projections_bit_exact(vla, ckdir, small):
    """q | k (from x + pos) and v (from x), and the decoder's cross k and v,
    run as one skinny GEMM launch per pair (gemm_i8_skinny_pair: each block
    runs its own product's code and sums); the forward must equal, bit for
    bit, the same forward with every product in its own launch
    (VLA_HIP_GEMM_PAIR=0). The full shape takes the 129-320-row route in the
    encoder (302 rows) and the panel route in the decoder (100 rows); the
    small one (50 rows) the panel route throughout."""
    ck = _ck()
    if small:
        c = dict(ck.ACT_BASE, n_enc=2, fh=6, fw=8)
        d = str(ckdir / "act_pair_small")
        ck.write_act(d, c)
    else:
        c = ck.ACT_BASE
        d = str(ckdir / "act")
        if not os.path.exists(os.path.join(d, "act.bin")):
            ck.write_act(d, c)
    feats, state = ck.act_inputs(c)
    run = lambda m: m.forward(feats, c["n_cams"], c["fh"], c["fw"], state)
    os.environ["VLA_HIP_GEMM_PAIR"] = "0"
    try:
        m0 = vla.ActTransformer(d, c["img_ch"], 31)
        ref = run(m0)
        ref2 = run(m0)  # the captured graph as well
    finally:
        del os.environ["VLA_HIP_GEMM_PAIR"]
    m1 = vla.ActTransformer(d, c["img_ch"], 31)
    got = run(m1)
    print(f"act paired projections small {small}: max |diff| {np.max(np.abs(got - ref)):.3e}, "
          f"nodes {m0.graph_nodes} -> {m1.graph_nodes}", flush=True)
    assert got.tobytes() == ref.tobytes() and ref2.tobytes() == ref.tobytes()
    _check_replay(lambda: run(m1), got)
    assert m1.graph_nodes < m0.graph_nodes


@pytest.mark.parametrize("mask", [0, 31])
def test_act_decoder_head_bit_exact(vla, ckdir, mask):
    """Decoder layer 0's self-attention block and norm1 read only the zero
    queries, dec_pos and weights: the graph computes them once per model and
    copies them in (dx and the cross-query input, fp32 rows at mask 0, int8
    bytes at 31). The forward must equal, bit for bit, the one that recomputes
    them every call (VLA_HIP_ACT_HEAD=0), on eager calls and graph replays."""
    ck = _ck()
    c = ck.ACT_BASE
    d = str(ckdir / "act")
    if not os.path.exists(os.path.join(d, "act.bin")):
        ck.write_act(d, c)
    feats, state = ck.act_inputs(c)
    feats2 = np.ascontiguousarray(feats[::-1])
    run = lambda m, f: m.forward(f, c["n_cams"], c["fh"], c["fw"], state)
    os.environ["VLA_HIP_ACT_HEAD"] = "0"
    try:
        m0 = vla.ActTransformer(d, c["img_ch"], mask)
        ref = [run(m0, feats), run(m0, feats2), run(m0, feats)]
    finally:
        del os.environ["VLA_HIP_ACT_HEAD"]
    m1 = vla.ActTransformer(d, c["img_ch"], mask)
    got = [run(m1, feats), run(m1, feats2), run(m1, feats)]
    for g, r in zip(got, ref):
        assert g.tobytes() == r.tobytes()
    print(f"act decoder head mask {mask}: nodes {m0.graph_nodes} -> {m1.graph_nodes}", flush=True)
    assert m1.graph_nodes < m0.graph_nodes


# -------------------------------------------------------------- IMPACT ----

@pytest.mark.parametrize("mask,n_real", [(0, 11), (31, 11), (31, 16), (31, 40), (31, 0), (15, 5)])
def test_impact_transformer(vla, ckdir, mask, n_real):
    """IMPACT's W8A8 transformer (impact_model.cpp:59-68): the ACT graph loaded
    with int8_state (the state projection joins mask bit 8,
    act_transformer.cpp:127-130) and run with its text tower's tokens and
    positions appended after the cameras, clamped to act.meta's n_text
    (build_tokens :212-250). Against the reference's ActTransformer loaded and
    run the same way; same bars as test_act_transformer."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = dict(ck.ACT_BASE, n_text=16, n_enc=2, fh=6, fw=8)
    d = str(ckdir / "impact")
    if not os.path.exists(os.path.join(d, "act.bin")):
        ck.write_act(d, c)
    feats, state = ck.act_inputs(c)
    import vla_simd_amd.synth as synth
    text = synth.normal("impact.text", (c["n_text"], c["dim"]), 1.0)
    tpos = synth.normal("impact.text_pos", (c["n_text"], c["dim"]), 0.02)
    print(f"impact mask {mask} n_text_real {n_real}", flush=True)
    r = ob.RefAct(d, c["img_ch"], mask, c["chunk"], c["action_dim"], int8_state=True)
    ref = r.forward_text(feats, 1, c["fh"], c["fw"], state, text, tpos, n_real)
    bar, sens = _bar(mask, lambda f: r.forward_text(f, 1, c["fh"], c["fw"], state, text, tpos, n_real), feats, ref)
    m = vla.ActTransformer(d, c["img_ch"], mask, int8_state=True)
    n_i8 = (2 * 4 if mask & 1 else 0) + (2 if mask & 2 else 0) + (2 if mask & 4 else 0) + \
           (2 if mask & 8 else 0) + (10 if mask & 16 else 0)
    assert m.n_text == 16 and m.int8_layers == n_i8
    got = m.forward_text(feats, 1, c["fh"], c["fw"], state, text, tpos, n_real)
    err = _rel(got, ref)
    print(f"impact mask {mask} n_text_real {n_real}: rel err {err:.3e} (reference ulp spread {sens:.3e})",
          flush=True)
    assert err <= bar
    _check_replay(lambda: m.forward_text(feats, 1, c["fh"], c["fw"], state, text, tpos, n_real), got)
    # without text the same handle is the plain ACT transformer (the reference with n_text_real = 0)
    if n_real == 0:
        assert m.forward(feats, 1, c["fh"], c["fw"], state).tobytes() == got.tobytes()


# ---------------------------------------------------------------- Octo ----

@pytest.mark.parametrize("mask,wrist,tmask", [(0, True, (1, 1)), (7, True, (1, 1)), (15, True, (1, 1)),
                                              (7, False, (1, 1)), (7, True, (0, 1))])
def test_octo_transformer(vla, ckdir, mask, wrist, tmask):
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = dict(ck.OCTO_BASE, repeat_task=1)  # the reference always repeats the task tokens
    d = str(ckdir / "octo")
    if not os.path.exists(os.path.join(d, "octo.bin")):
        ck.write_octo(d, c)
    t5, sp, sw, _ = ck.octo_inputs(c)
    tm = np.array(tmask, np.uint8)
    sw = sw if wrist else None
    print(f"octo mask {mask} wrist {wrist} tmask {tmask}", flush=True)
    r = ob.RefOcto(d, mask, c["d"])
    ref = r.forward(t5, sp, sw, 2, tm)
    bar, sens = _bar(mask, lambda x: r.forward(t5, x, sw, 2, tm), sp, ref)
    m = vla.OctoTransformer(d, mask)
    assert m.total_tokens(2) == 16 + 2 * (256 + 64 + 16 + 1)
    got = m.forward(t5, sp, sw, 2, tm)
    err = _rel(got, ref)
    print(f"octo mask {mask}: rel err {err:.3e} (reference ulp spread {sens:.3e})", flush=True)
    assert err <= bar
    _check_replay(lambda: m.forward(t5, sp, sw, 2, tm), got)


@pytest.mark.parametrize("mask,wrist,tmask", [(0, True, (1, 1)), (7, True, (1, 1)), (15, True, (1, 1)),
                                              (7, False, (1, 1)), (7, True, (0, 1))])
def test_octo_658_tokens(vla, ckdir, mask, wrist, tmask):
    """the Octo-base graph over the 658-token layout (16
    task tokens, then per timestep 256 primary + 64 wrist + 1 readout, with no
    per-step task copy; checkpoint meta repeat_task 0). The reference's
    forward() always repeats the task tokens, so the checker is the
    reference's own loaded layers driven over the 658-token layout
    (RefOcto.forward_layout, oracle/ref_models_shim.cpp), which reproduces
    forward() bit for bit at the 690-token layout (tests/test_ref_layouts.py).
    Same bars as the 690-token test."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = dict(ck.OCTO_BASE, repeat_task=0)
    d = str(ckdir / "octo658")
    if not os.path.exists(os.path.join(d, "octo.bin")):
        ck.write_octo(d, c)
    t5, sp, sw, _ = ck.octo_inputs(c)
    tm = np.array(tmask, np.uint8)
    sw = sw if wrist else None
    print(f"octo 658 mask {mask} wrist {wrist} tmask {tmask}", flush=True)
    r = ob.RefOcto(d, mask, c["d"])
    ref = r.forward_layout(t5, sp, sw, 2, tm, 0)
    bar, sens = _bar(mask, lambda x: r.forward_layout(t5, x, sw, 2, tm, 0), sp, ref)
    m = vla.OctoTransformer(d, mask)
    assert m.total_tokens(2) == 658
    got = m.forward(t5, sp, sw, 2, tm)
    err = _rel(got, ref)
    print(f"octo 658 mask {mask}: rel err {err:.3e} (reference ulp spread {sens:.3e}, bar {bar:.3e})", flush=True)
    assert err <= bar
    _check_replay(lambda: m.forward(t5, sp, sw, 2, tm), got)


# ------------------------------------------------------------- SmolVLA ----

@pytest.mark.parametrize("mask,n_pad", [(0, 0), (48, 0), (48, 5)])
def test_smolvla_chunk(vla, ckdir, mask, n_pad):
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = ck.SMOLVLA_BASE
    d = str(ckdir / "smol")
    if not os.path.exists(os.path.join(d, "aex.bin")):
        ck.write_smolvla(d, c)
    prefix, pad, noise = ck.smolvla_inputs(c, n_pad=n_pad)
    print(f"smolvla mask {mask} n_pad {n_pad}", flush=True)
    r = ob.RefSmolvla(d, mask)
    ref = r.run(prefix, pad, noise)
    bar, sens = _bar(mask, lambda x: r.run(x, pad, noise), prefix, ref)
    m = vla.SmolvlaChunk(d, mask)
    got = m.run(prefix, pad, noise)
    err = _rel(got, ref)
    print(f"smolvla mask {mask} n_pad {n_pad}: rel err {err:.3e} (reference ulp spread {sens:.3e})",
          flush=True)
    assert err <= bar
    _check_replay(lambda: m.run(prefix, pad, noise), got)


@pytest.mark.parametrize("mask", [0, 48])
def test_smolvla_short_chunk(vla, ckdir, mask):
    """A 12-action chunk (4 layers, 60 prefix tokens): the expert's int8 layers
    take at most 16 rows, so their RMSNorm / silu_gate / quantize row ops run
    inside the GEMM (gemm_i8_rowop) rather than as separate kernels; same bar."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = dict(ck.SMOLVLA_BASE, chunk=12, n_layers=4, expert_layers=4, n_prefix=60)
    d = str(ckdir / "smol12")
    if not os.path.exists(os.path.join(d, "aex.bin")):
        ck.write_smolvla(d, c)
    prefix, pad, noise = ck.smolvla_inputs(c, n_pad=3)
    print(f"smolvla chunk 12 mask {mask}", flush=True)
    r = ob.RefSmolvla(d, mask)
    ref = r.run(prefix, pad, noise)
    bar, sens = _bar(mask, lambda x: r.run(x, pad, noise), prefix, ref)
    m = vla.SmolvlaChunk(d, mask)
    got = m.run(prefix, pad, noise)
    err = _rel(got, ref)
    print(f"smolvla chunk 12 mask {mask}: rel err {err:.3e} (reference ulp spread {sens:.3e})", flush=True)
    assert err <= bar
    _check_replay(lambda: m.run(prefix, pad, noise), got)


@pytest.mark.parametrize("mask,short", [(32, False), (48, False), (48, True)])
def test_smolvla_rope_epilogue_bit_exact(vla, ckdir, mask, short):
    """The expert's int8 q|k|v and q projections rotate their q/k heads in the
    skinny GEMM's epilogue (each block owns 8 rotation pairs of a head); the
    chunk must equal, bit for bit, the same chunk with the GEMM storing plain
    outputs and the separate RoPE kernel rotating them
    (VLA_HIP_ROPE_FUSE=0): same epilogue floats, same rotation (rope.h)."""
    ck = _ck()
    if short:
        c = dict(ck.SMOLVLA_BASE, chunk=12, n_layers=4, expert_layers=4, n_prefix=60)
        d = str(ckdir / "smol12")
    else:
        c = ck.SMOLVLA_BASE
        d = str(ckdir / "smol")
    if not os.path.exists(os.path.join(d, "aex.bin")):
        ck.write_smolvla(d, c)
    prefix, pad, noise = ck.smolvla_inputs(c, n_pad=3)
    os.environ["VLA_HIP_ROPE_FUSE"] = "0"
    try:
        ref = vla.SmolvlaChunk(d, mask).run(prefix, pad, noise)
    finally:
        del os.environ["VLA_HIP_ROPE_FUSE"]
    got = vla.SmolvlaChunk(d, mask).run(prefix, pad, noise)
    print(f"smolvla rope epilogue mask {mask} short {short}: max |diff| {np.max(np.abs(got - ref)):.3e}",
          flush=True)
    assert got.tobytes() == ref.tobytes()


def test_models_load_from_gguf(vla, ckdir):
    """The device graphs loaded from a vla.simd GGUF (vla_ckpt_open's mount of
    the single-file checkpoint) give bit-identical outputs to the same graphs
    loaded from the converted directory; tests/test_gguf.py pins the file
    layer itself against the reference's reader."""
    ck = _ck()
    act = dict(ck.ACT_BASE, n_enc=2, fh=6, fw=8)
    d, g = str(ckdir / "act_g"), str(ckdir / "act_g.gguf")
    ck.write_act(d, act)
    ck.write_gguf(d, g, "act")
    feats, state = ck.act_inputs(act)
    outs = [vla.ActTransformer(p, act["img_ch"], 31).forward(feats, 1, 6, 8, state) for p in (d, g)]
    assert outs[0].tobytes() == outs[1].tobytes()

    octo = dict(ck.OCTO_BASE, n_layers=3, repeat_task=1)
    d, g = str(ckdir / "octo_g"), str(ckdir / "octo_g.gguf")
    ck.write_octo(d, octo)
    ck.write_gguf(d, g, "octo")
    t5, sp, sw, tm = ck.octo_inputs(octo)
    outs = [vla.OctoTransformer(p, 7).forward(t5, sp, sw, 2, tm) for p in (d, g)]
    assert outs[0].tobytes() == outs[1].tobytes()

    smol = dict(ck.SMOLVLA_BASE, n_layers=4, expert_layers=4)
    d, g = str(ckdir / "smol_g"), str(ckdir / "smol_g.gguf")
    ck.write_smolvla(d, smol)
    ck.write_gguf(d, g, "smolvla", layout=ck.smolvla_gguf_layout(smol))
    prefix, pad, noise = ck.smolvla_inputs(smol, n_pad=2)
    outs = [vla.SmolvlaChunk(p, 48).run(prefix, pad, noise) for p in (d, g)]
    assert outs[0].tobytes() == outs[1].tobytes()
    print("act / octo / smolvla from GGUF: identical to the directory loads", flush=True)


@pytest.mark.parametrize("line,ok", [("dim 512", True), ("dim   512   ", True), ("dim 512.0", False),
                                     ("dim 5e2", False), ("n_text -1", False), ("n_text 0", True),
                                     ("ln_eps 1e-5", True), ("ln_eps x", False), ("extra 1.5 junk", True)])
def test_act_meta_read_like_the_reference(vla, ckdir, line, ok):
    """act.meta values are read as the reference reads them
    (act_transformer.cpp:31-52: `ss >> int` per known key, nothing after it;
    n_text >= 0): the device loader accepts exactly what the reference accepts."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = dict(ck.ACT_BASE, n_enc=1, fh=2, fw=3)
    d = str(ckdir / f"actmeta_{abs(hash(line))}")
    ck.write_act(d, c)
    meta = os.path.join(d, "act.meta")
    key = line.split()[0]
    lines = [ln for ln in open(meta).read().splitlines() if ln.split()[0] != key] + [line]
    with open(meta, "w") as f:
        f.write("\n".join(lines) + "\n")
    try:
        ob.RefAct(d, c["img_ch"], 31, c["chunk"], c["action_dim"])
        ref_ok = True
    except RuntimeError:
        ref_ok = False
    try:
        vla.ActTransformer(d, c["img_ch"], 31).close()
        dev_ok = True
    except vla.VlaError:
        dev_ok = False
    assert ref_ok == ok and dev_ok == ok


def test_smolvla_pad_values_beyond_0_1_follow_the_reference(vla, ckdir):
    """A pad entry is a truth value in the masks and its raw value is summed
    into the positions (smolvla_model.cpp:224-246), so entries such as 2 or -1
    shift the RoPE positions of the tokens after them: the device graph takes
    them as the reference does (same bar as test_smolvla_chunk), and a layout
    change rebuilds the graph (the 0/1 pad of the same tokens gives another
    output)."""
    ck = _ck()
    from helpers import oracle
    ob = oracle()
    c = dict(ck.SMOLVLA_BASE, chunk=12, n_layers=2, expert_layers=2, n_prefix=20)
    d = str(ckdir / "smolpad")
    ck.write_smolvla(d, c)
    prefix, pad, noise = ck.smolvla_inputs(c, n_pad=2)
    m = vla.SmolvlaChunk(d, 0)
    r = ob.RefSmolvla(d, 0)
    plain = m.run(prefix, pad, noise)
    for vals in ([2, 1], [-1, 3], [5, 0]):
        odd = np.array(pad, np.int32)
        odd[0], odd[5] = vals
        ref = r.run(prefix, odd, noise)
        got = m.run(prefix, odd, noise)
        assert _rel(got, ref) <= 1e-3, vals
        assert not np.array_equal(got, plain), vals
        assert _rel(m.run(prefix, pad, noise), plain) == 0.0
    # the running sum must stay within int32
    huge = np.array(pad, np.int32)
    huge[:3] = 2**31 - 1
    out = np.empty((m.chunk, m.max_action_dim), np.float32)
    st = vla.lib().vla_smolvla_tf_chunk_run(m.h, vla._ptr(np.ascontiguousarray(prefix, np.float32)),
                                            vla._ptr(huge), prefix.shape[0],
                                            vla._ptr(np.ascontiguousarray(noise, np.float32)), vla._ptr(out))
    assert st == vla.VLA_ERR_ARG and b"overflow" in vla.lib().vla_last_error()