"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the GPU checker.

Each oracle function is checked against
  * the golden vectors written by the real reference kernels (tests/golden/,
    made by tests/golden/gen_golden.py from oracle/_ref), bit-exact for the
    int8 path;
  * the reference build itself where it is present (oracle/_ref travels with
    the tree);
  * what the mathematics fixes: brute-force integer sums, double-precision
    formulas, linearity, the fully-masked and zero-mask special cases;
and a planted mistake shows each golden comparison can fail.
"""

import math

import numpy as np
import pytest

from helpers import golden, load_masks, load_synth, max_rel, oracle, same_bits, sha

ob = oracle()
LOWEST = np.finfo(np.float32).min

TESTOPS_GEMM = [(1, 16, 3), (7, 48, 64), (50, 768, 1027), (13, 64, 17), (257, 96, 48)]
ATTN_CFGS = [(1, 50, 8, 2, 64), (50, 50, 8, 2, 64), (50, 113, 15, 5, 64), (17, 33, 4, 4, 72),
             (9, 20, 2, 1, 256), (256, 256, 12, 12, 64), (12, 512, 4, 2, 64)]
NORM_SHAPES = [(1, 768), (50, 960), (7, 6), (302, 512), (658, 768), (177, 960), (50, 720)]


# ------------------------------------------------------------ quantizer --

def test_quantizer_edge_cases_match_reference():
    g = golden("quant_edge.npz")
    for i in range(int(g["count"])):
        xq, s = ob.quantize_act_i8(g[f"x_{i}"])
        assert same_bits(xq, g[f"xq_{i}"]) and same_bits(s, g[f"s_{i}"]), f"edge case {i}"


def test_quantizer_closed_form():
    """Per row: s = max|x|/127 (floor FLT_MIN, 1 for a zero row); q = rne(x/s
    computed as x*(1/s)); |q*s - x| <= s/2; padding zero."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 37)) * np.logspace(-40, 3, 64)[:, None]).astype(np.float32)
    x[5] = 0
    xq, s = ob.quantize_act_i8(x, ldq=48)
    for t in range(64):
        amax = np.float32(np.max(np.abs(x[t])))
        want = np.float32(1.0) if amax == 0 else max(np.float32(amax / np.float32(127.0)),
                                                     np.float32(np.finfo(np.float32).tiny))
        assert s[t] == want
        inv = np.float32(1.0) / want
        q = np.clip(np.rint((x[t] * inv).astype(np.float32)), -127, 127).astype(np.int8)
        assert np.array_equal(xq[t, :37], q)
        assert np.all(xq[t, 37:] == 0)
        assert np.all(np.abs(xq[t, :37].astype(np.float64) * s[t] - x[t]) <= s[t] * 0.5 + 1e-45)


def test_weight_quantizer_is_the_reference_packer():
    """pack_weights_i8 (gemm_i8.cpp:56-89) == oracle weight quantizer + row layout."""
    fr = ob.Frand()
    W = fr.rv(48 * 70, -0.2, 0.2).reshape(48, 70)
    rows, ws, _ = ob.ref_pack_weights(W)
    q, s = ob.quantize_weights_i8(W)
    assert same_bits(q, rows) and same_bits(s, ws)


# ----------------------------------------------------------------- GEMM --

def _testops_inputs():
    fr = ob.Frand()
    for idx, (seq, N, K) in enumerate(TESTOPS_GEMM):
        x = fr.rv(seq * K).reshape(seq, K)
        W = fr.rv(N * K, -0.2, 0.2).reshape(N, K)
        b = fr.rv(N)
        fr.rv(seq * N)
        yield idx, seq, N, K, x, W, b


def test_gemm_testops_golden():
    g = golden("gemm_testops.npz")
    for idx, seq, N, K, x, W, b in _testops_inputs():
        Wq, ws = ob.quantize_weights_i8(W)
        xq, sa = ob.quantize_act_i8(x)
        assert sha(Wq) == str(g[f"wq_sha_{idx}"]) and same_bits(ws, g[f"ws_{idx}"])
        assert sha(xq) == str(g[f"xq_sha_{idx}"]) and same_bits(sa, g[f"sa_{idx}"])
        assert same_bits(ob.gemm_i8_acc(xq, Wq, K), g[f"acc_{idx}"]), "int32 accumulators"
        out = ob.dense_linear_i8_pre(xq, sa, Wq, ws, b, K)
        assert same_bits(out, g[f"out_ref_{idx}"]), "vs dense_linear_i8_ref"
        if f"out_pre_{idx}" in g:
            assert same_bits(out, g[f"out_pre_{idx}"]), "vs the AVX-VNNI kernel"


def test_gemm_golden_catches_a_planted_mistake():
    """A dropped bias term or a transposed operand must fail the same check."""
    g = golden("gemm_testops.npz")
    for idx, seq, N, K, x, W, b in _testops_inputs():
        if idx != 1:
            continue
        Wq, ws = ob.quantize_weights_i8(W)
        xq, sa = ob.quantize_act_i8(x)
        assert not same_bits(ob.dense_linear_i8_pre(xq, sa, Wq, ws, None, K), g[f"out_ref_{idx}"])
        Wt = np.ascontiguousarray(Wq[:, ::-1][:, -((K + 3) & ~3):])
        assert not same_bits(ob.gemm_i8_acc(xq, Wt, K), g[f"acc_{idx}"])


def test_int32_accumulators_brute_force_and_linearity():
    rng = np.random.default_rng(3)
    for seq, N, K in ((1, 1, 1), (3, 5, 7), (9, 17, 130), (2, 33, 4099)):
        ld = (K + 3) & ~3
        xq = np.zeros((seq, ld), np.int8)
        W1 = np.zeros((N, ld), np.int8)
        W2 = np.zeros((N, ld), np.int8)
        xq[:, :K] = rng.integers(-127, 128, (seq, K))
        W1[:, :K] = rng.integers(-63, 64, (N, K))
        W2[:, :K] = rng.integers(-63, 64, (N, K))
        brute = xq[:, :K].astype(np.int64) @ W1[:, :K].astype(np.int64).T
        a1 = ob.gemm_i8_acc(xq, W1, K)
        assert np.array_equal(a1, brute)
        a12 = ob.gemm_i8_acc(xq, (W1.astype(np.int16) + W2).astype(np.int8), K)
        assert np.array_equal(a12, a1 + ob.gemm_i8_acc(xq, W2, K))


def test_extreme_accumulator_values():
    """|acc| up to K*127*127 and the (float)acc rounding past 2^24 (RNE)."""
    K = 4096
    xq = np.full((2, K), 127, np.int8)
    xq[1] = -127
    Wq = np.full((3, K), 127, np.int8)
    Wq[1] = -127
    Wq[2, ::2] = -127
    acc = ob.gemm_i8_acc(xq, Wq, K)
    assert acc[0, 0] == K * 127 * 127 and acc[1, 0] == -K * 127 * 127 and acc[0, 2] == 0
    out = ob.dense_linear_i8_pre(xq, np.ones(2, np.float32), Wq, np.ones(3, np.float32), None, K)
    assert out[0, 0] == np.float32(K * 127 * 127)


SYNTH_SHAPES_FOR_ORACLE = [0] + [i for i in range(1, 31)]


def _baseline_shapes():
    g = golden("gemm_baseline.npz")
    return g, [tuple(int(v) for v in s) for s in g["shapes"]]


def test_synthetic_inputs_are_reproducible():
    """The generator reproduces the exact input bytes the golden outputs were made from."""
    synth = load_synth()
    g, shapes = _baseline_shapes()
    for idx, (M, K, N) in enumerate(shapes):
        if M * K > 2048 * 4096:
            continue
        x, Wq, ws, b = synth.linear_case(M, K, N)
        assert list(g[f"in_sha_{idx}"]) == [sha(x), sha(Wq), sha(ws), sha(b)], (M, K, N)


def test_baseline_linear_matches_reference():
    """configs[0] in full and every sweep shape the oracle finishes in seconds:
    oracle quantizer + oracle linear == the reference's dense_linear_i8 bytes."""
    synth = load_synth()
    g, shapes = _baseline_shapes()
    for idx, (M, K, N) in enumerate(shapes):
        if M * N * K > 512 * 960 * 2560:
            continue
        x, Wq, ws, b = synth.linear_case(M, K, N)
        xq, sa = ob.quantize_act_i8(x)
        assert sha(xq) == str(g[f"xq_sha_{idx}"]) and sha(sa) == str(g[f"sa_sha_{idx}"])
        out = ob.dense_linear_i8_pre(xq, sa, Wq, ws, b, K)
        assert sha(out) == str(g[f"out_sha_{idx}"]), (M, K, N)
    assert same_bits(ob.quantize_act_i8(synth.linear_case(*synth.CONFIG1)[0])[0], g["cfg1_xq"])


@pytest.mark.skipif(not ob.ref_available(), reason="oracle/_ref not built")
def test_oracle_matches_reference_build_directly():
    synth = load_synth()
    for M, K, N in ((5, 40, 32), (100, 512, 3200), (33, 1027, 48)):
        x, Wq, ws, b = synth.linear_case(M, K, N, tag="direct")
        xq, sa = ob.quantize_act_i8(x)
        rx, rs = ob.ref_quantize_act_i8(x)
        assert same_bits(xq, rx) and same_bits(sa, rs)
        blob = ob.ref_panels(Wq, K)
        Wp = np.zeros((N, (K + 3) & ~3), np.int8)
        Wp[:, :K] = Wq
        assert same_bits(ob.dense_linear_i8_pre(xq, sa, Wp, ws, b, K),
                         ob.ref_dense_linear_i8_ref(rx, rs, blob, ws, b, N, K))


# ------------------------------------------------------------ attention --

def naive(Q, K, V, sq, sk, nq, nkv, hd, scale, mask=None):
    Q = Q.reshape(sq, nq, hd).astype(np.float64)
    K = K.reshape(sk, nkv, hd).astype(np.float64)
    V = V.reshape(sk, nkv, hd).astype(np.float64)
    g = nq // nkv
    out = np.zeros((sq, nq, hd))
    for h in range(nq):
        s = Q[:, h, :] @ K[:, h // g, :].T * scale
        if mask is not None:
            s = np.where(mask == LOWEST, -np.inf, s + mask.astype(np.float64))
        mx = s.max(axis=1, keepdims=True)
        full = np.isneginf(mx[:, 0])
        e = np.where(np.isneginf(s), 0.0, np.exp(s - np.where(np.isneginf(mx), 0, mx)))
        o = (e @ V[:, h // g, :]) / np.maximum(e.sum(axis=1, keepdims=True), 1e-300)
        o[full] = V[:, h // g, :].mean(axis=0)
        out[:, h, :] = o
    return out.reshape(sq, nq * hd)


def _attn_inputs(sq, sk, nq, nkv, hd):
    fr = ob.Frand()
    return (fr.rv(sq * nq * hd).reshape(sq, nq * hd), fr.rv(sk * nkv * hd).reshape(sk, nkv * hd),
            fr.rv(sk * nkv * hd).reshape(sk, nkv * hd))


@pytest.mark.parametrize("idx", range(len(ATTN_CFGS)))
def test_attention_golden_and_closed_form(idx):
    g = golden("attention.npz")
    sq, sk, nq, nkv, hd = ATTN_CFGS[idx]
    Q, K, V = _attn_inputs(sq, sk, nq, nkv, hd)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    rows = g[f"rows_{idx}"]
    dense = ob.attention(Q, K, V, sq, sk, nq, nkv, hd, scale)
    assert max_rel(dense[rows], g[f"dense_{idx}"]) <= 2e-6
    assert max_rel(dense, naive(Q, K, V, sq, sk, nq, nkv, hd, scale)) <= 2e-6
    zero = ob.attention(Q, K, V, sq, sk, nq, nkv, hd, scale, np.zeros((sq, sk), np.float32))
    assert same_bits(dense, zero), "zero mask must equal no mask"
    i, j = np.arange(sq)[:, None], np.arange(sk)[None, :]
    causal = np.where(j > i + (sk - sq), -np.inf, 0.0).astype(np.float32)
    cz = ob.attention(Q, K, V, sq, sk, nq, nkv, hd, scale, causal)
    assert max_rel(cz[rows], g[f"causal_{idx}"]) <= 2e-6
    assert max_rel(cz, naive(Q, K, V, sq, sk, nq, nkv, hd, scale, causal)) <= 2e-6
    full = ob.attention(Q, K, V, sq, sk, nq, nkv, hd, scale, np.full((sq, sk), LOWEST, np.float32))
    assert max_rel(full[rows], g[f"full_{idx}"]) <= 2e-6
    mean = V.reshape(sk, nkv, hd).astype(np.float64).mean(axis=0)
    assert np.max(np.abs(full[0].reshape(nq, hd) - mean[np.arange(nq) // (nq // nkv)])) < 2e-6
    # planted mistake: a missing scale must fail the golden check
    bad = ob.attention(Q, K, V, sq, sk, nq, nkv, hd, 1.0)
    assert max_rel(bad[rows], g[f"dense_{idx}"]) > 1e-3


def test_model_masks_golden():
    g = golden("attention.npz")
    masks = load_masks()
    synth = load_synth()
    cases = []
    qg, kg, al, T = masks.octo_block_causal(wnd=2, repeat_task=False)
    cases.append(("octo658", T, T, 12, 12, masks.dense(masks.keep_from_groups(qg, kg, al))))
    lang = np.ones(48, np.uint8)
    lang[40:] = 0
    qg, kg, al, pad = masks.smolvla_prefix_lm(128, 48, lang)
    cases.append(("smol_prefix", len(pad), len(pad), 15, 5, masks.dense(masks.keep_from_groups(qg, kg, al))))
    q2, k2, a2, SK = masks.smolvla_denoise(pad, 50)
    cases.append(("smol_expert", 50, SK, 15, 5, masks.dense(masks.keep_from_groups(q2, k2, a2))))
    cases.append(("act_enc", 302, 302, 8, 8, None))
    cases.append(("act_cross", 100, 302, 8, 8, None))
    for name, sq, sk, nq, nkv, m in cases:
        Q = synth.normal(f"gold.{name}.q", (sq, nq * 64))
        K = synth.normal(f"gold.{name}.k", (sk, nkv * 64))
        V = synth.normal(f"gold.{name}.v", (sk, nkv * 64))
        o = ob.attention(Q, K, V, sq, sk, nq, nkv, 64, np.float32(0.125), m)
        rows = g[f"m_{name}_rows"]
        assert max_rel(o[rows], g[f"m_{name}_out"]) <= 2e-6, name


def _octo_keep_direct(n_task, tp, tw, nr, wnd, tsm, wrist, repeat):
    """octo_transformer.cpp:106-142 written out as loops, for the mask-builder check."""
    grp, ts, pad = [], [], []
    for _ in range(n_task):
        grp.append(0); ts.append(-1); pad.append(1)
    per = [(1, tp), (2, tw)] + ([(3, n_task)] if repeat else []) + [(4, nr)]
    for t in range(wnd):
        for gk, n in per:
            for _ in range(n):
                grp.append(gk); ts.append(t)
                pad.append(tsm[t] if gk == 1 else (int(wrist and tsm[t]) if gk == 2 else 1))
    T = len(grp)
    keep = np.zeros((T, T), bool)
    for i in range(T):
        for j in range(T):
            gi, ti, gj, tj = grp[i], ts[i], grp[j], ts[j]
            if gi == 0:
                a = gj == 0
            elif gj == 0:
                a = True
            elif gj <= 3:
                a = tj <= ti
            else:
                a = gi == 4 and gj == 4 and tj <= ti
            keep[i, j] = a and bool(pad[j])
    return keep


@pytest.mark.parametrize("tsm,wrist,repeat", [((1, 1), True, False), ((0, 1), True, True),
                                               ((1, 1), False, True)])
def test_octo_group_mask_equals_direct_rule(tsm, wrist, repeat):
    masks = load_masks()
    qg, kg, al, T = masks.octo_block_causal(n_task=4, tok_primary=6, tok_wrist=3, n_readout=1, wnd=2,
                                            timestep_mask=tsm, wrist=wrist, repeat_task=repeat)
    want = _octo_keep_direct(4, 6, 3, 1, 2, tsm, wrist, repeat)
    assert np.array_equal(masks.keep_from_groups(qg, kg, al), want)


def test_smolvla_group_masks_equal_direct_rule():
    masks = load_masks()
    lang = np.array([1, 1, 1, 0, 0], np.uint8)
    qg, kg, al, pad = masks.smolvla_prefix_lm(3, 5, lang)
    n = len(pad)
    att = np.zeros(n, int)
    att[-1] = 1
    want = np.array([[att[j] <= att[i] and pad[i] and pad[j] for j in range(n)] for i in range(n)])
    assert np.array_equal(masks.keep_from_groups(qg, kg, al), want)
    q2, k2, a2, SK = masks.smolvla_denoise(pad, 4)
    want2 = np.array([[bool(pad[j]) if j < n else (j - n) <= i for j in range(SK)] for i in range(4)])
    assert np.array_equal(masks.keep_from_groups(q2, k2, a2), want2)


# ------------------------------------------------------- norms, eltwise --

def _norm_inputs(seq, H):
    fr = ob.Frand()
    return fr.rv(seq * H, -3.0, 5.0).reshape(seq, H), fr.rv(H), fr.rv(H)


@pytest.mark.parametrize("idx", range(len(NORM_SHAPES)))
def test_norms_golden_and_double_formula(idx):
    g = golden("norms.npz")
    seq, H = NORM_SHAPES[idx]
    x, w, b = _norm_inputs(seq, H)
    rows = g[f"rows_{idx}"]
    ln = ob.layernorm(x, w, b, 1e-5)
    rms = ob.rmsnorm(x, w, 1e-6)
    assert np.max(np.abs(ln[rows] - g[f"ln_{idx}"])) <= 1e-6
    assert np.max(np.abs(ob.layernorm(x, w, None, 1e-6)[rows] - g[f"ln_nob_{idx}"])) <= 1e-6
    assert np.max(np.abs(rms[rows] - g[f"rms_{idx}"])) <= 1e-6
    xd = x.astype(np.float64)
    mu = xd.mean(axis=1, keepdims=True)
    ref_ln = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5) * w + b
    ref_rms = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(ln - ref_ln)) <= 1e-5 and np.max(np.abs(rms - ref_rms)) <= 1e-5


def test_eltwise_golden_and_libm():
    g = golden("eltwise.npz")
    x = ob.Frand().rv(20011, -30.0, 30.0)
    u = ob.Frand(12345).rv(20011, -2.0, 2.0)
    checks = {
        "gelu_tanh": (ob.gelu_tanh(x), lambda v: 0.5 * v * (1 + math.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))),
        "gelu_erf": (ob.gelu_erf(x), lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2)))),
        "relu": (ob.relu(x), lambda v: max(v, 0.0)),
    }
    for name, (got, f) in checks.items():
        assert max_rel(got, g[name]) <= 2e-6, name
        assert max_rel(got, np.array([f(float(v)) for v in x])) <= 2e-6, name
    sg = ob.silu_gate(x, u)
    assert max_rel(sg, g["silu_gate"]) <= 2e-6
    assert max_rel(sg, np.array([float(a) / (1 + math.exp(-float(a))) * float(c) for a, c in zip(x, u)])) <= 2e-6
    assert same_bits(ob.relu(x), g["relu"])


def test_rope_golden():
    g = golden("rope.npz")
    synth = load_synth()
    for idx, (seq, nh, hd) in enumerate(((177, 15, 64), (50, 5, 64), (7, 3, 16))):
        x = synth.normal(f"rope.{seq}", (seq, nh * hd))
        pos = np.arange(seq, dtype=np.int32) + 3
        got = ob.rope_neox(x, pos, nh, hd, 10000.0)[g[f"rows_{idx}"]]
        assert np.max(np.abs(got - g[f"rope_{idx}"])) <= 1e-6 * max(1.0, float(np.max(np.abs(got))))
        # closed form: rotation preserves each pair's norm
        xr = x.reshape(seq, nh, hd)
        gr = ob.rope_neox(x, pos, nh, hd, 10000.0).reshape(seq, nh, hd)
        h = hd // 2
        assert np.allclose(xr[..., :h] ** 2 + xr[..., h:] ** 2, gr[..., :h] ** 2 + gr[..., h:] ** 2, rtol=1e-5)
