"""GPU results against the golden vectors the real reference wrote (tests/golden/).

int8 path at BASELINE.json's full sizes (configs[0] and every configs[1] sweep
shape, up to 8192 x 4096 x 4096): the device quantizer and GEMM must give the
reference's exact bytes - compared through SHA-256 digests of the whole xq,
ascale and fp32 output, plus the stored samples. Inputs are regenerated here
from vla_simd_amd.synth and their digests checked first.

fp32 path (attention, norms, activations, RoPE): within 2e-5 of max(|ref|, 1)
of the reference's own outputs (BASELINE bar: 1e-3 relative).
"""

import numpy as np
import pytest

from helpers import golden, load_masks, load_synth, max_rel, sha

pytestmark = pytest.mark.gpu

_G = None


def _gemm_golden():
    global _G
    if _G is None:
        _G = golden("gemm_baseline.npz")
    return _G


@pytest.mark.parametrize("idx", range(31))
def test_baseline_gemm_bit_exact(vla, torch_cuda, idx):
    torch = torch_cuda
    g = _gemm_golden()
    M, K, N = (int(v) for v in g["shapes"][idx])
    synth = load_synth()
    x, Wq, ws, b = synth.linear_case(M, K, N)
    assert list(g[f"in_sha_{idx}"]) == [sha(x), sha(Wq), sha(ws), sha(b)], "synthetic inputs differ"
    print(f"case {M}x{K}x{N}", flush=True)
    lin = vla.LinearI8.from_i8(Wq, ws, b)
    dev = torch.device("cuda")
    xd = torch.from_numpy(x).to(dev)
    xq = torch.zeros((M, lin.ldw), dtype=torch.int8, device=dev)
    sa = torch.empty(M, dtype=torch.float32, device=dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    lin.forward_dev(out, xd, xq, sa)
    torch.cuda.synchronize()
    xq_h = np.ascontiguousarray(xq.cpu().numpy()[:, :K])
    assert sha(xq_h) == str(g[f"xq_sha_{idx}"]), "int8 activations differ from the reference"
    assert sha(sa.cpu().numpy()) == str(g[f"sa_sha_{idx}"]), "activation scales differ"
    o = out.cpu().numpy()
    assert np.array_equal(o.reshape(-1)[g[f"out_idx_{idx}"]], g[f"out_val_{idx}"])
    assert sha(o) == str(g[f"out_sha_{idx}"]), "fp32 output differs from the reference"
    lin.close()


def test_testops_gemm_golden(vla, orc):
    """test_ops.cpp:138 shapes through the host op forms, against the reference's
    dense_linear_i8_ref / VNNI outputs and its int32 accumulators."""
    g = golden("gemm_testops.npz")
    fr = orc.Frand()
    for idx, (seq, N, K) in enumerate([(1, 16, 3), (7, 48, 64), (50, 768, 1027), (13, 64, 17),
                                       (257, 96, 48)]):
        x = fr.rv(seq * K).reshape(seq, K)
        W = fr.rv(N * K, -0.2, 0.2).reshape(N, K)
        b = fr.rv(N)
        fr.rv(seq * N)
        Wq, ws = vla.pack_weights_i8(W)
        assert sha(Wq) == str(g[f"wq_sha_{idx}"]) and np.array_equal(ws, g[f"ws_{idx}"])
        xq, sa = vla.quantize_act_i8(x)
        assert sha(xq) == str(g[f"xq_sha_{idx}"]) and np.array_equal(sa, g[f"sa_{idx}"])
        assert np.array_equal(vla.gemm_i8_i32(xq, Wq, K), g[f"acc_{idx}"])
        out = vla.dense_linear_i8(x, Wq, ws, b)
        assert out.tobytes() == g[f"out_ref_{idx}"].tobytes()


CFGS = [(1, 50, 8, 2, 64), (50, 50, 8, 2, 64), (50, 113, 15, 5, 64), (17, 33, 4, 4, 72),
        (9, 20, 2, 1, 256), (256, 256, 12, 12, 64), (12, 512, 4, 2, 64)]
LOWEST = np.finfo(np.float32).min


def test_attention_golden(vla, orc):
    g = golden("attention.npz")
    for idx, (sq, sk, nq, nkv, hd) in enumerate(CFGS):
        fr = orc.Frand()
        Q = fr.rv(sq * nq * hd).reshape(sq, nq * hd)
        K = fr.rv(sk * nkv * hd).reshape(sk, nkv * hd)
        V = fr.rv(sk * nkv * hd).reshape(sk, nkv * hd)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        rows = g[f"rows_{idx}"]
        assert max_rel(vla.gqa_attention_dense(Q, K, V, sq, sk, nq, nkv, hd, scale)[rows], g[f"dense_{idx}"]) <= 2e-5
        i, j = np.arange(sq)[:, None], np.arange(sk)[None, :]
        causal = np.where(j > i + (sk - sq), -np.inf, 0.0).astype(np.float32)
        got = vla.gqa_attention_masked(Q, K, V, sq, sk, nq, nkv, hd, scale, causal)
        assert max_rel(got[rows], g[f"causal_{idx}"]) <= 2e-5
        full = vla.gqa_attention_masked(Q, K, V, sq, sk, nq, nkv, hd, scale,
                                        np.full((sq, sk), LOWEST, np.float32))
        assert max_rel(full[rows], g[f"full_{idx}"]) <= 2e-5


def test_model_mask_attention_golden(vla):
    g = golden("attention.npz")
    masks = load_masks()
    synth = load_synth()
    qg, kg, al, T = masks.octo_block_causal(wnd=2, repeat_task=False)
    lang = np.ones(48, np.uint8)
    lang[40:] = 0
    pq, pk, pa, pad = masks.smolvla_prefix_lm(128, 48, lang)
    eq, ek, ea, SK = masks.smolvla_denoise(pad, 50)
    cases = [("octo658", T, T, 12, 12, (qg, kg, al)), ("smol_prefix", len(pad), len(pad), 15, 5, (pq, pk, pa)),
             ("smol_expert", 50, SK, 15, 5, (eq, ek, ea)), ("act_enc", 302, 302, 8, 8, None),
             ("act_cross", 100, 302, 8, 8, None)]
    for name, sq, sk, nq, nkv, grp in cases:
        Q = synth.normal(f"gold.{name}.q", (sq, nq * 64))
        K = synth.normal(f"gold.{name}.k", (sk, nkv * 64))
        V = synth.normal(f"gold.{name}.v", (sk, nkv * 64))
        if grp is None:
            o = vla.gqa_attention_dense(Q, K, V, sq, sk, nq, nkv, 64, 0.125)
        else:
            o = vla.attention(Q, K, V, nq, nkv, 64, 0.125, kind=vla.MASK_GROUPS, q_group=grp[0],
                              k_group=grp[1], allow=grp[2])
        assert max_rel(o[g[f"m_{name}_rows"]], g[f"m_{name}_out"]) <= 2e-5, name


def test_norms_eltwise_rope_golden(vla, orc):
    g = golden("norms.npz")
    for idx, (seq, H) in enumerate([(1, 768), (50, 960), (7, 6), (302, 512), (658, 768), (177, 960), (50, 720)]):
        fr = orc.Frand()
        x = fr.rv(seq * H, -3.0, 5.0).reshape(seq, H)
        w, b = fr.rv(H), fr.rv(H)
        rows = g[f"rows_{idx}"]
        assert np.max(np.abs(vla.layernorm(x, w, b, 1e-5)[rows] - g[f"ln_{idx}"])) <= 2e-6
        assert np.max(np.abs(vla.layernorm(x, w, None, 1e-6)[rows] - g[f"ln_nob_{idx}"])) <= 2e-6
        assert np.max(np.abs(vla.rmsnorm(x, w, 1e-6)[rows] - g[f"rms_{idx}"])) <= 2e-6
    e = golden("eltwise.npz")
    x = orc.Frand().rv(20011, -30.0, 30.0)
    u = orc.Frand(12345).rv(20011, -2.0, 2.0)
    assert max_rel(vla.gelu_tanh(x), e["gelu_tanh"]) <= 2e-6
    assert max_rel(vla.gelu_erf(x), e["gelu_erf"]) <= 2e-6
    assert np.array_equal(vla.relu(x), e["relu"])
    assert max_rel(vla.silu_gate(x, u), e["silu_gate"]) <= 2e-6
    r = golden("rope.npz")
    synth = load_synth()
    for idx, (seq, nh, hd) in enumerate(((177, 15, 64), (50, 5, 64), (7, 3, 16))):
        xx = synth.normal(f"rope.{seq}", (seq, nh * hd))
        got = vla.rope_neox(xx, np.arange(seq, dtype=np.int32) + 3, nh, hd, 10000.0)[r[f"rows_{idx}"]]
        assert np.max(np.abs(got - r[f"rope_{idx}"])) <= 2e-6 * max(1.0, float(np.max(np.abs(got))))
