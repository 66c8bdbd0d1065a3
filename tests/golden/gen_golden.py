#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ from the REAL reference kernels.

Runs in the container that holds the reference sources: oracle/_ref/libvla_ref.so
is the reference's own hot-path translation units (gemm_i8.cpp, avx2/gemm_i8.cpp,
avx2/attn.cpp, common/attn.cpp, norms.cpp, eltwise.cpp, env.cpp) built by
oracle/Makefile, driven through its C shim. Nothing here is imported from the
reference at run time and the fixtures are data only: inputs are regenerated
by the tests from the same seeded generators (the xorshift frand of
tests/test_ops.cpp:31-35, or vla.simd_amd/synth.py), and the fixtures hold
the reference's outputs (whole arrays when small; SHA-256 digests plus samples
for the BASELINE-sized ones).

Fixtures
  quant_edge.npz     quantize_act_i8 on test_ops.cpp:93-112's edge rows
  gemm_testops.npz   pack_weights_i8 / quantize_act_i8 / dense_linear_i8_ref /
                     the AVX-VNNI dense_linear_i8_pre at test_ops.cpp:138 shapes
  gemm_baseline.npz  BASELINE configs[0] and the configs[1] sweep: digests of
                     the synthetic inputs and of the reference's xq, ascale and
                     fp32 output (dense_linear_i8 through the VNNI kernel)
  attention.npz      gqa_attention_dense / _masked (causal, fully masked) at
                     test_ops.cpp:221-223 configs, and the BASELINE model masks
  norms.npz          layernorm / rmsnorm at test_ops.cpp:296-321 shapes + model shapes
  eltwise.npz        gelu_tanh / gelu_erf / silu_gate / relu over [-30, 30]
  rope.npz           rope_neox
  manifest.json      provenance (backend, VNNI availability, shapes)

Usage: python tests/golden/gen_golden.py
"""

from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))

from helpers import load_masks, load_synth, oracle, sha  # noqa: E402

ob = oracle()
synth = load_synth()
masks = load_masks()
LOWEST = np.finfo(np.float32).min

TESTOPS_GEMM = [(1, 16, 3), (7, 48, 64), (50, 768, 1027), (13, 64, 17), (257, 96, 48)]
ATTN_CFGS = [(1, 50, 8, 2, 64), (50, 50, 8, 2, 64), (50, 113, 15, 5, 64), (17, 33, 4, 4, 72),
             (9, 20, 2, 1, 256), (256, 256, 12, 12, 64), (12, 512, 4, 2, 64)]
NORM_SHAPES = [(1, 768), (50, 960), (7, 6), (302, 512), (658, 768), (177, 960), (50, 720)]


def sample_idx(n, k=2048):
    return np.unique(np.linspace(0, n - 1, min(n, k)).astype(np.int64))


def gen_quant(out):
    d = {}
    mags = [0.0, float(np.finfo(np.float32).smallest_subnormal), 1e-37, 1.0]
    i = 0
    for mag in mags:
        for width in (3, 16, 33):
            x = np.array([(1 if j % 2 == 0 else -1) * mag for j in range(width)], np.float32)[None]
            xq, s = ob.ref_quantize_act_i8(x)
            d[f"x_{i}"], d[f"xq_{i}"], d[f"s_{i}"] = x, xq, s
            i += 1
    d["count"] = np.array(i)
    np.savez_compressed(os.path.join(out, "quant_edge.npz"), **d)


def gen_gemm_testops(out, vnni):
    d = {}
    fr = ob.Frand()
    for idx, (seq, N, K) in enumerate(TESTOPS_GEMM):
        # test_ops.cpp:140-141 draw order (x, W, b), then the x86 branch's acc
        # draw (:166) which advances the stream once more per shape
        x = fr.rv(seq * K).reshape(seq, K)
        W = fr.rv(N * K, -0.2, 0.2).reshape(N, K)
        b = fr.rv(N)
        fr.rv(seq * N)
        rows, ws, blob = ob.ref_pack_weights(W)
        xq, sa = ob.ref_quantize_act_i8(x)
        yr = ob.ref_dense_linear_i8_ref(xq, sa, blob, ws, b, N, K)
        # int32 accumulators through the reference itself: unit scales and no
        # bias make the fp32 output (float)acc, exact while |acc| < 2^24
        # (K <= 1027 here: |acc| <= 1027 * 127 * 127 < 2^24)
        accf = ob.ref_dense_linear_i8_ref(xq, np.ones(seq, np.float32), blob, np.ones(N, np.float32),
                                          None, N, K)
        assert np.all(np.abs(accf) < 2 ** 24)
        d[f"wq_sha_{idx}"], d[f"ws_{idx}"] = np.array(sha(rows)), ws
        d[f"wq_head_{idx}"] = rows[:8]
        d[f"xq_sha_{idx}"], d[f"sa_{idx}"] = np.array(sha(xq)), sa
        d[f"xq_head_{idx}"] = xq[:8]
        d[f"out_ref_{idx}"] = yr
        d[f"acc_{idx}"] = accf.astype(np.int32)
        if vnni:
            yp = ob.ref_dense_linear_i8_pre(xq, sa, blob, ws, b, N, K)
            assert yp.tobytes() == yr.tobytes(), "reference VNNI kernel != its scalar reference"
            d[f"out_pre_{idx}"] = yp
    np.savez_compressed(os.path.join(out, "gemm_testops.npz"), **d)


def gen_gemm_baseline(out, vnni):
    shapes = [synth.CONFIG1] + [(M, K, N) for (K, N) in synth.SWEEP_KN for M in synth.SWEEP_M]
    d = {"shapes": np.array(shapes, np.int64)}
    t0 = time.time()
    for idx, (M, K, N) in enumerate(shapes):
        x, Wq, ws, b = synth.linear_case(M, K, N)
        blob = ob.ref_panels(Wq, K)
        xq = np.empty((M, (K + 3) & ~3), np.int8)
        sa = np.empty(M, np.float32)
        y = ob.ref_dense_linear_i8(x, blob, ws, b, N, K, xq, sa)
        d[f"in_sha_{idx}"] = np.array([sha(x), sha(Wq), sha(ws), sha(b)])
        d[f"xq_sha_{idx}"] = np.array(sha(xq))
        d[f"sa_sha_{idx}"] = np.array(sha(sa))
        d[f"out_sha_{idx}"] = np.array(sha(y))
        si = sample_idx(y.size)
        d[f"out_idx_{idx}"] = si
        d[f"out_val_{idx}"] = y.reshape(-1)[si]
        if idx == 0:  # configs[0] in full
            d["cfg1_xq"], d["cfg1_sa"], d["cfg1_out"] = xq, sa, y
        print(f"  gemm {M}x{K}x{N} ({time.time() - t0:.1f}s)", flush=True)
    d["kernel"] = np.array("avx-vnni dense_linear_i8_pre" if vnni else "scalar dense_linear_i8_ref")
    np.savez_compressed(os.path.join(out, "gemm_baseline.npz"), **d)


def _row_subset(sq, k=24):
    return np.arange(sq) if sq <= k else np.unique(np.linspace(0, sq - 1, k).astype(np.int64))


def gen_attention(out):
    d = {}
    for idx, (sq, sk, nq, nkv, hd) in enumerate(ATTN_CFGS):
        fr = ob.Frand()
        Q = fr.rv(sq * nq * hd).reshape(sq, nq * hd)
        K = fr.rv(sk * nkv * hd).reshape(sk, nkv * hd)
        V = fr.rv(sk * nkv * hd).reshape(sk, nkv * hd)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        rows = _row_subset(sq)
        dense = ob.ref_attention(Q, K, V, sq, sk, nq, nkv, hd, scale)
        i = np.arange(sq)[:, None]
        j = np.arange(sk)[None, :]
        causal = np.where(j > i + (sk - sq), -np.inf, 0.0).astype(np.float32)
        cz = ob.ref_attention(Q, K, V, sq, sk, nq, nkv, hd, scale, causal)
        full = ob.ref_attention(Q, K, V, sq, sk, nq, nkv, hd, scale, np.full((sq, sk), LOWEST, np.float32))
        d[f"rows_{idx}"] = rows
        d[f"dense_{idx}"], d[f"causal_{idx}"], d[f"full_{idx}"] = dense[rows], cz[rows], full[rows]
    # BASELINE model-shaped attention with the graphs' masks
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
        o = ob.ref_attention(Q, K, V, sq, sk, nq, nkv, 64, np.float32(0.125), m)
        rows = _row_subset(sq)
        d[f"m_{name}_rows"], d[f"m_{name}_out"] = rows, o[rows]
    np.savez_compressed(os.path.join(out, "attention.npz"), **d)


def gen_norms(out):
    d = {}
    for idx, (seq, H) in enumerate(NORM_SHAPES):
        fr = ob.Frand()
        x = fr.rv(seq * H, -3.0, 5.0).reshape(seq, H)
        w = fr.rv(H)
        b = fr.rv(H)
        rows = _row_subset(seq, 16)
        d[f"rows_{idx}"] = rows
        d[f"ln_{idx}"] = ob.ref_layernorm(x, w, b, 1e-5)[rows]
        d[f"ln_nob_{idx}"] = ob.ref_layernorm(x, w, None, 1e-6)[rows]
        d[f"rms_{idx}"] = ob.ref_rmsnorm(x, w, 1e-6)[rows]
    np.savez_compressed(os.path.join(out, "norms.npz"), **d)


def gen_eltwise(out):
    x = ob.Frand().rv(20011, -30.0, 30.0)
    u = ob.Frand(12345).rv(20011, -2.0, 2.0)
    np.savez_compressed(os.path.join(out, "eltwise.npz"),
                        gelu_tanh=ob.ref_eltwise("ref_gelu_tanh", x),
                        gelu_erf=ob.ref_eltwise("ref_gelu_erf", x),
                        relu=ob.ref_eltwise("ref_relu", x),
                        silu_gate=ob.ref_silu_gate(x, u))


def gen_rope(out):
    d = {}
    for idx, (seq, nh, hd) in enumerate(((177, 15, 64), (50, 5, 64), (7, 3, 16))):
        x = synth.normal(f"rope.{seq}", (seq, nh * hd))
        pos = np.arange(seq, dtype=np.int32) + 3
        rows = _row_subset(seq, 16)
        d[f"rows_{idx}"] = rows
        d[f"rope_{idx}"] = ob.ref_rope_neox(x, pos, nh, hd, 10000.0)[rows]
    np.savez_compressed(os.path.join(out, "rope.npz"), **d)


def main():
    if not ob.ref_available():
        sys.exit("oracle/_ref/libvla_ref.so is not built (make -C oracle ref)")
    L = ob.ref()
    vnni = bool(L.ref_int8_available())
    print(f"reference backend {L.ref_backend_name().decode()}, AVX-VNNI {vnni}, "
          f"{L.ref_omp_max_threads()} OpenMP threads", flush=True)
    gen_quant(HERE)
    gen_gemm_testops(HERE, vnni)
    gen_gemm_baseline(HERE, vnni)
    gen_attention(HERE)
    gen_norms(HERE)
    gen_eltwise(HERE)
    gen_rope(HERE)
    json.dump({
        "generator": "tests/golden/gen_golden.py",
        "reference_build": "oracle/Makefile (reference hot-path TUs, -O3 -mavx2 -mfma -mf16c -ffp-contract=fast -fopenmp)",
        "backend": L.ref_backend_name().decode(),
        "avx_vnni": vnni,
        "frand_state": "0x243F6A8885A308D3 (tests/test_ops.cpp:31)",
        "synth_seed": synth.BASE_SEED,
    }, open(os.path.join(HERE, "manifest.json"), "w"), indent=1)
    print("golden vectors written", flush=True)


if __name__ == "__main__":
    main()
