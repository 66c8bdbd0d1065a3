#!/usr/bin/env python3
"""Benchmark of the MI355X int8 linear path on BASELINE.json's int8 GEMM sweep.

Workload: M in {1, 50, 100, 512, 2048, 8192} x
(K, N) in {(512,3200), (960,2560), (2560,960), (768,3072), (4096,4096)}, the
reference op path dense_linear_i8: fp32 activations ~N(0,1) quantized per row
on the device, int8 weights uniform in [-127,127] with per-channel scales
~U(1e-3,1e-2) and bias ~N(0,0.02), int32 accumulate, fp32 out. One step is one
pass over all 30 shapes (a quantize launch + a GEMM launch each, one launch
for the few-row shapes below), inputs and
weights resident in HBM; small shapes cycle through rotating copies of their
weights and outputs (>= 512 MiB per shape) so every launch streams from HBM
rather than from L2/MALL. For M <= 128 the quantize writes the library's
panel layout (vla_quantize_act_i8_panel_dev) and the GEMM reads it
(vla_dense_linear_i8_panel_dev): the same values, byte-identical output. For
M <= 16 with K <= 2048 the op is the library's op entry itself
(vla_dense_linear_i8_dev with caller-owned scratch), which quantizes inside
the GEMM: one launch, the same scratch bytes and output.
Each sweep row also carries the warm time (gemm_warm_us: the same launches
on one weight and output copy, operands resident in L2 / MALL) beside the
cold, rotating one (gemm_us), which is what frac and value use.

value = int8 TOPS of the whole step (sum of 2*M*N*K over the shapes / step
time). gemm_us is the GEMM launch alone (on the quantized rows), op_us the
whole op. roofline = the dominant kernel (the M=8192, K=N=4096 GEMM) measured
with HIP events on the stream it runs on. cpu_baseline = the reference's own
dense_linear_i8 (its AVX-VNNI kernel when the host CPU has AVX-VNNI, else its
scalar dense_linear_i8_ref) built from the reference sources into
oracle/_ref/, timed on this host on a bounded sample of the same shapes.

policy_latency_ms = the metric's second half, per-chunk latency at batch 1 of
BASELINE.json configs[2..4] (ACT transformer, Octo-base transformer, SmolVLA
chunk) on random-init checkpoints written in the reference's file layouts:
the device graph (one HIP-graph replay per forward, inputs resident in HBM,
HIP events) next to the reference's own graph on this host's cores.

conv_resnet18_480x640 = conv2d_i8 over ResNet-18's convolutions at 480 x 640
(ACT's backbone), per distinct layer: device time per call, its roofline
fraction, and the reference's conv2d_i8 on this host. Long-K GEMMs of a few
hundred rows in the sweep run with a split-K workspace (dense_linear_i8 takes
caller-owned scratch in the reference too); the values do not change.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# The CPUs this process may run on, read before any OpenMP runtime binds the
# main thread to one place (sched_getaffinity of a bound thread returns 1).
try:
    ALLOWED_CPUS = len(os.sched_getaffinity(0))
except (AttributeError, OSError):
    ALLOWED_CPUS = None

# The CPU legs follow the baseline protocol: OpenMP threads bound close, one
# per core (set before any OpenMP runtime in this process starts; a value the
# caller exported wins), 5 warm-up calls, then the median of >= 50 timed ones.
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")
CPU_WARMUP, CPU_TIMED = 5, 50

PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA (POP/s x 1000)
PEAK_HBM_GBS = 8000.0    # MI355X HBM3E
ROTATE_BYTES = 512 << 20


def load_pkg():
    import importlib.util

    d = os.path.join(ROOT, "vla.simd_amd")
    spec = importlib.util.spec_from_file_location("vla_simd_amd", os.path.join(d, "__init__.py"),
                                                  submodule_search_locations=[d])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["vla_simd_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def gemm_bytes(M, K, N):
    """Algorithmic HBM bytes of the GEMM kernel: int8 x and W in, scales and bias, fp32 out."""
    Kp = (K + 3) & ~3
    return M * Kp + N * Kp + 4 * M + 8 * N + 4 * M * N


def op_bytes(M, K, N):
    """The whole op from fp32 x (quantize reads 4*M*K and writes M*Kp + 4*M)."""
    Kp = (K + 3) & ~3
    return gemm_bytes(M, K, N) + 4 * M * K + M * Kp + 4 * M


def roof_us(M, K, N):
    ops = 2.0 * M * N * K
    t_mfma = ops / (PEAK_INT8_TOPS * 1e12) * 1e6
    t_hbm = gemm_bytes(M, K, N) / (PEAK_HBM_GBS * 1e9) * 1e6
    return max(t_mfma, t_hbm), ("mfma" if t_mfma >= t_hbm else "hbm")


class Shape:
    def __init__(self, vla, torch, synth, M, K, N):
        self.M, self.K, self.N = M, K, N
        dev = torch.device("cuda")
        x, Wq, ws, b = synth.linear_case(M, K, N)
        self.ldw = (((K + 3) & ~3) + 63) // 64 * 64
        per = self.ldw * N + 4 * M * N
        self.R = max(1, min(256, math.ceil(ROTATE_BYTES / per))) if per < ROTATE_BYTES else 1
        Wp = np.zeros((N, self.ldw), np.int8)
        Wp[:, :K] = Wq
        Wd = torch.from_numpy(Wp).to(dev)
        self.W = [Wd] + [Wd.clone() for _ in range(self.R - 1)]
        self.out = [torch.empty((M, N), dtype=torch.float32, device=dev) for _ in range(self.R)]
        self.x = torch.from_numpy(x).to(dev)
        # M <= 128: the library's panel layout for the quantized rows (the
        # skinny GEMM then reads each 16-row fragment as 1 KiB of contiguous
        # memory); the same quantize + GEMM arithmetic, bit-identical output
        self.panel = M <= 128
        if self.panel:
            self.xq = torch.zeros((vla.i8_panel_bytes(M, K),), dtype=torch.int8, device=dev)
        else:
            self.xq = torch.zeros((M, self.ldw), dtype=torch.int8, device=dev)
        self.sa = torch.empty(M, dtype=torch.float32, device=dev)
        self.ws = torch.from_numpy(ws).to(dev)
        self.b = torch.from_numpy(b).to(dev)
        # at most 16 rows the library's op entry (vla_dense_linear_i8_dev, the
        # reference's dense_linear_i8 with caller-owned scratch) quantizes inside
        # the GEMM: one launch per op, the same bytes in the scratch and out
        self.fused = M <= 16 and vla.rowop_linear_i8_fits(0, M, K)
        if self.fused:
            self.xq_op = torch.zeros((M, self.ldw), dtype=torch.int8, device=dev)
        # split-K workspace for long-K shapes whose tiles leave CUs idle (the
        # same values as the unsplit GEMM; the op API's caller-owned scratch)
        nsplit = 0 if self.panel else vla.gemm_i8_split_bytes(M, N, K)
        self.split = torch.empty(nsplit, dtype=torch.uint8, device=dev) if nsplit > 0 else None
        self.i = 0

    def quantize(self, vla, stream):
        if self.panel:
            vla.quantize_act_i8_panel_dev(self.x, self.xq, self.sa, stream)
        else:
            vla.quantize_act_i8_dev(self.x, self.xq, self.sa, stream)

    def gemm(self, vla, stream):
        r = self.i % self.R
        self.i += 1
        if self.panel:
            vla.dense_linear_i8_panel_dev(self.out[r], self.xq, self.sa, self.W[r], self.ws, self.b, self.K,
                                          stream=stream)
        elif self.split is not None:
            vla.dense_linear_i8_pre_split_dev(self.out[r], self.xq, self.sa, self.W[r], self.ws, self.b, self.K,
                                              self.split, stream=stream)
        else:
            vla.dense_linear_i8_pre_dev(self.out[r], self.xq, self.sa, self.W[r], self.ws, self.b, self.K,
                                        stream=stream)

    def gemm_warm(self, vla, stream):
        # the same weights and output every launch: operands warm in L2/MALL
        r, self.i = self.i, 0
        self.gemm(vla, stream)
        self.i = r

    def op(self, vla, stream):
        if self.fused:
            r = self.i % self.R
            self.i += 1
            vla.dense_linear_i8_dev(self.out[r], self.x, self.W[r], self.ws, self.b, self.K, self.xq_op, self.sa,
                                    stream=stream)
            return
        self.quantize(vla, stream)
        self.gemm(vla, stream)


def cur(torch):
    return torch.cuda.current_stream().cuda_stream


def capture(torch, fn, n):
    """A HIP graph of n calls of fn(stream) (torch.cuda.graph capture; the library's
    launches go to the capturing stream, so the graph holds exactly those kernels)."""
    fn(cur(torch))  # eager warm-up: grows any workspace outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n):
            fn(cur(torch))
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, replays, stream_obj):
    """Average us per replay, HIP events on the stream the replays run on."""
    g.replay()
    stream_obj.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream_obj)
    for _ in range(replays):
        g.replay()
    end.record(stream_obj)
    end.synchronize()
    return start.elapsed_time(end) * 1e3 / replays


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemm_i8_8192x4096x4096_traffic.txt")


def profiled_traffic():
    """HBM bytes per launch of the dominant GEMM, from the two rocprofv3 --pmc
    passes (FETCH_SIZE, WRITE_SIZE, calibrated) summarised in TRAFFIC_PROFILE."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def host_cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo, what lscpu prints as Model name)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_cores() -> dict:
    """The host's CPUs: logical CPUs, physical cores (distinct (package,
    core id) pairs of /proc/cpuinfo) and the CPUs this process may run on (the
    lease's share on a shared box, read at start-up)."""
    phys = set()
    pkg = core = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("physical id"):
                pkg = line.split(":", 1)[1].strip()
            elif line.startswith("core id"):
                core = line.split(":", 1)[1].strip()
            elif not line.strip():
                if core is not None:
                    phys.add((pkg, core))
                pkg = core = None
        if core is not None:
            phys.add((pkg, core))
    except OSError:
        pass
    return {"logical_cpus": os.cpu_count(), "physical_cores": len(phys) or None, "allowed_cpus": ALLOWED_CPUS}


def _median_ms(fn, warmup=CPU_WARMUP, timed=CPU_TIMED):
    """Median wall time in ms of `timed` calls of fn() after `warmup` calls."""
    for _ in range(warmup):
        fn()
    t = []
    for _ in range(timed):
        t0 = time.perf_counter()
        fn()
        t.append((time.perf_counter() - t0) * 1e3)
    return float(np.median(t))


def cpu_baseline(synth):
    """The reference's dense_linear_i8 on this host (oracle/_ref build): per
    shape the median of 50 calls after 5 warm-ups; value = sum of the shapes'
    ops / sum of their median times."""
    from oracle import bindings as ob

    if not ob.ref_available():
        return None
    L = ob.ref()
    sample = [(100, 512, 3200), (50, 960, 2560), (100, 2560, 960), (100, 768, 3072),
              (100, 4096, 4096), (512, 512, 3200), (512, 960, 2560), (512, 2560, 960),
              (512, 768, 3072), (512, 4096, 4096)]
    tot_ops, tot_ms, per = 0.0, 0.0, {}
    for M, K, N in sample:
        x, Wq, ws, b = synth.linear_case(M, K, N)
        blob = ob.ref_panels(Wq, K)
        xq = np.empty((M, (K + 3) & ~3), np.int8)
        sa = np.empty(M, np.float32)
        ms = _median_ms(lambda: ob.ref_dense_linear_i8(x, blob, ws, b, N, K, xq, sa))
        tot_ops += 2.0 * M * N * K
        tot_ms += ms
        per[f"{M}x{K}x{N}"] = round(ms, 4)
    vnni = bool(L.ref_int8_available())
    hc = host_cores()
    threads = int(L.ref_omp_max_threads())
    return {
        "value": round(tot_ops / (tot_ms * 1e-3) / 1e12, 4),
        "unit": "TOPS (int8, 2*M*N*K per dense_linear_i8 call)",
        "cores": threads,
        "host_cores": hc,
        "cores_note": (f"{threads} OpenMP threads: the host's {hc['physical_cores']} physical cores"
                       if threads == hc["physical_cores"] else
                       f"{threads} OpenMP threads = the CPUs this process may use ({hc['allowed_cpus']} allowed of "
                       f"{hc['logical_cpus']} logical, {hc['physical_cores']} physical cores; a shared box's lease "
                       f"limit, OMP_NUM_THREADS as the box sets it)"),
        "kind": "reference",
        "sample": f"reference dense_linear_i8 ({'AVX-VNNI' if vnni else 'scalar ref, no AVX-VNNI'}), "
                  f"{len(sample)} configs[1] shapes M<=512",
        "host_cpu": host_cpu_model(),
        "omp": {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OMP_PROC_BIND", "OMP_PLACES")},
        "protocol": f"{CPU_WARMUP} warm-up + median of {CPU_TIMED} calls per shape; sum ops / sum medians",
        "median_ms_per_shape": per,
    }


def _time_calls(torch, fn, stream_obj, min_calls=20, min_s=0.5):
    """ms per call of fn() (each call one replay of a captured policy graph),
    HIP events on the stream the graphs run on."""
    for _ in range(3):  # eager call, capture, first replay
        fn()
    stream_obj.synchronize()
    n, t = 0, 0.0
    while n < min_calls or t < min_s * 1e3:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream_obj)
        for _ in range(10):
            fn()
        end.record(stream_obj)
        end.synchronize()
        t += start.elapsed_time(end)
        n += 10
    return t / n


def _time_cpu(fn):
    """ms per call of a reference CPU leg: the baseline protocol's median of 50
    after 5 warm-ups."""
    return _median_ms(fn)


def _lat_act(vla, torch, ck, ob, tmp, stream_obj):
    """ACT: 4 x 302-token encoder, 100-query decoder, ACT_INT8=31."""
    dev, st = torch.device("cuda"), stream_obj.cuda_stream
    c = ck.ACT_BASE
    d = ck.write_act(os.path.join(tmp, "act"), c)
    f, s = ck.act_inputs(c)
    m = vla.ActTransformer(d, c["img_ch"], 31)
    tf, ts = torch.from_numpy(f).to(dev), torch.from_numpy(s).to(dev)
    ta = torch.empty((c["chunk"], c["action_dim"]), dtype=torch.float32, device=dev)
    gpu = _time_calls(torch, lambda: m.forward_dev(tf, 1, c["fh"], c["fw"], ts, ta, st), stream_obj)
    row = {"gpu_ms": round(gpu, 4), "tokens": m_tokens_act(c), "int8_mask": 31,
           "int8_layers": m.int8_layers, "graph_nodes": m.graph_nodes}
    if ob is not None:
        r = ob.RefAct(d, c["img_ch"], 31, c["chunk"], c["action_dim"])
        row["cpu_ref_ms"] = round(_time_cpu(lambda: r.forward(f, 1, c["fh"], c["fw"], s)), 3)
    return row


def _lat_act_model(vla, torch, ck, ob, tmp, stream_obj, act_int8):
    """ACT end to end (vla_act_predict_dev): one 480 x 640 uint8 camera ->
    normalization -> ResNet-18 -> the ACT_BASE transformer -> un-normalized
    actions; ACT_INT8 as given (31: transformer int8, 63: backbone too)."""
    dev, st = torch.device("cuda"), stream_obj.cuda_stream
    c = ck.ACT_MODEL_BASE
    d = os.path.join(tmp, "act_model")
    if not os.path.exists(os.path.join(d, "stats.bin")):
        ck.write_act_model(d, c)
    images, state = ck.act_model_inputs(c)
    saved = os.environ.get("ACT_INT8")
    os.environ["ACT_INT8"] = str(act_int8)
    try:
        m = vla.ActModel(d)
        r = ob.RefActModel(d) if ob is not None else None
    finally:
        if saved is None:
            os.environ.pop("ACT_INT8", None)
        else:
            os.environ["ACT_INT8"] = saved
    ti, ts = torch.from_numpy(images).to(dev), torch.from_numpy(state).to(dev)
    ta = torch.empty((c["chunk"], c["action_dim"]), dtype=torch.float32, device=dev)
    gpu = _time_calls(torch, lambda: m.predict_dev(ti, ts, ta, True, st), stream_obj)
    row = {"gpu_ms": round(gpu, 4), "image": f"{c['n_cams']}x{c['img_h']}x{c['img_w']}", "act_int8": act_int8,
           "int8_convs": m.int8_convs, "int8_layers": m.int8_layers, "graph_nodes": m.graph_nodes}
    # the backbone alone (vla_act_encode_dev: normalization + ResNet-18, one
    # graph replay per call)
    tf = torch.empty((m.n_cams * m.feat_h * m.feat_w, m.feat_ch), dtype=torch.float32, device=dev)
    row["backbone_gpu_ms"] = round(_time_calls(torch, lambda: m.encode_dev(ti, tf, st), stream_obj), 4)
    if r is not None:
        row["cpu_ref_ms"] = round(_time_cpu(lambda: r.predict(images, state)), 3)
        row["backbone_cpu_ref_ms"] = round(_time_cpu(lambda: r.encode(images)), 3)
    return row


def _lat_octo(vla, torch, ck, ob, tmp, stream_obj, repeat_task):
    """Octo-base: 12 x 768; repeat_task 0 is BASELINE's 658-token layout, 1 the
    reference's 690-token layout (the only one the reference runs)."""
    dev, st = torch.device("cuda"), stream_obj.cuda_stream
    c = dict(ck.OCTO_BASE, repeat_task=repeat_task)
    d = ck.write_octo(os.path.join(tmp, f"octo{repeat_task}"), c)
    t5, sp, sw, tm = ck.octo_inputs(c)
    m = vla.OctoTransformer(d, 7)
    a, b, w = (torch.from_numpy(v).to(dev) for v in (t5, sp, sw))
    o = torch.empty(c["d"], dtype=torch.float32, device=dev)
    gpu = _time_calls(torch, lambda: m.forward_dev(a, b, w, 2, tm, o, st), stream_obj)
    row = {"gpu_ms": round(gpu, 4), "tokens": m.total_tokens(2), "int8_mask": 7,
           "int8_layers": m.int8_layers, "graph_nodes": m.graph_nodes}
    if ob is not None and repeat_task:
        r = ob.RefOcto(d, 7, c["d"])
        row["cpu_ref_ms"] = round(_time_cpu(lambda: r.forward(t5, sp, sw, 2, tm)), 3)
    return row


def _lat_smolvla(vla, torch, ck, ob, tmp, stream_obj):
    """SmolVLA chunk: 16-layer prefix over 177 tokens + 10 Euler steps of the
    16-layer expert, SMOLVLA_INT8=48."""
    dev, st = torch.device("cuda"), stream_obj.cuda_stream
    c = ck.SMOLVLA_BASE
    d = ck.write_smolvla(os.path.join(tmp, "smol"), c)
    p, pad, n = ck.smolvla_inputs(c)
    m = vla.SmolvlaChunk(d, 48)
    tp, tn = torch.from_numpy(p).to(dev), torch.from_numpy(n).to(dev)
    ta = torch.empty((c["chunk"], c["max_action_dim"]), dtype=torch.float32, device=dev)
    gpu = _time_calls(torch, lambda: m.run_dev(tp, pad, tn, ta, st), stream_obj, min_calls=10)
    row = {"gpu_ms": round(gpu, 4), "prefix_tokens": c["n_prefix"], "steps": c["num_steps"],
           "int8_mask": 48, "int8_layers": m.int8_layers, "graph_nodes": m.graph_nodes}
    if ob is not None:
        r = ob.RefSmolvla(d, 48)
        row["cpu_ref_ms"] = round(_time_cpu(lambda: r.run(p, pad, n)), 3)
    return row


def _lat_siglip(vla, torch, ck, ob, tmp, stream_obj):
    """SmolVLA's SigLIP vision tower + connector per camera image: 12 x 768
    layers over 1024 patches (512 x 512), pixel shuffle to 64 tokens, the
    vision int8 bits 1|2|4|8 (SMOLVLA_INT8=15)."""
    dev, st = torch.device("cuda"), stream_obj.cuda_stream
    c = ck.SIGLIP_BASE
    d = ck.write_siglip(os.path.join(tmp, "vit"), c)
    px = ck.siglip_inputs(c)
    m = vla.SiglipVision(d, 15)
    tp = torch.from_numpy(px).to(dev)
    to = torch.empty((c["n_img_tok"], c["mm_out"]), dtype=torch.float32, device=dev)
    gpu = _time_calls(torch, lambda: m.encode_dev(tp, to, st), stream_obj)
    row = {"gpu_ms": round(gpu, 4), "patches": c["n_patches"], "int8_mask": 15,
           "int8_layers": m.int8_layers, "graph_nodes": m.graph_nodes}
    if ob is not None:
        r = ob.RefSiglip(d, 15, c["n_img_tok"], c["mm_out"])
        row["cpu_ref_ms"] = round(_time_cpu(lambda: r.encode(px)), 3)
    return row


def _lat_smolvla_model(vla, torch, ck, ob, tmp, stream_obj):
    """SmolVLA end to end through vla_smolvla_predict (host pointers, the
    caller's view): two 480 x 640 uint8 frames uploaded, resized to 512 x 512,
    SigLIP per view, a 48-token instruction, the state token, the 16-layer
    prefix tower and 10 Euler steps of the expert, actions downloaded;
    SMOLVLA_INT8=63. Wall-clock median of host calls (PCIe included)."""
    c = ck.SMOLVLA_MODEL_BASE
    d = os.path.join(tmp, "smol_model")
    if not os.path.exists(os.path.join(d, "heads.bin")):
        ck.write_smolvla_model(d, c)
    frames, state, noise = ck.smolvla_model_inputs(c)
    saved = os.environ.pop("SMOLVLA_INT8", None)
    try:
        r = ob.RefSmolvlaModel(d, int8_mask=63) if ob is not None else None  # the reference's latch stays 0
        os.environ["SMOLVLA_INT8"] = "63"
        m = vla.SmolvlaModel(d)
    finally:
        os.environ.pop("SMOLVLA_INT8", None)
        if saved is not None:
            os.environ["SMOLVLA_INT8"] = saved
    ids, lmask, _ = m.tokenize("pick up the red block and put it in the box, then " * 6)
    gpu = _median_ms(lambda: m.predict(frames, ids, lmask, state, noise=noise), warmup=3, timed=20)
    row = {"host_call_ms": round(gpu, 4), "frames": "2x480x640", "prefix_tokens": 2 * 64 + 48 + 1,
           "steps": c["tf"]["num_steps"], "smolvla_int8": 63, "int8_layers": m.int8_layers,
           "graph_nodes": m.graph_nodes}
    if r is not None:
        row["cpu_ref_ms"] = round(_median_ms(lambda: r.predict(frames, ids, lmask, state, m.chunk, m.action_dim,
                                                               noise=noise), warmup=2, timed=10), 3)
    return row


def _lat_octo_model(vla, torch, ck, ob, tmp, stream_obj):
    """Octo end to end through vla_octo_predict_ex (host pointers, the caller's
    view): two timesteps of 256 x 256 primary and 128 x 128 wrist uint8 frames
    (new frames every call: no stem reuse), the cached T5-base embedding of the
    instruction, the 12 x 768 transformer (690 tokens), the 20-step DDPM head;
    OCTO_INT8=63. Wall-clock median of host calls (PCIe included)."""
    c = ck.OCTO_MODEL_BASE
    d = os.path.join(tmp, "octo_model")
    if not os.path.exists(os.path.join(d, "head.bin")):
        ck.write_octo_model(d, c)
    frames = [ck.octo_model_inputs(c, seed=s) for s in (1, 2)]
    saved = os.environ.pop("OCTO_INT8", None)
    try:
        r = ob.RefOctoModel(d, int8_mask=63) if ob is not None else None  # the reference's latch stays 0
        os.environ["OCTO_INT8"] = "63"
        m = vla.OctoModel(d)
    finally:
        os.environ.pop("OCTO_INT8", None)
        if saved is not None:
            os.environ["OCTO_INT8"] = saved
    text = "pick up the red block"
    k = [0]

    def call():  # alternate two windows so every call runs the stems
        p, w, tm, n, z = frames[k[0] % 2]
        k[0] += 1
        return m.predict(p, w, tm, text, noise=n, z=z)
    gpu = _median_ms(call, warmup=3, timed=20)
    row = {"host_call_ms": round(gpu, 4), "frames": "2x(256x256 + 128x128)", "tokens": 690,
           "ddpm_steps": c["head"]["steps"], "octo_int8": 63, "int8_layers": m.int8_layers}
    if r is not None:
        p, w, tm, n, z = frames[0]
        row["cpu_ref_ms"] = round(_median_ms(lambda: r.predict(p, w, tm, text, noise=n, z=z), warmup=2, timed=10), 3)
    return row


def _lat_impact_model(vla, torch, ck, ob, tmp, stream_obj):
    """IMPACT end to end through vla_impact_predict (host pointers): one
    480 x 640 uint8 camera, the ACT_BASE-shaped transformer with its text
    tail, FiLM in the trunk; the instruction is encoded once and cached, as
    in a rollout; IMPACT_INT8=63. Wall-clock median of host calls."""
    c = ck.IMPACT_MODEL_BASE
    d = os.path.join(tmp, "impact_model")
    ck.write_impact_model(d, c)
    images, state = ck.act_model_inputs(c)
    saved = os.environ.get("IMPACT_INT8")
    os.environ["IMPACT_INT8"] = "63"
    try:
        m = vla.ImpactModel(d)
        r = ob.RefImpactModel(d) if ob is not None else None
    finally:
        if saved is None:
            os.environ.pop("IMPACT_INT8", None)
        else:
            os.environ["IMPACT_INT8"] = saved
    text = "pick up the red block"
    gpu = _median_ms(lambda: m.predict(images, state, text), warmup=3, timed=20)
    row = {"host_call_ms": round(gpu, 4), "image": f"{c['n_cams']}x{c['img_h']}x{c['img_w']}", "impact_int8": 63,
           "int8_layers": m.int8_layers, "int8_convs": m.int8_convs}
    if r is not None:
        row["cpu_ref_ms"] = round(_median_ms(lambda: r.predict(images, state, text), warmup=2, timed=10), 3)
    return row


def _lat_diffusion_model(vla, torch, ck, ob, tmp, stream_obj, mask, sched, steps):
    """Diffusion Policy end to end through vla_diffusion_predict (host
    pointers): lerobot's pusht-shaped policy (two 96 x 96 cameras cropped to
    84 x 84, GroupNorm ResNet-18 encoders, the 512/1024/2048 UNet over a
    16-step horizon) in a rollout's steady state (each query brings one new
    frame per camera, the older step's features come from the frame cache),
    DIFFUSION_INT8 = mask, the given sampler. Wall-clock median of host calls."""
    c = ck.DP_MODEL_BASE
    d = os.path.join(tmp, "diffusion_model")
    if not os.path.exists(os.path.join(d, "stats.bin")):
        ck.write_diffusion_model(d, c)
    pool, state, noise = ck.diffusion_model_inputs(dict(c, n_obs_steps=8))
    noise = noise[:1 + steps]
    saved = {k: os.environ.get(k) for k in ("DIFFUSION_INT8", "DP_SCHEDULER", "DP_STEPS")}
    os.environ.update(DIFFUSION_INT8=str(mask), DP_SCHEDULER=sched, DP_STEPS=str(steps))
    try:
        m = vla.DiffusionModel(d)
        r = ob.RefDiffusionModel(d) if ob is not None else None
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    n = c["n_obs_steps"]

    def roll(model):
        k = [0]

        def call():
            i = k[0] % (len(pool) - n + 1)
            k[0] += 1
            return model.predict(np.ascontiguousarray(pool[i:i + n]), state[i:i + n], noise)
        return call
    gpu = _median_ms(roll(m), warmup=3, timed=10 if steps > 20 else 20)
    row = {"host_call_ms": round(gpu, 4), "sampler": f"{sched}{steps}", "diffusion_int8": mask,
           "images": f"{n}x{c['n_cams']}x{c['img_h']}x{c['img_w']} (crop {c['crop_h']}x{c['crop_w']})",
           "int8_layers": m.int8_layers, "int8_convs": m.int8_convs, "graph_nodes": m.graph_nodes}
    if r is not None:
        row["cpu_ref_ms"] = round(_median_ms(roll(r), warmup=1, timed=3 if steps > 20 else 10), 3)
    return row


def policy_latency(vla, torch, stream_obj, with_cpu=True,
                   models=("act", "act_model", "octo", "smolvla", "siglip", "smolvla_model", "octo_model",
                           "impact_model", "diffusion_model")):
    """Per-chunk latency of BASELINE.json configs[2..4] at batch 1, and of
    SmolVLA's SigLIP vision tower per camera image: the device
    graphs (one captured HIP graph per forward, inputs resident in HBM) and the
    reference's own graphs (oracle/_ref) on this host, on the same random-init
    checkpoints and inputs."""
    import tempfile

    import vla_simd_amd.checkpoints as ck

    ob = None
    if with_cpu:
        from oracle import bindings as ob
        if not ob.ref_available():
            ob = None
    out = {}
    with tempfile.TemporaryDirectory(prefix="vla_ck_") as tmp:
        if "act" in models:
            out["act"] = _lat_act(vla, torch, ck, ob, tmp, stream_obj)
            print(f"  ACT transformer: {out['act']}", file=sys.stderr, flush=True)
        if "act_model" in models:
            for mask in (31, 63):
                out[f"act_model_int8_{mask}"] = _lat_act_model(vla, torch, ck, ob, tmp, stream_obj, mask)
                print(f"  ACT end to end (ACT_INT8={mask}): {out[f'act_model_int8_{mask}']}", file=sys.stderr,
                      flush=True)
        if "octo" in models:
            out["octo"] = _lat_octo(vla, torch, ck, ob, tmp, stream_obj, 0)
            print(f"  Octo transformer (658 tokens): {out['octo']}", file=sys.stderr, flush=True)
            out["octo_repeat_task"] = _lat_octo(vla, torch, ck, ob, tmp, stream_obj, 1)
            print(f"  Octo transformer (690 tokens): {out['octo_repeat_task']}", file=sys.stderr,
                  flush=True)
        if "smolvla" in models:
            out["smolvla"] = _lat_smolvla(vla, torch, ck, ob, tmp, stream_obj)
            print(f"  SmolVLA chunk: {out['smolvla']}", file=sys.stderr, flush=True)
        if "siglip" in models:
            out["siglip"] = _lat_siglip(vla, torch, ck, ob, tmp, stream_obj)
            print(f"  SigLIP vision tower: {out['siglip']}", file=sys.stderr, flush=True)
        if "smolvla_model" in models:
            out["smolvla_model"] = _lat_smolvla_model(vla, torch, ck, ob, tmp, stream_obj)
            print(f"  SmolVLA end to end: {out['smolvla_model']}", file=sys.stderr, flush=True)
        if "octo_model" in models:
            out["octo_model"] = _lat_octo_model(vla, torch, ck, ob, tmp, stream_obj)
            print(f"  Octo end to end: {out['octo_model']}", file=sys.stderr, flush=True)
        if "impact_model" in models:
            out["impact_model"] = _lat_impact_model(vla, torch, ck, ob, tmp, stream_obj)
            print(f"  IMPACT end to end: {out['impact_model']}", file=sys.stderr, flush=True)
        if "diffusion_model" in models:
            for mask, sched, steps in ((3, "DDPM", 100), (0, "DDPM", 100), (3, "DDIM", 10), (0, "DDIM", 10)):
                key = f"diffusion_{sched.lower()}{steps}_int8_{mask}"
                out[key] = _lat_diffusion_model(vla, torch, ck, ob, tmp, stream_obj, mask, sched, steps)
                print(f"  Diffusion Policy end to end ({sched} {steps}, DIFFUSION_INT8={mask}): {out[key]}",
                      file=sys.stderr, flush=True)
    if ob is not None:
        out["cpu_ref_threads"] = int(ob.ref().ref_omp_max_threads())
    return out


# ResNet-18 at 480 x 640 (ACT's backbone; src/models/act): (H, W, Cin, Cout, k, stride, pad, count)
RESNET18_480x640 = [(480, 640, 3, 64, 7, 2, 3, 1), (120, 160, 64, 64, 3, 1, 1, 4),
                    (120, 160, 64, 128, 3, 2, 1, 1), (60, 80, 128, 128, 3, 1, 1, 3),
                    (120, 160, 64, 128, 1, 2, 0, 1), (60, 80, 128, 256, 3, 2, 1, 1),
                    (30, 40, 256, 256, 3, 1, 1, 3), (60, 80, 128, 256, 1, 2, 0, 1),
                    (30, 40, 256, 512, 3, 2, 1, 1), (15, 20, 512, 512, 3, 1, 1, 3),
                    (30, 40, 256, 512, 1, 2, 0, 1)]


def conv_resnet18(vla, torch, stream_obj, with_cpu=True):
    """conv2d_i8 (section f.3 of the hot path) over ResNet-18's 20 convolutions at
    480 x 640: per distinct layer the device time per call (vla_conv2d_i8_dev,
    20 calls captured as a HIP graph, HIP events on the replay stream, inputs
    resident in HBM), its roofline
    (max(2*npix*Cout*K / int8 peak, algorithmic bytes / HBM peak) with bytes =
    4 H W Cin + Cout K + 8 Cout + 4 npix Cout), and the reference's conv2d_i8 on
    this host (oracle/_ref, weights packed once)."""
    ob = None
    if with_cpu:
        from oracle import bindings as ob
        if not ob.ref_available():
            ob = None
    st = stream_obj.cuda_stream
    rows, g_tot, c_tot = [], 0.0, 0.0
    for (H, Wd, Cin, Cout, k, s, p, count) in RESNET18_480x640:
        r = np.random.default_rng(H * 7 + Cin)
        x = r.normal(0.0, 1.0, (H, Wd, Cin)).astype(np.float32)
        K = k * k * Cin
        W = r.uniform(-0.2, 0.2, (Cout, K)).astype(np.float32)
        b = r.normal(0.0, 0.02, Cout).astype(np.float32)
        lin = vla.LinearI8.from_f32(W, b)
        Ho, Wo = (H + 2 * p - k) // s + 1, (Wd + 2 * p - k) // s + 1
        xd = torch.from_numpy(x).cuda()
        out = torch.empty((Ho, Wo, Cout), device="cuda")
        work = torch.empty(vla.conv2d_i8_workspace_bytes(H, Wd, Cin, Cout, k, s, p), dtype=torch.uint8,
                           device="cuda")
        # 20 calls captured as one HIP graph (as the sweep's GEMMs), so the
        # time is the device's, not the Python call's
        g = capture(torch, lambda cs: vla.conv2d_i8_dev(lin, out, xd, k, s, p, work, stream=cs), 20)
        us = time_graph(torch, g, 5, stream_obj) / 20
        npix = Ho * Wo
        ops = 2.0 * npix * Cout * K
        byt = 4.0 * H * Wd * Cin + Cout * K + 8.0 * Cout + 4.0 * npix * Cout
        roof = max(ops / (PEAK_INT8_TOPS * 1e12), byt / (PEAK_HBM_GBS * 1e9)) * 1e6
        row = {"layer": f"{H}x{Wd}x{Cin}->{Cout} k{k} s{s} p{p}", "count": count, "gpu_us": round(us, 2),
               "tops": round(ops / us / 1e6, 1), "roof_us": round(roof, 2), "frac": round(roof / us, 4)}
        g_tot += count * us
        if ob is not None:
            Wq, ws, blob = ob.ref_pack_weights(W) if Cout % 16 == 0 else (None, None, None)
            if blob is not None:
                o = np.empty((Ho, Wo, Cout), np.float32)
                L = ob.ref()
                f = lambda: L.ref_conv2d_i8_packed(ob._p(o), ob._p(x), ob._p(blob), ob._p(ws), ob._p(b), H, Wd,
                                                   Cin, Cout, k, s, p)
                row["cpu_ref_us"] = round(_time_cpu(f) * 1e3, 1)
                c_tot += count * row["cpu_ref_us"]
        rows.append(row)
        print(f"  conv {row}", file=sys.stderr, flush=True)
    out = {"layers": rows, "gpu_ms_total": round(g_tot / 1e3, 4)}
    if ob is not None:
        out["cpu_ref_ms_total"] = round(c_tot / 1e3, 3)
        out["cpu_ref_threads"] = int(ob.ref().ref_omp_max_threads())
    return out


def m_tokens_act(c):
    return c["n_1d"] + c["n_cams"] * c["fh"] * c["fw"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--shapes", default="", help="comma list MxKxN to restrict the sweep (debug)")
    ap.add_argument("--no-policy", action="store_true", help="skip the per-chunk policy latency leg")
    ap.add_argument("--policy-only", action="store_true",
                    help="only the per-chunk policy latency leg (for rocprofv3 runs)")
    ap.add_argument("--models", default="act,act_model,octo,smolvla,siglip,smolvla_model,octo_model,impact_model,"
                    "diffusion_model", help="policy graphs to time")
    ap.add_argument("--no-conv", action="store_true", help="skip the ResNet-18 conv2d_i8 leg")
    ap.add_argument("--conv-only", action="store_true", help="only the ResNet-18 conv2d_i8 leg")
    ap.add_argument("--profile-only", action="store_true",
                    help="only the dominant GEMM, back to back (for rocprofv3 runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the "
              "multi-GPU sharding of this path is a design, not a measured configuration",
              file=sys.stderr)
        sys.exit(2)

    import torch

    vla = load_pkg()
    vla.lib()
    if not vla.int8_available():
        print("bench.py: no gfx950 device visible", file=sys.stderr)
        sys.exit(1)
    import vla_simd_amd.synth as synth

    stream_obj = torch.cuda.Stream()
    torch.cuda.set_stream(stream_obj)
    stream = stream_obj.cuda_stream

    if args.conv_only:
        print(json.dumps({"conv_resnet18_480x640": conv_resnet18(vla, torch, stream_obj,
                                                                 with_cpu=not args.no_cpu)}), flush=True)
        return

    if args.policy_only:
        print(json.dumps({"policy_latency_ms": policy_latency(
            vla, torch, stream_obj, with_cpu=not args.no_cpu, models=args.models.split(","))}), flush=True)
        return

    shapes_spec = [(M, K, N) for (K, N) in synth.SWEEP_KN for M in synth.SWEEP_M]
    if args.shapes:  # any MxKxN list (A/B and scaling runs); the default is the sweep
        shapes_spec = [tuple(int(v) for v in s.split("x")) for s in args.shapes.split(",")]
    dominant = (8192, 4096, 4096)

    if args.profile_only:
        # the dominant GEMM, or the --shapes given, each quantized once and
        # launched 20 times eagerly (the profiler sees 20 dispatches per shape,
        # told apart by grid size)
        for spec in (shapes_spec if args.shapes else [dominant]):
            sh = Shape(vla, torch, synth, *spec)
            sh.quantize(vla, stream)
            for _ in range(20):
                sh.gemm(vla, stream)
        # calibration for the HBM byte counters: a plain device copy of 256 MiB
        # (reads 256 MiB, writes 256 MiB), well past the 256 MiB MALL
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_only": f"gemm {args.shapes or '8192x4096x4096'} x20 each, copy 256 MiB x3"}))
        return

    shapes = [Shape(vla, torch, synth, *s) for s in shapes_spec]
    torch.cuda.synchronize()
    print(f"bench: {len(shapes)} shapes resident on {vla.device_name()}", file=sys.stderr, flush=True)

    # per-shape kernel times: a graph of n back-to-back GEMM launches (cycling the
    # rotating copies), and a graph of n whole ops (quantize + GEMM)
    rows = []
    dom_us = None
    for sh in shapes:
        sh.quantize(vla, stream)
        torch.cuda.synchronize()
        n = max(sh.R, max(8, min(200, int(2000 / max(1.0, roof_us(sh.M, sh.K, sh.N)[0])))))
        g_gemm = capture(torch, lambda st: sh.gemm(vla, st), n)
        g_us = time_graph(torch, g_gemm, 3, stream_obj) / n
        g_op = capture(torch, lambda st: sh.op(vla, st), n)
        op_us = time_graph(torch, g_op, 3, stream_obj) / n
        # warm: the same n launches on one weight / output copy (L2 / MALL resident)
        g_warm = capture(torch, lambda st: sh.gemm_warm(vla, st), n)
        w_us = time_graph(torch, g_warm, 3, stream_obj) / n
        del g_gemm, g_op, g_warm
        ops = 2.0 * sh.M * sh.N * sh.K
        t_roof, bound = roof_us(sh.M, sh.K, sh.N)
        rows.append({
            "M": sh.M, "K": sh.K, "N": sh.N, "gemm_us": round(g_us, 3), "op_us": round(op_us, 3),
            "gemm_tops": round(ops / g_us / 1e6, 2),
            "gemm_gbs": round(gemm_bytes(sh.M, sh.K, sh.N) / g_us / 1e3, 1),
            "bound": bound, "roof_us": round(t_roof, 3), "frac": round(t_roof / g_us, 4),
            "gemm_warm_us": round(w_us, 3), "frac_warm": round(t_roof / w_us, 4),
            "rotating_copies": sh.R, "a_layout": "panel" if sh.panel else "row-major",
            "split_k": sh.split is not None,
        })
        if (sh.M, sh.K, sh.N) == dominant:
            dom_us = g_us
        print(f"  {sh.M}x{sh.K}x{sh.N}: gemm {g_us:.2f} us ({rows[-1]['gemm_tops']} TOPS, "
              f"{rows[-1]['gemm_gbs']} GB/s, {bound} frac {rows[-1]['frac']}), warm {w_us:.2f} us, op {op_us:.2f} us",
              file=sys.stderr, flush=True)

    # the step: every shape once (quantize + GEMM), captured as one graph
    def step(st):
        for sh in shapes:
            sh.op(vla, st)

    g_step = capture(torch, step, 1)
    for _ in range(args.warmup):
        g_step.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream_obj)
    for _ in range(args.steps):
        g_step.replay()
    end.record(stream_obj)
    end.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / args.steps
    total_ops = sum(2.0 * s.M * s.N * s.K for s in shapes)
    value = total_ops / (ms * 1e-3) / 1e12

    roofline = None
    if dom_us is not None:
        ach = 2.0 * 8192 * 4096 * 4096 / dom_us / 1e6
        roofline = {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_INT8_TOPS,
                    "unit": "TFLOP/s", "frac": round(ach / PEAK_INT8_TOPS, 4),
                    "traffic": profiled_traffic(),
                    "kernel": "int8 GEMM launch M=8192 K=4096 N=4096 (int8 ops = 2*M*N*K per "
                              "launch; unit TFLOP/s counts int8 ops)",
                    "avg_launch_us": round(dom_us, 3),
                    "algorithmic_bytes": gemm_bytes(*dominant),
                    "traffic_source": "profiles/gemm_i8_8192x4096x4096_traffic.txt"}

    cpu = None if args.no_cpu else cpu_baseline(synth)
    policy = None if args.no_policy else policy_latency(vla, torch, stream_obj, with_cpu=not args.no_cpu)
    conv = None if args.no_conv else conv_resnet18(vla, torch, stream_obj, with_cpu=not args.no_cpu)

    print(json.dumps({
        "metric": "int8 GEMM TOPS (% MFMA peak) + per-chunk policy latency ms, batch 1",
        "value": round(value, 3), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8 (int32 accumulate, fp32 out)",
        "data": "synthetic (seeded BASELINE distributions, vla.simd_amd/synth.py)",
        "config": {"workload": "int8 GEMM sweep, BASELINE.json configs[1]: 30 dense_linear_i8 "
                               "calls (device quantize + i8 MFMA GEMM) per step",
                   "shapes": len(shapes), "wall_s_timed": round(wall, 3)},
        "roofline": roofline, "cpu_baseline": cpu, "policy_latency_ms": policy, "sweep": rows,
        "conv_resnet18_480x640": conv,
    }), flush=True)


if __name__ == "__main__":
    main()
