"""Random-init checkpoints in the reference's own file layouts, for the graph
parity tests and the per-chunk latency bench (there is no network for real
checkpoints; BASELINE.json's configs 3-5 are random-init).

Each writer produces exactly what the reference's loader reads, in its order:

  ACT      act.meta ("key value" lines) + act.bin, the float arena walk of
           ActTransformer::load (src/models/act/act_transformer.cpp:29-170)
  Octo     octo.meta + octo.bin, OctoTransformer::load
           (src/models/octo/octo_transformer.cpp:17-99)
  SmolVLA  vlm.meta + vlm.bin (fp32 norms, then bf16 matrices,
           src/models/smolvla/smollm2_lm.cpp:17-83) and aex.meta + aex.bin
           (fp32, src/models/smolvla/action_expert.cpp:60-172)

Values come from vla_simd_amd.synth (seeded, machine-independent bytes):
linear weights U(-1/sqrt(K), 1/sqrt(K)) (torch nn.Linear's default scale),
biases N(0, 0.02^2), norm scales 1 + N(0, 0.02^2), norm biases N(0, 0.02^2),
learned position embeddings N(0, 0.02^2) (Octo, flax) or N(0, 1) (ACT, torch
nn.Embedding).
"""

from __future__ import annotations

import math
import os
import struct

import numpy as np

from . import synth

# ACT, encoder 4 x 302 tokens (15 x 20 feature grid
# + latent + state), d 512, 8 heads, FFN 3200 ReLU, decoder 1 x 100 queries,
# 14-dim action head.
ACT_BASE = dict(dim=512, heads=8, head_dim=64, ff=3200, n_enc=4, n_dec=1, chunk=100,
                state_dim=14, action_dim=14, n_1d=2, n_text=0, ln_eps=1e-5,
                img_ch=512, n_cams=1, fh=15, fw=20)

# Octo-base shape, 12 x 768, 12 heads, MLP 3072
# gelu-tanh, 2 timesteps of 256 primary + 64 wrist patches and one readout,
# 16 task tokens (658 tokens without the per-step task copy).
OCTO_BASE = dict(d=768, n_layers=12, heads=12, head_dim=64, mlp=3072, max_horizon=10, n_task=16,
                 tok_primary=256, tok_wrist=64, n_readout=1, t5_dim=768, stem_dim=512,
                 ln_eps=1e-6, gelu_erf=0, repeat_task=0, wnd=2)

# SmolVLA-shaped chunk, 16 text layers (960, 15q/5kv,
# hd 64, FFN 2560), prefix 2 x 64 image + 48 text + 1 state = 177 tokens,
# expert 16 layers of 720 (FFN 2048), chunk 50, 10 Euler steps.
SMOLVLA_BASE = dict(hidden=960, n_q=15, n_kv=5, head_dim=64, ffn=2560, eps=1e-5, rope_base=10000.0,
                    n_layers=16, expert_h=720, expert_ffn=2048, expert_layers=16,
                    self_attn_every_n=2, chunk=50, num_steps=10, max_action_dim=32,
                    min_period=4e-3, max_period=4.0, n_prefix=177)


class _Arena:
    """Collects float32 blocks in file order."""

    def __init__(self, tag: str, seed: int):
        self.tag, self.seed, self.parts = tag, seed, []

    def linear(self, name, N, K, bias=True):
        a = 1.0 / math.sqrt(K)
        self.parts.append(synth.uniform(f"{self.tag}.{name}.w", (N, K), -a, a, self.seed))
        if bias:
            self.parts.append(synth.normal(f"{self.tag}.{name}.b", (N,), 0.02, self.seed))

    def norm(self, name, n, bias=True):
        self.parts.append(1.0 + synth.normal(f"{self.tag}.{name}.s", (n,), 0.02, self.seed))
        if bias:
            self.parts.append(synth.normal(f"{self.tag}.{name}.b", (n,), 0.02, self.seed))

    def normal(self, name, shape, std):
        self.parts.append(synth.normal(f"{self.tag}.{name}", shape, std, self.seed))

    def write(self, path):
        with open(path, "wb") as f:
            for p in self.parts:
                f.write(np.ascontiguousarray(p, dtype=np.float32).tobytes())


def _meta(path, kv):
    with open(path, "w") as f:
        for k, v in kv.items():
            f.write(f"{k} {v}\n")


def write_act(dirpath: str, cfg: dict = ACT_BASE, seed: int = synth.BASE_SEED, tag: str = "act") -> str:
    """<tag>.meta / <tag>.bin as ActTransformer::load reads them (act.* for
    ACT, impact.* for IMPACT's transformer, impact_model.cpp:65)."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    d = c["dim"]
    _meta(os.path.join(dirpath, f"{tag}.meta"),
          {k: c[k] for k in ("dim", "heads", "head_dim", "ff", "n_enc", "n_dec", "chunk", "state_dim",
                             "action_dim", "n_1d", "n_text", "ln_eps")})
    a = _Arena("act", seed)
    a.linear("img_proj", d, c["img_ch"])
    a.linear("state_proj", d, c["state_dim"])
    a.normal("latent", (d,), 1.0)
    a.normal("pos1d", (c["n_1d"], d), 1.0)

    def mha(p):
        for w in ("q", "k", "v", "o"):
            a.linear(f"{p}.{w}", d, d)

    for i in range(c["n_enc"]):
        mha(f"enc{i}.attn")
        a.norm(f"enc{i}.n1", d)
        a.linear(f"enc{i}.w1", c["ff"], d)
        a.linear(f"enc{i}.w2", d, c["ff"])
        a.norm(f"enc{i}.n2", d)
    for i in range(c["n_dec"]):
        mha(f"dec{i}.self")
        a.norm(f"dec{i}.n1", d)
        mha(f"dec{i}.cross")
        a.norm(f"dec{i}.n2", d)
        a.linear(f"dec{i}.w1", c["ff"], d)
        a.linear(f"dec{i}.w2", d, c["ff"])
        a.norm(f"dec{i}.n3", d)
    a.normal("dec_pos", (c["chunk"], d), 1.0)
    a.norm("dec_norm", d)
    a.linear("head", c["action_dim"], d)
    a.write(os.path.join(dirpath, f"{tag}.bin"))
    return dirpath


def act_inputs(cfg: dict = ACT_BASE, seed: int = synth.BASE_SEED):
    feats = synth.normal("act.in.feats", (cfg["n_cams"] * cfg["fh"] * cfg["fw"], cfg["img_ch"]), 1.0, seed)
    state = synth.normal("act.in.state", (cfg["state_dim"],), 1.0, seed)
    return feats, state


# ACT end to end (ActModel, src/models/act/act_model.cpp): one 480 x 640
# camera through ResNet-18 (15 x 20 x 512 features) into ACT_BASE's
# transformer. width scales the trunk's channels (64 for ResNet-18).
ACT_MODEL_BASE = dict(ACT_BASE, img_h=480, img_w=640, n_cams=1, width=64, norm_eps=1e-8)


def resnet18_blocks(width: int = 64):
    """ResNet-18's basic blocks as backbone.meta lists them (cin, cout, stride,
    has_down): two per stage, the first of stages 2-4 strided with a 1x1
    projection (tools/_common.py:112-133)."""
    out, cin = [], width
    for si in range(4):
        cout = width << si
        for b in range(2):
            stride = 2 if si > 0 and b == 0 else 1
            down = int(stride != 1 or cin != cout)
            out.append((cin, cout, stride, down))
            cin = cout
    return out


def _write_resnet(dirpath: str, name: str, width: int, seed: int, film_after=(), gn_group_size: int = 0,
                  key: str = "bb") -> list:
    """<name>.meta / <name>.bin as ResNetBackbone::load reads them
    (resnet_backbone.cpp:49-154): ResNet-18 (weights NHWC [Cout][k][k][Cin])
    with BatchNorm folded into conv biases, or, with gn_group_size, a GroupNorm
    (scale, bias) after every bias-free conv; optional FiLM points. key names
    the weights' random streams."""
    blocks = resnet18_blocks(width)
    lines = ["in_ch 3", f"stem_out {width}", "stem_k 7", "stem_stride 2", "stem_pad 3", "pool_k 3",
             "pool_stride 2", "pool_pad 1"] + [f"block {a} {b} {st} {d}" for a, b, st, d in blocks]
    lines += [f"film_after {i}" for i in film_after]
    if gn_group_size:
        lines.append(f"gn_group_size {gn_group_size}")
    with open(os.path.join(dirpath, f"{name}.meta"), "w") as f:
        f.write("\n".join(lines) + "\n")
    a = _Arena(key, seed)

    def conv(name, cout, k, cin):
        bound = math.sqrt(3.0 / (k * k * cin))
        a.parts.append(synth.uniform(f"{key}.{name}.w", (cout, k, k, cin), -bound, bound, seed))
        if gn_group_size:
            a.parts.append(1.0 + synth.normal(f"{key}.{name}.gs", (cout,), 0.1, seed))
            a.parts.append(synth.normal(f"{key}.{name}.gb", (cout,), 0.05, seed))
        else:
            a.parts.append(synth.normal(f"{key}.{name}.b", (cout,), 0.05, seed))

    conv("stem", width, 7, 3)
    for i, (cin, cout, st, d) in enumerate(blocks):
        conv(f"b{i}.c1", cout, 3, cin)
        conv(f"b{i}.c2", cout, 3, cout)
        if d:
            conv(f"b{i}.down", cout, 1, cin)
    a.write(os.path.join(dirpath, f"{name}.bin"))
    return blocks


def _write_act_config(dirpath: str, c: dict, extra: str = ""):
    with open(os.path.join(dirpath, "config.txt"), "w") as f:
        f.write(f"img_h {c['img_h']}\nimg_w {c['img_w']}\nn_cams {c['n_cams']}\nnorm_eps {c['norm_eps']}\n")
        f.write(extra)
        for i in range(c["n_cams"]):
            f.write(f"cam{i} cam_{i}\n")


def _write_act_stats(dirpath: str, c: dict, seed: int):
    sd, ad = c["state_dim"], c["action_dim"]
    parts = [synth.normal("act.stats.state_mean", (sd,), 1.0, seed),
             0.5 + synth.uniform("act.stats.state_std", (sd,), 0.0, 1.0, seed),
             synth.normal("act.stats.action_mean", (ad,), 1.0, seed),
             0.5 + synth.uniform("act.stats.action_std", (ad,), 0.0, 1.0, seed)]
    for i in range(c["n_cams"]):
        parts.append(np.array([0.485, 0.456, 0.406], np.float32))
        parts.append(np.array([0.229, 0.224, 0.225], np.float32))
    np.concatenate([np.asarray(p, np.float32).reshape(-1) for p in parts]).tofile(
        os.path.join(dirpath, "stats.bin"))


def write_act_model(dirpath: str, cfg: dict = ACT_MODEL_BASE, seed: int = synth.BASE_SEED) -> str:
    """A whole ACT checkpoint as tools/convert_act.py writes it: config.txt,
    backbone.meta/.bin (BatchNorm folded into conv biases; weights NHWC
    [Cout][k][k][Cin]), act.meta/.bin (the transformer over the trunk's
    channels) and stats.bin (state, action, then per-camera image mean/std)."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    _write_act_config(dirpath, c)
    blocks = _write_resnet(dirpath, "backbone", c["width"], seed)
    write_act(dirpath, dict(c, img_ch=blocks[-1][1]), seed)
    _write_act_stats(dirpath, c, seed)
    return dirpath


# IMPACT end to end (ImpactModel, src/models/impact/impact_model.cpp): ACT's
# trunk with FiLM points at the end of each stage and its transformer with a
# text tail, conditioned on T5-small over a pruned vocabulary. The FiLM head is
# drawn small and non-zero here (a converted checkpoint starts it at zero,
# which would make the modulation the identity).
IMPACT_T5 = dict(d_model=512, n_layers=6, n_heads=8, d_kv=64, d_ff=2048, n_buckets=32, max_dist=128, eps=1e-6)
IMPACT_MODEL_BASE = dict(ACT_MODEL_BASE, n_text=32, film_after=(1, 3, 5, 7), t5=IMPACT_T5, unk_id=2,
                         keep=0.75)


def write_impact_model(dirpath: str, cfg: dict = IMPACT_MODEL_BASE, seed: int = synth.BASE_SEED) -> str:
    """A whole IMPACT checkpoint in the files ImpactModel::load reads:
    config.txt (with vocab_full and unk_id), vision.meta/.bin (the trunk and
    its film_after points), impact.meta/.bin (the transformer, n_text text
    slots), text.meta/.bin (T5-small over the pruned table, then the text
    projection [dim, d_model] + bias, the text positions [n_text, dim] and the
    FiLM head [2 film_total, d_model] + bias), vocab.txt (a SentencePiece
    vocabulary), vocab_map.bin (int32 per full id: its row in the pruned table
    or -1; a `keep` share of the ids kept, <unk> always) and stats.bin."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    write_t5_vocab(dirpath, seed=seed)
    with open(os.path.join(dirpath, "vocab.txt"), encoding="utf-8") as f:
        vocab_full = sum(1 for _ in f)
    r = np.random.default_rng(seed + 17)
    keep = r.random(vocab_full) < c["keep"]
    keep[c["unk_id"]] = True
    vmap = np.full(vocab_full, -1, np.int32)
    vmap[keep] = np.arange(int(keep.sum()), dtype=np.int32)
    vmap.tofile(os.path.join(dirpath, "vocab_map.bin"))
    _write_act_config(dirpath, c, f"vocab_full {vocab_full}\nunk_id {c['unk_id']}\n")
    blocks = _write_resnet(dirpath, "vision", c["width"], seed, c["film_after"])
    write_act(dirpath, dict(c, img_ch=blocks[-1][1]), seed, tag="impact")
    _write_act_stats(dirpath, c, seed)
    t5 = dict(c["t5"], vocab=int(keep.sum()))
    write_t5(dirpath, t5, stem="text", seed=seed)
    enc = os.path.getsize(os.path.join(dirpath, "text.bin")) // 4
    D, P, T = t5["d_model"], c["dim"], c["n_text"]
    F = sum(blocks[i][1] for i in c["film_after"])
    a = _Arena("text_heads", seed)
    a.linear("proj", P, D)
    a.normal("text_pos", (T, P), 0.5)
    a.parts.append(synth.normal("text_heads.film.w", (2 * F, D), 0.05 / math.sqrt(D), seed))
    a.parts.append(synth.normal("text_heads.film.b", (2 * F,), 0.02, seed))
    with open(os.path.join(dirpath, "text.bin"), "ab") as f:
        for part in a.parts:
            f.write(np.ascontiguousarray(part, dtype=np.float32).tobytes())
    with open(os.path.join(dirpath, "text.meta"), "a") as f:
        f.write(f"proj_dim {P}\nn_text {T}\nfilm_total {F}\nencoder_floats {enc}\n")
    return dirpath


def act_model_inputs(cfg: dict = ACT_MODEL_BASE, seed: int = synth.BASE_SEED):
    """uint8 frames [n_cams, img_h, img_w, 3] and a raw state [state_dim]."""
    u = synth.uniform("act.in.images", (cfg["n_cams"], cfg["img_h"], cfg["img_w"], 3), 0.0, 256.0, seed)
    images = np.clip(np.floor(u), 0, 255).astype(np.uint8)
    state = synth.normal("act.in.raw_state", (cfg["state_dim"],), 2.0, seed)
    return images, state


# Diffusion Policy's noise-prediction UNet (src/models/diffusion/unet1d.cpp)
# at lerobot's stock shape, and a small one for tests.
DP_UNET_BASE = dict(action_dim=6, horizon=64, down_dims=(512, 1024, 2048), kernel_size=5, n_groups=8,
                    step_embed_dim=128, film_scale=1, state_dim=6, n_cams=2, num_keypoints=32, n_obs_steps=2)


def dp_cond_dim(c: dict) -> int:
    """DPConfig::cond_dim (config.h:66-69): step embedding + (state + cameras) per obs step."""
    return c["step_embed_dim"] + (c["state_dim"] + c["n_cams"] * 2 * c["num_keypoints"]) * c["n_obs_steps"]


def write_dp_unet(dirpath: str, cfg: dict = DP_UNET_BASE, seed: int = synth.BASE_SEED) -> str:
    """unet.bin in the order DPUNet1d::load reads it (unet1d.cpp:18-34): step
    encoder, down blocks (two FiLM res blocks + a k3/s2 downsample but the
    last), two mid blocks, up blocks (two res blocks + a k4/s2 transposed conv),
    the final conv block and the 1x1 output conv."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    A, D, k, CD = c["action_dim"], c["step_embed_dim"], c["kernel_size"], dp_cond_dim(cfg)
    a = _Arena("unet", seed)
    n = [0]

    def lin(N, K, std=None):
        n[0] += 1
        bound = 1.0 / math.sqrt(K)
        a.parts.append(synth.uniform(f"unet.{n[0]}.w", (N, K), -bound, bound, seed))
        a.parts.append(synth.normal(f"unet.{n[0]}.b", (N,), 0.02, seed))

    def gn(C):
        n[0] += 1
        a.parts.append(1.0 + synth.normal(f"unet.{n[0]}.gs", (C,), 0.02, seed))
        a.parts.append(synth.normal(f"unet.{n[0]}.gb", (C,), 0.02, seed))

    def res(cin, cout):
        lin(cout, k * cin)
        gn(cout)
        lin(2 * cout if c["film_scale"] else cout, CD)
        lin(cout, k * cout)
        gn(cout)
        if cin != cout:
            lin(cout, cin)

    lin(4 * D, D)
    lin(D, 4 * D)
    dims = list(c["down_dims"])
    in_out = [(A, dims[0])] + [(dims[i], dims[i + 1]) for i in range(len(dims) - 1)]
    for i, (ci, co) in enumerate(in_out):
        res(ci, co)
        res(co, co)
        if i + 1 < len(in_out):
            lin(co, 3 * co)
    res(dims[-1], dims[-1])
    res(dims[-1], dims[-1])
    for ind in range(len(in_out) - 1):
        dim_out, dim_in = in_out[len(in_out) - 1 - ind]
        res(dim_in * 2, dim_out)
        res(dim_out, dim_out)
        n[0] += 1
        bound = 1.0 / math.sqrt(4 * dim_out)
        a.parts.append(synth.uniform(f"unet.{n[0]}.up", (dim_out, 4, dim_out), -bound, bound, seed))
        a.parts.append(synth.normal(f"unet.{n[0]}.upb", (dim_out,), 0.02, seed))
    lin(dims[0], k * dims[0])
    gn(dims[0])
    lin(A, dims[0])
    a.write(os.path.join(dirpath, "unet.bin"))
    return dirpath


# Diffusion Policy end to end (DiffusionModel, src/models/diffusion/): lerobot's
# stock pusht-shaped policy, two 96 x 96 cameras centre-cropped to 84 x 84,
# GroupNorm ResNet-18 encoders (16 channels per group), 32 keypoints, the
# 512/1024/2048 UNet over a 16-step horizon, DDPM with 100 steps.
DP_MODEL_BASE = dict(DP_UNET_BASE, horizon=16, n_action_steps=8, img_h=96, img_w=96, crop_h=84, crop_w=84,
                     width=64, gn_group_size=16, separate_encoders=1, scheduler="DDPM", num_train_timesteps=100,
                     num_inference_steps=100, beta_schedule="squaredcos_cap_v2", clip_sample=1,
                     clip_sample_range=1.0)


def write_diffusion_model(dirpath: str, cfg: dict = DP_MODEL_BASE, seed: int = synth.BASE_SEED) -> str:
    """A whole Diffusion Policy checkpoint as tools/convert_diffusion.py
    writes it: diffusion.meta, per encoder rgb_encoder<i>_backbone.meta/.bin
    (GroupNorm ResNet-18) and rgb_encoder<i>.bin (the 1x1 keypoint conv
    [K, C] + bias, the output Linear [2K, 2K] + bias), unet.bin and stats.bin
    (state min / max, action min / max, per camera image mean / std)."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    keys = ("n_obs_steps", "n_cams", "img_h", "img_w", "crop_h", "crop_w", "state_dim", "action_dim", "horizon",
            "n_action_steps", "num_keypoints", "kernel_size", "n_groups", "step_embed_dim", "num_train_timesteps",
            "num_inference_steps", "beta_schedule", "clip_sample", "clip_sample_range", "film_scale",
            "separate_encoders", "scheduler")
    with open(os.path.join(dirpath, "diffusion.meta"), "w") as f:
        for k in keys:
            f.write(f"{k} {c[k]}\n")
        f.write("prediction_type epsilon\n")
        f.write("down_dims " + " ".join(str(d) for d in c["down_dims"]) + "\n")
        for i in range(c["n_cams"]):
            f.write(f"cam observation.images.cam{i}\n")
    K, F = c["num_keypoints"], 2 * c["num_keypoints"]
    for e in range(c["n_cams"] if c["separate_encoders"] else 1):
        blocks = _write_resnet(dirpath, f"rgb_encoder{e}_backbone", c["width"], seed,
                               gn_group_size=c["gn_group_size"], key=f"dp.enc{e}")
        C = blocks[-1][1]
        a = _Arena(f"dp.enc{e}.head", seed)
        a.linear("kp", K, C)
        a.linear("out", F, F)
        a.write(os.path.join(dirpath, f"rgb_encoder{e}.bin"))
    write_dp_unet(dirpath, c, seed)
    sd, ad = c["state_dim"], c["action_dim"]
    smin = synth.normal("dp.stats.state_min", (sd,), 1.0, seed)
    amin = synth.normal("dp.stats.action_min", (ad,), 1.0, seed)
    parts = [smin, smin + 0.5 + synth.uniform("dp.stats.state_range", (sd,), 0.0, 1.0, seed),
             amin, amin + 0.5 + synth.uniform("dp.stats.action_range", (ad,), 0.0, 1.0, seed)]
    for i in range(c["n_cams"]):
        parts.append(np.array([0.485, 0.456, 0.406], np.float32))
        parts.append(np.array([0.229, 0.224, 0.225], np.float32))
    np.concatenate([np.asarray(p, np.float32).reshape(-1) for p in parts]).tofile(
        os.path.join(dirpath, "stats.bin"))
    return dirpath


def diffusion_model_inputs(cfg: dict = DP_MODEL_BASE, seed: int = synth.BASE_SEED, tag: str = "q0"):
    """uint8 frames [n_obs, n_cams, img_h, img_w, 3], raw states [n_obs,
    state_dim] inside the stats' ranges, and the sampler's noise [1 +
    num_inference_steps, horizon, action_dim] (the prior, then one buffer per
    DDPM step)."""
    c = cfg
    u = synth.uniform(f"dp.in.{tag}.frames", (c["n_obs_steps"], c["n_cams"], c["img_h"], c["img_w"], 3),
                      0.0, 256.0, seed)
    frames = np.clip(np.floor(u), 0, 255).astype(np.uint8)
    state = synth.normal(f"dp.in.{tag}.state", (c["n_obs_steps"], c["state_dim"]), 1.0, seed)
    noise = synth.normal(f"dp.in.{tag}.noise", (1 + c["num_inference_steps"], c["horizon"], c["action_dim"]),
                         1.0, seed)
    return frames, state, noise


def write_octo(dirpath: str, cfg: dict = OCTO_BASE, seed: int = synth.BASE_SEED) -> str:
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    D = c["d"]
    keys = ("d", "n_layers", "heads", "head_dim", "mlp", "max_horizon", "n_task", "tok_primary",
            "tok_wrist", "n_readout", "t5_dim", "stem_dim", "ln_eps", "gelu_erf", "repeat_task")
    _meta(os.path.join(dirpath, "octo.meta"), {k: c[k] for k in keys if k in c})
    a = _Arena("octo", seed)
    a.linear("proj_task", D, c["t5_dim"])
    a.linear("proj_prim", D, c["stem_dim"])
    a.linear("proj_wrist", D, c["stem_dim"])
    a.normal("pos_task", (c["n_task"], D), 0.02)
    a.normal("pos_prim", (c["max_horizon"], c["tok_primary"], D), 0.02)
    a.normal("pos_wrist", (c["max_horizon"], c["tok_wrist"], D), 0.02)
    a.normal("pos_readout", (c["max_horizon"], c["n_readout"], D), 0.02)
    for i in range(c["n_layers"]):
        a.norm(f"l{i}.ln1", D)
        for w in ("q", "k", "v", "o"):
            a.linear(f"l{i}.{w}", D, D)
        a.norm(f"l{i}.ln2", D)
        a.linear(f"l{i}.w1", c["mlp"], D)
        a.linear(f"l{i}.w2", D, c["mlp"])
    a.norm("final", D)
    a.write(os.path.join(dirpath, "octo.bin"))
    return dirpath


def octo_inputs(cfg: dict = OCTO_BASE, seed: int = synth.BASE_SEED):
    w = cfg["wnd"]
    t5 = synth.normal("octo.in.t5", (cfg["n_task"], cfg["t5_dim"]), 1.0, seed)
    sp = synth.normal("octo.in.prim", (w, cfg["tok_primary"], cfg["stem_dim"]), 1.0, seed)
    sw = synth.normal("octo.in.wrist", (w, cfg["tok_wrist"], cfg["stem_dim"]), 1.0, seed)
    tmask = np.ones(w, np.uint8)
    return t5, sp, sw, tmask


def _bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (what a bf16 checkpoint holds)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def write_smolvla(dirpath: str, cfg: dict = SMOLVLA_BASE, seed: int = synth.BASE_SEED) -> str:
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    H, NL, F = c["hidden"], c["n_layers"], c["ffn"]
    QF, KV = c["n_q"] * c["head_dim"], c["n_kv"] * c["head_dim"]
    _meta(os.path.join(dirpath, "vlm.meta"),
          {"hidden": H, "n_q": c["n_q"], "n_kv": c["n_kv"], "head_dim": c["head_dim"], "ffn": F,
           "eps": c["eps"], "rope_base": c["rope_base"], "n_layers": NL})
    norms = []
    for L in range(NL):
        norms.append(1.0 + synth.normal(f"vlm.l{L}.ln_in", (H,), 0.02, seed))
        norms.append(1.0 + synth.normal(f"vlm.l{L}.ln_post", (H,), 0.02, seed))
    norms.append(1.0 + synth.normal("vlm.out_norm", (H,), 0.02, seed))
    with open(os.path.join(dirpath, "vlm.bin"), "wb") as f:
        for p in norms:
            f.write(np.asarray(p, np.float32).tobytes())
        for L in range(NL):
            for name, (N, K) in (("q", (QF, H)), ("k", (KV, H)), ("v", (KV, H)), ("o", (H, QF)),
                                 ("gate", (F, H)), ("up", (F, H)), ("down", (H, F))):
                a = 1.0 / math.sqrt(K)
                f.write(_bf16(synth.uniform(f"vlm.l{L}.{name}", (N, K), -a, a, seed)).tobytes())

    EH, EF, ENL = c["expert_h"], c["expert_ffn"], c["expert_layers"]
    MAD, san = c["max_action_dim"], c["self_attn_every_n"]
    _meta(os.path.join(dirpath, "aex.meta"),
          {"expert_h": EH, "expert_ffn": EF, "n_q": c["n_q"], "n_kv": c["n_kv"],
           "head_dim": c["head_dim"], "eps": c["eps"], "rope_base": c["rope_base"], "n_layers": ENL,
           "self_attn_every_n": san, "chunk": c["chunk"], "num_steps": c["num_steps"],
           "max_action_dim": MAD, "min_period": c["min_period"], "max_period": c["max_period"]})
    a = _Arena("aex", seed)
    for L in range(ENL):
        self_attn = san > 0 and L % san == 0
        kk = EH if self_attn else KV
        a.norm(f"l{L}.ln_in", EH, bias=False)
        a.linear(f"l{L}.q", QF, EH, bias=False)
        a.linear(f"l{L}.k", KV, kk, bias=False)
        a.linear(f"l{L}.v", KV, kk, bias=False)
        a.linear(f"l{L}.o", EH, QF, bias=False)
        a.norm(f"l{L}.ln_post", EH, bias=False)
        a.linear(f"l{L}.gate", EF, EH, bias=False)
        a.linear(f"l{L}.up", EF, EH, bias=False)
        a.linear(f"l{L}.down", EH, EF, bias=False)
    a.norm("out_norm", EH, bias=False)
    a.linear("action_in", EH, MAD)
    a.linear("action_time_in", EH, 2 * EH)
    a.linear("action_time_out", EH, EH)
    a.linear("action_out", MAD, EH)
    a.write(os.path.join(dirpath, "aex.bin"))
    return dirpath


# SmolVLM2-500M's SigLIP vision tower (src/models/smolvla/siglip_vision.h:23-38):
# 512 x 512 images, 16 x 16 patches (1024), 12 layers of 768 (12 heads, MLP
# 3072 gelu-tanh), pixel shuffle by 4 into 64 tokens, projection to 960.
SIGLIP_BASE = dict(hidden=768, n_heads=12, head_dim=64, inter=3072, n_layers=12, patch=16, img=512,
                   n_patches=1024, ln_eps=1e-6, scale_factor=4, mm_out=960, n_img_tok=64)


def write_siglip(dirpath: str, cfg: dict = SIGLIP_BASE, seed: int = synth.BASE_SEED) -> str:
    """vit.meta + vit.bin as SiglipVision::load reads them
    (src/models/smolvla/siglip_vision.cpp:21-140): an fp32 region (patch bias,
    position embedding, per layer ln1 w/b, q/k/v/o biases, ln2 w/b, fc1/fc2
    biases, post-LN w/b) then a bf16 region (patch weight [H, 3 p p], per
    layer Wq Wk Wv Wo fc1 fc2, the modality projection [mm_out, H sf sf])."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    H, I, NL, P = c["hidden"], c["inter"], c["n_layers"], c["patch"]
    PD, NP, SD = 3 * P * P, c["n_patches"], c["hidden"] * c["scale_factor"] ** 2
    _meta(os.path.join(dirpath, "vit.meta"), {k: c[k] for k in (
        "hidden", "n_heads", "head_dim", "inter", "n_layers", "patch", "img", "n_patches", "ln_eps",
        "scale_factor", "mm_out", "n_img_tok")})
    f32 = [synth.normal("vit.patch.b", (H,), 0.02, seed), synth.normal("vit.pos", (NP, H), 0.02, seed)]
    for L in range(NL):
        f32 += [1.0 + synth.normal(f"vit.l{L}.ln1.s", (H,), 0.02, seed),
                synth.normal(f"vit.l{L}.ln1.b", (H,), 0.02, seed)]
        f32 += [synth.normal(f"vit.l{L}.b{n}", (H,), 0.02, seed) for n in "qkvo"]
        f32 += [1.0 + synth.normal(f"vit.l{L}.ln2.s", (H,), 0.02, seed),
                synth.normal(f"vit.l{L}.ln2.b", (H,), 0.02, seed),
                synth.normal(f"vit.l{L}.fc1.b", (I,), 0.02, seed),
                synth.normal(f"vit.l{L}.fc2.b", (H,), 0.02, seed)]
    f32 += [1.0 + synth.normal("vit.post.s", (H,), 0.02, seed), synth.normal("vit.post.b", (H,), 0.02, seed)]

    def w(name, N, K):
        a = 1.0 / math.sqrt(K)
        return _bf16(synth.uniform(name, (N, K), -a, a, seed))

    with open(os.path.join(dirpath, "vit.bin"), "wb") as f:
        for p in f32:
            f.write(np.asarray(p, np.float32).tobytes())
        f.write(w("vit.patch.w", H, PD).tobytes())
        for L in range(NL):
            for n in "qkvo":
                f.write(w(f"vit.l{L}.w{n}", H, H).tobytes())
            f.write(w(f"vit.l{L}.fc1.w", I, H).tobytes())
            f.write(w(f"vit.l{L}.fc2.w", H, I).tobytes())
        f.write(w("vit.mm_proj", c["mm_out"], SD).tobytes())
    return dirpath


def siglip_inputs(cfg: dict = SIGLIP_BASE, seed: int = synth.BASE_SEED):
    """pixels [3, img, img] CHW, uniform in [-1, 1] (normalized image)."""
    return synth.uniform("vit.in.pixels", (3, cfg["img"], cfg["img"]), -1.0, 1.0, seed)


def siglip_gguf_layout(cfg: dict = SIGLIP_BASE) -> dict:
    """vit.bin as the converter stores it: the fp32 region, then bf16."""
    H, I, NL, NP = cfg["hidden"], cfg["inter"], cfg["n_layers"], cfg["n_patches"]
    n_f32 = H + NP * H + NL * (2 * H + 4 * H + 2 * H + I + H) + 2 * H
    return {"vit.bin": [("F32", n_f32 * 4), ("BF16", None)]}


def smolvla_inputs(cfg: dict = SMOLVLA_BASE, seed: int = synth.BASE_SEED, n_pad: int = 0):
    """prefix [n_prefix, hidden] ~ N(0,1), pad [n_prefix] (n_pad text slots
    before the state token marked as padding), noise [chunk, max_action_dim] ~ N(0,1)."""
    n = cfg["n_prefix"]
    prefix = synth.normal("smolvla.in.prefix", (n, cfg["hidden"]), 1.0, seed)
    pad = np.ones(n, np.int32)
    if n_pad:
        pad[n - 1 - n_pad:n - 1] = 0
    noise = synth.normal("smolvla.in.noise", (cfg["chunk"], cfg["max_action_dim"]), 1.0, seed)
    return prefix, pad, noise


# ------------------------------------------------------------ tokenizer --
# A byte-level BPE tokenizer directory (vocab.txt "id<TAB>token", merges.txt
# "left right", the files src/tokenizer/tokenizer.cpp:122-151 reads), trained
# here on a small corpus so the merges exercise letters, spaces, digits and
# punctuation. Token ids 0..255 are the 256 byte symbols in byte order.

def gpt2_byte_symbols() -> list:
    """The byte alphabet: bytes 33-126, 161-172, 174-255 stand for
    themselves, the rest for code points 256, 257, ... in byte order."""
    keep = set(range(33, 127)) | set(range(161, 173)) | set(range(174, 256))
    out, n = [], 0
    for b in range(256):
        if b in keep:
            out.append(chr(b))
        else:
            out.append(chr(256 + n))
            n += 1
    return out


TOK_CORPUS = ("pick up the red block and put it in the box. place the cup on the plate, then open the "
              "drawer. push the green button twice; don't drop the sponge! move the arm 10 cm to the "
              "left and grasp the handle. the robot picks the blue cube, stacks it on top of the "
              "yellow one and returns home. wipe the table with the cloth and fold the towel.")


def write_bpe_tokenizer(dirpath: str, n_merges: int = 160, corpus: str = TOK_CORPUS) -> str:
    os.makedirs(dirpath, exist_ok=True)
    sym = gpt2_byte_symbols()
    words = []
    for i, w in enumerate(corpus.split(" ")):
        b = ((" " if i else "") + w).encode()
        words.append([sym[x] for x in b])
    merges = []
    for _ in range(n_merges):
        counts = {}
        for w in words:
            for a, b in zip(w, w[1:]):
                counts[(a, b)] = counts.get((a, b), 0) + 1
        if not counts:
            break
        best = max(sorted(counts), key=lambda k: counts[k])
        merges.append(best)
        for w in words:
            i = 0
            while i + 1 < len(w):
                if (w[i], w[i + 1]) == best:
                    w[i:i + 2] = [w[i] + w[i + 1]]
                i += 1
    vocab = list(sym) + [a + b for a, b in merges]
    seen, rows = set(), []
    for t in vocab:
        if t not in seen:
            seen.add(t)
            rows.append(t)
    with open(os.path.join(dirpath, "vocab.txt"), "w", encoding="utf-8", newline="\n") as f:
        for i, t in enumerate(rows):
            f.write(f"{i}\t{t}\n")
    with open(os.path.join(dirpath, "merges.txt"), "w", encoding="utf-8", newline="\n") as f:
        f.write("#version: 0.2\n")
        for a, b in merges:
            f.write(f"{a} {b}\n")
    return dirpath


def write_t5_vocab(dirpath: str, corpus: str = TOK_CORPUS, seed: int = synth.BASE_SEED) -> str:
    """A SentencePiece unigram vocab.txt ("piece<TAB>score" per line, line =
    id; src/tokenizer/t5_tokenizer.cpp:46-72): <pad> </s> <unk> (score 0),
    then the corpus's words (U+2581-prefixed) and their prefixes and suffixes,
    single characters, a literal special piece <extra_id_0> (score 0), a
    score-0 ordinary piece (unusable) and a duplicate line (the first wins)."""
    os.makedirs(dirpath, exist_ok=True)
    r = np.random.default_rng(seed)
    sp = "▁"
    pieces = {}
    for w in corpus.replace(",", " ,").replace(".", " .").replace(";", " ;").replace("!", " !").split():
        w = sp + w
        for k in range(1, len(w) + 1):
            pieces.setdefault(w[:k], -2.0 - 0.5 * (len(w) - k) - float(r.random()))
            pieces.setdefault(w[-k:], -3.0 - 0.5 * (len(w) - k) - float(r.random()))
    for ch in "abcdefghijklmnopqrstuvwxyz0123456789.,;!?'-" + sp:
        pieces.setdefault(ch, -8.0 - float(r.random()))
    lines = ["<pad>\t0", "</s>\t0", "<unk>\t0"]
    lines += [f"{p}\t{v:.6f}" for p, v in pieces.items()]
    lines += ["<extra_id_0>\t0", "zzz\t0", f"{sp}the\t-0.5", "notab line"]
    with open(os.path.join(dirpath, "vocab.txt"), "w", encoding="utf-8", newline="\n") as f:
        f.write("\n".join(lines) + "\n")
    return dirpath


# ---------------------------------------------------------------- Octo model --
# The whole Octo checkpoint OctoModel::load reads (src/models/octo/
# octo_model.cpp:64-98, tools/convert_octo.py's file set): the T5 encoder
# (t5.meta/.bin, fp32), two SmallStems (stem_{primary,wrist}.meta/.bin), the
# block transformer (octo.meta/.bin, the reference's repeated-task layout),
# the DDPM head (head.meta/.bin), the action statistics and a SentencePiece
# vocab in tok/.
T5_BASE = dict(d_model=768, n_layers=12, n_heads=12, d_kv=64, d_ff=3072, vocab=32128, n_buckets=32,
               max_dist=128, eps=1e-6)
OCTO_STEM_BASE = dict(features=(32, 96, 192, 384), embed_dim=512, gn_groups=32, gn_eps=1e-6)
OCTO_HEAD_BASE = dict(action_dim=7, horizon=4, time_dim=32, num_blocks=3, hidden=256, steps=20, max_action=5.0)
OCTO_MODEL_BASE = dict(t5=T5_BASE, stem=OCTO_STEM_BASE, tf=dict(OCTO_BASE, repeat_task=1), head=OCTO_HEAD_BASE)


def write_t5(dirpath: str, cfg: dict = T5_BASE, stem: str = "t5", seed: int = synth.BASE_SEED) -> str:
    """<stem>.meta + <stem>.bin as T5Encoder::load reads them
    (src/nn/t5_encoder.cpp:20-63): embedding, relative bias [n_buckets,
    n_heads], per layer ln1, Wq, Wk, Wv, Wo, ln2, Wi [d_ff, d], Wo2 [d, d_ff],
    the final norm; fp32, no biases."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    D, FF = c["d_model"], c["d_ff"]
    _meta(os.path.join(dirpath, f"{stem}.meta"), {k: c[k] for k in (
        "d_model", "n_layers", "n_heads", "d_kv", "d_ff", "vocab", "n_buckets", "max_dist", "eps")})
    a = _Arena(stem, seed)
    a.normal("emb", (c["vocab"], D), 1.0)
    a.normal("rel", (c["n_buckets"], c["n_heads"]), 0.5)
    for L in range(c["n_layers"]):
        a.norm(f"l{L}.ln1", D, bias=False)
        for w in ("q", "k", "v"):
            a.linear(f"l{L}.{w}", D, D, bias=False)
        # T5 folds 1/sqrt(d_kv) into its query weights: keep the logits tame
        a.parts[-3] = a.parts[-3] / math.sqrt(c["d_kv"])
        a.linear(f"l{L}.o", D, D, bias=False)
        a.norm(f"l{L}.ln2", D, bias=False)
        a.linear(f"l{L}.wi", FF, D, bias=False)
        a.linear(f"l{L}.wo", D, FF, bias=False)
    a.norm("final", D, bias=False)
    a.write(os.path.join(dirpath, f"{stem}.bin"))
    return dirpath


def write_octo_stem(dirpath: str, name: str, cfg: dict = OCTO_STEM_BASE, seed: int = synth.BASE_SEED) -> str:
    """<name>.meta + <name>.bin as SmallStem::load reads them
    (src/models/octo/small_stem.cpp:19-82): per layer the 3x3 stride-2 conv
    [cout, 3, 3, cin] + bias, GroupNorm scale + bias; then the embedding."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    feats = list(c["features"])
    with open(os.path.join(dirpath, f"{name}.meta"), "w") as f:
        f.write(f"in_ch 6\nn_layers {len(feats)}\nk 3\nstride 2\npad 1\n")
        f.write("features " + " ".join(map(str, feats)) + "\n")
        f.write(f"embed_dim {c['embed_dim']}\ngn_groups {c['gn_groups']}\ngn_eps {c['gn_eps']}\n")
    a = _Arena(name, seed)
    cin = 6
    for i, cout in enumerate(feats):
        k = 9 * cin
        bound = 1.0 / math.sqrt(k)
        a.parts.append(synth.uniform(f"{name}.c{i}.w", (cout, 3, 3, cin), -bound, bound, seed))
        a.parts.append(synth.normal(f"{name}.c{i}.b", (cout,), 0.02, seed))
        a.norm(f"c{i}.gn", cout)
        cin = cout
    a.linear("embed", c["embed_dim"], cin)
    a.write(os.path.join(dirpath, f"{name}.bin"))
    return dirpath


def write_octo_head(dirpath: str, emb: int, cfg: dict = OCTO_HEAD_BASE, seed: int = synth.BASE_SEED) -> str:
    """head.meta + head.bin as DiffusionHead::load reads them
    (src/models/octo/diffusion_head.cpp:17-118): Fourier weights, the cond
    MLP, in_proj, blocks (LN, d0 [4H, H], d1 [H, 4H]), out_proj, then the
    betas / alphas / alpha_hats of a linear schedule."""
    os.makedirs(dirpath, exist_ok=True)
    c = cfg
    TD, H, FLAT, S = c["time_dim"], c["hidden"], c["action_dim"] * c["horizon"], c["steps"]
    _meta(os.path.join(dirpath, "head.meta"),
          {"emb": emb, "action_dim": c["action_dim"], "horizon": c["horizon"], "time_dim": TD,
           "num_blocks": c["num_blocks"], "hidden": H, "steps": S, "max_action": c["max_action"]})
    a = _Arena("head", seed)
    a.normal("fourier", (TD // 2,), 0.2)
    a.linear("cond0", 2 * TD, TD)
    a.linear("cond1", TD, 2 * TD)
    a.linear("in_proj", H, TD + emb + FLAT)
    for b in range(c["num_blocks"]):
        a.norm(f"b{b}.ln", H)
        a.linear(f"b{b}.d0", 4 * H, H)
        a.linear(f"b{b}.d1", H, 4 * H)
    a.linear("out_proj", FLAT, H)
    betas = np.linspace(1e-4, 0.02, S, dtype=np.float64)
    alphas = 1.0 - betas
    a.parts += [betas.astype(np.float32), alphas.astype(np.float32), np.cumprod(alphas).astype(np.float32)]
    a.write(os.path.join(dirpath, "head.bin"))
    return dirpath


def write_octo_model(dirpath: str, cfg: dict = OCTO_MODEL_BASE, seed: int = synth.BASE_SEED) -> str:
    c = cfg
    write_t5(dirpath, c["t5"], "t5", seed)
    write_octo_stem(dirpath, "stem_primary", c["stem"], seed)
    write_octo_stem(dirpath, "stem_wrist", dict(c["stem"]), seed + 1)
    write_octo(dirpath, c["tf"], seed)
    write_octo_head(dirpath, c["tf"]["d"], c["head"], seed)
    ad = c["head"]["action_dim"]
    mean = synth.normal("octo.act_mean", (ad,), 1.0, seed).astype(np.float32)
    std = synth.uniform("octo.act_std", (ad,), 0.5, 2.0, seed).astype(np.float32)
    mask = np.ones(ad, np.float32)
    mask[-1] = 0.0  # the gripper dimension stays normalized, as in the reference's stats
    for name, v in (("mean", mean), ("std", std), ("mask", mask)):
        v.tofile(os.path.join(dirpath, f"stats_action_{name}.bin"))
    write_t5_vocab(os.path.join(dirpath, "tok"))
    return dirpath


def octo_model_inputs(cfg: dict = OCTO_MODEL_BASE, wnd: int = 2, seed: int = synth.BASE_SEED):
    """primary [wnd, 256, 256, 3], wrist [wnd, 128, 128, 3] uint8, timestep
    mask [wnd], noise [flat], z [steps, flat]."""
    r = np.random.default_rng(seed)
    primary = r.integers(0, 256, size=(wnd, 256, 256, 3), dtype=np.uint8)
    wrist = r.integers(0, 256, size=(wnd, 128, 128, 3), dtype=np.uint8)
    h = cfg["head"]
    flat = h["action_dim"] * h["horizon"]
    noise = synth.normal("octo.in.noise", (flat,), 1.0, seed).astype(np.float32)
    z = synth.normal("octo.in.z", (h["steps"], flat), 1.0, seed).astype(np.float32)
    return primary, wrist, np.ones(wnd, np.uint8), noise, z


# ------------------------------------------------------------- SmolVLA model --
# The whole SmolVLA checkpoint SmolvlaModel::load reads
# (src/models/smolvla/smolvla_model.cpp:53-113, smolvla_capi.cpp:43-84): the
# vision tower, the text tower and expert, heads.meta, the bf16 token
# embedding table, the state projection, the normalization statistics,
# config.txt and a tokenizer directory tok/.
SMOLVLA_MODEL_BASE = dict(vit=SIGLIP_BASE, tf=dict(SMOLVLA_BASE), vocab=49152, max_state_dim=32,
                          real_state_dim=6, real_action_dim=6, n_views=2, norm_eps=1e-8, tok_maxlen=48,
                          pad_id=2)


def write_smolvla_model(dirpath: str, cfg: dict = SMOLVLA_MODEL_BASE, seed: int = synth.BASE_SEED) -> str:
    c = cfg
    write_siglip(dirpath, c["vit"], seed)
    write_smolvla(dirpath, c["tf"], seed)
    H, V, MSD = c["tf"]["hidden"], c["vocab"], c["max_state_dim"]
    assert c["vit"]["mm_out"] == H
    _meta(os.path.join(dirpath, "heads.meta"),
          {"vocab": V, "hidden": H, "max_state_dim": MSD, "real_state_dim": c["real_state_dim"],
           "real_action_dim": c["real_action_dim"], "n_views": c["n_views"], "norm_eps": c["norm_eps"]})
    with open(os.path.join(dirpath, "emb.bin"), "wb") as f:
        f.write(_bf16(synth.normal("smolvla.emb", (V, H), 0.05, seed)).tobytes())
    a = 1.0 / math.sqrt(MSD)
    with open(os.path.join(dirpath, "heads.bin"), "wb") as f:
        f.write(synth.uniform("smolvla.state_proj.w", (H, MSD), -a, a, seed).astype(np.float32).tobytes())
        f.write(synth.normal("smolvla.state_proj.b", (H,), 0.02, seed).astype(np.float32).tobytes())
    sd, ad = c["real_state_dim"], c["real_action_dim"]
    for name, n, kind in (("state_mean", sd, 0), ("state_std", sd, 1), ("action_mean", ad, 0),
                          ("action_std", ad, 1)):
        v = (synth.uniform(f"smolvla.{name}", (n,), 0.5, 2.0, seed) if kind
             else synth.normal(f"smolvla.{name}", (n,), 1.0, seed))
        with open(os.path.join(dirpath, f"stats_{name}.bin"), "wb") as f:
            f.write(np.asarray(v, np.float32).tobytes())
    with open(os.path.join(dirpath, "config.txt"), "w") as f:
        f.write("instruction pick up the red block\n")
        f.write(f"tokenizer_max_length {c['tok_maxlen']}\n")
        f.write(f"pad_token_id {c['pad_id']}\n")
    write_bpe_tokenizer(os.path.join(dirpath, "tok"))
    return dirpath


def smolvla_model_inputs(cfg: dict = SMOLVLA_MODEL_BASE, height: int = 480, width: int = 640,
                         seed: int = synth.BASE_SEED):
    """frames [n_views, height, width, 3] uint8, raw state [real_state_dim],
    noise [chunk, max_action_dim] ~ N(0, 1)."""
    nv = cfg["n_views"]
    r = np.random.default_rng(seed)
    frames = r.integers(0, 256, size=(nv, height, width, 3), dtype=np.uint8)
    state = synth.normal("smolvla.in.state", (cfg["real_state_dim"],), 1.0, seed).astype(np.float32)
    noise = synth.normal("smolvla.in.noise", (cfg["tf"]["chunk"], cfg["tf"]["max_action_dim"]), 1.0, seed)
    return frames, state, np.asarray(noise, np.float32)


# ------------------------------------------------------------ vla.simd GGUF --
# The single-file form of a converted directory that the reference's
# converters write (tools/_gguf.py:6-28) and its engine mounts
# (src/io/gguf_vla_simd.cpp:29-77): GGUF v3, general.architecture "vla-simd",
# vla_simd.format 1, every text file as the string vla_simd.file.<path>, every
# .bin as a 1-D tensor <path> (F32 unless a layout says otherwise) or, when it
# mixes element types, as parts <path>:0, <path>:1, ... in order; tensor data
# 32-byte aligned.

GGUF_TYPES = {"F32": (0, 4), "F16": (1, 2), "BF16": (30, 2), "I8": (24, 1), "I32": (26, 4)}
_KV_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
           11: "<q", 12: "<d"}


class GgufBuilder:
    """Byte-level GGUF writer: metadata of any type, tensors with explicit dims,
    element type and (optionally forced) offsets. write_gguf is built on it;
    the reader tests use it to make malformed files too."""

    def __init__(self, version: int = 3, align: int = 32):
        self.version, self.align = version, align
        self.kv, self.infos, self.blobs = [], [], []

    @staticmethod
    def _s(text) -> bytes:
        b = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        return struct.pack("<Q", len(b)) + b

    def string(self, key, value):
        self.kv.append(self._s(key) + struct.pack("<I", 8) + self._s(value))

    def scalar(self, key, gtype: int, value):
        self.kv.append(self._s(key) + struct.pack("<I", gtype) + struct.pack(_KV_FMT[gtype], value))

    def array(self, key, elem: int, values):
        body = b"".join(self._s(v) for v in values) if elem == 8 else \
            b"".join(struct.pack(_KV_FMT[elem], v) for v in values)
        self.kv.append(self._s(key) + struct.pack("<IIQ", 9, elem, len(values)) + body)

    def raw_kv(self, data: bytes):
        self.kv.append(bytes(data))

    def tensor(self, name, data: bytes, ggml_type: int, dims=None, offset=None):
        """dims (ggml order) default to the element count of data."""
        if dims is None:
            size = next(s for t, s in GGUF_TYPES.values() if t == ggml_type)
            dims = [len(data) // size]
        self.infos.append([name, list(dims), ggml_type, offset])
        self.blobs.append(bytes(data))

    def tobytes(self) -> bytes:
        head = b"GGUF" + struct.pack("<IQQ", self.version, len(self.infos), len(self.kv)) + b"".join(self.kv)
        offsets, off = [], 0
        for (name, dims, ty, forced), blob in zip(self.infos, self.blobs):
            off = (off + self.align - 1) // self.align * self.align
            offsets.append(off if forced is None else forced)
            head += self._s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            head += struct.pack("<IQ", ty, offsets[-1])
            off += len(blob)
        head += b"\0" * (-len(head) % self.align)
        data = bytearray()
        for o, blob in zip(offsets, self.blobs):
            if o < len(data):  # a forced offset may point anywhere; keep the data where the file asks
                continue
            data += b"\0" * (o - len(data))
            data += blob
        return head + bytes(data)


def write_gguf(src_dir: str, path: str, model: str, source: str = "", layout: dict | None = None,
               version: int = 3) -> str:
    """Pack a converted directory into one vla.simd GGUF. layout maps a .bin
    (relative path) to [(type, nbytes or None for the rest), ...] when it is not
    all F32, e.g. SmolVLA's vlm.bin = fp32 norms then bf16 matrices."""
    layout = layout or {}
    g = GgufBuilder(version)
    g.string("general.architecture", "vla-simd")
    g.string("general.name", os.path.splitext(os.path.basename(path))[0])
    g.string("vla_simd.model", model)
    g.scalar("vla_simd.format", 4, 1)
    g.string("vla_simd.source", source)
    files = []
    for d, dirs, names in os.walk(src_dir):
        dirs.sort()
        for n in sorted(names):
            full = os.path.join(d, n)
            files.append((os.path.relpath(full, src_dir).replace(os.sep, "/"), full))
    for rel, full in files:
        with open(full, "rb") as f:
            data = f.read()
        if not rel.endswith(".bin") or not data:
            g.string(f"vla_simd.file.{rel}", data.decode("utf-8"))
            continue
        parts = layout.get(rel, [("F32", None)])
        at = 0
        for i, (ty, n) in enumerate(parts):
            n = len(data) - at if n is None else n
            tid, size = GGUF_TYPES[ty]
            if n <= 0 or n % size or at + n > len(data):
                raise ValueError(f"{rel}: invalid {ty} part {i} of {n} bytes")
            g.tensor(rel if len(parts) == 1 else f"{rel}:{i}", data[at:at + n], tid)
            at += n
        if at != len(data):
            raise ValueError(f"{rel}: layout covers {at} of {len(data)} bytes")
    with open(path, "wb") as f:
        f.write(g.tobytes())
    return path


def smolvla_gguf_layout(cfg: dict = SMOLVLA_BASE) -> dict:
    """vlm.bin as the converter stores it: the fp32 norms, then bf16 matrices."""
    n_norm = (2 * cfg["n_layers"] + 1) * cfg["hidden"] * 4
    return {"vlm.bin": [("F32", n_norm), ("BF16", None)]}
