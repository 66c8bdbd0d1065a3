"""vla.simd_amd - MI355X (gfx950) backend of vla.simd's int8 linear + attention path.

The product is the C-ABI shared library ``libvla_simd_hip.so`` built from
``csrc/`` (declared in ``include/vla_simd_hip.h``). This module is its Python
face: a ctypes loader plus numpy-level wrappers named after the reference op
API (``tcpu::quantize_act_i8``, ``tcpu::dense_linear_i8``, ... in
src/ops/quant_ops.h and src/ops/lm_ops.h of the reference), the way the
reference's own Python layer drives its libraries through ctypes
(vla_simd/policy_server.py:203-273).

There is no CPU fallback: if the library is missing, or no gfx950 device is
present, the calls raise.

Load it by path (the directory name is not an importable identifier)::

    import importlib.util, sys
    spec = importlib.util.spec_from_file_location(
        "vla_simd_amd", "<repo>/vla.simd_amd/__init__.py",
        submodule_search_locations=["<repo>/vla.simd_amd"])
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_size_t, c_uint8, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvla_simd_hip.so")

VLA_OK, VLA_ERR_ARG, VLA_ERR_SHAPE, VLA_ERR_EXCEPTION = 0, -1, -2, -3
ACT = {"none": 0, "relu": 1, "gelu_tanh": 2, "gelu_erf": 3}
MASK_NONE, MASK_DENSE, MASK_CAUSAL, MASK_GROUPS = 0, 1, 2, 3

# Every symbol include/vla_simd_hip.h declares, in declaration order.
EXPORTS = (
    "vla_abi_version", "vla_backend_name", "vla_int8_available", "vla_last_error",
    "vla_hip_malloc", "vla_hip_free", "vla_hip_memcpy_h2d", "vla_hip_memcpy_d2h",
    "vla_hip_memset", "vla_hip_synchronize", "vla_hip_device_name",
    "vla_i8_kpad", "vla_quantize_act_i8", "vla_quantize_act_i8_dev", "vla_pack_weights_i8",
    "vla_quantize_span_i8", "vla_quantize_span_i8_dev",
    "vla_dense_linear_i8_pre", "vla_dense_linear_i8", "vla_dense_linear_i8_dev", "vla_dense_linear_i8_pre_dev",
    "vla_dense_linear_i8_noalloc_dev", "vla_dense_linear_i8_noalloc_max_bytes",
    "vla_i8_panel_bytes", "vla_quantize_act_i8_panel_dev", "vla_dense_linear_i8_panel_dev",
    "vla_dense_linear_i8_panel_split_dev",
    "vla_rowop_quantize_i8_panel_dev", "vla_rowop_linear_i8_fits", "vla_rowop_linear_i8_dev",
    "vla_ckpt_open", "vla_ckpt_free", "vla_ckpt_is_gguf", "vla_ckpt_file_size", "vla_ckpt_read",
    "vla_ckpt_names", "vla_conv2d_i8", "vla_conv2d_i8_workspace_bytes", "vla_conv2d_i8_dev",
    "vla_gemm_i8_split_bytes", "vla_dense_linear_i8_pre_split_dev",
    "vla_gemm_i8_i32", "vla_gemm_i8_i32_dev",
    "vla_linear_i8_create", "vla_linear_i8_create_q", "vla_linear_i8_free",
    "vla_linear_i8_weights", "vla_linear_i8_wscale", "vla_linear_i8_ldw",
    "vla_linear_i8_forward_dev", "vla_linear_i8_forward_quantized_dev",
    "vla_linear_i8_download", "vla_linear_i8_set_bias", "vla_linear_i8_forward", "vla_linear_i8_forward_quantized",
    "vla_conv2d_i8_resident", "vla_h2d_bytes",
    "vla_gqa_attention_masked", "vla_gqa_attention_dense", "vla_attention_dev", "vla_attention",
    "vla_layernorm", "vla_layernorm_dev", "vla_rmsnorm", "vla_rmsnorm_dev",
    "vla_rope_neox", "vla_rope_neox_dev",
    "vla_gelu_tanh", "vla_gelu_erf", "vla_relu", "vla_silu_gate",
    "vla_gelu_tanh_dev", "vla_gelu_erf_dev", "vla_relu_dev", "vla_silu_gate_dev", "vla_add_dev",
    "vla_dense_linear", "vla_dense_linear_dev",
    "vla_act_tf_load", "vla_act_tf_free", "vla_act_tf_chunk", "vla_act_tf_action_dim",
    "vla_act_tf_state_dim", "vla_act_tf_dim", "vla_act_tf_int8_layers", "vla_act_tf_graph_nodes",
    "vla_act_tf_forward", "vla_act_tf_forward_dev", "vla_act_tf_load_ex", "vla_act_tf_n_text",
    "vla_act_tf_forward_text", "vla_act_tf_forward_text_dev",
    "vla_octo_tf_load", "vla_octo_tf_free", "vla_octo_tf_dim", "vla_octo_tf_total_tokens",
    "vla_octo_tf_readout_index", "vla_octo_tf_config", "vla_octo_tf_int8_layers", "vla_octo_tf_graph_nodes",
    "vla_octo_tf_forward", "vla_octo_tf_forward_dev",
    "vla_smolvla_tf_load", "vla_smolvla_tf_free", "vla_smolvla_tf_chunk",
    "vla_smolvla_tf_max_action_dim", "vla_smolvla_tf_hidden", "vla_smolvla_tf_int8_layers",
    "vla_smolvla_tf_graph_nodes", "vla_smolvla_tf_chunk_run", "vla_smolvla_tf_chunk_dev",
    "vla_siglip_tf_load", "vla_siglip_tf_free", "vla_siglip_tf_img", "vla_siglip_tf_n_tokens",
    "vla_siglip_tf_out_dim", "vla_siglip_tf_int8_layers", "vla_siglip_tf_graph_nodes",
    "vla_siglip_tf_encode", "vla_siglip_tf_encode_dev",
    "vla_probe_begin", "vla_probe_end", "vla_probe_count", "vla_probe_shape", "vla_probe_read",
    "vla_act_load", "vla_act_free", "vla_act_chunk", "vla_act_action_dim", "vla_act_state_dim",
    "vla_act_n_cams", "vla_act_img_h", "vla_act_img_w", "vla_act_predict", "vla_act_predict_dev",
    "vla_act_encode", "vla_act_encode_dev", "vla_act_feat_shape", "vla_act_int8_convs", "vla_act_int8_layers",
    "vla_act_graph_nodes",
    "vla_impact_load", "vla_impact_free", "vla_impact_chunk", "vla_impact_action_dim", "vla_impact_state_dim",
    "vla_impact_n_cams", "vla_impact_img_h", "vla_impact_img_w", "vla_impact_n_text", "vla_impact_set_instruction",
    "vla_impact_predict", "vla_impact_tokens", "vla_impact_film", "vla_impact_predict_dev",
    "vla_impact_int8_layers", "vla_impact_int8_convs",
    "vla_diffusion_load", "vla_diffusion_free", "vla_diffusion_chunk", "vla_diffusion_horizon",
    "vla_diffusion_action_dim", "vla_diffusion_state_dim", "vla_diffusion_n_cams", "vla_diffusion_n_obs_steps",
    "vla_diffusion_img_h", "vla_diffusion_img_w", "vla_diffusion_num_steps", "vla_diffusion_is_ddim",
    "vla_diffusion_predict", "vla_diffusion_int8_layers", "vla_diffusion_int8_convs", "vla_diffusion_graph_nodes",
    "vla_smolvla_load", "vla_smolvla_free", "vla_smolvla_chunk", "vla_smolvla_action_dim",
    "vla_smolvla_state_dim", "vla_smolvla_n_views", "vla_smolvla_img_size", "vla_smolvla_tok_maxlen",
    "vla_smolvla_tokenize", "vla_smolvla_predict", "vla_smolvla_predict_rtc", "vla_smolvla_preprocess",
    "vla_smolvla_int8_layers", "vla_smolvla_graph_nodes", "vla_bpe_load", "vla_bpe_free", "vla_bpe_encode",
    "vla_unigram_load", "vla_unigram_free", "vla_unigram_encode",
    "vla_octo_load", "vla_octo_free", "vla_octo_horizon", "vla_octo_action_dim", "vla_octo_max_window",
    "vla_octo_predict", "vla_octo_predict_ex", "vla_octo_lang", "vla_octo_int8_layers",
)


class VlaError(RuntimeError):
    """A libvla_simd_hip call returned a status other than VLA_OK."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} -> {status}: {msg}")
        self.status = status


class VlaMask(ctypes.Structure):
    """vla_mask (include/vla_simd_hip.h)."""

    _fields_ = [
        ("kind", c_int32),
        ("dense", c_void_p),
        ("causal_offset", c_int32),
        ("n_groups", c_int32),
        ("q_group", c_void_p),
        ("k_group", c_void_p),
        ("allow", c_void_p),
    ]


_lib = None


def _declare(L):
    P = c_void_p
    i32, f32, i64 = c_int32, c_float, c_int64
    sig = {
        "vla_abi_version": (i32, []),
        "vla_backend_name": (c_char_p, []),
        "vla_int8_available": (i32, []),
        "vla_last_error": (c_char_p, []),
        "vla_hip_malloc": (i32, [POINTER(c_void_p), c_size_t]),
        "vla_hip_free": (i32, [P]),
        "vla_hip_memcpy_h2d": (i32, [P, P, c_size_t]),
        "vla_hip_memcpy_d2h": (i32, [P, P, c_size_t]),
        "vla_hip_memset": (i32, [P, i32, c_size_t]),
        "vla_hip_synchronize": (i32, []),
        "vla_hip_device_name": (i32, [c_char_p, i32]),
        "vla_i8_kpad": (i32, [i32]),
        "vla_quantize_act_i8": (i32, [P, P, P, i32, i32]),
        "vla_quantize_act_i8_dev": (i32, [P, P, i32, P, i32, i32, P]),
        "vla_pack_weights_i8": (i32, [P, P, P, i32, i32]),
        "vla_dense_linear_i8_pre": (i32, [P, P, P, P, P, P, i32, i32, i32]),
        "vla_dense_linear_i8": (i32, [P, P, P, P, P, i32, i32, i32]),
        "vla_dense_linear_i8_pre_dev": (i32, [P, i32, P, i32, P, P, i32, P, P, i32, i32, i32, i32, i32, P]),
        "vla_dense_linear_i8_dev": (i32, [P, i32, P, i32, P, i32, P, P, i32, i32, i32, P, i32, P, i32, i32, P]),
        "vla_quantize_span_i8": (i32, [P, P, i64, f32]),
        "vla_quantize_span_i8_dev": (i32, [P, P, i64, f32, P]),
        "vla_dense_linear_i8_noalloc_dev": (i32, [P, i32, P, i32, P, i32, P, P, i32, i32, i32, i32, i32, P]),
        "vla_dense_linear_i8_noalloc_max_bytes": (i64, []),
        "vla_i8_panel_bytes": (ctypes.c_int64, [i32, i32]),
        "vla_quantize_act_i8_panel_dev": (i32, [P, i32, P, P, i32, i32, P]),
        "vla_dense_linear_i8_panel_dev": (i32, [P, i32, P, P, P, i32, P, P, i32, i32, i32, i32, i32, P]),
        "vla_dense_linear_i8_panel_split_dev": (i32, [P, i32, P, P, P, i32, P, P, i32, i32, i32, i32, i32, P,
                                                      c_int64, P]),
        "vla_rowop_quantize_i8_panel_dev": (i32, [i32, P, i32, P, i32, P, ctypes.c_float, P, P, i32, i32, P]),
        "vla_rowop_linear_i8_fits": (i32, [i32, i32, i32]),
        "vla_conv2d_i8": (i32, [P, P, P, P, P, i32, i32, i32, i32, i32, i32, i32]),
        "vla_conv2d_i8_workspace_bytes": (ctypes.c_int64, [i32, i32, i32, i32, i32, i32, i32]),
        "vla_gemm_i8_split_bytes": (ctypes.c_int64, [i32, i32, i32]),
        "vla_dense_linear_i8_pre_split_dev": (i32, [P, i32, P, i32, P, P, i32, P, P, i32, i32, i32, i32, i32, P,
                                                    ctypes.c_int64, P]),
        "vla_conv2d_i8_dev": (i32, [P, P, P, i32, i32, i32, i32, i32, i32, P, ctypes.c_int64, P]),
        "vla_ckpt_open": (P, [c_char_p]),
        "vla_ckpt_free": (None, [P]),
        "vla_ckpt_is_gguf": (i32, [P]),
        "vla_ckpt_file_size": (ctypes.c_int64, [P, c_char_p]),
        "vla_ckpt_read": (i32, [P, c_char_p, P, ctypes.c_int64]),
        "vla_ckpt_names": (ctypes.c_int64, [P, c_char_p, ctypes.c_int64]),
        "vla_rowop_linear_i8_dev": (i32, [P, i32, i32, P, i32, P, i32, P, ctypes.c_float, P, i32, P, P, i32,
                                          i32, i32, i32, i32, P]),
        "vla_gemm_i8_i32": (i32, [P, P, P, i32, i32, i32]),
        "vla_gemm_i8_i32_dev": (i32, [P, P, i32, P, i32, i32, i32, i32, P]),
        "vla_linear_i8_create": (P, [P, P, i32, i32]),
        "vla_linear_i8_create_q": (P, [P, P, P, i32, i32]),
        "vla_linear_i8_free": (None, [P]),
        "vla_linear_i8_weights": (P, [P]),
        "vla_linear_i8_wscale": (P, [P]),
        "vla_linear_i8_ldw": (i32, [P]),
        "vla_linear_i8_forward_dev": (i32, [P, P, P, i32, P, P, i32, i32, P]),
        "vla_linear_i8_forward_quantized_dev": (i32, [P, P, P, i32, P, i32, i32, i32, P]),
        "vla_linear_i8_download": (i32, [P, P, i32, P]),
        "vla_linear_i8_set_bias": (i32, [P, P]),
        "vla_linear_i8_forward": (i32, [P, P, P, i32, P, i32, P]),
        "vla_linear_i8_forward_quantized": (i32, [P, P, P, i32, P, i32]),
        "vla_conv2d_i8_resident": (i32, [P, P, P, i32, i32, i32, i32, i32, i32]),
        "vla_h2d_bytes": (ctypes.c_int64, [i32]),
        "vla_gqa_attention_masked": (i32, [P, P, P, P, i32, i32, i32, i32, i32, f32, P]),
        "vla_gqa_attention_dense": (i32, [P, P, P, P, i32, i32, i32, i32, i32, f32]),
        "vla_attention_dev": (i32, [P, i32, P, i32, P, i32, P, i32, i32, i32, i32, i32, i32, f32,
                                    POINTER(VlaMask), P]),
        "vla_attention": (i32, [P, P, P, P, i32, i32, i32, i32, i32, f32, POINTER(VlaMask)]),
        "vla_layernorm": (i32, [P, P, P, P, i32, i32, f32]),
        "vla_layernorm_dev": (i32, [P, P, P, P, i32, i32, f32, P]),
        "vla_rmsnorm": (i32, [P, P, P, i32, i32, f32]),
        "vla_rmsnorm_dev": (i32, [P, P, P, i32, i32, f32, P]),
        "vla_rope_neox": (i32, [P, P, i32, i32, i32, f32]),
        "vla_rope_neox_dev": (i32, [P, i32, P, i32, i32, i32, f32, P]),
        "vla_gelu_tanh": (i32, [P, i32]),
        "vla_gelu_erf": (i32, [P, i32]),
        "vla_relu": (i32, [P, i32]),
        "vla_silu_gate": (i32, [P, P, P, i32]),
        "vla_gelu_tanh_dev": (i32, [P, i64, P]),
        "vla_gelu_erf_dev": (i32, [P, i64, P]),
        "vla_relu_dev": (i32, [P, i64, P]),
        "vla_silu_gate_dev": (i32, [P, P, P, i64, P]),
        "vla_add_dev": (i32, [P, P, P, i64, P]),
        "vla_dense_linear": (i32, [P, P, P, P, i32, i32, i32]),
        "vla_dense_linear_dev": (i32, [P, i32, P, i32, P, i32, P, i32, i32, i32, i32, i32, f32, P]),
        "vla_act_tf_load": (P, [c_char_p, i32, i32]),
        "vla_act_tf_free": (None, [P]),
        "vla_act_tf_chunk": (i32, [P]),
        "vla_act_tf_action_dim": (i32, [P]),
        "vla_act_tf_state_dim": (i32, [P]),
        "vla_act_tf_dim": (i32, [P]),
        "vla_act_tf_int8_layers": (i32, [P]),
        "vla_act_tf_graph_nodes": (i32, [P]),
        "vla_act_tf_forward": (i32, [P, P, i32, i32, i32, P, P]),
        "vla_act_tf_forward_dev": (i32, [P, P, i32, i32, i32, P, P, P]),
        "vla_act_tf_load_ex": (P, [c_char_p, i32, i32, i32]),
        "vla_act_tf_n_text": (i32, [P]),
        "vla_act_tf_forward_text": (i32, [P, P, i32, i32, i32, P, P, P, i32, P]),
        "vla_act_tf_forward_text_dev": (i32, [P, P, i32, i32, i32, P, P, P, i32, P, P]),
        "vla_octo_tf_load": (P, [c_char_p, i32]),
        "vla_octo_tf_free": (None, [P]),
        "vla_octo_tf_dim": (i32, [P]),
        "vla_octo_tf_total_tokens": (i32, [P, i32]),
        "vla_octo_tf_readout_index": (i32, [P, i32]),
        "vla_octo_tf_config": (i32, [P, P]),
        "vla_octo_tf_int8_layers": (i32, [P]),
        "vla_octo_tf_graph_nodes": (i32, [P]),
        "vla_octo_tf_forward": (i32, [P, P, P, P, i32, P, P]),
        "vla_octo_tf_forward_dev": (i32, [P, P, P, P, i32, P, P, P]),
        "vla_smolvla_tf_load": (P, [c_char_p, i32]),
        "vla_smolvla_tf_free": (None, [P]),
        "vla_smolvla_tf_chunk": (i32, [P]),
        "vla_smolvla_tf_max_action_dim": (i32, [P]),
        "vla_smolvla_tf_hidden": (i32, [P]),
        "vla_smolvla_tf_int8_layers": (i32, [P]),
        "vla_smolvla_tf_graph_nodes": (i32, [P]),
        "vla_smolvla_tf_chunk_run": (i32, [P, P, P, i32, P, P]),
        "vla_smolvla_tf_chunk_dev": (i32, [P, P, P, i32, P, P, P]),
        "vla_siglip_tf_load": (P, [c_char_p, i32]),
        "vla_siglip_tf_free": (None, [P]),
        "vla_siglip_tf_img": (i32, [P]),
        "vla_siglip_tf_n_tokens": (i32, [P]),
        "vla_siglip_tf_out_dim": (i32, [P]),
        "vla_siglip_tf_int8_layers": (i32, [P]),
        "vla_siglip_tf_graph_nodes": (i32, [P]),
        "vla_siglip_tf_encode": (i32, [P, P, P]),
        "vla_siglip_tf_encode_dev": (i32, [P, P, P, P]),
        "vla_act_load": (P, [c_char_p]),
        "vla_act_free": (None, [P]),
        "vla_act_chunk": (i32, [P]),
        "vla_act_action_dim": (i32, [P]),
        "vla_act_state_dim": (i32, [P]),
        "vla_act_n_cams": (i32, [P]),
        "vla_act_img_h": (i32, [P]),
        "vla_act_img_w": (i32, [P]),
        "vla_act_predict": (i32, [P, P, P, i32, P]),
        "vla_act_predict_dev": (i32, [P, P, P, i32, P, P]),
        "vla_act_encode": (i32, [P, P, P]),
        "vla_act_encode_dev": (i32, [P, P, P, P]),
        "vla_act_feat_shape": (i32, [P, P, P, P]),
        "vla_act_int8_convs": (i32, [P]),
        "vla_act_int8_layers": (i32, [P]),
        "vla_act_graph_nodes": (i32, [P]),
        "vla_impact_load": (P, [c_char_p]),
        "vla_impact_free": (None, [P]),
        "vla_impact_chunk": (i32, [P]),
        "vla_impact_action_dim": (i32, [P]),
        "vla_impact_state_dim": (i32, [P]),
        "vla_impact_n_cams": (i32, [P]),
        "vla_impact_img_h": (i32, [P]),
        "vla_impact_img_w": (i32, [P]),
        "vla_impact_n_text": (i32, [P]),
        "vla_impact_set_instruction": (i32, [P, c_char_p]),
        "vla_impact_predict": (i32, [P, P, P, c_char_p, i32, P]),
        "vla_impact_tokens": (i32, [P, P, P, P, i32]),
        "vla_impact_film": (i32, [P, P, P, i32]),
        "vla_impact_predict_dev": (i32, [P, P, P, i32, P, P]),
        "vla_impact_int8_layers": (i32, [P]),
        "vla_impact_int8_convs": (i32, [P]),
        "vla_diffusion_load": (P, [c_char_p]),
        "vla_diffusion_free": (None, [P]),
        **{f"vla_diffusion_{k}": (i32, [P]) for k in (
            "chunk", "horizon", "action_dim", "state_dim", "n_cams", "n_obs_steps", "img_h", "img_w", "num_steps",
            "is_ddim", "int8_layers", "int8_convs", "graph_nodes")},
        "vla_diffusion_predict": (i32, [P, P, P, i32, P, P]),
        "vla_smolvla_load": (P, [c_char_p, c_char_p]),
        "vla_smolvla_free": (None, [P]),
        "vla_smolvla_chunk": (i32, [P]),
        "vla_smolvla_action_dim": (i32, [P]),
        "vla_smolvla_state_dim": (i32, [P]),
        "vla_smolvla_n_views": (i32, [P]),
        "vla_smolvla_img_size": (i32, [P]),
        "vla_smolvla_tok_maxlen": (i32, [P]),
        "vla_smolvla_int8_layers": (i32, [P]),
        "vla_smolvla_graph_nodes": (i32, [P]),
        "vla_smolvla_tokenize": (i32, [P, c_char_p, P, P]),
        "vla_smolvla_predict": (i32, [P, P, i32, i32, i32, P, P, i32, P, P, ctypes.c_uint64, P]),
        "vla_smolvla_predict_rtc": (i32, [P, P, i32, i32, i32, P, P, i32, P, P, ctypes.c_uint64, P, P, i32, P,
                                          c_float]),
        "vla_smolvla_preprocess": (i32, [P, P, i32, i32, i32, P]),
        "vla_bpe_load": (P, [c_char_p]),
        "vla_bpe_free": (None, [P]),
        "vla_bpe_encode": (i32, [P, c_char_p, P, i32]),
        "vla_octo_load": (P, [c_char_p, c_char_p]),
        "vla_octo_free": (None, [P]),
        "vla_octo_horizon": (i32, [P]),
        "vla_octo_action_dim": (i32, [P]),
        "vla_octo_max_window": (i32, [P]),
        "vla_octo_int8_layers": (i32, [P]),
        "vla_octo_predict": (i32, [P, P, P, i32, P, c_char_p, ctypes.c_uint64, i32, P]),
        "vla_octo_predict_ex": (i32, [P, P, P, i32, P, c_char_p, P, P, ctypes.c_uint64, i32, P]),
        "vla_octo_lang": (i32, [P, c_char_p, P, i64]),
        "vla_unigram_load": (P, [c_char_p]),
        "vla_unigram_free": (None, [P]),
        "vla_unigram_encode": (i32, [P, c_char_p, i32, P]),
        "vla_probe_begin": (i32, [i32]),
        "vla_probe_end": (i32, []),
        "vla_probe_count": (i32, []),
        "vla_probe_shape": (i32, [i32, P]),
        "vla_probe_read": (i32, [i32, i32, P, i64]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def lib(path: str | None = None):
    """Load libvla_simd_hip.so (once). Raises if it is not built.

    PyTorch wheels for ROCm carry their own libamdhip64.so.7. Whichever copy a
    process loads first serves every later library with that soname, so torch
    is imported (when installed) before this library: the process then holds a
    single HIP runtime and torch's device pointers and streams are valid here.
    """
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        p = path or os.environ.get("VLA_SIMD_HIP_LIB", LIB_PATH)
        if not os.path.exists(p):
            raise RuntimeError(f"{p} is not built: run __graft_entry__.build() (make -C vla.simd_amd/csrc)")
        L = ctypes.CDLL(p)
        _declare(L)
        _lib = L
    return _lib


def check(fn: str, status: int) -> None:
    if status != VLA_OK:
        raise VlaError(fn, status, (lib().vla_last_error() or b"").decode(errors="replace"))


def _call(name: str, *args) -> int:
    st = getattr(lib(), name)(*args)
    check(name, st)
    return st


def _ptr(a):
    if a is None:
        return None
    return a.ctypes.data_as(c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i8(a):
    return np.ascontiguousarray(a, dtype=np.int8)


# ------------------------------------------------------------- handshake --

def abi_version() -> int:
    return lib().vla_abi_version()


def backend_name() -> str:
    return lib().vla_backend_name().decode()


def int8_available() -> bool:
    return bool(lib().vla_int8_available())


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    _call("vla_hip_device_name", buf, 256)
    return buf.value.decode()


def i8_kpad(K: int) -> int:
    return (K + 3) & ~3


# ------------------------------------------------- host-pointer op forms --

def quantize_act_i8(x):
    """tcpu::quantize_act_i8: x [seq, K] -> (xq [seq, i8_kpad(K)] int8, ascale [seq])."""
    x = _f32(x)
    seq, K = x.shape
    xq = np.empty((seq, i8_kpad(K)), np.int8)
    s = np.empty(seq, np.float32)
    _call("vla_quantize_act_i8", _ptr(x), _ptr(xq), _ptr(s), seq, K)
    return xq, s


def pack_weights_i8(W):
    """tcpu::pack_weights_i8 formula, device row layout: W [N,K] -> (Wq [N, Kp], wscale [N])."""
    W = _f32(W)
    N, K = W.shape
    Wq = np.empty((N, i8_kpad(K)), np.int8)
    s = np.empty(N, np.float32)
    _call("vla_pack_weights_i8", _ptr(W), _ptr(Wq), _ptr(s), N, K)
    return Wq, s


def _pad_rows(a, Kp):
    a = _i8(a)
    if a.shape[1] == Kp:
        return a
    out = np.zeros((a.shape[0], Kp), np.int8)
    out[:, : a.shape[1]] = a
    return out


def dense_linear_i8_pre(xq, ascale, Wq, wscale, bias, K):
    """tcpu::dense_linear_i8_pre with row-major Wq [N, K or Kp]."""
    Kp = i8_kpad(K)
    xq, Wq = _pad_rows(xq, Kp), _pad_rows(Wq, Kp)
    seq, N = xq.shape[0], Wq.shape[0]
    ascale, wscale = _f32(ascale), _f32(wscale)
    b = None if bias is None else _f32(bias)
    out = np.empty((seq, N), np.float32)
    _call("vla_dense_linear_i8_pre", _ptr(out), _ptr(xq), _ptr(ascale), _ptr(Wq), _ptr(wscale),
          _ptr(b), seq, N, K)
    return out


def dense_linear_i8(x, Wq, wscale, bias):
    """tcpu::dense_linear_i8: quantize x per row, then the int8 GEMM."""
    x = _f32(x)
    seq, K = x.shape
    Wq = _pad_rows(Wq, i8_kpad(K))
    N = Wq.shape[0]
    wscale = _f32(wscale)
    b = None if bias is None else _f32(bias)
    out = np.empty((seq, N), np.float32)
    _call("vla_dense_linear_i8", _ptr(out), _ptr(x), _ptr(Wq), _ptr(wscale), _ptr(b), seq, N, K)
    return out


def gemm_i8_i32(xq, Wq, K):
    """Exact int32 accumulators [seq, N]."""
    Kp = i8_kpad(K)
    xq, Wq = _pad_rows(xq, Kp), _pad_rows(Wq, Kp)
    seq, N = xq.shape[0], Wq.shape[0]
    acc = np.empty((seq, N), np.int32)
    _call("vla_gemm_i8_i32", _ptr(acc), _ptr(xq), _ptr(Wq), seq, N, K)
    return acc


def _mask_struct(kind=MASK_NONE, dense=None, causal_offset=0, q_group=None, k_group=None, allow=None):
    keep = []
    m = VlaMask()
    m.kind = kind
    if dense is not None:
        d = _f32(dense)
        keep.append(d)
        m.dense = d.ctypes.data
    m.causal_offset = causal_offset
    if kind == MASK_GROUPS:
        qg = np.ascontiguousarray(q_group, np.uint8)
        kg = np.ascontiguousarray(k_group, np.uint8)
        al = np.ascontiguousarray(allow, np.uint8)
        keep += [qg, kg, al]
        m.n_groups = int(round(np.sqrt(al.size)))
        m.q_group, m.k_group, m.allow = qg.ctypes.data, kg.ctypes.data, al.ctypes.data
    return m, keep


def attention(Q, K, V, n_q, n_kv, head_dim, scale, kind=MASK_NONE, dense=None, causal_offset=0,
              q_group=None, k_group=None, allow=None):
    """Fused attention, host arrays. Q [seq_q, n_q*hd], K/V [seq_k, n_kv*hd]."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    sq = Q.size // (n_q * head_dim)
    sk = K.size // (n_kv * head_dim)
    out = np.empty((sq, n_q * head_dim), np.float32)
    m, keep = _mask_struct(kind, dense, causal_offset, q_group, k_group, allow)
    _call("vla_attention", _ptr(out), _ptr(Q), _ptr(K), _ptr(V), sq, sk, n_q, n_kv, head_dim,
          float(scale), ctypes.byref(m))
    del keep
    return out


def gqa_attention_masked(Q, K, V, seq_q, seq_k, n_q, n_kv, head_dim, scale, mask):
    """tcpu::gqa_attention_masked (mask [seq_q, seq_k] additive or None)."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    out = np.empty((seq_q, n_q * head_dim), np.float32)
    m = None if mask is None else _f32(mask)
    _call("vla_gqa_attention_masked", _ptr(out), _ptr(Q), _ptr(K), _ptr(V), seq_q, seq_k, n_q,
          n_kv, head_dim, float(scale), _ptr(m))
    return out


def gqa_attention_dense(Q, K, V, seq_q, seq_k, n_q, n_kv, head_dim, scale):
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    out = np.empty((seq_q, n_q * head_dim), np.float32)
    _call("vla_gqa_attention_dense", _ptr(out), _ptr(Q), _ptr(K), _ptr(V), seq_q, seq_k, n_q,
          n_kv, head_dim, float(scale))
    return out


def layernorm(x, w, b, eps):
    x = _f32(x).copy()
    seq, H = x.shape
    bb = None if b is None else _f32(b)
    _call("vla_layernorm", _ptr(x), _ptr(x), _ptr(_f32(w)), _ptr(bb), seq, H, float(eps))
    return x


def rmsnorm(x, w, eps):
    x = _f32(x).copy()
    seq, H = x.shape
    _call("vla_rmsnorm", _ptr(x), _ptr(x), _ptr(_f32(w)), seq, H, float(eps))
    return x


def rope_neox(x, pos, n_heads, head_dim, base):
    x = _f32(x).copy()
    p = np.ascontiguousarray(pos, np.int32)
    _call("vla_rope_neox", _ptr(x), _ptr(p), len(p), n_heads, head_dim, float(base))
    return x


def _eltwise(name, x):
    x = _f32(x).copy()
    _call(name, _ptr(x), x.size)
    return x


def gelu_tanh(x):
    return _eltwise("vla_gelu_tanh", x)


def gelu_erf(x):
    return _eltwise("vla_gelu_erf", x)


def relu(x):
    return _eltwise("vla_relu", x)


def silu_gate(g, u):
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    _call("vla_silu_gate", _ptr(out), _ptr(g), _ptr(u), g.size)
    return out


# ------------------------------------------- device forms (torch tensors) --

def _dp(t):
    return None if t is None else c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        return c_void_p(torch.cuda.current_stream().cuda_stream)
    return c_void_p(stream)


def quantize_act_i8_dev(x, xq, ascale, stream=None):
    seq, K = x.shape
    _call("vla_quantize_act_i8_dev", _dp(x), _dp(xq), xq.shape[1], _dp(ascale), seq, K,
          _stream(stream))


def dense_linear_i8_pre_dev(out, xq, ascale, Wq, wscale, bias, K, act=0, accumulate=0, stream=None):
    seq, N = out.shape[0], Wq.shape[0]
    _call("vla_dense_linear_i8_pre_dev", _dp(out), out.stride(0), _dp(xq), xq.stride(0),
          _dp(ascale), _dp(Wq), Wq.stride(0), _dp(wscale), _dp(bias), seq, N, K, act, accumulate,
          _stream(stream))


def quantize_span_i8(x, inv):
    """tcpu::quantize_span_i8: clamp(rne(x * inv), +-127) with one shared inverse scale."""
    x = _f32(x)
    q = np.empty(x.shape, np.int8)
    _call("vla_quantize_span_i8", _ptr(x), _ptr(q), x.size, float(inv))
    return q


def dense_linear_i8_dev(out, x, Wq, wscale, bias, K, xq_scratch, ascale_scratch, act=0, accumulate=0,
                        stream=None):
    """tcpu::dense_linear_i8 on device tensors with the caller-owned scratch the
    reference takes: xq_scratch [seq, ldq >= i8_kpad(K)] int8, ascale_scratch [seq]."""
    seq, N = out.shape[0], Wq.shape[0]
    _call("vla_dense_linear_i8_dev", _dp(out), out.stride(0), _dp(x), x.stride(0), _dp(Wq), Wq.stride(0),
          _dp(wscale), _dp(bias), seq, N, K, _dp(xq_scratch), xq_scratch.stride(0), _dp(ascale_scratch),
          act, accumulate, _stream(stream))


def dense_linear_i8_noalloc_dev(out, x, Wq, wscale, bias, K, act=0, accumulate=0, stream=None):
    """dense_linear_i8_dev with the library's fixed device scratch instead of
    caller scratch: allocates nothing. Calls that overlap on one GPU race."""
    seq, N = out.shape[0], Wq.shape[0]
    _call("vla_dense_linear_i8_noalloc_dev", _dp(out), out.stride(0), _dp(x), x.stride(0), _dp(Wq),
          Wq.stride(0), _dp(wscale), _dp(bias), seq, N, K, act, accumulate, _stream(stream))


def i8_panel_bytes(seq: int, K: int) -> int:
    """Bytes of the panel layout of [seq, K] int8 activations (seq <= 128)."""
    return int(lib().vla_i8_panel_bytes(seq, K))


def quantize_act_i8_panel_dev(x, xq, ascale, stream=None):
    """quantize_act_i8 of x [seq, K] into the panel layout (xq: >= i8_panel_bytes bytes)."""
    seq, K = x.shape
    _call("vla_quantize_act_i8_panel_dev", _dp(x), x.stride(0), _dp(xq), _dp(ascale), seq, K,
          _stream(stream))


def dense_linear_i8_panel_dev(out, xq, ascale, Wq, wscale, bias, K, act=0, accumulate=0, stream=None):
    """dense_linear_i8_pre_dev with panel-layout activations (seq = out rows <= 128)."""
    seq, N = out.shape[0], Wq.shape[0]
    _call("vla_dense_linear_i8_panel_dev", _dp(out), out.stride(0), _dp(xq), _dp(ascale), _dp(Wq),
          Wq.stride(0), _dp(wscale), _dp(bias), seq, N, K, act, accumulate, _stream(stream))


def dense_linear_i8_panel_split_dev(out, xq, ascale, Wq, wscale, bias, K, work, act=0, accumulate=0,
                                    stream=None):
    """dense_linear_i8_panel_dev with a split-K workspace (a device byte tensor or None)."""
    seq, N = out.shape[0], Wq.shape[0]
    nbytes = 0 if work is None else work.numel() * work.element_size()
    _call("vla_dense_linear_i8_panel_split_dev", _dp(out), out.stride(0), _dp(xq), _dp(ascale), _dp(Wq),
          Wq.stride(0), _dp(wscale), _dp(bias), seq, N, K, act, accumulate, _dp(work), nbytes,
          _stream(stream))


ROWOP_IDENTITY, ROWOP_RMSNORM, ROWOP_SILU_GATE = 0, 2, 3


def rowop_quantize_i8_panel_dev(op, x, xq, ascale, u=None, w=None, eps=0.0, stream=None):
    """op(x) quantized into the panel layout: op 0 identity, 2 RMSNorm(w, eps),
    3 silu_gate(x, u); x and u are [seq, K] fp32 views (row-strided)."""
    seq, K = x.shape
    _call("vla_rowop_quantize_i8_panel_dev", op, _dp(x), x.stride(0), _dp(u), u.stride(0) if u is not None else 0,
          _dp(w), float(eps), _dp(xq), _dp(ascale), seq, K, _stream(stream))


def rowop_linear_i8_fits(op: int, seq: int, K: int) -> bool:
    """Whether rowop_linear_i8_dev supports this row op and shape."""
    return bool(lib().vla_rowop_linear_i8_fits(op, seq, K))


def rowop_linear_i8_dev(out, op, x, Wq, wscale, bias, u=None, w=None, eps=0.0, act=0, accumulate=0,
                        stream=None):
    """out (+)= the int8 linear of op(x) (rowop_quantize_i8_panel_dev, then
    dense_linear_i8_panel_dev) in one kernel; out [seq, N] must not overlap x or u."""
    seq, K = x.shape
    N = Wq.shape[0]
    _call("vla_rowop_linear_i8_dev", _dp(out), out.stride(0), op, _dp(x), x.stride(0), _dp(u),
          u.stride(0) if u is not None else 0, _dp(w), float(eps), _dp(Wq), Wq.stride(0), _dp(wscale),
          _dp(bias), seq, N, K, act, accumulate, _stream(stream))


def gemm_i8_i32_dev(acc, xq, Wq, K, stream=None):
    seq, N = acc.shape
    _call("vla_gemm_i8_i32_dev", _dp(acc), _dp(xq), xq.stride(0), _dp(Wq), Wq.stride(0), seq, N,
          K, _stream(stream))


def attention_dev(out, Q, K, V, n_q, n_kv, head_dim, scale, mask: VlaMask | None = None,
                  stream=None):
    _call("vla_attention_dev", _dp(out), out.stride(0), _dp(Q), Q.stride(0), _dp(K), K.stride(0),
          _dp(V), V.stride(0), Q.shape[0], K.shape[0], n_q, n_kv, head_dim, float(scale),
          None if mask is None else ctypes.byref(mask), _stream(stream))


class LinearI8:
    """Device-resident int8 linear (vla_linear_i8_*)."""

    def __init__(self, handle, N, K):
        self.h = c_void_p(handle)
        self.N, self.K = N, K
        self.ldw = lib().vla_linear_i8_ldw(self.h)

    @classmethod
    def from_f32(cls, W, bias=None):
        W = _f32(W)
        N, K = W.shape
        b = None if bias is None else _f32(bias)
        h = lib().vla_linear_i8_create(_ptr(W), _ptr(b), N, K)
        if not h:
            raise VlaError("vla_linear_i8_create", VLA_ERR_ARG, lib().vla_last_error().decode())
        return cls(h, N, K)

    @classmethod
    def from_i8(cls, Wq, wscale, bias=None):
        Wq = _i8(Wq)
        N, K = Wq.shape
        b = None if bias is None else _f32(bias)
        h = lib().vla_linear_i8_create_q(_ptr(Wq), _ptr(_f32(wscale)), _ptr(b), N, K)
        if not h:
            raise VlaError("vla_linear_i8_create_q", VLA_ERR_ARG, lib().vla_last_error().decode())
        return cls(h, N, K)

    def forward_dev(self, out, x, xq_scratch, ascale_scratch, act=0, accumulate=0, stream=None):
        _call("vla_linear_i8_forward_dev", self.h, _dp(out), _dp(x), x.shape[0], _dp(xq_scratch),
              _dp(ascale_scratch), act, accumulate, _stream(stream))

    def forward_quantized_dev(self, out, xq, ascale, act=0, accumulate=0, stream=None):
        _call("vla_linear_i8_forward_quantized_dev", self.h, _dp(out), _dp(xq), xq.stride(0),
              _dp(ascale), xq.shape[0], act, accumulate, _stream(stream))

    def forward(self, x):
        """Host arrays over the resident weights (vla_linear_i8_forward):
        returns (out [seq, N], the quantized rows [seq, i8_kpad(K)], their scales)."""
        x = _f32(x)
        if x.ndim != 2 or x.shape[1] != self.K:
            raise ValueError(f"x must be [seq, {self.K}], got {x.shape}")
        kp = (self.K + 3) & ~3
        out = np.empty((x.shape[0], self.N), np.float32)
        xq = np.empty((x.shape[0], kp), np.int8)
        sa = np.empty(x.shape[0], np.float32)
        _call("vla_linear_i8_forward", self.h, _ptr(out), _ptr(x), x.shape[0], _ptr(xq), kp, _ptr(sa))
        return out, xq, sa

    def forward_quantized(self, xq, ascale):
        """Host int8 rows xq [seq, >= i8_kpad(K)] and scales (vla_linear_i8_forward_quantized)."""
        xq = np.ascontiguousarray(xq, np.int8)
        out = np.empty((xq.shape[0], self.N), np.float32)
        _call("vla_linear_i8_forward_quantized", self.h, _ptr(out), _ptr(xq), xq.shape[1], _ptr(_f32(ascale)),
              xq.shape[0])
        return out

    def download(self):
        """The resident rows [N, i8_kpad(K)] and scales (vla_linear_i8_download)."""
        kp = (self.K + 3) & ~3
        Wq = np.empty((self.N, kp), np.int8)
        ws = np.empty(self.N, np.float32)
        _call("vla_linear_i8_download", self.h, _ptr(Wq), kp, _ptr(ws))
        return Wq, ws

    def set_bias(self, bias=None):
        _call("vla_linear_i8_set_bias", self.h, _ptr(None if bias is None else _f32(bias)))

    def conv2d(self, x, k, stride, pad):
        """conv2d_i8 with host x [H, W, Cin] over these resident weights (vla_conv2d_i8_resident)."""
        x = _f32(x)
        H, Wd, Cin = x.shape
        Ho, Wo = (H + 2 * pad - k) // stride + 1, (Wd + 2 * pad - k) // stride + 1
        out = np.empty((Ho, Wo, self.N), np.float32)
        _call("vla_conv2d_i8_resident", self.h, _ptr(out), _ptr(x), H, Wd, Cin, k, stride, pad)
        return out

    def close(self):
        if self.h:
            lib().vla_linear_i8_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------ fp32 linear ------

def dense_linear(x, W, bias=None):
    """tcpu::dense_linear: x [seq, K] fp32, W [N, K] -> out [seq, N]."""
    x, W = _f32(x), _f32(W)
    b = None if bias is None else _f32(bias)
    out = np.empty((x.shape[0], W.shape[0]), np.float32)
    _call("vla_dense_linear", _ptr(out), _ptr(x), _ptr(W), _ptr(b), x.shape[0], W.shape[0], W.shape[1])
    return out


def dense_linear_dev(out, x, W, bias=None, act=0, accumulate=0, alpha=1.0, stream=None):
    _call("vla_dense_linear_dev", _dp(out), out.stride(0), _dp(x), x.stride(0), _dp(W), W.stride(0),
          _dp(bias), x.shape[0], W.shape[0], W.shape[1], act, accumulate, float(alpha), _stream(stream))


# ------------------------------------------------ device policy graphs ----

class _Handle:
    _free = ""

    def __init__(self, h):
        if not h:
            raise VlaError(self._load, VLA_ERR_ARG, (lib().vla_last_error() or b"").decode())
        self.h = c_void_p(h)

    def close(self):
        if getattr(self, "h", None):
            getattr(lib(), self._free)(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def conv2d_i8(x, Wq, wscale, bias, k, stride, pad):
    """conv2d_i8 of x [H, Wd, Cin] (host arrays): Wq [Cout, i8_kpad(k*k*Cin)]
    from pack_weights_i8 -> out [Hout, Wout, Cout]."""
    x = _f32(x)
    H, Wd, Cin = x.shape
    Wq = np.ascontiguousarray(Wq, np.int8)
    Cout = Wq.shape[0]
    Ho, Wo = (H + 2 * pad - k) // stride + 1, (Wd + 2 * pad - k) // stride + 1
    out = np.empty((Ho, Wo, Cout), np.float32)
    _call("vla_conv2d_i8", _ptr(out), _ptr(x), _ptr(Wq), _ptr(_f32(wscale)), _ptr(None if bias is None else _f32(bias)),
          H, Wd, Cin, Cout, k, stride, pad)
    return out


def conv2d_i8_workspace_bytes(H, Wd, Cin, Cout, k, stride, pad) -> int:
    return int(lib().vla_conv2d_i8_workspace_bytes(H, Wd, Cin, Cout, k, stride, pad))


def gemm_i8_split_bytes(seq: int, N: int, K: int) -> int:
    """Split-K workspace bytes dense_linear_i8_pre_split_dev uses for this shape (0: unsplit)."""
    return int(lib().vla_gemm_i8_split_bytes(seq, N, K))


def dense_linear_i8_pre_split_dev(out, xq, ascale, Wq, wscale, bias, K, work, act=0, accumulate=0, stream=None):
    """dense_linear_i8_pre_dev with a split-K workspace (a device byte tensor or None)."""
    seq, N = out.shape[0], Wq.shape[0]
    nbytes = 0 if work is None else work.numel() * work.element_size()
    _call("vla_dense_linear_i8_pre_split_dev", _dp(out), out.stride(0), _dp(xq), xq.stride(0), _dp(ascale),
          _dp(Wq), Wq.stride(0), _dp(wscale), _dp(bias), seq, N, K, act, accumulate, _dp(work), nbytes,
          _stream(stream))


def conv2d_i8_dev(lin, out, x, k, stride, pad, work, stream=None):
    """Device conv2d_i8: lin a LinearI8 over [Cout, k*k*Cin], x [H, Wd, Cin] and
    out [Hout, Wout, Cout] torch tensors, work a device byte buffer."""
    H, Wd, Cin = x.shape
    _call("vla_conv2d_i8_dev", lin.h, _dp(out), _dp(x), H, Wd, Cin, k, stride, pad, _dp(work),
          work.numel() * work.element_size(), _stream(stream))


class CkptFiles(_Handle):
    """The files of a model path as the policy loaders read them (vla_ckpt_*):
    a converted directory, or a vla.simd GGUF that carries them."""

    _load, _free = "vla_ckpt_open", "vla_ckpt_free"

    def __init__(self, path: str):
        super().__init__(lib().vla_ckpt_open(str(path).encode()))

    @property
    def gguf(self) -> bool:
        return bool(lib().vla_ckpt_is_gguf(self.h))

    def names(self):
        L = lib()
        n = L.vla_ckpt_names(self.h, None, 0)
        buf = ctypes.create_string_buffer(int(n))
        L.vla_ckpt_names(self.h, buf, n)
        text = buf.value.decode()
        return text.split("\n") if text else []

    def size(self, rel: str) -> int:
        return int(lib().vla_ckpt_file_size(self.h, rel.encode()))

    def read(self, rel: str) -> bytes:
        n = self.size(rel)
        if n < 0:
            raise VlaError("vla_ckpt_read", VLA_ERR_ARG, f"no file {rel}")
        buf = ctypes.create_string_buffer(max(n, 1))
        _call("vla_ckpt_read", self.h, rel.encode(), ctypes.cast(buf, c_void_p), n)
        return buf.raw[:n]


def _need_size(name, a, n, at_least=False):
    """Raise ValueError unless array a holds n elements (at least n with at_least)."""
    size = int(np.asarray(a).size)
    if size < n if at_least else size != n:
        raise ValueError(f"{name} holds {size} values, the model reads {'at least ' if at_least else ''}{n}")


class ActTransformer(_Handle):
    """Device ACT transformer (vla_act_tf_*, ActTransformer of the reference)."""

    _load, _free = "vla_act_tf_load", "vla_act_tf_free"

    def __init__(self, dirpath: str, img_ch: int, int8_mask: int = 31, int8_state: bool = False):
        super().__init__(lib().vla_act_tf_load_ex(dirpath.encode(), img_ch, int8_mask, int(bool(int8_state))))
        L = lib()
        self.n_text = L.vla_act_tf_n_text(self.h)
        self.chunk, self.action_dim = L.vla_act_tf_chunk(self.h), L.vla_act_tf_action_dim(self.h)
        self.state_dim, self.img_ch = L.vla_act_tf_state_dim(self.h), img_ch
        self.dim = L.vla_act_tf_dim(self.h)
        self.int8_layers = L.vla_act_tf_int8_layers(self.h)

    @property
    def graph_nodes(self):
        return lib().vla_act_tf_graph_nodes(self.h)

    def _check(self, feats, n_cams, fh, fw, state):
        """The sizes the C ABI reads from the host buffers (it cannot see them)."""
        if min(n_cams, fh, fw) < 1:
            raise ValueError(f"need n_cams, fh, fw >= 1, got {n_cams}, {fh}, {fw}")
        _need_size("feats", feats, n_cams * fh * fw * self.img_ch)
        _need_size("state", state, self.state_dim)

    def forward(self, feats, n_cams, fh, fw, state):
        feats, state = _f32(feats), _f32(state)
        self._check(feats, n_cams, fh, fw, state)
        out = np.empty((self.chunk, self.action_dim), np.float32)
        _call("vla_act_tf_forward", self.h, _ptr(feats), n_cams, fh, fw, _ptr(state), _ptr(out))
        return out

    def forward_dev(self, feats, n_cams, fh, fw, state, out, stream=None):
        _call("vla_act_tf_forward_dev", self.h, _dp(feats), n_cams, fh, fw, _dp(state), _dp(out),
              _stream(stream))

    def forward_text(self, feats, n_cams, fh, fw, state, text, text_pos, n_text_real):
        """IMPACT's form: the text tail (its T5 tower's tokens and positions) after the cameras."""
        feats, state = _f32(feats), _f32(state)
        self._check(feats, n_cams, fh, fw, state)
        nt = max(0, min(int(n_text_real), self.n_text))
        text, text_pos = _f32(text), _f32(text_pos)
        _need_size("text", text, nt * self.dim, at_least=True)
        _need_size("text_pos", text_pos, nt * self.dim, at_least=True)
        out = np.empty((self.chunk, self.action_dim), np.float32)
        _call("vla_act_tf_forward_text", self.h, _ptr(feats), n_cams, fh, fw, _ptr(state), _ptr(text),
              _ptr(text_pos), int(n_text_real), _ptr(out))
        return out


class ActModel(_Handle):
    """ACT end to end on the device through the reference's own entry points
    (vla_act_load / vla_act_predict): uint8 frames + raw state -> actions."""

    _load, _free = "vla_act_load", "vla_act_free"

    def __init__(self, dirpath: str):
        super().__init__(lib().vla_act_load(dirpath.encode()))
        L = lib()
        self.chunk, self.action_dim = L.vla_act_chunk(self.h), L.vla_act_action_dim(self.h)
        self.state_dim, self.n_cams = L.vla_act_state_dim(self.h), L.vla_act_n_cams(self.h)
        self.img_h, self.img_w = L.vla_act_img_h(self.h), L.vla_act_img_w(self.h)
        fh, fw, ch = (c_int32(), c_int32(), c_int32())
        _call("vla_act_feat_shape", self.h, ctypes.byref(fh), ctypes.byref(fw), ctypes.byref(ch))
        self.feat_h, self.feat_w, self.feat_ch = fh.value, fw.value, ch.value
        self.int8_convs, self.int8_layers = L.vla_act_int8_convs(self.h), L.vla_act_int8_layers(self.h)

    @property
    def graph_nodes(self):
        return lib().vla_act_graph_nodes(self.h)

    def _check(self, images, state):
        _need_size("images", images, self.n_cams * self.img_h * self.img_w * 3)
        _need_size("state", state, self.state_dim)

    def predict(self, images, state, unnormalize=True):
        images = np.ascontiguousarray(images, np.uint8)
        state = _f32(state)
        self._check(images, state)
        out = np.empty((self.chunk, self.action_dim), np.float32)
        _call("vla_act_predict", self.h, _ptr(images), _ptr(state), int(bool(unnormalize)), _ptr(out))
        return out

    def predict_dev(self, images, state, out, unnormalize=True, stream=None):
        _call("vla_act_predict_dev", self.h, _dp(images), _dp(state), int(bool(unnormalize)), _dp(out),
              _stream(stream))

    def encode(self, images):
        images = np.ascontiguousarray(images, np.uint8)
        _need_size("images", images, self.n_cams * self.img_h * self.img_w * 3)
        out = np.empty((self.n_cams * self.feat_h * self.feat_w, self.feat_ch), np.float32)
        _call("vla_act_encode", self.h, _ptr(images), _ptr(out))
        return out

    def encode_dev(self, images, out, stream=None):
        """The backbone on device tensors: images uint8 [n_cams, img_h, img_w, 3],
        out float32 [n_cams * feat_h * feat_w, feat_ch], on the given stream."""
        n_in, n_out = self.n_cams * self.img_h * self.img_w * 3, self.n_cams * self.feat_h * self.feat_w * self.feat_ch
        if images.numel() != n_in or images.element_size() != 1 or not images.is_contiguous():
            raise ValueError(f"images: need {n_in} contiguous uint8 values on the device")
        if out.numel() != n_out or out.element_size() != 4 or not out.is_contiguous():
            raise ValueError(f"out: need {n_out} contiguous float32 values on the device")
        _call("vla_act_encode_dev", self.h, _dp(images), _dp(out), _stream(stream))


class ImpactModel(_Handle):
    """IMPACT end to end on the device through the reference's own entry points
    (vla_impact_load / _set_instruction / _predict / _tokens / _film): uint8
    frames + raw state + an instruction -> actions."""

    _load, _free = "vla_impact_load", "vla_impact_free"

    def __init__(self, dirpath: str):
        super().__init__(lib().vla_impact_load(dirpath.encode()))
        L = lib()
        self.chunk, self.action_dim = L.vla_impact_chunk(self.h), L.vla_impact_action_dim(self.h)
        self.state_dim, self.n_cams = L.vla_impact_state_dim(self.h), L.vla_impact_n_cams(self.h)
        self.img_h, self.img_w = L.vla_impact_img_h(self.h), L.vla_impact_img_w(self.h)
        self.n_text = L.vla_impact_n_text(self.h)
        self.int8_layers, self.int8_convs = L.vla_impact_int8_layers(self.h), L.vla_impact_int8_convs(self.h)

    def set_instruction(self, instruction: str):
        _call("vla_impact_set_instruction", self.h, instruction.encode())

    def predict(self, frames, state, instruction: str, unnormalize=True):
        frames = np.ascontiguousarray(frames, np.uint8)
        state = _f32(state)
        _need_size("frames", frames, self.n_cams * self.img_h * self.img_w * 3)
        _need_size("state", state, self.state_dim)
        out = np.empty((self.chunk, self.action_dim), np.float32)
        _call("vla_impact_predict", self.h, _ptr(frames), _ptr(state), instruction.encode(),
              int(bool(unnormalize)), _ptr(out))
        return out

    def predict_dev(self, frames, state, out, unnormalize=True, stream=None):
        _call("vla_impact_predict_dev", self.h, _dp(frames), _dp(state), int(bool(unnormalize)), _dp(out),
              _stream(stream))

    def tokens(self):
        """(ids, compact ids, mask) of the current instruction, [n_text] int32 each."""
        ids, comp, mask = (np.empty(self.n_text, np.int32) for _ in range(3))
        n = lib().vla_impact_tokens(self.h, _ptr(ids), _ptr(comp), _ptr(mask), self.n_text)
        if n != self.n_text:
            raise VlaError("vla_impact_tokens", n, "no instruction set")
        return ids, comp, mask

    def film(self):
        """(gamma, beta) of the current instruction, [film_total] float32 each."""
        L = lib()
        n = L.vla_impact_film(self.h, None, None, 1 << 30)  # null buffers: the count
        if n < 0:
            raise VlaError("vla_impact_film", n, "no instruction set")
        gamma, beta = np.empty(n, np.float32), np.empty(n, np.float32)
        got = L.vla_impact_film(self.h, _ptr(gamma), _ptr(beta), n)
        if got != n:
            raise VlaError("vla_impact_film", got, "copy failed")
        return gamma, beta


class DiffusionModel(_Handle):
    """Diffusion Policy end to end on the device through the reference's own
    entry points (vla_diffusion_load / _predict): an observation history of
    uint8 frames and raw states (+ the sampler's noise) -> actions."""

    _load, _free = "vla_diffusion_load", "vla_diffusion_free"

    def __init__(self, dirpath: str):
        super().__init__(lib().vla_diffusion_load(dirpath.encode()))
        L = lib()
        for k in ("chunk", "horizon", "action_dim", "state_dim", "n_cams", "n_obs_steps", "img_h", "img_w",
                  "num_steps", "int8_layers", "int8_convs"):
            setattr(self, k, getattr(L, f"vla_diffusion_{k}")(self.h))
        self.is_ddim = bool(L.vla_diffusion_is_ddim(self.h))

    @property
    def graph_nodes(self):
        return lib().vla_diffusion_graph_nodes(self.h)

    def predict(self, frames, state, noise=None, unnormalize=True):
        """frames [n_obs, n_cams, H, W, 3] uint8, state [n_obs, state_dim],
        noise [1 + num_steps, horizon, action_dim] or None -> [chunk, action_dim]."""
        frames = np.ascontiguousarray(frames, np.uint8)
        state = _f32(state)
        _need_size("frames", frames, self.n_obs_steps * self.n_cams * self.img_h * self.img_w * 3)
        _need_size("state", state, self.n_obs_steps * self.state_dim)
        if noise is not None:
            noise = _f32(noise)
            _need_size("noise", noise, (1 + self.num_steps) * self.horizon * self.action_dim)
        out = np.empty((self.chunk, self.action_dim), np.float32)
        _call("vla_diffusion_predict", self.h, _ptr(frames), _ptr(state), int(bool(unnormalize)), _ptr(out),
              None if noise is None else _ptr(noise))
        return out


class SmolvlaModel(_Handle):
    """SmolVLA end to end on the device through the reference's own entry
    points (vla_smolvla_load / _tokenize / _predict / _predict_rtc): native
    uint8 frames + language ids + raw state -> actions."""

    _load, _free = "vla_smolvla_load", "vla_smolvla_free"

    def __init__(self, dirpath: str, tok_dir: str | None = None):
        tok_dir = tok_dir or os.path.join(dirpath, "tok")
        super().__init__(lib().vla_smolvla_load(dirpath.encode(), tok_dir.encode()))
        L = lib()
        self.chunk, self.action_dim = L.vla_smolvla_chunk(self.h), L.vla_smolvla_action_dim(self.h)
        self.state_dim, self.n_views = L.vla_smolvla_state_dim(self.h), L.vla_smolvla_n_views(self.h)
        self.img_size, self.tok_maxlen = L.vla_smolvla_img_size(self.h), L.vla_smolvla_tok_maxlen(self.h)
        self.int8_layers = L.vla_smolvla_int8_layers(self.h)

    @property
    def graph_nodes(self):
        return lib().vla_smolvla_graph_nodes(self.h)

    def tokenize(self, text: str):
        ids = np.zeros(self.tok_maxlen, np.int32)
        mask = np.zeros(self.tok_maxlen, np.int32)
        n = lib().vla_smolvla_tokenize(self.h, text.encode(), _ptr(ids), _ptr(mask))
        check("vla_smolvla_tokenize", min(n, 0))
        return ids, mask, n

    def preprocess(self, frames):
        frames = np.ascontiguousarray(frames, np.uint8)
        if frames.ndim != 4 or frames.shape[3] != 3:
            raise ValueError(f"frames must be [n_views, height, width, 3], got {frames.shape}")
        out = np.empty((frames.shape[0], 3, self.img_size, self.img_size), np.float32)
        _call("vla_smolvla_preprocess", self.h, _ptr(frames), frames.shape[0], frames.shape[1], frames.shape[2],
              _ptr(out))
        return out

    def predict(self, frames, ids, mask, state, noise=None, seed=0, prev=None, weights=None, max_guidance=0.0):
        frames = np.ascontiguousarray(frames, np.uint8)
        if frames.ndim != 4 or frames.shape[3] != 3:
            raise ValueError(f"frames must be [n_views, height, width, 3], got {frames.shape}")
        ids = np.ascontiguousarray(ids, np.int32)
        mask = np.ascontiguousarray(mask, np.int32)
        if ids.shape != mask.shape or ids.ndim != 1:
            raise ValueError("ids and mask must be 1-D arrays of one length")
        state = _f32(state)
        _need_size("state", state, self.state_dim)
        if noise is not None:
            noise = _f32(noise)
        out = np.empty((self.chunk, self.action_dim), np.float32)
        args = [self.h, _ptr(frames), frames.shape[0], frames.shape[1], frames.shape[2], _ptr(ids), _ptr(mask),
                ids.size, _ptr(state), _ptr(noise), ctypes.c_uint64(seed), _ptr(out)]
        if prev is None:
            _call("vla_smolvla_predict", *args)
        else:
            prev, weights = _f32(prev), _f32(weights)
            if prev.size % self.action_dim:
                raise ValueError("prev must be [n_prev, action_dim]")
            _need_size("weights", weights, self.chunk)
            _call("vla_smolvla_predict_rtc", *args, _ptr(prev), prev.size // self.action_dim, _ptr(weights),
                  float(max_guidance))
        return out


class BpeTokenizer(_Handle):
    """SmolVLA's byte-level BPE tokenizer alone (vla_bpe_*), host code."""

    _load, _free = "vla_bpe_load", "vla_bpe_free"

    def __init__(self, tok_dir: str):
        super().__init__(lib().vla_bpe_load(tok_dir.encode()))

    def encode(self, text) -> list:
        b = text.encode() if isinstance(text, str) else bytes(text)
        n = lib().vla_bpe_encode(self.h, b, None, 0)
        check("vla_bpe_encode", min(n, 0))
        ids = np.zeros(max(n, 1), np.int32)
        lib().vla_bpe_encode(self.h, b, _ptr(ids), n)
        return [int(v) for v in ids[:n]]


class OctoModel(_Handle):
    """Octo end to end on the device through the reference's own entry points
    (vla_octo_load / vla_octo_predict / vla_octo_predict_ex): pre-resized
    uint8 frames + an instruction -> actions."""

    _load, _free = "vla_octo_load", "vla_octo_free"

    def __init__(self, dirpath: str, tok_dir: str | None = None):
        tok_dir = tok_dir or os.path.join(dirpath, "tok")
        super().__init__(lib().vla_octo_load(dirpath.encode(), tok_dir.encode()))
        L = lib()
        self.horizon, self.action_dim = L.vla_octo_horizon(self.h), L.vla_octo_action_dim(self.h)
        self.max_window, self.int8_layers = L.vla_octo_max_window(self.h), L.vla_octo_int8_layers(self.h)

    def predict(self, primary, wrist, timestep_mask, instruction: str, noise=None, z=None, seed=0,
                unnormalize=True):
        primary = np.ascontiguousarray(primary, np.uint8)
        if primary.ndim != 4 or primary.shape[1:] != (256, 256, 3):
            raise ValueError(f"primary must be [wnd, 256, 256, 3], got {primary.shape}")
        wnd = primary.shape[0]
        if wrist is not None:
            wrist = np.ascontiguousarray(wrist, np.uint8)
            if wrist.shape != (wnd, 128, 128, 3):
                raise ValueError(f"wrist must be [{wnd}, 128, 128, 3], got {wrist.shape}")
        tm = np.ascontiguousarray(timestep_mask, np.uint8)
        _need_size("timestep_mask", tm, wnd)
        out = np.empty((self.horizon, self.action_dim), np.float32)
        if (noise is None) != (z is None):
            raise ValueError("pass both noise and z, or neither")
        if noise is None:
            _call("vla_octo_predict", self.h, _ptr(primary), _ptr(wrist), wnd, _ptr(tm), instruction.encode(),
                  ctypes.c_uint64(seed), int(bool(unnormalize)), _ptr(out))
        else:
            noise, z = _f32(noise), _f32(z)
            _need_size("noise", noise, self.horizon * self.action_dim)
            if z.size % (self.horizon * self.action_dim):
                raise ValueError("z must be [steps, horizon * action_dim]")
            _call("vla_octo_predict_ex", self.h, _ptr(primary), _ptr(wrist), wnd, _ptr(tm), instruction.encode(),
                  _ptr(noise), _ptr(z), ctypes.c_uint64(seed), int(bool(unnormalize)), _ptr(out))
        return out

    def lang(self, instruction: str, n_task: int, t5_dim: int):
        out = np.empty((n_task, t5_dim), np.float32)
        _call("vla_octo_lang", self.h, instruction.encode(), _ptr(out), out.size)
        return out


class UnigramTokenizer(_Handle):
    """Octo's SentencePiece unigram tokenizer alone (vla_unigram_*), host code."""

    _load, _free = "vla_unigram_load", "vla_unigram_free"

    def __init__(self, tok_dir: str):
        super().__init__(lib().vla_unigram_load(tok_dir.encode()))

    def encode(self, text, max_len: int = 16) -> list:
        b = text.encode() if isinstance(text, str) else bytes(text)
        ids = np.zeros(max_len, np.int32)
        _call("vla_unigram_encode", self.h, b, max_len, _ptr(ids))
        return [int(v) for v in ids]


class OctoTransformer(_Handle):
    """Device Octo block transformer (vla_octo_tf_*)."""

    _load, _free = "vla_octo_tf_load", "vla_octo_tf_free"

    def __init__(self, dirpath: str, int8_mask: int = 7):
        super().__init__(lib().vla_octo_tf_load(dirpath.encode(), int8_mask))
        self.d = lib().vla_octo_tf_dim(self.h)
        self.int8_layers = lib().vla_octo_tf_int8_layers(self.h)
        cfg = np.zeros(7, np.int32)
        _call("vla_octo_tf_config", self.h, _ptr(cfg))
        (_, self.n_task, self.t5_dim, self.stem_dim, self.tok_primary, self.tok_wrist,
         self.max_horizon) = (int(v) for v in cfg)

    def _check(self, t5, stem_p, stem_w, wnd, tm):
        if not 1 <= wnd <= self.max_horizon:
            raise ValueError(f"wnd must be in [1, {self.max_horizon}], got {wnd}")
        _need_size("timestep_mask", tm, wnd, at_least=True)
        _need_size("t5", t5, self.n_task * self.t5_dim)
        _need_size("stem_p", stem_p, wnd * self.tok_primary * self.stem_dim)
        if stem_w is not None:
            _need_size("stem_w", stem_w, wnd * self.tok_wrist * self.stem_dim)

    @property
    def graph_nodes(self):
        return lib().vla_octo_tf_graph_nodes(self.h)

    def total_tokens(self, wnd):
        return lib().vla_octo_tf_total_tokens(self.h, wnd)

    def readout_index(self, wnd):
        return lib().vla_octo_tf_readout_index(self.h, wnd)

    def forward(self, t5, stem_p, stem_w, wnd, tmask):
        t5, stem_p = _f32(t5), _f32(stem_p)
        stem_w = None if stem_w is None else _f32(stem_w)
        tm = np.ascontiguousarray(tmask, dtype=np.uint8)
        self._check(t5, stem_p, stem_w, wnd, tm)
        out = np.empty(self.d, np.float32)
        _call("vla_octo_tf_forward", self.h, _ptr(t5), _ptr(stem_p), _ptr(stem_w), wnd, _ptr(tm),
              _ptr(out))
        return out

    def forward_dev(self, t5, stem_p, stem_w, wnd, tmask, out, stream=None):
        tm = np.ascontiguousarray(tmask, dtype=np.uint8)
        _call("vla_octo_tf_forward_dev", self.h, _dp(t5), _dp(stem_p), _dp(stem_w), wnd, _ptr(tm),
              _dp(out), _stream(stream))


class SmolvlaChunk(_Handle):
    """Device SmolVLA action chunk: text-tower prefix + expert denoise (vla_smolvla_tf_*)."""

    _load, _free = "vla_smolvla_tf_load", "vla_smolvla_tf_free"

    def __init__(self, dirpath: str, int8_mask: int = 48):
        super().__init__(lib().vla_smolvla_tf_load(dirpath.encode(), int8_mask))
        L = lib()
        self.chunk, self.max_action_dim = L.vla_smolvla_tf_chunk(self.h), L.vla_smolvla_tf_max_action_dim(self.h)
        self.hidden = L.vla_smolvla_tf_hidden(self.h)
        self.int8_layers = L.vla_smolvla_tf_int8_layers(self.h)

    @property
    def graph_nodes(self):
        return lib().vla_smolvla_tf_graph_nodes(self.h)

    def _check(self, prefix, pad, noise):
        if prefix.ndim != 2 or prefix.shape[1] != self.hidden:
            raise ValueError(f"prefix must be [n_prefix, {self.hidden}], got {prefix.shape}")
        _need_size("pad", pad, prefix.shape[0])
        _need_size("noise", noise, self.chunk * self.max_action_dim)

    def run(self, prefix, pad, noise):
        prefix, noise = _f32(prefix), _f32(noise)
        pad = np.ascontiguousarray(pad, dtype=np.int32)
        self._check(prefix, pad, noise)
        out = np.empty((self.chunk, self.max_action_dim), np.float32)
        _call("vla_smolvla_tf_chunk_run", self.h, _ptr(prefix), _ptr(pad), prefix.shape[0], _ptr(noise),
              _ptr(out))
        return out

    def run_dev(self, prefix, pad, noise, out, stream=None):
        pad = np.ascontiguousarray(pad, dtype=np.int32)
        _call("vla_smolvla_tf_chunk_dev", self.h, _dp(prefix), _ptr(pad), prefix.shape[0], _dp(noise),
              _dp(out), _stream(stream))


class SiglipVision(_Handle):
    """Device SigLIP vision tower + connector of SmolVLA (vla_siglip_tf_*)."""

    _load, _free = "vla_siglip_tf_load", "vla_siglip_tf_free"

    def __init__(self, dirpath: str, int8_mask: int = 15):
        super().__init__(lib().vla_siglip_tf_load(dirpath.encode(), int8_mask))
        L = lib()
        self.img, self.n_tokens = L.vla_siglip_tf_img(self.h), L.vla_siglip_tf_n_tokens(self.h)
        self.out_dim = L.vla_siglip_tf_out_dim(self.h)
        self.int8_layers = L.vla_siglip_tf_int8_layers(self.h)

    @property
    def graph_nodes(self):
        return lib().vla_siglip_tf_graph_nodes(self.h)

    def encode(self, pixels):
        pixels = _f32(pixels)
        if pixels.shape != (3, self.img, self.img):
            raise ValueError(f"pixels must be [3, {self.img}, {self.img}]")
        out = np.empty((self.n_tokens, self.out_dim), np.float32)
        _call("vla_siglip_tf_encode", self.h, _ptr(pixels), _ptr(out))
        return out

    def encode_dev(self, pixels, out, stream=None):
        _call("vla_siglip_tf_encode_dev", self.h, _dp(pixels), _dp(out), _stream(stream))


# ------------------------------------------------------ int8-step probe --

_PROBE_FIELDS = {"src": (0, np.float32, "MK"), "xq": (1, np.int8, "MK"), "ascale": (2, np.float32, "M"),
                 "before": (3, np.float32, "MN"), "after": (4, np.float32, "MN"), "W": (5, np.int8, "NK"),
                 "wscale": (6, np.float32, "N"), "bias": (7, np.float32, "N")}


def probe_records(run, max_records=512):
    """Runs run() with the int8-step probe on; returns one dict per int8 GEMM
    the pass ran (M, K, N, act, acc and the arrays of _PROBE_FIELDS)."""
    _call("vla_probe_begin", max_records)
    try:
        run()
        recs = []
        for i in range(int(lib().vla_probe_count())):
            sh = np.zeros(7, np.int32)
            _call("vla_probe_shape", i, _ptr(sh))
            M, K, N, act, acc, has_bias, has_src = (int(v) for v in sh)
            r = dict(M=M, K=K, N=N, act=act, acc=acc)
            dims = {"M": M, "K": K, "N": N}
            for name, (what, dt, shape) in _PROBE_FIELDS.items():
                if (name == "bias" and not has_bias) or (name == "src" and not has_src):
                    r[name] = None
                    continue
                a = np.empty(tuple(dims[c] for c in shape), dt)
                _call("vla_probe_read", i, what, _ptr(a), a.nbytes)
                r[name] = a
            recs.append(r)
        return recs
    finally:
        _call("vla_probe_end")
