"""ctypes bindings of the CPU checker. TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg. Two libraries, both built by oracle/Makefile:

  liboracle.so          this repo's C restatement (oracle.c)
  _ref/libvla_ref.so    the real reference kernels + ref_shim.cpp (built in the
                        container that holds the reference sources; the .so
                        travels with the tree)
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_size_t, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libvla_ref.so")

_orc = None
_ref = None


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def kpad(K: int) -> int:
    return (K + 3) & ~3


def oracle():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError(f"{ORACLE_PATH} missing: run make -C oracle")
        L = ctypes.CDLL(ORACLE_PATH)
        P, i, f = c_void_p, c_int, c_float
        L.orc_i8_kpad.argtypes, L.orc_i8_kpad.restype = [i], i
        L.orc_frand_fill.argtypes = [ctypes.POINTER(c_uint64), P, c_size_t, f, f]
        L.orc_quantize_act_i8.argtypes = [P, P, P, i, i, i]
        L.orc_quantize_weights_i8.argtypes = [P, P, P, i, i, i]
        L.orc_gemm_i8_acc.argtypes = [P, P, i, P, i, i, i, i]
        L.orc_dense_linear_i8_pre.argtypes = [P, P, i, P, P, i, P, P, i, i, i]
        L.orc_apply_act.argtypes = [P, c_size_t, i]
        L.orc_gqa_attention_masked.argtypes = [P, P, P, P, i, i, i, i, i, f, P]
        L.orc_layernorm.argtypes = [P, P, P, P, i, i, f]
        L.orc_rmsnorm.argtypes = [P, P, P, i, i, f]
        L.orc_rope_neox.argtypes = [P, P, i, i, i, f]
        L.orc_gelu_tanh.argtypes = [P, c_size_t]
        L.orc_gelu_erf.argtypes = [P, c_size_t]
        L.orc_silu_gate.argtypes = [P, P, P, c_size_t]
        L.orc_relu.argtypes = [P, c_size_t]
        L.orc_quantize_tensor_i8.argtypes, L.orc_quantize_tensor_i8.restype = [P, P, c_size_t, f], f
        L.orc_im2col_i8.argtypes = [P, i, P, i, i, i, i, i, i]
        L.orc_conv2d_i8.argtypes = [P, P, P, i, P, P, i, i, i, i, i, i, i, f]
        _orc = L
    return _orc


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_PATH} missing: run make -C oracle ref (needs the reference sources)")
        L = ctypes.CDLL(REF_PATH)
        P, i, f = c_void_p, c_int, c_float
        L.ref_int8_available.restype = i
        L.ref_backend_name.restype = ctypes.c_char_p
        L.ref_omp_max_threads.restype = i
        L.ref_i8_kpad.argtypes, L.ref_i8_kpad.restype = [i], i
        L.ref_packed_i8_words.argtypes, L.ref_packed_i8_words.restype = [i, i], c_size_t
        L.ref_pack_weights_i8.argtypes = [P, P, P, i, i]
        L.ref_panels_from_rows.argtypes = [P, i, i, i, P]
        L.ref_rows_from_panels.argtypes = [P, i, i, P, i]
        L.ref_quantize_act_i8.argtypes = [P, P, P, i, i]
        L.ref_dense_linear_i8.argtypes = [P, P, P, P, P, i, i, i, P, P]
        L.ref_dense_linear_i8_pre.argtypes = [P, P, P, P, P, P, i, i, i]
        L.ref_dense_linear_i8_ref.argtypes = [P, P, P, P, P, P, i, i, i]
        L.ref_gqa_attention_masked.argtypes = [P, P, P, P, i, i, i, i, i, f, P]
        L.ref_gqa_attention_dense.argtypes = [P, P, P, P, i, i, i, i, i, f]
        L.ref_layernorm.argtypes = [P, P, P, P, i, i, f]
        L.ref_rmsnorm.argtypes = [P, P, P, i, i, f]
        L.ref_rope_neox.argtypes = [P, P, i, i, i, f]
        L.ref_gelu_tanh.argtypes = [P, i]
        L.ref_gelu_erf.argtypes = [P, i]
        L.ref_silu_gate.argtypes = [P, P, P, i]
        L.ref_relu.argtypes = [P, i]
        L.ref_dense_linear.argtypes = [P, P, P, P, i, i, i]
        L.ref_conv2d_i8.argtypes = [P, P, P, P, i, i, i, i, i, i, i]
        L.ref_conv2d_i8_packed.argtypes = [P, P, P, P, P, i, i, i, i, i, i, i]
        _ref = L
    return _ref


# -------------------------------------- the reference's nn on two backends --

REF_HIP_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libvla_ref_hip.so")
_nn_libs = {}


def ref_hip_available() -> bool:
    return os.path.exists(REF_HIP_PATH)


def ref_nn(backend: str):
    """The reference's own nn::Linear / MhaQKV driven by oracle/ref_nn_shim.cpp,
    on its CPU op backend ("cpu": _ref/libvla_ref.so) or on
    vla.simd_amd/hal/ops_hip.cpp over libvla_simd_hip.so ("hip":
    _ref/libvla_ref_hip.so; load the vla package first so one HIP runtime and
    one copy of libvla_simd_hip.so serve the process)."""
    if backend not in _nn_libs:
        L = ref() if backend == "cpu" else ctypes.CDLL(REF_HIP_PATH)
        P, i = c_void_p, c_int
        L.ref_nn_linear_forward.argtypes = [P, P, i, i, i, P, i, P]
        L.ref_nn_linear_forward.restype = i
        L.ref_nn_mha_forward.argtypes = [i, i, P, P, i, P, P, P, i, i, P, P, P, P]
        L.ref_nn_mha_forward.restype = i
        L.ref_nn_pre_vs_ref.argtypes = [P, i, i, P, i, P, P, P]
        L.ref_nn_pre_vs_ref.restype = i
        L.ref_unet_load.argtypes, L.ref_unet_load.restype = [ctypes.c_char_p, P, i, P], P
        L.ref_unet_free.argtypes = [P]
        L.ref_unet_forward.argtypes, L.ref_unet_forward.restype = [P, P, P, P, i], i
        L.ref_nn_linear_load.argtypes, L.ref_nn_linear_load.restype = [P, P, i, i, i, P], P
        L.ref_nn_linear_run.argtypes, L.ref_nn_linear_run.restype = [P, P, P, P, i, P], i
        L.ref_nn_linear_free.argtypes = [P]
        L.ref_nn_mha_load.argtypes, L.ref_nn_mha_load.restype = [i, i, P, P, i], P
        L.ref_nn_mha_run.argtypes, L.ref_nn_mha_run.restype = [P, P, P, P, i, i, P], i
        L.ref_nn_mha_free.argtypes = [P]
        L.ref_nn_conv_load.argtypes, L.ref_nn_conv_load.restype = [P, P, i, i, i, i, P], P
        L.ref_nn_conv_run.argtypes, L.ref_nn_conv_run.restype = [P, P, i, i, i, i, P], i
        L.ref_nn_conv_free.argtypes = [P]
        _nn_libs[backend] = L
    return _nn_libs[backend]


def nn_linear_forward(backend, W, b, x, int8=1):
    W, x = _f32(W), _f32(x)
    N, K = W.shape
    out = np.empty((x.shape[0], N), np.float32)
    q = ref_nn(backend).ref_nn_linear_forward(_p(W), _p(None if b is None else _f32(b)), N, K, int8, _p(x),
                                              x.shape[0], _p(out))
    if q < 0:
        raise RuntimeError("ref_nn_linear_forward failed")
    return out, bool(q)


def nn_mha_forward(backend, dim, heads, W, b, xq, xk, xv, rows, seq_kv, int8=1):
    """MhaQKV.forward(out, xq, xk, xv, rows, seq_kv): pass the same array object
    for aliased inputs (the shared-quantization branches key on pointer
    equality). Returns out, q, k, v."""
    out = np.empty((rows, dim), np.float32)
    q = np.empty((rows, dim), np.float32)
    k = np.zeros((seq_kv, dim), np.float32)
    v = np.empty((seq_kv, dim), np.float32)
    st = ref_nn(backend).ref_nn_mha_forward(dim, heads, _p(W), _p(b), int8, _p(xq), _p(xk), _p(xv), rows, seq_kv,
                                           _p(out), _p(q), _p(k), _p(v))
    if st != 0:
        raise RuntimeError("ref_nn_mha_forward failed")
    return out, q, k, v


class NnLinear:
    """A reference nn::Linear kept across calls on one op backend."""

    def __init__(self, backend, W, b, int8=1):
        self.L = ref_nn(backend)
        self.W, self.N, self.K = _f32(W), W.shape[0], W.shape[1]
        q = np.zeros(1, np.int32)
        self.h = self.L.ref_nn_linear_load(_p(self.W), _p(None if b is None else _f32(b)), self.N, self.K,
                                           int(int8), _p(q))
        if not self.h:
            raise RuntimeError("ref_nn_linear_load failed")
        self.int8 = bool(q[0])

    def forward(self, x):
        x = _f32(x)
        out = np.empty((x.shape[0], self.N), np.float32)
        if self.L.ref_nn_linear_run(self.h, _p(x), None, None, x.shape[0], _p(out)) != 0:
            raise RuntimeError("ref_nn_linear_run failed")
        return out

    def forward_quantized(self, xq, scales):
        xq = np.ascontiguousarray(xq, np.int8)
        out = np.empty((xq.shape[0], self.N), np.float32)
        if self.L.ref_nn_linear_run(self.h, None, _p(xq), _p(_f32(scales)), xq.shape[0], _p(out)) != 0:
            raise RuntimeError("ref_nn_linear_run failed")
        return out

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_nn_linear_free(self.h)


class NnMha:
    """A reference nn::MhaQKV (four dim x dim projections sharing W, b) kept
    across calls; forward(xq, xk, xv, rows, seq_kv) keys its shared
    quantization on which inputs are the same array."""

    def __init__(self, backend, dim, heads, W, b, int8=1):
        self.L = ref_nn(backend)
        self.dim = dim
        self.h = self.L.ref_nn_mha_load(dim, heads, _p(_f32(W)), _p(_f32(b)), int(int8))
        if not self.h:
            raise RuntimeError("ref_nn_mha_load failed")

    def forward(self, xq, xk, xv, rows, seq_kv):
        out = np.empty((rows, self.dim), np.float32)
        if self.L.ref_nn_mha_run(self.h, _p(xq), _p(xk), _p(xv), rows, seq_kv, _p(out)) != 0:
            raise RuntimeError("ref_nn_mha_run failed")
        return out

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_nn_mha_free(self.h)


class NnConv:
    """A reference nn::Conv2d (W [Cout, k, k, Cin], NHWC) kept across calls."""

    def __init__(self, backend, W, b, int8=1):
        self.L = ref_nn(backend)
        self.Cout, self.k, _, self.Cin = W.shape
        q = np.zeros(1, np.int32)
        self.h = self.L.ref_nn_conv_load(_p(_f32(W)), _p(None if b is None else _f32(b)), self.Cout, self.k,
                                         self.Cin, int(int8), _p(q))
        if not self.h:
            raise RuntimeError("ref_nn_conv_load failed")
        self.int8 = bool(q[0])

    def forward(self, x, stride, pad):
        x = _f32(x)
        H, Wd = x.shape[0], x.shape[1]
        Ho, Wo = (H + 2 * pad - self.k) // stride + 1, (Wd + 2 * pad - self.k) // stride + 1
        out = np.empty((Ho, Wo, self.Cout), np.float32)
        if self.L.ref_nn_conv_run(self.h, _p(x), H, Wd, stride, pad, _p(out)) != 0:
            raise RuntimeError("ref_nn_conv_run failed")
        return out

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_nn_conv_free(self.h)


class NnUnet:
    """The reference's Diffusion Policy UNet (DPUNet1d) on one op backend."""

    def __init__(self, backend, dirpath, cfg, int8):
        self.L = ref_nn(backend)
        vals = np.array([cfg[k] for k in ("action_dim", "horizon")] + list(cfg["down_dims"]) +
                        [cfg[k] for k in ("kernel_size", "n_groups", "step_embed_dim", "film_scale", "state_dim",
                                          "n_cams", "num_keypoints")], np.int32)
        n = np.zeros(1, np.int32)
        self.h = self.L.ref_unet_load(dirpath.encode(), _p(vals), int(int8), _p(n))
        if not self.h:
            raise RuntimeError(f"reference DPUNet1d::load failed for {dirpath}")
        self.n_int8 = int(n[0])
        self.cfg = cfg

    def forward(self, sample, gc, t):
        c = self.cfg
        eps = np.empty((c["horizon"], c["action_dim"]), np.float32)
        if self.L.ref_unet_forward(self.h, _p(eps), _p(_f32(sample)), _p(_f32(gc)), int(t)) != 0:
            raise RuntimeError("ref_unet_forward failed")
        return eps

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_unet_free(self.h)


def nn_pre_vs_ref(backend, W, x, bias):
    W, x = _f32(W), _f32(x)
    N, K = W.shape
    pre = np.empty((x.shape[0], N), np.float32)
    refo = np.empty((x.shape[0], N), np.float32)
    st = ref_nn(backend).ref_nn_pre_vs_ref(_p(W), N, K, _p(x), x.shape[0], _p(None if bias is None else _f32(bias)),
                                          _p(pre), _p(refo))
    if st != 0:
        raise RuntimeError("ref_nn_pre_vs_ref failed")
    return pre, refo


# ------------------------------------------------------------------ frand --

class Frand:
    """tests/test_ops.cpp:31-40 xorshift64 stream (state 0x243F6A8885A308D3)."""

    def __init__(self, state: int = 0x243F6A8885A308D3):
        self.state = c_uint64(state)

    def rv(self, n: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
        v = np.empty(n, np.float32)
        oracle().orc_frand_fill(ctypes.byref(self.state), _p(v), n, lo, hi)
        return v


# ------------------------------------------------------------ oracle ops --

def quantize_act_i8(x, ldq=None):
    x = _f32(x)
    seq, K = x.shape
    ldq = ldq or kpad(K)
    xq = np.empty((seq, ldq), np.int8)
    s = np.empty(seq, np.float32)
    oracle().orc_quantize_act_i8(_p(x), _p(xq), _p(s), seq, K, ldq)
    return xq, s


def quantize_weights_i8(W, ldq=None):
    W = _f32(W)
    N, K = W.shape
    ldq = ldq or kpad(K)
    Wq = np.empty((N, ldq), np.int8)
    s = np.empty(N, np.float32)
    oracle().orc_quantize_weights_i8(_p(W), _p(Wq), _p(s), N, K, ldq)
    return Wq, s


def gemm_i8_acc(xq, Wq, K):
    xq = np.ascontiguousarray(xq, np.int8)
    Wq = np.ascontiguousarray(Wq, np.int8)
    seq, N = xq.shape[0], Wq.shape[0]
    acc = np.empty((seq, N), np.int32)
    oracle().orc_gemm_i8_acc(_p(acc), _p(xq), xq.shape[1], _p(Wq), Wq.shape[1], seq, N, K)
    return acc


def dense_linear_i8_pre(xq, ascale, Wq, wscale, bias, K):
    xq = np.ascontiguousarray(xq, np.int8)
    Wq = np.ascontiguousarray(Wq, np.int8)
    seq, N = xq.shape[0], Wq.shape[0]
    out = np.empty((seq, N), np.float32)
    b = None if bias is None else _f32(bias)
    oracle().orc_dense_linear_i8_pre(_p(out), _p(xq), xq.shape[1], _p(_f32(ascale)), _p(Wq),
                                     Wq.shape[1], _p(_f32(wscale)), _p(b), seq, N, K)
    return out


def apply_act(x, act: int):
    x = _f32(x).copy()
    oracle().orc_apply_act(_p(x), x.size, act)
    return x


def attention(Q, K, V, seq_q, seq_k, n_q, n_kv, head_dim, scale, mask=None):
    out = np.empty((seq_q, n_q * head_dim), np.float32)
    m = None if mask is None else _f32(mask)
    oracle().orc_gqa_attention_masked(_p(out), _p(_f32(Q)), _p(_f32(K)), _p(_f32(V)), seq_q, seq_k,
                                      n_q, n_kv, head_dim, scale, _p(m))
    return out


def layernorm(x, w, b, eps):
    x = _f32(x)
    out = np.empty_like(x)
    oracle().orc_layernorm(_p(out), _p(x), _p(_f32(w)), _p(None if b is None else _f32(b)),
                           x.shape[0], x.shape[1], eps)
    return out


def rmsnorm(x, w, eps):
    x = _f32(x)
    out = np.empty_like(x)
    oracle().orc_rmsnorm(_p(out), _p(x), _p(_f32(w)), x.shape[0], x.shape[1], eps)
    return out


def rope_neox(x, pos, n_heads, head_dim, base):
    x = _f32(x).copy()
    p = np.ascontiguousarray(pos, np.int32)
    oracle().orc_rope_neox(_p(x), _p(p), len(p), n_heads, head_dim, base)
    return x


def gelu_tanh(x):
    x = _f32(x).copy()
    oracle().orc_gelu_tanh(_p(x), x.size)
    return x


def gelu_erf(x):
    x = _f32(x).copy()
    oracle().orc_gelu_erf(_p(x), x.size)
    return x


def relu(x):
    x = _f32(x).copy()
    oracle().orc_relu(_p(x), x.size)
    return x


def silu_gate(g, u):
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    oracle().orc_silu_gate(_p(out), _p(g), _p(u), g.size)
    return out


def conv_out(H, Wd, k, stride, pad):
    return (H + 2 * pad - k) // stride + 1, (Wd + 2 * pad - k) // stride + 1


def quantize_tensor_i8(x, clip=1.0):
    x = _f32(x)
    q = np.empty(x.shape, np.int8)
    s = oracle().orc_quantize_tensor_i8(_p(x), _p(q), x.size, clip)
    return q, np.float32(s)


def im2col_i8(xq, k, stride, pad, ldc=None):
    """xq int8 [H, Wd, Cin] -> [Hout*Wout, ldc] patch rows [ky][kx][ci]."""
    xq = np.ascontiguousarray(xq, np.int8)
    H, Wd, Cin = xq.shape
    Ho, Wo = conv_out(H, Wd, k, stride, pad)
    ldc = ldc or kpad(k * k * Cin)
    col = np.empty((Ho * Wo, ldc), np.int8)
    oracle().orc_im2col_i8(_p(col), ldc, _p(xq), H, Wd, Cin, k, stride, pad)
    return col


def conv2d_i8(x, Wq, wscale, bias, k, stride, pad, clip=1.0):
    """x fp32 [H, Wd, Cin], Wq int8 [Cout, >= k*k*Cin] -> out [Hout, Wout, Cout]."""
    x = _f32(x)
    H, Wd, Cin = x.shape
    Wq = np.ascontiguousarray(Wq, np.int8)
    Cout = Wq.shape[0]
    Ho, Wo = conv_out(H, Wd, k, stride, pad)
    out = np.empty((Ho, Wo, Cout), np.float32)
    b = None if bias is None else _f32(bias)
    oracle().orc_conv2d_i8(_p(out), _p(x), _p(Wq), Wq.shape[1], _p(_f32(wscale)), _p(b), H, Wd, Cin, Cout,
                           k, stride, pad, clip)
    return out


# ------------------------------------------------------ reference (real) --

def ref_pack_weights(W):
    """The reference packer: returns (row-major Wq [N, Kp], wscale, panel blob)."""
    W = _f32(W)
    N, K = W.shape
    L = ref()
    words = L.ref_packed_i8_words(N, K)
    blob = np.zeros(words * 4, np.int8)
    ws = np.empty(N, np.float32)
    L.ref_pack_weights_i8(_p(W), _p(blob), _p(ws), N, K)
    rows = np.empty((N, kpad(K)), np.int8)
    L.ref_rows_from_panels(_p(blob), N, K, _p(rows), kpad(K))
    return rows, ws, blob


def ref_panels(Wrows, K):
    """Row-major int8 [N, >=K] -> the reference's panel blob (+ row sums)."""
    Wrows = np.ascontiguousarray(Wrows, np.int8)
    N = Wrows.shape[0]
    L = ref()
    blob = np.zeros(L.ref_packed_i8_words(N, K) * 4, np.int8)
    L.ref_panels_from_rows(_p(Wrows), Wrows.shape[1], N, K, _p(blob))
    return blob


def ref_quantize_act_i8(x):
    x = _f32(x)
    seq, K = x.shape
    xq = np.empty((seq, kpad(K)), np.int8)
    s = np.empty(seq, np.float32)
    ref().ref_quantize_act_i8(_p(x), _p(xq), _p(s), seq, K)
    return xq, s


def ref_dense_linear_i8_ref(xq, ascale, blob, wscale, bias, N, K):
    seq = xq.shape[0]
    out = np.empty((seq, N), np.float32)
    ref().ref_dense_linear_i8_ref(_p(out), _p(np.ascontiguousarray(xq, np.int8)), _p(_f32(ascale)),
                                  _p(blob), _p(_f32(wscale)), _p(None if bias is None else _f32(bias)),
                                  seq, N, K)
    return out


def ref_dense_linear_i8_pre(xq, ascale, blob, wscale, bias, N, K):
    seq = xq.shape[0]
    out = np.empty((seq, N), np.float32)
    ref().ref_dense_linear_i8_pre(_p(out), _p(np.ascontiguousarray(xq, np.int8)), _p(_f32(ascale)),
                                  _p(blob), _p(_f32(wscale)), _p(None if bias is None else _f32(bias)),
                                  seq, N, K)
    return out


def ref_dense_linear_i8(x, blob, wscale, bias, N, K, xq_scratch=None, as_scratch=None):
    x = _f32(x)
    seq = x.shape[0]
    out = np.empty((seq, N), np.float32)
    xq = xq_scratch if xq_scratch is not None else np.empty((seq, kpad(K)), np.int8)
    s = as_scratch if as_scratch is not None else np.empty(seq, np.float32)
    ref().ref_dense_linear_i8(_p(out), _p(x), _p(blob), _p(_f32(wscale)),
                              _p(None if bias is None else _f32(bias)), seq, N, K, _p(xq), _p(s))
    return out


def ref_attention(Q, K, V, seq_q, seq_k, n_q, n_kv, head_dim, scale, mask=None):
    out = np.empty((seq_q, n_q * head_dim), np.float32)
    if mask is None:
        ref().ref_gqa_attention_dense(_p(out), _p(_f32(Q)), _p(_f32(K)), _p(_f32(V)), seq_q, seq_k,
                                      n_q, n_kv, head_dim, scale)
    else:
        ref().ref_gqa_attention_masked(_p(out), _p(_f32(Q)), _p(_f32(K)), _p(_f32(V)), seq_q, seq_k,
                                       n_q, n_kv, head_dim, scale, _p(_f32(mask)))
    return out


def ref_layernorm(x, w, b, eps):
    x = _f32(x)
    out = np.empty_like(x)
    ref().ref_layernorm(_p(out), _p(x), _p(_f32(w)), _p(None if b is None else _f32(b)), x.shape[0],
                        x.shape[1], eps)
    return out


def ref_rmsnorm(x, w, eps):
    x = _f32(x)
    out = np.empty_like(x)
    ref().ref_rmsnorm(_p(out), _p(x), _p(_f32(w)), x.shape[0], x.shape[1], eps)
    return out


def ref_rope_neox(x, pos, n_heads, head_dim, base):
    x = _f32(x).copy()
    p = np.ascontiguousarray(pos, np.int32)
    ref().ref_rope_neox(_p(x), _p(p), len(p), n_heads, head_dim, base)
    return x


def ref_eltwise(name, x):
    x = _f32(x).copy()
    getattr(ref(), name)(_p(x), x.size)
    return x


def ref_conv2d_i8(x, W, bias, k, stride, pad):
    """The reference's conv2d_i8 with its own pack_weights_i8 of fp32 W [Cout, k, k, Cin]."""
    x = _f32(x)
    H, Wd, Cin = x.shape
    W = _f32(W)
    Cout = W.shape[0]
    Ho, Wo = conv_out(H, Wd, k, stride, pad)
    out = np.empty((Ho, Wo, Cout), np.float32)
    b = None if bias is None else _f32(bias)
    ref().ref_conv2d_i8(_p(out), _p(x), _p(W), _p(b), H, Wd, Cin, Cout, k, stride, pad)
    return out


def ref_silu_gate(g, u):
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    ref().ref_silu_gate(_p(out), _p(g), _p(u), g.size)
    return out


# ------------------------------------------- reference policy graphs ------
# ref_models_shim.cpp: the reference's own ActTransformer / OctoTransformer /
# SmollmVlm + ActionExpert, loading the same checkpoint files as the device
# graphs.

def _ref_models():
    L = ref()
    if getattr(L, "_models_declared", False):
        return L
    P, i = c_void_p, c_int
    L.ref_act_load.argtypes, L.ref_act_load.restype = [ctypes.c_char_p, i, i], P
    L.ref_act_free.argtypes = [P]
    L.ref_act_forward.argtypes, L.ref_act_forward.restype = [P, P, i, i, i, P, P], i
    L.ref_octo_load.argtypes, L.ref_octo_load.restype = [ctypes.c_char_p, i], P
    L.ref_octo_free.argtypes = [P]
    L.ref_octo_forward.argtypes, L.ref_octo_forward.restype = [P, P, P, P, i, P, P], i
    L.ref_octo_total_tokens.argtypes, L.ref_octo_total_tokens.restype = [P, i], i
    L.ref_octo_forward_layout.argtypes = [P, P, P, P, i, P, i, P]
    L.ref_octo_forward_layout.restype = i
    L.ref_smolvla_load.argtypes, L.ref_smolvla_load.restype = [ctypes.c_char_p, i], P
    L.ref_smolvla_free.argtypes = [P]
    L.ref_smolvla_chunk.argtypes, L.ref_smolvla_chunk.restype = [P, P, P, i, P, P], i
    L.ref_smolvla_chunk_len.argtypes, L.ref_smolvla_chunk_len.restype = [P], i
    L.ref_smolvla_max_action_dim.argtypes, L.ref_smolvla_max_action_dim.restype = [P], i
    L.ref_siglip_load.argtypes, L.ref_siglip_load.restype = [ctypes.c_char_p, i], P
    L.ref_siglip_free.argtypes = [P]
    L.ref_siglip_encode.argtypes = [P, P, P]
    L.ref_act_load_ex.argtypes, L.ref_act_load_ex.restype = [ctypes.c_char_p, i, i, i], P
    L.ref_act_forward_text.argtypes, L.ref_act_forward_text.restype = [P, P, i, i, i, P, P, P, i, P], i
    L.ref_act_model_load.argtypes, L.ref_act_model_load.restype = [ctypes.c_char_p], P
    L.ref_act_model_free.argtypes = [P]
    L.ref_act_model_dims.argtypes = [P, P]
    L.ref_act_model_predict.argtypes, L.ref_act_model_predict.restype = [P, P, P, i, P], i
    L.ref_act_model_encode.argtypes, L.ref_act_model_encode.restype = [P, P, P], i
    L.ref_mount_read.argtypes = [ctypes.c_char_p, ctypes.c_char_p, P, ctypes.c_longlong]
    L.ref_mount_read.restype = ctypes.c_longlong
    L.ref_smolvla_model_load.argtypes, L.ref_smolvla_model_load.restype = [ctypes.c_char_p, i], P
    L.ref_smolvla_model_free.argtypes = [P]
    L.ref_smolvla_model_predict.argtypes = [P, P, i, i, i, P, P, i, P, P, P, P, i, P, c_float, i]
    L.ref_smolvla_model_predict.restype = i
    L.ref_resize_with_pad.argtypes = [P, i, i, i, P]
    L.ref_bpe_load.argtypes, L.ref_bpe_load.restype = [ctypes.c_char_p], P
    L.ref_bpe_free.argtypes = [P]
    L.ref_bpe_encode.argtypes, L.ref_bpe_encode.restype = [P, ctypes.c_char_p, P, i], i
    L.ref_octo_model_load.argtypes, L.ref_octo_model_load.restype = [ctypes.c_char_p, ctypes.c_char_p, i], P
    L.ref_octo_model_free.argtypes = [P]
    L.ref_octo_model_dims.argtypes = [P, P]
    L.ref_octo_model_lang.argtypes = [P, ctypes.c_char_p, P]
    L.ref_octo_model_predict.argtypes = [P, P, P, i, P, ctypes.c_char_p, P, P, i, P, i]
    L.vla_octo_load.argtypes, L.vla_octo_load.restype = [ctypes.c_char_p, ctypes.c_char_p], P
    L.vla_octo_free.argtypes, L.vla_octo_free.restype = [P], None
    for n in ("horizon", "action_dim", "max_window"):
        f = getattr(L, f"vla_octo_{n}")
        f.argtypes, f.restype = [P], ctypes.c_int32
    L.vla_octo_predict_ex.argtypes = [P, P, P, ctypes.c_int32, P, ctypes.c_char_p, P, P, c_uint64, ctypes.c_int32, P]
    L.vla_octo_predict_ex.restype = ctypes.c_int32
    L.ref_t5tok_load.argtypes, L.ref_t5tok_load.restype = [ctypes.c_char_p], P
    L.ref_t5tok_free.argtypes = [P]
    L.ref_t5tok_encode.argtypes = [P, ctypes.c_char_p, i, P]
    # the reference's own SmolVLA entry points (smolvla_capi.cpp)
    i32 = ctypes.c_int32
    L.vla_smolvla_load.argtypes, L.vla_smolvla_load.restype = [ctypes.c_char_p, ctypes.c_char_p], P
    L.vla_smolvla_free.argtypes, L.vla_smolvla_free.restype = [P], None
    for n in ("chunk", "action_dim", "state_dim", "n_views", "img_size", "tok_maxlen"):
        f = getattr(L, f"vla_smolvla_{n}")
        f.argtypes, f.restype = [P], i32
    L.vla_smolvla_tokenize.argtypes, L.vla_smolvla_tokenize.restype = [P, ctypes.c_char_p, P, P], i32
    L.vla_smolvla_predict_rtc.argtypes = [P, P, i32, i32, i32, P, P, i32, P, P, c_uint64, P, P, i32, P, c_float]
    L.vla_smolvla_predict_rtc.restype = i32
    # the reference's own IMPACT entry points (impact_capi.cpp)
    L.vla_impact_load.argtypes, L.vla_impact_load.restype = [ctypes.c_char_p], P
    L.vla_impact_free.argtypes, L.vla_impact_free.restype = [P], None
    for n in ("chunk", "action_dim", "state_dim", "n_cams", "img_h", "img_w", "n_text"):
        f = getattr(L, f"vla_impact_{n}")
        f.argtypes, f.restype = [P], i32
    L.vla_impact_set_instruction.argtypes, L.vla_impact_set_instruction.restype = [P, ctypes.c_char_p], i32
    L.vla_impact_predict.argtypes = [P, P, P, ctypes.c_char_p, i32, P]
    L.vla_impact_predict.restype = i32
    L.vla_impact_tokens.argtypes, L.vla_impact_tokens.restype = [P, P, P, P, i32], i32
    L.vla_impact_film.argtypes, L.vla_impact_film.restype = [P, P, P, i32], i32
    # the reference's own Diffusion Policy entry points (diffusion_capi.cpp)
    L.vla_diffusion_load.argtypes, L.vla_diffusion_load.restype = [ctypes.c_char_p], P
    L.vla_diffusion_free.argtypes, L.vla_diffusion_free.restype = [P], None
    for n in ("chunk", "horizon", "action_dim", "state_dim", "n_cams", "n_obs_steps", "img_h", "img_w",
              "num_steps", "is_ddim"):
        f = getattr(L, f"vla_diffusion_{n}")
        f.argtypes, f.restype = [P], i32
    L.vla_diffusion_predict.argtypes, L.vla_diffusion_predict.restype = [P, P, P, i32, P, P], i32
    L._models_declared = True
    return L


class RefSiglip:
    """The reference's SigLIP vision tower + connector (SiglipVision::encode)."""

    def __init__(self, dirpath, int8_mask, n_tok, mm_out):
        L = _ref_models()
        self.h = L.ref_siglip_load(dirpath.encode(), int8_mask)
        if not self.h:
            raise RuntimeError(f"reference SiglipVision::load failed for {dirpath}")
        self.n_tok, self.mm_out = n_tok, mm_out

    def encode(self, pixels):
        out = np.empty((self.n_tok, self.mm_out), np.float32)
        px = _f32(pixels)
        _ref_models().ref_siglip_encode(self.h, _p(px), _p(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().ref_siglip_free(self.h)


def ref_mount_read(path, rel):
    """The bytes of <path>/<rel> through the reference's own model-file layer
    (io::Mount + io::InFile: a vla.simd GGUF's embedded file, else the file on
    disk). None when there is no such file; raises when the path does not
    mount (a GGUF the reference rejects)."""
    L = _ref_models()
    n = L.ref_mount_read(str(path).encode(), rel.encode(), None, 0)
    if n == -2:
        raise ValueError(f"reference mount failed for {path}")
    if n < 0:
        return None
    buf = ctypes.create_string_buffer(max(int(n), 1))
    L.ref_mount_read(str(path).encode(), rel.encode(), ctypes.cast(buf, c_void_p), n)
    return buf.raw[:n]


class RefAct:
    def __init__(self, dirpath, img_ch, int8_mask, chunk, action_dim, int8_state=False):
        L = _ref_models()
        self.h = L.ref_act_load_ex(dirpath.encode(), img_ch, int8_mask, int(bool(int8_state)))
        if not self.h:
            raise RuntimeError(f"reference ActTransformer::load failed for {dirpath}")
        self.chunk, self.action_dim = chunk, action_dim

    def forward_text(self, feats, n_cams, fh, fw, state, text, text_pos, n_text_real):
        out = np.empty((self.chunk, self.action_dim), np.float32)
        _ref_models().ref_act_forward_text(self.h, _p(_f32(feats)), n_cams, fh, fw, _p(_f32(state)),
                                           _p(_f32(text)), _p(_f32(text_pos)), int(n_text_real), _p(out))
        return out

    def forward(self, feats, n_cams, fh, fw, state):
        out = np.empty((self.chunk, self.action_dim), np.float32)
        f, s = _f32(feats), _f32(state)
        _ref_models().ref_act_forward(self.h, _p(f), n_cams, fh, fw, _p(s), _p(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().ref_act_free(self.h)


class RefActModel:
    """The reference's ActModel (backbone + transformer + stats); ACT_INT8 is
    read from the environment at load, as the reference reads it."""

    def __init__(self, dirpath):
        L = _ref_models()
        self.h = L.ref_act_model_load(dirpath.encode())
        if not self.h:
            raise RuntimeError(f"reference ActModel::load failed for {dirpath}")
        d = np.zeros(9, np.int32)
        L.ref_act_model_dims(self.h, _p(d))
        (self.chunk, self.action_dim, self.state_dim, self.n_cams, self.img_h, self.img_w, self.feat_h,
         self.feat_w, self.feat_ch) = (int(v) for v in d)

    def predict(self, images, state, unnormalize=True):
        out = np.empty((self.chunk, self.action_dim), np.float32)
        _ref_models().ref_act_model_predict(self.h, _p(np.ascontiguousarray(images, np.uint8)), _p(_f32(state)),
                                            int(bool(unnormalize)), _p(out))
        return out

    def encode(self, images):
        out = np.empty((self.n_cams * self.feat_h * self.feat_w, self.feat_ch), np.float32)
        _ref_models().ref_act_model_encode(self.h, _p(np.ascontiguousarray(images, np.uint8)), _p(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().ref_act_model_free(self.h)


class RefOcto:
    def __init__(self, dirpath, int8_mask, d):
        L = _ref_models()
        self.h = L.ref_octo_load(dirpath.encode(), int8_mask)
        if not self.h:
            raise RuntimeError(f"reference OctoTransformer::load failed for {dirpath}")
        self.d = d

    def forward(self, t5, stem_p, stem_w, wnd, tmask):
        L = _ref_models()
        total = L.ref_octo_total_tokens(self.h, wnd)
        out = np.zeros((total, self.d), np.float32)
        a, b = _f32(t5), _f32(stem_p)
        c = None if stem_w is None else _f32(stem_w)
        tm = np.ascontiguousarray(tmask, dtype=np.uint8)
        ro = L.ref_octo_forward(self.h, _p(a), _p(b), _p(c), wnd, _p(tm), _p(out))
        return out[ro].copy()

    def forward_layout(self, t5, stem_p, stem_w, wnd, tmask, repeat_task):
        """The reference's own layers over either token layout (ref_octo_forward_layout):
        repeat_task 1 is forward()'s layout, 0 drops the per-step task copy."""
        L = _ref_models()
        out = np.zeros(self.d, np.float32)
        a, b = _f32(t5), _f32(stem_p)
        c = None if stem_w is None else _f32(stem_w)
        tm = np.ascontiguousarray(tmask, dtype=np.uint8)
        L.ref_octo_forward_layout(self.h, _p(a), _p(b), _p(c), wnd, _p(tm), int(repeat_task), _p(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().ref_octo_free(self.h)


class RefSmolvla:
    def __init__(self, dirpath, int8_mask):
        L = _ref_models()
        self.h = L.ref_smolvla_load(dirpath.encode(), int8_mask)
        if not self.h:
            raise RuntimeError(f"reference SmolVLA load failed for {dirpath}")
        self.chunk = L.ref_smolvla_chunk_len(self.h)
        self.mad = L.ref_smolvla_max_action_dim(self.h)

    def run(self, prefix, pad, noise):
        out = np.empty((self.chunk, self.mad), np.float32)
        p, n = _f32(prefix), _f32(noise)
        pd = np.ascontiguousarray(pad, dtype=np.int32)
        _ref_models().ref_smolvla_chunk(self.h, _p(p), _p(pd), p.shape[0], _p(n), _p(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().ref_smolvla_free(self.h)


def ref_dense_linear(x, W, bias=None):
    """The reference's fp32 dense_linear (Linear::Role::Generic)."""
    x, W = _f32(x), _f32(W)
    b = None if bias is None else _f32(bias)
    out = np.empty((x.shape[0], W.shape[0]), np.float32)
    ref().ref_dense_linear(_p(out), _p(x), _p(W), _p(b), x.shape[0], W.shape[0], W.shape[1])
    return out


class RefSmolvlaModel:
    """The reference's SmolvlaModel. int8_mask None: through its own C ABI
    (vla_smolvla_load / _tokenize / _predict_rtc, SMOLVLA_INT8 as the
    environment had it at the process's first load); an int mask: loaded by
    ref_smolvla_model_load with that mask's groups and run by the body of
    vla_smolvla_predict_rtc (ref_smolvla_model_predict, noise required)."""

    def __init__(self, dirpath, tok_dir=None, int8_mask=None):
        L = _ref_models()
        self.abi = int8_mask is None
        if self.abi:
            tok_dir = tok_dir or os.path.join(dirpath, "tok")
            self.h = L.vla_smolvla_load(dirpath.encode(), tok_dir.encode())
        else:
            self.h = L.ref_smolvla_model_load(dirpath.encode(), int8_mask)
        if not self.h:
            raise RuntimeError(f"reference SmolvlaModel::load failed for {dirpath}")

    def dims(self):
        L = _ref_models()
        assert self.abi
        return {n: getattr(L, f"vla_smolvla_{n}")(self.h)
                for n in ("chunk", "action_dim", "state_dim", "n_views", "img_size", "tok_maxlen")}

    def tokenize(self, text, maxlen):
        ids = np.zeros(maxlen, np.int32)
        mask = np.zeros(maxlen, np.int32)
        n = _ref_models().vla_smolvla_tokenize(self.h, text.encode(), _p(ids), _p(mask))
        return ids, mask, n

    def predict(self, frames, ids, mask, state, chunk, action_dim, noise=None, seed=0, prev=None, weights=None,
                max_guidance=0.0, perturb=0):
        """-> (status, actions [chunk, action_dim]); perturb > 0 (shim path
        only) moves the preprocessed pixels by seeded 1-ulp steps"""
        L = _ref_models()
        frames = np.ascontiguousarray(frames, np.uint8)
        ids, mask = np.ascontiguousarray(ids, np.int32), np.ascontiguousarray(mask, np.int32)
        out = np.zeros((chunk, action_dim), np.float32)
        noise = None if noise is None else _f32(noise)
        prev = None if prev is None else _f32(prev)
        weights = None if weights is None else _f32(weights)
        n_prev = 0 if prev is None else prev.size // action_dim
        nv, h, w = frames.shape[:3]
        if self.abi:
            st = L.vla_smolvla_predict_rtc(self.h, _p(frames), nv, h, w, _p(ids), _p(mask), ids.size,
                                           _p(_f32(state)), _p(noise), seed, _p(out), _p(prev), n_prev,
                                           _p(weights), float(max_guidance))
        else:
            assert noise is not None
            st = L.ref_smolvla_model_predict(self.h, _p(frames), nv, h, w, _p(ids), _p(mask), ids.size,
                                             _p(_f32(state)), _p(noise), _p(out), _p(prev), n_prev, _p(weights),
                                             float(max_guidance), int(perturb))
        return int(st), out

    def __del__(self):
        if getattr(self, "h", None):
            L = _ref_models()
            (L.vla_smolvla_free if self.abi else L.ref_smolvla_model_free)(self.h)


def ref_resize_with_pad(frame, S):
    """src/preprocess/image.cpp resize_with_pad: [h, w, 3] uint8 -> [3, S, S]"""
    frame = np.ascontiguousarray(frame, np.uint8)
    out = np.empty((3, S, S), np.float32)
    _ref_models().ref_resize_with_pad(_p(frame), frame.shape[0], frame.shape[1], S, _p(out))
    return out


class RefBpe:
    """The reference's Tokenizer (src/tokenizer/tokenizer.cpp)."""

    def __init__(self, tok_dir):
        self.h = _ref_models().ref_bpe_load(tok_dir.encode())
        if not self.h:
            raise RuntimeError(f"reference Tokenizer::load failed for {tok_dir}")

    def encode(self, text):
        b = text.encode() if isinstance(text, str) else bytes(text)
        L = _ref_models()
        n = L.ref_bpe_encode(self.h, b, None, 0)
        ids = np.zeros(max(n, 1), np.int32)
        L.ref_bpe_encode(self.h, b, _p(ids), n)
        return [int(v) for v in ids[:n]]

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().ref_bpe_free(self.h)


class RefT5Tok:
    """The reference's T5Tokenizer (src/tokenizer/t5_tokenizer.cpp)."""

    def __init__(self, tok_dir):
        self.h = _ref_models().ref_t5tok_load(tok_dir.encode())
        if not self.h:
            raise RuntimeError(f"reference T5Tokenizer::load failed for {tok_dir}")

    def encode(self, text, max_len=16):
        b = text.encode() if isinstance(text, str) else bytes(text)
        ids = np.zeros(max_len, np.int32)
        _ref_models().ref_t5tok_encode(self.h, b, max_len, _p(ids))
        return [int(v) for v in ids]

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().ref_t5tok_free(self.h)


class RefImpactModel:
    """The reference's ImpactModel through its own C ABI (vla_impact_load /
    _set_instruction / _predict / _tokens / _film, IMPACT_INT8 as the process
    environment holds it at load)."""

    def __init__(self, dirpath):
        L = _ref_models()
        self.h = L.vla_impact_load(dirpath.encode())
        if not self.h:
            raise RuntimeError(f"reference ImpactModel::load failed for {dirpath}")
        self.chunk, self.action_dim = L.vla_impact_chunk(self.h), L.vla_impact_action_dim(self.h)
        self.state_dim, self.n_cams = L.vla_impact_state_dim(self.h), L.vla_impact_n_cams(self.h)
        self.img_h, self.img_w, self.n_text = L.vla_impact_img_h(self.h), L.vla_impact_img_w(self.h), \
            L.vla_impact_n_text(self.h)

    def set_instruction(self, instruction):
        return int(_ref_models().vla_impact_set_instruction(self.h, instruction.encode()))

    def predict(self, frames, state, instruction, unnormalize=True):
        """-> (status, actions [chunk, action_dim])"""
        frames = np.ascontiguousarray(frames, np.uint8)
        state = _f32(state)
        out = np.zeros((self.chunk, self.action_dim), np.float32)
        st = _ref_models().vla_impact_predict(self.h, _p(frames), _p(state), instruction.encode(),
                                              int(bool(unnormalize)), _p(out))
        return int(st), out

    def tokens(self):
        ids, comp, mask = (np.zeros(self.n_text, np.int32) for _ in range(3))
        n = _ref_models().vla_impact_tokens(self.h, _p(ids), _p(comp), _p(mask), self.n_text)
        return int(n), ids, comp, mask

    def film(self):
        L = _ref_models()
        n = L.vla_impact_film(self.h, None, None, 1 << 30)
        if n <= 0:
            return int(n), None, None
        g, b = np.zeros(n, np.float32), np.zeros(n, np.float32)
        L.vla_impact_film(self.h, _p(g), _p(b), n)
        return int(n), g, b

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().vla_impact_free(self.h)
            self.h = None


class RefDiffusionModel:
    """The reference's DiffusionModel through its own C ABI (vla_diffusion_load
    / _predict; DIFFUSION_INT8, DP_STEPS and DP_SCHEDULER as the process
    environment holds them at load)."""

    DIMS = ("chunk", "horizon", "action_dim", "state_dim", "n_cams", "n_obs_steps", "img_h", "img_w", "num_steps",
            "is_ddim")

    def __init__(self, dirpath):
        L = _ref_models()
        self.h = L.vla_diffusion_load(dirpath.encode())
        if not self.h:
            raise RuntimeError(f"reference DiffusionModel::load failed for {dirpath}")
        for k in self.DIMS:
            setattr(self, k, int(getattr(L, f"vla_diffusion_{k}")(self.h)))

    def predict(self, frames, state, noise=None, unnormalize=True):
        """-> (status, actions [chunk, action_dim])"""
        frames = np.ascontiguousarray(frames, np.uint8)
        state = _f32(state)
        out = np.zeros((self.chunk, self.action_dim), np.float32)
        noise = None if noise is None else _f32(noise)  # held until the call returns
        st = _ref_models().vla_diffusion_predict(self.h, _p(frames), _p(state), int(bool(unnormalize)), _p(out),
                                                 None if noise is None else _p(noise))
        return int(st), out

    def __del__(self):
        if getattr(self, "h", None):
            _ref_models().vla_diffusion_free(self.h)
            self.h = None


class RefOctoModel:
    """The reference's OctoModel. int8_mask None: through its own C ABI
    (vla_octo_load / vla_octo_predict_ex, OCTO_INT8 as the process latched
    it); an int mask: ref_octo_model_load with that mask's groups and
    ref_octo_model_predict (noise and z required, optional stem-token ulp
    perturbation)."""

    def __init__(self, dirpath, tok_dir=None, int8_mask=None):
        L = _ref_models()
        tok_dir = tok_dir or os.path.join(dirpath, "tok")
        self.abi = int8_mask is None
        self.h = (L.vla_octo_load(dirpath.encode(), tok_dir.encode()) if self.abi
                  else L.ref_octo_model_load(dirpath.encode(), tok_dir.encode(), int8_mask))
        if not self.h:
            raise RuntimeError(f"reference OctoModel::load failed for {dirpath}")
        self._shim = None if self.abi else self.h
        d = np.zeros(6, np.int32)
        if not self.abi:
            L.ref_octo_model_dims(self.h, _p(d))
            self.horizon, self.action_dim, self.max_window, self.n_task, self.t5_dim, self.steps = (int(v) for v in d)
        else:
            self.horizon, self.action_dim = L.vla_octo_horizon(self.h), L.vla_octo_action_dim(self.h)
            self.max_window = L.vla_octo_max_window(self.h)

    def predict(self, primary, wrist, tmask, instruction, noise=None, z=None, seed=0, unnormalize=True, perturb=0):
        """-> (status, actions [horizon, action_dim])"""
        L = _ref_models()
        primary = np.ascontiguousarray(primary, np.uint8)
        wrist = None if wrist is None else np.ascontiguousarray(wrist, np.uint8)
        tm = np.ascontiguousarray(tmask, np.uint8)
        noise = None if noise is None else _f32(noise)
        z = None if z is None else _f32(z)
        out = np.zeros((self.horizon, self.action_dim), np.float32)
        wnd = primary.shape[0]
        if self.abi:
            st = L.vla_octo_predict_ex(self.h, _p(primary), _p(wrist), wnd, _p(tm), instruction.encode(), _p(noise),
                                       _p(z), seed, int(bool(unnormalize)), _p(out))
            return int(st), out
        assert noise is not None and z is not None
        L.ref_octo_model_predict(self.h, _p(primary), _p(wrist), wnd, _p(tm), instruction.encode(), _p(noise), _p(z),
                                 int(bool(unnormalize)), _p(out), int(perturb))
        return 0, out

    def lang(self, instruction):
        assert not self.abi
        out = np.zeros((self.n_task, self.t5_dim), np.float32)
        _ref_models().ref_octo_model_lang(self.h, instruction.encode(), _p(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            L = _ref_models()
            (L.vla_octo_free if self.abi else L.ref_octo_model_free)(self.h)
