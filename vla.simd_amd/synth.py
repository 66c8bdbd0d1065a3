"""Seeded synthetic inputs for the BASELINE configs (numpy, host side).

One generator feeds the GPU path, the CPU baseline and the parity tests, so
all three see identical bytes. Each tensor gets its own splitmix64 stream,
seeded from the base seed and an FNV-1a hash of the tensor's name; uniform
draws are the top 53 bits scaled to [0, 1); normal draws are Box-Muller over
pairs of uniforms.

The bytes must not depend on the machine that runs this (the fixtures under
tests/golden/ store hashes of both inputs and outputs, and the GPU box
regenerates the inputs). Vectorised transcendental functions may round
differently on different CPUs, so Box-Muller here uses only IEEE-exact
operations (+ - * / sqrt, frexp, floor) on float64: ln by frexp and the atanh
series, sin/cos by octant reduction and Taylor series, both accurate to a few
ulp of float64 - far below the float32 rounding that follows.

The distributions are the ones BASELINE.json states for the int8 linear
configs: activations ~ N(0, 1), int8 weights uniform integers in [-127, 127],
per-output-channel weight scales ~ U(1e-3, 1e-2), bias ~ N(0, 0.02^2).
"""

from __future__ import annotations

import numpy as np

BASE_SEED = 20261201
_M64 = (1 << 64) - 1


def _fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & _M64
    return h


def _splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start+1 .. start+n of the splitmix64 stream seeded with seed."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed & _M64) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def _seed(name: str, seed: int) -> int:
    return (seed ^ _fnv1a64(name)) & _M64


def uniform(name: str, shape, lo=0.0, hi=1.0, seed: int = BASE_SEED) -> np.ndarray:
    n = int(np.prod(shape))
    u = (_splitmix64(_seed(name, seed), n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


_LN2 = 0.6931471805599453
# cos/sin of the octant centres (2k+1)*pi/8, k = 0..7
_C8 = np.array([0.9238795325112867, 0.38268343236508984, -0.3826834323650897, -0.9238795325112867,
                -0.9238795325112868, -0.38268343236509034, 0.38268343236509, 0.9238795325112865])
_S8 = np.array([0.3826834323650898, 0.9238795325112867, 0.9238795325112867, 0.3826834323650899,
                -0.38268343236508967, -0.9238795325112864, -0.9238795325112867, -0.38268343236509045])


_INV_ODD = [1.0 / k for k in range(23, 0, -2)]  # 1/23, 1/21, ..., 1/1
_COS_C = []  # (-1)^j / (2j)!, j = 9 .. 0 (Horner order)
_SIN_C = []  # (-1)^j / (2j+1)!, j = 9 .. 0
for _j in range(9, -1, -1):
    _f2, _f3 = 1.0, 1.0
    for _t in range(1, 2 * _j + 1):
        _f2 *= _t
    _f3 = _f2 * (2 * _j + 1)
    _COS_C.append((-1.0) ** _j / _f2)
    _SIN_C.append((-1.0) ** _j / _f3)


def _ln(u: np.ndarray) -> np.ndarray:
    """ln(u), u > 0, from exact frexp and the series ln m = 2 atanh((m-1)/(m+1))."""
    m, e = np.frexp(u)  # u = m * 2^e, m in [0.5, 1)
    small = m < 0.7071067811865476
    m[small] *= 2.0
    e = (e - small).astype(np.float64)
    s = (m - 1.0) / (m + 1.0)
    s2 = s * s
    acc = np.full_like(s, _INV_ODD[0])
    for c in _INV_ODD[1:]:
        acc *= s2
        acc += c
    acc *= s
    acc *= 2.0
    e *= _LN2
    acc += e
    return acc


def _sincos_turns(t: np.ndarray):
    """(cos, sin) of 2*pi*t for t in [0, 1)."""
    x = t * 8.0
    k = np.floor(x)
    a = x - k
    a -= 0.5
    a *= np.pi / 4.0  # [-pi/8, pi/8)
    a2 = a * a
    c = np.full_like(a, _COS_C[0])
    sn = np.full_like(a, _SIN_C[0])
    for cc, sc in zip(_COS_C[1:], _SIN_C[1:]):
        c *= a2
        c += cc
        sn *= a2
        sn += sc
    sn *= a
    ki = np.minimum(k.astype(np.int64), 7)
    C, S = _C8[ki], _S8[ki]
    return C * c - S * sn, S * c + C * sn


def normal(name: str, shape, std=1.0, seed: int = BASE_SEED) -> np.ndarray:
    """Draw 2i and 2i+1 of the stream form pair i; pair i gives element i
    (cos branch) and element m + i (sin branch), m = ceil(n/2). Computed in
    cache-sized chunks of pairs; every step is elementwise, so chunking does
    not change a value."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    sd = _seed(name, seed)
    v = np.empty(2 * m, np.float64)
    CH = 1 << 16
    for p0 in range(0, m, CH):
        p1 = min(m, p0 + CH)
        z = _splitmix64(sd, 2 * (p1 - p0), 2 * p0) >> np.uint64(11)
        u1 = (z[0::2].astype(np.float64) + 1.0) * (1.0 / (1 << 53))  # (0, 1]
        u2 = z[1::2].astype(np.float64) * (1.0 / (1 << 53))
        r = np.sqrt(-2.0 * _ln(u1))
        cs, sn = _sincos_turns(u2)
        v[p0:p1] = r * cs
        v[m + p0:m + p1] = r * sn
    return (std * v[:n]).astype(np.float32).reshape(shape)


def int8_uniform(name: str, shape, seed: int = BASE_SEED) -> np.ndarray:
    n = int(np.prod(shape))
    z = _splitmix64(_seed(name, seed), n)
    return ((z % np.uint64(255)).astype(np.int64) - 127).astype(np.int8).reshape(shape)


def linear_case(M: int, K: int, N: int, tag: str = "lin", seed: int = BASE_SEED):
    """One int8 linear of the BASELINE distributions: (x, Wq, wscale, bias)."""
    x = normal(f"{tag}.x.{M}x{K}", (M, K), 1.0, seed)
    Wq = int8_uniform(f"{tag}.w.{N}x{K}", (N, K), seed)
    ws = uniform(f"{tag}.ws.{N}", (N,), 1e-3, 1e-2, seed)
    b = normal(f"{tag}.b.{N}", (N,), 0.02, seed)
    return x, Wq, ws, b


# BASELINE.json configs[0] and configs[1]
CONFIG1 = (100, 512, 3200)  # (M, K, N): ACT action-decoder linear
SWEEP_M = (1, 50, 100, 512, 2048, 8192)
SWEEP_KN = ((512, 3200), (960, 2560), (2560, 960), (768, 3072), (4096, 4096))
