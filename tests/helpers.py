"""Shared test plumbing: repo paths, package and oracle loaders, comparison helpers."""

from __future__ import annotations

import hashlib
import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")

if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def load_pkg():
    """Import vla.simd_amd/ as module ``vla_simd_amd`` (its directory name has a dot)."""
    if "vla_simd_amd" in sys.modules:
        return sys.modules["vla_simd_amd"]
    d = os.path.join(ROOT, "vla.simd_amd")
    spec = importlib.util.spec_from_file_location("vla_simd_amd", os.path.join(d, "__init__.py"),
                                                  submodule_search_locations=[d])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["vla_simd_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_synth():
    load_pkg()
    import vla_simd_amd.synth as synth  # noqa: E402
    return synth


def load_masks():
    load_pkg()
    import vla_simd_amd.masks as masks  # noqa: E402
    return masks


def oracle():
    import oracle.bindings as ob  # noqa: E402
    return ob


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def golden(name: str):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """test_ops.cpp:41-43: equal shape and identical bytes."""
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()


def max_rel(got: np.ndarray, ref: np.ndarray, floor: float = 1.0) -> float:
    """max |got - ref| / max(|ref|, floor), rejecting non-finite values (test_ops.cpp:59-70)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if got.shape != ref.shape or not np.all(np.isfinite(got)) or not np.all(np.isfinite(ref)):
        return float("inf")
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), floor))) if got.size else 0.0
