"""CPU checks of the C-ABI boundary: the library loads without a GPU and
exports every symbol include/*.h declares (no compute calls here)."""

import ctypes
import os
import re

from helpers import ROOT, load_pkg


def declared_symbols():
    names = []
    inc = os.path.join(ROOT, "include")
    for f in sorted(os.listdir(inc)):
        if f.endswith(".h"):
            text = open(os.path.join(inc, f)).read()
            names += re.findall(r"VLA_API\s+[^;(]*?\b(vla_\w+)\s*\(", text)
    return names


def test_header_declares_the_python_export_list():
    pkg = load_pkg()
    assert sorted(set(declared_symbols())) == sorted(set(pkg.EXPORTS))


def test_library_exports_every_declared_symbol():
    pkg = load_pkg()
    L = ctypes.CDLL(pkg.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing


def test_handshake_without_gpu():
    pkg = load_pkg()
    assert pkg.abi_version() == 1
    assert pkg.backend_name() == "hip-gfx950"
    # no device in this container: the int8 path must report itself unavailable
    if not os.path.exists("/dev/kfd"):
        assert pkg.int8_available() is False


def test_argument_errors_need_no_device():
    """Preconditions are checked before any device work, and come back as
    VLA_ERR_ARG with a message (include/vla_simd.h:15-20 error contract)."""
    import numpy as np
    import pytest

    pkg = load_pkg()
    with pytest.raises(pkg.VlaError) as e:
        pkg.quantize_act_i8(np.zeros((2, 0), np.float32))
    assert e.value.status == pkg.VLA_ERR_ARG
    K = 2147483647 // (255 * 127) + 1
    st = pkg.lib().vla_dense_linear_i8_pre(None, None, None, None, None, None, 1, 16, K)
    assert st == pkg.VLA_ERR_ARG
    assert b"accumulator bound" in pkg.lib().vla_last_error()
