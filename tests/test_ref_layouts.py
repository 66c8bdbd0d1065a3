"""CPU pin of the reference-side driver the 658-token Octo parity test uses.

RefOcto.forward_layout (oracle/ref_models_shim.cpp) drives the reference's own
loaded OctoTransformer layers over a token layout with or without the per-step
task copy. At the reference's own layout (repeat_task 1) it must reproduce
OctoTransformer::forward (src/models/octo/octo_transformer.cpp:144-219) bit for
bit, fp32 and int8; the 658-token layout must differ from it (the layouts are
different inputs), and a planted mistake in the 658 driver's inputs must show.
"""

import os

import numpy as np
import pytest

from helpers import load_pkg


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


@pytest.fixture(scope="module")
def octo_dir(tmp_path_factory):
    ck = _ck()
    d = str(tmp_path_factory.mktemp("ref_layout") / "octo")
    ck.write_octo(d, dict(ck.OCTO_BASE, n_layers=3, repeat_task=1))
    return d


@pytest.mark.parametrize("mask,wrist,tmask", [(0, True, (1, 1)), (7, True, (1, 1)), (15, False, (1, 1)),
                                              (7, True, (0, 1))])
def test_layout_driver_reproduces_reference_forward(octo_dir, mask, wrist, tmask):
    from helpers import oracle
    ob = oracle()
    if not ob.ref_available():
        pytest.skip("oracle/_ref/libvla_ref.so is not built")
    ck = _ck()
    c = dict(ck.OCTO_BASE, n_layers=3, repeat_task=1)
    t5, sp, sw, _ = ck.octo_inputs(c)
    sw = sw if wrist else None
    tm = np.array(tmask, np.uint8)
    r = ob.RefOcto(octo_dir, mask, c["d"])
    ref = r.forward(t5, sp, sw, 2, tm)
    got = r.forward_layout(t5, sp, sw, 2, tm, 1)
    assert got.tobytes() == ref.tobytes()
    # the 658-token layout is a different input: its readout row differs
    other = r.forward_layout(t5, sp, sw, 2, tm, 0)
    assert np.max(np.abs(other - ref)) > 1e-3 * np.max(np.abs(ref))
    # a planted mistake (one stem row perturbed) moves the driver's output
    sp2 = np.array(sp, copy=True)
    sp2[1, 7, :] += 0.5
    assert r.forward_layout(t5, sp2, sw, 2, tm, 0).tobytes() != other.tobytes()
