"""SmolVLA's SigLIP vision tower + connector on the device against the
reference's own SiglipVision (src/models/smolvla/siglip_vision.cpp, compiled
from the reference sources into oracle/_ref/libvla_ref.so).

Both sides load the same synthetic vit.meta / vit.bin (written in the
reference's layout by vla_simd_amd.checkpoints.write_siglip) and encode the
same seeded image. The bars are those of the other device graphs
(tests/test_gpu_graphs.py): int8 mask 0 agrees to 1e-3 of the output scale;
int8 masks sit within twice the reference's own spread under 1-ulp input
perturbations. Replays of the captured graph reproduce the eager call bit for
bit, and a GGUF of the checkpoint gives the directory load's bytes.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from helpers import load_pkg, oracle
from test_gpu_graphs import _bar, _check_replay, _rel

pytestmark = pytest.mark.gpu

# the reference geometry at reduced depth/width: 128x128 images, 64 patches,
# pixel shuffle by 2 into 16 tokens
SMALL = dict(hidden=192, n_heads=3, head_dim=64, inter=768, n_layers=2, patch=16, img=128, n_patches=64,
             ln_eps=1e-6, scale_factor=2, mm_out=256, n_img_tok=16)


def _ck():
    load_pkg()
    import vla_simd_amd.checkpoints as ck
    return ck


@pytest.fixture(scope="module")
def ckdir(tmp_path_factory):
    return tmp_path_factory.mktemp("vit")


def _dir(ck, ckdir, name, cfg):
    d = str(ckdir / name)
    if not os.path.exists(os.path.join(d, "vit.bin")):
        ck.write_siglip(d, cfg)
    return d


@pytest.mark.parametrize("cfg_name,mask", [("small", 0), ("small", 15), ("small", 1), ("deep2", 15)])
def test_siglip_encode(vla, ckdir, cfg_name, mask):
    ck = _ck()
    ob = oracle()
    # deep2: the full SmolVLM2 tower geometry (512x512, 1024 patches, hidden
    # 768, pixel shuffle by 4 into 64 tokens of 12288) at two layers
    cfg = SMALL if cfg_name == "small" else dict(ck.SIGLIP_BASE, n_layers=2)
    d = _dir(ck, ckdir, cfg_name, cfg)
    px = ck.siglip_inputs(cfg)
    print(f"siglip {cfg_name} mask {mask}", flush=True)
    r = ob.RefSiglip(d, mask, cfg["n_img_tok"], cfg["mm_out"])
    ref = r.encode(px)
    bar, sens = _bar(mask, r.encode, px, ref)
    m = vla.SiglipVision(d, mask)
    assert (m.img, m.n_tokens, m.out_dim) == (cfg["img"], cfg["n_img_tok"], cfg["mm_out"])
    assert m.int8_layers == cfg["n_layers"] * ((4 if mask & 1 else 0) + bool(mask & 2) + bool(mask & 4)) + \
        (2 if mask & 8 else 0)
    got = m.encode(px)
    err = _rel(got, ref)
    print(f"siglip {cfg_name} mask {mask}: rel err {err:.3e} (reference ulp spread {sens:.3e})", flush=True)
    assert err <= bar
    _check_replay(lambda: m.encode(px), got)


def test_siglip_dev_form_and_gguf(vla, ckdir, torch_cuda):
    """encode_dev on device buffers equals the host form; the GGUF of the
    checkpoint (fp32 region then bf16, as the converter stores vit.bin) loads
    to the same bytes."""
    torch = torch_cuda
    ck = _ck()
    d = _dir(ck, ckdir, "small", SMALL)
    g = str(ckdir / "small.gguf")
    ck.write_gguf(d, g, "smolvla-vision", layout=ck.siglip_gguf_layout(SMALL))
    px = ck.siglip_inputs(SMALL)
    m = vla.SiglipVision(d, 15)
    want = m.encode(px)
    out = torch.full((SMALL["n_img_tok"], SMALL["mm_out"]), 3.0, device="cuda")
    m.encode_dev(torch.from_numpy(px).cuda(), out)
    torch.cuda.synchronize()
    assert out.cpu().numpy().tobytes() == want.tobytes()
    assert vla.SiglipVision(g, 15).encode(px).tobytes() == want.tobytes()


def test_siglip_rejects_bad_meta(vla, ckdir):
    """A vit.meta whose grids do not close is refused at load (the reference's
    siglip_vision.cpp:43-70 checks), as is a vit.bin of the wrong size."""
    ck = _ck()
    bad = dict(SMALL, n_img_tok=9)  # 8x8 patches shuffled by 2 give 16 tokens, not 9
    d = str(ckdir / "bad")
    ck.write_siglip(d, bad)
    with pytest.raises(vla.VlaError):
        vla.SiglipVision(d, 15)
    d2 = str(ckdir / "short")
    ck.write_siglip(d2, SMALL)
    with open(os.path.join(d2, "vit.bin"), "r+b") as f:
        f.truncate(os.path.getsize(os.path.join(d2, "vit.bin")) - 2)
    with pytest.raises(vla.VlaError):
        vla.SiglipVision(d2, 15)
