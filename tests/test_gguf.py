"""The model-file layer (vla_ckpt_*): converted directories and vla.simd GGUFs.

Checked against the reference's own reader: oracle/_ref/libvla_ref.so carries
src/io/{files,gguf,gguf_vla_simd,gguf_models}.cpp, and ref_mount_read returns
what its io::Mount + io::InFile serve for a path, as its model loaders read it
(act_model.cpp:23). Every GGUF here is written by vla_simd_amd.checkpoints
(write_gguf / GgufBuilder); the reference reading it back byte for byte, and
its loaders giving bit-identical outputs from it and from the directory, pin
the writer. The reader then has to agree with the reference on every file,
malformed ones included (the cases of the reference's tests/test_gguf.cpp
:170-230 and :262-300: truncation, bad version, duplicates, misaligned or
overflowing tensors, bad alignment, unsafe paths, misordered parts). No GPU.
"""

from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from helpers import load_pkg


@pytest.fixture(scope="module")
def vla():
    return load_pkg()


@pytest.fixture(scope="module")
def ck(vla):
    import vla_simd_amd.checkpoints as ck
    return ck


@pytest.fixture(scope="module")
def ob():
    from helpers import oracle
    o = oracle()
    if not o.ref_available():
        pytest.skip("oracle/_ref/libvla_ref.so is not built")
    return o


ACT_SMALL = dict(dim=128, heads=2, head_dim=64, ff=256, n_enc=2, n_dec=1, chunk=10, state_dim=14,
                 action_dim=14, n_1d=2, n_text=0, ln_eps=1e-5, img_ch=64, n_cams=1, fh=3, fw=4)
OCTO_SMALL = dict(d=128, n_layers=2, heads=2, head_dim=64, mlp=256, max_horizon=10, n_task=4,
                  tok_primary=16, tok_wrist=4, n_readout=1, t5_dim=64, stem_dim=32, ln_eps=1e-6,
                  gelu_erf=0, repeat_task=1, wnd=2)


@pytest.fixture(scope="module")
def models(ck, tmp_path_factory):
    """Small ACT / Octo / SmolVLA checkpoints as directories and as GGUFs."""
    root = tmp_path_factory.mktemp("gguf")
    smol = dict(ck.SMOLVLA_BASE, chunk=12, n_layers=2, expert_layers=2, n_prefix=60)
    vit = dict(hidden=192, n_heads=3, head_dim=64, inter=768, n_layers=2, patch=16, img=128, n_patches=64,
               ln_eps=1e-6, scale_factor=2, mm_out=256, n_img_tok=16)
    out = {}
    for name, write, cfg, layout in (("act", ck.write_act, ACT_SMALL, None),
                                     ("octo", ck.write_octo, OCTO_SMALL, None),
                                     ("smolvla", ck.write_smolvla, smol, ck.smolvla_gguf_layout(smol)),
                                     ("siglip", ck.write_siglip, vit, ck.siglip_gguf_layout(vit))):
        d = str(root / name)
        write(d, cfg)
        g = str(root / f"{name}.gguf")
        ck.write_gguf(d, g, name, source="synthetic", layout=layout)
        out[name] = (d, g, cfg)
    return out


def _disk_files(d):
    return sorted(n for n in os.listdir(d) if os.path.isfile(os.path.join(d, n)))


@pytest.mark.parametrize("name", ["act", "octo", "smolvla", "siglip"])
def test_gguf_serves_the_directory_bytes(vla, ob, models, name):
    d, g, _ = models[name]
    f = vla.CkptFiles(g)
    assert f.gguf
    assert f.names() == _disk_files(d)
    for rel in f.names():
        disk = open(os.path.join(d, rel), "rb").read()
        assert f.size(rel) == len(disk)
        assert f.read(rel) == disk, rel
        assert ob.ref_mount_read(g, rel) == disk, f"the reference reads {rel} differently"
    plain = vla.CkptFiles(d)
    assert not plain.gguf and plain.names() == []
    assert plain.read(f.names()[0]) == open(os.path.join(d, f.names()[0]), "rb").read()


def test_smolvla_bin_is_stored_in_typed_parts(ck, models):
    """vlm.bin mixes fp32 norms and bf16 matrices: two tensors vlm.bin:0 (F32)
    and vlm.bin:1 (BF16), concatenated on read."""
    _, g, cfg = models["smolvla"]
    raw = open(g, "rb").read()
    assert b"vlm.bin:0" in raw and b"vlm.bin:1" in raw and b"aex.bin:0" not in raw


def test_reference_loaders_read_the_gguf(ob, models, ck):
    """The reference's own ActTransformer / OctoTransformer / SmolVLA loaders
    give bit-identical outputs from the GGUF and from the directory."""
    d, g, c = models["act"]
    feats, state = ck.act_inputs(c)
    outs = [ob.RefAct(p, c["img_ch"], 31, c["chunk"], c["action_dim"]).forward(feats, 1, c["fh"], c["fw"], state)
            for p in (d, g)]
    assert outs[0].tobytes() == outs[1].tobytes()
    d, g, c = models["octo"]
    t5, sp, sw, tm = ck.octo_inputs(c)
    outs = [ob.RefOcto(p, 7, c["d"]).forward(t5, sp, sw, 2, tm) for p in (d, g)]
    assert outs[0].tobytes() == outs[1].tobytes()
    d, g, c = models["smolvla"]
    prefix, pad, noise = ck.smolvla_inputs(c, n_pad=2)
    outs = [ob.RefSmolvla(p, 48).run(prefix, pad, noise) for p in (d, g)]
    assert outs[0].tobytes() == outs[1].tobytes()
    d, g, c = models["siglip"]
    px = ck.siglip_inputs(c)
    outs = [ob.RefSiglip(p, 15, c["n_img_tok"], c["mm_out"]).encode(px) for p in (d, g)]
    assert outs[0].tobytes() == outs[1].tobytes()


def test_mount_rule_and_sidecars(vla, ob, models, tmp_path):
    """A directory with exactly one .gguf and no .meta mounts the GGUF; with a
    .meta (a converted directory) or two GGUFs it is a plain directory. A
    file the GGUF does not carry is read from disk beside it."""
    _, g, _ = models["act"]
    d = tmp_path / "m"
    d.mkdir()
    (d / "model.gguf").write_bytes(open(g, "rb").read())
    (d / "config.txt").write_text("fps 30\n")
    f = vla.CkptFiles(str(d))
    assert f.gguf and "act.meta" in f.names()
    assert f.read("config.txt") == b"fps 30\n"                     # sidecar
    assert ob.ref_mount_read(str(d), "config.txt") == b"fps 30\n"
    assert f.size("nope.bin") == -1 and ob.ref_mount_read(str(d), "nope.bin") is None
    with pytest.raises(vla.VlaError):
        f.read("nope.bin")
    f2 = vla.CkptFiles(str(d / "model.gguf") + "/")                 # the file itself, trailing slash
    assert f2.gguf and f2.read("config.txt") == b"fps 30\n"
    (d / "other.meta").write_text("x 1\n")                          # now a converted directory
    f3 = vla.CkptFiles(str(d))
    assert not f3.gguf and f3.size("act.meta") == -1
    assert ob.ref_mount_read(str(d), "act.meta") is None
    (d / "other.meta").unlink()
    (d / "second.gguf").write_bytes(b"GGUF")                         # two GGUFs: a directory
    assert not vla.CkptFiles(str(d)).gguf


# ------------------------------------------------------------- malformed --

def _valid(ck, files=None, tensors=None, version=3):
    b = ck.GgufBuilder(version)
    b.string("general.architecture", "vla-simd")
    b.scalar("vla_simd.format", 4, 1)
    for rel, text in ({"a.meta": "k 1\n"} if files is None else files).items():
        b.string(f"vla_simd.file.{rel}", text)
    if tensors is None:
        tensors = [("w.bin", np.arange(8, dtype=np.float32).tobytes())]
    for name, data in tensors:
        b.tensor(name, data, 0)
    return b


def _builders(ck):
    """(label, bytes) of GGUFs both readers must refuse."""
    w = np.arange(8, dtype=np.float32).tobytes()
    whole = _valid(ck).tobytes()
    out = [(f"truncated at {cut}", whole[:cut]) for cut in (3, 20, 30, len(whole) // 2, len(whole) - 1)]
    out.append(("bad magic", b"GGUX" + whole[4:]))
    for v in (1, 4, 9):
        out.append((f"version {v}", whole[:4] + struct.pack("<I", v) + whole[8:]))
    b = _valid(ck)
    b.scalar("dup", 4, 1)
    b.scalar("dup", 4, 2)
    out.append(("duplicate metadata", b.tobytes()))
    out.append(("duplicate tensor", _valid(ck, tensors=[("w.bin", w), ("w.bin", w)]).tobytes()))
    b = _valid(ck, tensors=[])
    b.tensor("w.bin", w, 0, offset=4)
    out.append(("misaligned offset", b.tobytes()))
    b = _valid(ck, tensors=[])
    b.tensor("w.bin", w, 0, dims=[1 << 32, 1 << 32])
    out.append(("overflowing shape", b.tobytes()))
    b = _valid(ck, tensors=[])
    b.tensor("w.bin", w, 0, dims=[1 << 20])
    out.append(("tensor past the end", b.tobytes()))
    for label, ty, val in (("alignment 0", 4, 0), ("alignment 48", 4, 48), ("alignment as f64", 12, 32.0)):
        b = _valid(ck)
        b.scalar("general.alignment", ty, val)
        out.append((label, b.tobytes()))
    for rel in ("../escape.txt", "/absolute.txt", "tok/../../escape", "./here.txt", "dir/"):
        out.append((f"unsafe path {rel!r}", _valid(ck, files={rel: "x"}).tobytes()))
        out.append((f"unsafe tensor path {rel!r}", _valid(ck, tensors=[(rel, w)]).tobytes()))
    for names in (["w.bin:1"], ["w.bin:0", "w.bin:2"], ["w.bin", "w.bin:0"], ["w.bin:0", "w.bin"],
                  ["w.bin:00"]):
        out.append((f"parts {names}", _valid(ck, tensors=[(n, w) for n in names]).tobytes()))
    out.append(("text file and tensor of one name", _valid(ck, files={"w.bin": "x"}).tobytes()))
    b = ck.GgufBuilder()
    b.string("general.architecture", "vla-simd")
    b.scalar("vla_simd.format", 4, 2)
    b.tensor("w.bin", w, 0)
    out.append(("format 2", b.tobytes()))
    b = ck.GgufBuilder()
    b.string("general.architecture", "vla-simd")
    b.tensor("w.bin", w, 0)
    out.append(("no format", b.tobytes()))
    b = ck.GgufBuilder()
    b.string("general.architecture", "llama")
    b.scalar("vla_simd.format", 4, 1)
    b.tensor("w.bin", w, 0)
    out.append(("another architecture", b.tobytes()))
    b = _valid(ck, tensors=[])
    b.tensor("w.bin", bytes(18), 2, dims=[32])  # Q4_0 blocks: no fixed element size
    out.append(("quantized tensor type", b.tobytes()))
    b = _valid(ck)
    b.scalar("vla_simd.file.n.txt", 4, 3)
    out.append(("embedded file that is not a string", b.tobytes()))
    b = ck.GgufBuilder()
    b.string("general.architecture", "vla-simd")
    b.scalar("vla_simd.format", 4, 1)
    out.append(("no files", b.tobytes()))
    b = _valid(ck)
    b.raw_kv(ck.GgufBuilder._s("nested") + struct.pack("<IIQ", 9, 9, 1) + struct.pack("<IQ", 4, 0))
    out.append(("nested array", b.tobytes()))
    b = _valid(ck)
    b.raw_kv(ck.GgufBuilder._s("big") + struct.pack("<IIQ", 9, 12, 1000000))
    out.append(("truncated metadata array", b.tobytes()))
    return out


def test_malformed_ggufs_are_refused_like_the_reference(vla, ob, ck, tmp_path):
    for label, data in _builders(ck):
        p = tmp_path / "bad.gguf"
        p.write_bytes(data)
        with pytest.raises(vla.VlaError) as e:
            vla.CkptFiles(str(p))
        assert e.value.status == vla.VLA_ERR_ARG, label
        with pytest.raises(ValueError):
            ob.ref_mount_read(str(p), "a.meta")
        print(f"refused ({label}): {e.value}")


def test_valid_variants_accepted_like_the_reference(vla, ob, ck, tmp_path):
    """GGUF v2, a 64-byte alignment, metadata arrays of strings and numbers, an
    I8 + I32 + F16 .bin in parts, nested directories and an empty text file."""
    i8 = np.arange(-5, 6, dtype=np.int8).tobytes()
    i32 = np.array([7, -9], np.int32).tobytes()
    f16 = np.array([1.5, -2.0, 65504.0], np.float16).tobytes()
    for version, align in ((2, 32), (3, 64)):
        b = ck.GgufBuilder(version, align)
        b.string("general.architecture", "vla-simd")
        b.scalar("vla_simd.format", 10, 1)                   # u64 format
        if align != 32:
            b.scalar("general.alignment", 4, align)
        b.array("tokens", 8, ["a", "bb", ""])
        b.array("ids", 5, [1, -2, 3])
        b.string("vla_simd.file.tok/vocab.txt", "a\nbb\n")
        b.string("vla_simd.file.empty.bin", "")
        b.tensor("mix.bin:0", i8, 24)
        b.tensor("mix.bin:1", i32, 26)
        b.tensor("mix.bin:2", f16, 1)
        p = tmp_path / f"ok{version}.gguf"
        p.write_bytes(b.tobytes())
        f = vla.CkptFiles(str(p))
        assert f.names() == ["empty.bin", "mix.bin", "tok/vocab.txt"]
        assert f.read("mix.bin") == i8 + i32 + f16 == ob.ref_mount_read(str(p), "mix.bin")
        assert f.read("tok/vocab.txt") == b"a\nbb\n" == ob.ref_mount_read(str(p), "tok/vocab.txt")
        assert f.read("empty.bin") == b"" == ob.ref_mount_read(str(p), "empty.bin")
