"""SmolVLA's byte-level BPE tokenizer (vla_bpe_*, host code in
libvla_simd_hip.so) against the reference's own Tokenizer
(src/tokenizer/tokenizer.cpp, compiled into oracle/_ref/libvla_ref.so), on a
tokenizer directory trained by vla_simd_amd.checkpoints.write_bpe_tokenizer.

The cases cover each rule of the pre-tokenizer: contractions (lower case
only), letter / number / other runs with an optional leading space, digits
one per piece, whitespace runs that leave their last character to the next
piece, the non-ASCII letter / number / space tables, 4-byte characters, and
malformed UTF-8 (a lone continuation byte, a truncated sequence, 0xF8-0xFF
lead bytes), plus seeded random strings over a mixed alphabet. The ids must be
identical. No device is needed.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import load_pkg, oracle

CASES = [
    "", " ", "a", "pick up the red block\n", "Pick Up THE Red Block",
    "don't", "I'll we're you've she'd it's they'm", "DON'T 'S 'Ll", "'", "''", "'x", "rock'n'roll",
    "12345", "move 10 cm, then 2.5 cm", "a1b2c3", " 7", "x  9",
    "a   b", "   leading", "trailing   ", "\t\n mixed \r\n\tspace", "a \n b", "  \n", "end\n\n\n",
    "café niño über", "Привет мир", "日本語のテキスト", "한국어", "ελληνικά", "עברית", "عربى",
    "٣٤٥ ²³ ½ ① ０１２", "x y　z w v", "\u0085next",
    "emoji 🤖 robot 🦾 arm", "mixed🤖123abc!!", "tab\tsep\tvalues",
    "!!!???...", " !?", "path/to/file.txt", "a-b_c=d+e", "(nested [brackets] {here})",
]

BAD_BYTES = [b"\x80abc", b"abc\xe2\x82", b"\xff\xfe ok", b"\xf8\x88\x80\x80\x80", b"\xc3", b"x\xc3(y",
             b"\xe2\x28\xa1", b"\xf0\x9f\xa4", b" \xed\xa0\x80 surrogate"]


@pytest.fixture(scope="module")
def toks(tmp_path_factory):
    pkg = load_pkg()
    import vla_simd_amd.checkpoints as ck
    ob = oracle()
    d = ck.write_bpe_tokenizer(str(tmp_path_factory.mktemp("tok")))
    return pkg.BpeTokenizer(d), ob.RefBpe(d), d


def test_cases_match_reference(toks):
    ours, ref, _ = toks
    for text in CASES:
        assert ours.encode(text) == ref.encode(text), repr(text)
    for b in BAD_BYTES:
        assert ours.encode(b) == ref.encode(b), repr(b)


def test_merges_are_applied(toks):
    """The trained merges really fire (a sentence from the corpus takes far
    fewer ids than bytes), so the comparison covers the merge loop."""
    ours, _, _ = toks
    s = "pick up the red block and put it in the box."
    assert len(ours.encode(s)) < len(s.encode()) // 2


def test_random_strings_match_reference(toks):
    ours, ref, _ = toks
    alphabet = list("abcdefghij ABC  \t\n'0123456789.,!?-") + ["é", "ж", "語", "٣", " ", "🤖", "ß"]
    r = np.random.default_rng(7)
    for _ in range(300):
        n = int(r.integers(0, 40))
        text = "".join(alphabet[int(k)] for k in r.integers(0, len(alphabet), size=n))
        assert ours.encode(text) == ref.encode(text), repr(text)


def test_load_errors(tmp_path):
    pkg = load_pkg()
    with pytest.raises(pkg.VlaError):
        pkg.BpeTokenizer(str(tmp_path / "missing"))
    (tmp_path / "vocab.txt").write_text("0\ta\n")
    (tmp_path / "merges.txt").write_text("#nospace\n")  # no line with a space: no merges
    with pytest.raises(pkg.VlaError):
        pkg.BpeTokenizer(str(tmp_path))
