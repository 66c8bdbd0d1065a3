"""Octo's SentencePiece unigram tokenizer (vla_unigram_*, host code in
libvla_simd_hip.so) against the reference's own T5Tokenizer
(src/tokenizer/t5_tokenizer.cpp, compiled into oracle/_ref/libvla_ref.so), on
a vocab written by vla_simd_amd.checkpoints.write_t5_vocab.

The cases cover the normalization (controls deleted, full-width ASCII folded,
the compatibility decompositions, every whitespace code point, U+FFFD for
ill-formed UTF-8), the Viterbi with <unk> fallback and <unk> collapsing,
literal special pieces, the score-0 rule, duplicate pieces, truncation to
max_len - 1 + </s>, padding, and seeded random strings. No device is needed.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import load_pkg, oracle

CASES = [
    "", " ", "pick up the red block", "Pick Up The Red Block", "  pick   up\tthe\nred\r\nblock  ",
    "place the cup on the plate, then open the drawer.", "push the green button twice; don't drop it!",
    "ＰＩＣＫ ｕｐ！", "½ cup ² … ‼ ⁇ ﬁ ĳ ſ", "\x01pick\x7fup\x1f", "a　b c﻿d e▁f",
    "xyzzy qqq", "unknown ЖЖЖ 日本 🤖🤖", "<extra_id_0> pick <extra_id_0>", "<unk> <pad> </s>", "<notapiece>",
    "a<b>c", "<<extra_id_0>>", "zzz", "the the the the the the the the the the the the the the the the the",
]
BAD = [b"\xff\xfe pick", b"up\xc3", b"\xe2\x28\xa1 the", b"\xed\xa0\x80x", b"\xf0\x9f\xa4 box", b"\xf5\x80\x80"]


@pytest.fixture(scope="module")
def toks(tmp_path_factory):
    pkg = load_pkg()
    import vla_simd_amd.checkpoints as ck
    d = ck.write_t5_vocab(str(tmp_path_factory.mktemp("t5tok")))
    return pkg.UnigramTokenizer(d), oracle().RefT5Tok(d)


@pytest.mark.parametrize("max_len", [1, 4, 16, 40])
def test_cases_match_reference(toks, max_len):
    ours, ref = toks
    for t in CASES:
        assert ours.encode(t, max_len) == ref.encode(t, max_len), repr(t)
    for b in BAD:
        assert ours.encode(b, max_len) == ref.encode(b, max_len), repr(b)


def test_pieces_and_unknowns(toks):
    ours, _ = toks
    ids = ours.encode("pick up the red block", 16)
    assert ids[:5].count(2) == 0 and 1 in ids and ids[-1] == 0  # known pieces, </s>, padding
    ids = ours.encode("ЖЖЖ", 8)  # the word marker, one <unk> for the run, then </s>
    assert ids[1:3] == [2, 1] and ids[0] != 2


def test_random_strings_match_reference(toks):
    ours, ref = toks
    alphabet = list("pickuthredblos  \t\n.,!<>'") + ["Ж", "½", "Ｐ", "　", "\x01", "…", "🤖", "▁"]
    r = np.random.default_rng(11)
    for _ in range(300):
        n = int(r.integers(0, 30))
        text = "".join(alphabet[int(k)] for k in r.integers(0, len(alphabet), size=n))
        assert ours.encode(text, 16) == ref.encode(text, 16), repr(text)


def test_crafted_vocab_matches_reference(tmp_path):
    """A vocab a SentencePiece export never writes, chosen so that a slip in
    the segmentation or the file rules fails: a repeated piece whose later,
    lower score still lowers the <unk> score (the first line keeps the id and
    score; with the <unk> score at -50 the four one-byte pieces of U+1F916 win
    at -24, with it at -17 the single <unk> would), equal-score segmentations
    (the first candidate found wins), pieces that end inside a UTF-8
    character, an unusable score-0 line before a usable line of the same
    piece, and a special piece with a '<' inside it."""
    pkg = load_pkg()
    lines = [b"<pad>\t0", b"</s>\t0", b"<unk>\t0",
             "\u2581ab\t-2".encode(), "\u2581a\t-1".encode(), b"b\t-1", b"ab\t-1.5",
             "\u2581\t-0.5".encode(), b"a\t-1",
             "\u2581a\t-40".encode(),          # repeat: ignored, but lowers the <unk> score
             b"c\t0", b"c\t-3",                 # unusable, then usable
             b"\xe2\x96\t-7",                  # the first two bytes of U+2581
             b"\xf0\t-6", b"\x9f\t-6", b"\xa4\t-6", b"\x96\t-6",
             b"<a<b>\t0", b"<b>\t0", b"<x>\t-1"]
    (tmp_path / "vocab.txt").write_bytes(b"\n".join(lines) + b"\n")
    ours, ref = pkg.UnigramTokenizer(str(tmp_path)), oracle().RefT5Tok(str(tmp_path))
    texts = ["ab", "a b", "abab c", "cab", "\u0416 ab", "<a<b>", "x<a<b>y<b>z", "<b><b>", "<x> <b>", "a<b",
             "<a<b>>", "ab ab ab ab", "\u0416\u0416 c \u0416\u0416", "\U0001F916", "a\U0001F916b"]
    for t in texts:
        for max_len in (1, 3, 12):
            assert ours.encode(t, max_len) == ref.encode(t, max_len), (t, max_len)
    # the byte pieces of U+1F916 win over one <unk> (lowest score -40, not -7)
    assert ours.encode("\U0001F916", 8)[1:5] == [13, 14, 15, 16]
