// tokenizer.h - the byte-level BPE tokenizer SmolVLA's language prompt goes
// through before its token ids index the embedding table
// (src/tokenizer/tokenizer.{h,cpp}, called from smolvla_capi.cpp's
// vla_smolvla_tokenize).
//
// Behaviour kept from the reference, since the ids must be the same:
//   * files: vocab.txt lines "<id>\t<token>" (std::stoi of the id; lines with
//     no tab are skipped; a later line for the same token wins), merges.txt
//     lines "<left> <right>" split at the first space, ranked by their order
//     among the lines that have a space;
//   * the GPT-2 byte alphabet: bytes 33-126, 161-172 and 174-255 stand for
//     themselves, the other 68 bytes for code points 256, 257, ... in byte
//     order, each written as UTF-8;
//   * pre-tokenization: every digit is a piece of its own; the text between
//     digits splits into the GPT-2 pieces (the contractions 's 't 'm 'd 're
//     've 'll, an optional space + a run of letters or of other symbols, and
//     whitespace runs that leave their last character to the next piece),
//     with the reference's code-point tables for what counts as a letter,
//     a number and a space outside ASCII;
//   * merging: repeatedly merge the leftmost adjacent pair of lowest rank, one
//     pair per round; symbols missing from the vocabulary are dropped.
// Host code: tokenization is string work on a few dozen bytes per query.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace vla {
namespace hip {

class BpeTokenizer {
public:
    // the text of vocab.txt and merges.txt; false when either table is empty
    // (the reference's load result); std::stoi's exceptions propagate
    bool load(const std::string& vocab_txt, const std::string& merges_txt);
    std::vector<int32_t> encode(const std::string& text) const;
    size_t vocab_size() const { return vocab_.size(); }

private:
    void encode_piece(const char* p, size_t n, std::vector<int32_t>& out) const;
    std::unordered_map<std::string, int32_t> vocab_;
    std::unordered_map<std::string, int32_t> rank_;  // key "left right" (left holds no space)
    std::string byte_sym_[256];
};

// Octo's SentencePiece unigram tokenizer for its T5 language tower
// (src/tokenizer/t5_tokenizer.{h,cpp}, called by OctoModel::lang_encode).
// Behaviour kept from the reference:
//   * vocab.txt lines "<piece>\t<score>" split at the last tab, the id the
//     line's index among lines with a tab (std::stod of the score); a piece of
//     score 0 is usable only when written "<...>" (the special pieces); the
//     first line of a piece wins;
//   * normalization: UTF-8 decoded with U+FFFD for ill-formed sequences
//     (maximal subparts), C0/C1 controls deleted, full-width ASCII folded,
//     a table of compatibility decompositions, whitespace runs -> one U+2581
//     before the next word;
//   * Viterbi over the bytes of the normalized text, each piece scored by its
//     vocab score, one UTF-8 character as <unk> at (lowest score - 10), ties
//     to the earlier candidate; consecutive <unk> collapse to one;
//   * special pieces written literally ("<...>" of score 0) are emitted as
//     themselves; the ids are cut to max_len - 1, </s> (1) appended, <pad> (0)
//     to max_len.
class UnigramTokenizer {
public:
    // false when vocab.txt has no "piece\tscore" line; std::stod's exceptions propagate
    bool load(const std::string& vocab_txt);
    std::vector<int32_t> encode(const std::string& text, int max_len) const;
    static constexpr int32_t kPad = 0, kEos = 1, kUnk = 2;

private:
    void encode_words(const std::string& text, std::vector<int32_t>& ids) const;
    std::unordered_map<std::string, int32_t> piece_;
    std::vector<double> score_;
    int max_len_ = 1;
    double min_score_ = 0.0;
};

}  // namespace hip
}  // namespace vla
