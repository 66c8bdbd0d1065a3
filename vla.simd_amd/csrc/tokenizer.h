// tokenizer.h - the two host tokenizers the model-level entry points need
// before token ids index an embedding table on the device:
//   * BpeTokenizer: SmolVLA's byte-level BPE (src/tokenizer/tokenizer.{h,cpp},
//     called from smolvla_capi.cpp's vla_smolvla_tokenize);
//   * UnigramTokenizer: Octo's SentencePiece unigram model for its T5 tower
//     (src/tokenizer/t5_tokenizer.{h,cpp}, called by OctoModel::lang_encode).
// Host code: tokenization is string work on a few dozen bytes per query.
//
// BPE behaviour kept from the reference, since the ids must be the same:
//   * files: vocab.txt lines "<id>\t<token>" (std::stoi of the id; lines with
//     no tab are skipped; a later line for the same token wins), merges.txt
//     lines "<left> <right>" split at the first space, ranked by their order
//     among the lines that have a space (a repeated pair keeps its last rank);
//   * the GPT-2 byte alphabet: bytes 33-126, 161-172 and 174-255 stand for
//     themselves, the other 68 bytes for code points 256, 257, ... in byte
//     order, each written as UTF-8;
//   * pre-tokenization: every digit is a piece of its own; the text between
//     digits splits into the GPT-2 pieces (the contractions 's 't 'm 'd 're
//     've 'll, an optional space + a run of letters or of other symbols, and
//     whitespace runs that leave their last character to the next piece),
//     with the reference's code-point tables for what counts as a letter,
//     a number and a space outside ASCII;
//   * merging: repeatedly merge the adjacent pair of lowest rank, the leftmost
//     one on a tie, one pair per round; symbols missing from the vocabulary
//     are dropped.
//
// Design: symbols are interned strings, a merge rule maps a pair of symbol ids
// to (rank, merged id), a word is a linked list of symbol nodes, and the pairs
// wait in a min-heap ordered by (rank, position) with stale entries dropped
// when popped. The pre-tokenizer decodes the text once into characters with a
// class each and precomputed run ends.
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
    size_t vocab_size() const { return n_vocab_; }

private:
    struct Rule {
        int32_t rank;
        int32_t merged;  // symbol id of left + right
    };
    int32_t intern(const std::string& s);
    void merge_word(const unsigned char* bytes, size_t n, std::vector<int32_t>& out) const;

    std::unordered_map<std::string, int32_t> sym_of_;  // symbol text -> symbol id
    std::vector<int32_t> vocab_of_sym_;                // symbol id -> token id, or -1
    std::unordered_map<uint64_t, Rule> rules_;         // (left id << 32 | right id) -> rule
    int32_t byte_sym_[256] = {};
    size_t n_vocab_ = 0;
};

// Octo's SentencePiece unigram tokenizer.
// Behaviour kept from the reference:
//   * vocab.txt lines "<piece>\t<score>" split at the last tab, the id the
//     line's index among lines with a tab (std::stod of the score); a piece of
//     score 0 is usable only when written "<...>" (the special pieces); the
//     first line of a piece wins;
//   * normalization: UTF-8 decoded with U+FFFD for ill-formed sequences
//     (maximal subparts), C0/C1 controls deleted, full-width ASCII folded,
//     a table of compatibility decompositions, whitespace runs -> one U+2581
//     before the next word;
//   * best segmentation of the bytes of the normalized text, each piece scored
//     by its vocab score, one UTF-8 character as <unk> at (lowest score - 10),
//     ties to the candidate found first (shorter pieces first, the <unk>
//     character last); consecutive <unk> collapse to one;
//   * special pieces written literally ("<...>" of score 0) are emitted as
//     themselves; the ids are cut to max_len - 1, </s> (1) appended, <pad> (0)
//     to max_len.
// Design: the usable pieces sit in a byte trie, so the segmentation walks the
// trie from each reachable position instead of looking up every substring.
class UnigramTokenizer {
public:
    // false when vocab.txt has no "piece\tscore" line; std::stod's exceptions propagate
    bool load(const std::string& vocab_txt);
    std::vector<int32_t> encode(const std::string& text, int max_len) const;
    static constexpr int32_t kPad = 0, kEos = 1, kUnk = 2;

private:
    void segment(const std::string& text, std::vector<int32_t>& ids) const;
    int32_t child(int32_t node, unsigned char b) const;

    // trie: node 0 is the root; edges keyed (node << 8 | byte)
    std::unordered_map<uint64_t, int32_t> edge_;
    std::vector<int32_t> node_piece_;  // piece id ending at a node, or -1
    std::vector<double> score_;        // by piece id (every line with a tab)
    size_t longest_ = 1;               // bytes of the longest usable piece
    double lowest_ = 0.0;              // lowest usable score (at most 0)
};

}  // namespace hip
}  // namespace vla
