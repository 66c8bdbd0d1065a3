// tokenizer.cpp - byte-level BPE (see tokenizer.h). Follows
// src/tokenizer/tokenizer.cpp: the byte alphabet (:16-49), the character
// classes (:51-95), the piece rule (:97-120), the tables (:122-151) and the
// merge loop (:153-180).
#include "tokenizer.h"

#include <algorithm>
#include <climits>
#include <limits>
#include <sstream>

namespace vla {
namespace hip {

namespace {

enum class Cls { Letter, Number, Space, Other };

struct Range {
    uint32_t lo, hi;
};

// The code points outside ASCII the reference treats as whitespace, numbers
// and letters (tokenizer.cpp:73-93): a fixed approximation of \s, \p{N} and
// \p{L}, kept as is so both sides split a prompt the same way.
constexpr Range kSpace[] = {{0x85, 0x85},     {0xA0, 0xA0},     {0x1680, 0x1680}, {0x2000, 0x200A},
                            {0x2028, 0x2029}, {0x202F, 0x202F}, {0x205F, 0x205F}, {0x3000, 0x3000}};
constexpr Range kNumber[] = {{0xB2, 0xB3},     {0xB9, 0xB9},     {0xBC, 0xBE},     {0x660, 0x669},
                             {0x6F0, 0x6F9},   {0x966, 0x96F},   {0x2070, 0x2070}, {0x2074, 0x2079},
                             {0x2080, 0x2089}, {0x2150, 0x2182}, {0x2185, 0x2189}, {0x2460, 0x249B},
                             {0x24EA, 0x24FF}, {0x2776, 0x2793}, {0x3007, 0x3007}, {0x3021, 0x3029},
                             {0xFF10, 0xFF19}};
constexpr Range kLetter[] = {{0xAA, 0xAA},     {0xB5, 0xB5},     {0xBA, 0xBA},     {0xC0, 0xD6},
                             {0xD8, 0xF6},     {0xF8, 0x2C1},    {0x370, 0x373},   {0x376, 0x377},
                             {0x37B, 0x37D},   {0x386, 0x386},   {0x388, 0x3FF},   {0x400, 0x481},
                             {0x48A, 0x52F},   {0x531, 0x556},   {0x561, 0x587},   {0x5D0, 0x5EA},
                             {0x620, 0x64A},   {0x1E00, 0x1FBC}, {0x3041, 0x3096}, {0x30A1, 0x30FA},
                             {0x3400, 0x4DBF}, {0x4E00, 0x9FFF}, {0xAC00, 0xD7A3}, {0xF900, 0xFAFF},
                             {0xFF21, 0xFF3A}, {0xFF41, 0xFF5A}};

template <size_t N>
bool in(const Range (&t)[N], uint32_t cp) {
    for (const Range& r : t)
        if (cp >= r.lo && cp <= r.hi) return true;
    return false;
}

// The class of the character at s[i] (i < end) and its length in bytes. A
// malformed or truncated UTF-8 sequence is one byte of class Other.
Cls classify(const std::string& s, size_t i, size_t end, size_t* len) {
    const unsigned char c = (unsigned char)s[i];
    *len = 1;
    if (c < 0x80) {
        if ((c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z')) return Cls::Letter;
        if (c >= '0' && c <= '9') return Cls::Number;
        if (c == ' ' || (c >= '\t' && c <= '\r')) return Cls::Space;
        return Cls::Other;
    }
    // the lead byte alone decides the length (0xF8..0xFF read as four bytes)
    size_t n = 0;
    if (c >= 0xF0) n = 4;
    else if (c >= 0xE0) n = 3;
    else if (c >= 0xC0) n = 2;
    if (n == 0 || n > end - i) return Cls::Other;
    uint32_t cp = c & (0x7Fu >> n);
    for (size_t k = 1; k < n; k++) {
        const unsigned char d = (unsigned char)s[i + k];
        if ((d & 0xC0) != 0x80) return Cls::Other;
        cp = (cp << 6) | (d & 0x3Fu);
    }
    *len = n;
    if (in(kSpace, cp)) return Cls::Space;
    if (in(kNumber, cp)) return Cls::Number;
    if (in(kLetter, cp)) return Cls::Letter;
    return Cls::Other;
}

// end of the run of class `want` starting at i
size_t run_end(const std::string& s, size_t i, size_t end, Cls want) {
    size_t n;
    while (i < end && classify(s, i, end, &n) == want) i += n;
    return i;
}

// Length of the piece starting at i in a digit-free span [i, end):
// the GPT-2 rule  's|'t|'re|'ve|'m|'ll|'d| ?L+| ?N+| ?O+|\s+(?!\S)|\s+
size_t piece_len(const std::string& s, size_t i, size_t end) {
    if (s[i] == '\'' && i + 1 < end) {
        const char a = s[i + 1];
        const char b = i + 2 < end ? s[i + 2] : '\0';
        if (a == 's' || a == 't' || a == 'm' || a == 'd') return 2;
        if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) return 3;
    }
    size_t n;
    const size_t j = s[i] == ' ' ? i + 1 : i;  // an optional leading space
    if (j < end) {
        const Cls cj = classify(s, j, end, &n);
        if (cj != Cls::Space) return run_end(s, j, end, cj) - i;
    }
    // whitespace: to the end of the text, or up to (not including) the last
    // whitespace character before the next non-space, when that leaves any
    const size_t k = run_end(s, i, end, Cls::Space);
    if (k == end) return k - i;
    size_t last = i;
    for (size_t p = i; p < k; p += n) {
        classify(s, p, end, &n);
        last = p;
    }
    return last > i ? last - i : k - i;
}

void utf8_append(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
        out += (char)cp;
    } else {  // cp < 0x800 for every symbol of the byte alphabet
        out += (char)(0xC0 | (cp >> 6));
        out += (char)(0x80 | (cp & 0x3F));
    }
}

}  // namespace

bool BpeTokenizer::load(const std::string& vocab_txt, const std::string& merges_txt) {
    vocab_.clear();
    rank_.clear();
    uint32_t shifted = 256;
    for (int b = 0; b < 256; b++) {
        const bool self = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
        byte_sym_[b].clear();
        utf8_append(byte_sym_[b], self ? (uint32_t)b : shifted++);
    }
    std::istringstream vf(vocab_txt);
    std::string line;
    while (std::getline(vf, line)) {
        const size_t tab = line.find('\t');
        if (tab == std::string::npos) continue;
        vocab_[line.substr(tab + 1)] = (int32_t)std::stoi(line.substr(0, tab));
    }
    std::istringstream mf(merges_txt);
    int32_t r = 0;
    while (std::getline(mf, line)) {
        if (line.find(' ') == std::string::npos) continue;
        rank_[line] = r++;  // "left right": the key is the line itself
    }
    return !vocab_.empty() && !rank_.empty();
}

void BpeTokenizer::encode_piece(const char* p, size_t n, std::vector<int32_t>& out) const {
    std::vector<std::string> sym(n);
    for (size_t i = 0; i < n; i++) sym[i] = byte_sym_[(unsigned char)p[i]];
    std::string key;
    while (sym.size() > 1) {
        int32_t best = INT_MAX;
        size_t at = 0;
        bool found = false;
        for (size_t i = 0; i + 1 < sym.size(); i++) {
            key.assign(sym[i]).append(1, ' ').append(sym[i + 1]);
            const auto it = rank_.find(key);
            if (it != rank_.end() && it->second < best) {
                best = it->second;
                at = i;
                found = true;
            }
        }
        if (!found) break;
        sym[at] += sym[at + 1];
        sym.erase(sym.begin() + (ptrdiff_t)at + 1);
    }
    for (const std::string& s : sym) {
        const auto it = vocab_.find(s);
        if (it != vocab_.end()) out.push_back(it->second);
    }
}

std::vector<int32_t> BpeTokenizer::encode(const std::string& text) const {
    std::vector<int32_t> ids;
    const size_t N = text.size();
    size_t b = 0;
    while (b < N) {
        size_t n;
        if (classify(text, b, N, &n) == Cls::Number) {  // one piece per digit
            encode_piece(text.data() + b, n, ids);
            b += n;
            continue;
        }
        size_t e = b;
        while (e < N && classify(text, e, N, &n) != Cls::Number) e += n;
        for (size_t i = b; i < e;) {
            const size_t len = piece_len(text, i, e);
            encode_piece(text.data() + i, len, ids);
            i += len;
        }
        b = e;
    }
    return ids;
}

}  // namespace hip
}  // namespace vla

// ---------------------------------------------------------------- unigram --
// src/tokenizer/t5_tokenizer.cpp: normalization tables (:13-44), load
// (:46-72), Viterbi (:82-137), specials and padding (:139-157).

namespace vla {
namespace hip {

namespace {

// The compatibility decompositions the reference applies (t5_tokenizer.cpp:
// 13-26): a code point and the up to five it becomes (0 ends the list).
constexpr uint32_t kCompat[][6] = {
    {0xA8, ' ', 0x308},  {0xAA, 'a'},  {0xAF, ' ', 0x304},  {0xB2, '2'},  {0xB3, '3'},  {0xB4, ' ', 0x301},
    {0xB5, 0x3BC},       {0xB8, ' ', 0x327}, {0xB9, '1'}, {0xBA, 'o'},   {0xBC, '1', 0x2044, '4'},
    {0xBD, '1', 0x2044, '2'}, {0xBE, '3', 0x2044, '4'}, {0x132, 'I', 'J'}, {0x133, 'i', 'j'},
    {0x13F, 'L', 0xB7},  {0x140, 'l', 0xB7}, {0x149, 0x2BC, 'n'}, {0x17F, 's'}, {0x340, 0x300},
    {0x341, 0x301},      {0x343, 0x313}, {0x344, 0x308, 0x301}, {0x2011, 0x2010}, {0x2017, ' ', 0x333},
    {0x2024, '.'},       {0x2025, '.', '.'}, {0x2026, '.', '.', '.'}, {0x2033, 0x2032, 0x2032},
    {0x2034, 0x2032, 0x2032, 0x2032}, {0x2036, 0x2035, 0x2035}, {0x2037, 0x2035, 0x2035, 0x2035},
    {0x203C, '!', '!'},  {0x203E, ' ', 0x305}, {0x2047, '?', '?'}, {0x2048, '?', '!'},
    {0x2049, '!', '?'},  {0x2057, 0x2032, 0x2032, 0x2032, 0x2032},
};

bool deleted_cp(uint32_t cp) {
    return (cp >= 1 && cp <= 8) || cp == 0xB || (cp >= 0xE && cp <= 0x1F) || cp == 0x7F || cp == 0x8F || cp == 0x9F;
}

bool space_cp(uint32_t cp) {
    switch (cp) {
    case ' ': case '\t': case '\n': case '\f': case '\r': case 0x85: case 0xA0: case 0x1680: case 0x2028:
    case 0x2029: case 0x202F: case 0x205F: case 0x2581: case 0x3000: case 0xFEFF: case 0xFFFD:
        return true;
    default:
        return cp >= 0x2000 && cp <= 0x200F;
    }
}

// UTF-8 -> code points; each maximal ill-formed subpart becomes U+FFFD (the
// Unicode well-formed byte table: lead C2..F4, second-byte limits for E0, ED,
// F0, F4)
std::vector<uint32_t> decode_utf8(const std::string& s) {
    std::vector<uint32_t> out;
    out.reserve(s.size());
    size_t i = 0;
    while (i < s.size()) {
        const unsigned char c = (unsigned char)s[i++];
        int need;
        if (c < 0x80) need = 0;
        else if (c >= 0xC2 && c <= 0xDF) need = 1;
        else if (c >= 0xE0 && c <= 0xEF) need = 2;
        else if (c >= 0xF0 && c <= 0xF4) need = 3;
        else {
            out.push_back(0xFFFD);
            continue;
        }
        uint32_t cp = need == 0 ? c : c & (0x3Fu >> need);
        unsigned char lo = 0x80, hi = 0xBF;
        if (c == 0xE0) lo = 0xA0;
        else if (c == 0xED) hi = 0x9F;
        else if (c == 0xF0) lo = 0x90;
        else if (c == 0xF4) hi = 0x8F;
        while (need > 0 && i < s.size()) {
            const unsigned char d = (unsigned char)s[i];
            if (d < lo || d > hi) break;
            cp = (cp << 6) | (d & 0x3Fu);
            i++;
            need--;
            lo = 0x80;
            hi = 0xBF;
        }
        out.push_back(need ? 0xFFFD : cp);
    }
    return out;
}

void encode_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
        out += (char)cp;
    } else if (cp < 0x800) {
        out += (char)(0xC0 | (cp >> 6));
        out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out += (char)(0xE0 | (cp >> 12));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    } else {
        out += (char)(0xF0 | (cp >> 18));
        out += (char)(0x80 | ((cp >> 12) & 0x3F));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    }
}

// bytes of the character a lead byte starts (1 for anything else)
int char_bytes(unsigned char c) {
    if ((c & 0x80) == 0) return 1;
    if ((c & 0xE0) == 0xC0) return 2;
    if ((c & 0xF0) == 0xE0) return 3;
    if ((c & 0xF8) == 0xF0) return 4;
    return 1;
}

}  // namespace

bool UnigramTokenizer::load(const std::string& vocab_txt) {
    piece_.clear();
    score_.clear();
    max_len_ = 1;
    min_score_ = 0.0;
    std::istringstream in(vocab_txt);
    std::string line;
    int32_t id = 0;
    while (std::getline(in, line)) {
        const size_t tab = line.rfind('\t');
        if (tab == std::string::npos) continue;
        const std::string piece = line.substr(0, tab);
        const double sc = std::stod(line.substr(tab + 1));
        const int32_t my = id++;
        score_.push_back(sc);
        const bool special = piece.size() >= 2 && piece.front() == '<' && piece.back() == '>';
        if (sc == 0.0 && !special) continue;
        piece_.emplace(piece, my);  // the first line of a piece keeps it
        if ((int)piece.size() > max_len_) max_len_ = (int)piece.size();
        if (sc < min_score_) min_score_ = sc;
    }
    return id > 0;
}

void UnigramTokenizer::encode_words(const std::string& text, std::vector<int32_t>& ids) const {
    // normalized text: every word preceded by U+2581 (UTF-8 E2 96 81)
    std::string s;
    bool at_space = true;
    auto emit = [&](uint32_t cp) {
        if (space_cp(cp)) {
            at_space = true;
            return;
        }
        if (at_space) {
            s += "\xE2\x96\x81";
            at_space = false;
        }
        encode_utf8(s, cp);
    };
    for (uint32_t cp : decode_utf8(text)) {
        if (deleted_cp(cp)) continue;
        if (cp >= 0xFF01 && cp <= 0xFF5D) cp -= 0xFEE0;  // full-width ASCII
        bool mapped = false;
        for (const auto& row : kCompat)
            if (row[0] == cp) {
                for (int k = 1; k < 6 && row[k]; k++) emit(row[k]);
                mapped = true;
            }
        if (!mapped) emit(cp);
    }

    // Viterbi: best[i] the top score of a segmentation of s[0, i)
    const int n = (int)s.size();
    const double NEG = -std::numeric_limits<double>::infinity(), unk = min_score_ - 10.0;
    std::vector<double> best(n + 1, NEG);
    std::vector<int> from(n + 1, -1);
    std::vector<int32_t> tok(n + 1, kUnk);
    best[0] = 0.0;
    std::string key;
    for (int i = 0; i < n; i++) {
        if (best[i] == NEG) continue;
        const int lmax = std::min(max_len_, n - i);
        for (int l = 1; l <= lmax; l++) {
            key.assign(s, i, l);
            const auto it = piece_.find(key);
            if (it == piece_.end()) continue;
            const double sc = best[i] + score_[it->second];
            if (sc > best[i + l]) {
                best[i + l] = sc;
                from[i + l] = i;
                tok[i + l] = it->second;
            }
        }
        const int l = char_bytes((unsigned char)s[i]);
        if (best[i] + unk > best[i + l]) {
            best[i + l] = best[i] + unk;
            from[i + l] = i;
            tok[i + l] = kUnk;
        }
    }
    std::vector<int32_t> rev;
    for (int i = n; i > 0; i = from[i])
        if (tok[i] != kUnk || rev.empty() || rev.back() != kUnk) rev.push_back(tok[i]);
    ids.insert(ids.end(), rev.rbegin(), rev.rend());
}

std::vector<int32_t> UnigramTokenizer::encode(const std::string& text, int max_len) const {
    if (max_len < 1) return {};
    std::vector<int32_t> ids;
    size_t done = 0;
    // special pieces written literally: "<...>" shorter than the longest
    // piece, in the vocabulary with score 0; the search resumes one byte
    // after each '<'
    for (size_t i = text.find('<'); i != std::string::npos; i = text.find('<', i + 1)) {
        const size_t j = text.find('>', i);
        if (j == std::string::npos) break;
        if (j - i >= (size_t)max_len_) continue;
        const auto it = piece_.find(text.substr(i, j + 1 - i));
        if (it == piece_.end() || score_[(size_t)it->second] != 0.0) continue;
        encode_words(text.substr(done, i - done), ids);
        ids.push_back(it->second);
        done = j + 1;
    }
    encode_words(text.substr(done), ids);
    if ((int)ids.size() > max_len - 1) ids.resize((size_t)(max_len - 1));
    ids.push_back(kEos);
    while ((int)ids.size() < max_len) ids.push_back(kPad);
    return ids;
}

}  // namespace hip
}  // namespace vla
