// tokenizer.cpp - byte-level BPE and SentencePiece unigram tokenizers (see
// tokenizer.h for the rules they keep). The ids must equal those of
// src/tokenizer/tokenizer.cpp (byte alphabet :16-49, character classes
// :51-95, piece rule :97-120, files :122-151, merge rule :153-180) and
// src/tokenizer/t5_tokenizer.cpp (tables :13-44, file :46-72, segmentation
// :82-137, specials and padding :139-157); the data structures are this
// file's own.
#include "tokenizer.h"

#include <algorithm>
#include <limits>
#include <queue>
#include <tuple>

namespace vla {
namespace hip {

namespace {

// Calls fn(line) for each '\n'-separated line of text (a trailing newline
// adds no line; every caller skips empty lines anyway).
template <class Fn>
void for_each_line(const std::string& text, Fn fn) {
    size_t at = 0;
    while (at < text.size()) {
        size_t nl = text.find('\n', at);
        if (nl == std::string::npos) nl = text.size();
        fn(text.substr(at, nl - at));
        at = nl + 1;
    }
}

void put_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
        out.push_back((char)cp);
        return;
    }
    int tail = cp < 0x800 ? 1 : cp < 0x10000 ? 2 : 3;
    static const unsigned char lead[4] = {0, 0xC0, 0xE0, 0xF0};
    out.push_back((char)(lead[tail] | (cp >> (6 * tail))));
    while (tail-- > 0) out.push_back((char)(0x80 | ((cp >> (6 * tail)) & 0x3F)));
}

// ------------------------------------------------------------ BPE classes --

enum Cls : uint8_t { kLetter, kNumber, kSpace, kOther };

struct ClassRange {
    uint32_t lo, hi;
    Cls cls;
};

// The code points above ASCII that the reference treats as whitespace,
// numbers and letters (tokenizer.cpp:73-93, a fixed approximation of \s,
// \p{N} and \p{L}), merged into one table sorted by code point; everything
// else above ASCII is "other".
constexpr ClassRange kClassTable[] = {
    {0x85, 0x85, kSpace},       {0xA0, 0xA0, kSpace},       {0xAA, 0xAA, kLetter},      {0xB2, 0xB3, kNumber},
    {0xB5, 0xB5, kLetter},      {0xB9, 0xB9, kNumber},      {0xBA, 0xBA, kLetter},      {0xBC, 0xBE, kNumber},
    {0xC0, 0xD6, kLetter},      {0xD8, 0xF6, kLetter},      {0xF8, 0x2C1, kLetter},     {0x370, 0x373, kLetter},
    {0x376, 0x377, kLetter},    {0x37B, 0x37D, kLetter},    {0x386, 0x386, kLetter},    {0x388, 0x3FF, kLetter},
    {0x400, 0x481, kLetter},    {0x48A, 0x52F, kLetter},    {0x531, 0x556, kLetter},    {0x561, 0x587, kLetter},
    {0x5D0, 0x5EA, kLetter},    {0x620, 0x64A, kLetter},    {0x660, 0x669, kNumber},    {0x6F0, 0x6F9, kNumber},
    {0x966, 0x96F, kNumber},    {0x1680, 0x1680, kSpace},   {0x1E00, 0x1FBC, kLetter},  {0x2000, 0x200A, kSpace},
    {0x2028, 0x2029, kSpace},   {0x202F, 0x202F, kSpace},   {0x205F, 0x205F, kSpace},   {0x2070, 0x2070, kNumber},
    {0x2074, 0x2079, kNumber},  {0x2080, 0x2089, kNumber},  {0x2150, 0x2182, kNumber},  {0x2185, 0x2189, kNumber},
    {0x2460, 0x249B, kNumber},  {0x24EA, 0x24FF, kNumber},  {0x2776, 0x2793, kNumber},  {0x3000, 0x3000, kSpace},
    {0x3007, 0x3007, kNumber},  {0x3021, 0x3029, kNumber},  {0x3041, 0x3096, kLetter},  {0x30A1, 0x30FA, kLetter},
    {0x3400, 0x4DBF, kLetter},  {0x4E00, 0x9FFF, kLetter},  {0xAC00, 0xD7A3, kLetter},  {0xF900, 0xFAFF, kLetter},
    {0xFF10, 0xFF19, kNumber},  {0xFF21, 0xFF3A, kLetter},  {0xFF41, 0xFF5A, kLetter},
};

constexpr bool class_table_sorted() {
    for (size_t i = 0; i < sizeof(kClassTable) / sizeof(kClassTable[0]); i++) {
        if (kClassTable[i].lo > kClassTable[i].hi) return false;
        if (i > 0 && kClassTable[i].lo <= kClassTable[i - 1].hi) return false;
    }
    return true;
}
static_assert(class_table_sorted(), "class ranges must be sorted and disjoint (binary search)");

Cls class_of_cp(uint32_t cp) {
    const ClassRange* end = kClassTable + sizeof(kClassTable) / sizeof(kClassTable[0]);
    const ClassRange* r =
        std::upper_bound(kClassTable, end, cp, [](uint32_t v, const ClassRange& e) { return v < e.lo; });
    if (r == kClassTable) return kOther;
    --r;
    return cp <= r->hi ? r->cls : kOther;
}

Cls class_of_ascii(unsigned char c) {
    if ((c | 0x20) >= 'a' && (c | 0x20) <= 'z') return kLetter;
    if (c >= '0' && c <= '9') return kNumber;
    if (c == ' ' || (c >= 0x09 && c <= 0x0D)) return kSpace;
    return kOther;
}

struct Char {
    uint32_t off;  // first byte
    uint8_t len;   // bytes
    Cls cls;
};

// The text as characters: the lead byte alone fixes the length (0xC0-0xDF
// two, 0xE0-0xEF three, 0xF0-0xFF four); a stray continuation byte, a
// sequence cut by the end of the text or one with a bad continuation byte is
// one byte of class "other".
std::vector<Char> split_chars(const std::string& t) {
    std::vector<Char> out;
    out.reserve(t.size());
    const size_t n = t.size();
    size_t i = 0;
    while (i < n) {
        const unsigned char c = (unsigned char)t[i];
        Char ch{(uint32_t)i, 1, kOther};
        if (c < 0x80) {
            ch.cls = class_of_ascii(c);
        } else if (c >= 0xC0) {
            const size_t len = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : 2;
            bool ok = i + len <= n;
            uint32_t cp = c & (0x7Fu >> len);
            for (size_t k = 1; ok && k < len; k++) {
                const unsigned char d = (unsigned char)t[i + k];
                ok = (d & 0xC0) == 0x80;
                cp = (cp << 6) | (d & 0x3Fu);
            }
            if (ok) {
                ch.len = (uint8_t)len;
                ch.cls = class_of_cp(cp);
            }
        }
        out.push_back(ch);
        i += ch.len;
    }
    return out;
}

bool contraction_letter(char a) { return a == 's' || a == 't' || a == 'm' || a == 'd'; }
bool contraction_pair(char a, char b) {
    return (a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l');
}

}  // namespace

int32_t BpeTokenizer::intern(const std::string& s) {
    const auto ins = sym_of_.emplace(s, (int32_t)sym_of_.size());
    return ins.first->second;
}

bool BpeTokenizer::load(const std::string& vocab_txt, const std::string& merges_txt) {
    sym_of_.clear();
    rules_.clear();
    vocab_of_sym_.clear();
    // the byte alphabet: printable Latin-1 bytes keep their code point, the
    // rest take 256, 257, ... in byte order
    uint32_t spare = 256;
    for (int b = 0; b < 256; b++) {
        const bool keeps = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || b >= 174;
        std::string s;
        put_utf8(s, keeps ? (uint32_t)b : spare++);
        byte_sym_[b] = intern(s);
    }
    std::unordered_map<std::string, int32_t> token_id;
    for_each_line(vocab_txt, [&](const std::string& line) {
        const size_t tab = line.find('\t');
        if (tab != std::string::npos) token_id[line.substr(tab + 1)] = (int32_t)std::stoi(line.substr(0, tab));
    });
    int32_t rank = 0;
    for_each_line(merges_txt, [&](const std::string& line) {
        const size_t sp = line.find(' ');
        if (sp == std::string::npos) return;
        const std::string left = line.substr(0, sp), right = line.substr(sp + 1);
        const int32_t l = intern(left), r = intern(right);
        const int32_t m = intern(left + right);
        rules_[(uint64_t)(uint32_t)l << 32 | (uint32_t)r] = Rule{rank++, m};
    });
    vocab_of_sym_.assign(sym_of_.size(), -1);
    for (const auto& kv : sym_of_) {
        const auto t = token_id.find(kv.first);
        if (t != token_id.end()) vocab_of_sym_[(size_t)kv.second] = t->second;
    }
    n_vocab_ = token_id.size();
    return !token_id.empty() && !rules_.empty();
}

void BpeTokenizer::merge_word(const unsigned char* bytes, size_t n, std::vector<int32_t>& out) const {
    // one node per byte; a merge keeps the left node and unlinks the right
    std::vector<int32_t> sym(n), next(n), prev(n);
    for (size_t i = 0; i < n; i++) {
        sym[i] = byte_sym_[bytes[i]];
        next[i] = i + 1 < n ? (int32_t)(i + 1) : -1;
        prev[i] = (int32_t)i - 1;
    }
    // candidate pairs by (rank, left node): the left node's index is its
    // first byte, so the smaller index is the leftmost pair
    using Cand = std::tuple<int32_t, int32_t, int32_t, int32_t, int32_t>;  // rank, left, right, lsym, rsym
    std::priority_queue<Cand, std::vector<Cand>, std::greater<Cand>> heap;
    auto offer = [&](int32_t l) {
        if (l < 0) return;
        const int32_t r = next[(size_t)l];
        if (r < 0) return;
        const auto it = rules_.find((uint64_t)(uint32_t)sym[(size_t)l] << 32 | (uint32_t)sym[(size_t)r]);
        if (it != rules_.end()) heap.emplace(it->second.rank, l, r, sym[(size_t)l], sym[(size_t)r]);
    };
    for (size_t i = 0; i + 1 < n; i++) offer((int32_t)i);
    while (!heap.empty()) {
        int32_t rank, l, r, ls, rs;
        std::tie(rank, l, r, ls, rs) = heap.top();
        heap.pop();
        // stale: either node took part in a later merge
        if (next[(size_t)l] != r || sym[(size_t)l] != ls || sym[(size_t)r] != rs) continue;
        sym[(size_t)l] = rules_.at((uint64_t)(uint32_t)ls << 32 | (uint32_t)rs).merged;
        next[(size_t)l] = next[(size_t)r];
        if (next[(size_t)r] >= 0) prev[(size_t)next[(size_t)r]] = l;
        next[(size_t)r] = -2;  // unlinked: no pair starting at r validates again
        offer(prev[(size_t)l]);
        offer(l);
    }
    for (int32_t i = n ? 0 : -1; i >= 0; i = next[(size_t)i]) {
        const int32_t id = vocab_of_sym_[(size_t)sym[(size_t)i]];
        if (id >= 0) out.push_back(id);
    }
}

std::vector<int32_t> BpeTokenizer::encode(const std::string& text) const {
    std::vector<int32_t> ids;
    const std::vector<Char> ch = split_chars(text);
    const size_t n = ch.size();
    // run_end[c]: one past the last character of the same class as c that
    // follows c without a break
    std::vector<uint32_t> run_end(n);
    for (size_t c = n; c-- > 0;)
        run_end[c] = (c + 1 < n && ch[c + 1].cls == ch[c].cls) ? run_end[c + 1] : (uint32_t)(c + 1);

    // the end (in characters) of the piece starting at c
    auto piece_end = [&](size_t c) -> size_t {
        const Cls k = ch[c].cls;
        if (k == kNumber) return c + 1;  // digits are pieces of their own
        const size_t b = ch[c].off;
        if (text[b] == '\'' && b + 1 < text.size()) {
            if (contraction_letter(text[b + 1])) return c + 2;
            if (b + 2 < text.size() && contraction_pair(text[b + 1], text[b + 2])) return c + 3;
        }
        // a space joins the letter or symbol run after it
        if (text[b] == ' ' && c + 1 < n && (ch[c + 1].cls == kLetter || ch[c + 1].cls == kOther))
            return run_end[c + 1];
        if (k != kSpace) return run_end[c];
        // whitespace: all of it before a digit or the end of the text,
        // otherwise all but its last character, which starts the next piece
        const size_t q = run_end[c];
        if (q == n || ch[q].cls == kNumber) return q;
        return q - c >= 2 ? q - 1 : q;
    };

    for (size_t c = 0; c < n;) {
        const size_t e = piece_end(c);
        const size_t b0 = ch[c].off, b1 = ch[e - 1].off + ch[e - 1].len;
        merge_word(reinterpret_cast<const unsigned char*>(text.data()) + b0, b1 - b0, ids);
        c = e;
    }
    return ids;
}

// ---------------------------------------------------------------- unigram --

namespace {

// The compatibility decompositions the reference applies (t5_tokenizer.cpp:
// 13-26), sorted by code point: a code point and the up to five it becomes
// (0 ends the list).
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
constexpr size_t kCompatRows = sizeof(kCompat) / sizeof(kCompat[0]);

constexpr bool compat_sorted() {
    for (size_t i = 1; i < kCompatRows; i++)
        if (kCompat[i][0] <= kCompat[i - 1][0]) return false;
    return true;
}
static_assert(compat_sorted(), "compatibility rows must be sorted (binary search)");

const uint32_t* compat_row(uint32_t cp) {
    size_t lo = 0, hi = kCompatRows;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (kCompat[mid][0] < cp) lo = mid + 1;
        else hi = mid;
    }
    return lo < kCompatRows && kCompat[lo][0] == cp ? kCompat[lo] : nullptr;
}

// C0/C1 controls the normalizer deletes (tab, newline, form feed and
// carriage return are whitespace instead)
bool is_deleted_cp(uint32_t cp) {
    if (cp == 0x7F || cp == 0x8F || cp == 0x9F || cp == 0x0B) return true;
    return (cp >= 0x01 && cp <= 0x08) || (cp >= 0x0E && cp <= 0x1F);
}

bool is_blank_cp(uint32_t cp) {
    if (cp < 0x80) return cp == ' ' || cp == '\t' || cp == '\n' || cp == '\f' || cp == '\r';
    if (cp >= 0x2000 && cp <= 0x200F) return true;
    static constexpr uint32_t kOthers[] = {0x85,   0xA0,   0x1680, 0x2028, 0x2029, 0x202F,
                                           0x205F, 0x2581, 0x3000, 0xFEFF, 0xFFFD};
    return std::binary_search(std::begin(kOthers), std::end(kOthers), cp);
}

// UTF-8 -> code points, each maximal ill-formed subpart replaced by one
// U+FFFD (Unicode 3.9, table 3-7 of well-formed byte sequences: the lead
// byte fixes the length and the range allowed for the first continuation
// byte; a byte outside it ends the subpart without being consumed).
std::vector<uint32_t> utf8_code_points(const std::string& s) {
    struct Lead {
        uint8_t tail, lo, hi;
    };
    auto lead_of = [](unsigned char c) -> Lead {
        if (c >= 0xC2 && c <= 0xDF) return {1, 0x80, 0xBF};
        if (c == 0xE0) return {2, 0xA0, 0xBF};
        if (c == 0xED) return {2, 0x80, 0x9F};
        if (c >= 0xE1 && c <= 0xEF) return {2, 0x80, 0xBF};
        if (c == 0xF0) return {3, 0x90, 0xBF};
        if (c == 0xF4) return {3, 0x80, 0x8F};
        if (c >= 0xF1 && c <= 0xF3) return {3, 0x80, 0xBF};
        return {0, 0, 0};  // not a lead byte
    };
    std::vector<uint32_t> cps;
    cps.reserve(s.size());
    const size_t n = s.size();
    for (size_t i = 0; i < n;) {
        const unsigned char c = (unsigned char)s[i++];
        if (c < 0x80) {
            cps.push_back(c);
            continue;
        }
        const Lead ld = lead_of(c);
        if (ld.tail == 0) {
            cps.push_back(0xFFFD);
            continue;
        }
        uint32_t cp = c & (0x3Fu >> ld.tail);
        int got = 0;
        for (unsigned char lo = ld.lo, hi = ld.hi; got < ld.tail && i < n; lo = 0x80, hi = 0xBF) {
            const unsigned char d = (unsigned char)s[i];
            if (d < lo || d > hi) break;
            cp = (cp << 6) | (d & 0x3Fu);
            i++;
            got++;
        }
        cps.push_back(got == ld.tail ? cp : 0xFFFD);
    }
    return cps;
}

// The normalized text: each word (a run of non-whitespace after deletions,
// folding and decompositions) preceded by U+2581.
std::string normalize_words(const std::string& text) {
    std::string s;
    bool gap = true;
    auto put = [&](uint32_t cp) {
        if (is_blank_cp(cp)) {
            gap = true;
            return;
        }
        if (gap) s += "\xE2\x96\x81";
        gap = false;
        put_utf8(s, cp);
    };
    for (uint32_t cp : utf8_code_points(text)) {
        if (is_deleted_cp(cp)) continue;
        if (cp >= 0xFF01 && cp <= 0xFF5D) cp -= 0xFEE0;  // full-width ASCII
        if (const uint32_t* row = compat_row(cp)) {
            for (int k = 1; k < 6 && row[k]; k++) put(row[k]);
        } else {
            put(cp);
        }
    }
    return s;
}

// bytes of the character a lead byte starts; 1 for continuation bytes and
// 0xF8-0xFF
int lead_length(unsigned char c) {
    switch (c >> 4) {
    case 0xC: case 0xD: return 2;
    case 0xE: return 3;
    case 0xF: return c < 0xF8 ? 4 : 1;
    default: return 1;
    }
}

}  // namespace

int32_t UnigramTokenizer::child(int32_t node, unsigned char b) const {
    const auto it = edge_.find((uint64_t)(uint32_t)node << 8 | b);
    return it == edge_.end() ? -1 : it->second;
}

bool UnigramTokenizer::load(const std::string& vocab_txt) {
    edge_.clear();
    node_piece_.assign(1, -1);
    score_.clear();
    longest_ = 1;
    lowest_ = 0.0;
    for_each_line(vocab_txt, [&](const std::string& line) {
        const size_t tab = line.rfind('\t');
        if (tab == std::string::npos) return;
        const int32_t id = (int32_t)score_.size();
        const double sc = std::stod(line.substr(tab + 1));
        score_.push_back(sc);
        const bool bracketed = tab >= 2 && line[0] == '<' && line[tab - 1] == '>';
        if (sc == 0.0 && !bracketed) return;  // unusable: no score and not a special piece
        int32_t node = 0;
        for (size_t k = 0; k < tab; k++) {
            const uint64_t key = (uint64_t)(uint32_t)node << 8 | (unsigned char)line[k];
            auto it = edge_.find(key);
            if (it == edge_.end()) {
                it = edge_.emplace(key, (int32_t)node_piece_.size()).first;
                node_piece_.push_back(-1);
            }
            node = it->second;
        }
        if (node_piece_[(size_t)node] < 0) node_piece_[(size_t)node] = id;  // the first line of a piece
        longest_ = std::max(longest_, tab);
        lowest_ = std::min(lowest_, sc);
    });
    return !score_.empty();
}

void UnigramTokenizer::segment(const std::string& text, std::vector<int32_t>& ids) const {
    const std::string s = normalize_words(text);
    const size_t n = s.size();
    const double kNone = -std::numeric_limits<double>::infinity();
    const double unk_score = lowest_ - 10.0;
    // best[p]: top score of a segmentation of s[0, p); how[p]: its last piece
    // (start, id)
    std::vector<double> best(n + 1, kNone);
    std::vector<std::pair<int32_t, int32_t>> how(n + 1, {-1, kUnk});
    best[0] = 0.0;
    auto offer = [&](size_t from, size_t to, int32_t id, double sc) {
        if (sc > best[to]) {
            best[to] = sc;
            how[to] = {(int32_t)from, id};
        }
    };
    for (size_t i = 0; i < n; i++) {
        if (best[i] == kNone) continue;
        // every vocabulary piece that starts here, shortest first
        int32_t node = 0;
        for (size_t p = i; p < n && (node = child(node, (unsigned char)s[p])) >= 0; p++) {
            const int32_t id = node_piece_[(size_t)node];
            if (id >= 0) offer(i, p + 1, id, best[i] + score_[(size_t)id]);
        }
        // one character as <unk>
        offer(i, i + (size_t)lead_length((unsigned char)s[i]), kUnk, best[i] + unk_score);
    }
    std::vector<int32_t> path;
    for (size_t p = n; p > 0; p = (size_t)how[p].first) path.push_back(how[p].second);
    bool prev_unk = false;
    for (auto it = path.rbegin(); it != path.rend(); ++it) {
        if (*it == kUnk && prev_unk) continue;  // a run of <unk> is one <unk>
        prev_unk = *it == kUnk;
        ids.push_back(*it);
    }
}

std::vector<int32_t> UnigramTokenizer::encode(const std::string& text, int max_len) const {
    if (max_len < 1) return {};
    std::vector<int32_t> ids;
    // Special pieces written literally: from each '<', the text up to the next
    // '>' when it is shorter than the longest piece and is a score-0 piece.
    // The scan goes on from the byte after each '<' (a '<' inside a matched
    // piece is tried too; the text before such a match is then everything
    // after the previous match, as the reference's substr with a wrapped
    // length gives).
    size_t done = 0;
    for (size_t i = text.find('<'); i != std::string::npos; i = text.find('<', i + 1)) {
        const size_t j = text.find('>', i);
        if (j == std::string::npos) break;
        if (j - i >= longest_) continue;
        int32_t node = 0;
        for (size_t k = i; k <= j && node >= 0; k++) node = child(node, (unsigned char)text[k]);
        const int32_t id = node >= 0 ? node_piece_[(size_t)node] : -1;
        if (id < 0 || score_[(size_t)id] != 0.0) continue;
        segment(i >= done ? text.substr(done, i - done) : text.substr(done), ids);
        ids.push_back(id);
        done = j + 1;
    }
    segment(text.substr(done), ids);
    if (ids.size() > (size_t)max_len - 1) ids.resize((size_t)max_len - 1);
    ids.push_back(kEos);
    ids.resize((size_t)max_len, kPad);
    return ids;
}

}  // namespace hip
}  // namespace vla
