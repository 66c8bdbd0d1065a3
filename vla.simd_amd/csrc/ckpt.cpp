// ckpt.cpp - see ckpt.h.
#include "ckpt.h"

#include "common.h"

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <limits>
#include <set>
#include <sstream>

namespace vla {
namespace hip {

namespace {

// GGUF metadata value types (the GGUF spec's gguf_type) and the byte size of
// each scalar one; 0 marks string and array.
constexpr uint32_t kString = 8, kArray = 9, kU32 = 4;
size_t scalar_bytes(uint32_t t) {
    static const size_t s[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return t < 13 ? s[t] : 0;
}

// Tensor element types with a fixed size (ggml_type F32, F16, I8, I32, BF16);
// quantized block types have none and are refused.
size_t element_bytes(uint32_t t) {
    switch (t) {
    case 0: return 4;
    case 1: return 2;
    case 24: return 1;
    case 26: return 4;
    case 30: return 2;
    default: return 0;
    }
}

bool ends_with(const std::string& s, const char* suffix) {
    const size_t n = std::strlen(suffix);
    return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
}

std::string without_trailing_slash(std::string p) {
    while (p.size() > 1 && p.back() == '/') p.pop_back();
    return p;
}

std::string parent_dir(const std::string& p) {
    const size_t s = p.rfind('/');
    if (s == std::string::npos) return ".";
    return s == 0 ? "/" : p.substr(0, s);
}

// An embedded file name must stay inside the model directory: relative, no
// empty, "." or ".." component, no NUL.
bool safe_relative(const std::string& rel) {
    if (rel.empty() || rel[0] == '/' || rel.find('\0') != std::string::npos) return false;
    size_t a = 0;
    while (true) {
        const size_t b = rel.find('/', a);
        const std::string part = rel.substr(a, b == std::string::npos ? std::string::npos : b - a);
        if (part.empty() || part == "." || part == "..") return false;
        if (b == std::string::npos) return true;
        a = b + 1;
    }
}

// Little-endian reads over the mapping; running past its end is an error.
class Cursor {
public:
    Cursor(const uint8_t* p, size_t n, const std::string& what) : p_(p), n_(n), what_(what) {}
    void need(uint64_t k) const {
        if (k > n_ - at_) throw ArgError(what_ + ": truncated GGUF");
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p_ + at_, sizeof(T));
        at_ += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        need(n);
        std::string s(reinterpret_cast<const char*>(p_ + at_), (size_t)n);
        at_ += (size_t)n;
        return s;
    }
    void skip(uint64_t k) {
        need(k);
        at_ += (size_t)k;
    }
    size_t at() const { return at_; }

private:
    const uint8_t* p_;
    size_t n_, at_ = 0;
    const std::string& what_;
};

// A scalar metadata value as a double (what vla_simd.format and
// general.alignment need).
double scalar_value(Cursor& c, uint32_t t) {
    switch (t) {
    case 0: return c.get<uint8_t>();
    case 1: return c.get<int8_t>();
    case 2: return c.get<uint16_t>();
    case 3: return c.get<int16_t>();
    case 4: return c.get<uint32_t>();
    case 5: return c.get<int32_t>();
    case 6: return c.get<float>();
    case 7: return c.get<uint8_t>() != 0;
    case 10: return (double)c.get<uint64_t>();
    case 11: return (double)c.get<int64_t>();
    case 12: return c.get<double>();
    default: return 0.0;
    }
}

}  // namespace

// The mount rule of the reference's io::Mount (find_gguf, src/io/files.cpp:91-108):
// a model path names a vla.simd GGUF when it is a regular file whose name ends
// in ".gguf", or a directory in which exactly one entry ends in ".gguf" and no
// entry ends in ".meta" (a converted .meta/.bin directory is read as files even
// with a GGUF beside it). Anything else, or a path that does not exist, is not
// a GGUF: "" is returned.
std::string find_gguf(const std::string& path_in) {
    namespace fs = std::filesystem;
    const fs::path p(without_trailing_slash(path_in));
    std::error_code ec;
    if (p.empty()) return {};
    const fs::file_status st = fs::status(p, ec);  // follows links, as stat() does
    if (ec) return {};
    if (fs::is_regular_file(st)) return ends_with(p.string(), ".gguf") ? p.string() : std::string();
    if (!fs::is_directory(st)) return {};
    std::vector<std::string> ggufs;
    bool has_meta = false;
    for (fs::directory_iterator it(p, ec), end; !ec && it != end; it.increment(ec)) {
        const std::string name = it->path().filename().string();
        if (ends_with(name, ".gguf")) ggufs.push_back(name);
        else if (ends_with(name, ".meta")) has_meta = true;
    }
    if (ec || has_meta || ggufs.size() != 1) return {};
    return p.string() + "/" + ggufs.front();
}

CkptFiles::CkptFiles(const std::string& path) : where_(without_trailing_slash(path)) {
    VLA_REQUIRE(!where_.empty(), "checkpoint: empty model path");
    const std::string file = find_gguf(where_);
    if (file.empty()) {
        disk_ = where_;
        return;
    }
    disk_ = file == where_ ? parent_dir(where_) : where_;
    const int fd = ::open(file.c_str(), O_RDONLY);
    VLA_REQUIRE(fd >= 0, "checkpoint: cannot open " + file);
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        throw ArgError(file + ": not a GGUF file (too short)");
    }
    void* m = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    VLA_REQUIRE(m != MAP_FAILED, "checkpoint: cannot map " + file);
    map_ = m;
    len_ = (size_t)st.st_size;
    try {
        parse(file);
    } catch (...) {
        ::munmap(map_, len_);
        map_ = nullptr;
        throw;
    }
}

CkptFiles::~CkptFiles() {
    if (map_) ::munmap(map_, len_);
}

void CkptFiles::parse(const std::string& file) {
    const uint8_t* base = static_cast<const uint8_t*>(map_);
    Cursor c(base, len_, file);
    VLA_REQUIRE(std::memcmp(base, "GGUF", 4) == 0, file + ": bad magic, not a GGUF file");
    c.skip(4);
    const uint32_t version = c.get<uint32_t>();
    VLA_REQUIRE(version == 2 || version == 3,
                file + ": GGUF version " + std::to_string(version) + " is not supported (2 or 3)");
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    // every key and tensor entry takes at least 12 bytes
    VLA_REQUIRE(n_tensors <= len_ / 12 && n_kv <= len_ / 12, file + ": corrupt header counts");

    // metadata: keep what the vla.simd format uses, walk past the rest
    std::set<std::string> keys;
    std::string arch;
    double format = 0.0;
    uint64_t align = 32;
    std::vector<std::pair<std::string, std::string>> texts;
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key = c.str();
        const uint32_t type = c.get<uint32_t>();
        VLA_REQUIRE(keys.insert(key).second, file + ": duplicate metadata " + key);
        const bool is_file = key.compare(0, 14, "vla_simd.file.") == 0;
        VLA_REQUIRE(!is_file || type == kString, file + ": embedded file " + key.substr(14) + " is not a string");
        if (type == kString) {
            std::string v = c.str();
            if (key == "general.architecture") arch = v;
            if (is_file) texts.emplace_back(key.substr(14), std::move(v));
        } else if (type == kArray) {
            const uint32_t elem = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            if (elem == kString) {
                for (uint64_t j = 0; j < n; j++) c.skip(c.get<uint64_t>());
            } else {
                const size_t eb = scalar_bytes(elem);
                VLA_REQUIRE(eb != 0, file + ": bad array element type at key '" + key + "'");
                VLA_REQUIRE(n <= len_ / eb, file + ": truncated GGUF");
                c.skip(n * eb);
            }
        } else {
            VLA_REQUIRE(scalar_bytes(type) != 0, file + ": bad metadata type at key '" + key + "'");
            const double v = scalar_value(c, type);
            if (key == "vla_simd.format") format = v;
            if (key == "general.alignment") {
                VLA_REQUIRE(type == kU32, file + ": general.alignment must be uint32");
                align = (uint64_t)v;
                VLA_REQUIRE(align != 0 && (align & (align - 1)) == 0, file + ": bad general.alignment");
            }
        }
    }

    struct Info {
        std::string name;
        size_t bytes;
        uint64_t off;
        bool typed;
    };
    std::vector<Info> infos;
    std::set<std::string> names;
    for (uint64_t i = 0; i < n_tensors; i++) {
        Info t;
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        VLA_REQUIRE(nd >= 1 && nd <= 4, file + ": bad tensor info for " + t.name);
        uint64_t numel = 1;
        for (uint32_t d = 0; d < nd; d++) {
            const uint64_t dim = c.get<uint64_t>();
            VLA_REQUIRE(dim >= 1 && dim <= ((uint64_t)1 << 40) && numel <= ((uint64_t)1 << 62) / dim,
                        file + ": bad or overflowing shape for " + t.name);
            numel *= dim;
        }
        const uint32_t type = c.get<uint32_t>();
        t.off = c.get<uint64_t>();
        const size_t eb = element_bytes(type);
        t.typed = eb != 0;
        VLA_REQUIRE(!t.typed || numel <= len_ / eb, file + ": tensor " + t.name + " runs past the end of the file");
        t.bytes = (size_t)numel * eb;
        VLA_REQUIRE(names.insert(t.name).second, file + ": duplicate tensor " + t.name);
        infos.push_back(std::move(t));
    }
    const size_t data = (c.at() + align - 1) / align * align;
    VLA_REQUIRE(data <= len_, file + ": truncated alignment padding");
    for (const Info& t : infos) {
        if (!t.typed) continue;
        VLA_REQUIRE(t.off % align == 0, file + ": misaligned tensor " + t.name);
        VLA_REQUIRE(t.off <= len_ - data && t.bytes <= len_ - data - t.off,
                    file + ": tensor " + t.name + " runs past the end of the file");
    }

    // the vla.simd format on top
    VLA_REQUIRE(arch == "vla-simd", file + ": GGUF architecture '" + arch +
                                        "' is not supported (vla-simd, the converted-checkpoint GGUF, is)");
    VLA_REQUIRE(format == 1.0, file + ": vla.simd GGUF format " + std::to_string(format) + " is not supported (1 is)");
    for (auto& [rel, text] : texts) {
        VLA_REQUIRE(safe_relative(rel), file + ": invalid embedded file " + rel);
        Entry e;
        e.is_text = true;
        e.text = std::move(text);
        files_.emplace(rel, std::move(e));
    }
    for (const Info& t : infos) {
        VLA_REQUIRE(t.typed, file + ": tensor " + t.name + " has an element type vla.simd does not write");
        std::string rel = t.name;
        const size_t colon = rel.rfind(':');
        const bool part = colon != std::string::npos && colon + 1 < rel.size() &&
                          rel.find_first_not_of("0123456789", colon + 1) == std::string::npos;
        if (part) {
            // <rel>:0, <rel>:1, ... in order, for a .bin made of parts only
            const std::string index = rel.substr(colon + 1);
            rel.resize(colon);
            auto it = files_.find(rel);
            const bool next = it == files_.end()
                                  ? index == "0"
                                  : it->second.parted && index == std::to_string(it->second.parts.size());
            VLA_REQUIRE(next, file + ": invalid tensor part " + t.name);
        } else {
            VLA_REQUIRE(files_.find(rel) == files_.end(), file + ": duplicate embedded file " + rel);
        }
        VLA_REQUIRE(safe_relative(rel), file + ": invalid embedded file " + rel);
        Entry& e = files_[rel];
        e.parts.push_back({base + data + t.off, t.bytes});
        e.parted = part;
    }
    VLA_REQUIRE(!files_.empty(), file + ": vla.simd GGUF holds no files");
}

std::vector<std::string> CkptFiles::names() const {
    std::vector<std::string> out;
    for (const auto& kv : files_) out.push_back(kv.first);
    return out;
}

std::string CkptFiles::disk_path(const std::string& rel) const { return disk_ + "/" + rel; }

int64_t CkptFiles::size(const std::string& rel) const {
    auto it = files_.find(rel);
    if (it != files_.end()) {
        if (it->second.is_text) return (int64_t)it->second.text.size();
        int64_t n = 0;
        for (const Piece& p : it->second.parts) n += (int64_t)p.n;
        return n;
    }
    struct stat st;
    if (::stat(disk_path(rel).c_str(), &st) != 0 || !S_ISREG(st.st_mode)) return -1;
    return (int64_t)st.st_size;
}

std::vector<char> CkptFiles::bytes(const std::string& rel) const {
    auto it = files_.find(rel);
    if (it != files_.end()) {
        const Entry& e = it->second;
        if (e.is_text) return std::vector<char>(e.text.begin(), e.text.end());
        std::vector<char> out((size_t)size(rel));
        size_t at = 0;
        for (const Piece& p : e.parts) {
            std::memcpy(out.data() + at, p.p, p.n);
            at += p.n;
        }
        return out;
    }
    const std::string path = disk_path(rel);
    std::ifstream f(path, std::ios::binary);
    VLA_REQUIRE(f, "cannot open " + (map_ ? where_ + "/" + rel : path));
    f.seekg(0, std::ios::end);
    const std::streamoff n = f.tellg();
    f.seekg(0);
    std::vector<char> d((size_t)n);
    if (n > 0) f.read(d.data(), n);
    VLA_REQUIRE(f, "cannot read " + path);
    return d;
}

std::map<std::string, double> CkptFiles::meta(const std::string& rel) const {
    const std::vector<char> raw = bytes(rel);
    std::istringstream in(std::string(raw.begin(), raw.end()));
    std::map<std::string, double> m;
    std::string key;
    double v;
    while (in >> key) {
        VLA_REQUIRE(static_cast<bool>(in >> v), rel + ": key " + key + " has no numeric value");
        m[key] = v;
    }
    return m;
}

std::vector<std::pair<std::string, std::string>> CkptFiles::meta_lines(const std::string& rel) const {
    const std::vector<char> raw = bytes(rel);
    std::istringstream in(std::string(raw.begin(), raw.end()));
    std::vector<std::pair<std::string, std::string>> out;
    std::string line;
    while (std::getline(in, line)) {
        std::istringstream ls(line);
        std::string key;
        if (!(ls >> key)) continue;
        std::string rest;
        std::getline(ls, rest);
        out.emplace_back(key, rest);
    }
    return out;
}

int meta_value_int(const std::string& file, const std::string& key, const std::string& text) {
    std::istringstream ss(text);
    int v = 0;
    ss >> v;
    VLA_REQUIRE(!ss.fail() && (ss >> std::ws).eof(), file + " key " + key + " is not a plain integer: '" + text + "'");
    return v;
}

float meta_value_float(const std::string& file, const std::string& key, const std::string& text) {
    std::istringstream ss(text);
    float v = 0.0f;
    ss >> v;
    VLA_REQUIRE(!ss.fail() && (ss >> std::ws).eof(), file + " key " + key + " is not a number: '" + text + "'");
    return v;
}

int meta_int(const std::map<std::string, double>& m, const char* file, const char* k, int def) {
    auto it = m.find(k);
    if (it == m.end()) return def;
    const double v = it->second;
    VLA_REQUIRE(std::isfinite(v) && v == std::trunc(v) && v >= -2147483648.0 && v <= 2147483647.0,
                std::string(file) + " key " + k + " is not an integer");
    return (int)v;
}

}  // namespace hip
}  // namespace vla
