// ckpt.h - the files of a model path: a converted directory of the
// reference's .meta / .bin files, or a vla.simd GGUF that carries them.
//
// Follows the reference's model-file access (src/io/files.h:8-17, the mount
// rule of files.cpp find_gguf, the vla.simd GGUF of tools/_gguf.py:6-28 read
// by src/io/gguf.cpp and src/io/gguf_vla_simd.cpp:29-77):
//   * a path is a GGUF when it is a regular file named *.gguf, or a directory
//     holding exactly one *.gguf and no *.meta; anything else is a directory;
//   * a vla.simd GGUF (general.architecture "vla-simd", vla_simd.format 1)
//     stores every text file as a string `vla_simd.file.<path>` and every .bin
//     as a tensor named <path>, or as parts <path>:0, <path>:1, ... (in file
//     order) when it mixes element types; the files come back byte for byte;
//   * a file the GGUF does not carry is read from disk beside it.
// The GGUF is memory-mapped; a .bin is copied out of the mapping once, when
// a loader asks for it. The file is untrusted input: every count, offset and
// size is checked against the mapping before use, and any defect (truncation,
// a bad version, duplicate keys or tensors, misaligned or overflowing
// tensors, an unsafe embedded path, misordered parts) is an ArgError.
// Other GGUF architectures (the vla.cpp smolvla / octo / turbovla layouts the
// reference re-lays out in src/io/gguf_{smolvla,octo,turbovla}.cpp) are
// rejected by name.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <utility>
#include <vector>

namespace vla {
namespace hip {

class CkptFiles {
public:
    explicit CkptFiles(const std::string& path);
    ~CkptFiles();
    CkptFiles(const CkptFiles&) = delete;
    CkptFiles& operator=(const CkptFiles&) = delete;

    bool gguf() const { return map_ != nullptr; }
    // The files the GGUF carries, sorted (empty for a directory).
    std::vector<std::string> names() const;
    // Size of <rel> (in the GGUF, else on disk); -1 when there is none.
    int64_t size(const std::string& rel) const;
    // The bytes of <rel>; ArgError when there is none.
    std::vector<char> bytes(const std::string& rel) const;
    // "key value" pairs of a .meta file (whitespace separated, numeric values).
    std::map<std::string, double> meta(const std::string& rel) const;
    // The lines of a .meta file as (key, rest of the line), in file order, for
    // loaders that read each value as the reference's getline + `ss >> value` +
    // end-of-line check does (blank lines skipped).
    std::vector<std::pair<std::string, std::string>> meta_lines(const std::string& rel) const;

private:
    struct Piece {
        const uint8_t* p;
        size_t n;
    };
    struct Entry {
        std::string text;          // a text file
        std::vector<Piece> parts;  // a .bin: its tensor(s), in order
        bool is_text = false;
        bool parted = false;       // stored as <path>:0, <path>:1, ...
    };
    void parse(const std::string& file);
    std::string disk_path(const std::string& rel) const;

    std::string where_;  // the path as given, for messages
    std::string disk_;   // directory that files not in a GGUF come from
    void* map_ = nullptr;
    size_t len_ = 0;
    std::map<std::string, Entry> files_;
};

// Whether `path` mounts as a GGUF, and which file ("" otherwise).
std::string find_gguf(const std::string& path);

// One value of a meta_lines() line read the reference's way: `ss >> int` (or
// float) must succeed and leave nothing but whitespace ("512.0" and "1e3" are
// not integers); otherwise ArgError naming the file and key.
int meta_value_int(const std::string& file, const std::string& key, const std::string& text);
float meta_value_float(const std::string& file, const std::string& key, const std::string& text);

// The integer value of key k of a parsed .meta file (def when absent), with
// the reference's metadata_int bounds (src/models/arena.h:21-25): a finite
// integer in int range, else an error naming `file`.
int meta_int(const std::map<std::string, double>& m, const char* file, const char* k, int def);

}  // namespace hip
}  // namespace vla
