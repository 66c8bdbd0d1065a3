// loader.h - small helpers the policy loaders share: the reference's shape
// bounds, its integer environment knobs and its `key values...` line parsing,
// and a cursor over a .bin's floats.
#pragma once

#include "common.h"

#include <climits>
#include <cstdlib>
#include <initializer_list>
#include <sstream>
#include <string>

namespace vla {
namespace hip {

// resnet_backbone.cpp:23-27: output size of a strided window, 0 when none fits
inline int conv_out(int in, int k, int stride, int pad) {
    const long long num = (long long)in + 2LL * pad - k;
    if (in <= 0 || stride <= 0 || num < 0 || num / stride >= INT_MAX) return 0;
    return (int)(num / stride + 1);
}

// arena.h shape_fits: every dim positive and the product within int
inline bool shape_fits(std::initializer_list<int> dims) {
    int count = 1;
    for (int d : dims) {
        if (d <= 0 || count > INT_MAX / d) return false;
        count *= d;
    }
    return true;
}

// hal::env::int_env (src/hal/common/env.cpp:23-29): a whole decimal integer,
// else the default
inline int int_env(const char* name, int dflt) {
    const char* e = std::getenv(name);
    if (!e || !*e) return dflt;
    char* end = nullptr;
    const long long v = std::strtoll(e, &end, 10);
    return *end || v < INT_MIN || v > INT_MAX ? dflt : (int)v;
}

// The values after a key, read as the reference's loaders read them: each
// `ss >> v` must succeed and nothing but whitespace may follow the last one.
template <class... T>
void read_values(const std::string& file, const std::string& key, const std::string& text, T&... v) {
    std::istringstream ss(text);
    (ss >> ... >> v);
    VLA_REQUIRE(!ss.fail() && (ss >> std::ws).eof(), file + ": bad value for key " + key + ": '" + text + "'");
}

// Consecutive float arrays of a .bin, each checked against what is left.
struct Floats {
    const float* p;
    size_t n, off = 0;
    const float* take(size_t k, const char* what) {
        if (k > n - off) throw ArgError(std::string(what) + " is shorter than its .meta says");
        const float* r = p + off;
        off += k;
        return r;
    }
    bool done() const { return off == n; }
};

}  // namespace hip
}  // namespace vla
