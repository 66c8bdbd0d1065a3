// runtime.cpp - error plumbing, library stream, staging arena, device check.
#include "runtime.h"

#include <atomic>

#include <cstdio>

namespace vla {
namespace hip {

namespace {
thread_local std::string t_last_error;
}

void set_last_error(const std::string& msg) { t_last_error = msg; }
const char* last_error() { return t_last_error.c_str(); }

[[noreturn]] void throw_hip(hipError_t e, const char* what, const char* file, int line) {
    char buf[512];
    std::snprintf(buf, sizeof buf, "%s failed: %s (%d) at %s:%d", what, hipGetErrorString(e),
                  (int)e, file, line);
    throw HipError(buf);
}

hipStream_t library_stream() {
    // One stream per process for the host-pointer forms, default priority.
    static hipStream_t s = [] {
        hipStream_t st = nullptr;
        VLA_HIP_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        return st;
    }();
    return s;
}

bool device_is_gfx950() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return false;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

void Staging::reset(size_t total_bytes) {
    used_ = 0;
    if (total_bytes <= cap_) return;
    if (base_) {
        VLA_HIP_CHECK(hipStreamSynchronize(library_stream()));
        VLA_HIP_CHECK(hipFree(base_));
        base_ = nullptr;
        cap_ = 0;
    }
    size_t cap = 1 << 20;
    while (cap < total_bytes) cap <<= 1;
    VLA_HIP_CHECK(hipMalloc(&base_, cap));
    cap_ = cap;
}

void* Staging::take(size_t bytes) {
    const size_t b = align256(bytes ? bytes : 1);
    if (used_ + b > cap_) throw HipError("staging arena overflow (size computed too small)");
    void* p = base_ + used_;
    used_ += b;
    return p;
}

namespace {
std::atomic<uint64_t> g_h2d_all{0}, g_h2d_weights{0};
}

void count_h2d(size_t bytes, bool weights) {
    g_h2d_all.fetch_add(bytes, std::memory_order_relaxed);
    if (weights) g_h2d_weights.fetch_add(bytes, std::memory_order_relaxed);
}

uint64_t h2d_bytes(bool weights_only) {
    return (weights_only ? g_h2d_weights : g_h2d_all).load(std::memory_order_relaxed);
}

Staging& staging() {
    static Staging s;
    return s;
}

}  // namespace hip
}  // namespace vla
