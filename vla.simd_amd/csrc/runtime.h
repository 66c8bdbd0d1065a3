// runtime.h - host-side runtime of the C ABI: per-thread error text, the
// library stream and staging arena used by the host-pointer op forms, and the
// guard that turns C++ exceptions into vla_status codes.
#pragma once

#include "common.h"

#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace vla {
namespace hip {

void set_last_error(const std::string& msg);
const char* last_error();

// Runs f; returns 0 (VLA_OK), -1 (VLA_ERR_ARG) for ArgError, -3
// (VLA_ERR_EXCEPTION) for anything else. Exceptions never escape.
template <class F>
int32_t guarded(const char* where, F&& f) {
    try {
        f();
        return 0;
    } catch (const ArgError& e) {
        set_last_error(std::string(where) + ": " + e.what());
        return -1;
    } catch (const ShapeError& e) {
        set_last_error(std::string(where) + ": " + e.what());
        return -2;
    } catch (const std::exception& e) {
        set_last_error(std::string(where) + ": " + e.what());
        return -3;
    } catch (...) {
        set_last_error(std::string(where) + ": unknown exception");
        return -3;
    }
}

// Grow-only device staging for the host-pointer forms. take() hands out
// 256-byte aligned slices of one allocation; reset() at the start of a call.
// Host-to-device bytes the library has issued: all of them, and the part
// that carried weights (int8 rows, weight scales, biases, fp32 weights). The
// host-pointer op forms upload a layer's weights on every call; resident
// layers (vla_linear_i8_*) upload them once.
void count_h2d(size_t bytes, bool weights);
uint64_t h2d_bytes(bool weights_only);

class Staging {
public:
    std::unique_lock<std::mutex> lock() { return std::unique_lock<std::mutex>(mu_); }
    void reset(size_t total_bytes);
    void* take(size_t bytes);
    // weights: count the bytes as weight bytes too
    template <class T>
    T* upload(const T* host, size_t count, hipStream_t st, bool weights = false) {
        if (!host) return nullptr;
        T* d = static_cast<T*>(take(count * sizeof(T)));
        if (count) {
            VLA_HIP_CHECK(hipMemcpyAsync(d, host, count * sizeof(T), hipMemcpyHostToDevice, st));
            count_h2d(count * sizeof(T), weights);
        }
        return d;
    }
    template <class T>
    T* alloc(size_t count) {
        return static_cast<T*>(take(count * sizeof(T)));
    }

private:
    std::mutex mu_;
    char* base_ = nullptr;
    size_t cap_ = 0, used_ = 0;
};

Staging& staging();

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace hip
}  // namespace vla
