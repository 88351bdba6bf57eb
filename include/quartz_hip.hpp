// quartz_hip.hpp -- C++17 host layer over the C ABI of libquartz_hip (quartz_hip.h).
//
// The counterpart of the reference's Rust host types for the GEMV path
// (src/cuda.rs:57-150, :250-281), for C++ hosts:
//   GpuBuf            RAII device buffer (GpuBuf::upload / alloc_f32, freed on
//                     destruction): src/cuda.rs:59-89
//   GpuScratch        reusable x / y device vectors; gemv copies x in, runs one
//                     GEMV and copies y out: src/cuda.rs:93-127
//   gpu_expert_slice  expert e of a stacked MoE tensor: src/cuda.rs:250-258
//   GpuScratch::gemv_slice                              src/cuda.rs:260-281
//   verify_gemv_hip   a fresh upload + one GEMV, for --verify-gemv:
//                     src/cuda.rs:142-150
//   verify_input / verify_ok   the --verify-gemv x pattern and pass criterion
//                     (src/main.rs:2644-2662)
// Differences from the reference: failures throw quartz_hip::Error (status code
// and hip_last_error() text) where Rust asserts or ignores the void return; the
// IQ codebooks are compiled into the library, so there is no ensure_iq_grids
// step (hip_set_* remain for callers that upload their own tables).
#pragma once
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "quartz_hip.h"

namespace quartz_hip {

class Error : public std::runtime_error {
public:
    Error(const std::string& what, int status)
        : std::runtime_error(what + ": " + hip_status_string(status) + " " + hip_last_error()), status_(status) {}
    int status() const { return status_; }

private:
    int status_;
};

inline void check(const char* what, int status) {
    if (status != QH_OK) throw Error(what, status);
}

// Device buffer owned by the host object (move-only).
class GpuBuf {
public:
    GpuBuf() = default;
    static GpuBuf upload(const void* data, size_t bytes) {
        GpuBuf b = alloc_bytes(bytes);
        if (bytes) check("hip_h2d", hip_h2d(b.ptr_, data, bytes));
        return b;
    }
    static GpuBuf alloc_f32(size_t n) { return alloc_bytes(n * sizeof(float)); }
    static GpuBuf alloc_bytes(size_t bytes) {
        GpuBuf b;
        if (bytes) {
            b.ptr_ = hip_alloc(bytes);
            if (!b.ptr_) throw Error("hip_alloc of " + std::to_string(bytes) + " bytes", QH_ERR_HIP);
        }
        b.bytes_ = bytes;
        return b;
    }
    GpuBuf(GpuBuf&& o) noexcept : ptr_(std::exchange(o.ptr_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
    GpuBuf& operator=(GpuBuf&& o) noexcept {
        if (this != &o) {
            reset();
            ptr_ = std::exchange(o.ptr_, nullptr);
            bytes_ = std::exchange(o.bytes_, 0);
        }
        return *this;
    }
    GpuBuf(const GpuBuf&) = delete;
    GpuBuf& operator=(const GpuBuf&) = delete;
    ~GpuBuf() { reset(); }

    void* ptr() const { return ptr_; }
    size_t bytes() const { return bytes_; }
    template <class T>
    std::vector<T> download(size_t n) const {
        if (n * sizeof(T) > bytes_) throw Error("download past the buffer", QH_ERR_RANGE);
        std::vector<T> out(n);
        if (n) check("hip_d2h", hip_d2h(out.data(), ptr_, n * sizeof(T)));
        return out;
    }

private:
    void reset() {
        if (ptr_) hip_drop(ptr_);
        ptr_ = nullptr;
        bytes_ = 0;
    }
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
};

// A typed view of expert weights inside a stacked tensor.
struct GpuSlice {
    const uint8_t* ptr;
    uint32_t ggml_type;
};

// Expert e of a tensor holding n_experts slices of n_elems_per_expert elements.
inline GpuSlice gpu_expert_slice(const GpuBuf& buf, uint32_t ggml_type, size_t expert, size_t n_elems_per_expert) {
    const size_t bytes = hip_type_size(ggml_type, n_elems_per_expert);
    if (bytes == 0) throw Error("gpu_expert_slice: unknown type", QH_ERR_TYPE);
    if ((expert + 1) * bytes > buf.bytes()) throw Error("gpu_expert_slice: expert past the buffer", QH_ERR_RANGE);
    return GpuSlice{static_cast<const uint8_t*>(buf.ptr()) + expert * bytes, ggml_type};
}

// x and y device vectors reused across GEMV calls (one caller at a time).
class GpuScratch {
public:
    GpuScratch(size_t max_in, size_t max_out)
        : d_x_(GpuBuf::alloc_f32(max_in)), d_y_(GpuBuf::alloc_f32(max_out)), max_in_(max_in), max_out_(max_out) {}

    std::vector<float> gemv(const float* x, size_t nx, const GpuBuf& data, uint32_t ggml_type, int in_dim,
                            int out_dim) const {
        return run(x, nx, static_cast<const uint8_t*>(data.ptr()), ggml_type, in_dim, out_dim);
    }
    std::vector<float> gemv_slice(const float* x, size_t nx, const GpuSlice& s, int in_dim, int out_dim) const {
        return run(x, nx, s.ptr, s.ggml_type, in_dim, out_dim);
    }

private:
    std::vector<float> run(const float* x, size_t nx, const uint8_t* w, uint32_t t, int in_dim, int out_dim) const {
        if (nx > max_in_ || in_dim < 0 || (size_t)in_dim > max_in_ || out_dim < 0 || (size_t)out_dim > max_out_)
            throw Error("GpuScratch: vector past the scratch size", QH_ERR_RANGE);
        if (nx) check("hip_h2d", hip_h2d(d_x_.ptr(), x, nx * sizeof(float)));
        check("hip_gemv", hip_gemv(t, w, static_cast<const float*>(d_x_.ptr()), static_cast<float*>(d_y_.ptr()),
                                   in_dim, out_dim));
        std::vector<float> out(out_dim);
        if (out_dim) check("hip_d2h", hip_d2h(out.data(), d_y_.ptr(), (size_t)out_dim * sizeof(float)));
        check("hip_sync", hip_sync());
        return out;
    }
    GpuBuf d_x_, d_y_;
    size_t max_in_, max_out_;
};

// One GEMV on a freshly uploaded tensor (the --verify-gemv helper).
inline std::vector<float> verify_gemv_hip(const float* x, size_t nx, const void* data, size_t bytes,
                                          uint32_t ggml_type, int in_dim, int out_dim) {
    const GpuBuf buf = GpuBuf::upload(data, bytes);
    const GpuScratch sc((size_t)in_dim, (size_t)out_dim);
    return sc.gemv(x, nx, buf, ggml_type, in_dim, out_dim);
}

// --verify-gemv's input: ((i * 2654435761) >> 8) & 0x3FF, scaled to [-1, 1).
inline std::vector<float> verify_input(size_t in_dim) {
    std::vector<float> x(in_dim);
    for (size_t i = 0; i < in_dim; i++) {
        const uint64_t s = (((uint64_t)i * 2654435761ull) >> 8) & 0x3FFu;
        x[i] = (float)s / 512.0f - 1.0f;
    }
    return x;
}

// --verify-gemv's criterion: max |cpu - gpu| / max(1e-6, max |cpu|) < 1e-3.  A
// NaN difference fails here (the reference's f32::max fold skips it).
struct VerifyResult {
    float maxdiff, rel;
    bool ok;
};
inline VerifyResult verify_ok(const std::vector<float>& cpu, const std::vector<float>& gpu) {
    float maxdiff = 0.f, maxmag = 1e-6f;
    bool nan = false;
    for (size_t i = 0; i < cpu.size() && i < gpu.size(); i++) {
        const float d = cpu[i] > gpu[i] ? cpu[i] - gpu[i] : gpu[i] - cpu[i];
        nan = nan || d != d;
        maxdiff = d > maxdiff ? d : maxdiff;
        const float m = cpu[i] < 0 ? -cpu[i] : cpu[i];
        maxmag = m > maxmag ? m : maxmag;
    }
    const float rel = maxdiff / maxmag;
    return VerifyResult{maxdiff, rel, !nan && rel < 1e-3f && cpu.size() == gpu.size()};
}

}  // namespace quartz_hip
