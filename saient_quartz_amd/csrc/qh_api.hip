// qh_api.hip -- the C ABI declared in include/quartz_hip.h.
//
// Argument checking, dispatch and status codes.  Reference: the `extern "C"`
// block of src/cuda_kernels.cu:1025-1125.  Unlike the reference (void returns,
// no error checks), every HIP call is checked and turned into a status code.
#include <atomic>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/quartz_hip.h"
#include "qh_internal.h"

extern __device__ uint64_t qh_g_iq2xxs[256];
extern __device__ uint64_t qh_g_iq2xs[512];
extern __device__ uint64_t qh_g_iq2s[1024];
extern __device__ uint32_t qh_g_iq3s[512];

static thread_local char qh_errbuf[256];

// Message for hip_last_error() from host-side code (the GGUF reader/writer).
void qh_set_error(const char* msg) { snprintf(qh_errbuf, sizeof qh_errbuf, "%s", msg); }

bool qh_force_valu() {
    static const bool v = [] {
        const char* e = getenv("QUARTZ_HIP_KERNEL");
        return e && strcmp(e, "valu") == 0;
    }();
    return v;
}

static int qh_fail(hipError_t e, const char* what) {
    snprintf(qh_errbuf, sizeof qh_errbuf, "%s: %s", what, hipGetErrorString(e));
    return QH_ERR_HIP;
}
#define QH_CHECK(call, what)                         \
    do {                                             \
        hipError_t qh_e_ = (call);                   \
        if (qh_e_ != hipSuccess) return qh_fail(qh_e_, what); \
    } while (0)

static int qh_check_dims(uint32_t type, int in_dim, int out_dim) {
    const int qk = qh_block_elems(type);
    if (qk == 0) return QH_ERR_TYPE;
    if (in_dim <= 0 || out_dim < 0 || in_dim % qk) return QH_ERR_DIMS;
    return QH_OK;
}

// Unknown type: zero y and say so, as cuda_gemv does (src/cuda_kernels.cu:1070-1074).
static int qh_unknown_type(const char* fn, uint32_t type, float* y, size_t n, hipStream_t st) {
    fprintf(stderr, "%s: unsupported ggml_type %u\n", fn, type);
    // The library's zero-fill kernel rather than hipMemsetAsync, so a call made
    // under HIP graph capture records a kernel node, not a memset node.
    for (size_t off = 0; y && off < n; off += (size_t)1 << 30) {
        const size_t m = n - off < ((size_t)1 << 30) ? n - off : ((size_t)1 << 30);
        hipError_t e = qh_glue_vec(2, y + off, nullptr, 0.f, (int)m, st);
        if (e != hipSuccess) {
            qh_fail(e, fn);
            break;
        }
    }
    return QH_ERR_TYPE;
}

extern "C" {

const char* hip_status_string(int s) {
    switch (s) {
        case QH_OK: return "ok";
        case QH_ERR_TYPE: return "unsupported ggml_type";
        case QH_ERR_DIMS: return "bad dimensions (in_dim must be a positive multiple of the block size)";
        case QH_ERR_NULL: return "null device pointer";
        case QH_ERR_HIP: return "HIP runtime error";
        case QH_ERR_RANGE: return "argument out of range";
        case QH_ERR_FORMAT: return "malformed or unsupported GGUF file";
        case QH_ERR_IO: return "file I/O error";
        default: return "unknown status";
    }
}

const char* hip_last_error(void) { return qh_errbuf; }

size_t hip_type_size(uint32_t type, size_t n) { return qh_type_size(type, n); }

int hip_gemv_async(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                   void* stream) {
    hipStream_t st = (hipStream_t)stream;
    int rc = qh_check_dims(type, in_dim, out_dim);
    if (rc == QH_ERR_TYPE) return qh_unknown_type("hip_gemv", type, out_dim > 0 ? y : nullptr, (size_t)(out_dim > 0 ? out_dim : 0), st);
    if (rc) return rc;
    if (out_dim == 0) return QH_OK;
    if (!W || !x || !y) return QH_ERR_NULL;
    QH_CHECK(qh_launch_gemv(type, W, x, y, in_dim, out_dim, st), "hip_gemv");
    return QH_OK;
}

int hip_gemv(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim) {
    return hip_gemv_async(type, W, x, y, in_dim, out_dim, nullptr);
}

int hip_gemv_multi_async(uint32_t type, int count, const uint8_t* const* W, float* const* y, const int* out_dims,
                         const float* x, int in_dim, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    if (count < 1 || count > 4 || !W || !y || !out_dims) return QH_ERR_RANGE;
    const int qk = qh_block_elems(type);
    if (qk == 0) {
        int rc = QH_ERR_TYPE;
        for (int k = 0; k < count; k++)
            rc = qh_unknown_type("hip_gemv_multi", type, out_dims[k] > 0 ? y[k] : nullptr,
                                 (size_t)(out_dims[k] > 0 ? out_dims[k] : 0), st);
        return rc;
    }
    for (int k = 0; k < count; k++) {
        int rc = qh_check_dims(type, in_dim, out_dims[k]);
        if (rc) return rc;
        if (out_dims[k] > 0 && (!W[k] || !y[k])) return QH_ERR_NULL;
    }
    if (!x) return QH_ERR_NULL;
    if (!qh_force_valu()) {
        hipError_t e = qh_launch_mmv16_multi(type, W, y, out_dims, count, x, in_dim, st, nullptr, 0);
        if (e == hipSuccess) return QH_OK;
        if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemv_multi");
    }
    // no fused kernel for this type/shape: one launch per matrix
    for (int k = 0; k < count; k++) {
        int rc = hip_gemv_async(type, W[k], x, y[k], in_dim, out_dims[k], stream);
        if (rc) return rc;
    }
    return QH_OK;
}

int hip_gemv_multi(uint32_t type, int count, const uint8_t* const* W, float* const* y, const int* out_dims,
                   const float* x, int in_dim) {
    return hip_gemv_multi_async(type, count, W, y, out_dims, x, in_dim, nullptr);
}

int hip_gemv_fused_async(uint32_t type, int count, const uint8_t* const* W, float* const* y, const int* out_dims,
                         const float* x, const float* norm_w, int accumulate, int in_dim, float* scratch,
                         void* stream) {
    hipStream_t st = (hipStream_t)stream;
    if (count < 1 || count > 4 || !W || !y || !out_dims) return QH_ERR_RANGE;
    if (!norm_w && !accumulate) return hip_gemv_multi_async(type, count, W, y, out_dims, x, in_dim, stream);
    const int qk = qh_block_elems(type);
    if (qk == 0) {
        int rc = QH_ERR_TYPE;
        for (int k = 0; k < count; k++)
            rc = qh_unknown_type("hip_gemv_fused", type, out_dims[k] > 0 ? y[k] : nullptr,
                                 (size_t)(out_dims[k] > 0 ? out_dims[k] : 0), st);
        return rc;
    }
    int max_out = 0;
    for (int k = 0; k < count; k++) {
        int rc = qh_check_dims(type, in_dim, out_dims[k]);
        if (rc) return rc;
        if (out_dims[k] > 0 && (!W[k] || !y[k])) return QH_ERR_NULL;
        if (out_dims[k] > max_out) max_out = out_dims[k];
    }
    if (!x) return QH_ERR_NULL;
    if (!qh_force_valu()) {
        hipError_t e = qh_launch_mmv16_multi(type, W, y, out_dims, count, x, in_dim, st, norm_w, accumulate ? 1 : 0);
        if (e == hipSuccess) return QH_OK;
        if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemv_fused");
    }
    // No fused kernel for this type/shape: the reference's sequence of separate
    // kernels, through the caller's scratch (in_dim + max out_dim floats).
    if (!scratch) return QH_ERR_NULL;
    const float* xs = x;
    if (norm_w) {
        QH_CHECK(qh_glue_rms_norm(scratch, x, norm_w, in_dim, st), "hip_gemv_fused");
        xs = scratch;
    }
    for (int k = 0; k < count; k++) {
        if (out_dims[k] == 0) continue;
        float* out = accumulate ? scratch + in_dim : y[k];
        int rc = hip_gemv_async(type, W[k], xs, out, in_dim, out_dims[k], stream);
        if (rc) return rc;
        if (accumulate) QH_CHECK(qh_glue_vec(0, y[k], out, 0.f, out_dims[k], st), "hip_gemv_fused");
    }
    (void)max_out;
    return QH_OK;
}

int hip_gemv_group_async(int count, const uint32_t* types, const uint8_t* const* W, float* const* y,
                         const int* out_dims, const float* x, const float* norm_w, int accumulate, int in_dim,
                         float* scratch, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    if (count < 1 || count > 8 || !types || !W || !y || !out_dims) return QH_ERR_RANGE;
    // the distinct types in first-seen order, each with its matrices
    uint32_t ut[8];
    int nut = 0, idx[8][8], cnt[8] = {0};
    for (int k = 0; k < count; k++) {
        int u = 0;
        while (u < nut && ut[u] != types[k]) u++;
        if (u == nut) ut[nut++] = types[k];
        idx[u][cnt[u]++] = k;
    }
    auto gather = [&](int u, const uint8_t** w, float** yy, int* o) {
        for (int i = 0; i < cnt[u]; i++) {
            w[i] = W[idx[u][i]];
            yy[i] = y[idx[u][i]];
            o[i] = out_dims[idx[u][i]];
        }
    };
    if (nut == 2 && cnt[0] <= 4 && cnt[1] <= 4 && x && !qh_force_valu()) {
        bool ok = true;
        for (int k = 0; k < count; k++)
            ok = ok && qh_check_dims(types[k], in_dim, out_dims[k]) == QH_OK && out_dims[k] > 0 && W[k] && y[k];
        if (ok) {
            const uint8_t *w0[4], *w1[4];
            float *y0[4], *y1[4];
            int o0[4], o1[4];
            gather(0, w0, y0, o0);
            gather(1, w1, y1, o1);
            hipError_t e = qh_launch_mmv16_mix(ut[0], w0, y0, o0, cnt[0], ut[1], w1, y1, o1, cnt[1], x, in_dim,
                                               norm_w, accumulate ? 1 : 0, st);
            if (e == hipSuccess) return QH_OK;
            if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemv_group");
        }
    }
    for (int u = 0; u < nut; u++) {
        const uint8_t* w[8];
        float* yy[8];
        int o[8];
        gather(u, w, yy, o);
        for (int i0 = 0; i0 < cnt[u]; i0 += 4) {
            const int n = cnt[u] - i0 < 4 ? cnt[u] - i0 : 4;
            int rc = hip_gemv_fused_async(ut[u], n, w + i0, yy + i0, o + i0, x, norm_w, accumulate, in_dim, scratch,
                                          stream);
            if (rc) return rc;
        }
    }
    return QH_OK;
}

int hip_gemv_swiglu_async(uint32_t type, const uint8_t* W_gate, const uint8_t* W_up, float* act, int ffn_dim,
                          const float* x, const float* norm_w, int in_dim, float* scratch, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    int rc = qh_check_dims(type, in_dim, ffn_dim);
    if (rc == QH_ERR_TYPE) return qh_unknown_type("hip_gemv_swiglu", type, ffn_dim > 0 ? act : nullptr,
                                                  (size_t)(ffn_dim > 0 ? ffn_dim : 0), st);
    if (rc) return rc;
    if (ffn_dim == 0) return QH_OK;
    if (!W_gate || !W_up || !act || !x) return QH_ERR_NULL;
    if (!qh_force_valu()) {
        const uint8_t* W[2] = {W_gate, W_up};
        float* y[2] = {act, act};
        const int outs[2] = {ffn_dim, ffn_dim};
        hipError_t e = qh_launch_mmv16_multi(type, W, y, outs, 2, x, in_dim, st, norm_w, 0, true);
        if (e == hipSuccess) return QH_OK;
        if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemv_swiglu");
    }
    // separate kernels through scratch: [normed x (in_dim)] [gate (ffn)] [up (ffn)]
    if (!scratch) return QH_ERR_NULL;
    const float* xs = x;
    if (norm_w) {
        QH_CHECK(qh_glue_rms_norm(scratch, x, norm_w, in_dim, st), "hip_gemv_swiglu");
        xs = scratch;
    }
    float* g = scratch + in_dim;
    float* u = g + ffn_dim;
    rc = hip_gemv_async(type, W_gate, xs, g, in_dim, ffn_dim, stream);
    if (rc) return rc;
    rc = hip_gemv_async(type, W_up, xs, u, in_dim, ffn_dim, stream);
    if (rc) return rc;
    QH_CHECK(qh_glue_swiglu(0, act, g, u, ffn_dim, st), "hip_gemv_swiglu");
    return QH_OK;
}

int hip_gemm_async(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim, int n,
                   void* stream) {
    hipStream_t st = (hipStream_t)stream;
    int rc = qh_check_dims(type, in_dim, out_dim);
    if (rc == QH_ERR_TYPE) {
        const size_t cnt = (out_dim > 0 && n > 0) ? (size_t)out_dim * (size_t)n : 0;
        return qh_unknown_type("hip_gemm", type, cnt ? y : nullptr, cnt, st);
    }
    if (rc) return rc;
    if (n < 0) return QH_ERR_DIMS;
    if (out_dim == 0 || n == 0) return QH_OK;
    if (!W || !x || !y) return QH_ERR_NULL;
    QH_CHECK(qh_launch_gemm(type, W, x, y, in_dim, out_dim, n, st), "hip_gemm");
    return QH_OK;
}

int hip_gemm(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim, int n) {
    return hip_gemm_async(type, W, x, y, in_dim, out_dim, n, nullptr);
}

int hip_gemm_grouped_async(uint32_t type, int count, const uint8_t* const* W, const float* const* x, float* const* y,
                           const int* n, const int* out_dims, int in_dim, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    if (count < 0) return QH_ERR_RANGE;
    if (count == 0) return QH_OK;
    if (!W || !x || !y || !n || !out_dims) return QH_ERR_NULL;
    if (qh_block_elems(type) == 0) {
        int rc = QH_ERR_TYPE;
        for (int k = 0; k < count; k++) {
            const size_t cnt = (out_dims[k] > 0 && n[k] > 0) ? (size_t)out_dims[k] * (size_t)n[k] : 0;
            rc = qh_unknown_type("hip_gemm_grouped", type, cnt ? y[k] : nullptr, cnt, st);
        }
        return rc;
    }
    bool batched = false;
    for (int k = 0; k < count; k++) {
        int rc = qh_check_dims(type, in_dim, out_dims[k]);
        if (rc) return rc;
        if (n[k] < 0) return QH_ERR_DIMS;
        if (n[k] > 0 && out_dims[k] > 0 && (!W[k] || !x[k] || !y[k])) return QH_ERR_NULL;
        batched = batched || (n[k] > 1 && out_dims[k] > 0);
    }
    if (batched && !qh_force_valu()) {
        hipError_t e = qh_launch_mmq_grouped(type, count, W, x, y, n, out_dims, in_dim, st);
        if (e == hipSuccess) return QH_OK;
        if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemm_grouped");
    }
    // single tokens only, or no grouped kernel for this type/shape: one call per matrix
    for (int k = 0; k < count; k++) {
        int rc = hip_gemm_async(type, W[k], x[k], y[k], in_dim, out_dims[k], n[k], stream);
        if (rc) return rc;
    }
    return QH_OK;
}

int hip_gemm_grouped(uint32_t type, int count, const uint8_t* const* W, const float* const* x, float* const* y,
                     const int* n, const int* out_dims, int in_dim) {
    return hip_gemm_grouped_async(type, count, W, x, y, n, out_dims, in_dim, nullptr);
}

int hip_gemm_grouped_ex_async(uint32_t type, int count, const uint8_t* const* W, const float* const* x,
                              const float* const* x_up, float* const* y, const int* n, const int* out_dims,
                              int in_dim, int accumulate, float* scratch, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    if (!x_up && !accumulate) return hip_gemm_grouped_async(type, count, W, x, y, n, out_dims, in_dim, stream);
    if (count < 0) return QH_ERR_RANGE;
    if (count == 0) return QH_OK;
    if (!W || !x || !y || !n || !out_dims) return QH_ERR_NULL;
    if (qh_block_elems(type) == 0) {
        int rc = QH_ERR_TYPE;
        for (int k = 0; k < count; k++) {
            const size_t cnt = (out_dims[k] > 0 && n[k] > 0) ? (size_t)out_dims[k] * (size_t)n[k] : 0;
            rc = qh_unknown_type("hip_gemm_grouped_ex", type, cnt ? y[k] : nullptr, cnt, st);
        }
        return rc;
    }
    bool batched = true;
    for (int k = 0; k < count; k++) {
        int rc = qh_check_dims(type, in_dim, out_dims[k]);
        if (rc) return rc;
        if (n[k] < 0) return QH_ERR_DIMS;
        if (n[k] > 0 && out_dims[k] > 0 && (!W[k] || !x[k] || !y[k] || (x_up && !x_up[k]))) return QH_ERR_NULL;
        batched = batched && n[k] > 1;
    }
    if (batched && !qh_force_valu()) {
        hipError_t e = qh_launch_mmq_grouped(type, count, W, x, y, n, out_dims, in_dim, st, x_up, accumulate ? 1 : 0);
        if (e == hipSuccess) return QH_OK;
        if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemm_grouped_ex");
    }
    // separate kernels through scratch: [act (n in_dim)] [product (n out_dim)]
    if (!scratch) return QH_ERR_NULL;
    for (int k = 0; k < count; k++) {
        if (n[k] == 0 || out_dims[k] == 0) continue;
        const size_t nx = (size_t)n[k] * (size_t)in_dim;
        const float* xk = x[k];
        if (x_up) {
            QH_CHECK(qh_glue_swiglu(0, scratch, x[k], x_up[k], (int)nx, st), "hip_gemm_grouped_ex");
            xk = scratch;
        }
        float* yk = accumulate ? scratch + (x_up ? nx : 0) : y[k];
        int rc = hip_gemm_async(type, W[k], xk, yk, in_dim, out_dims[k], n[k], stream);
        if (rc) return rc;
        if (accumulate) QH_CHECK(qh_glue_vec(0, y[k], yk, 0.f, n[k] * out_dims[k], st), "hip_gemm_grouped_ex");
    }
    return QH_OK;
}

int hip_gemm_group_norm_async(int count, const uint32_t* types, const uint8_t* const* W, const float* x,
                              const float* norm_w, float* const* y, int n, const int* out_dims, int in_dim,
                              float* scratch, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    if (count < 1 || count > 8 || n < 0) return QH_ERR_RANGE;
    if (n == 0) return QH_OK;
    if (!types || !W || !x || !norm_w || !y || !out_dims) return QH_ERR_NULL;
    uint32_t ut[8];
    int nut = 0, idx[8][8], cnt[8] = {0};
    for (int k = 0; k < count; k++) {
        int u = 0;
        while (u < nut && ut[u] != types[k]) u++;
        if (u == nut) ut[nut++] = types[k];
        idx[u][cnt[u]++] = k;
    }
    const uint8_t* wu[8][8];
    float* yu[8][8];
    int ou[8][8];
    for (int u = 0; u < nut; u++)
        for (int i = 0; i < cnt[u]; i++) {
            wu[u][i] = W[idx[u][i]];
            yu[u][i] = y[idx[u][i]];
            ou[u][i] = out_dims[idx[u][i]];
        }
    if (n >= 2 && n <= 4 && nut == 2 && cnt[0] <= 4 && cnt[1] <= 4 && !qh_force_valu()) {
        bool ok = true;
        for (int k = 0; k < count; k++)
            ok = ok && qh_check_dims(types[k], in_dim, out_dims[k]) == QH_OK && out_dims[k] > 0 && W[k] && y[k];
        // The per-type call takes 3-4 tokens through the GEMV kernel only up to
        // 16 MB of weights per type (qh_launch_mmq_grouped); the mixed launch
        // follows the same rule, so each type's result is the per-type call's.
        for (int u = 0; ok && n > 2 && u < 2; u++) {
            int64_t wb = 0;
            for (int i = 0; i < cnt[u]; i++) wb += (int64_t)qh_type_size(ut[u], (size_t)in_dim) * ou[u][i];
            ok = wb <= ((int64_t)16 << 20);
        }
        if (ok) {
            hipError_t e = qh_launch_mmv16_mix_tokens(ut[0], wu[0], yu[0], ou[0], ou[0], cnt[0], ut[1], wu[1], yu[1],
                                                      ou[1], ou[1], cnt[1], x, in_dim, n, in_dim, norm_w, 0, st);
            if (e == hipSuccess) return QH_OK;
            if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemm_group_norm");
        }
    }
    // 5-32 tokens of two types (a layer's q/k in Q4_K and v in Q6_K): the rows
    // normalised once (into the x images; for 5-16 tokens into scratch when
    // that does not fit), then both types in one batched launch.
    if (n >= 5 && n <= 32 && nut == 2 && scratch && !qh_force_valu()) {
        bool ok = true;
        for (int k = 0; k < count; k++)
            ok = ok && qh_check_dims(types[k], in_dim, out_dims[k]) == QH_OK && out_dims[k] > 0 && W[k] && y[k];
        if (ok) {
            // the norm fused into the images (one launch), then both types
            hipError_t e = qh_launch_mmq_mixed(ut[0], cnt[0], wu[0], yu[0], ou[0], ut[1], cnt[1], wu[1], yu[1], ou[1],
                                               x, n, in_dim, st, norm_w);
            if (e == hipSuccess) return QH_OK;
            if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemm_group_norm");
            ok = n <= 16;  // 17-32 tokens: the per-type fused images below
        }
        if (ok) {
            QH_CHECK(qh_glue_rms_norm(scratch, x, norm_w, in_dim, st, n), "hip_gemm_group_norm");
            hipError_t e;
            e = qh_launch_mmq_mixed(ut[0], cnt[0], wu[0], yu[0], ou[0], ut[1], cnt[1], wu[1], yu[1], ou[1], scratch, n,
                                    in_dim, st);
            if (e == hipSuccess) return QH_OK;
            if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemm_group_norm");
            // scratch holds the normalised rows: one grouped call per type
            for (int u = 0; u < nut; u++) {
                const float* xs[8];
                int ns[8];
                for (int i = 0; i < cnt[u]; i++) {
                    xs[i] = scratch;
                    ns[i] = n;
                }
                int rc = hip_gemm_grouped_async(ut[u], cnt[u], wu[u], xs, yu[u], ns, ou[u], in_dim, stream);
                if (rc) return rc;
            }
            return QH_OK;
        }
    }
    // 5-16 tokens of one type (a layer's gate and up, the output head), or 3-4
    // tokens over more than 16 MB of weights (which the per-type call also
    // takes to the batched kernel): the norm fused into the images (one
    // launch), then the batched kernel on them
    int64_t wb1 = 0;
    for (int k = 0; k < count; k++)
        wb1 += (int64_t)qh_type_size(types[k], (size_t)in_dim) * (out_dims[k] > 0 ? out_dims[k] : 0);
    // 17-32 tokens (one 32-token pass, two image halves) of any number of
    // types: the norm fused into the images once, then one launch per type
    // on them
    int u0 = 0;
    if (n >= 3 && n <= 32 && (n >= 5 || wb1 > ((int64_t)16 << 20)) && (nut == 1 || n > 16) && !qh_force_valu()) {
        bool ok = true;
        for (int k = 0; k < count; k++)
            ok = ok && qh_check_dims(types[k], in_dim, out_dims[k]) == QH_OK && out_dims[k] > 0 && W[k] && y[k];
        for (; ok && u0 < nut; u0++) {
            hipError_t e =
                qh_launch_mmq_norm(ut[u0], cnt[u0], wu[u0], yu[u0], ou[u0], x, norm_w, n, in_dim, st, u0 > 0);
            if (e == hipErrorNotSupported) break;  // this type and the rest: the per-type calls
            if (e != hipSuccess) return qh_fail(e, "hip_gemm_group_norm");
        }
        if (u0 == nut) return QH_OK;
    }
    for (int u = u0; u < nut; u++) {
        int rc = hip_gemm_grouped_norm_async(ut[u], cnt[u], wu[u], x, norm_w, yu[u], n, ou[u], in_dim, scratch, stream);
        if (rc) return rc;
    }
    return QH_OK;
}

int hip_gemm_grouped_norm_async(uint32_t type, int count, const uint8_t* const* W, const float* x,
                                const float* norm_w, float* const* y, int n, const int* out_dims, int in_dim,
                                float* scratch, void* stream) {
    hipStream_t st = (hipStream_t)stream;
    if (count < 0 || n < 0) return QH_ERR_RANGE;
    if (count == 0 || n == 0) return QH_OK;
    if (!W || !x || !norm_w || !y || !out_dims) return QH_ERR_NULL;
    if (in_dim <= 0) return QH_ERR_DIMS;
    if (qh_block_elems(type) != 0) {
        for (int k = 0; k < count; k++) {
            int rc = qh_check_dims(type, in_dim, out_dims[k]);
            if (rc) return rc;
            if (out_dims[k] > 0 && (!W[k] || !y[k])) return QH_ERR_NULL;
        }
        if (!qh_force_valu() && count <= 16) {
            hipError_t e = hipErrorNotSupported;
            if (n == 1 && count <= 4)
                e = qh_launch_mmv16_multi(type, W, y, out_dims, count, x, in_dim, st, norm_w, 0, false);
            else if (n >= 2) {
                const float* xs[16];
                int ns[16];
                for (int k = 0; k < count; k++) {
                    xs[k] = x;
                    ns[k] = n;
                }
                e = qh_launch_mmq_grouped(type, count, W, xs, y, ns, out_dims, in_dim, st, nullptr, 0, norm_w);
            }
            if (e == hipSuccess) return QH_OK;
            if (e != hipErrorNotSupported) return qh_fail(e, "hip_gemm_grouped_norm");
        }
    }
    // the normalised rows into scratch (n in_dim floats), then one grouped call
    // (matrices sharing x share its digitisation)
    if (!scratch) return QH_ERR_NULL;
    QH_CHECK(qh_glue_rms_norm(scratch, x, norm_w, in_dim, st, n), "hip_gemm_grouped_norm");
    for (int k0 = 0; k0 < count; k0 += 16) {
        const int cnt = count - k0 < 16 ? count - k0 : 16;
        const float* xs[16];
        int ns[16];
        for (int k = 0; k < cnt; k++) {
            xs[k] = scratch;
            ns[k] = n;
        }
        int rc = hip_gemm_grouped_async(type, cnt, W + k0, xs, y + k0, ns, out_dims + k0, in_dim, stream);
        if (rc) return rc;
    }
    return QH_OK;
}

// Device scratch of hip_gemm_grouped_norm_static_async: the normalised token
// rows, at most QH_NORM_SCRATCH_FLOATS floats (4 MB; 64 tokens of 16384).  One
// array per device, held until the process ends.  Host code uses only the
// device address hipGetSymbolAddress returns for it (per device, looked up once
// with that device current), never the array's name.
#define QH_NORM_SCRATCH_FLOATS (1 << 20)
static __device__ __align__(256) float qh_norm_scratch[QH_NORM_SCRATCH_FLOATS];

static float* qh_norm_scratch_ptr() {
    static std::atomic<float*> ptrs[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    float* p = ptrs[dev].load(std::memory_order_acquire);
    if (!p) {
        void* a = nullptr;
        hipError_t e = hipGetSymbolAddress(&a, HIP_SYMBOL(qh_norm_scratch));
        if (e != hipSuccess) {
            qh_fail(e, "hip_gemm_grouped_norm_static: hipGetSymbolAddress");
            return nullptr;
        }
        p = static_cast<float*>(a);
        ptrs[dev].store(p, std::memory_order_release);
    }
    return p;
}

int hip_gemm_grouped_norm_static_async(uint32_t type, int count, const uint8_t* const* W, const float* x,
                                       const float* norm_w, float* const* y, int n, const int* out_dims, int in_dim,
                                       void* stream) {
    if (count < 0 || n < 0) return QH_ERR_RANGE;
    if (count == 0 || n == 0) return QH_OK;
    if (in_dim <= 0) return QH_ERR_DIMS;
    if ((int64_t)n * in_dim > QH_NORM_SCRATCH_FLOATS) {
        snprintf(qh_errbuf, sizeof qh_errbuf,
                 "hip_gemm_grouped_norm_static: n * in_dim = %lld floats exceeds the static scratch (%d floats)",
                 (long long)n * in_dim, QH_NORM_SCRATCH_FLOATS);
        return QH_ERR_RANGE;
    }
    float* s = qh_norm_scratch_ptr();
    if (!s) return QH_ERR_HIP;
    return hip_gemm_grouped_norm_async(type, count, W, x, norm_w, y, n, out_dims, in_dim, s, stream);
}

int hip_gemm_q8_1_mmq_async(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                            int rows, int reference_rows, int multiprocessors, void* stream) {
    if (type != QT_Q4_K && type != QT_Q6_K) return QH_ERR_TYPE;
    if (in_dim <= 0 || in_dim % 256 || out_dim < 0 || rows < 0 || reference_rows < 0 || multiprocessors < 0)
        return QH_ERR_DIMS;
    if (rows == 0 || out_dim == 0) return QH_OK;
    if (!W || !x || !y) return QH_ERR_NULL;
    if ((uintptr_t)x & 15u) return QH_ERR_RANGE;
    QH_CHECK(qh_launch_mmq_q81(type, W, x, y, in_dim, out_dim, rows, reference_rows, multiprocessors,
                               (hipStream_t)stream),
             "hip_gemm_q8_1_mmq");
    return QH_OK;
}
int hip_gemm_q8_1_mmq(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim, int rows,
                      int reference_rows, int multiprocessors) {
    return hip_gemm_q8_1_mmq_async(type, W, x, y, in_dim, out_dim, rows, reference_rows, multiprocessors, nullptr);
}

int hip_gemm_moe_async(uint32_t type, const uint8_t* experts, int n_sel, const int* expert_ids, const int* tok_off,
                       const float* x, float* y, int in_dim, int out_dim, void* stream) {
    if (n_sel < 0) return QH_ERR_RANGE;
    if (n_sel == 0) return QH_OK;
    if (!expert_ids || !tok_off) return QH_ERR_NULL;
    const int qk = qh_block_elems(type);
    const size_t slice = (qk && in_dim > 0 && out_dim >= 0 && in_dim % qk == 0)
                             ? qh_type_size(type, (size_t)in_dim * (size_t)out_dim)
                             : 0;
    const uint8_t* Ws[16];
    const float* Xs[16];
    float* Ys[16];
    int ns[16], outs[16];
    for (int k0 = 0; k0 < n_sel; k0 += 16) {
        const int cnt = n_sel - k0 < 16 ? n_sel - k0 : 16;
        for (int k = 0; k < cnt; k++) {
            const int e = expert_ids[k0 + k], a = tok_off[k0 + k], b = tok_off[k0 + k + 1];
            if (e < 0 || a < 0 || b < a) return QH_ERR_RANGE;
            Ws[k] = experts ? experts + (size_t)e * slice : nullptr;
            Xs[k] = x ? x + (size_t)a * (size_t)(in_dim > 0 ? in_dim : 0) : nullptr;
            Ys[k] = y ? y + (size_t)a * (size_t)(out_dim > 0 ? out_dim : 0) : nullptr;
            ns[k] = b - a;
            outs[k] = out_dim;
        }
        int rc = hip_gemm_grouped_async(type, cnt, Ws, Xs, Ys, ns, outs, in_dim, stream);
        if (rc) return rc;
    }
    return QH_OK;
}

int hip_gemm_moe_dev_async(uint32_t type, int n_sets, const uint8_t* const* experts, float* const* y, int n_exp,
                           const int* tok_off, int max_tokens, const float* x, const float* x_up, int in_dim,
                           int out_dim, int accumulate, void* stream) {
    if (n_sets < 1 || n_sets > 2 || n_exp < 0 || max_tokens < 0) return QH_ERR_RANGE;
    if (n_exp == 0 || max_tokens == 0) return QH_OK;
    if (!experts || !y || !tok_off || !x) return QH_ERR_NULL;
    for (int s = 0; s < n_sets; s++)
        if (!experts[s] || !y[s]) return QH_ERR_NULL;
    if (qh_block_elems(type) == 0) return QH_ERR_TYPE;
    int rc = qh_check_dims(type, in_dim, out_dim);
    if (rc) return rc;
    hipError_t e = qh_launch_mmq_moe_dev(type, n_sets, experts, y, n_exp, tok_off, max_tokens, x, x_up, in_dim,
                                         out_dim, accumulate ? 1 : 0, (hipStream_t)stream);
    if (e == hipErrorNotSupported) {
        qh_set_error("hip_gemm_moe_dev: this type or shape has no device-driven kernel (Q4_K, Q5_K, Q6_K, IQ3_S, "
                     "IQ2_XXS with in_dim % 256 == 0 and 16-byte aligned x)");
        return QH_ERR_TYPE;
    }
    if (e != hipSuccess) return qh_fail(e, "hip_gemm_moe_dev");
    return QH_OK;
}

int hip_gemm_moe(uint32_t type, const uint8_t* experts, int n_sel, const int* expert_ids, const int* tok_off,
                 const float* x, float* y, int in_dim, int out_dim) {
    return hip_gemm_moe_async(type, experts, n_sel, expert_ids, tok_off, x, y, in_dim, out_dim, nullptr);
}

int hip_gemv_moe4(uint32_t type, const uint8_t* w0, const uint8_t* w1, const uint8_t* w2, const uint8_t* w3,
                  const float* xi0, const float* xi1, const float* xi2, const float* xi3, float* o0, float* o1,
                  float* o2, float* o3, int n_act, int in_dim, int out_dim) {
    if (n_act < 0 || n_act > 4) return QH_ERR_RANGE;
    const uint8_t* ws[4] = {w0, w1, w2, w3};
    const float* xs[4] = {xi0, xi1, xi2, xi3};
    float* os[4] = {o0, o1, o2, o3};
    for (int e = 0; e < n_act; e++) {
        int rc = hip_gemv_async(type, ws[e], xs[e], os[e], in_dim, out_dim, nullptr);
        if (rc) return rc;
    }
    return QH_OK;
}

// ---------------------------------------------------------------- decode-step glue
// Twins of the reference's forward-pass helpers (src/cuda_kernels.cu:1129-1290,
// Rust decls src/cuda.rs:20-55); the plain forms run on the default stream.
#define QH_GLUE(call, what)                                  \
    do {                                                     \
        hipError_t qh_e_ = (call);                           \
        if (qh_e_ != hipSuccess) return qh_fail(qh_e_, what); \
        return QH_OK;                                        \
    } while (0)

int hip_vec_add_async(float* dst, const float* src, int n, void* s) {
    if (n > 0 && (!dst || !src)) return QH_ERR_NULL;
    QH_GLUE(qh_glue_vec(0, dst, src, 0.f, n, (hipStream_t)s), "hip_vec_add");
}
int hip_vec_add(float* dst, const float* src, int n) { return hip_vec_add_async(dst, src, n, nullptr); }
int hip_vec_scale_add_async(float* dst, const float* src, float scale, int n, void* s) {
    if (n > 0 && (!dst || !src)) return QH_ERR_NULL;
    QH_GLUE(qh_glue_vec(1, dst, src, scale, n, (hipStream_t)s), "hip_vec_scale_add");
}
int hip_vec_scale_add(float* dst, const float* src, float scale, int n) {
    return hip_vec_scale_add_async(dst, src, scale, n, nullptr);
}
int hip_vec_zero_async(float* dst, int n, void* s) {
    if (n > 0 && !dst) return QH_ERR_NULL;
    QH_GLUE(qh_glue_vec(2, dst, nullptr, 0.f, n, (hipStream_t)s), "hip_vec_zero");
}
int hip_vec_zero(float* dst, int n) { return hip_vec_zero_async(dst, n, nullptr); }

int hip_rms_norm_async(float* out, const float* x, const float* w, int n, void* s) {
    if (n <= 0) return n == 0 ? QH_OK : QH_ERR_DIMS;
    if (!out || !x || !w) return QH_ERR_NULL;
    QH_GLUE(qh_glue_rms_norm(out, x, w, n, (hipStream_t)s), "hip_rms_norm");
}
int hip_rms_norm(float* out, const float* x, const float* w, int n) { return hip_rms_norm_async(out, x, w, n, nullptr); }
int hip_rms_norm_rows_async(float* out, const float* x, const float* w, int rows, int n, void* s) {
    if (n <= 0 || rows < 0) return (n == 0 || rows == 0) && rows >= 0 && n >= 0 ? QH_OK : QH_ERR_DIMS;
    if (!out || !x || !w) return QH_ERR_NULL;
    QH_GLUE(qh_glue_rms_norm(out, x, w, n, (hipStream_t)s, rows), "hip_rms_norm_rows");
}

int hip_rope_yarn_async(float* x, int n_heads, int head_dim, int pos, float theta, float yarn_scale,
                        int yarn_orig_ctx, int neox, void* s) {
    if (n_heads < 0 || head_dim < 0 || head_dim % 2) return QH_ERR_DIMS;
    if (n_heads * head_dim > 0 && !x) return QH_ERR_NULL;
    QH_GLUE(qh_glue_rope(x, n_heads, head_dim, pos, theta, yarn_scale, yarn_orig_ctx, neox, (hipStream_t)s),
            "hip_rope_yarn");
}
int hip_rope_yarn(float* x, int n_heads, int head_dim, int pos, float theta, float yarn_scale, int yarn_orig_ctx,
                  int neox) {
    return hip_rope_yarn_async(x, n_heads, head_dim, pos, theta, yarn_scale, yarn_orig_ctx, neox, nullptr);
}

int hip_kv_append_async(float* k_cache, float* v_cache, const float* k, const float* v, int pos, int kv_dim, void* s) {
    if (pos < 0 || kv_dim < 0) return QH_ERR_DIMS;
    if (kv_dim == 0) return QH_OK;
    if (!k_cache || !v_cache || !k || !v) return QH_ERR_NULL;
    QH_GLUE(qh_glue_kv_append(k_cache, v_cache, k, v, pos, kv_dim, (hipStream_t)s), "hip_kv_append");
}
int hip_kv_append(float* k_cache, float* v_cache, const float* k, const float* v, int pos, int kv_dim) {
    return hip_kv_append_async(k_cache, v_cache, k, v, pos, kv_dim, nullptr);
}

static int qh_attn_dims(int n_heads, int n_kv, int seq, int hd, int kv_dim, int max_seq) {
    if (n_heads < 0 || n_kv <= 0 || seq < 0 || hd <= 0 || seq > max_seq) return QH_ERR_DIMS;
    if ((int64_t)n_kv * hd > kv_dim) return QH_ERR_DIMS;
    return QH_OK;
}

int hip_attn_score_all_async(float* scores, const float* q, const float* k_cache, int n_heads, int n_kv_heads,
                             int seq_len, int head_dim, int kv_dim, int max_seq, float scale, void* s) {
    int rc = qh_attn_dims(n_heads, n_kv_heads, seq_len, head_dim, kv_dim, max_seq);
    if (rc) return rc;
    if (n_heads && seq_len && (!scores || !q || !k_cache)) return QH_ERR_NULL;
    QH_GLUE(qh_glue_attn(0, scores, q, k_cache, nullptr, n_heads, n_kv_heads, seq_len, head_dim, kv_dim, max_seq,
                         scale, (hipStream_t)s), "hip_attn_score_all");
}
int hip_attn_score_all(float* scores, const float* q, const float* k_cache, int n_heads, int n_kv_heads, int seq_len,
                       int head_dim, int kv_dim, int max_seq, float scale) {
    return hip_attn_score_all_async(scores, q, k_cache, n_heads, n_kv_heads, seq_len, head_dim, kv_dim, max_seq,
                                    scale, nullptr);
}
int hip_softmax_sink_all_async(float* scores, int n_heads, int seq_len, int max_seq, const float* sinks, void* s) {
    if (n_heads < 0 || seq_len < 0 || seq_len > max_seq) return QH_ERR_DIMS;
    if (n_heads && seq_len && !scores) return QH_ERR_NULL;
    QH_GLUE(qh_glue_attn(1, scores, nullptr, nullptr, sinks, n_heads, 1, seq_len, 1, 1, max_seq, -1e30f,
                         (hipStream_t)s), "hip_softmax_sink_all");
}
int hip_softmax_sink_all(float* scores, int n_heads, int seq_len, int max_seq, const float* sinks) {
    return hip_softmax_sink_all_async(scores, n_heads, seq_len, max_seq, sinks, nullptr);
}
int hip_attn_values_all_async(float* out, const float* scores, const float* v_cache, int n_heads, int n_kv_heads,
                              int seq_len, int head_dim, int kv_dim, int max_seq, void* s) {
    int rc = qh_attn_dims(n_heads, n_kv_heads, seq_len, head_dim, kv_dim, max_seq);
    if (rc) return rc;
    if (n_heads && (!out || !scores || !v_cache)) return QH_ERR_NULL;
    if (seq_len == 0) return hip_vec_zero_async(out, n_heads * head_dim, s);
    QH_GLUE(qh_glue_attn(2, out, scores, v_cache, nullptr, n_heads, n_kv_heads, seq_len, head_dim, kv_dim, max_seq,
                         0.f, (hipStream_t)s), "hip_attn_values_all");
}
int hip_attn_values_all(float* out, const float* scores, const float* v_cache, int n_heads, int n_kv_heads,
                        int seq_len, int head_dim, int kv_dim, int max_seq) {
    return hip_attn_values_all_async(out, scores, v_cache, n_heads, n_kv_heads, seq_len, head_dim, kv_dim, max_seq,
                                     nullptr);
}

// Single-head forms (cuda_attn_score / cuda_softmax_sink / cuda_attn_values).
int hip_attn_score(float* scores, const float* q, const float* k_cache, int seq_len, int head_dim, int kv_dim,
                   int kv_head_off, float scale) {
    if (kv_head_off < 0 || kv_head_off + head_dim > kv_dim) return QH_ERR_DIMS;
    return hip_attn_score_all_async(scores, q, k_cache ? k_cache + kv_head_off : nullptr, 1, 1, seq_len, head_dim,
                                    kv_dim, seq_len, scale, nullptr);
}
int hip_softmax_sink(float* x, int n, float sink) {
    if (n < 0) return QH_ERR_DIMS;
    if (n && !x) return QH_ERR_NULL;
    QH_GLUE(qh_glue_attn(1, x, nullptr, nullptr, nullptr, 1, 1, n, 1, 1, n, sink, nullptr), "hip_softmax_sink");
}
int hip_attn_values(float* out, const float* scores, const float* v_cache, int seq_len, int head_dim, int kv_dim,
                    int kv_head_off) {
    if (kv_head_off < 0 || kv_head_off + head_dim > kv_dim) return QH_ERR_DIMS;
    return hip_attn_values_all_async(out, scores, v_cache ? v_cache + kv_head_off : nullptr, 1, 1, seq_len, head_dim,
                                     kv_dim, seq_len, nullptr);
}

int hip_attention_decode_async(float* out, const float* q, const float* k_cache, const float* v_cache,
                               const float* sinks, int n_heads, int n_kv_heads, int seq_len, int head_dim, int kv_dim,
                               float scale, void* s) {
    int rc = qh_attn_dims(n_heads, n_kv_heads, seq_len, head_dim, kv_dim, seq_len);
    if (rc) return rc;
    if (n_heads && (!out || !q || !k_cache || !v_cache)) return QH_ERR_NULL;
    if (seq_len == 0) return hip_vec_zero_async(out, n_heads * head_dim, s);
    hipError_t e = qh_glue_attention_decode(out, q, k_cache, v_cache, sinks, n_heads, n_kv_heads, seq_len, head_dim,
                                            kv_dim, scale, (hipStream_t)s);
    if (e == hipErrorNotSupported) return QH_ERR_RANGE;  // seq_len beyond the kernel's LDS score buffer
    if (e != hipSuccess) return qh_fail(e, "hip_attention_decode");
    return QH_OK;
}
int hip_attention_decode(float* out, const float* q, const float* k_cache, const float* v_cache, const float* sinks,
                         int n_heads, int n_kv_heads, int seq_len, int head_dim, int kv_dim, float scale) {
    return hip_attention_decode_async(out, q, k_cache, v_cache, sinks, n_heads, n_kv_heads, seq_len, head_dim, kv_dim,
                                      scale, nullptr);
}

static int qh_attention_step(float* out, const float* q, const float* k, const float* v, float* k_cache,
                             float* v_cache, const float* sinks, int n_seq, size_t cache_stride, int n_heads,
                             int n_kv_heads, int head_dim, int kv_dim, int pos, const int* d_pos, float theta,
                             float yarn_scale, int yarn_orig_ctx, int neox, float scale, void* s) {
    if (pos < 0 || n_seq < 0) return QH_ERR_DIMS;
    int rc = qh_attn_dims(n_heads, n_kv_heads, pos + 1, head_dim, kv_dim, pos + 1);
    if (rc) return rc;
    if (n_kv_heads > n_heads && n_heads > 0) return QH_ERR_DIMS;
    if (n_seq > 1 && cache_stride < (size_t)(pos + 1) * (size_t)kv_dim) return QH_ERR_DIMS;
    if (n_heads == 0 || n_seq == 0) return QH_OK;
    if (!out || !q || !k || !v || !k_cache || !v_cache) return QH_ERR_NULL;
    hipError_t e = qh_glue_attention_step(out, q, k, v, k_cache, v_cache, sinks, n_heads, n_kv_heads, head_dim,
                                          kv_dim, pos, theta, yarn_scale, yarn_orig_ctx, neox, scale, (hipStream_t)s,
                                          n_seq, cache_stride, d_pos);
    if (e == hipErrorNotSupported) return QH_ERR_RANGE;
    if (e != hipSuccess) return qh_fail(e, "hip_attention_step");
    return QH_OK;
}

int hip_attention_step_batched_async(float* out, const float* q, const float* k, const float* v, float* k_cache,
                                     float* v_cache, const float* sinks, int n_seq, size_t cache_stride, int n_heads,
                                     int n_kv_heads, int head_dim, int kv_dim, int pos, float theta, float yarn_scale,
                                     int yarn_orig_ctx, int neox, float scale, void* s) {
    return qh_attention_step(out, q, k, v, k_cache, v_cache, sinks, n_seq, cache_stride, n_heads, n_kv_heads,
                             head_dim, kv_dim, pos, nullptr, theta, yarn_scale, yarn_orig_ctx, neox, scale, s);
}

int hip_attention_step_dev_async(float* out, const float* q, const float* k, const float* v, float* k_cache,
                                 float* v_cache, const float* sinks, int n_seq, size_t cache_stride, int n_heads,
                                 int n_kv_heads, int head_dim, int kv_dim, const int* d_pos, int max_pos, float theta,
                                 float yarn_scale, int yarn_orig_ctx, int neox, float scale, void* s) {
    if (!d_pos && n_heads > 0 && n_seq > 0) return QH_ERR_NULL;
    return qh_attention_step(out, q, k, v, k_cache, v_cache, sinks, n_seq, cache_stride, n_heads, n_kv_heads,
                             head_dim, kv_dim, max_pos, d_pos, theta, yarn_scale, yarn_orig_ctx, neox, scale, s);
}

int hip_attention_step_async(float* out, const float* q, const float* k, const float* v, float* k_cache,
                             float* v_cache, const float* sinks, int n_heads, int n_kv_heads, int head_dim,
                             int kv_dim, int pos, float theta, float yarn_scale, int yarn_orig_ctx, int neox,
                             float scale, void* s) {
    return hip_attention_step_batched_async(out, q, k, v, k_cache, v_cache, sinks, 1, 0, n_heads, n_kv_heads,
                                            head_dim, kv_dim, pos, theta, yarn_scale, yarn_orig_ctx, neox, scale, s);
}

int hip_moe_route_async(const float* logits, const float* router_bias, int n_tok, int n_exp, int k, int renorm,
                        int* ids, float* weights, void* s) {
    if (n_tok < 0 || n_exp < 1 || n_exp > 256 || k < 1 || k > 16 || k > n_exp) return QH_ERR_DIMS;
    if (n_tok > 0 && (!logits || !ids || !weights)) return QH_ERR_NULL;
    QH_GLUE(qh_moe_route(logits, router_bias, n_tok, n_exp, k, renorm, ids, weights, (hipStream_t)s),
            "hip_moe_route");
}
int hip_moe_plan_async(const int* ids, int n_tok, int k, int n_exp, int* tok_off, int* slot_of, int* slot_tok,
                       int* slot_exp, void* s) {
    if (n_tok < 0 || n_exp < 1 || n_exp > 256 || k < 1 || k > 16 || (int64_t)n_tok * k > (1 << 24))
        return QH_ERR_DIMS;
    if (!tok_off || (n_tok > 0 && (!ids || !slot_of || !slot_tok || !slot_exp))) return QH_ERR_NULL;
    QH_GLUE(qh_moe_plan(ids, n_tok, k, n_exp, tok_off, slot_of, slot_tok, slot_exp, (hipStream_t)s),
            "hip_moe_plan");
}
int hip_moe_gather_async(float* xg, const float* x, const int* slot_tok, int n_slots, int dim, void* s) {
    if (n_slots < 0 || dim < 0) return QH_ERR_DIMS;
    if (n_slots > 0 && dim > 0 && (!xg || !x || !slot_tok)) return QH_ERR_NULL;
    QH_GLUE(qh_moe_gather(xg, x, slot_tok, n_slots, dim, (hipStream_t)s), "hip_moe_gather");
}
int hip_moe_swiglu_async(float* act, const float* gate, const float* up, const float* gate_bias, const float* up_bias,
                         const int* slot_exp, int n_slots, int ffn_dim, int oai, void* s) {
    if (n_slots < 0 || ffn_dim < 0) return QH_ERR_DIMS;
    if (n_slots > 0 && ffn_dim > 0 && (!act || !gate || !up || ((gate_bias || up_bias) && !slot_exp)))
        return QH_ERR_NULL;
    QH_GLUE(qh_moe_swiglu(act, gate, up, gate_bias, up_bias, slot_exp, n_slots, ffn_dim, oai, (hipStream_t)s),
            "hip_moe_swiglu");
}
int hip_moe_combine_async(float* out, const float* y_slots, const int* slot_of, const float* weights, const int* ids,
                          const float* down_bias, int n_tok, int k, int dim, int accumulate, void* s) {
    if (n_tok < 0 || k < 1 || dim < 0) return QH_ERR_DIMS;
    if (n_tok > 0 && dim > 0 && (!out || !y_slots || !slot_of || !weights || (down_bias && !ids))) return QH_ERR_NULL;
    QH_GLUE(qh_moe_combine(out, y_slots, slot_of, weights, ids, down_bias, n_tok, k, dim, accumulate, (hipStream_t)s),
            "hip_moe_combine");
}

int hip_swiglu_async(float* out, const float* gate, const float* up, int n, void* s) {
    if (n > 0 && (!out || !gate || !up)) return QH_ERR_NULL;
    QH_GLUE(qh_glue_swiglu(0, out, gate, up, n, (hipStream_t)s), "hip_swiglu");
}
int hip_swiglu(float* out, const float* gate, const float* up, int n) { return hip_swiglu_async(out, gate, up, n, nullptr); }
int hip_swiglu_oai_async(float* out, const float* gate, const float* up, int n, void* s) {
    if (n > 0 && (!out || !gate || !up)) return QH_ERR_NULL;
    QH_GLUE(qh_glue_swiglu(1, out, gate, up, n, (hipStream_t)s), "hip_swiglu_oai");
}
int hip_swiglu_oai(float* out, const float* gate, const float* up, int n) {
    return hip_swiglu_oai_async(out, gate, up, n, nullptr);
}

int hip_embed_lookup_async(float* out, const uint8_t* data, uint32_t ggml_type, int token, int embed_dim, void* s) {
    const int qk = qh_block_elems(ggml_type);
    if (qk == 0) return QH_ERR_TYPE;
    if (token < 0 || embed_dim <= 0 || embed_dim % qk) return QH_ERR_DIMS;
    if (!out || !data) return QH_ERR_NULL;
    QH_GLUE(qh_glue_embed(out, 0, data, ggml_type, &token, 1, embed_dim, (hipStream_t)s), "hip_embed_lookup");
}
int hip_embed_lookup_batched_async(float* out, size_t out_stride, const uint8_t* data, uint32_t ggml_type,
                                   const int* tokens, int n_tok, int embed_dim, void* s) {
    const int qk = qh_block_elems(ggml_type);
    if (qk == 0) return QH_ERR_TYPE;
    if (n_tok < 0 || embed_dim <= 0 || embed_dim % qk || (n_tok > 1 && out_stride < (size_t)embed_dim))
        return QH_ERR_DIMS;
    if (n_tok == 0) return QH_OK;
    if (!out || !data || !tokens) return QH_ERR_NULL;
    for (int i = 0; i < n_tok; i++)
        if (tokens[i] < 0) return QH_ERR_DIMS;
    QH_GLUE(qh_glue_embed(out, out_stride, data, ggml_type, tokens, n_tok, embed_dim, (hipStream_t)s),
            "hip_embed_lookup_batched");
}
int hip_embed_lookup_dev_async(float* out, size_t out_stride, const uint8_t* data, uint32_t ggml_type,
                               const int* d_tokens, int n_tok, int n_vocab, int embed_dim, void* s) {
    const int qk = qh_block_elems(ggml_type);
    if (qk == 0) return QH_ERR_TYPE;
    if (n_tok < 0 || n_vocab < 0 || embed_dim <= 0 || embed_dim % qk ||
        (n_tok > 1 && out_stride < (size_t)embed_dim))
        return QH_ERR_DIMS;
    if (n_tok == 0) return QH_OK;
    if (!out || !data || !d_tokens) return QH_ERR_NULL;
    QH_GLUE(qh_glue_embed(out, out_stride, data, ggml_type, nullptr, n_tok, embed_dim, (hipStream_t)s, d_tokens,
                          n_vocab),
            "hip_embed_lookup_dev");
}
int hip_greedy_next_async(const float* logits, size_t row_stride, int rows, int n, int* d_tokens, int* d_pos,
                          void* s) {
    if (rows < 0 || n < 0 || (rows > 1 && row_stride < (size_t)n)) return QH_ERR_DIMS;
    if (rows == 0 || n == 0) return QH_OK;
    if (!logits || !d_tokens) return QH_ERR_NULL;
    QH_GLUE(qh_glue_greedy(logits, row_stride, rows, n, d_tokens, d_pos, (hipStream_t)s), "hip_greedy_next");
}
int hip_embed_lookup(float* out, const uint8_t* data, uint32_t ggml_type, int token, int embed_dim) {
    return hip_embed_lookup_async(out, data, ggml_type, token, embed_dim, nullptr);
}

int hip_dequant_async(uint32_t type, const uint8_t* W, float* out, size_t n, void* stream) {
    const int qk = qh_block_elems(type);
    if (qk == 0) return QH_ERR_TYPE;
    if (n % (size_t)qk) return QH_ERR_DIMS;
    if (n == 0) return QH_OK;
    if (!W || !out) return QH_ERR_NULL;
    QH_CHECK(qh_launch_dequant(type, W, out, n, (hipStream_t)stream), "hip_dequant");
    return QH_OK;
}

int hip_dequant(uint32_t type, const uint8_t* W, float* out, size_t n) {
    return hip_dequant_async(type, W, out, n, nullptr);
}

void* hip_alloc(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    return p;
}

void hip_drop(void* p) {
    if (p) (void)hipFree(p);
}

int hip_h2d(void* dst, const void* src, size_t bytes) {
    QH_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hip_h2d");
    return QH_OK;
}

int hip_h2d_async(void* dst, const void* src, size_t bytes, void* s) {
    if (bytes && (!dst || !src)) return QH_ERR_NULL;
    QH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)s), "hip_h2d_async");
    return QH_OK;
}
int hip_d2h_async(void* dst, const void* src, size_t bytes, void* s) {
    if (bytes && (!dst || !src)) return QH_ERR_NULL;
    QH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)s), "hip_d2h_async");
    return QH_OK;
}

int hip_d2h(void* dst, const void* src, size_t bytes) {
    QH_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hip_d2h");
    return QH_OK;
}

__global__ void qh_timestamp_k(uint64_t* dst) { *dst = __builtin_amdgcn_s_memrealtime(); }

int hip_timestamp_async(uint64_t* dst, void* stream) {
    if (!dst) return QH_ERR_NULL;
    hipLaunchKernelGGL(qh_timestamp_k, dim3(1), dim3(1), 0, (hipStream_t)stream, dst);
    QH_CHECK(hipGetLastError(), "hip_timestamp_async");
    return QH_OK;
}

// Stream capture into a HIP graph for hosts that drive the library through
// the C ABI only (hipStreamBeginCapture / hipStreamEndCapture /
// hipGraphInstantiate / hipGraphLaunch).
int hip_graph_begin(void* stream) {
    if (!stream) return QH_ERR_NULL;  // the null stream cannot be captured
    QH_CHECK(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal), "hip_graph_begin");
    return QH_OK;
}
int hip_graph_end(void* stream, void** exec) {
    if (!stream || !exec) return QH_ERR_NULL;
    *exec = nullptr;
    hipGraph_t g = nullptr;
    QH_CHECK(hipStreamEndCapture((hipStream_t)stream, &g), "hip_graph_end");
    hipGraphExec_t x = nullptr;
    const hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    QH_CHECK(e, "hip_graph_end");
    *exec = (void*)x;
    return QH_OK;
}
int hip_graph_launch(void* exec, void* stream) {
    if (!exec) return QH_ERR_NULL;
    QH_CHECK(hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream), "hip_graph_launch");
    return QH_OK;
}
void hip_graph_destroy(void* exec) {
    if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
}
int hip_stream_create(void** stream) {
    if (!stream) return QH_ERR_NULL;
    hipStream_t st = nullptr;
    QH_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hip_stream_create");
    *stream = (void*)st;
    return QH_OK;
}
int hip_stream_sync(void* stream) {
    QH_CHECK(hipStreamSynchronize((hipStream_t)stream), "hip_stream_sync");
    return QH_OK;
}
void hip_stream_destroy(void* stream) {
    if (stream) (void)hipStreamDestroy((hipStream_t)stream);
}

int hip_wallclock_khz(void) {
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
        return 0;
    return khz;
}

int hip_sync(void) {
    QH_CHECK(hipDeviceSynchronize(), "hip_sync");
    return QH_OK;
}

int hip_mem_info(size_t* free_b, size_t* total_b) {
    QH_CHECK(hipMemGetInfo(free_b, total_b), "hip_mem_info");
    return QH_OK;
}

int hip_set_iq3s_grid(const uint32_t* host) {
    if (!host) return QH_ERR_NULL;
    QH_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(qh_g_iq3s), host, sizeof(qh_g_iq3s)), "hip_set_iq3s_grid");
    return QH_OK;
}
int hip_set_iq2s_grid(const uint64_t* host) {
    if (!host) return QH_ERR_NULL;
    QH_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(qh_g_iq2s), host, sizeof(qh_g_iq2s)), "hip_set_iq2s_grid");
    return QH_OK;
}
int hip_set_iq2xxs_grid(const uint64_t* host) {
    if (!host) return QH_ERR_NULL;
    QH_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(qh_g_iq2xxs), host, sizeof(qh_g_iq2xxs)), "hip_set_iq2xxs_grid");
    return QH_OK;
}
int hip_set_iq2xs_grid(const uint64_t* host) {
    if (!host) return QH_ERR_NULL;
    QH_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(qh_g_iq2xs), host, sizeof(qh_g_iq2xs)), "hip_set_iq2xs_grid");
    return QH_OK;
}
int hip_set_ksigns(const uint8_t* host) {
    if (!host) return QH_ERR_NULL;
    for (uint32_t i = 0; i < 128; i++)
        if (host[i] != (uint8_t)(i | ((uint32_t)__builtin_parity(i) << 7))) return QH_ERR_RANGE;
    return QH_OK;
}

}  // extern "C"
