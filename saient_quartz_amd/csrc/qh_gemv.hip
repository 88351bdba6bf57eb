// qh_gemv.hip -- batch-1 dequant-GEMV kernels for gfx950 (y = W x, f32 accumulate).
//
// One 256-thread workgroup = 4 wavefronts; each wavefront owns R consecutive
// output rows.  Lane l owns the 64-weight units u = l, l+64, ... of every one of
// its R rows (see qh_formats.h), so a wavefront streams whole rows with
// per-lane 16-byte buffer loads while the 64 activations a unit pairs with are
// read ONCE from LDS and reused for all R rows.  x is staged into LDS in tiles of
// QH_XTILE elements (16-byte chunks, XOR-swizzled against bank conflicts).
// Per-row partial sums are reduced across the wavefront with DPP.
//
// Reference counterpart: the warp-per-row kernels dispatched by cuda_gemv,
// src/cuda_kernels.cu:1046-1077 (and their CPU twins in src/dequant.rs:18-31).
#include "qh_formats.h"
#include "qh_internal.h"

#define QH_XTILE 8192  // activations per LDS tile (32 KB)

QH_DEV int qh_swz(int c) { return c ^ ((c >> 4) & 7); }

template <class F, int R>
__global__ __launch_bounds__(256) void qh_gemv_unit(const uint8_t* __restrict__ W, uint32_t wbytes,
                                                    const float* __restrict__ x, float* __restrict__ y,
                                                    int in_dim, int out_dim, uint32_t row_bytes) {
    extern __shared__ float4 qh_xl[];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const QhBuf wb = qh_buf(W, wbytes);
    const int row0 = (blockIdx.x * 4 + wid) * R;
    const int U = in_dim >> 6;
    constexpr int UT = QH_XTILE / 64;

    uint32_t roff[R];
#pragma unroll
    for (int r = 0; r < R; r++) roff[r] = (uint32_t)min(row0 + r, out_dim - 1) * row_bytes;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

    for (int t0 = 0; t0 < U; t0 += UT) {
        const int tu = min(UT, U - t0);
        uint32_t raw[R][F::NRAW];
        // Issue this lane's first weight loads before staging x so HBM traffic starts at once.
        if (lane < tu) {
#pragma unroll
            for (int r = 0; r < R; r++) F::load(wb, roff[r], t0 + lane, raw[r]);
        }
        if (t0) __syncthreads();
        const float4* xg = reinterpret_cast<const float4*>(x) + t0 * 16;
        for (int c = tid; c < tu * 16; c += 256) qh_xl[qh_swz(c)] = xg[c];
        __syncthreads();
        for (int ul = lane; ul < tu; ul += 64) {
            if (ul != lane) {
#pragma unroll
                for (int r = 0; r < R; r++) F::load(wb, roff[r], t0 + ul, raw[r]);
            }
            const int u = t0 + ul;
            float xv[64];
#pragma unroll
            for (int c = 0; c < 16; c++) {
                const float4 v = qh_xl[qh_swz(F::xoff(u, c) / 4 - t0 * 16)];
                xv[4 * c] = v.x; xv[4 * c + 1] = v.y; xv[4 * c + 2] = v.z; xv[4 * c + 3] = v.w;
            }
            float xs[F::NXS > 0 ? F::NXS : 1];
            F::xsums(xv, xs);
#pragma unroll
            for (int r = 0; r < R; r++) acc[r] += F::dot(raw[r], xv, xs, roff[r], u);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = qh_wave_sum63(acc[r]);
        if (lane == 63 && row0 + r < out_dim) y[row0 + r] = v;
    }
}

// ---------------------------------------------------------------- fallback
// Any (type, in_dim) the unit kernel does not cover (in_dim % 64 != 0, or an
// activation pointer that is not 16-byte aligned): one wavefront per row, lanes
// stride over blocks, each lane decodes its block element by element with the
// bit-exact decoder.  Correct for every supported type, not tuned.
__global__ __launch_bounds__(256) void qh_gemv_generic(uint32_t type, const uint8_t* __restrict__ W,
                                                       const float* __restrict__ x, float* __restrict__ y,
                                                       int in_dim, int out_dim, uint32_t row_bytes, int qk,
                                                       uint32_t blk_bytes) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= out_dim) return;  // wave-uniform
    const uint8_t* rp = W + (size_t)row * row_bytes;
    const int nb = in_dim / qk;
    float acc = 0.f;
    float vals[256];
    for (int b = lane; b < nb; b += 64) {
        qh_decode_block(type, rp + (size_t)b * blk_bytes, vals);
        const float* xb = x + (size_t)b * qk;
        for (int i = 0; i < qk; i++) acc = fmaf(xb[i], vals[i], acc);
    }
    const float v = qh_wave_sum63(acc);
    if (lane == 63) y[row] = v;
}

// ---------------------------------------------------------------- launch

template <class F, int R>
static hipError_t launch_unit(const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                              uint32_t row_bytes, hipStream_t st) {
    const int rows_per_block = 4 * R;
    const int U = in_dim >> 6;
    const int tile_units = U < QH_XTILE / 64 ? U : QH_XTILE / 64;
    const size_t lds = (size_t)tile_units * 256;
    // Rows are processed in chunks whose weight bytes fit one 31-bit buffer range.
    const int64_t max_rows = ((int64_t)1 << 31) / row_bytes;
    int64_t chunk = max_rows - (max_rows % rows_per_block);
    if (chunk < rows_per_block) return hipErrorInvalidValue;
    for (int64_t r0 = 0; r0 < out_dim; r0 += chunk) {
        const int rows = (int)((out_dim - r0) < chunk ? (out_dim - r0) : chunk);
        // Record count rounded up to a dword: a 4-byte load that holds the last
        // byte of a 2-byte-aligned tensor must not be range-checked to zero.
        // (The straddling dword lies in the same 4-aligned, hence mapped, span.)
        const uint32_t wbytes = (uint32_t)(((uint64_t)rows * row_bytes + 3) & ~(uint64_t)3);
        dim3 grid((rows + rows_per_block - 1) / rows_per_block);
        hipLaunchKernelGGL((qh_gemv_unit<F, R>), grid, dim3(256), lds, st, W + (size_t)r0 * row_bytes, wbytes, x,
                           y + r0, in_dim, rows, row_bytes);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t qh_launch_gemv(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                          hipStream_t st) {
    if (!qh_force_valu()) {
        hipError_t e = qh_launch_mmv16(type, W, x, y, in_dim, out_dim, st);
        if (e != hipErrorNotSupported) return e;
        e = qh_launch_mmv(type, W, x, y, in_dim, out_dim, st);
        if (e != hipErrorNotSupported) return e;
    }
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    const bool unit_ok = (in_dim % 64) == 0 && ((uintptr_t)x & 15u) == 0;
    if (unit_ok) {
        switch (type) {
            case QT_Q4_K: return launch_unit<FmtQ4K, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_Q5_K: return launch_unit<FmtQ5K, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_Q6_K: return launch_unit<FmtQ6K, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_Q2_K: return launch_unit<FmtQ2K, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_Q8_0: return launch_unit<FmtQ8_0, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_Q5_0: return launch_unit<FmtQ5_0, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_Q5_1: return launch_unit<FmtQ5_1, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_Q4_0: return launch_unit<FmtQ4_0, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_Q4_1: return launch_unit<FmtQ4_1, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_IQ4_NL: return launch_unit<FmtIQ4NL, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_IQ2_XXS: return launch_unit<FmtIQ2XXS, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_IQ2_XS: return launch_unit<FmtIQ2XS, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_IQ2_S: return launch_unit<FmtIQ2S, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_IQ3_S: return launch_unit<FmtIQ3S, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_F32: return launch_unit<FmtF32, 1>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_F16: return launch_unit<FmtF16, 2>(W, x, y, in_dim, out_dim, row_bytes, st);
            case QT_BF16: return launch_unit<FmtBF16, 2>(W, x, y, in_dim, out_dim, row_bytes, st);
            default: break;
        }
    }
    const int qk = qh_block_elems(type);
    if (qk == 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(qh_gemv_generic, dim3((out_dim + 3) / 4), dim3(256), 0, st, type, W, x, y, in_dim, out_dim,
                       row_bytes, qk, (uint32_t)qh_type_size(type, (size_t)qk));
    return hipGetLastError();
}

// Batched tokens: the matrix-core kernel (one weight pass per 16 tokens) where
// it covers the type and shape, else one batch-1 pass per token.
hipError_t qh_launch_gemm(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                          int n, hipStream_t st) {
    if (n == 1) return qh_launch_gemv(type, W, x, y, in_dim, out_dim, st);
    // f32 weights (routers): one launch for all tokens
    if (type == QT_F32) return qh_launch_gemm_f32(reinterpret_cast<const float*>(W), x, y, in_dim, out_dim, n, st);
    if (!qh_force_valu()) {
        hipError_t e = qh_launch_mmq(type, W, x, y, in_dim, out_dim, n, st);
        if (e != hipErrorNotSupported) return e;
    }
    for (int t = 0; t < n; t++) {
        hipError_t e = qh_launch_gemv(type, W, x + (size_t)t * in_dim, y + (size_t)t * out_dim, in_dim, out_dim, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
