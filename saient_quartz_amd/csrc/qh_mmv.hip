// qh_mmv.hip -- matrix-core dequant-GEMV for gfx950 (y = W x, W GGUF-quantized).
//
// The dot products run on the int8 matrix cores (v_mfma_i32_32x32x32_i8):
//   * B operand = the quantized weights themselves as int8 (a Q4_K nibble plane is
//     `w & 0x0F0F0F0F`, a Q8_0 block is already int8, IQ codebook values are int8),
//     so no per-weight float conversion is needed;
//   * A operand = the activations as three balanced int8 digits per element:
//     a wavefront picks one exponent s for its slice of x (max|x| * 2^s < 2^22),
//     rounds x * 2^s to a 23-bit integer with one FMA against a magic constant and
//     splits it into digits d0 + 256 d1 + 65536 d2 (each in [-128, 127]).  The
//     int32 MFMA sums are exact, so the only rounding relative to an f32 dot is
//     x's own rounding to 23 bits (<= 2^-23 of the slice's largest |x|).
// A 32-weight "unit" (Q4_K sub-block, Q8_0 block, Q6_K (half, k) group, ...) is
// one MFMA: 32 rows x 32 k.  Units whose two 16-weight halves carry different
// scales (Q6_K, Q2_K, IQ2_XS, IQ2_S) put the digits of positions 0-15 in A rows
// 0-2 and of positions 16-31 in A rows 4-6, so the two halves land in lanes 0-31
// and 32-63 of the result and each lane applies its own half's scale.
//
// Grid: one workgroup per 32 output rows; its 8 wavefronts split K (groups of 256
// weights) and reduce through LDS at the end.  Each wavefront issues the loads of
// its next group before decoding the current one.
//
// Reference counterpart: the warp-per-row kernels behind cuda_gemv,
// src/cuda_kernels.cu:1046-1077 (scalar FMA per weight, one row per warp).
#include "qh_formats.h"
#include "qh_internal.h"

typedef int32_t qh_i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t qh_i32x16 __attribute__((ext_vector_type(16)));

#define QH_MMV_WAVES 8
#define QH_UNIT_LDS 128  // per 32-element x unit: 3 digit planes, 2 half sums, 16 zero bytes

// ---------------------------------------------------------------- activations

// Quantize this wavefront's slice of x (ngroups x 256 elements starting at x0)
// into LDS: per 32-element unit u, digit planes at lds[u*128 + 32p + pos], the f32
// sums of positions 0-15 / 16-31 at lds[u*128 + 96 / 100] and 16 zero bytes at
// lds[u*128 + 112] (the A operand of lanes that carry no digits).  Returns 2^-s.
QH_DEV float qh_prep_x(const float* __restrict__ x, int x0, int ngroups, unsigned char* lds, int lane) {
    float m = 0.f;
    for (int t = 0; t < ngroups; t++) {
        const float4 v = *reinterpret_cast<const float4*>(x + x0 + 256 * t + 4 * lane);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    // wave max (DPP), result broadcast from lane 63
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x140, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x142, 0xA, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x143, 0xC, 0xF, false)));
    m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 63));
    int e = 0;
    (void)frexpf(m, &e);                   // m < 2^e
    const int s = m > 0.f ? 22 - e : 0;    // |x| 2^s < 2^22
    const float sc = ldexpf(1.0f, s);
    // round(x 2^s) + 2^22 + 0x808080 as the low 24 bits of (x 2^s + 1.5 * 2^23); the
    // xor with 0x808080 then leaves the three balanced digits in bytes 0..2.
    const float magic = 12582912.0f;
    const uint32_t bias = 0x4B400000u - 0x808080u;
    for (int t = 0; t < ngroups; t++) {
        const float4 v = *reinterpret_cast<const float4*>(x + x0 + 256 * t + 4 * lane);
        const uint32_t a0 = (__float_as_uint(fmaf(v.x, sc, magic)) - bias) ^ 0x808080u;
        const uint32_t a1 = (__float_as_uint(fmaf(v.y, sc, magic)) - bias) ^ 0x808080u;
        const uint32_t a2 = (__float_as_uint(fmaf(v.z, sc, magic)) - bias) ^ 0x808080u;
        const uint32_t a3 = (__float_as_uint(fmaf(v.w, sc, magic)) - bias) ^ 0x808080u;
        const uint32_t t01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
        const uint32_t t23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
        const uint32_t u01 = __builtin_amdgcn_perm(a1, a0, 0x06020602u);
        const uint32_t u23 = __builtin_amdgcn_perm(a3, a2, 0x06020602u);
        const uint32_t p0 = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
        const uint32_t p1 = __builtin_amdgcn_perm(t23, t01, 0x07060302u);
        const uint32_t p2 = __builtin_amdgcn_perm(u23, u01, 0x05040100u);
        // lane covers positions 4*(lane%8) .. +3 of unit u = 8t + lane/8
        const int u = 8 * t + (lane >> 3), pos = 4 * (lane & 7);
        unsigned char* ub = lds + u * QH_UNIT_LDS;
        *reinterpret_cast<uint32_t*>(ub + pos) = p0;
        *reinterpret_cast<uint32_t*>(ub + 32 + pos) = p1;
        *reinterpret_cast<uint32_t*>(ub + 64 + pos) = p2;
        float h = (v.x + v.y) + (v.z + v.w);
        h += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(h), 0xB1, 0xF, 0xF, false));
        h += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(h), 0x4E, 0xF, 0xF, false));
        if ((lane & 3) == 0) *reinterpret_cast<float*>(ub + 96 + 4 * ((lane >> 2) & 1)) = h;
        if ((lane & 7) == 0) *reinterpret_cast<qh_i32x4*>(ub + 112) = qh_i32x4{0, 0, 0, 0};
    }
    return ldexpf(1.0f, -s);
}

// LDS offset (within a unit) of this lane's A operand: digit p of positions
// [16h, 16h+16) for the lanes that carry A rows, the zero slot for all others.
//   one-scale units: A rows 0-2 (lanes 0-2) <- positions 0-15, lanes 32-34 <- 16-31
//   two-scale units: A rows 0-2 (lanes 0-2) <- 0-15, rows 4-6 (lanes 36-38) <- 16-31
template <bool TWO>
QH_DEV uint32_t qh_aoff(int lane) {
    const int m = lane & 31, g = lane >> 5;
    int p;
    bool on;
    if (TWO) {
        p = g ? m - 4 : m;
        on = g ? (m >= 4 && m < 7) : (m < 3);
    } else {
        p = m;
        on = m < 3;
    }
    return on ? (uint32_t)(32 * p + 16 * g) : 112u;
}

// One unit on the matrix cores: D = A B with C = 0 (an inline constant, so
// nothing is zeroed); returns the unit's digit dot d0 + 256 d1 + 65536 d2 (before
// the 2^-s factor).  |d1 * 256 + d0| < 2^31 always; the f32 conversions round to
// 24 bits at most once each.
QH_DEV float qh_unit_dot(qh_i32x4 a, qh_i32x4 b) {
    const qh_i32x16 z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const qh_i32x16 D = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
    return fmaf((float)D[2], 65536.0f, (float)(D[1] * 256 + D[0]));
}

// ---------------------------------------------------------------- formats
// Each policy decodes one 256-weight group of its row (lane: row n = lane%32,
// half g = lane/32) from NRAW raw dwords:
//   load(buf, roff, grp, g, raw)     issue the loads
//   unit(raw, j, g, roff, grp, B, scale, mm)   B fragment of unit j (16 int8),
//        the scale multiplying the unit's digit dot, and mm multiplying the
//        half's x sum (offsets / mins).
//   TWO: units whose halves have different scales.

// Q4_K (src/dequant.rs:1482-1519): unit j = sub-block j (32 weights, one 6-bit scale).
struct MQ4K {
    static constexpr uint32_t GB = 144;  // group bytes (one superblock)
    static constexpr int NRAW = 20;
    static constexpr bool TWO = false;
    QH_DEV static void load(QhBuf b, uint32_t roff, int grp, int g, uint32_t* r) {
        const uint32_t base = roff + GB * (uint32_t)grp;
        qh_ldn<4>(b, base, r);
#pragma unroll
        for (int p = 0; p < 4; p++) qh_ldn<4>(b, base + 16 + 32 * p + 16 * g, r + 4 + 4 * p);
    }
    QH_DEV static void unit(const uint32_t* r, int j, int g, uint32_t, int, qh_i32x4& B, float& scale,
                            float& mm) {
        const int p = j >> 1;
        const uint32_t sh = (j & 1) ? 4u : 0u;
#pragma unroll
        for (int i = 0; i < 4; i++) B[i] = (int)((r[4 + 4 * p + i] >> sh) & 0x0F0F0F0Fu);
        uint32_t sc1, m1, sc2, m2;
        qh_scale_pair(r[1], r[2], r[3], p, sc1, m1, sc2, m2);
        const uint32_t sc = (j & 1) ? sc2 : sc1, mn = (j & 1) ? m2 : m1;
        scale = qh_f16_lo(r[0]) * (float)sc;
        mm = -(qh_f16_hi(r[0]) * (float)mn);
    }
};

// Q6_K (src/dequant.rs:1583-1631): unit j = (h = j/4, k = j%4), weights
// y[128h + 32k + l]; half g = l/16 has scale sc[8h + 2k + g]; B = the unsigned
// 6-bit q, the -32 offset goes through the half sums.
struct MQ6K {
    static constexpr uint32_t GB = 210;
    static constexpr int NRAW = 36;
    static constexpr bool TWO = true;
    QH_DEV static void load(QhBuf b, uint32_t roff, int grp, int g, uint32_t* r) {
        const uint32_t base = roff + GB * (uint32_t)grp;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            qh_ldwin<4>(b, base + 64 * h + 16 * g, r + 10 * h);           // ql[64h + 16g ..]
            qh_ldwin<4>(b, base + 64 * h + 32 + 16 * g, r + 10 * h + 5);  // ql[64h + 32 + 16g ..]
            qh_ldwin<4>(b, base + 128 + 32 * h + 16 * g, r + 20 + 5 * h); // qh[32h + 16g ..]
        }
        qh_ldwin<4>(b, base + 192, r + 30);  // sc[0..16)
        r[35] = qh_ld32(b, (base + 208) & ~3u);
    }
    QH_DEV static void unit(const uint32_t* r, int j, int g, uint32_t roff, int grp, qh_i32x4& B, float& scale,
                            float& mm) {
        const uint32_t base = roff + GB * (uint32_t)grp;
        const uint32_t sh = base & 3u;
        const int h = j >> 2, k = j & 3;
        const uint32_t* qlw = r + 10 * h + 5 * (k & 1);
        const uint32_t* qhw = r + 20 + 5 * h;
        const uint32_t nsh = (k & 2) ? 4u : 0u;
        const uint32_t hsh = 2u * (uint32_t)k;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t ql = __builtin_amdgcn_alignbyte(qlw[i + 1], qlw[i], sh);
            const uint32_t qh = __builtin_amdgcn_alignbyte(qhw[i + 1], qhw[i], sh);
            B[i] = (int)(((ql >> nsh) & 0x0F0F0F0Fu) | (((qh >> hsh) & 0x03030303u) << 4));
        }
        const int si = 8 * h + 2 * k + g;  // scale byte index
        const uint32_t sw = __builtin_amdgcn_alignbyte(r[30 + (si >> 2) + 1], r[30 + (si >> 2)], sh);
        const float d = (base & 2u) ? qh_f16_hi(r[35]) : qh_f16_lo(r[35]);
        scale = d * (float)(int8_t)(sw >> (8 * (si & 3)));
        mm = -32.0f * scale;
    }
};

// Q8_0 (src/dequant.rs:1450-1463): unit j = block j of the group (8 x 34 B).
struct MQ8_0 {
    static constexpr uint32_t GB = 272;
    static constexpr int NRAW = 48;
    static constexpr bool TWO = false;
    QH_DEV static void load(QhBuf b, uint32_t roff, int grp, int g, uint32_t* r) {
        const uint32_t base = roff + GB * (uint32_t)grp;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            qh_ldwin<4>(b, base + 34 * j + 2 + 16 * g, r + 6 * j);
            r[6 * j + 5] = qh_ld32(b, (base + 34 * j) & ~3u);
        }
    }
    QH_DEV static void unit(const uint32_t* r, int j, int, uint32_t roff, int grp, qh_i32x4& B, float& scale,
                            float& mm) {
        const uint32_t blk = roff + GB * (uint32_t)grp + 34 * j;
        const uint32_t sh = (blk + 2) & 3u;
#pragma unroll
        for (int i = 0; i < 4; i++) B[i] = (int)__builtin_amdgcn_alignbyte(r[6 * j + i + 1], r[6 * j + i], sh);
        scale = (blk & 2u) ? qh_f16_hi(r[6 * j + 5]) : qh_f16_lo(r[6 * j + 5]);
        mm = 0.f;
    }
};

// ---------------------------------------------------------------- kernel

// The 8 units of local group t for the T column tiles of this wavefront.
template <class F, int T>
QH_DEV void qh_mmv_group(const uint32_t (&raw)[T][F::NRAW], const unsigned char* lds, uint32_t aoff, int g,
                         const uint32_t (&roff)[T], int grp, int t, float (&acc)[T], float (&accm)[T]) {
    const unsigned char* ub = lds + 8 * t * QH_UNIT_LDS;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const qh_i32x4 a = *reinterpret_cast<const qh_i32x4*>(ub + j * QH_UNIT_LDS + aoff);
        const float xh = *reinterpret_cast<const float*>(ub + j * QH_UNIT_LDS + 96 + 4 * g);
#pragma unroll
        for (int c = 0; c < T; c++) {
            qh_i32x4 B;
            float scale, mm;
            F::unit(raw[c], j, g, roff[c], grp, B, scale, mm);
            acc[c] = fmaf(scale, qh_unit_dot(a, B), acc[c]);
            accm[c] = fmaf(mm, xh, accm[c]);
        }
        // Keep the scheduler from hoisting later units' MFMAs: each 32x32 result is
        // 16 registers and only 3 of them are read.
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Workgroup = 8 wavefronts splitting K; rows = T column tiles of `rt` rows.
template <class F, int T>
__global__ __launch_bounds__(64 * QH_MMV_WAVES) void qh_mmv(const uint8_t* __restrict__ W, uint32_t wbytes,
                                                          const float* __restrict__ x, float* __restrict__ y,
                                                          int out_dim, uint32_t row_bytes, int ngroups, int gpw,
                                                          int rt) {
    extern __shared__ __align__(16) unsigned char qh_lds[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n = lane & 31, g = lane >> 5;
    const QhBuf wb = qh_buf(W, wbytes);
    int row[T];
    bool live[T];
    uint32_t roff[T];
#pragma unroll
    for (int c = 0; c < T; c++) {
        row[c] = (blockIdx.x * T + c) * rt + n;
        live[c] = n < rt && row[c] < out_dim;
        // Rows outside the matrix read past the buffer's record count: zeros, no traffic.
        roff[c] = live[c] ? (uint32_t)row[c] * row_bytes : 0x80000000u;
    }
    const int g0 = w * gpw;
    const int gn = max(0, min(gpw, ngroups - g0));
    unsigned char* lds = qh_lds + w * gpw * 8 * QH_UNIT_LDS;
    const uint32_t aoff = qh_aoff<F::TWO>(lane);

    float acc[T], accm[T];
#pragma unroll
    for (int c = 0; c < T; c++) {
        acc[c] = 0.f;
        accm[c] = 0.f;
    }
    float xs = 0.f;
    if (gn > 0) {
        // Two statically named buffers.  The first two groups are requested before
        // the activation quantization (which waits on x), later ones one group ahead.
        uint32_t ra[T][F::NRAW], rb[T][F::NRAW];
#pragma unroll
        for (int c = 0; c < T; c++) F::load(wb, roff[c], g0, g, ra[c]);
        if (gn > 1) {
#pragma unroll
            for (int c = 0; c < T; c++) F::load(wb, roff[c], g0 + 1, g, rb[c]);
        }
        xs = qh_prep_x(x, 256 * g0, gn, lds, lane);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int t = 0; t < gn; t += 2) {
            qh_mmv_group<F, T>(ra, lds, aoff, g, roff, g0 + t, t, acc, accm);
            if (t + 2 < gn) {
#pragma unroll
                for (int c = 0; c < T; c++) F::load(wb, roff[c], g0 + t + 2, g, ra[c]);
            }
            if (t + 1 >= gn) break;
            qh_mmv_group<F, T>(rb, lds, aoff, g, roff, g0 + t + 1, t + 1, acc, accm);
            if (t + 3 < gn) {
#pragma unroll
                for (int c = 0; c < T; c++) F::load(wb, roff[c], g0 + t + 3, g, rb[c]);
            }
        }
    }
    // Each row's total: both lane halves, all wavefronts.
    float v[T];
#pragma unroll
    for (int c = 0; c < T; c++) {
        v[c] = fmaf(acc[c], xs, accm[c]);
        v[c] += __shfl_xor(v[c], 32);
    }
    __syncthreads();
    float* red = reinterpret_cast<float*>(qh_lds);
    if (g == 0) {
#pragma unroll
        for (int c = 0; c < T; c++) red[(w * T + c) * 32 + n] = v[c];
    }
    __syncthreads();
    if (w < T && g == 0) {
        const int c = w;
        const int r = (blockIdx.x * T + c) * rt + n;
        if (n < rt && r < out_dim) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < QH_MMV_WAVES; i++) s += red[(i * T + c) * 32 + n];
            y[r] = s;
        }
    }
}

// Rows per column tile: at most 32, chosen so the workgroups (T tiles each)
// spread evenly over the device's CUs (14336 rows, T=2 -> 28-row tiles, 256 WGs).
static int qh_tile_rows(int out_dim, int T) {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        hipDeviceProp_t prop;
        cus = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
                  ? prop.multiProcessorCount
                  : 256;
    }
    const int64_t per_round = 32LL * T * cus;
    const int64_t rounds = ((int64_t)out_dim + per_round - 1) / per_round;
    const int64_t r = ((int64_t)out_dim + rounds * T * cus - 1) / (rounds * T * cus);
    return (int)(r < 1 ? 1 : (r > 32 ? 32 : r));
}

template <class F, int T>
static hipError_t launch_mmv(const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                             uint32_t row_bytes, hipStream_t st) {
    const int ngroups = in_dim / 256;
    const int gpw = (ngroups + QH_MMV_WAVES - 1) / QH_MMV_WAVES;
    size_t lds = (size_t)QH_MMV_WAVES * gpw * 8 * QH_UNIT_LDS;
    if (lds < (size_t)QH_MMV_WAVES * T * 32 * sizeof(float)) lds = (size_t)QH_MMV_WAVES * T * 32 * sizeof(float);
    const int rt = qh_tile_rows(out_dim, T);
    const int64_t wg_rows = (int64_t)T * rt;
    const int64_t max_rows = (((int64_t)1 << 31) / row_bytes) / wg_rows * wg_rows;
    if (max_rows < wg_rows) return hipErrorInvalidValue;
    for (int64_t r0 = 0; r0 < out_dim; r0 += max_rows) {
        const int rows = (int)((out_dim - r0) < max_rows ? (out_dim - r0) : max_rows);
        const uint32_t wbytes = (uint32_t)(((uint64_t)rows * row_bytes + 3) & ~(uint64_t)3);
        hipLaunchKernelGGL((qh_mmv<F, T>), dim3((unsigned)((rows + wg_rows - 1) / wg_rows)),
                           dim3(64 * QH_MMV_WAVES), lds, st, W + (size_t)r0 * row_bytes, wbytes, x, y + r0, rows,
                           row_bytes, ngroups, gpw, rt);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Returns hipErrorNotSupported when the type/shape has no matrix-core kernel.
hipError_t qh_launch_mmv(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                         hipStream_t st) {
    if (in_dim % 256 || ((uintptr_t)x & 15u)) return hipErrorNotSupported;
    const int gpw = (in_dim / 256 + QH_MMV_WAVES - 1) / QH_MMV_WAVES;
    if ((size_t)QH_MMV_WAVES * gpw * 8 * QH_UNIT_LDS > 64 * 1024) return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    switch (type) {
        case QT_Q4_K: return launch_mmv<MQ4K, 1>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q6_K: return launch_mmv<MQ6K, 1>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q8_0: return launch_mmv<MQ8_0, 1>(W, x, y, in_dim, out_dim, row_bytes, st);
        default: return hipErrorNotSupported;
    }
}
