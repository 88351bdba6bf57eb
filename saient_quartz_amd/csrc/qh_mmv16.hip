// qh_mmv16.hip -- staged matrix-core GEMV for the 256-weight superblock formats
// (Q4_K, Q5_K, Q6_K) on v_mfma_i32_16x16x64_i8.
//
// Workgroup = ROWS (<= 16) output rows x W wavefronts that split K.  A wavefront
// works on chunks of GPW superblock columns ("groups" of 256 weights):
//   1. it loads the chunk's x first (one float4 per lane per group), then the
//      chunk's weight bytes with fully coalesced 16-byte buffer loads: lane q of a
//      group's load covers slice q % CH of row q / CH (ROWS x CH x 16 bytes);
//   2. x is turned into three balanced int8 digit planes in LDS (the exponent is
//      per wavefront and chunk, so the int32 MFMA sums are exact);
//   3. per group, the wavefront writes its slices into a private LDS tile (one
//      RS-byte line per row, 16-byte aligned whatever the block alignment in
//      memory) and reads them back transposed: lane (n = lane % 16, kg = lane / 16)
//      takes the 16 weights k = 16 kg .. 16 kg + 15 of each 64-weight slice p of
//      row n as the B operand (column n).  The A operand holds digit m of those x
//      values in row 4 kg + m only, so result row 4 kg + m, column n (which the
//      MFMA returns in lane 16 kg + n, register m) is the digit-m dot of exactly
//      that lane's 16-weight group: every lane then applies its own group's
//      integer scale, with no shuffles.
//   4. sums over lanes and wavefronts finish through DPP/LDS.
//
// Reference counterpart: the warp-per-row cuda_gemv kernels of
// src/cuda_kernels.cu:1046-1077 (one f32 FMA per weight).
#include "qh_formats.h"
#include "qh_internal.h"

typedef int32_t qh_i32x4 __attribute__((ext_vector_type(4)));

#define QH_XU 256   // LDS bytes per 64-element x slice
#define QH_XU_SUM 192  // 4 f32 sums of 16 elements
#define QH_XU_ZERO 208 // 16 zero bytes: the A operand of lanes that carry no digits
#define QH_RS 240   // LDS line per row: 15 x 16 bytes, conflict-free b128 reads over 16 rows

// ---------------------------------------------------------------- formats
// Each format gives: BYTES (per superblock), CH (16-byte slices loaded per row and
// superblock), ROWS, a header decoded once per group (hdr), the B operand of
// slice p for this lane (bop), the lane's integer scale (scl) and the integer
// weight of its f32 x-sum (mn), and the two f32 factors of the group result:
//   y += d * 2^-s * sum(scl * digit dots) - dm * sum(mn * x16).

// Q4_K: d, dmin, scales[12], qs[128] (src/dequant.rs:1471-1519).  Weight = d*sc*q - dmin*m.
struct M16Q4K {
    static constexpr int BYTES = 144, CH = 9, ROWS = 14;
    struct H { uint32_t sc0, sc1, mn0, mn1; float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) {
        const qh_u32x4 h = *reinterpret_cast<const qh_u32x4*>(r);
        H o;
        o.sc0 = h.y & 0x3F3F3F3Fu;
        o.mn0 = h.z & 0x3F3F3F3Fu;
        o.sc1 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        o.mn1 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
        o.d = qh_f16_lo(h.x);
        o.dm = qh_f16_hi(h.x);
        return o;
    }
    // Slice p covers sub-blocks 2p (k < 32) and 2p+1: qs[32p + 16(kg&1) + e], nibble kg>>1.
    template <int P>
    static QH_DEV qh_i32x4 bop(const unsigned char* r, int kg, const H&) {
        const qh_u32x4 q = *reinterpret_cast<const qh_u32x4*>(r + 16 + 32 * P + 16 * (kg & 1));
        const uint32_t sh = 4u * (uint32_t)(kg >> 1);
        return qh_i32x4{(int)((q.x >> sh) & 0x0F0F0F0Fu), (int)((q.y >> sh) & 0x0F0F0F0Fu),
                        (int)((q.z >> sh) & 0x0F0F0F0Fu), (int)((q.w >> sh) & 0x0F0F0F0Fu)};
    }
    template <int P>
    static QH_DEV int scl(const H& h, int kg) {
        return (int)(((P < 2 ? h.sc0 : h.sc1) >> (16 * (P & 1) + 8 * (kg >> 1))) & 0xFFu);
    }
    template <int P>
    static QH_DEV int mn(const H& h, int kg) {
        return (int)(((P < 2 ? h.mn0 : h.mn1) >> (16 * (P & 1) + 8 * (kg >> 1))) & 0xFFu);
    }
};

// Q5_K: d, dmin, scales[12], qh[32], qs[128] (src/dequant.rs:1146-1182).
// Weight of sub-block j, position l: d*sc*(nibble + 16*bit_j(qh[l])) - dmin*m.
struct M16Q5K {
    static constexpr int BYTES = 176, CH = 11, ROWS = 11;
    using H = M16Q4K::H;
    static QH_DEV H hdr(const unsigned char* r) { return M16Q4K::hdr(r); }
    template <int P>
    static QH_DEV qh_i32x4 bop(const unsigned char* r, int kg, const H&) {
        const qh_u32x4 q = *reinterpret_cast<const qh_u32x4*>(r + 48 + 32 * P + 16 * (kg & 1));
        const qh_u32x4 u = *reinterpret_cast<const qh_u32x4*>(r + 16 + 16 * (kg & 1));
        const uint32_t sh = 4u * (uint32_t)(kg >> 1), j = 2u * P + (uint32_t)(kg >> 1);
        return qh_i32x4{(int)(((q.x >> sh) & 0x0F0F0F0Fu) | (((u.x >> j) & 0x01010101u) << 4)),
                        (int)(((q.y >> sh) & 0x0F0F0F0Fu) | (((u.y >> j) & 0x01010101u) << 4)),
                        (int)(((q.z >> sh) & 0x0F0F0F0Fu) | (((u.z >> j) & 0x01010101u) << 4)),
                        (int)(((q.w >> sh) & 0x0F0F0F0Fu) | (((u.w >> j) & 0x01010101u) << 4))};
    }
    template <int P>
    static QH_DEV int scl(const H& h, int kg) { return M16Q4K::scl<P>(h, kg); }
    template <int P>
    static QH_DEV int mn(const H& h, int kg) { return M16Q4K::mn<P>(h, kg); }
};

// Q6_K: ql[128], qh[64], scales[16] (int8), d (src/dequant.rs:1583-1620).
// Slice p = (half n = p/2, nibble p%2): position k = 16kg + e has
// q = nibble(ql[64n + 16kg + e]) | bits(qh[32n + 16(kg&1) + e] >> (4(p%2) + 2(kg>>1))) << 4,
// scale index 4p + kg and weight d*sc*(q - 32): the -32 goes through the x sums.
struct M16Q6K {
    static constexpr int BYTES = 210, CH = 14, ROWS = 16;
    struct H { qh_u32x4 s; float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) {
        H o;
        o.s = *reinterpret_cast<const qh_u32x4*>(r + 192);
        o.d = qh_f16_lo(*reinterpret_cast<const uint32_t*>(r + 208));
        o.dm = 32.0f * o.d;
        return o;
    }
    template <int P>
    static QH_DEV qh_i32x4 bop(const unsigned char* r, int kg, const H&) {
        const qh_u32x4 l = *reinterpret_cast<const qh_u32x4*>(r + 64 * (P >> 1) + 16 * kg);
        const qh_u32x4 u = *reinterpret_cast<const qh_u32x4*>(r + 128 + 32 * (P >> 1) + 16 * (kg & 1));
        constexpr uint32_t ls = 4u * (P & 1);
        const uint32_t us = ls + 2u * (uint32_t)(kg >> 1);
        return qh_i32x4{(int)(((l.x >> ls) & 0x0F0F0F0Fu) | (((u.x >> us) & 0x03030303u) << 4)),
                        (int)(((l.y >> ls) & 0x0F0F0F0Fu) | (((u.y >> us) & 0x03030303u) << 4)),
                        (int)(((l.z >> ls) & 0x0F0F0F0Fu) | (((u.z >> us) & 0x03030303u) << 4)),
                        (int)(((l.w >> ls) & 0x0F0F0F0Fu) | (((u.w >> us) & 0x03030303u) << 4))};
    }
    template <int P>
    static QH_DEV int scl(const H& h, int kg) {
        return ((int)(h.s[P] >> (8 * kg)) << 24) >> 24;
    }
    template <int P>
    static QH_DEV int mn(const H& h, int kg) { return scl<P>(h, kg); }
};

// ---------------------------------------------------------------- kernel

QH_DEV float qh_dpp_max(float m) {
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x140, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x142, 0xA, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x143, 0xC, 0xF, false)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 63));
}

template <class F, int W, int GPW>
__global__ __launch_bounds__(64 * W) void qh_mmv16(const uint8_t* __restrict__ Wt, uint32_t wbytes,
                                                   const float* __restrict__ x, float* __restrict__ y, int out_dim,
                                                   uint32_t row_bytes, int ngroups) {
    constexpr int ROWS = F::ROWS, CH = F::CH;
    constexpr int NH = (ROWS * CH + 63) / 64;  // 16-byte loads per lane and group
    static_assert(ROWS <= 16 && 16 * CH < QH_RS, "tile shape");
    __shared__ __align__(16) unsigned char lds[W * ROWS * QH_RS + W * GPW * 4 * QH_XU];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const QhBuf wb = qh_buf(Wt, wbytes);
    const int row0 = blockIdx.x * ROWS;
    unsigned char* wl = lds + w * (ROWS * QH_RS);
    unsigned char* xl = lds + W * ROWS * QH_RS + w * (GPW * 4 * QH_XU);

    uint32_t goff[NH], soff[NH];
    bool sok[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) {
        const int q = 64 * h + lane, r = q / CH, c = q - CH * r;
        sok[h] = q < ROWS * CH;
        goff[h] = (sok[h] && row0 + r < out_dim) ? (uint32_t)(row0 + r) * row_bytes + 16u * c : 0x80000000u;
        soff[h] = (uint32_t)(r * QH_RS + 16 * c);
    }
    const int n = lane & 15, kg = lane >> 4;
    const unsigned char* wrow = wl + (n < ROWS ? n : 0) * QH_RS;
    const uint32_t aoff = ((n >> 2) == kg && (n & 3) < 3) ? 64u * (n & 3) + 16u * kg : QH_XU_ZERO;
    const uint32_t bias = 0x4B400000u - 0x808080u;

    float tot = 0.f, bad = 0.f;
    for (int cg = w * GPW; cg < ngroups; cg += W * GPW) {
        float4 xv[GPW];
#pragma unroll
        for (int t = 0; t < GPW; t++)
            xv[t] = (cg + t < ngroups) ? *reinterpret_cast<const float4*>(x + 256 * (cg + t) + 4 * lane)
                                       : float4{0.f, 0.f, 0.f, 0.f};
        qh_u32x4 wr[GPW * NH];
#pragma unroll
        for (int t = 0; t < GPW; t++)
#pragma unroll
            for (int h = 0; h < NH; h++) {
                const uint32_t off = (cg + t < ngroups ? goff[h] : 0x80000000u) + (uint32_t)F::BYTES * (uint32_t)(cg + t);
                if (F::BYTES % 16 == 0 || off + 16u <= wbytes || off >= 0x80000000u) {
                    wr[t * NH + h] = qh_ld128(wb, off);
                } else {
                    // A slice that runs past the end of the tensor (the last block of a
                    // 210-byte format): a dword straddling the range end reads as zero,
                    // so load aligned dwords and realign.
                    uint32_t raw[5], v[4];
                    qh_ldwin<4>(wb, off, raw);
                    qh_fix<4>(raw, off, v);
                    wr[t * NH + h] = qh_u32x4{v[0], v[1], v[2], v[3]};
                }
            }

        // x -> digits.  One exponent per wavefront and chunk: max|x| * 2^s < 2^22.
        float m = 0.f;
#pragma unroll
        for (int t = 0; t < GPW; t++) {
            m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[t].x), fabsf(xv[t].y)), fmaxf(fabsf(xv[t].z), fabsf(xv[t].w))));
            bad += ((xv[t].x * 0.f + xv[t].y * 0.f) + (xv[t].z * 0.f + xv[t].w * 0.f));  // NaN iff x not finite
        }
        m = qh_dpp_max(m);
        int e = 0;
        (void)frexpf(m, &e);
        int s = m > 0.f ? 22 - e : 0;
        s = s > 126 ? 126 : s;
        const float scx = ldexpf(1.0f, s);
#pragma unroll
        for (int t = 0; t < GPW; t++) {
            const float4 v = xv[t];
            const uint32_t a0 = (__float_as_uint(fmaf(v.x, scx, 12582912.0f)) - bias) ^ 0x808080u;
            const uint32_t a1 = (__float_as_uint(fmaf(v.y, scx, 12582912.0f)) - bias) ^ 0x808080u;
            const uint32_t a2 = (__float_as_uint(fmaf(v.z, scx, 12582912.0f)) - bias) ^ 0x808080u;
            const uint32_t a3 = (__float_as_uint(fmaf(v.w, scx, 12582912.0f)) - bias) ^ 0x808080u;
            const uint32_t t01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
            const uint32_t t23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
            const uint32_t u01 = __builtin_amdgcn_perm(a1, a0, 0x06020602u);
            const uint32_t u23 = __builtin_amdgcn_perm(a3, a2, 0x06020602u);
            // lane holds x[256t + 4 lane .. +3]: slice lane/16, 16-group (lane/4)%4.
            unsigned char* ub = xl + (4 * t + (lane >> 4)) * QH_XU;
            const int pos = 4 * (lane & 15);
            *reinterpret_cast<uint32_t*>(ub + pos) = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
            *reinterpret_cast<uint32_t*>(ub + 64 + pos) = __builtin_amdgcn_perm(t23, t01, 0x07060302u);
            *reinterpret_cast<uint32_t*>(ub + 128 + pos) = __builtin_amdgcn_perm(u23, u01, 0x05040100u);
            float hs = (v.x + v.y) + (v.z + v.w);
            hs += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(hs), 0xB1, 0xF, 0xF, false));
            hs += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(hs), 0x4E, 0xF, 0xF, false));
            if ((lane & 3) == 0) *reinterpret_cast<float*>(ub + QH_XU_SUM + (lane & 12)) = hs;
            if ((lane & 15) == 0) *reinterpret_cast<qh_u32x4*>(ub + QH_XU_ZERO) = qh_u32x4{0, 0, 0, 0};
        }

        float acc = 0.f, accm = 0.f;
#pragma unroll
        for (int t = 0; t < GPW; t++) {
            // Stage group t.  The tile is reused per group: LDS operations of one
            // wavefront complete in order, so these writes follow the previous reads.
#pragma unroll
            for (int h = 0; h < NH; h++)
                if (sok[h]) *reinterpret_cast<qh_u32x4*>(wl + soff[h]) = wr[t * NH + h];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const typename F::H hd = F::hdr(wrow);
            int i0 = 0, i1 = 0, i2 = 0;
            float fm = 0.f;
            const unsigned char* xt = xl + 4 * t * QH_XU;
            auto slice = [&](auto PC) {
                constexpr int P = decltype(PC)::value;
                const qh_i32x4 B = F::template bop<P>(wrow, kg, hd);
                const qh_i32x4 a = *reinterpret_cast<const qh_i32x4*>(xt + P * QH_XU + aoff);
                const qh_i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, B, qh_i32x4{0, 0, 0, 0}, 0, 0, 0);
                const int sc = F::template scl<P>(hd, kg);
                i0 += __mul24(sc, D[0]);
                i1 += __mul24(sc, D[1]);
                i2 += __mul24(sc, D[2]);
                const float xs = *reinterpret_cast<const float*>(xt + P * QH_XU + QH_XU_SUM + 4 * kg);
                fm = fmaf((float)F::template mn<P>(hd, kg), xs, fm);
                __builtin_amdgcn_sched_barrier(0);
            };
            slice(std::integral_constant<int, 0>{});
            slice(std::integral_constant<int, 1>{});
            slice(std::integral_constant<int, 2>{});
            slice(std::integral_constant<int, 3>{});
            const float P = fmaf((float)i2, 65536.0f, fmaf((float)i1, 256.0f, (float)i0));
            acc = fmaf(hd.d, P, acc);
            accm = fmaf(hd.dm, fm, accm);
        }
        tot += fmaf(acc, ldexpf(1.0f, -s), -accm);
    }
    float v = tot + bad;
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    __syncthreads();
    float* red = reinterpret_cast<float*>(lds);
    if (lane < 16) red[w * 16 + lane] = v;
    __syncthreads();
    if (w == 0 && lane < ROWS && row0 + lane < out_dim) {
        float r = 0.f;
#pragma unroll
        for (int i = 0; i < W; i++) r += red[i * 16 + lane];
        y[row0 + lane] = r;
    }
}

template <class F, int W, int GPW>
static hipError_t launch_mmv16(const uint8_t* Wt, const float* x, float* y, int in_dim, int out_dim,
                               uint32_t row_bytes, hipStream_t st) {
    const int ngroups = in_dim / 256;
    // Rows are processed in chunks whose weight bytes fit a 31-bit buffer range.
    const int64_t max_rows = (((int64_t)1 << 31) - 4096) / row_bytes / F::ROWS * F::ROWS;
    if (max_rows < F::ROWS) return hipErrorNotSupported;
    for (int64_t r0 = 0; r0 < out_dim; r0 += max_rows) {
        const int rows = (int)((out_dim - r0) < max_rows ? (out_dim - r0) : max_rows);
        // Record count rounded up to a dword (the last 2-byte field of a 210-byte
        // block shares its dword with the byte after the tensor).
        const uint32_t wbytes = (uint32_t)(((uint64_t)rows * row_bytes + 3) & ~(uint64_t)3);
        hipLaunchKernelGGL((qh_mmv16<F, W, GPW>), dim3((unsigned)((rows + F::ROWS - 1) / F::ROWS)), dim3(64 * W), 0,
                           st, Wt + (size_t)r0 * row_bytes, wbytes, x, y + r0, rows, row_bytes, ngroups);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Returns hipErrorNotSupported when the type/shape has no kernel here.
hipError_t qh_launch_mmv16(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                           hipStream_t st) {
    if (in_dim % 256 || ((uintptr_t)x & 15u)) return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    switch (type) {
        case QT_Q4_K: return launch_mmv16<M16Q4K, 4, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q5_K: return launch_mmv16<M16Q5K, 4, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q6_K: return launch_mmv16<M16Q6K, 4, 4>(W, x, y, in_dim, out_dim, row_bytes, st);
        default: return hipErrorNotSupported;
    }
}
