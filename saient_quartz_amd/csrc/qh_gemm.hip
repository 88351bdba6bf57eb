// qh_gemm.hip -- batched dequant-GEMM for n = 2..16 tokens on the int8 matrix
// cores (v_mfma_i32_32x32x32_i8), Q4_K / Q5_K / Q6_K / IQ3_S / IQ2_XXS.
//
// Y[t][j] = sum_k W[j,k] X[t][k], X and Y token-major.  One pass over the weights
// serves every token: the weights are the B operand (32 weight rows = the 32
// MFMA columns), the tokens are the A operand (A row 2t + m = digit m of token
// t's x), so a lane's 16 results all belong to one weight row and one scale.
//   * x as two balanced int8 digits: per token and K chunk, s = 14 - exponent of
//     max|x|, x * 2^s is rounded to an integer of at most 2^14 in magnitude (one
//     FMA against a magic constant) and split into d0 + 256 d1.  The int32 MFMA
//     sums are exact; x's rounding (<= 2^-15 of the chunk's largest |x| per token)
//     is the only error added (measured ~3e-5 relative L2 against the oracle,
//     against the 1e-3 bar).
//   * Q4_K / Q5_K: one MFMA per 32-weight sub-block (one scale), 16 tokens each.
//     Q6_K: 16-weight scale groups, so a 32-weight chunk carries two scales: A
//     rows 0-15 hold tokens' digits for k < 16 and rows 16-31 for k >= 16, 8
//     tokens per MFMA, and result registers 0-7 / 8-15 take the two scales.
//   * mins (Q4_K/Q5_K dmin * m_j * sum(x)): one more MFMA per group whose B
//     operand is the 8 mins and whose A operand is the per-token sums of x over
//     the sub-blocks, digitised the same way.  Q6_K's -32 is in its B operand
//     (q - 32 is a signed byte), so its sums are not needed.
// Weights are read with the same coalesced, LDS-staged, persistent pipeline as
// qh_mmv16.hip (tiles of 32 rows; the next item's loads are in flight while the
// current one is computed).  Every item re-digitises x for its K chunk and all
// tokens (4 NT elements per lane).
//
// Reference counterpart: dequant::gemm (src/dequant.rs:143-200) with
// q4k_row_batched / q6k_row_batched (:38-122); the reference has no GPU
// batched path.
#include "qh_formats.h"
#include "qh_internal.h"

typedef int32_t qh_i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t qh_i32x16 __attribute__((ext_vector_type(16)));

#define QG_MAXT 4  // row tiles per workgroup (their results wait in LDS until the end)

// ---------------------------------------------------------------- formats

// Q4_K (src/dequant.rs:1471-1519): sub-block sb = 2p + nibble uses qs[32p + l].
struct GQ4K {
    static constexpr int BYTES = 144, CH = 9, RS = 144, LAST = 128;
    static constexpr int SUMK = 32, SUMSH = 5;  // x sums over 32 (the mins' pieces)
    static constexpr bool SUMS = true;
    static constexpr int KIND = 0, GRID = 0;  // sub-block pairs from one qs load
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
    // B operands of sub-blocks 2p, 2p+1 for lane half hh (k = 16 hh + e).
    template <int P>
    static QH_DEV void bpair(const unsigned char* r, int hh, qh_i32x4& b0, qh_i32x4& b1) {
        const qh_u32x4 q = *reinterpret_cast<const qh_u32x4*>(r + 16 + 32 * P + 16 * hh);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            b0[i] = (int)(q[i] & 0x0F0F0F0Fu);
            b1[i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
        }
    }
    template <int SB>
    static QH_DEV int scl(const H& h) { return (int)(((SB < 4 ? h.sc0 : h.sc1) >> (8 * (SB & 3))) & 0xFFu); }
    // B operand of the sums MFMA: the 8 mins in k = 0..7 (lanes of half 0).
    static QH_DEV qh_i32x4 bmin(const unsigned char*, const H& h, int hh) {
        return hh == 0 ? qh_i32x4{(int)h.mn0, (int)h.mn1, 0, 0} : qh_i32x4{0, 0, 0, 0};
    }
};

// Q5_K (src/dequant.rs:1146-1182): as Q4_K plus bit sb of qh[l] as bit 4.
struct GQ5K {
    static constexpr int BYTES = 176, CH = 11, RS = 176, LAST = 160;
    static constexpr int SUMK = 32, SUMSH = 5;
    static constexpr bool SUMS = true;
    static constexpr int KIND = 0, GRID = 0;
    using H = GQ4K::H;
    static QH_DEV H hdr(const unsigned char* r) { return GQ4K::hdr(r); }
    template <int P>
    static QH_DEV void bpair(const unsigned char* r, int hh, qh_i32x4& b0, qh_i32x4& b1) {
        const qh_u32x4 q = *reinterpret_cast<const qh_u32x4*>(r + 48 + 32 * P + 16 * hh);
        const qh_u32x4 u = *reinterpret_cast<const qh_u32x4*>(r + 16 + 16 * hh);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v = u[i] >> (2 * P);
            b0[i] = (int)((q[i] & 0x0F0F0F0Fu) | ((v & 0x01010101u) << 4));
            b1[i] = (int)(((q[i] >> 4) & 0x0F0F0F0Fu) | ((v & 0x02020202u) << 3));
        }
    }
    template <int SB>
    static QH_DEV int scl(const H& h) { return GQ4K::scl<SB>(h); }
    static QH_DEV qh_i32x4 bmin(const unsigned char* r, const H& h, int hh) { return GQ4K::bmin(r, h, hh); }
};

// Q6_K (src/dequant.rs:1583-1631): chunk c = 4 half + quarter covers 32
// consecutive weights: ql[64 half + 32 (quarter&1) + l] nibble quarter>>1, qh[32
// half + l] bits 2 quarter..; scales 2c (l < 16) and 2c + 1 (l >= 16).
struct GQ6K {
    static constexpr int BYTES = 210, CH = 14, RS = 240, LAST = 194;  // d lands at 222
    static constexpr int SUMK = 16, SUMSH = 4;
    static constexpr bool SUMS = false;  // the -32 is in the B operand
    static constexpr int KIND = 2, GRID = 0;  // two scales per 32 weights
    struct H { qh_u32x4 s; float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) {
        H o;
        o.s = *reinterpret_cast<const qh_u32x4*>(r + 192);
        o.d = qh_h2f(*reinterpret_cast<const uint16_t*>(r + 222));
        o.dm = 0.f;
        return o;
    }
    template <int C>
    static QH_DEV qh_i32x4 bop(const unsigned char* r, int hh) {
        constexpr int half = C >> 2, qu = C & 3;
        const qh_u32x4 l = *reinterpret_cast<const qh_u32x4*>(r + 64 * half + 32 * (qu & 1) + 16 * hh);
        const qh_u32x4 u = *reinterpret_cast<const qh_u32x4*>(r + 128 + 32 * half + 16 * hh);
        qh_i32x4 b;
#pragma unroll
        for (int i = 0; i < 4; i++)
            // q in 0..63 per byte; (q + 0x60) ^ 0x80 is q - 32 as a signed byte (no carries)
            b[i] = (int)(((((l[i] >> (4 * (qu >> 1))) & 0x0F0F0F0Fu) | (((u[i] >> (2 * qu)) & 0x03030303u) << 4)) +
                          0x60606060u) ^ 0x80808080u);
        return b;
    }
    template <int G>
    static QH_DEV int scl(const H& h) { return ((int)(h.s[G >> 2] >> (8 * (G & 3))) << 24) >> 24; }
};


// IQ3_S (src/dequant.rs:1184-1237), 110-byte blocks: d, qs[64], qh[8],
// signs[32], scales[4].  Sub-block k (32 weights, scale d (1 + 2 nibble)):
// 8-weight group l has grid indices qs[8k + 2l], qs[8k + 2l + 1] with bits 2l,
// 2l+1 of qh[k] as bit 8, and sign byte signs[4k + l].  Weights are signed grid
// bytes, so the B operand holds the dequantized value / (d scale) exactly.
// The 7th 16-byte slice is loaded from block bytes 94-109: block byte b >= 96
// sits at LDS b + 2.
extern __device__ uint32_t qh_g_iq3s[512];
extern __device__ uint64_t qh_g_iq2xxs[256];

QH_DEV uint32_t qh_rd16(const unsigned char* p, int o) { return *reinterpret_cast<const uint16_t*>(p + o); }

struct GIQ3S {
    static constexpr int BYTES = 110, CH = 7, RS = 112, LAST = 94;
    static constexpr int SUMK = 32, SUMSH = 5;
    static constexpr bool SUMS = false;
    static constexpr int KIND = 1, GRID = 1;  // one scale per 32 weights; IQ3S codebook in LDS
    struct H { float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) { return H{qh_h2f(qh_rd16(r, 0)), 0.f}; }
    static QH_DEV int at(int o) { return o >= 96 ? o + 2 : o; }
    template <int K>
    static QH_DEV void bop(const unsigned char* r, int hh, const unsigned char* grid, qh_i32x4& b, int& sc) {
        const int oq = 2 + 8 * K + 4 * hh;  // 4 index bytes of groups 2hh, 2hh+1
        const uint32_t q = qh_rd16(r, oq) | (qh_rd16(r, oq + 2) << 16);
        const uint32_t qh = (uint32_t)r[66 + K] >> (4 * hh);
        const uint32_t sg = qh_rd16(r, at(74 + 4 * K + 2 * hh));
        const uint32_t* g32 = reinterpret_cast<const uint32_t*>(grid);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t idx = ((q >> (8 * m)) & 0xFFu) | (((qh >> m) & 1u) << 8);
            b[m] = (int)qh_negbytes(g32[idx], qh_signmask4(sg >> (4 * m)));
        }
        sc = 1 + 2 * (int)((r[at(106 + K / 2)] >> (4 * (K & 1))) & 0xFu);
    }
};

// IQ2_XXS (src/dequant.rs:1011-1041), 66-byte blocks: d, then per sub-block k 4
// grid indices (bytes 2+8k..) and a u32 (bytes 6+8k..) holding four 7-bit sign
// fields and the scale in bits 28-31: weight = d/8 (2 scale + 1) grid * sign.
// The 5th slice is loaded from block bytes 50-65: block byte b >= 64 sits at LDS
// b + 14.
struct GIQ2XXS {
    static constexpr int BYTES = 66, CH = 5, RS = 80, LAST = 50;
    static constexpr int SUMK = 32, SUMSH = 5;
    static constexpr bool SUMS = false;
    static constexpr int KIND = 1, GRID = 2;  // IQ2XXS codebook in LDS
    struct H { float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) { return H{0.125f * qh_h2f(qh_rd16(r, 0)), 0.f}; }
    static QH_DEV int at(int o) { return o >= 64 ? o + 14 : o; }
    template <int K>
    static QH_DEV void bop(const unsigned char* r, int hh, const unsigned char* grid, qh_i32x4& b, int& sc) {
        const uint32_t a0 = qh_rd16(r, 2 + 8 * K + 2 * hh);  // indices of groups 2hh, 2hh+1
        const uint32_t a1 = qh_rd16(r, at(6 + 8 * K)) | (qh_rd16(r, at(8 + 8 * K)) << 16);
        const uint64_t* g64 = reinterpret_cast<const uint64_t*>(grid);
#pragma unroll
        for (int l = 0; l < 2; l++) {
            const uint64_t g = g64[(a0 >> (8 * l)) & 0xFFu];
            const uint32_t s8 = qh_ksigns((a1 >> (7 * (2 * hh + l))) & 127u);
            b[2 * l] = (int)qh_negbytes((uint32_t)g, qh_signmask4(s8));
            b[2 * l + 1] = (int)qh_negbytes((uint32_t)(g >> 32), qh_signmask4(s8 >> 4));
        }
        sc = 2 * (int)(a1 >> 28) + 1;
    }
};

template <class F>
struct IsQ6 { static constexpr bool value = false; };
template <>
struct IsQ6<GQ6K> { static constexpr bool value = true; };

// ---------------------------------------------------------------- kernel

// LDS per wavefront: x digits of one group for NT tokens -- plane 2t+m (digit m
// of token t, 256 bytes) at PS (2t+m), sum digits of plane 2t+m at
// SUMS + 16 (2t+m) (8 or 16 bytes used, the rest stays zero), 256 zero bytes, and
// 2^-s / 2^-(s - SUMSH) per token.
template <int NT>
struct XL {
    static constexpr int PS = 272;  // plane stride: 256 bytes + 16, conflict-free b128 reads over 16 rows
    static constexpr int SUMS = 2 * PS * NT;
    static constexpr int ZERO = SUMS + 32 * NT;
    static constexpr int RS_ = ZERO + 256;
    static constexpr int BYTES = RS_ + 8 * NT;
};

template <class F, int NT, int W>
__global__ __launch_bounds__(64 * W) void qh_mmq(const uint8_t* __restrict__ Wt, uint32_t wbytes,
                                                 const float* __restrict__ x, float* __restrict__ y, int out_dim,
                                                 uint32_t row_bytes, int ngroups, int in_dim, int n, int ldy) {
    constexpr int CH = F::CH, RS = F::RS;
    constexpr int NH = (32 * CH + 63) / 64;  // 16-byte loads per lane per group
    constexpr int TILE = 32 * RS + 16;
    constexpr int LPT = 64 / NT, EPL = 4 * NT;  // lanes per token, x elements per lane
    constexpr int NV = EPL / 4;                  // float4 per lane
    static_assert(NT == 2 || NT == 4 || NT == 8 || NT == 16, "NT");
    using X = XL<NT>;
    constexpr int GRIDB = F::GRID ? 2048 : 0;  // codebook (IQ3S: 512 x u32, IQ2XXS: 256 x u64)
    __shared__ __align__(16) unsigned char lds[W * TILE + W * X::BYTES + W * NT * 32 * 4 + QG_MAXT * NT * 32 * 4 +
                                               GRIDB];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int R = lane & 31, hh = lane >> 5;
    unsigned char* wl = lds + w * TILE;
    unsigned char* xl = lds + W * TILE + w * X::BYTES;
    float* red = reinterpret_cast<float*>(lds + W * TILE + W * X::BYTES);
    float* res = red + W * NT * 32;
    unsigned char* gridl = reinterpret_cast<unsigned char*>(res + QG_MAXT * NT * 32);
    if constexpr (F::GRID != 0) {
        const uint32_t* src = F::GRID == 1 ? qh_g_iq3s : reinterpret_cast<const uint32_t*>(qh_g_iq2xxs);
        for (int i = threadIdx.x; i < 512; i += 64 * W) reinterpret_cast<uint32_t*>(gridl)[i] = src[i];
        __syncthreads();
    }
    const QhBuf wb = qh_buf(Wt, wbytes);
    const QhBuf xb = qh_buf(x, 4u * (uint32_t)n * (uint32_t)in_dim);
    const int ntiles = (out_dim + 31) / 32;
    const int nch = (ngroups + W - 1) / W;

    // Zero this wavefront's x area once: sum-digit padding and the zero area are
    // never written afterwards.
    for (int i = lane * 16; i < X::BYTES; i += 64 * 16)
        if (i + 16 <= X::BYTES) *reinterpret_cast<qh_u32x4*>(xl + i) = qh_u32x4{0, 0, 0, 0};

    // Weight slices of this lane: row rr[h] of the tile, byte offset goff[h] from
    // the tile's first row, LDS offset soff[h] (lanes past 32 * CH: spare bytes).
    uint32_t goff[NH], soff[NH];
    int rr[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) {
        const int q = 64 * h + lane, r = q / CH, c = q - CH * r;
        rr[h] = q < 32 * CH ? r : 1 << 30;
        goff[h] = (uint32_t)r * row_bytes + (c == CH - 1 ? F::LAST : 16u * c);
        soff[h] = q < 32 * CH ? (uint32_t)(r * RS + 16 * c) : (uint32_t)(32 * RS);
    }
    // x slice of this lane: token tx, elements EPL * part .. of the group.
    const int tx = lane / LPT, part = lane % LPT;

    auto load_w = [&](int tile, int ch, qh_u32x4* wo) {
        const int g = ch * W + w;
        const uint32_t base = (uint32_t)(tile * 32) * row_bytes;
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const bool ok = tile * 32 + rr[h] < out_dim && g < ngroups;
            wo[h] = qh_ld128(wb, (ok ? base + goff[h] : 0x80000000u) + (uint32_t)F::BYTES * (uint32_t)g);
        }
    };
    auto load_x = [&](int ch, float4* xo) {
        const int g = ch * W + w;
        const uint32_t off = (g < ngroups && tx < n)
                                 ? 4u * ((uint32_t)tx * (uint32_t)in_dim + 256u * (uint32_t)g + (uint32_t)(EPL * part))
                                 : 0x80000000u;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const qh_u32x4 v = qh_ld128(xb, off + 16u * i);
            xo[i] = float4{__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
        }
    };
    // x -> two digit planes per token + digitised sums over SUMK.
    //   fmaf(x, 2^s, 12615808) = 1.5 * 2^23 + 0x8080 + n (n = round(x 2^s), |n| <=
    //   2^14), so the float's low 16 bits are n + 0x8080 and its bytes XOR 0x80
    //   are the balanced digits; the sums are exact integer sums of those n (sum
    //   of the float bits minus k * 0x4B408080, mod 2^32).
    //   A token whose chunk holds Inf or NaN (max|x| is Inf, or a bit sum falls
    //   outside the range finite values allow) gets 2^-s = NaN, so exactly its
    //   outputs are NaN, as in the reference's f32 dot.
    auto prep_x = [&](const float4* xv) {
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            // v_max3_f32 with |.| source modifiers: one instruction per two elements
            // (NaN is caught by the bit-sum check below, not by the max).
            __asm__("v_max3_f32 %0, |%1|, |%2|, %0" : "+v"(m) : "v"(xv[i].x), "v"(xv[i].y));
            __asm__("v_max3_f32 %0, |%1|, |%2|, %0" : "+v"(m) : "v"(xv[i].z), "v"(xv[i].w));
        }
#pragma unroll
        for (int o = 1; o < LPT; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
        int e = 0;
        (void)frexpf(m, &e);
        // |x| * 2^s <= 2^14: even after rounding, n + 0x8080 stays below 2^16.
        int s = m > 0.f ? 14 - e : 0;
        s = s > 126 ? 126 : (s < -126 ? -126 : s);
        const float scx = ldexpf(1.0f, s);
        const float magic = 12615808.0f;  // 0x4B408080
        unsigned char* p0 = xl + X::PS * (2 * tx) + EPL * part;
        constexpr int PIECE = F::SUMS ? F::SUMK : EPL;  // elements per checked bit sum
        constexpr int PL = PIECE < EPL ? PIECE : EPL;    // of which in this lane
        uint32_t psum = 0;
        bool nonfinite = !(m <= 3.0e38f);
        auto piece_done = [&](int j) {
            uint32_t ps = psum;
            if constexpr (PIECE > EPL) {
#pragma unroll
                for (int o = 1; o < PIECE / EPL; o <<= 1) ps += (uint32_t)__shfl_xor((int)ps, o);
            }
            const int sn = (int)(ps - (uint32_t)PIECE * 0x4B408080u);
            nonfinite |= sn > PIECE * 16384 || sn < -PIECE * 16384;
            if constexpr (F::SUMS) {
                if (PIECE <= EPL || (part % (PIECE / EPL)) == 0) {
                    // sum of n in units of 2^SUMSH (|result| <= 2^14)
                    const int ns = (sn + (1 << (F::SUMSH - 1))) >> F::SUMSH;
                    const uint32_t u = (uint32_t)(ns + 0x8080);
                    xl[X::SUMS + 16 * (2 * tx) + j] = (unsigned char)((u & 0xFFu) ^ 0x80u);
                    xl[X::SUMS + 16 * (2 * tx + 1) + j] = (unsigned char)(((u >> 8) & 0xFFu) ^ 0x80u);
                }
            }
            psum = 0;
        };
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const float4 v = xv[i];
            const uint32_t a0 = __float_as_uint(fmaf(v.x, scx, magic));
            const uint32_t a1 = __float_as_uint(fmaf(v.y, scx, magic));
            const uint32_t a2 = __float_as_uint(fmaf(v.z, scx, magic));
            const uint32_t a3 = __float_as_uint(fmaf(v.w, scx, magic));
            const uint32_t t01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
            const uint32_t t23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
            *reinterpret_cast<uint32_t*>(p0 + 4 * i) = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
            *reinterpret_cast<uint32_t*>(p0 + X::PS + 4 * i) =
                __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
            psum += a0 + a1 + a2 + a3;
            if ((4 * i + 4) % PL == 0) piece_done((EPL * part + 4 * i) / PIECE);
        }
        // every lane of the token agrees on the flag
        int nf = nonfinite ? 1 : 0;
#pragma unroll
        for (int o = 1; o < LPT; o <<= 1) nf |= __shfl_xor(nf, o);
        if (part == 0) {
            reinterpret_cast<float*>(xl + X::RS_)[tx] = nf ? __builtin_nanf("") : ldexpf(1.0f, -s);
            reinterpret_cast<float*>(xl + X::RS_)[NT + tx] = ldexpf(1.0f, F::SUMSH - s);
        }
    };
    auto stage = [&](const qh_u32x4* wr) {
#pragma unroll
        for (int h = 0; h < NH; h++) *reinterpret_cast<qh_u32x4*>(wl + soff[h]) = wr[h];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // Token slots of this lane: t = 4q + 2hh + r (q < 4, r < 2); result register
    // 4q + 2r + m of a 16-token MFMA holds digit m of slot (q, r).
    float tot[8];
#pragma unroll
    for (int i = 0; i < 8; i++) tot[i] = 0.f;
    const unsigned char* wrow = wl + R * RS;
    // A operand offsets.  Main (Q4_K/Q5_K): plane R (token R/2, digit R%2).
    const uint32_t aoffm = (R >> 1) < NT ? (uint32_t)X::PS * R + 16u * hh : (uint32_t)X::ZERO;
    // Sums MFMA: plane R's sum digits in k = 0..15 (half 0 only).
    const uint32_t aoffs = (hh == 0 && (R >> 1) < NT) ? (uint32_t)(X::SUMS + 16 * R) : (uint32_t)X::ZERO;
    // Q6_K: MFMA u covers tokens 8u..8u+7; rows R < 16 take k < 16, rows >= 16 k >= 16.
    uint32_t aoff6[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int t = 8 * u + ((R & 15) >> 1);
        aoff6[u] = ((R >> 4) == hh && t < NT) ? (uint32_t)X::PS * (16 * u + (R & 15)) + 16u * hh : (uint32_t)X::ZERO;
    }

    auto compute = [&]() {
        const typename F::H hd = F::hdr(wrow);
        const float* rsv = reinterpret_cast<const float*>(xl + X::RS_);
        int acc[16];
        int acc2[16];
#pragma unroll
        for (int j = 0; j < 16; j++) acc[j] = acc2[j] = 0;
        if constexpr (F::KIND == 1) {
            auto sub = [&](auto KC) {
                constexpr int K = decltype(KC)::value;
                qh_i32x4 b;
                int sc;
                F::template bop<K>(wrow, hh, gridl, b, sc);
                const qh_i32x4 a = *reinterpret_cast<const qh_i32x4*>(xl + aoffm + 32 * K);
                const qh_i32x16 z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
                const qh_i32x16 d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4 * (NT < 4 ? 1 : NT / 4); j++) acc[j] += __mul24(sc, d[j]);
                __builtin_amdgcn_sched_barrier(0);
            };
            sub(std::integral_constant<int, 0>{});
            sub(std::integral_constant<int, 1>{});
            sub(std::integral_constant<int, 2>{});
            sub(std::integral_constant<int, 3>{});
            sub(std::integral_constant<int, 4>{});
            sub(std::integral_constant<int, 5>{});
            sub(std::integral_constant<int, 6>{});
            sub(std::integral_constant<int, 7>{});
        } else if constexpr (!IsQ6<F>::value) {
            auto pair = [&](auto PC) {
                constexpr int P = decltype(PC)::value;
                qh_i32x4 b0, b1;
                F::template bpair<P>(wrow, hh, b0, b1);
                const qh_i32x4 a0 = *reinterpret_cast<const qh_i32x4*>(xl + aoffm + 64 * P);
                const qh_i32x4 a1 = *reinterpret_cast<const qh_i32x4*>(xl + aoffm + 64 * P + 32);
                const qh_i32x16 z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
                const qh_i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, z, 0, 0, 0);
                const int s0 = F::template scl<2 * P>(hd);
#pragma unroll
                for (int j = 0; j < 4 * (NT < 4 ? 1 : NT / 4); j++) acc[j] += __mul24(s0, d0[j]);
                __builtin_amdgcn_sched_barrier(0);
                const qh_i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, z, 0, 0, 0);
                const int s1 = F::template scl<2 * P + 1>(hd);
#pragma unroll
                for (int j = 0; j < 4 * (NT < 4 ? 1 : NT / 4); j++) acc[j] += __mul24(s1, d1[j]);
                __builtin_amdgcn_sched_barrier(0);
            };
            pair(std::integral_constant<int, 0>{});
            pair(std::integral_constant<int, 1>{});
            pair(std::integral_constant<int, 2>{});
            pair(std::integral_constant<int, 3>{});
        } else {
            auto chunk = [&](auto CC) {
                constexpr int C = decltype(CC)::value;
                const qh_i32x4 b = F::template bop<C>(wrow, hh);
                const int slo = F::template scl<2 * C>(hd), shi = F::template scl<2 * C + 1>(hd);
                const qh_i32x16 z = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
                {
                    const qh_i32x4 a = *reinterpret_cast<const qh_i32x4*>(xl + aoff6[0] + 32 * C);
                    const qh_i32x16 d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 8; j++) acc[j] += __mul24(slo, d[j]) + __mul24(shi, d[j + 8]);
                }
                if constexpr (NT > 8) {
                    const qh_i32x4 a = *reinterpret_cast<const qh_i32x4*>(xl + aoff6[1] + 32 * C);
                    const qh_i32x16 d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 8; j++) acc2[j] += __mul24(slo, d[j]) + __mul24(shi, d[j + 8]);
                }
                __builtin_amdgcn_sched_barrier(0);
            };
            chunk(std::integral_constant<int, 0>{});
            chunk(std::integral_constant<int, 1>{});
            chunk(std::integral_constant<int, 2>{});
            chunk(std::integral_constant<int, 3>{});
            chunk(std::integral_constant<int, 4>{});
            chunk(std::integral_constant<int, 5>{});
            chunk(std::integral_constant<int, 6>{});
            chunk(std::integral_constant<int, 7>{});
        }
        // sums MFMA: the mins (Q4_K/Q5_K)
        qh_i32x16 dm = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        if constexpr (F::SUMS) {
            const qh_i32x4 as = *reinterpret_cast<const qh_i32x4*>(xl + aoffs);
            dm = __builtin_amdgcn_mfma_i32_32x32x32_i8(as, F::bmin(wrow, hd, hh), dm, 0, 0, 0);
        }
        // finish: slot (q, r) = token 4q + 2hh + r
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int t = 4 * q + 2 * hh + r;
                if (4 * q >= NT) continue;  // slot beyond the tokens for both lane halves
                int i0, i1;
                if constexpr (!IsQ6<F>::value) {
                    i0 = acc[4 * q + 2 * r];
                    i1 = acc[4 * q + 2 * r + 1];
                } else {
                    // Q6_K: MFMA u = q/2 holds slot q in register 4 (q%2) + 2r + m
                    const int* a = (q < 2) ? acc : acc2;
                    i0 = a[4 * (q & 1) + 2 * r];
                    i1 = a[4 * (q & 1) + 2 * r + 1];
                }
                const float P = fmaf((float)i1, 256.0f, (float)i0);
                const int tt = t < NT ? t : 0;
                if constexpr (F::SUMS) {
                    const float Pm = fmaf((float)dm[4 * q + 2 * r + 1], 256.0f, (float)dm[4 * q + 2 * r]);
                    tot[2 * q + r] += fmaf(hd.d * P, rsv[tt], -hd.dm * Pm * rsv[NT + tt]);
                } else {
                    tot[2 * q + r] += hd.d * P * rsv[tt];
                }
            }
    };

    int tile = blockIdx.x, ch = 0, done = 0;
    if (tile >= ntiles) return;  // uniform over the workgroup
    qh_u32x4 wr[NH];
    float4 xv[NV];
    load_x(0, xv);
    load_w(tile, 0, wr);
    for (;;) {
        prep_x(xv);
        int ntile = tile, nc = ch + 1;
        if (nc == nch) { nc = 0; ntile += gridDim.x; }
        load_x(nc, xv);  // next item's x (L2-resident), in flight during the compute
        stage(wr);
        load_w(ntile, nc, wr);  // past the last tile: all offsets out of range, no traffic
        compute();
        if (nc == 0) {
            // Tile finished: lanes hold (token slot, weight row R); sum the wavefronts.
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const int t = 4 * q + 2 * hh + r;
                    if (t < NT) red[(w * NT + t) * 32 + R] = tot[2 * q + r];
                    tot[2 * q + r] = 0.f;
                }
            __syncthreads();
            // y is written after the loop: a store inside it would make the
            // compiler drain all loads in flight (stores and loads share vmcnt).
            for (int i = threadIdx.x; i < NT * 32; i += 64 * W) {
                float v = 0.f;
#pragma unroll
                for (int k = 0; k < W; k++) v += red[k * NT * 32 + i];
                res[done * NT * 32 + i] = v;
            }
            __syncthreads();
            done++;
        }
        if (ntile >= ntiles) break;
        tile = ntile;
        ch = nc;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < done * NT * 32; i += 64 * W) {
        const int k = i / (NT * 32), t = (i / 32) % NT, r = i & 31;
        const int row = (blockIdx.x + k * gridDim.x) * 32 + r;
        if (t < n && row < out_dim) y[(size_t)t * ldy + row] = res[i];
    }
}

template <class F, int NT, int W>
static hipError_t launch_mmq(const uint8_t* Wt, const float* x, float* y, int in_dim, int out_dim, int n,
                             uint32_t row_bytes, hipStream_t st) {
    static int resident = 0;
    if (!resident) {
        int dev = 0, per_cu = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, qh_mmq<F, NT, W>, 64 * W, 0) != hipSuccess ||
            per_cu < 1)
            return hipErrorNotSupported;
        resident = per_cu * prop.multiProcessorCount;
    }
    const int ngroups = in_dim / 256;
    const int64_t max_rows = (((int64_t)1 << 31) - 4096) / row_bytes / 32 * 32;
    if (max_rows < 32 || (int64_t)n * in_dim * 4 >= ((int64_t)1 << 31)) return hipErrorNotSupported;
    for (int64_t r0 = 0; r0 < out_dim; r0 += max_rows) {
        const int rows = (int)((out_dim - r0) < max_rows ? (out_dim - r0) : max_rows);
        const uint32_t wbytes = (uint32_t)(((uint64_t)rows * row_bytes + 3) & ~(uint64_t)3);
        const int ntiles = (rows + 31) / 32;
        int grid = ntiles < resident ? ntiles : resident;
        if ((ntiles + grid - 1) / grid > QG_MAXT) grid = (ntiles + QG_MAXT - 1) / QG_MAXT;
        // y rows r0.. of every token: y + r0 with the token stride out_dim.
        hipLaunchKernelGGL((qh_mmq<F, NT, W>), dim3((unsigned)grid), dim3(64 * W), 0, st,
                           Wt + (size_t)r0 * row_bytes, wbytes, x, y + r0, rows, row_bytes, ngroups, in_dim, n,
                           out_dim);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// QUARTZ_HIP_MMQ_WAVES=4|8 forces the workgroup size (tuning).
static int qh_mmq_waves_env() {
    static const int v = [] {
        const char* e = getenv("QUARTZ_HIP_MMQ_WAVES");
        return e ? atoi(e) : 0;
    }();
    return v;
}

// Batched tokens on the matrix cores; hipErrorNotSupported when the type/shape
// has no kernel here.  Tokens go in chunks of up to 16 (one weight pass each).
hipError_t qh_launch_mmq(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim, int n,
                         hipStream_t st) {
    if (in_dim % 256 || ((uintptr_t)x & 15u) || n < 2) return hipErrorNotSupported;
    if (type != QT_Q4_K && type != QT_Q5_K && type != QT_Q6_K && type != QT_IQ3_S && type != QT_IQ2_XXS)
        return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    for (int t0 = 0; t0 < n; t0 += 16) {
        const int nt = n - t0 < 16 ? n - t0 : 16;
        const float* xs = x + (size_t)t0 * in_dim;
        float* ys = y + (size_t)t0 * out_dim;
        hipError_t e;
        // 8 wavefronts per workgroup when the row tiles alone give few workgroups
        // (measured faster for Q4_K/Q5_K at 4096 rows); Q6_K's 16-token kernel
        // does not fit 8 wavefronts' registers.
        const bool w8 = qh_mmq_waves_env() == 8 ||
                        (qh_mmq_waves_env() != 4 && type != QT_Q6_K && (out_dim + 31) / 32 < 256);
#define QG_NT(F, NT_)                                                                                 \
    e = w8 ? launch_mmq<F, NT_, 8>(W, xs, ys, in_dim, out_dim, nt, row_bytes, st)                     \
           : launch_mmq<F, NT_, 4>(W, xs, ys, in_dim, out_dim, nt, row_bytes, st);
#define QG_CASE(F)                                                                                   \
    if (nt <= 2) { QG_NT(F, 2) } else if (nt <= 4) { QG_NT(F, 4) } else if (nt <= 8) { QG_NT(F, 8) } \
    else { QG_NT(F, 16) }
        if (type == QT_Q4_K) { QG_CASE(GQ4K) }
        else if (type == QT_Q5_K) { QG_CASE(GQ5K) }
        else if (type == QT_IQ3_S) { QG_CASE(GIQ3S) }
        else if (type == QT_IQ2_XXS) { QG_CASE(GIQ2XXS) }
        else { QG_CASE(GQ6K) }
#undef QG_CASE
#undef QG_NT
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
