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
#include <climits>

#include "qh_formats.h"
#include "qh_internal.h"

typedef int32_t qh_i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t qh_i32x16 __attribute__((ext_vector_type(16)));

#define QG_WAVES 4          // wavefronts per workgroup
#define QG_TARGET_WGS 256   // workgroups a launch aims for (measured best: one per CU; more split K further and lose)
#define QG_PART_TILES 2048  // (row tile, K split) partials the scratch holds

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


// IQ3_S and IQ2_XXS: the B operand of sub-block K, lane half hh, is the
// qh_iq3s_piece / qh_iq2xxs_piece of the staged block (signed codebook bytes,
// the dequantized value / (d scale) exactly), with the codebooks in LDS.
extern __device__ uint32_t qh_g_iq3s[512];
extern __device__ uint64_t qh_g_iq2xxs[256];

struct GIQ3S {
    static constexpr int BYTES = 110, CH = 7, RS = 112, LAST = 94;
    static constexpr int SUMK = 32, SUMSH = 5;
    static constexpr bool SUMS = false;
    static constexpr int KIND = 1, GRID = 1;  // one scale per 32 weights; IQ3S codebook in LDS
    struct H { float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) { return H{qh_h2f(qh_rd16(r, 0)), 0.f}; }
    template <int K>
    static QH_DEV void bop(const unsigned char* r, int hh, const unsigned char* grid, qh_i32x4& b, int& sc) {
        uint32_t v[4];
        qh_iq3s_piece(r, K, hh, reinterpret_cast<const uint32_t*>(grid), v, sc);
#pragma unroll
        for (int m = 0; m < 4; m++) b[m] = (int)v[m];
    }
};

struct GIQ2XXS {
    static constexpr int BYTES = 66, CH = 5, RS = 80, LAST = 50;
    static constexpr int SUMK = 32, SUMSH = 5;
    static constexpr bool SUMS = false;
    static constexpr int KIND = 1, GRID = 2;  // IQ2XXS codebook in LDS
    struct H { float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) { return H{0.125f * qh_h2f(qh_rd16(r, 0)), 0.f}; }
    template <int K>
    static QH_DEV void bop(const unsigned char* r, int hh, const unsigned char* grid, qh_i32x4& b, int& sc) {
        uint32_t v[4];
        qh_iq2xxs_piece(r, K, hh, reinterpret_cast<const uint64_t*>(grid), v, sc);
#pragma unroll
        for (int m = 0; m < 4; m++) b[m] = (int)v[m];
    }
};

template <class F>
struct IsQ6 { static constexpr bool value = false; };
template <>
struct IsQ6<GQ6K> { static constexpr bool value = true; };

// ---------------------------------------------------------------- x image

// The x operand of one 256-element group for 16 token slots ("image"), written
// once per call by qh_mmq_ximg and read by every workgroup with coalesced loads:
// chunk c is the A operand of one MFMA, lane L's 16 bytes at 1024 c + 16 L
// (lane L = row L % 32, k half L / 32 of the 32x32x32 MFMA).
//   KIND 0 / 1 (one scale per 32 weights): chunk k < 8 = sub-block k, row 2t+m =
//     digit m of token t; KIND 0 adds chunk 8, the sum digits of the 8
//     sub-blocks (row 2t+m, k half 0, bytes 0..7).
//   KIND 2 (Q6_K, scales per 16): chunk 8u+c = 32-weight chunk c for tokens
//     8u..8u+7 (so <= 8 tokens need only chunks 0..7): row 2(t%8)+m takes k < 16, row 16 + 2(t%8)+m takes k >= 16, the
//     other k half of each row is zero.
// Then 16 bytes: the digit exponent s of each token slot (127: Inf/NaN seen).
template <int KIND, bool SUMS>
struct XImg {
    static constexpr int CHUNKS = KIND == 2 ? 16 : (SUMS ? 9 : 8);
    static constexpr int EXP = 1024 * CHUNKS;
    static constexpr int BYTES = EXP + 256;  // per group
};
#define QG_MAX_GROUPS 256                     // in_dim <= 65536 on the matrix-core path
#define QG_SCRATCH (4 * QG_MAX_GROUPS * (16 * 1024 + 256))  // 16.6 MB: 4 slots at the largest in_dim
static __device__ __align__(256) unsigned char qh_mmq_scratch[QG_SCRATCH];
// Split-K partials (16 tokens x 32 rows per (tile, split)) and per-tile arrival
// counters; every counter is back at zero when a launch ends.
static __device__ __align__(256) float qh_mmq_part[QG_PART_TILES * 16 * 32];
static __device__ __align__(256) unsigned int qh_mmq_cnt[QG_PART_TILES];

#define QG_MAXG 16  // matrices (or row chunks) per grouped launch
struct QgXs {        // the distinct token blocks of one grouped launch
    const float* x[QG_MAXG];
    const float* x2[QG_MAXG];  // SwiGLU: x is silu(x) * x2 (gate, up) when non-null
    int n[QG_MAXG];  // tokens (<= 16)
};
struct QgGroups {    // the matrices of one grouped launch
    const uint8_t* w[QG_MAXG];
    float* y[QG_MAXG];
    uint32_t wbytes[QG_MAXG];  // buffer range of each matrix's weights
    int rows[QG_MAXG];
    int n[QG_MAXG];            // tokens of the matrix's x block
    int ldy[QG_MAXG];          // y token stride
    int slot[QG_MAXG];         // x image slot
    int bstart[QG_MAXG + 1];   // first workgroup of each matrix; entries past the count are INT_MAX
    int accum;                 // y += result (the residual add) instead of y = result
};

// One workgroup (256 threads) per group: thread T digitises elements 16 (T%16)
// .. +15 of token T/16 (zeros past n), building the image in LDS, then copies it
// out.  Digits: fmaf(x, 2^s, 12615808) = 1.5 * 2^23 + 0x8080 + n with n =
// round(x 2^s), |n| <= 2^14 (s = 14 - exponent of the token's max |x| over the
// group), so the float's low bytes XOR 0x80 are the balanced digits of n.
// Sums: exact integer sums of n over each sub-block, in units of 2^SUMSH.
// Grid (groups, slots): slot s digitises the n[s] tokens at x[s] into image
// slot s (img + s * ngroups * XI::BYTES).
template <int KIND, bool SUMS, int SUMSH>
__global__ __launch_bounds__(256) void qh_mmq_ximg(const QgXs xs, unsigned char* __restrict__ img, int in_dim) {
    using XI = XImg<KIND, SUMS>;
    __shared__ __align__(16) unsigned char im[XI::BYTES];
    const int T = threadIdx.x, g = blockIdx.x;
    const float* __restrict__ x = xs.x[blockIdx.y];
    const int n = xs.n[blockIdx.y];
    img += (size_t)blockIdx.y * gridDim.x * XI::BYTES;
    const int t = T >> 4, p = T & 15;
    for (int i = 16 * T; i < XI::BYTES; i += 16 * 256) *reinterpret_cast<qh_u32x4*>(im + i) = qh_u32x4{0, 0, 0, 0};
    __syncthreads();  // the zero fill lands before any thread's image writes
    float4 v[4];
    const QhBuf xb = qh_buf(x, 4u * (uint32_t)n * (uint32_t)in_dim);
    const uint32_t off = t < n ? 4u * ((uint32_t)t * (uint32_t)in_dim + 256u * (uint32_t)g + 16u * p) : 0x80000000u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const qh_u32x4 u = qh_ld128(xb, off + 16u * i);
        v[i] = float4{__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w)};
    }
    if (const float* x2 = xs.x2[blockIdx.y]) {
        // SwiGLU fused in: x = silu(gate) * up, qg_swiglu's expression
        const QhBuf ub = qh_buf(x2, 4u * (uint32_t)n * (uint32_t)in_dim);
        auto sw = [](float gv, float uv) { return (gv / (1.f + expf(-gv))) * uv; };
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const qh_u32x4 u = qh_ld128(ub, off + 16u * i);
            v[i] = float4{sw(v[i].x, __uint_as_float(u.x)), sw(v[i].y, __uint_as_float(u.y)),
                          sw(v[i].z, __uint_as_float(u.z)), sw(v[i].w, __uint_as_float(u.w))};
        }
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    // max over the 16 threads (one DPP row) of the token
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x140, 0xF, 0xF, false)));
    int e = 0;
    (void)frexpf(m, &e);
    int s = m > 0.f ? 14 - e : 0;
    s = s > 126 ? 126 : (s < -126 ? -126 : s);
    const float scx = ldexpf(1.0f, s);
    uint32_t a[16];
    uint32_t hi_or = 0, sum = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[4 * i + 0] = __float_as_uint(fmaf(v[i].x, scx, 12615808.0f));
        a[4 * i + 1] = __float_as_uint(fmaf(v[i].y, scx, 12615808.0f));
        a[4 * i + 2] = __float_as_uint(fmaf(v[i].z, scx, 12615808.0f));
        a[4 * i + 3] = __float_as_uint(fmaf(v[i].w, scx, 12615808.0f));
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        hi_or |= (a[i] >> 16) ^ 0x4B40u;  // nonzero iff a value was not finite (or out of range)
        sum += a[i];
    }
    // 16 bytes of digit m, in element order
    qh_u32x4 d0, d1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t t01 = __builtin_amdgcn_perm(a[4 * i + 1], a[4 * i], 0x05010400u);
        const uint32_t t23 = __builtin_amdgcn_perm(a[4 * i + 3], a[4 * i + 2], 0x05010400u);
        d0[i] = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
        d1[i] = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
    }
    const int c32 = p >> 1, kh = p & 1;  // 32-element piece of the group, k half
    if constexpr (KIND == 2) {
        const int u = t >> 3, r = 16 * kh + 2 * (t & 7);
        *reinterpret_cast<qh_u32x4*>(im + 1024 * (8 * u + c32) + 16 * (32 * kh + r)) = d0;
        *reinterpret_cast<qh_u32x4*>(im + 1024 * (8 * u + c32) + 16 * (32 * kh + r + 1)) = d1;
    } else {
        *reinterpret_cast<qh_u32x4*>(im + 1024 * c32 + 16 * (32 * kh + 2 * t)) = d0;
        *reinterpret_cast<qh_u32x4*>(im + 1024 * c32 + 16 * (32 * kh + 2 * t + 1)) = d1;
    }
    if constexpr (SUMS) {
        // integer sum of n over the sub-block (this thread and its neighbour)
        sum += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)sum, 0xB1, 0xF, 0xF, false);
        if (kh == 0) {
            const int sn = (int)(sum - 32u * 0x4B408080u);
            const int ns = (sn + (1 << (SUMSH - 1))) >> SUMSH;
            const uint32_t uu = (uint32_t)(ns + 0x8080);
            im[1024 * 8 + 16 * (2 * t) + c32] = (unsigned char)((uu & 0xFFu) ^ 0x80u);
            im[1024 * 8 + 16 * (2 * t + 1) + c32] = (unsigned char)(((uu >> 8) & 0xFFu) ^ 0x80u);
        }
    }
    // the token's non-finite flag, over its 16 threads
    uint32_t f = hi_or;
    f |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)f, 0xB1, 0xF, 0xF, false);
    f |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)f, 0x4E, 0xF, 0xF, false);
    f |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)f, 0x141, 0xF, 0xF, false);
    f |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)f, 0x140, 0xF, 0xF, false);
    __syncthreads();
    if (p == 0) im[XI::EXP + t] = (unsigned char)(signed char)(f ? 127 : s);
    __syncthreads();
    unsigned char* dst = img + (size_t)g * XI::BYTES;
    for (int i = 16 * T; i < XI::BYTES; i += 16 * 256)
        *reinterpret_cast<qh_u32x4*>(dst + i) = *reinterpret_cast<const qh_u32x4*>(im + i);
}

// ---------------------------------------------------------------- kernel

QH_DEV qh_i32x4 qh_as_i32x4(const qh_u32x4& v) { return qh_i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w}; }

// One workgroup of W wavefronts per (row tile of 32 rows, K split): wavefront w
// takes the split's groups w, w + W, ...  Per group ("item") it stages the tile's
// weight slices through its LDS tile (coalesced 16-byte loads, the next item's
// in flight during the compute) and loads the group's x image straight into
// the A-operand registers (L2-resident, issued before the weights are staged).
// The wavefronts' partials meet in LDS at the end; with more than one split,
// each split stores its partial tile to `part` and the last split to arrive
// (per-tile counter in `cnt`) adds the splits in order 0, 1, ... and writes y,
// so the result does not depend on which split finishes last.
template <class F, int NT, int W>
__global__ __launch_bounds__(64 * W) void qh_mmq(const QgGroups gs, const unsigned char* __restrict__ img,
                                                 uint32_t row_bytes, int ngroups, int splits,
                                                 float* __restrict__ part, unsigned int* __restrict__ cnt) {
    constexpr int CH = F::CH, RS = F::RS;
    constexpr int NH = (32 * CH + 63) / 64;  // 16-byte loads per lane per group
    constexpr int TILE = 32 * RS + 16;
    static_assert(NT == 2 || NT == 4 || NT == 8 || NT == 16, "NT");
    static_assert(TILE >= NT * 32 * 4, "the wavefront partials reuse the staging tile");
    using XI = XImg<F::KIND, F::SUMS>;
    // Image chunks this kernel reads: Q6_K with <= 8 tokens needs only u = 0.
    constexpr int NC = (F::KIND == 2) ? (NT > 8 ? 16 : 8) : XI::CHUNKS;
    constexpr int GRIDB = F::GRID ? 2048 : 0;  // codebook (IQ3S: 512 x u32, IQ2XXS: 256 x u64)
    __shared__ __align__(16) unsigned char lds[W * TILE + GRIDB];
    __shared__ int last_split;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int R = lane & 31, hh = lane >> 5;
    unsigned char* wl = lds + w * TILE;
    unsigned char* gridl = lds + W * TILE;
    if constexpr (F::GRID != 0) {
        const uint32_t* src = F::GRID == 1 ? qh_g_iq3s : reinterpret_cast<const uint32_t*>(qh_g_iq2xxs);
        for (int i = threadIdx.x; i < 512; i += 64 * W) reinterpret_cast<uint32_t*>(gridl)[i] = src[i];
        __syncthreads();
    }
    // This workgroup's matrix (uniform), row tile and K split.  Every matrix's
    // workgroups start at a multiple of `splits`, so blockIdx / splits is a
    // launch-wide tile index (for the split counters and partials).
    int gi = 0;
#pragma unroll
    for (int k = 1; k < QG_MAXG; k++) gi += (int)blockIdx.x >= gs.bstart[k];
    const int out_dim = gs.rows[gi], n = gs.n[gi], ldy = gs.ldy[gi];
    float* __restrict__ y = gs.y[gi];
    const QhBuf wb = qh_buf(gs.w[gi], gs.wbytes[gi]);
    const QhBuf ib = qh_buf(img + (size_t)gs.slot[gi] * ngroups * XI::BYTES, (uint32_t)ngroups * XI::BYTES);
    const int lb = blockIdx.x - gs.bstart[gi];
    const int tile = lb / splits, sp = lb - tile * splits, gt = blockIdx.x / splits;
    const int g0 = (int)((int64_t)ngroups * sp / splits), g1 = (int)((int64_t)ngroups * (sp + 1) / splits);

    // Weight slices of this lane: row rr[h] of the tile, byte offset goff[h] from
    // the tile's first row, LDS offset soff[h] (lanes past 32 * CH: spare bytes).
    uint32_t goff[NH], soff[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) {
        const int q = 64 * h + lane, r = q / CH, c = q - CH * r;
        const bool ok = q < 32 * CH && tile * 32 + r < out_dim;
        goff[h] = ok ? (uint32_t)(tile * 32 + r) * row_bytes + (c == CH - 1 ? F::LAST : 16u * c) : 0x80000000u;
        soff[h] = q < 32 * CH ? (uint32_t)(r * RS + 16 * c) : (uint32_t)(32 * RS);
    }
    auto load_w = [&](int g, qh_u32x4* wo) {
        const uint32_t go = g < g1 ? (uint32_t)F::BYTES * (uint32_t)g : 0x80000000u;
#pragma unroll
        for (int h = 0; h < NH; h++) wo[h] = qh_ld128(wb, goff[h] + go);
    };
    // The group's image chunks (1 KB each, coalesced) and its exponents.
    // Lanes whose A row holds a token slot >= NT load nothing (out of range: zeros).
    const bool xrow = F::KIND == 2 ? ((R & 15) >> 1) < NT : (R >> 1) < NT;
    auto load_x = [&](int g, qh_u32x4* xo, qh_u32x4& eo) {
        const uint32_t base = (uint32_t)g * XI::BYTES;
        const uint32_t lb = xrow ? base + 16u * lane : 0x80000000u;
#pragma unroll
        for (int c = 0; c < NC; c++) xo[c] = qh_ld128(ib, lb + 1024u * c);
        eo = qh_ld128(ib, base + XI::EXP);
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

    auto compute = [&](const qh_u32x4& ex, const qh_u32x4* xa) {
        const typename F::H hd = F::hdr(wrow);
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
                const qh_i32x4 a = qh_as_i32x4(xa[K]);
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
        } else if constexpr (F::KIND == 0) {
            auto pair = [&](auto PC) {
                constexpr int P = decltype(PC)::value;
                qh_i32x4 b0, b1;
                F::template bpair<P>(wrow, hh, b0, b1);
                const qh_i32x4 a0 = qh_as_i32x4(xa[2 * P]);
                const qh_i32x4 a1 = qh_as_i32x4(xa[2 * P + 1]);
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
                    const qh_i32x4 a = qh_as_i32x4(xa[C]);
                    const qh_i32x16 d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 8; j++) acc[j] += __mul24(slo, d[j]) + __mul24(shi, d[j + 8]);
                }
                if constexpr (NT > 8) {
                    const qh_i32x4 a = qh_as_i32x4(xa[8 + C]);
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
            const qh_i32x4 as = qh_as_i32x4(xa[8]);
            dm = __builtin_amdgcn_mfma_i32_32x32x32_i8(as, F::bmin(wrow, hd, hh), dm, 0, 0, 0);
        }
        // finish: slot (q, r) = token 4q + 2hh + r, exponent byte t of the image
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int r = 0; r < 2; r++) {
                if (4 * q >= NT) continue;  // slot beyond the tokens for both lane halves
                const int t = 4 * q + 2 * hh + r;
                const int se = ((int)(ex[t >> 2] << (24 - 8 * (t & 3)))) >> 24;
                const float rs = se == 127 ? __builtin_nanf("") : ldexpf(1.0f, -se);
                int i0, i1;
                if constexpr (F::KIND != 2) {
                    i0 = acc[4 * q + 2 * r];
                    i1 = acc[4 * q + 2 * r + 1];
                } else {
                    // Q6_K: MFMA u = q/2 holds slot q in register 4 (q%2) + 2r + m
                    const int* ap = (q < 2) ? acc : acc2;
                    i0 = ap[4 * (q & 1) + 2 * r];
                    i1 = ap[4 * (q & 1) + 2 * r + 1];
                }
                const float P = fmaf((float)i1, 256.0f, (float)i0);
                if constexpr (F::SUMS) {
                    const float Pm = fmaf((float)dm[4 * q + 2 * r + 1], 256.0f, (float)dm[4 * q + 2 * r]);
                    tot[2 * q + r] += (hd.d * P - hd.dm * Pm * (float)(1 << F::SUMSH)) * rs;
                } else {
                    tot[2 * q + r] += hd.d * P * rs;
                }
            }
    };

    // This wavefront's groups g0 + w + W j, j < nw, taken from j = rot on
    // (rotating with the workgroup): workgroups that run together then read
    // different groups' x images instead of all hitting the same L2 lines.
    const int nw = g1 - g0 > w ? (g1 - g0 - w + W - 1) / W : 0;
    const int rot = nw ? (int)(blockIdx.x % (unsigned)nw) : 0;
    auto grp = [&](int k) { return k < nw ? g0 + w + W * (k + rot < nw ? k + rot : k + rot - nw) : g1; };
    qh_u32x4 wr[NH], xr[NC], er;
    load_w(grp(0), wr);
    for (int k = 0; k < nw; k++) {
        const int g = grp(k);
        load_x(g, xr, er);
        // Keep the x loads ahead of the stage's wait for the weights (left to
        // itself the compiler issues them after it, exposing their latency).
        __builtin_amdgcn_sched_barrier(0);
        stage(wr);
        load_w(grp(k + 1), wr);  // past the last group: all offsets out of range, no traffic
        compute(er, xr);
    }
    // Wavefront partials -> this wavefront's staging tile (its own LDS), then
    // the sum over wavefronts in order 0..W-1.
    float* red = reinterpret_cast<float*>(wl);
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int t = 4 * q + 2 * hh + r;
            if (t < NT) red[t * 32 + R] = tot[2 * q + r];
        }
    __syncthreads();
    float v[(NT * 32 + 64 * W - 1) / (64 * W)];
#pragma unroll
    for (int j = 0; j < (NT * 32 + 64 * W - 1) / (64 * W); j++) {
        const int i = threadIdx.x + 64 * W * j;
        float a = 0.f;
        if (i < NT * 32) {
#pragma unroll
            for (int k = 0; k < W; k++) a += reinterpret_cast<const float*>(lds + k * TILE)[i];
        }
        v[j] = a;
    }
    auto put = [&](int i, float a) {
        const int t = i >> 5, row = tile * 32 + (i & 31);
        if (t < n && row < out_dim) {
            float* yp = y + (size_t)t * ldy + row;
            *yp = gs.accum ? *yp + a : a;
        }
    };
    if (splits == 1) {
#pragma unroll
        for (int j = 0; j < (NT * 32 + 64 * W - 1) / (64 * W); j++) {
            const int i = threadIdx.x + 64 * W * j;
            if (i < NT * 32) put(i, v[j]);
        }
        return;
    }
    float* mine = part + (size_t)blockIdx.x * (NT * 32);
#pragma unroll
    for (int j = 0; j < (NT * 32 + 64 * W - 1) / (64 * W); j++) {
        const int i = threadIdx.x + 64 * W * j;
        if (i < NT * 32) __hip_atomic_store(mine + i, v[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Agent-scope stores and loads of the partials reach the device's point of
    // coherence without writing back or invalidating whole L2s (which a
    // release/acquire fence per workgroup would, at a cost measured in tens of
    // microseconds per launch).  Every thread's stores have completed (vmcnt 0)
    // before the barrier, and the counter is bumped only after it.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0)
        last_split = __hip_atomic_fetch_add(&cnt[gt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (unsigned)(splits - 1);
    __syncthreads();
    if (!last_split) return;
    const float* tp = part + (size_t)gt * splits * (NT * 32);
#pragma unroll
    for (int j = 0; j < (NT * 32 + 64 * W - 1) / (64 * W); j++) {
        const int i = threadIdx.x + 64 * W * j;
        if (i < NT * 32) {
            float a = 0.f;
            for (int k = 0; k < splits; k++)
                a += __hip_atomic_load(tp + k * (NT * 32) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            put(i, a);
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(&cnt[gt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
}

// Device addresses of the library's static scratch, per device (hipGetSymbolAddress once).
struct QgScratch { unsigned char* img; float* part; unsigned int* cnt; };
static const QgScratch* qh_mmq_scratch_ptrs() {
    static QgScratch ptrs[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    QgScratch& p = ptrs[dev];
    if (!p.img) {
        void *a = nullptr, *b = nullptr, *c = nullptr;
        if (hipGetSymbolAddress(&a, HIP_SYMBOL(qh_mmq_scratch)) != hipSuccess ||
            hipGetSymbolAddress(&b, HIP_SYMBOL(qh_mmq_part)) != hipSuccess ||
            hipGetSymbolAddress(&c, HIP_SYMBOL(qh_mmq_cnt)) != hipSuccess)
            return nullptr;
        p.part = static_cast<float*>(b);
        p.cnt = static_cast<unsigned int*>(c);
        p.img = static_cast<unsigned char*>(a);
    }
    return &p;
}

// QUARTZ_HIP_MMQ_WAVES=4|8|16 forces the wavefronts per workgroup (tuning).
static int qh_mmq_waves_env() {
    static const int v = [] {
        const char* e = getenv("QUARTZ_HIP_MMQ_WAVES");
        return e ? atoi(e) : 0;
    }();
    return v;
}

// QUARTZ_HIP_MMQ_SPLITS=k forces the K splits per row tile (tuning).
static int qh_mmq_splits_env() {
    static const int v = [] {
        const char* e = getenv("QUARTZ_HIP_MMQ_SPLITS");
        return e ? atoi(e) : 0;
    }();
    return v;
}

template <class F, int NT, int W>
static void launch_mmq(const QgGroups& gs, int wgs, int splits, const QgScratch& sc, uint32_t row_bytes, int ngroups,
                       hipStream_t st) {
    hipLaunchKernelGGL((qh_mmq<F, NT, W>), dim3((unsigned)wgs), dim3(64 * W), 0, st, gs, sc.img, row_bytes, ngroups,
                       splits, sc.part, sc.cnt);
}

template <class F, int NT>
static void launch_mmq_w(int waves, const QgGroups& gs, int wgs, int splits, const QgScratch& sc, uint32_t row_bytes,
                         int ngroups, hipStream_t st) {
    if (waves == 16) launch_mmq<F, NT, 16>(gs, wgs, splits, sc, row_bytes, ngroups, st);
    else if (waves == 8) launch_mmq<F, NT, 8>(gs, wgs, splits, sc, row_bytes, ngroups, st);
    else launch_mmq<F, NT, 4>(gs, wgs, splits, sc, row_bytes, ngroups, st);
}

template <class F>
static void launch_mmq_nt(int nt, int waves, const QgGroups& gs, int wgs, int splits, const QgScratch& sc,
                          uint32_t row_bytes, int ngroups, hipStream_t st) {
    if (nt <= 2) launch_mmq_w<F, 2>(waves, gs, wgs, splits, sc, row_bytes, ngroups, st);
    else if (nt <= 4) launch_mmq_w<F, 4>(waves, gs, wgs, splits, sc, row_bytes, ngroups, st);
    else if (nt <= 8) launch_mmq_w<F, 8>(waves, gs, wgs, splits, sc, row_bytes, ngroups, st);
    else launch_mmq_w<F, 16>(waves, gs, wgs, splits, sc, row_bytes, ngroups, st);
}

// Bytes of one x image slot (all groups of in_dim) for a type's kernel.
static size_t qg_slot_bytes(uint32_t type, int ngroups) {
    const size_t per = type == QT_Q6_K ? XImg<2, false>::BYTES
                       : (type == QT_IQ3_S || type == QT_IQ2_XXS) ? XImg<1, false>::BYTES
                                                                  : XImg<0, true>::BYTES;
    return per * (size_t)ngroups;
}

struct QgEntry {  // one matrix (or row chunk of one) and its <= 16 tokens
    const uint8_t* w;
    const float* x;
    const float* x2;  // SwiGLU up (x is the gate), or null
    float* y;
    int n, rows, ldy;
};

// One grouped launch pair: the prologue digitises every distinct token block
// into its image slot, then the main kernel covers every entry's row tiles.
static hipError_t qg_run(uint32_t type, const QgEntry* en, int cnt, int in_dim, uint32_t row_bytes,
                         const QgScratch& sc, hipStream_t st, int accum) {
    const int ngroups = in_dim / 256;
    const int waves = qh_mmq_waves_env() ? qh_mmq_waves_env() : QG_WAVES;
    QgXs xs = {};
    QgGroups gs = {};
    int nslots = 0, ntmax = 0, tiles = 0;
    for (int i = 0; i < cnt; i++) {
        int j = 0;
        while (j < nslots && !(xs.x[j] == en[i].x && xs.x2[j] == en[i].x2 && xs.n[j] == en[i].n)) j++;
        if (j == nslots) {
            xs.x[j] = en[i].x;
            xs.x2[j] = en[i].x2;
            xs.n[j] = en[i].n;
            nslots++;
        }
        gs.w[i] = en[i].w;
        gs.y[i] = en[i].y;
        gs.wbytes[i] = (uint32_t)(((uint64_t)en[i].rows * row_bytes + 3) & ~(uint64_t)3);
        gs.rows[i] = en[i].rows;
        gs.n[i] = en[i].n;
        gs.ldy[i] = en[i].ldy;
        gs.slot[i] = j;
        ntmax = en[i].n > ntmax ? en[i].n : ntmax;
        tiles += (en[i].rows + 31) / 32;
    }
    // K splits: enough workgroups to fill the chip (about QG_TARGET_WGS), at
    // least one group per wavefront, and partials within the scratch.
    int splits = qh_mmq_splits_env();
    if (splits <= 0) {
        splits = (QG_TARGET_WGS + tiles - 1) / tiles;
        const int cap = ngroups / waves > 1 ? ngroups / waves : 1;
        splits = splits < cap ? splits : cap;
    }
    splits = splits < ngroups ? splits : ngroups;
    if ((int64_t)tiles * splits > QG_PART_TILES) splits = QG_PART_TILES / tiles;
    if (splits < 1) splits = 1;
    int wgs = 0;
    for (int i = 0; i < QG_MAXG; i++) {
        gs.bstart[i] = i < cnt ? wgs : INT_MAX;
        if (i < cnt) wgs += (en[i].rows + 31) / 32 * splits;
    }
    gs.bstart[QG_MAXG] = INT_MAX;
    gs.accum = accum;

    const dim3 pg((unsigned)ngroups, (unsigned)nslots);
    if (type == QT_Q6_K)
        hipLaunchKernelGGL((qh_mmq_ximg<2, false, 4>), pg, dim3(256), 0, st, xs, sc.img, in_dim);
    else if (type == QT_IQ3_S || type == QT_IQ2_XXS)
        hipLaunchKernelGGL((qh_mmq_ximg<1, false, 5>), pg, dim3(256), 0, st, xs, sc.img, in_dim);
    else
        hipLaunchKernelGGL((qh_mmq_ximg<0, true, 5>), pg, dim3(256), 0, st, xs, sc.img, in_dim);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (type) {
        case QT_Q4_K: launch_mmq_nt<GQ4K>(ntmax, waves, gs, wgs, splits, sc, row_bytes, ngroups, st); break;
        case QT_Q5_K: launch_mmq_nt<GQ5K>(ntmax, waves, gs, wgs, splits, sc, row_bytes, ngroups, st); break;
        case QT_IQ3_S: launch_mmq_nt<GIQ3S>(ntmax, waves, gs, wgs, splits, sc, row_bytes, ngroups, st); break;
        case QT_IQ2_XXS: launch_mmq_nt<GIQ2XXS>(ntmax, waves, gs, wgs, splits, sc, row_bytes, ngroups, st); break;
        default: launch_mmq_nt<GQ6K>(ntmax, waves, gs, wgs, splits, sc, row_bytes, ngroups, st); break;
    }
    return hipGetLastError();
}

// Batched tokens on the matrix cores for `count` matrices of one type and
// in_dim: Y[i][t][:] = W[i] X[i][t][:] for t < n[i] (token-major, y token stride
// out_dims[i]); hipErrorNotSupported when the type/shape has no kernel here.
// Tokens go in chunks of up to 16 (one weight pass each); matrices whose
// weights pass 2 GB go in row chunks.  Per launch, qh_mmq_ximg writes the x
// images to the library's device scratch and qh_mmq reads them; the scratch is
// one array per device, so calls that overlap on one device (different
// streams) must be serialised by the caller.
hipError_t qh_launch_mmq_grouped(uint32_t type, int count, const uint8_t* const* W, const float* const* X,
                                 float* const* Y, const int* n, const int* out_dims, int in_dim, hipStream_t st,
                                 const float* const* X2, int accum, const float* nw) {
    if (in_dim % 256 || in_dim / 256 > QG_MAX_GROUPS || count < 1) return hipErrorNotSupported;
    // an RMS norm fuses only into the 2-4 token GEMV path (the batched kernel's
    // 15-bit x image measured less accurate with x * w digitised before the scale)
    if (nw && X2) return hipErrorNotSupported;
    if (!X2 && count <= 4) {
        // 2-4 tokens of one x shared by up to 4 matrices: the GEMV kernel carries
        // the tokens (no x-image prologue, the weights read once)
        bool same = n[0] >= 2 && n[0] <= 4;
        for (int i = 1; i < count; i++) same = same && X[i] == X[0] && n[i] == n[0];
        // 3-4 tokens: the four MFMAs per token and group make big matrices
        // compute-bound in the GEMV kernel (measured slower above ~16 MB)
        int64_t wbytes = 0;
        for (int i = 0; i < count; i++) wbytes += (int64_t)qh_type_size(type, (size_t)in_dim) * (out_dims[i] > 0 ? out_dims[i] : 0);
        if (same && (n[0] == 2 || wbytes <= ((int64_t)16 << 20))) {
            hipError_t e = qh_launch_mmv16_tokens(type, count, W, Y, out_dims, out_dims, X[0], in_dim, n[0], in_dim,
                                                  accum, st, nw);
            if (e != hipErrorNotSupported) return e;
        }
    }
    if (nw) return hipErrorNotSupported;  // the caller normalises first
    if (type != QT_Q4_K && type != QT_Q5_K && type != QT_Q6_K && type != QT_IQ3_S && type != QT_IQ2_XXS)
        return hipErrorNotSupported;
    const QgScratch* sc = qh_mmq_scratch_ptrs();
    if (!sc) return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    const int ngroups = in_dim / 256;
    int max_slots = (int)(QG_SCRATCH / qg_slot_bytes(type, ngroups));
    max_slots = max_slots < QG_MAXG ? max_slots : QG_MAXG;
    if (max_slots < 1) return hipErrorNotSupported;
    const int64_t max_rows = (((int64_t)1 << 31) - 4096) / row_bytes / 32 * 32;
    if (max_rows < 32) return hipErrorNotSupported;
    // Entries go matrix-major: a matrix's token chunks follow each other, so
    // its weights are read from HBM once and from the MALL (256 MB) for the
    // chunks after the first, instead of once per chunk pass over all matrices.
    QgEntry batch[QG_MAXG];
    int cnt = 0, slots = 0;
    const float* last_x = nullptr;
    for (int i = 0; i < count; i++) {
        if (out_dims[i] <= 0) continue;
        for (int t0 = 0; t0 < n[i]; t0 += 16) {
            const int nt = n[i] - t0 < 16 ? n[i] - t0 : 16;
            const float* xs = X[i] + (size_t)t0 * in_dim;
            const float* xs2 = X2 && X2[i] ? X2[i] + (size_t)t0 * in_dim : nullptr;
            for (int64_t r0 = 0; r0 < out_dims[i]; r0 += max_rows) {
                // a new slot unless the previous entry's x is the same
                const bool new_slot = !(cnt > 0 && xs == last_x && batch[cnt - 1].x2 == xs2 && batch[cnt - 1].n == nt);
                if (cnt == QG_MAXG || (new_slot && slots == max_slots)) {
                    hipError_t e = qg_run(type, batch, cnt, in_dim, row_bytes, *sc, st, accum);
                    if (e != hipSuccess) return e;
                    cnt = 0;
                    slots = 0;
                }
                if (new_slot) slots++;
                const int rows = (int)(out_dims[i] - r0 < max_rows ? out_dims[i] - r0 : max_rows);
                batch[cnt++] = QgEntry{W[i] + (size_t)r0 * row_bytes, xs, xs2, Y[i] + (size_t)t0 * out_dims[i] + r0,
                                       nt, rows, out_dims[i]};
                last_x = xs;
            }
        }
    }
    if (cnt) {
        hipError_t e = qg_run(type, batch, cnt, in_dim, row_bytes, *sc, st, accum);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t qh_launch_mmq(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim, int n,
                         hipStream_t st) {
    if (n < 2) return hipErrorNotSupported;
    return qh_launch_mmq_grouped(type, 1, &W, &x, &y, &n, &out_dim, in_dim, st, nullptr, 0, nullptr);
}
