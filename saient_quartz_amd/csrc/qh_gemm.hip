// qh_gemm.hip -- batched dequant-GEMM for n = 2..32 tokens per weight pass on the f16 matrix
// cores (v_mfma_f32_32x32x16_f16), Q4_K / Q5_K / Q6_K / IQ3_S / IQ2_XXS.
//
// Y[t][j] = sum_k W[j,k] X[t][k], X and Y token-major.  One pass over the weights
// serves every token: the weights are the B operand (32 weight rows = the 32
// MFMA columns), the tokens' x the A operand, so a lane's results all belong to
// one weight row.
//   * x as two f16 per element: per token and 256-element group, x' = x 2^s
//     (s = 14 - exponent of max|x|, so |x'| < 2^14) is split into hi = f16(x')
//     and lo = f16(x' - hi) (both rounded toward zero), 21-22 significant bits
//     per element whatever the group's other values (an outlier costs its
//     neighbours nothing).  A rows
//     2t and 2t + 1 hold token t's hi and lo parts.
//   * B = the integer weight times its integer scale as f16, exact (|B| <=
//     2048, or a short integer times a power of two): one K-block of 16 weights
//     shares one scale in every format (Q6_K's scale groups are 16 weights), so
//     the MFMA accumulates a whole superblock without per-scale epilogue work.
//     Bytes become f16 with v_perm into 0x64xx (1024 + byte) and one packed FMA
//     against (scale, -(1024 + offset) scale), exact as long as that constant
//     fits f16 (Q6_K uses an add and a multiply instead).
//   * Q4_K / Q5_K mins (dmin * m_sb * sum(x over sb)): one more f16 MFMA whose A
//     operand is each token's per-sub-block x sums (hi + lo, scaled by 2^(s-5))
//     and whose B operand is the 8 mins.
//   * Products and sums accumulate in f32; the superblock's f16 scale d (and
//     dmin) multiply the f32 results once per superblock.
// A launch first digitises each token block's x once (qg_ximage, into the
// library's image array); the GEMM's workgroups then stream the images of their
// K split group by group into an LDS pair shared by their W wavefronts (one
// 32-row tile each), while each wavefront's weight slices stream through its
// own LDS tile with QG_NBUF items in flight.
//
// Reference counterpart: dequant::gemm (src/dequant.rs:143-200) with
// q4k_row_batched / q6k_row_batched (:38-122); the reference has no GPU
// batched path.
#include <climits>
#include <mutex>

#include "qh_formats.h"
#include "qh_internal.h"

typedef float qh_f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 qh_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 qh_f16x2 __attribute__((ext_vector_type(2)));

#ifndef QG_WAVES
#define QG_WAVES 8          // wavefronts (32-row tiles) per workgroup
#endif
#define QG_TARGET_WGS 256   // workgroups a launch aims for (one per CU)
#define QG_PART_TILES 8192  // row blocks with split-K counters (one per wavefront)
#define QG_NBUF 2           // items of weights in flight per wavefront (register sets)
#ifndef QG_GMAX
#define QG_GMAX 5           // groups per K split (their x images stay in LDS)
#endif
#define QG_GMAX2 3          // the same for 32-token launches (two image halves per group)
#define QG_DIG_BLOCKS 128   // row blocks per token block up to which a launch digitises x in the kernel
#define QG_MAX_GROUPS 256   // in_dim <= 65536 on the matrix-core path

// ---------------------------------------------------------------- f16 operands

QH_DEV uint32_t qg_h2u(qh_f16x2 v) { return __builtin_bit_cast(uint32_t, v); }
QH_DEV qh_f16x2 qg_u2h(uint32_t u) { return __builtin_bit_cast(qh_f16x2, u); }
// bytes (b0, b1) or (b2, b3) of w as the f16 pair (1024 + b, 1024 + b')
#define QG_SEL01 0x04010400u
#define QG_SEL23 0x04030402u
QH_DEV qh_f16x2 qg_b2h(uint32_t w, uint32_t sel) { return qg_u2h(__builtin_amdgcn_perm(0x64646464u, w, sel)); }
// (f, f) for an integer |f| <= 1024 given as a byte-biased value: the f16 pair
// of byte k of w, minus bias
QH_DEV qh_f16x2 qg_dup(uint32_t w, int k, _Float16 bias) {
    const uint32_t sel = (uint32_t)k | 0x0400u | ((uint32_t)k << 16) | 0x04000000u;
    return qg_u2h(__builtin_amdgcn_perm(0x64646464u, w, sel)) - qh_f16x2{bias, bias};
}
// 8 unsigned bytes (w0, w1) -> B operand sc * (byte - off): fma(1024 + b, sc,
// c) with c = -(1024 + off) sc, exact when |c| <= 65504 and |sc (b - off)| is
// an f16 integer.
QH_DEV qh_f16x8 qg_cvt8(uint32_t w0, uint32_t w1, qh_f16x2 scv, qh_f16x2 cv) {
    qh_f16x8 o;
    const qh_f16x2 a = __builtin_elementwise_fma(qg_b2h(w0, QG_SEL01), scv, cv);
    const qh_f16x2 b = __builtin_elementwise_fma(qg_b2h(w0, QG_SEL23), scv, cv);
    const qh_f16x2 c = __builtin_elementwise_fma(qg_b2h(w1, QG_SEL01), scv, cv);
    const qh_f16x2 d = __builtin_elementwise_fma(qg_b2h(w1, QG_SEL23), scv, cv);
    o[0] = a[0]; o[1] = a[1]; o[2] = b[0]; o[3] = b[1];
    o[4] = c[0]; o[5] = c[1]; o[6] = d[0]; o[7] = d[1];
    return o;
}

// ---------------------------------------------------------------- formats
// Each format gives BYTES, CH (16-byte slices staged per row and superblock,
// the last from byte LAST), RS (LDS line per row), the header decoded once per
// group (hdr: d, dmin, scales) and bop<J>: lane half hh's B operand of K-block
// J (weights 16 J + 8 hh .. + 7 of the lane's row) from the staged line r.

// Q4_K (src/dequant.rs:1471-1519): sub-block sb = 2p + nibble uses qs[32p + l].
struct GQ4K {
    static constexpr int BYTES = 144, CH = 9, RS = 144, LAST = 128;
    static constexpr bool SUMS = true;
    static constexpr int GRID = 0;
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
    template <int J>
    static QH_DEV qh_f16x8 bop(const unsigned char* r, int hh, const H& h, const unsigned char*) {
        constexpr int sb = J >> 1, jj = J & 1, p = sb >> 1, nib = sb & 1;
        const qh_u32x2 w = *reinterpret_cast<const qh_u32x2*>(r + 16 + 32 * p + 16 * jj + 8 * hh);
        const uint32_t q0 = nib ? (w.x >> 4) & 0x0F0F0F0Fu : w.x & 0x0F0F0F0Fu;
        const uint32_t q1 = nib ? (w.y >> 4) & 0x0F0F0F0Fu : w.y & 0x0F0F0F0Fu;
        const qh_f16x2 scv = qg_dup(sb < 4 ? h.sc0 : h.sc1, sb & 3, (_Float16)1024.0f);
        return qg_cvt8(q0, q1, scv, scv * (_Float16)-1024.0f);
    }
    // B operand of the mins MFMA for lane half hh: mins 4 hh .. 4 hh + 3, each
    // twice (for the hi and lo parts of the x sums)
    static QH_DEV qh_f16x8 minh(const H& h, int hh) {
        const uint32_t m = hh ? h.mn1 : h.mn0;
        const qh_f16x2 a = qg_dup(m, 0, (_Float16)1024.0f), b = qg_dup(m, 1, (_Float16)1024.0f);
        const qh_f16x2 c = qg_dup(m, 2, (_Float16)1024.0f), d = qg_dup(m, 3, (_Float16)1024.0f);
        return qh_f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    }
};

// Q5_K (src/dequant.rs:1146-1182): as Q4_K plus bit sb of qh[l] as bit 4.
struct GQ5K {
    static constexpr int BYTES = 176, CH = 11, RS = 176, LAST = 160;
    static constexpr bool SUMS = true;
    static constexpr int GRID = 0;
    using H = GQ4K::H;
    static QH_DEV H hdr(const unsigned char* r) { return GQ4K::hdr(r); }
    template <int J>
    static QH_DEV qh_f16x8 bop(const unsigned char* r, int hh, const H& h, const unsigned char*) {
        constexpr int sb = J >> 1, jj = J & 1, p = sb >> 1, nib = sb & 1;
        const qh_u32x2 w = *reinterpret_cast<const qh_u32x2*>(r + 48 + 32 * p + 16 * jj + 8 * hh);
        const qh_u32x2 u = *reinterpret_cast<const qh_u32x2*>(r + 16 + 16 * jj + 8 * hh);
        const uint32_t q0 = (nib ? (w.x >> 4) & 0x0F0F0F0Fu : w.x & 0x0F0F0F0Fu) | (((u.x >> sb) & 0x01010101u) << 4);
        const uint32_t q1 = (nib ? (w.y >> 4) & 0x0F0F0F0Fu : w.y & 0x0F0F0F0Fu) | (((u.y >> sb) & 0x01010101u) << 4);
        const qh_f16x2 scv = qg_dup(sb < 4 ? h.sc0 : h.sc1, sb & 3, (_Float16)1024.0f);
        return qg_cvt8(q0, q1, scv, scv * (_Float16)-1024.0f);
    }
    static QH_DEV qh_f16x8 minh(const H& h, int hh) { return GQ4K::minh(h, hh); }
};

// Q6_K (src/dequant.rs:1583-1631): weight 128 h + 32 k + l (h < 2, k < 4, l <
// 32) is ql[64 h + 32 (k & 1) + l] nibble k >> 1 with bits 2k, 2k+1 of qh[32 h
// + l] on top, minus 32, times sc[(128 h + 32 k + l) / 16].  K-block J = 8 h + 2 k
// + l / 16.  The line is staged with its last slice from byte 194, so d sits at
// 222 in LDS.
struct GQ6K {
    static constexpr int BYTES = 210, CH = 14, RS = 240, LAST = 194;
    static constexpr bool SUMS = false;
    static constexpr int GRID = 0;
    struct H { qh_u32x4 s; float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) {
        H o;
        o.s = *reinterpret_cast<const qh_u32x4*>(r + 192);
        o.d = qh_h2f(*reinterpret_cast<const uint16_t*>(r + 222));
        o.dm = 0.f;
        return o;
    }
    template <int J>
    static QH_DEV qh_f16x8 bop(const unsigned char* r, int hh, const H& h, const unsigned char*) {
        constexpr int hf = J >> 3, k = (J >> 1) & 3, l0 = 16 * (J & 1);
        const qh_u32x2 ql = *reinterpret_cast<const qh_u32x2*>(r + 64 * hf + 32 * (k & 1) + l0 + 8 * hh);
        const qh_u32x2 qh = *reinterpret_cast<const qh_u32x2*>(r + 128 + 32 * hf + l0 + 8 * hh);
        const uint32_t q0 = ((ql.x >> (4 * (k >> 1))) & 0x0F0F0F0Fu) | (((qh.x >> (2 * k)) & 0x03030303u) << 4);
        const uint32_t q1 = ((ql.y >> (4 * (k >> 1))) & 0x0F0F0F0Fu) | (((qh.y >> (2 * k)) & 0x03030303u) << 4);
        // the signed scale as an f16 pair: byte ^ 0x80 is sc + 128
        const qh_f16x2 scv = qg_dup(h.s[J >> 2] ^ 0x80808080u, J & 3, (_Float16)1152.0f);
        const qh_f16x2 m32 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
        const qh_f16x2 a = (qg_b2h(q0, QG_SEL01) + m32) * scv, b = (qg_b2h(q0, QG_SEL23) + m32) * scv;
        const qh_f16x2 c = (qg_b2h(q1, QG_SEL01) + m32) * scv, d = (qg_b2h(q1, QG_SEL23) + m32) * scv;
        return qh_f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    }
};

// IQ3_S (src/dequant.rs:1184-1237) and IQ2_XXS (:1011-1041): K-block J is half
// J & 1 of sub-block J >> 1; the lane's 8 weights are two codebook entries
// (IQ3_S) or one (IQ2_XXS) with their 8 sign bits, times the sub-block's odd
// scale.  Two tables in LDS, built once per workgroup (qg_iq_tables), make
// this a few lookups: the codebook as f16 (entry e at 8 e bytes for IQ3_S's 4
// values, 16 e for IQ2_XXS's 8), and for each sign byte the four f16-pair sign
// masks of its 8 weights (16 bytes each, at IQT_SIGN).
extern __device__ uint32_t qh_g_iq3s[512];
extern __device__ uint64_t qh_g_iq2xxs[256];
#define IQT_SIGN 4096  // sign masks after the 4 KB f16 codebook
#define IQT_BYTES 8192

struct GIQ3S {
    static constexpr int BYTES = 110, CH = 7, RS = 112, LAST = 94;
    static constexpr bool SUMS = false;
    static constexpr int GRID = 1;
    struct H { float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) { return H{qh_h2f(qh_rd16(r, 0)), 0.f}; }
    template <int J>
    static QH_DEV qh_f16x8 bop(const unsigned char* r, int hh, const H&, const unsigned char* tab) {
        constexpr int K = J >> 1, jj = J & 1;
        const uint32_t q = qh_rd16(r, 2 + 8 * K + 4 * jj + 2 * hh);                   // 2 grid indices
        const uint32_t qh = (uint32_t)r[66 + K] >> (4 * jj + 2 * hh);                  // their 9th bits
        const uint32_t sg = (uint32_t)r[qh_iq3s_at(74 + 4 * K + 2 * jj + hh)];         // 8 sign bits
        const qh_u32x2 g0 = *reinterpret_cast<const qh_u32x2*>(tab + 8 * ((q & 0xFFu) | ((qh & 1u) << 8)));
        const qh_u32x2 g1 = *reinterpret_cast<const qh_u32x2*>(tab + 8 * (((q >> 8) & 0xFFu) | ((qh & 2u) << 7)));
        const qh_u32x4 m = *reinterpret_cast<const qh_u32x4*>(tab + IQT_SIGN + 16 * sg);
        const int sc = 1 + 2 * (int)((r[qh_iq3s_at(106 + K / 2)] >> (4 * (K & 1))) & 0xFu);
        const qh_f16x2 scv = {(_Float16)sc, (_Float16)sc};
        const qh_f16x2 a = qg_u2h(g0.x ^ m.x) * scv, b = qg_u2h(g0.y ^ m.y) * scv;
        const qh_f16x2 c = qg_u2h(g1.x ^ m.z) * scv, d = qg_u2h(g1.y ^ m.w) * scv;
        return qh_f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    }
};

struct GIQ2XXS {
    static constexpr int BYTES = 66, CH = 5, RS = 80, LAST = 50;
    static constexpr bool SUMS = false;
    static constexpr int GRID = 2;
    struct H { float d, dm; };
    static QH_DEV H hdr(const unsigned char* r) { return H{0.125f * qh_h2f(qh_rd16(r, 0)), 0.f}; }
    template <int J>
    static QH_DEV qh_f16x8 bop(const unsigned char* r, int hh, const H&, const unsigned char* tab) {
        constexpr int K = J >> 1, jj = J & 1;
        const uint32_t idx = r[2 + 8 * K + 2 * jj + hh];
        const uint32_t a1 = qh_rd16(r, qh_iq2xxs_at(6 + 8 * K)) | (qh_rd16(r, qh_iq2xxs_at(8 + 8 * K)) << 16);
        const qh_u32x4 g = *reinterpret_cast<const qh_u32x4*>(tab + 16 * idx);
        const uint32_t s8 = qh_ksigns((a1 >> (7 * (2 * jj + hh))) & 127u);
        const qh_u32x4 m = *reinterpret_cast<const qh_u32x4*>(tab + IQT_SIGN + 16 * s8);
        const int sc = 2 * (int)(a1 >> 28) + 1;
        const qh_f16x2 scv = {(_Float16)sc, (_Float16)sc};
        const qh_f16x2 a = qg_u2h(g.x ^ m.x) * scv, b = qg_u2h(g.y ^ m.y) * scv;
        const qh_f16x2 c = qg_u2h(g.z ^ m.z) * scv, d = qg_u2h(g.w ^ m.w) * scv;
        return qh_f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    }
};

// Build the IQ tables of format GRID (1: IQ3_S, 2: IQ2_XXS) in LDS at tab:
// thread i < 512 converts codebook bytes to f16, i < 256 writes sign byte i's
// masks (bit k of the byte -> the sign bit of f16 k, pairs per dword).
template <int GRIDT>
QH_DEV void qg_iq_tables(unsigned char* tab, int tid, int nthreads) {
    for (int i = tid; i < 512; i += nthreads) {
        if constexpr (GRIDT == 1) {
            const uint32_t e = qh_g_iq3s[i];
            const qh_u32x2 v = {__builtin_amdgcn_perm(0x64646464u, e, QG_SEL01), __builtin_amdgcn_perm(0x64646464u, e, QG_SEL23)};
            const qh_f16x2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
            *reinterpret_cast<qh_u32x2*>(tab + 8 * i) =
                qh_u32x2{qg_h2u(qg_u2h(v.x) - k1024), qg_h2u(qg_u2h(v.y) - k1024)};
        } else if (i < 256) {
            const uint64_t e = qh_g_iq2xxs[i];
            const uint32_t lo = (uint32_t)e, hi = (uint32_t)(e >> 32);
            const qh_f16x2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
            *reinterpret_cast<qh_u32x4*>(tab + 16 * i) =
                qh_u32x4{qg_h2u(qg_b2h(lo, QG_SEL01) - k1024), qg_h2u(qg_b2h(lo, QG_SEL23) - k1024),
                         qg_h2u(qg_b2h(hi, QG_SEL01) - k1024), qg_h2u(qg_b2h(hi, QG_SEL23) - k1024)};
        }
        if (i < 256) {
            qh_u32x4 m;
#pragma unroll
            for (int k = 0; k < 4; k++)
                m[k] = (((uint32_t)i >> (2 * k)) & 1u) << 15 | (((uint32_t)i >> (2 * k + 1)) & 1u) << 31;
            *reinterpret_cast<qh_u32x4*>(tab + IQT_SIGN + 16 * i) = m;
        }
    }
}

// ---------------------------------------------------------------- x image in LDS

// The x operand of one 256-element group for 16 token slots, built in LDS by
// the workgroup that reads it.  A-operand order of v_mfma_f32_32x32x16_f16:
// lane L's 16 bytes are row L % 32, k = 8 (L / 32) .. + 7.
//   XA: K-block j (16 weights) at 1024 j: row 2t + part holds token t's hi
//     (part 0) or lo (part 1) f16 of elements 16 j + k.
//   SUM (Q4_K / Q5_K): token t's sum of x over sub-block sb, times 2^(s - 5),
//     as hi and lo f16, the A operand of the mins MFMA: row rho(t) = 8 (t >> 2)
//     + 4 ((t >> 1) & 1) + (t & 1) (so its results land where token t's main
//     results are), k = 8 (sb >> 2) + 2 (sb & 3) + part, stored at 16 (t + 16
//     (sb >> 2)) + 2 (2 (sb & 3) + part).
//   RSF: 2^-s of each token slot as f32 (NaN: x not finite), token t at float
//     8 ((t >> 1) & 1) + 2 (t >> 2) + (t & 1), so lane half hh reads its eight
//     tokens' factors (t = 4q + 2hh + r) as two 16-byte words.
struct XImg {
    static constexpr int SUM = 16384, RSF = 16896, BYTES = 16960;  // BYTES: a multiple of 16
};

#define QG_MAXG 16  // matrices (or row chunks) per grouped launch
struct QgXs {        // the distinct token blocks of one grouped launch
    const float* x[QG_MAXG];
    const float* x2[QG_MAXG];  // SwiGLU: x is silu(x) * x2 (gate, up) when non-null
    int n[QG_MAXG];  // tokens (<= 16 halves)
    const unsigned char* img;  // their x images: slot s, group g, half h at ((s ngroups + g) halves + h) XImg::BYTES
    uint32_t img_bytes;
    // Token ranges on the device (expert layers): when tok_off is set, slot s is
    // chunk c = s % moe_c of expert e = s / moe_c, tokens tok_off[e] + 16 c ..
    // min(+16, tok_off[e + 1]) of the gathered x[0] (and x2[0]); n[] is unused.
    const int* tok_off;
    int moe_c;
    // 16-token halves per token block (2: 32-token launches); a device-range
    // chunk then holds 32 tokens, and qg_ximage writes both halves' images
    // next to each other ((slot ngroups + g) halves + h)
    int halves;
};
// The tokens of slot s: x (and x2) of its first token, their count (<= 16 halves)
// and the index a of the first one in the gathered rows (0 for host slots).
struct QgTok {
    const float* x;
    const float* x2;
    int n, a;
};
// A workgroup-uniform value held in scalar registers (the compiler cannot
// prove uniformity through a dynamically indexed argument array or a loaded
// offset, and would wrap every buffer load built on it in a waterfall loop).
template <class T>
QH_DEV T* qg_uni(T* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return (T*)(((uint64_t)hi << 32) | lo);
}
QH_DEV int qg_uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
QH_DEV QgTok qg_tokens(const QgXs& xs, int slot, int in_dim) {
    if (!xs.tok_off) return QgTok{qg_uni(xs.x[slot]), qg_uni(xs.x2[slot]), qg_uni(xs.n[slot]), 0};
    const int e = slot / xs.moe_c, c = slot - e * xs.moe_c;
    const int ct = 16 * xs.halves;  // tokens per chunk
    const int a = qg_uni(xs.tok_off[e]) + ct * c;
    int n = qg_uni(xs.tok_off[e + 1]) - a;
    n = n < 0 ? 0 : (n > ct ? ct : n);
    const size_t off = (size_t)a * (size_t)in_dim;
    return QgTok{xs.x[0] + off, xs.x2[0] ? xs.x2[0] + off : nullptr, n, a};
}
struct QgGroups {    // the matrices of one grouped launch
    const uint8_t* w[QG_MAXG];
    float* y[QG_MAXG];
    uint32_t wbytes[QG_MAXG];  // buffer range of each matrix's weights
    int rows[QG_MAXG];
    int ldy[QG_MAXG];          // y token stride
    int slot[QG_MAXG];         // x block (QgXs entry)
    int bstart[QG_MAXG + 1];   // first workgroup of each matrix (launch-wide); entries from the count on
                               // hold the total
    // each matrix's tokens (what QgXs holds per slot), so a workgroup reads
    // them in the same round of argument loads as its matrix
    const float* x[QG_MAXG];
    const float* x2[QG_MAXG];
    int n[QG_MAXG];
    int accum;                 // y += result (the residual add) instead of y = result
};
// The tokens of matrix gi's token block `slot` (host blocks: the matrix's own
// fields; device ranges: slot = expert chunk, as qg_tokens).
QH_DEV QgTok qg_tokens(const QgGroups& gs, int gi, const QgXs& xs, int slot, int in_dim) {
    if (!xs.tok_off) return QgTok{qg_uni(gs.x[gi]), qg_uni(gs.x2[gi]), qg_uni(gs.n[gi]), 0};
    return qg_tokens(xs, slot, in_dim);
}
// Split-K partials (per (row block, split): W wavefronts x TPW tiles x NT
// tokens (16 or 32) x 32 rows)
// and per-(block, wavefront) arrival counters; every counter is back at zero
// when a launch ends.
#define QG_PART_FLOATS (16 * 1024 * 1024)
static __device__ __align__(256) float qh_mmq_part[QG_PART_FLOATS];
// x images of one launch's token blocks (qg_ximage)
#define QG_IMG_BYTES (40u << 20)
static __device__ __align__(256) unsigned char qh_mmq_img[QG_IMG_BYTES];
static __device__ __align__(256) unsigned int qh_mmq_cnt[QG_PART_TILES * QG_WAVES];

// ---------------------------------------------------------------- x images

// qg_ximage: the x operand of token block `slot` (blockIdx.y), 256-element
// group g (blockIdx.x), for the batched kernel, written once per launch to the
// library's image array and read by every row block.  Thread tid takes token t
// = tid / 32, elements 8 c .. 8 c + 7 (c = tid % 32) of the group, i.e.
// K-block c / 2, k half c % 2.  Per token and group, x' = x 2^s (s = 14 -
// exponent of max|x|) as hi = rtz(x') and lo = rtz(x' - hi); the layout is
// XImg's:
//   K-block j (16 weights) at 1024 j: row 2t + part holds token t's hi (part
//     0) or lo (part 1) f16 of elements 16 j + k (the A operand order of
//     v_mfma_f32_32x32x16_f16: lane L's 16 bytes are row L % 32, k = 8 (L / 32)
//     .. + 7);
//   SUM: token t's sum of x over sub-block sb, times 2^(s - 5), as hi and lo
//     f16 (the A operand of the Q4_K/Q5_K mins MFMA): row rho(t) = 8 (t >> 2) +
//     4 ((t >> 1) & 1) + (t & 1), k = 8 (sb >> 2) + 2 (sb & 3) + part, stored
//     at 16 (t + 16 (sb >> 2)) + 2 (2 (sb & 3) + part);
//   RSF: 2^-s of each token as f32 (NaN when the group holds an Inf or NaN,
//     which makes the token's results NaN).
// Tokens past the block's n write nothing (their rows are never read back
// into results).
// Digitise one 8-element chunk of the image: token t = xt, elements 8 xc ..
// 8 xc + 7 of the group (xc < 32), values v; the 32 lanes of a token form one
// half of a wavefront and must all take part (lanes with `on` false hold
// zeros and write nothing).  `im` is the group's image (global or LDS).
QH_DEV void qg_digitise(const float* v, bool on, int lane, int xt, int xc, unsigned char* im) {
    float m = 0.f, sum = 0.f;
    bool fin = true;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        m = fmaxf(m, fabsf(v[i]));
        sum += v[i];
        fin = fin && __builtin_isfinite(v[i]);
    }
    // max over the token's 32 lanes (a DPP row of 16, then the other row)
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x140, 0xF, 0xF, false)));
    m = fmaxf(m, __shfl_xor(m, 16));
    const uint64_t bad = __ballot(!fin);
    const bool fb = ((bad >> (lane & 32)) & 0xFFFFFFFFull) != 0;
    int e = 0;
    (void)frexpf(m, &e);
    int s = m > 0.f ? 14 - e : 0;
    s = s > 126 ? 126 : (s < -126 ? -126 : s);
    const float scx = ldexpf(1.0f, s);
    uint32_t hi4[4], lo4[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = v[2 * i] * scx, b = v[2 * i + 1] * scx;
        const auto hp = __builtin_amdgcn_cvt_pkrtz(a, b);
        const auto lp = __builtin_amdgcn_cvt_pkrtz(a - (float)hp[0], b - (float)hp[1]);
        hi4[i] = __builtin_bit_cast(uint32_t, hp);
        lo4[i] = __builtin_bit_cast(uint32_t, lp);
    }
    const int u = xc >> 1, c = xc & 1;
    // sub-block sb = xc / 4: the sum over 4 lanes (a DPP quad)
    sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0xB1, 0xF, 0xF, false));
    sum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sum), 0x4E, 0xF, 0xF, false));
    const float s5 = sum * ldexpf(1.0f, s - 5);
    const auto p5 = __builtin_amdgcn_cvt_pkrtz(s5, 0.f);
    const auto q5 = __builtin_amdgcn_cvt_pkrtz(s5 - (float)p5[0], 0.f);
    if (!on) return;
    *reinterpret_cast<qh_u32x4*>(im + 1024 * u + 16 * (2 * xt + 32 * c)) = qh_u32x4{hi4[0], hi4[1], hi4[2], hi4[3]};
    *reinterpret_cast<qh_u32x4*>(im + 1024 * u + 16 * (2 * xt + 1 + 32 * c)) = qh_u32x4{lo4[0], lo4[1], lo4[2], lo4[3]};
    const int sb = xc >> 2;
    if ((xc & 3) == 0) {
        const uint32_t pair = (uint32_t)__builtin_bit_cast(uint16_t, p5[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, q5[0]) << 16);
        *reinterpret_cast<uint32_t*>(im + XImg::SUM + 16 * (xt + 16 * (sb >> 2)) + 4 * (sb & 3)) = pair;
    }
    if (xc == 0)
        reinterpret_cast<float*>(im + XImg::RSF)[8 * ((xt >> 1) & 1) + 2 * (xt >> 2) + (xt & 1)] =
            fb ? __builtin_nanf("") : ldexpf(1.0f, -s);
}

// x (and the SwiGLU up operand x2) of one token chunk: 8 floats at p (and p2).
QH_DEV void qg_chunk(const qh_u32x4* xr, const qh_u32x4* ur, bool swiglu, float* v) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[i] = __uint_as_float(xr[0][i]);
        v[4 + i] = __uint_as_float(xr[1][i]);
    }
    if (swiglu) {
        // SwiGLU fused in: x = silu(gate) * up, qg_swiglu's expression
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = (v[i] / (1.f + expf(-v[i]))) * __uint_as_float(ur[0][i]);
            v[4 + i] = (v[4 + i] / (1.f + expf(-v[4 + i]))) * __uint_as_float(ur[1][i]);
        }
    }
}

__global__ __launch_bounds__(512) void qg_ximage(const QgXs xs, unsigned char* __restrict__ img, int in_dim) {
    // blockIdx.y = slot * halves + half h: tokens 16 h .. of the slot
    const int g = blockIdx.x, half = (int)blockIdx.y % xs.halves, slot = (int)blockIdx.y / xs.halves;
    const int ngroups = in_dim >> 8;
    const int lane = threadIdx.x & 63, xt = threadIdx.x >> 5, xc = threadIdx.x & 31;
    const QgTok tk = qg_tokens(xs, slot, in_dim);
    int n = tk.n - 16 * half;
    n = n > 16 ? 16 : n;
    if (xt >= n) return;  // whole half-wavefronts: the reductions stay within live lanes
    const size_t t0 = (size_t)(16 * half) * (size_t)in_dim;
    const uint32_t off = 4u * ((uint32_t)xt * (uint32_t)in_dim + 256u * (uint32_t)g + 8u * (uint32_t)xc);
    const QhBuf xb = qh_buf(tk.x + t0, 4u * (uint32_t)n * (uint32_t)in_dim);
    qh_u32x4 xr[2] = {qh_ld128(xb, off), qh_ld128(xb, off + 16u)}, ur[2] = {};
    if (tk.x2) {
        const QhBuf ub = qh_buf(tk.x2 + t0, 4u * (uint32_t)n * (uint32_t)in_dim);
        ur[0] = qh_ld128(ub, off);
        ur[1] = qh_ld128(ub, off + 16u);
    }
    float v[8];
    qg_chunk(xr, ur, tk.x2 != nullptr, v);
    qg_digitise(v, true, lane, xt, xc, img + (((size_t)slot * ngroups + g) * xs.halves + half) * XImg::BYTES);
}

// ---------------------------------------------------------------- kernel

QH_DEV qh_u32x4 qh_lds128(const unsigned char* p) { return *reinterpret_cast<const qh_u32x4*>(p); }

// One workgroup of W wavefronts per (row block of 32 W rows, K split).  Wavefront
// w owns one 32-row tile and streams its weights group by group through its own
// LDS tile (coalesced 16-byte loads, QG_NBUF groups in flight in register sets).
// The x images (qg_ximage's) go through a pair of LDS slots shared by the
// workgroup, one group ahead of the weights: while group i is computed, group
// i + 1's image (loaded one iteration earlier) is stored, and group i + 2's
// image loads go out with the weights.  One workgroup barrier per group orders
// the slot pair.
// A wavefront's results belong to its own rows, so no reduction over
// wavefronts is needed, and split-K partials are combined per wavefront (see
// the end).
template <class F, int NT, int W, int MODE>
constexpr int qh_mmq_lds() {
    return (MODE != 0 ? (NT > 16 ? QG_GMAX2 : QG_GMAX) : 2) * (NT > 16 ? 2 : 1) * XImg::BYTES + W * (32 * F::RS + 16) +
           (F::GRID ? IQT_BYTES : 0);
}

// The kernel body for workgroup lb of matrix gi (a launch may run two formats'
// bodies side by side, see qh_mmq_mix); lds holds qh_mmq_lds<...>() bytes.
// Launches are two-dimensional (blockIdx.y = matrix, blockIdx.x = its
// workgroup), so every per-matrix argument is read in the first round of
// argument loads; workgroups past a matrix's count exit at once.
template <class F, int NT, int W, int MODE>
__device__ __forceinline__ void qh_mmq_body(const QgGroups& gs, const QgXs& xs, uint32_t row_bytes, int in_dim,
                                            int splits, float* __restrict__ part, unsigned int* __restrict__ cnt,
                                            unsigned char* lds, const int gi, int lb) {
    constexpr int CH = F::CH, RS = F::RS;
    constexpr int NH = (32 * CH + 63) / 64;  // 16-byte weight loads per lane per group
    constexpr int TILE = 32 * RS + 16;
    static_assert(NT == 4 || NT == 8 || NT == 16 || NT == 32, "NT");
    using XI = XImg;
    // 32 tokens: two 16-token halves, each its own image and MFMA accumulator
    // against the same converted weights (streamed images, or digitised in the
    // kernel)
    constexpr int NTH = NT > 16 ? 2 : 1;
    static_assert(NTH == 1 || MODE != 1, "32-token launches: streamed or digitised images");
    constexpr int NQ = (NT > 16 ? 16 : NT) / 4;  // slot quads per half (tokens 16h + 4q .. + 3)
    constexpr int TPW = 1;                     // 32-row tiles per wavefront
    constexpr int GRIDB = F::GRID ? IQT_BYTES : 0;  // IQ codebook and sign tables
    constexpr int IMB = NTH * XI::BYTES;  // a group's images (both halves, adjacent)
    constexpr bool RES = MODE != 0;
    constexpr int NSLOT = RES ? (NTH == 2 ? QG_GMAX2 : QG_GMAX) : 2;  // image slots in LDS
    static_assert(qh_mmq_lds<F, NT, W, MODE>() == NSLOT * IMB + W * TILE + GRIDB, "LDS layout");
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int R = lane & 31, hh = lane >> 5;
    unsigned char* wl = lds + NSLOT * IMB + w * TILE;
    unsigned char* gridl = lds + NSLOT * IMB + W * TILE;
    if constexpr (F::GRID != 0) qg_iq_tables<F::GRID>(gridl, threadIdx.x, 64 * W);
    // This workgroup's row block and K split.  Every matrix's workgroups start
    // at a multiple of `splits` in the launch-wide count bx, so bx / splits is
    // a launch-wide block index (for the split counters and partials).
    const int b0 = gs.bstart[gi];
    if (lb >= gs.bstart[gi + 1] - b0) return;  // past this matrix (uniform, before any barrier)
    const int bx = b0 + lb;
    const int out_dim = gs.rows[gi], ldy = gs.ldy[gi];
    const int ngroups = in_dim >> 8;
    int slot = gs.slot[gi];
    if (xs.tok_off) {
        // expert layers: entry gi is expert gs.slot[gi]; its workgroups cover
        // moe_c token chunks, each over all row blocks and splits
        const int per = (out_dim + 32 * W - 1) / (32 * W) * splits;
        const int c = lb / per;
        lb -= c * per;
        slot = slot * xs.moe_c + c;
    }
    const QgTok tk = qg_tokens(gs, gi, xs, slot, in_dim);
    const int n = tk.n;
    if (n <= 0) return;  // an empty token chunk (uniform over the workgroup, before any barrier)
    float* __restrict__ y = gs.y[gi] + (size_t)tk.a * (size_t)ldy;
    const QhBuf wb = qh_buf(gs.w[gi], gs.wbytes[gi]);
    const int blk = lb / splits, sp = lb - blk * splits, gblk = bx / splits;
    const int tile0 = blk * W + w;  // this wavefront's tile
    const int g0 = ngroups * sp / splits, g1 = ngroups * (sp + 1) / splits;  // ngroups <= 256
    const int nk = g1 - g0;
    // Row blocks walk their split's groups from different starting points, so
    // concurrent workgroups read different parts of x (spreading the L2 load).
    const int rot = nk > 0 ? blk % nk : 0;
    auto grp = [&](int i) { const int j = i + rot; return g0 + (j >= nk ? j - nk : j); };

    // Weight slices of this lane: row q / CH of the tile, slice q % CH, byte
    // offset goff[h], LDS offset soff[h] (lanes past 32 * CH: the spare 16
    // bytes at the tile's end); bit h of okb: the slice's row exists.
    uint32_t goff[NH], soff[NH], okb = 0;
#pragma unroll
    for (int h = 0; h < NH; h++) {
        const int q = 64 * h + lane, r = q / CH, c = q - CH * r;
        okb |= (q < 32 * CH && tile0 * 32 + r < out_dim) ? 1u << h : 0u;
        goff[h] = (uint32_t)(tile0 * 32 + r) * row_bytes + (c == CH - 1 ? F::LAST : 16u * c);
        soff[h] = q < 32 * CH ? (uint32_t)(r * RS + 16 * c) : (uint32_t)(32 * RS);
    }
    // Past the split (i >= nk) the offsets get bit 31 (out of the buffer's
    // range: no traffic, zeros) by arithmetic, not a branch: a branch here
    // leaves the compiler's load counting at the joins conservative, and its
    // waits for one register set then also wait for the other set's loads.
    auto load_w = [&](int i, qh_u32x4* wo) {  // item i: group grp(i)
        const uint32_t go = (uint32_t)F::BYTES * (uint32_t)grp(i) | ((uint32_t)(nk - 1 - i) & 0x80000000u);
#pragma unroll
        for (int h = 0; h < NH; h++) wo[h] = qh_ld128(wb, ((okb >> h) & 1u) ? goff[h] + go : 0x80000000u);
    };
    auto stage_w = [&](const qh_u32x4* wr) {
#pragma unroll
        for (int h = 0; h < NH; h++) *reinterpret_cast<qh_u32x4*>(wl + soff[h]) = wr[h];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // ---- x images (built by qg_ximage), 16-byte chunk id = tid + 64 W p
    // (pass p < XP) of a group's image per thread.
    //   MODE 1: the split's nk <= QG_GMAX images are copied to LDS once (item
    //     i's at slot i): all their loads go out first, then the first weight
    //     items, and only the image loads are waited for.  The item loop then
    //     runs without workgroup barriers.
    //   MODE 2: as MODE 1, but the workgroup digitises the split's x (and
    //     SwiGLU operand) itself: no qg_ximage launch; thread tid < 32 NT
    //     takes token tid / 32, elements 8 (tid % 32) .. + 7 of each group
    //     (32 tokens: tokens tid / 32 and 16 + tid / 32, one per half).
    //   MODE 0: one group at a time through a slot pair, loaded with the
    //     weights one iteration ahead; one workgroup barrier per group orders
    //     the pair.
    constexpr int NCH = IMB / 16;
    constexpr int XP = (NCH + 64 * W - 1) / (64 * W);
    const QhBuf xb = qh_buf(xs.img, xs.img_bytes);
    const uint32_t ibase = (uint32_t)slot * (uint32_t)ngroups * (uint32_t)IMB + 16u * threadIdx.x;
    auto load_x = [&](int i, qh_u32x4* xr) {  // item i: group grp(i)
#pragma unroll
        for (int p = 0; p < XP; p++) {
            const int id = threadIdx.x + 64 * W * p;
            xr[p] = qh_ld128(xb, (id < NCH && i < nk) ? ibase + (uint32_t)IMB * (uint32_t)grp(i) + 1024u * W * p
                                                       : 0x80000000u);
        }
    };
    auto store_x = [&](unsigned char* im, const qh_u32x4* xr) {
#pragma unroll
        for (int p = 0; p < XP; p++) {
            const int id = threadIdx.x + 64 * W * p;
            if (id < NCH) *reinterpret_cast<qh_u32x4*>(im + 16 * id) = xr[p];
        }
    };
    qh_u32x4 wr[QG_NBUF][NH];
    qh_u32x4 xq[RES ? 1 : XP];  // streamed: the next group's image
    if constexpr (MODE == 2) {
        constexpr int TH = NT > 16 ? 16 : NT;  // tokens per half
        static_assert(32 * TH <= 64 * W, "one chunk per thread and half");
        const int xt = threadIdx.x >> 5, xc = threadIdx.x & 31;
        const QhBuf fb = qh_buf(tk.x, 4u * (uint32_t)n * (uint32_t)in_dim);
        const QhBuf ub = qh_buf(tk.x2, 4u * (uint32_t)n * (uint32_t)in_dim);
        const bool swiglu = tk.x2 != nullptr;
        const uint32_t xo = 4u * ((uint32_t)xt * (uint32_t)in_dim + 8u * (uint32_t)xc);
        bool xon[NTH];
#pragma unroll
        for (int p = 0; p < NTH; p++) xon[p] = (int)threadIdx.x < 32 * TH && xt + 16 * p < n;
        qh_u32x4 xd[NSLOT][NTH][2], ud[NSLOT][NTH][2];
#pragma unroll
        for (int k = 0; k < NSLOT; k++)
#pragma unroll
            for (int p = 0; p < NTH; p++) {
                const uint32_t off = (xon[p] && k < nk)
                                         ? xo + 64u * (uint32_t)p * (uint32_t)in_dim + 1024u * (uint32_t)grp(k)
                                         : 0x80000000u;
                xd[k][p][0] = qh_ld128(fb, off);
                xd[k][p][1] = qh_ld128(fb, off + 16u);
                const uint32_t uoff = swiglu ? off : 0x80000000u;
                ud[k][p][0] = qh_ld128(ub, uoff);
                ud[k][p][1] = qh_ld128(ub, uoff + 16u);
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < QG_NBUF; b++) load_w(b, wr[b]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < NSLOT; k++)
            if (k < nk) {
#pragma unroll
                for (int p = 0; p < NTH; p++) {
                    float v[8];
                    qg_chunk(xd[k][p], ud[k][p], swiglu, v);
                    qg_digitise(v, xon[p], lane, xt, xc, lds + k * IMB + p * XI::BYTES);
                }
            }
    } else if constexpr (RES) {
        qh_u32x4 xr[NSLOT][XP];
#pragma unroll
        for (int k = 0; k < NSLOT; k++) load_x(k < nk ? k : nk, xr[k]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < QG_NBUF; b++) load_w(b, wr[b]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < NSLOT; k++)
            if (k < nk) store_x(lds + k * IMB, xr[k]);
    } else {
        // group 0's image, the first QG_NBUF groups' weights, group 0's image
        // to LDS (waiting only for its loads), then group 1's image loads
        load_x(0, xq);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < QG_NBUF; b++) load_w(b, wr[b]);
        __builtin_amdgcn_sched_barrier(0);
        store_x(lds, xq);
        load_x(1, xq);
    }
    __syncthreads();  // images (and the codebook) visible to every wavefront

    // Result slots of this lane: slot (q, r) of tile tt is token t = 4q + 2hh + r
    // of the tile's row R.
    // Result slot h 2NQ + 2q + r of tile tt is token 16h + 4q + 2hh + r.
    float tot[TPW][NTH * 2 * NQ];
#pragma unroll
    for (int tt = 0; tt < TPW; tt++)
#pragma unroll
        for (int i = 0; i < NTH * 2 * NQ; i++) tot[tt][i] = 0.f;
    const unsigned char* wrow = wl + R * RS;
    // compact index of this lane's row in the sums (rows rho(t))
    const int cidx = 4 * (R >> 3) + 2 * ((R >> 2) & 1) + (R & 1) + 16 * hh;

    auto compute = [&](const unsigned char* im, float* tot) {
        const typename F::H hd = F::hdr(wrow);
        qh_f32x16 c[NTH], dm[NTH];
#pragma unroll
        for (int h = 0; h < NTH; h++) {
            c[h] = qh_f32x16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            dm[h] = c[h];
        }
        auto kb = [&](auto JC) {
            constexpr int J = decltype(JC)::value;
            const qh_f16x8 b = F::template bop<J>(wrow, hh, hd, gridl);
#pragma unroll
            for (int h = 0; h < NTH; h++) {
                const qh_f16x8 a = __builtin_bit_cast(qh_f16x8, qh_lds128(im + h * XI::BYTES + 1024 * J + 16 * lane));
                c[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[h], 0, 0, 0);
            }
        };
        kb(std::integral_constant<int, 0>{});
        kb(std::integral_constant<int, 1>{});
        kb(std::integral_constant<int, 2>{});
        kb(std::integral_constant<int, 3>{});
        kb(std::integral_constant<int, 4>{});
        kb(std::integral_constant<int, 5>{});
        kb(std::integral_constant<int, 6>{});
        kb(std::integral_constant<int, 7>{});
        kb(std::integral_constant<int, 8>{});
        kb(std::integral_constant<int, 9>{});
        kb(std::integral_constant<int, 10>{});
        kb(std::integral_constant<int, 11>{});
        kb(std::integral_constant<int, 12>{});
        kb(std::integral_constant<int, 13>{});
        kb(std::integral_constant<int, 14>{});
        kb(std::integral_constant<int, 15>{});
        if constexpr (F::SUMS) {
            const qh_f16x8 mb = F::minh(hd, hh);
#pragma unroll
            for (int h = 0; h < NTH; h++) {
                const qh_f16x8 sv = __builtin_bit_cast(qh_f16x8, qh_lds128(im + h * XI::BYTES + XI::SUM + 16 * cidx));
                dm[h] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sv, mb, dm[h], 0, 0, 0);
            }
        }
        // finish: slot (q, r) = token 4q + 2hh + r of the half (rows 2t, 2t + 1:
        // registers 4q + 2r, 4q + 2r + 1), its 2^-s at float 8 hh + 2q + r of
        // the half's image
#pragma unroll
        for (int h = 0; h < NTH; h++) {
            const unsigned char* ih = im + h * XI::BYTES;
            const qh_u32x4 rs0 = qh_lds128(ih + XI::RSF + 32 * hh), rs1 = qh_lds128(ih + XI::RSF + 32 * hh + 16);
            const uint32_t rsw[8] = {rs0.x, rs0.y, rs0.z, rs0.w, rs1.x, rs1.y, rs1.z, rs1.w};
#pragma unroll
            for (int q = 0; q < NQ; q++)
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const float rs = __uint_as_float(rsw[2 * q + r]);
                    const float P = c[h][4 * q + 2 * r] + c[h][4 * q + 2 * r + 1];
                    if constexpr (F::SUMS)
                        tot[h * 2 * NQ + 2 * q + r] += (hd.d * P - hd.dm * 32.0f * dm[h][4 * q + r]) * rs;
                    else
                        tot[h * 2 * NQ + 2 * q + r] += hd.d * P * rs;
                }
        }
    };

    // Item i in register set i % QG_NBUF, refilled with item i + QG_NBUF as
    // soon as it is staged (past the split: out of range, no traffic).
    // Streamed images: image (i + 1) % 2 is stored from the loads of one
    // iteration ago (every wavefront finished reading that slot before the
    // last barrier) and group i + 2's image loads go out before the weights
    // (a wait for them then leaves the weight loads in flight).
    // The pair loop's body is straight-line and an odd last item runs after
    // it: with a conditional second item the compiler's load counting at the
    // loop header assumes the shorter path, and the first set's wait would
    // also wait for the second set's loads (memory and compute serialised).
    static_assert(QG_NBUF == 2, "item pairs");
    auto item = [&](int b, int i) {
        // keep each item's stage (and its load wait) after the previous item's
        // compute: hoisted, it would wait for the newest loads too
        __builtin_amdgcn_sched_barrier(0);
        stage_w(wr[b]);
        if constexpr (!RES) {
            if (i + 1 < nk) store_x(lds + ((i + 1) & 1) * IMB, xq);
            load_x(i + 2, xq);
        }
        load_w(i + QG_NBUF, wr[b]);
        __builtin_amdgcn_sched_barrier(0);  // the refill goes out before the compute
        compute(lds + (RES ? i : (i & 1)) * IMB, tot[0]);
        if constexpr (!RES) __syncthreads();
    };
    int i0 = 0;
    for (; i0 + 1 < nk; i0 += 2) {
        item(0, i0);
        item(1, i0 + 1);
    }
    if (i0 < nk) item(0, i0);
    // Results: this wavefront's 32 rows x NT tokens; slot i of a tile holds
    // token stok(i) (half i / 2NQ, quad (i % 2NQ) / 2, r = i % 2).
    constexpr int NSL = NTH * 2 * NQ;  // result slots per lane and tile
    auto stok = [&](int i) { return 16 * (i / (2 * NQ)) + 4 * ((i % (2 * NQ)) >> 1) + 2 * hh + (i & 1); };
    auto put = [&](int t, int row, float a) {
        if (t < n && row < out_dim) {
            float* yp = y + (size_t)t * ldy + row;
            *yp = gs.accum ? *yp + a : a;
        }
    };
    if (splits == 1) {
#pragma unroll
        for (int tt = 0; tt < TPW; tt++)
#pragma unroll
            for (int i = 0; i < NSL; i++) put(stok(i), (tile0 + tt) * 32 + R, tot[tt][i]);
        return;
    }
    // Split K: each wavefront stores its partial (NT tokens x 32 rows), and the
    // last of the splits' wavefronts for the same rows to arrive (counter per
    // (block, wavefront)) adds the splits in order 0, 1, ... and writes y, so
    // the result does not depend on which split finishes last.  Wavefronts do
    // this independently, without workgroup barriers.
    constexpr int PW = TPW * NT * 32;  // floats of one wavefront partial
    const size_t wslot = (size_t)gblk * W + w;
    float* mine = part + (wslot * splits + sp) * PW;
#pragma unroll
    for (int tt = 0; tt < TPW; tt++)
#pragma unroll
        for (int i = 0; i < NSL; i++)
            __hip_atomic_store(mine + (tt * NT + stok(i)) * 32 + R, tot[tt][i], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    // Agent-scope stores and loads of the partials reach the device's point of
    // coherence without writing back or invalidating whole L2s (which a
    // release/acquire fence would, at a cost measured in tens of microseconds
    // per launch).  This wavefront's stores have completed (vmcnt 0) before its
    // counter moves.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    unsigned old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(&cnt[wslot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
    if (old != (unsigned)(splits - 1)) return;
    // The partials are read with SC1 buffer loads (the coherence bit of an
    // agent-scope load, so no stale L2 line of an earlier launch is seen),
    // which unlike atomic loads issue back to back: every slot of 4 splits in
    // flight at once, summed in split order.
    const QhBuf pbuf = qh_buf(part, 4u * QG_PART_FLOATS);
    const uint32_t bbase = 4u * (uint32_t)(wslot * splits * PW);
    constexpr int NS = TPW * NSL;  // result slots per lane
    float a[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) a[i] = 0.f;
    // A residual launch's y values go out with the first round of partial loads
    // (one round trip for both, not one more at the end).
    float yv[NS];
#pragma unroll
    for (int tt = 0; tt < TPW; tt++)
#pragma unroll
        for (int i = 0; i < NSL; i++) {
            const int t = stok(i), row = (tile0 + tt) * 32 + R;
            yv[tt * NSL + i] = gs.accum && t < n && row < out_dim ? y[(size_t)t * ldy + row] : 0.f;
        }
    for (int k0 = 0; k0 < splits; k0 += 4) {
        uint32_t v[NS][4];
#pragma unroll
        for (int tt = 0; tt < TPW; tt++)
#pragma unroll
            for (int i = 0; i < NSL; i++)
#pragma unroll
                for (int uu = 0; uu < 4; uu++) {
                    const uint32_t off = k0 + uu < splits
                                             ? bbase + 4u * (uint32_t)((k0 + uu) * PW + (tt * NT + stok(i)) * 32 + R)
                                             : 0x80000000u;
                    v[tt * NSL + i][uu] = __builtin_amdgcn_raw_buffer_load_b32(pbuf.rs, (int)off, 0, 16);
                }
#pragma unroll
        for (int i = 0; i < NS; i++)
#pragma unroll
            for (int uu = 0; uu < 4; uu++)
                if (k0 + uu < splits) a[i] += __uint_as_float(v[i][uu]);
    }
#pragma unroll
    for (int tt = 0; tt < TPW; tt++)
#pragma unroll
        for (int i = 0; i < NSL; i++) {
            const int t = stok(i), row = (tile0 + tt) * 32 + R;
            if (t < n && row < out_dim) y[(size_t)t * ldy + row] = gs.accum ? yv[tt * NSL + i] + a[tt * NSL + i] : a[tt * NSL + i];
        }
    if (lane == 0) __hip_atomic_store(&cnt[wslot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
}

template <class F, int NT, int W, int MODE>
__global__ __launch_bounds__(64 * W) void qh_mmq(const QgGroups gs, const QgXs xs, uint32_t row_bytes, int in_dim,
                                                 int splits, float* __restrict__ part, unsigned int* __restrict__ cnt) {
    __shared__ __align__(16) unsigned char lds[qh_mmq_lds<F, NT, W, MODE>()];
    qh_mmq_body<F, NT, W, MODE>(gs, xs, row_bytes, in_dim, splits, part, cnt, lds, (int)blockIdx.y, (int)blockIdx.x);
}

// Two formats sharing x in one launch (a layer's q/k in Q4_K and v in Q6_K),
// both with resident images (MODE 2: digitised in the kernel; MODE 1: built by
// qg_norm_image before the launch): matrices (blockIdx.y)
// below c1 run F1's body on gs1, the others F2's on gs2, each with its own
// splits and its own region of the split-K partials and counters.
template <class F1, class F2, int NT, int W, int MODE>
__global__ __launch_bounds__(64 * W) void qh_mmq_mix(const QgGroups gs1, const QgGroups gs2, const QgXs xs,
                                                     uint32_t rb1, uint32_t rb2, int in_dim, int s1, int s2, int c1,
                                                     float* __restrict__ part, unsigned int* __restrict__ cnt,
                                                     float* __restrict__ part2, unsigned int* __restrict__ cnt2) {
    constexpr int L1 = qh_mmq_lds<F1, NT, W, MODE>(), L2 = qh_mmq_lds<F2, NT, W, MODE>();
    __shared__ __align__(16) unsigned char lds[L1 > L2 ? L1 : L2];
    if ((int)blockIdx.y < c1)
        qh_mmq_body<F1, NT, W, MODE>(gs1, xs, rb1, in_dim, s1, part, cnt, lds, (int)blockIdx.y, (int)blockIdx.x);
    else
        qh_mmq_body<F2, NT, W, MODE>(gs2, xs, rb2, in_dim, s2, part2, cnt2, lds, (int)blockIdx.y - c1,
                                     (int)blockIdx.x);
}

// Device addresses of the library's static scratch, per device (hipGetSymbolAddress once).
struct QgScratch { float* part; unsigned int* cnt; unsigned char* img; };
static const QgScratch* qh_mmq_scratch_ptrs() {
    // filled once per device (std::call_once: host threads may race here)
    static QgScratch ptrs[64] = {};
    static std::once_flag once[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::call_once(once[dev], [&] {
        void *b = nullptr, *c = nullptr, *im = nullptr;
        if (hipGetSymbolAddress(&b, HIP_SYMBOL(qh_mmq_part)) == hipSuccess &&
            hipGetSymbolAddress(&c, HIP_SYMBOL(qh_mmq_cnt)) == hipSuccess &&
            hipGetSymbolAddress(&im, HIP_SYMBOL(qh_mmq_img)) == hipSuccess)
            ptrs[dev] = QgScratch{static_cast<float*>(b), static_cast<unsigned int*>(c),
                                  static_cast<unsigned char*>(im)};
    });
    return ptrs[dev].part ? &ptrs[dev] : nullptr;
}

// QUARTZ_HIP_MMQ_MODE=m forces the image mode (0 streamed, 1 resident, 2
// resident and digitised in the kernel) where it applies (tuning).
static int qh_mmq_mode_env() {
    static const int v = [] {
        const int m = qh_env_int("QUARTZ_HIP_MMQ_MODE", -1);
        return m >= 0 && m <= 2 ? m : -1;
    }();
    return v;
}

// QUARTZ_HIP_MMQ_SPLITS=k forces the K splits per row block (tuning).
static int qh_mmq_splits_env() {
    static const int v = [] {
        const int k = qh_env_int("QUARTZ_HIP_MMQ_SPLITS", 0);
        return k > 0 ? k : 0;
    }();
    return v;
}

// Launch shape: QG_WAVES wavefronts (32-row tiles) per workgroup.
// grid: (the largest matrix's workgroups, matrices); bstart[cnt] = the total.
template <class F, int NT>
static void launch_mmq_t(int mode, const QgGroups& gs, const QgXs& xs, dim3 grid, int splits, const QgScratch& sc,
                         uint32_t row_bytes, int in_dim, hipStream_t st) {
    if (mode == 2)
        hipLaunchKernelGGL((qh_mmq<F, NT, QG_WAVES, 2>), grid, dim3(64 * QG_WAVES), 0, st, gs, xs, row_bytes, in_dim,
                           splits, sc.part, sc.cnt);
    else if (mode == 1)
        hipLaunchKernelGGL((qh_mmq<F, NT, QG_WAVES, 1>), grid, dim3(64 * QG_WAVES), 0, st, gs, xs, row_bytes, in_dim,
                           splits, sc.part, sc.cnt);
    else
        hipLaunchKernelGGL((qh_mmq<F, NT, QG_WAVES, 0>), grid, dim3(64 * QG_WAVES), 0, st, gs, xs, row_bytes, in_dim,
                           splits, sc.part, sc.cnt);
}

template <class F>
static void launch_mmq_nt(int nt, int mode, const QgGroups& gs, const QgXs& xs, dim3 grid, int splits,
                          const QgScratch& sc, uint32_t row_bytes, int in_dim, hipStream_t st) {
    if (nt <= 4) launch_mmq_t<F, 4>(mode, gs, xs, grid, splits, sc, row_bytes, in_dim, st);
    else if (nt <= 8) launch_mmq_t<F, 8>(mode, gs, xs, grid, splits, sc, row_bytes, in_dim, st);
    else if (nt <= 16) launch_mmq_t<F, 16>(mode, gs, xs, grid, splits, sc, row_bytes, in_dim, st);
    else if (mode == 2)  // 17-32 tokens: digitised in the kernel, or streamed
        hipLaunchKernelGGL((qh_mmq<F, 32, QG_WAVES, 2>), grid, dim3(64 * QG_WAVES), 0, st, gs, xs, row_bytes, in_dim,
                           splits, sc.part, sc.cnt);
    else
        hipLaunchKernelGGL((qh_mmq<F, 32, QG_WAVES, 0>), grid, dim3(64 * QG_WAVES), 0, st, gs, xs, row_bytes, in_dim,
                           splits, sc.part, sc.cnt);
}

struct QgEntry {  // one matrix (or row chunk of one) and its <= 32 tokens
    const uint8_t* w;
    const float* x;
    const float* x2;  // SwiGLU up (x is the gate), or null
    float* y;
    int n, rows, ldy;
};

// K splits per row block: the count s (at least ngroups / gmax) that
// minimises the rounds of `target` workgroups times (3 + the groups each one
// walks), plus the merge's rounds of partial loads, the fewest splits on ties.
static int qg_pick_splits(int blocks, int ngroups, int gmax, int target) {
    const int smin = (ngroups + gmax - 1) / gmax;
    const int cap = ngroups > smin ? ngroups : smin;
    int best = smin;
    int64_t best_cost = INT64_MAX;
    for (int s = smin; s <= cap; s++) {
        const int64_t rounds = ((int64_t)blocks * s + target - 1) / target;
        // a workgroup's fixed costs (pipeline fill, split merge) weigh about
        // as much as 3 groups of weights (measured: 14336 x 4096 Q4_K at 16
        // tokens 21.7 us with 4 splits of 4 groups, 29.7 with 8 of 2 in two
        // rounds; 1024 x 4096 Q6_K 20.6 us with 4 splits on 16 workgroups)
        // plus half a group per round of the merging wavefront's partial loads
        // (4 splits per round; in half-group units: 4096 x 4096 Q4_K at 16
        // tokens 16.1 us with 16 splits, 13.6 with 8; a full group per round
        // moved 4096 x 14336 from 14 to 12 splits, 25.5 -> 26.2 us)
        const int gps = (ngroups + s - 1) / s;
        const int64_t cost = 2 * rounds * (3 + gps) + (s + 3) / 4;
        if (cost < best_cost) {
            best_cost = cost;
            best = s;
        }
    }
    return best;
}

// One grouped launch: every entry's row blocks, each workgroup digitising its
// own K split of its entry's x.
// img_ready: the launch's one token block already has its images in slot 0
// (qg_norm_image), so no image launch and no in-kernel digitisation.
static hipError_t qg_run(uint32_t type, const QgEntry* en, int cnt, int in_dim, uint32_t row_bytes,
                         const QgScratch& sc, hipStream_t st, int accum, bool img_ready = false) {
    const int ngroups = in_dim / 256;
    QgXs xs = {};
    xs.halves = 1;
    QgGroups gs = {};
    int nslots = 0, ntmax = 0;
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
        gs.ldy[i] = en[i].ldy;
        gs.slot[i] = j;
        gs.x[i] = en[i].x;
        gs.x2[i] = en[i].x2;
        gs.n[i] = en[i].n;
        ntmax = en[i].n > ntmax ? en[i].n : ntmax;
    }
    // One 32-row tile per wavefront, QG_WAVES per workgroup.  Splits: enough
    // workgroups for one per CU (the kernel's registers allow no second).
    const int brows = 32 * QG_WAVES;
    int blocks = 0;
    for (int i = 0; i < cnt; i++) blocks += (en[i].rows + brows - 1) / brows;
    // Splits for streamed images; when they leave at most QG_GMAX groups per
    // split (launches of about one round), the split's images stay resident
    // in LDS instead and the item loop needs no workgroup barriers.
    int splits = qh_mmq_splits_env();
    if (splits <= 0) splits = qg_pick_splits(blocks, ngroups, ngroups, QG_TARGET_WGS);
    splits = splits < ngroups ? splits : ngroups;
    // 17-32 tokens per block: two image halves per group, QG_GMAX2 groups of
    // them resident in LDS
    const int halves = ntmax > 16 ? 2 : 1;
    const bool res = (ngroups + splits - 1) / splits <= (halves == 2 ? QG_GMAX2 : QG_GMAX);
    // Resident images are digitised in the kernel (no image launch) when few
    // row blocks share each token block's x; otherwise qg_ximage digitises
    // each block's x once.
    int mode = res ? (blocks <= QG_DIG_BLOCKS * nslots ? 2 : 1) : 0;
    const int fm = qh_mmq_mode_env();
    if (fm == 0) mode = 0;
    else if (fm >= 1 && fm <= 2 && res) mode = fm;
    if (img_ready) {
        if (nslots != 1) return hipErrorNotSupported;
        mode = res ? 1 : 0;
    }
    // two halves: no resident copy of ready images (MODE 1); ready images are
    // the two-half layout qg_norm_image writes past 16 tokens
    if (halves == 2 && mode == 1) mode = 0;
    const int64_t pb = (int64_t)(brows / 32) * 16 * halves * 32;  // floats of one partial block (token bound)
    // The partials and the per-block counters must hold the launch: otherwise
    // halve the batch (or, for one entry, its rows) and run the halves in turn.
    const bool img_fits = (int64_t)nslots * halves * ngroups * XImg::BYTES <= (int64_t)QG_IMG_BYTES;
    if (!img_fits || (splits > 1 && ((int64_t)blocks * splits * pb > QG_PART_FLOATS || blocks > QG_PART_TILES))) {
        if (cnt > 1) {
            hipError_t e = qg_run(type, en, cnt / 2, in_dim, row_bytes, sc, st, accum, img_ready);
            return e != hipSuccess ? e
                                   : qg_run(type, en + cnt / 2, cnt - cnt / 2, in_dim, row_bytes, sc, st, accum,
                                            img_ready);
        }
        const int half = (en[0].rows / 2 + brows - 1) / brows * brows;
        QgEntry a = en[0], b = en[0];
        a.rows = half;
        b.rows = en[0].rows - half;
        b.w += (size_t)half * row_bytes;
        b.y += half;
        hipError_t e = qg_run(type, &a, 1, in_dim, row_bytes, sc, st, accum, img_ready);
        return e != hipSuccess ? e : qg_run(type, &b, 1, in_dim, row_bytes, sc, st, accum, img_ready);
    }
    int wgs = 0, maxw = 0;
    for (int i = 0; i < cnt; i++) {
        gs.bstart[i] = wgs;
        const int wi = (en[i].rows + brows - 1) / brows * splits;
        wgs += wi;
        maxw = wi > maxw ? wi : maxw;
    }
    for (int i = cnt; i <= QG_MAXG; i++) gs.bstart[i] = wgs;
    gs.accum = accum;
    const dim3 grid((unsigned)maxw, (unsigned)cnt);
    // the token blocks' x images, once per launch
    xs.img = sc.img;
    xs.halves = halves;
    xs.img_bytes = (uint32_t)(nslots * halves * ngroups * XImg::BYTES);
    if (mode != 2 && !img_ready)
        hipLaunchKernelGGL(qg_ximage, dim3((unsigned)ngroups, (unsigned)(nslots * halves)), dim3(512), 0, st, xs, sc.img,
                           in_dim);
    switch (type) {
        case QT_Q4_K: launch_mmq_nt<GQ4K>(ntmax, mode, gs, xs, grid, splits, sc, row_bytes, in_dim, st); break;
        case QT_Q5_K: launch_mmq_nt<GQ5K>(ntmax, mode, gs, xs, grid, splits, sc, row_bytes, in_dim, st); break;
        case QT_IQ3_S: launch_mmq_nt<GIQ3S>(ntmax, mode, gs, xs, grid, splits, sc, row_bytes, in_dim, st); break;
        case QT_IQ2_XXS: launch_mmq_nt<GIQ2XXS>(ntmax, mode, gs, xs, grid, splits, sc, row_bytes, in_dim, st); break;
        default: launch_mmq_nt<GQ6K>(ntmax, mode, gs, xs, grid, splits, sc, row_bytes, in_dim, st); break;
    }
    return hipGetLastError();
}

// Batched tokens on the matrix cores for `count` matrices of one type and
// in_dim: Y[i][t][:] = W[i] X[i][t][:] for t < n[i] (token-major, y token stride
// out_dims[i]); hipErrorNotSupported when the type/shape has no kernel here.
// Tokens go in chunks of up to 16 (one weight pass each); matrices whose
// weights pass 2 GB go in row chunks.  The split-K partials and counters are
// one array per device, so calls that overlap on one device (different
// streams) must be serialised by the caller.
hipError_t qh_launch_mmq_grouped(uint32_t type, int count, const uint8_t* const* W, const float* const* X,
                                 float* const* Y, const int* n, const int* out_dims, int in_dim, hipStream_t st,
                                 const float* const* X2, int accum, const float* nw) {
    if (in_dim % 256 || in_dim / 256 > QG_MAX_GROUPS || count < 1) return hipErrorNotSupported;
    // an RMS norm fuses only into the 2-4 token GEMV path (the batched path
    // normalises into scratch first)
    if (nw && X2) return hipErrorNotSupported;
    if (!X2 && count <= 4) {
        // 2-4 tokens of one x shared by up to 4 matrices: the GEMV kernel carries
        // the tokens (the weights read once)
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
    const int max_slots = QG_MAXG;
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
        for (int t0 = 0; t0 < n[i]; t0 += 32) {
            // blocks of up to 32 tokens (17-32: one weight pass on two halves)
            const int nt = n[i] - t0 < 32 ? n[i] - t0 : 32;
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

hipError_t qh_launch_mmq_norm(uint32_t type, int count, const uint8_t* const* W, float* const* Y, const int* out_dims,
                              const float* x, const float* nw, int n, int in_dim, hipStream_t st, bool img_done) {
    if (n < 2 || n > 32 || count < 1 || count > QG_MAXG || in_dim % 256 || in_dim > 4096 || !nw)
        return hipErrorNotSupported;
    if (type != QT_Q4_K && type != QT_Q5_K && type != QT_Q6_K && type != QT_IQ3_S && type != QT_IQ2_XXS)
        return hipErrorNotSupported;
    const QgScratch* sc = qh_mmq_scratch_ptrs();
    if (!sc) return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    QgEntry en[QG_MAXG];
    int cnt = 0;
    for (int i = 0; i < count; i++) {
        if (out_dims[i] <= 0) continue;
        if ((int64_t)out_dims[i] * row_bytes >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
        en[cnt++] = QgEntry{W[i], x, nullptr, Y[i], n, out_dims[i], out_dims[i]};
    }
    if (cnt == 0) return hipSuccess;
    if (!img_done) {
        hipError_t e = qh_glue_norm_image(sc->img, x, nw, n, in_dim, st);
        if (e != hipSuccess) return e;
    }
    return qg_run(type, en, cnt, in_dim, row_bytes, *sc, st, 0, true);
}

// Two weight types sharing one x of n <= 16 tokens (a layer's q, k in Q4_K and
// v in Q6_K; n <= 32 with nw, 17-32 on two streamed image halves) in one
// launch, images digitised in the kernel or by qg_norm_image: Y1[i] = W1[i] X,
// Y2[i] = W2[i] X (token-major, token stride out_dims).  Splits are chosen
// jointly: the pair (s1, s2) minimising the rounds of 256 workgroups over both
// formats times (3 + the longer split), the fewest workgroups on ties.
// hipErrorNotSupported when the pair, shapes or scratch do not fit; the caller
// then makes one call per type.
template <class F1, class F2, int NT>
static void launch_mmq_mix(const QgGroups& g1s, const QgGroups& g2s, const QgXs& xs, uint32_t rb1, uint32_t rb2,
                           int in_dim, int s1, int s2, int c1, dim3 grid, const QgScratch& sc, size_t poff, int coff,
                           hipStream_t st, bool img_ready) {
    if constexpr (NT > 16)  // two image halves, streamed from qg_norm_image's images
        hipLaunchKernelGGL((qh_mmq_mix<F1, F2, NT, QG_WAVES, 0>), grid, dim3(64 * QG_WAVES), 0, st, g1s, g2s, xs, rb1,
                           rb2, in_dim, s1, s2, c1, sc.part, sc.cnt, sc.part + poff, sc.cnt + coff);
    else if (img_ready)
        hipLaunchKernelGGL((qh_mmq_mix<F1, F2, NT, QG_WAVES, 1>), grid, dim3(64 * QG_WAVES), 0, st, g1s, g2s, xs, rb1,
                           rb2, in_dim, s1, s2, c1, sc.part, sc.cnt, sc.part + poff, sc.cnt + coff);
    else
        hipLaunchKernelGGL((qh_mmq_mix<F1, F2, NT, QG_WAVES, 2>), grid, dim3(64 * QG_WAVES), 0, st, g1s, g2s, xs, rb1,
                           rb2, in_dim, s1, s2, c1, sc.part, sc.cnt, sc.part + poff, sc.cnt + coff);
}

hipError_t qh_launch_mmq_mixed(uint32_t t1, int c1, const uint8_t* const* W1, float* const* Y1, const int* o1,
                               uint32_t t2, int c2, const uint8_t* const* W2, float* const* Y2, const int* o2,
                               const float* x, int n, int in_dim, hipStream_t st, const float* nw) {
    if (t1 == QT_Q6_K && t2 == QT_Q4_K)
        return qh_launch_mmq_mixed(t2, c2, W2, Y2, o2, t1, c1, W1, Y1, o1, x, n, in_dim, st, nw);
    if (t1 != QT_Q4_K || t2 != QT_Q6_K) return hipErrorNotSupported;
    // 17-32 tokens only from images qg_norm_image writes (two halves, streamed)
    if (n < 2 || n > (nw ? 32 : 16) || c1 < 1 || c2 < 1 || c1 > QG_MAXG || c2 > QG_MAXG || in_dim % 256 ||
        in_dim / 256 > QG_MAX_GROUPS || ((uintptr_t)x & 15u))
        return hipErrorNotSupported;
    const int halves = n > 16 ? 2 : 1;
    const QgScratch* sc = qh_mmq_scratch_ptrs();
    if (!sc) return hipErrorNotSupported;
    const int ngroups = in_dim / 256, brows = 32 * QG_WAVES;
    const uint32_t rb1 = (uint32_t)qh_type_size(t1, (size_t)in_dim), rb2 = (uint32_t)qh_type_size(t2, (size_t)in_dim);
    int b1 = 0, b2 = 0;
    for (int i = 0; i < c1; i++) {
        if (o1[i] <= 0 || (int64_t)o1[i] * rb1 >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
        b1 += (o1[i] + brows - 1) / brows;
    }
    for (int i = 0; i < c2; i++) {
        if (o2[i] <= 0 || (int64_t)o2[i] * rb2 >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
        b2 += (o2[i] + brows - 1) / brows;
    }
    const int smin = (ngroups + QG_GMAX - 1) / QG_GMAX;
    int s1 = 0, s2 = 0;
    int64_t best = INT64_MAX, best_wgs = INT64_MAX;
    for (int a = smin; a <= ngroups; a++)
        for (int b = smin; b <= ngroups; b++) {
            const int64_t wgs = (int64_t)b1 * a + (int64_t)b2 * b;
            const int64_t rounds = (wgs + QG_TARGET_WGS - 1) / QG_TARGET_WGS;
            const int gps = (ngroups + a - 1) / a > (ngroups + b - 1) / b ? (ngroups + a - 1) / a : (ngroups + b - 1) / b;
            const int merge = (a > b ? a : b) + 3;
            const int64_t cost = 2 * rounds * (3 + gps) + merge / 4;
            if (cost < best || (cost == best && wgs < best_wgs)) {
                best = cost;
                best_wgs = wgs;
                s1 = a;
                s2 = b;
            }
        }
    const int wgs1 = b1 * s1, wgs = wgs1 + b2 * s2;
    const int64_t pw = (int64_t)QG_WAVES * 16 * halves * 32;  // floats of one workgroup's partials (token bound)
    if ((int64_t)wgs * pw > QG_PART_FLOATS || b1 + b2 > QG_PART_TILES) return hipErrorNotSupported;
    QgXs xs = {};
    xs.halves = halves;
    xs.x[0] = x;
    xs.n[0] = n;
    // nw: x's rows RMS-normalised with nw and digitised by qg_norm_image into
    // image slot 0 first; the kernel then copies the images (MODE 1)
    const bool img_ready = nw != nullptr;
    if (img_ready) {
        hipError_t e = qh_glue_norm_image(sc->img, x, nw, n, in_dim, st);
        if (e != hipSuccess) return e;
        xs.img = sc->img;
        xs.img_bytes = (uint32_t)(halves * ngroups * XImg::BYTES);
    }
    int maxw = 0;
    auto fill = [&](QgGroups& g, int c, const uint8_t* const* Wt, float* const* Y, const int* o, uint32_t rb, int s) {
        g = QgGroups{};
        int w = 0;
        for (int i = 0; i < c; i++) {
            g.bstart[i] = w;
            g.w[i] = Wt[i];
            g.y[i] = Y[i];
            g.wbytes[i] = (uint32_t)(((uint64_t)o[i] * rb + 3) & ~(uint64_t)3);
            g.rows[i] = o[i];
            g.ldy[i] = o[i];
            g.slot[i] = 0;
            g.x[i] = x;
            g.n[i] = n;
            const int wi = (o[i] + brows - 1) / brows * s;
            w += wi;
            maxw = wi > maxw ? wi : maxw;
        }
        for (int i = c; i <= QG_MAXG; i++) g.bstart[i] = w;
        g.accum = 0;
    };
    QgGroups g1s, g2s;
    fill(g1s, c1, W1, Y1, o1, rb1, s1);
    fill(g2s, c2, W2, Y2, o2, rb2, s2);
    const size_t poff = (size_t)wgs1 * pw;
    const int coff = b1 * QG_WAVES;
    const dim3 grid((unsigned)maxw, (unsigned)(c1 + c2));
    if (n <= 4) launch_mmq_mix<GQ4K, GQ6K, 4>(g1s, g2s, xs, rb1, rb2, in_dim, s1, s2, c1, grid, *sc, poff, coff, st,
                                              img_ready);
    else if (n <= 8) launch_mmq_mix<GQ4K, GQ6K, 8>(g1s, g2s, xs, rb1, rb2, in_dim, s1, s2, c1, grid, *sc, poff, coff, st,
                                              img_ready);
    else if (n <= 16) launch_mmq_mix<GQ4K, GQ6K, 16>(g1s, g2s, xs, rb1, rb2, in_dim, s1, s2, c1, grid, *sc, poff, coff,
                                                     st, img_ready);
    else launch_mmq_mix<GQ4K, GQ6K, 32>(g1s, g2s, xs, rb1, rb2, in_dim, s1, s2, c1, grid, *sc, poff, coff, st,
                                        img_ready);
    return hipGetLastError();
}

// Expert layers with token ranges on the device: for s < sets and e < n_exp,
// Y[s][t] = E[s][e] X[t] for the gathered rows t = tok_off[e] .. tok_off[e + 1]
// - 1 (X[t] = silu(X[t]) * X2[t] with X2), expert e's weights at E[s] + e *
// slice.  Every expert gets max_tokens / 16 (rounded up) token chunks of
// workgroups; chunks past an expert's tokens exit at once, so nothing is read
// back to the host (the launch can sit in a captured graph).  Experts go in
// batches of up to QG_MAXG / sets.
hipError_t qh_launch_mmq_moe_dev(uint32_t type, int sets, const uint8_t* const* E, float* const* Y, int n_exp,
                                 const int* tok_off, int max_tokens, const float* X, const float* X2, int in_dim,
                                 int out_dim, int accum, hipStream_t st) {
    if (type != QT_Q4_K && type != QT_Q5_K && type != QT_Q6_K && type != QT_IQ3_S && type != QT_IQ2_XXS)
        return hipErrorNotSupported;
    if (sets < 1 || sets > 2 || n_exp < 1 || max_tokens < 1 || in_dim % 256 || in_dim / 256 > QG_MAX_GROUPS ||
        out_dim < 1 || ((uintptr_t)X & 15u) || ((uintptr_t)X2 & 15u))
        return hipErrorNotSupported;
    const QgScratch* sc = qh_mmq_scratch_ptrs();
    if (!sc) return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    if ((int64_t)out_dim * row_bytes >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
    const size_t slice = (size_t)row_bytes * (size_t)out_dim;
    const int ngroups = in_dim / 256, brows = 32 * QG_WAVES, blocks = (out_dim + brows - 1) / brows;
    // experts of more than 16 tokens: 32-token chunks on two image halves (one
    // weight pass for up to 32 tokens), streamed images
    const int halves = max_tokens > 16 ? 2 : 1;
    const int C = (max_tokens + 16 * halves - 1) / (16 * halves);
    const int pw = QG_WAVES * 16 * halves * 32;  // floats of one workgroup's partials (token bound)
    for (int e0 = 0; e0 < n_exp;) {
        // experts of this launch: bounded by the entries, the partials and the images
        int ne = n_exp - e0 < QG_MAXG / sets ? n_exp - e0 : QG_MAXG / sets;
        int splits = 1, mode = 0;
        for (;; ne--) {
            if (ne < 1) return hipErrorNotSupported;
            const int bl = sets * ne * blocks;  // row blocks with one chunk per expert
            splits = qh_mmq_splits_env();
            if (splits <= 0) splits = qg_pick_splits(bl, ngroups, ngroups, QG_TARGET_WGS);
            splits = splits < ngroups ? splits : ngroups;
            const bool res = (ngroups + splits - 1) / splits <= QG_GMAX;
            mode = res ? (bl <= QG_DIG_BLOCKS * ne ? 2 : 1) : 0;
            if (halves == 2) mode = 0;
            const int64_t wgs = (int64_t)sets * ne * C * blocks * splits;
            const bool fits = wgs * pw <= QG_PART_FLOATS && (int64_t)sets * ne * C * blocks <= QG_PART_TILES &&
                              (mode == 2 || (int64_t)ne * C * halves * ngroups * XImg::BYTES <= (int64_t)QG_IMG_BYTES);
            if (fits) break;
        }
        QgXs xs = {};
        xs.halves = halves;
        xs.x[0] = X;
        xs.x2[0] = X2;
        xs.tok_off = tok_off + e0;
        xs.moe_c = C;
        xs.img = sc->img;
        xs.img_bytes = (uint32_t)((int64_t)ne * C * halves * ngroups * XImg::BYTES);
        QgGroups gs = {};
        int wgs = 0;
        const int per = C * blocks * splits;  // workgroups of each (set, expert)
        for (int i = 0; i < sets * ne; i++) {
            const int s = i / ne, e = i - s * ne;
            gs.bstart[i] = wgs;
            gs.w[i] = E[s] + (size_t)(e0 + e) * slice;
            gs.y[i] = Y[s];
            gs.wbytes[i] = (uint32_t)((slice + 3) & ~(size_t)3);
            gs.rows[i] = out_dim;
            gs.ldy[i] = out_dim;
            gs.slot[i] = e;
            wgs += per;
        }
        for (int i = sets * ne; i <= QG_MAXG; i++) gs.bstart[i] = wgs;
        gs.accum = accum;
        const dim3 grid((unsigned)per, (unsigned)(sets * ne));
        if (mode != 2)
            hipLaunchKernelGGL(qg_ximage, dim3((unsigned)ngroups, (unsigned)(ne * C * halves)), dim3(512), 0, st, xs,
                               sc->img, in_dim);
        switch (type) {
            case QT_Q4_K: launch_mmq_nt<GQ4K>(16 * halves, mode, gs, xs, grid, splits, *sc, row_bytes, in_dim, st); break;
            case QT_Q5_K: launch_mmq_nt<GQ5K>(16 * halves, mode, gs, xs, grid, splits, *sc, row_bytes, in_dim, st); break;
            case QT_IQ3_S: launch_mmq_nt<GIQ3S>(16 * halves, mode, gs, xs, grid, splits, *sc, row_bytes, in_dim, st); break;
            case QT_IQ2_XXS: launch_mmq_nt<GIQ2XXS>(16 * halves, mode, gs, xs, grid, splits, *sc, row_bytes, in_dim, st); break;
            default: launch_mmq_nt<GQ6K>(16 * halves, mode, gs, xs, grid, splits, *sc, row_bytes, in_dim, st); break;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        e0 += ne;
    }
    return hipSuccess;
}
