// qh_formats.h -- per-format "unit" decoders for the batch-1 GEMV kernel.
//
// A unit is 64 consecutive-in-storage weights of one row that one lane owns:
// a quarter superblock for the 256-element formats, two blocks for the
// 32-element formats, 64 elements for F32/F16/BF16.  Every policy provides
//
//   NRAW             dwords of raw weight bytes per unit (loaded first, decoded later)
//   NXS              partial sums of x the decode needs (shared by every row)
//   xoff(u, c)       row-relative element index of the c-th 4-float chunk of x
//                    that pairs with unit u (c = 0..15), i.e. the order in which
//                    dot() consumes the 64 activations
//   load(b, roff, u, raw)   issue the buffer loads for unit u of the row at byte roff
//   xsums(xv, xs)    the NXS partial sums of the 64 activations
//   dot(raw, xv, xs, roff, u)   sum over the unit of x * w, in f32
//
// The decode expressions are those of src/dequant.rs (block layouts at the
// lines cited per policy); dot() reassociates the sums (factored scales, offset
// folding), which the 1e-3 relative-L2 GEMV tolerance allows.  The bit-exact
// per-element decode lives in qh_dequant.hip.
#pragma once
#include "qh_device.h"

// IQ codebooks, one copy per device, initialised from iq_grids.h and
// overwritable through hip_set_*_grid (src/cuda_kernels.cu:814-818, 1027-1041).
extern __device__ uint64_t qh_g_iq2xxs[256];
extern __device__ uint64_t qh_g_iq2xs[512];
extern __device__ uint64_t qh_g_iq2s[1024];
extern __device__ uint32_t qh_g_iq3s[512];

// ---------------------------------------------------------------- helpers

// Q4_K / Q5_K 6-bit (scale, min) pair for sub-blocks 2p and 2p+1, from the 12
// packed bytes held in dwords s0 (bytes 0-3), s1 (4-7), s2 (8-11).
// Restates get_scale_min_k4 (src/dequant.rs:1471-1480) for j = 2p, 2p+1.
QH_DEV void qh_scale_pair(uint32_t s0, uint32_t s1, uint32_t s2, int p,
                          uint32_t& sc1, uint32_t& m1, uint32_t& sc2, uint32_t& m2) {
    const uint32_t sh = 16u * (uint32_t)(p & 1);
    const uint32_t A = s0 >> sh, B = s1 >> sh, C = s2 >> sh;
    if (p < 2) {
        sc1 = A & 63u;         m1 = B & 63u;
        sc2 = (A >> 8) & 63u;  m2 = (B >> 8) & 63u;
    } else {
        sc1 = (C & 15u) | ((A >> 2) & 0x30u);
        m1 = ((C >> 4) & 15u) | ((B >> 2) & 0x30u);
        sc2 = ((C >> 8) & 15u) | ((A >> 10) & 0x30u);
        m2 = ((C >> 12) & 15u) | ((B >> 10) & 0x30u);
    }
}

QH_DEV float qh_sum(const float* v, int n) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < n; i += 2) { a += v[i]; b += v[i + 1]; }
    return a + b;
}

// ================================================================ K-quants

// Q4_K: [d f16][dmin f16][12 B scales][128 B qs], 144 B / 256 (src/dequant.rs:1482-1519).
// Unit u = superblock s = u/4, sub-block pair p = u%4 (sub-blocks 2p, 2p+1):
// header (16 B) + qs[32p .. 32p+32) (32 B).  Weight 64p+l is qs[32p+l]&15,
// weight 64p+32+l is qs[32p+l]>>4.
struct FmtQ4K {
    static constexpr uint32_t QK = 256, BLK = 144;
    static constexpr int NRAW = 12, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2), p = (uint32_t)(u & 3);
        qh_ldn<4>(b, base, r);
        qh_ldn<8>(b, base + 16 + 32 * p, r + 4);
    }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int u) {
        const float d = qh_f16_lo(r[0]), dmin = qh_f16_hi(r[0]);
        uint32_t sc1, m1, sc2, m2;
        qh_scale_pair(r[1], r[2], r[3], u & 3, sc1, m1, sc2, m2);
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            slo = qh_dot4u(xv + 4 * i, r[4 + i] & 0x0F0F0F0Fu, slo);
            shi = qh_dot4u(xv + 32 + 4 * i, (r[4 + i] >> 4) & 0x0F0F0F0Fu, shi);
        }
        return (d * (float)sc1) * slo - (dmin * (float)m1) * xs[0] + (d * (float)sc2) * shi -
               (dmin * (float)m2) * xs[1];
    }
};

// Q5_K: [d][dmin][12 B scales][qh 32 B][qs 128 B], 176 B / 256 (src/dequant.rs:1146-1181).
// Unit u = superblock s, jb = u%4: ql = qs[32jb..+32], high bits = qh bits 2jb / 2jb+1.
struct FmtQ5K {
    static constexpr uint32_t QK = 256, BLK = 176;
    static constexpr int NRAW = 20, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2), jb = (uint32_t)(u & 3);
        qh_ldn<4>(b, base, r);
        qh_ldn<8>(b, base + 16, r + 4);
        qh_ldn<8>(b, base + 48 + 32 * jb, r + 12);
    }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int u) {
        const int jb = u & 3;
        const float d = qh_f16_lo(r[0]), dmin = qh_f16_hi(r[0]);
        uint32_t sc1, m1, sc2, m2;
        qh_scale_pair(r[1], r[2], r[3], jb, sc1, m1, sc2, m2);
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t ql = r[12 + i], qh = r[4 + i];
            const uint32_t lo = (ql & 0x0F0F0F0Fu) | (((qh >> (2 * jb)) & 0x01010101u) << 4);
            const uint32_t hi = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * jb + 1)) & 0x01010101u) << 4);
            slo = qh_dot4u(xv + 4 * i, lo, slo);
            shi = qh_dot4u(xv + 32 + 4 * i, hi, shi);
        }
        return (d * (float)sc1) * slo - (dmin * (float)m1) * xs[0] + (d * (float)sc2) * shi -
               (dmin * (float)m2) * xs[1];
    }
};

// Q6_K: [ql 128][qh 64][sc 16 x i8][d f16], 210 B / 256 (src/dequant.rs:1583-1631).
// Unit u = superblock s = u/4, half h = (u/2)%2, position group g = u%2 (l in
// [16g, 16g+16)).  The unit's weights are y[128h + 32k + l], k = 0..3, using
// ql[64h+l] (k=0 low, k=2 high nibble), ql[64h+32+l] (k=1 low, k=3 high),
// qh[32h+l] bits 2k..2k+1 and scale sc[8h + l/16 + 2k] = sc[8h + g + 2k].
// Superblocks sit at 2-byte alignment, hence the window loads.
struct FmtQ6K {
    static constexpr uint32_t QK = 256, BLK = 210;
    static constexpr int NRAW = 19, NXS = 4;
    QH_DEV static int xoff(int u, int c) {
        const int s = u >> 2, h = (u >> 1) & 1, g = u & 1, k = c >> 2, i = c & 3;
        return 256 * s + 128 * h + 32 * k + 16 * g + 4 * i;
    }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2);
        const uint32_t h = (uint32_t)((u >> 1) & 1), g = (uint32_t)(u & 1);
        const uint32_t o1 = base + 64 * h + 16 * g;
        qh_ldwin<4>(b, o1, r);
        qh_ldwin<4>(b, o1 + 32, r + 5);
        qh_ldwin<4>(b, base + 128 + 32 * h + 16 * g, r + 10);
        qh_ldwin<2>(b, base + 192 + 8 * h, r + 15);
        r[18] = qh_ld32(b, (base + 208) & ~3u);
    }
    QH_DEV static void xsums(const float* xv, float* xs) {
#pragma unroll
        for (int k = 0; k < 4; k++) xs[k] = qh_sum(xv + 16 * k, 16);
    }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t roff, int u) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2);
        const uint32_t g = (uint32_t)(u & 1);
        uint32_t a[4], bq[4], q[4], sc[2];
        qh_fix<4>(r, base, a);
        qh_fix<4>(r + 5, base, bq);
        qh_fix<4>(r + 10, base, q);
        qh_fix<2>(r + 15, base, sc);
        const float d = (base & 2u) ? qh_f16_hi(r[18]) : qh_f16_lo(r[18]);
        float S[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q0 = (a[i] & 0x0F0F0F0Fu) | ((q[i] << 4) & 0x30303030u);
            const uint32_t q1 = (bq[i] & 0x0F0F0F0Fu) | ((q[i] << 2) & 0x30303030u);
            const uint32_t q2 = ((a[i] >> 4) & 0x0F0F0F0Fu) | (q[i] & 0x30303030u);
            const uint32_t q3 = ((bq[i] >> 4) & 0x0F0F0F0Fu) | ((q[i] >> 2) & 0x30303030u);
            S[0] = qh_dot4u(xv + 0 + 4 * i, q0, S[0]);
            S[1] = qh_dot4u(xv + 16 + 4 * i, q1, S[1]);
            S[2] = qh_dot4u(xv + 32 + 4 * i, q2, S[2]);
            S[3] = qh_dot4u(xv + 48 + 4 * i, q3, S[3]);
        }
        const uint32_t shb = 8u * g;
        const float s0 = (float)(int8_t)(sc[0] >> shb), s1 = (float)(int8_t)(sc[0] >> (shb + 16));
        const float s2 = (float)(int8_t)(sc[1] >> shb), s3 = (float)(int8_t)(sc[1] >> (shb + 16));
        return d * (s0 * (S[0] - 32.f * xs[0]) + s1 * (S[1] - 32.f * xs[1]) + s2 * (S[2] - 32.f * xs[2]) +
                    s3 * (S[3] - 32.f * xs[3]));
    }
};

// Q2_K: [scales 16][qs 64][d f16][dmin f16], 84 B / 256 (src/dequant.rs:1113-1144).
// Unit u = superblock s, n = (u/2)%2 (128-element half), jp = u%2: shifts
// j = 2jp, 2jp+1 over q = qs[32n..+32]; scales is = 8n + 4jp + 0..3.
struct FmtQ2K {
    static constexpr uint32_t QK = 256, BLK = 84;
    static constexpr int NRAW = 10, NXS = 4;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2);
        const uint32_t n = (uint32_t)((u >> 1) & 1), jp = (uint32_t)(u & 1);
        qh_ldn<8>(b, base + 16 + 32 * n, r);
        r[8] = qh_ld32(b, base + 8 * n + 4 * jp);
        r[9] = qh_ld32(b, base + 80);
    }
    QH_DEV static void xsums(const float* xv, float* xs) {
#pragma unroll
        for (int k = 0; k < 4; k++) xs[k] = qh_sum(xv + 16 * k, 16);
    }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int u) {
        const uint32_t sh0 = 4u * (uint32_t)(u & 1), sh1 = sh0 + 2;
        const float d = qh_f16_lo(r[9]), dmin = qh_f16_hi(r[9]);
        float G[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            G[0] = qh_dot4u(xv + 4 * i, (r[i] >> sh0) & 0x03030303u, G[0]);
            G[1] = qh_dot4u(xv + 16 + 4 * i, (r[4 + i] >> sh0) & 0x03030303u, G[1]);
            G[2] = qh_dot4u(xv + 32 + 4 * i, (r[i] >> sh1) & 0x03030303u, G[2]);
            G[3] = qh_dot4u(xv + 48 + 4 * i, (r[4 + i] >> sh1) & 0x03030303u, G[3]);
        }
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t sc = (r[8] >> (8 * k)) & 0xFFu;
            acc += (d * (float)(sc & 15u)) * G[k] - (dmin * (float)(sc >> 4)) * xs[k];
        }
        return acc;
    }
};

// ================================================================ 32-element blocks (unit = 2 blocks)

// Q8_0: [d f16][32 x i8], 34 B / 32 (src/dequant.rs:1450-1463).  68 B per unit.
struct FmtQ8_0 {
    static constexpr uint32_t QK = 32, BLK = 34;
    static constexpr int NRAW = 17, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<17>(b, roff + 68u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int) {
        const float d0 = qh_f16_lo(r[0]), d1 = qh_f16_hi(r[8]);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s0 = qh_dot4u(xv + 4 * i, __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2) ^ 0x80808080u, s0);
            s1 = qh_dot4u(xv + 32 + 4 * i, r[9 + i] ^ 0x80808080u, s1);
        }
        return d0 * (s0 - 128.f * xs[0]) + d1 * (s1 - 128.f * xs[1]);
    }
};

// Q5_0 block part shared by Q5_0/Q5_1: 5-bit q = nibble | qh bit << 4, weights
// j (low nibble of qs[j], qh bit j) and j+16 (high nibble, qh bit j+16).
QH_DEV float qh_q5_block(const uint32_t* qs, uint32_t qh, const float* xv) {
    float s = 0.f, t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = (qs[i] & 0x0F0F0F0Fu) | (qh_spread4((qh >> (4 * i)) & 15u) << 4);
        const uint32_t hi = ((qs[i] >> 4) & 0x0F0F0F0Fu) | (qh_spread4((qh >> (16 + 4 * i)) & 15u) << 4);
        s = qh_dot4u(xv + 4 * i, lo, s);
        t = qh_dot4u(xv + 16 + 4 * i, hi, t);
    }
    return s + t;
}

// Q5_0: [d f16][qh u32][qs 16], 22 B / 32 (src/dequant.rs:1381-1409); v = (q - 16) d.
struct FmtQ5_0 {
    static constexpr uint32_t QK = 32, BLK = 22;
    static constexpr int NRAW = 11, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<11>(b, roff + 44u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int) {
        uint32_t qs0[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qs0[i] = __builtin_amdgcn_alignbyte(r[i + 2], r[i + 1], 2);
        const uint32_t qh0 = __builtin_amdgcn_alignbyte(r[1], r[0], 2);
        const float d0 = qh_f16_lo(r[0]), d1 = qh_f16_hi(r[5]);
        const float s0 = qh_q5_block(qs0, qh0, xv), s1 = qh_q5_block(r + 7, r[6], xv + 32);
        return d0 * (s0 - 16.f * xs[0]) + d1 * (s1 - 16.f * xs[1]);
    }
};

// Q5_1: [d f16][m f16][qh u32][qs 16], 24 B / 32 (src/dequant.rs:1419-1443); v = q d + m.
struct FmtQ5_1 {
    static constexpr uint32_t QK = 32, BLK = 24;
    static constexpr int NRAW = 12, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<12>(b, roff + 48u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int) {
        const float s0 = qh_q5_block(r + 2, r[1], xv), s1 = qh_q5_block(r + 8, r[7], xv + 32);
        return qh_f16_lo(r[0]) * s0 + qh_f16_hi(r[0]) * xs[0] + qh_f16_lo(r[6]) * s1 + qh_f16_hi(r[6]) * xs[1];
    }
};

QH_DEV float qh_q4_block(const uint32_t* qs, const float* xv) {
    float s = 0.f, t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        s = qh_dot4u(xv + 4 * i, qs[i] & 0x0F0F0F0Fu, s);
        t = qh_dot4u(xv + 16 + 4 * i, (qs[i] >> 4) & 0x0F0F0F0Fu, t);
    }
    return s + t;
}

// Q4_0 (GGUF layout, not in Quartz): [d f16][qs 16], 18 B / 32; v = (q - 8) d.
struct FmtQ4_0 {
    static constexpr uint32_t QK = 32, BLK = 18;
    static constexpr int NRAW = 9, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<9>(b, roff + 36u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int) {
        uint32_t qs0[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qs0[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);
        const float s0 = qh_q4_block(qs0, xv), s1 = qh_q4_block(r + 5, xv + 32);
        return qh_f16_lo(r[0]) * (s0 - 8.f * xs[0]) + qh_f16_hi(r[4]) * (s1 - 8.f * xs[1]);
    }
};

// Q4_1 (GGUF layout, not in Quartz): [d f16][m f16][qs 16], 20 B / 32; v = q d + m.
struct FmtQ4_1 {
    static constexpr uint32_t QK = 32, BLK = 20;
    static constexpr int NRAW = 10, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<10>(b, roff + 40u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int) {
        const float s0 = qh_q4_block(r + 1, xv), s1 = qh_q4_block(r + 6, xv + 32);
        return qh_f16_lo(r[0]) * s0 + qh_f16_hi(r[0]) * xs[0] + qh_f16_lo(r[5]) * s1 + qh_f16_hi(r[5]) * xs[1];
    }
};

// IQ4_NL: [d f16][qs 16], 18 B / 32 (src/dequant.rs:1527-1574); v = d * T[q].
// T + 128 as bytes, looked up four at a time with v_perm_b32.
QH_DEV uint32_t qh_iq4nl_lut(uint32_t idx) {
    // T[i] + 128 for i = 0..15: 1 24 45 63 | 79 93 106 118 | 129 141 153 166 | 181 197 217 241
    const uint32_t t0 = 0x3F2D1801u, t1 = 0x766A5D4Fu, t2 = 0xA6998D81u, t3 = 0xF1D9C5B5u;
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}
QH_DEV float qh_iq4nl_block(const uint32_t* qs, const float* xv) {
    float s = 0.f, t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        s = qh_dot4u(xv + 4 * i, qh_iq4nl_lut(qs[i] & 0x0F0F0F0Fu), s);
        t = qh_dot4u(xv + 16 + 4 * i, qh_iq4nl_lut((qs[i] >> 4) & 0x0F0F0F0Fu), t);
    }
    return s + t;
}
struct FmtIQ4NL {
    static constexpr uint32_t QK = 32, BLK = 18;
    static constexpr int NRAW = 9, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<9>(b, roff + 36u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t, int) {
        uint32_t qs0[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qs0[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], 2);
        const float s0 = qh_iq4nl_block(qs0, xv), s1 = qh_iq4nl_block(r + 5, xv + 32);
        return qh_f16_lo(r[0]) * (s0 - 128.f * xs[0]) + qh_f16_hi(r[4]) * (s1 - 128.f * xs[1]);
    }
};

// ================================================================ IQ codebook formats

// 8 signed codebook values (grid entry g, 8 sign bits) dotted with 8 activations.
// Values are made unsigned by +128 (byte xor 0x80); the caller subtracts 128*sum(x).
QH_DEV float qh_grid8(uint64_t g, uint32_t signs, const float* xv, float s) {
    const uint32_t lo = qh_signbytes((uint32_t)g, signs & 0xFu) ^ 0x80808080u;
    const uint32_t hi = qh_signbytes((uint32_t)(g >> 32), (signs >> 4) & 0xFu) ^ 0x80808080u;
    s = qh_dot4u(xv, lo, s);
    return qh_dot4u(xv + 4, hi, s);
}

// IQ2_XXS: [d f16][qs 64], 66 B / 256 (src/dequant.rs:1011-1041).
// Unit u = superblock s, pair pr = u%4: groups ib32 = 2pr, 2pr+1 (8 B each:
// 4 grid indices + u32 of 4x7 sign bits and a 4-bit scale).
struct FmtIQ2XXS {
    static constexpr uint32_t QK = 256, BLK = 66;
    static constexpr int NRAW = 6, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2);
        qh_ldwin<4>(b, base + 2 + 16 * (uint32_t)(u & 3), r);
        r[5] = qh_ld32(b, base & ~3u);
    }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t roff, int u) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2);
        uint32_t w[4];
        qh_fix<4>(r, base + 2, w);
        const float d = (base & 2u) ? qh_f16_hi(r[5]) : qh_f16_lo(r[5]);
        float acc = 0.f;
#pragma unroll
        for (int gi = 0; gi < 2; gi++) {
            const uint32_t a0 = w[2 * gi], a1 = w[2 * gi + 1];
            const float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
            float s = 0.f;
#pragma unroll
            for (int l = 0; l < 4; l++)
                s = qh_grid8(qh_g_iq2xxs[(a0 >> (8 * l)) & 255u], qh_ksigns((a1 >> (7 * l)) & 127u),
                             xv + 32 * gi + 8 * l, s);
            acc += db * (s - 128.f * xs[gi]);
        }
        return acc;
    }
};

// IQ2_XS: [d f16][qs 32 x u16][scales 8], 74 B / 256 (src/dequant.rs:1043-1075).
struct FmtIQ2XS {
    static constexpr uint32_t QK = 256, BLK = 74;
    static constexpr int NRAW = 7, NXS = 4;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2), pr = (uint32_t)(u & 3);
        qh_ldwin<4>(b, base + 2 + 16 * pr, r);
        r[5] = qh_ld32(b, base & ~3u);
        r[6] = qh_ld32(b, (base + 66 + 2 * pr) & ~3u);
    }
    QH_DEV static void xsums(const float* xv, float* xs) {
#pragma unroll
        for (int k = 0; k < 4; k++) xs[k] = qh_sum(xv + 16 * k, 16);
    }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t roff, int u) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2), pr = (uint32_t)(u & 3);
        uint32_t w[4];
        qh_fix<4>(r, base + 2, w);
        const float d = (base & 2u) ? qh_f16_hi(r[5]) : qh_f16_lo(r[5]);
        const uint32_t sc2 = r[6] >> (8u * ((base + 66 + 2 * pr) & 3u));  // scales[2pr], scales[2pr+1]
        float acc = 0.f;
#pragma unroll
        for (int gi = 0; gi < 2; gi++) {
            const uint32_t sb = (sc2 >> (8 * gi)) & 0xFFu;
            const float db0 = d * (0.5f + (float)(sb & 15u)) * 0.25f;
            const float db1 = d * (0.5f + (float)(sb >> 4)) * 0.25f;
            float s[2] = {0.f, 0.f};
#pragma unroll
            for (int l = 0; l < 4; l++) {
                const uint32_t q = (w[2 * gi + (l >> 1)] >> (16 * (l & 1))) & 0xFFFFu;
                s[l >> 1] = qh_grid8(qh_g_iq2xs[q & 511u], qh_ksigns(q >> 9), xv + 32 * gi + 8 * l, s[l >> 1]);
            }
            acc += db0 * (s[0] - 128.f * xs[2 * gi]) + db1 * (s[1] - 128.f * xs[2 * gi + 1]);
        }
        return acc;
    }
};

// IQ2_S: [d f16][qs 32 idx + 32 signs][qh 8][scales 8], 82 B / 256 (src/dequant.rs:1077-1110).
struct FmtIQ2S {
    static constexpr uint32_t QK = 256, BLK = 82;
    static constexpr int NRAW = 9, NXS = 4;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2), pr = (uint32_t)(u & 3);
        qh_ldwin<2>(b, base + 2 + 8 * pr, r);
        qh_ldwin<2>(b, base + 34 + 8 * pr, r + 3);
        r[6] = qh_ld32(b, (base + 66 + 2 * pr) & ~3u);
        r[7] = qh_ld32(b, (base + 74 + 2 * pr) & ~3u);
        r[8] = qh_ld32(b, base & ~3u);
    }
    QH_DEV static void xsums(const float* xv, float* xs) {
#pragma unroll
        for (int k = 0; k < 4; k++) xs[k] = qh_sum(xv + 16 * k, 16);
    }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t roff, int u) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2), pr = (uint32_t)(u & 3);
        uint32_t idx[2], sg[2];
        qh_fix<2>(r, base + 2, idx);
        qh_fix<2>(r + 3, base + 34, sg);
        const uint32_t qh2 = r[6] >> (8u * ((base + 66 + 2 * pr) & 3u));
        const uint32_t sc2 = r[7] >> (8u * ((base + 74 + 2 * pr) & 3u));
        const float d = (base & 2u) ? qh_f16_hi(r[8]) : qh_f16_lo(r[8]);
        float acc = 0.f;
#pragma unroll
        for (int gi = 0; gi < 2; gi++) {
            const uint32_t sb = (sc2 >> (8 * gi)) & 0xFFu, qhb = (qh2 >> (8 * gi)) & 0xFFu;
            const float db0 = d * (0.5f + (float)(sb & 15u)) * 0.25f;
            const float db1 = d * (0.5f + (float)(sb >> 4)) * 0.25f;
            float s[2] = {0.f, 0.f};
#pragma unroll
            for (int l = 0; l < 4; l++) {
                const uint32_t i = ((idx[gi] >> (8 * l)) & 0xFFu) | ((qhb << (8 - 2 * l)) & 0x300u);
                s[l >> 1] = qh_grid8(qh_g_iq2s[i], (sg[gi] >> (8 * l)) & 0xFFu, xv + 32 * gi + 8 * l, s[l >> 1]);
            }
            acc += db0 * (s[0] - 128.f * xs[2 * gi]) + db1 * (s[1] - 128.f * xs[2 * gi + 1]);
        }
        return acc;
    }
};

// IQ3_S: [d f16][qs 64][qh 8][signs 32][scales 4], 110 B / 256 (src/dequant.rs:1184-1237).
// Unit u = superblock s, it = u%4 (ib32 = 2it, 2it+1).
struct FmtIQ3S {
    static constexpr uint32_t QK = 256, BLK = 110;
    static constexpr int NRAW = 11, NXS = 2;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2), it = (uint32_t)(u & 3);
        qh_ldwin<4>(b, base + 2 + 16 * it, r);
        r[5] = qh_ld32(b, (base + 66 + 2 * it) & ~3u);
        qh_ldwin<2>(b, base + 74 + 8 * it, r + 6);
        r[9] = qh_ld32(b, (base + 106 + it) & ~3u);
        r[10] = qh_ld32(b, base & ~3u);
    }
    QH_DEV static void xsums(const float* xv, float* xs) { xs[0] = qh_sum(xv, 32); xs[1] = qh_sum(xv + 32, 32); }
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float* xs, uint32_t roff, int u) {
        const uint32_t base = roff + BLK * (uint32_t)(u >> 2), it = (uint32_t)(u & 3);
        uint32_t qs[4], sg[2];
        qh_fix<4>(r, base + 2, qs);
        qh_fix<2>(r + 6, base + 74, sg);
        const uint32_t qh2 = r[5] >> (8u * ((base + 66 + 2 * it) & 3u));
        const uint32_t scb = (r[9] >> (8u * ((base + 106 + it) & 3u))) & 0xFFu;
        const float d = (base & 2u) ? qh_f16_hi(r[10]) : qh_f16_lo(r[10]);
        float acc = 0.f;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const float db = d * (1.0f + 2.0f * (float)(half ? (scb >> 4) : (scb & 15u)));
            const uint32_t qhb = (qh2 >> (8 * half)) & 0xFFu;
            float s = 0.f;
#pragma unroll
            for (int l = 0; l < 4; l++) {
                const uint32_t qw = qs[2 * half + (l >> 1)] >> (16 * (l & 1));
                const uint32_t i0 = (qw & 0xFFu) | ((qhb << (8 - 2 * l)) & 256u);
                const uint32_t i1 = ((qw >> 8) & 0xFFu) | ((qhb << (7 - 2 * l)) & 256u);
                const uint32_t sb = (sg[half] >> (8 * l)) & 0xFFu;
                const uint64_t g = (uint64_t)qh_g_iq3s[i0] | ((uint64_t)qh_g_iq3s[i1] << 32);
                s = qh_grid8(g, sb, xv + 32 * half + 8 * l, s);
            }
            acc += db * (s - 128.f * xs[half]);
        }
        return acc;
    }
};

// ================================================================ plain floats

// F32 / F16 / BF16 rows (src/dequant.rs:946-981, 1321-1371): unit = 64 elements.
struct FmtF32 {
    static constexpr uint32_t QK = 1, BLK = 4;
    static constexpr int NRAW = 64, NXS = 0;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<64>(b, roff + 256u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float*, float*) {}
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float*, uint32_t, int) {
        float s = 0.f, t = 0.f;
#pragma unroll
        for (int i = 0; i < 64; i += 2) { s = fmaf(xv[i], qh_bits(r[i]), s); t = fmaf(xv[i + 1], qh_bits(r[i + 1]), t); }
        return s + t;
    }
};
struct FmtF16 {
    static constexpr uint32_t QK = 1, BLK = 2;
    static constexpr int NRAW = 32, NXS = 0;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<32>(b, roff + 128u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float*, float*) {}
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float*, uint32_t, int) {
        float s = 0.f, t = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) { s = fmaf(xv[2 * i], qh_f16_lo(r[i]), s); t = fmaf(xv[2 * i + 1], qh_f16_hi(r[i]), t); }
        return s + t;
    }
};
struct FmtBF16 {
    static constexpr uint32_t QK = 1, BLK = 2;
    static constexpr int NRAW = 32, NXS = 0;
    QH_DEV static int xoff(int u, int c) { return 64 * u + 4 * c; }
    QH_DEV static void load(QhBuf b, uint32_t roff, int u, uint32_t* r) { qh_ldn<32>(b, roff + 128u * (uint32_t)u, r); }
    QH_DEV static void xsums(const float*, float*) {}
    QH_DEV static float dot(const uint32_t* r, const float* xv, const float*, uint32_t, int) {
        float s = 0.f, t = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            s = fmaf(xv[2 * i], qh_bits(r[i] << 16), s);
            t = fmaf(xv[2 * i + 1], qh_bits(r[i] & 0xFFFF0000u), t);
        }
        return s + t;
    }
};
