/*
 * quartz_oracle.c -- CPU restatement of Quartz's quantized GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP library, never
 * part of it: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load liboracle.so.  Nothing under saient_quartz_amd/ links or calls it.
 *
 * Every function follows /root/reference/src/dequant.rs (Quartz) line by line:
 *   - same decode expressions (so dequantized values are bit-identical; every
 *     product of an f16 scale and a <=8-bit integer is exact in f32, the only
 *     rounding is the final "- m" / "+ m" of Q4_K/Q5_K/Q2_K/Q5_1/Q4_1),
 *   - same f32 summation order as the Rust (Rust never contracts a*b+c into an
 *     FMA, so this file is compiled with -ffp-contract=off and no -ffast-math),
 *   - rows computed in parallel (OpenMP), as rayon does: no cross-row reduction,
 *     so results do not depend on the thread count.
 *
 * Q4_0 / Q4_1 (GGML types 2, 3) do not exist in Quartz; they follow the public
 * GGUF block layout only (parity unpinned by the reference, pinned by the
 * closed-form tests in tests/test_oracle.py).
 *
 * Bit-identity of the f32 sums (o_gemv / o_gemm) with the Rust binary: parity
 * unpinned -- rustc is not available to run the reference; the sums are pinned
 * to the float64 dot of the exact dequantized values (relative L2 < 1e-5) and
 * the summation order is restated from the cited lines.
 */
#include "quartz_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "../saient_quartz_amd/csrc/iq_grids.h"

/* ---------------------------------------------------------------- helpers -- */

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }

/* src/dequant.rs:1329-1349 f16_to_f32 (subnormals normalised by a loop, Inf/NaN keep payload) */
float o_f16_to_f32(uint16_t bits) {
    uint32_t sign = bits >> 15, exp = (bits >> 10) & 0x1F, mant = bits & 0x3FF;
    if (exp == 0) {
        if (mant == 0) return bits_f32(sign << 31);
        uint32_t e = 0, m = mant;
        while ((m & 0x400) == 0) { m <<= 1; e += 1; }
        return bits_f32((sign << 31) | ((127 - 15 - e + 1) << 23) | ((m & 0x3FF) << 13));
    }
    if (exp == 31) return bits_f32((sign << 31) | 0x7F800000u | (mant << 13));
    return bits_f32((sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13));
}

/* src/dequant.rs:1471-1480 get_scale_min_k4 */
void o_get_scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* ksigns_iq2xs[i]: the 7 sign bits of i plus an even-parity 8th bit
 * (the closed form of KSIGNS_IQ2XS, src/iq2_tables.rs:9). */
static inline uint8_t ksigns(uint32_t i) {
    return (uint8_t)(i | ((uint32_t)__builtin_parity(i) << 7));
}
/* KMASK_IQ2XS[j] = 1 << j (src/iq2_tables.rs:11) */
#define KMASK(j) (1u << (j))

/* src/gguf.rs:172-191 ggml_type_size (+ Q4_0/Q4_1 from the GGUF layout) */
size_t o_type_size(uint32_t t, size_t n) {
    switch (t) {
        case 0: return n * 4;
        case 1: return n * 2;
        case 2: return (n / 32) * 18;
        case 3: return (n / 32) * 20;
        case 6: return (n / 32) * 22;
        case 7: return (n / 32) * 24;
        case 8: return (n / 32) * 34;
        case 10: return (n / 256) * 84;
        case 12: return (n / 256) * 144;
        case 13: return (n / 256) * 176;
        case 14: return (n / 256) * 210;
        case 16: return (n / 256) * 66;
        case 17: return (n / 256) * 74;
        case 20: return (n / 32) * 18;
        case 21: return (n / 256) * 110;
        case 22: return (n / 256) * 82;
        case 30: return n * 2;
        default: return 0;
    }
}

int o_block_elems(uint32_t t) {
    switch (t) {
        case 0: case 1: case 30: return 1;
        case 2: case 3: case 6: case 7: case 8: case 20: return 32;
        case 10: case 12: case 13: case 14: case 16: case 17: case 21: case 22: return 256;
        default: return 0;
    }
}

/* ------------------------------------------------------------ block codecs -- */
/* Each decodes ONE block into out[QK]. */

/* src/dequant.rs:1450-1463 */
static void blk_q8_0(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b));
    for (int i = 0; i < 32; i++) o[i] = d * (float)(int8_t)b[2 + i];
}

/* src/dequant.rs:1381-1409 */
static void blk_q5_0(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b));
    uint32_t qh = rd32(b + 2);
    const uint8_t* qs = b + 6;
    for (int j = 0; j < 16; j++) {
        uint32_t xh0 = ((qh >> j) << 4) & 0x10;
        uint32_t xh1 = (qh >> (j + 12)) & 0x10;
        int32_t x0 = (int32_t)((qs[j] & 0x0F) | xh0) - 16;
        int32_t x1 = (int32_t)((qs[j] >> 4) | xh1) - 16;
        o[j] = (float)x0 * d;
        o[j + 16] = (float)x1 * d;
    }
}

/* src/dequant.rs:1419-1443 */
static void blk_q5_1(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b)), m = o_f16_to_f32(rd16(b + 2));
    uint32_t qh = rd32(b + 4);
    const uint8_t* qs = b + 8;
    for (int j = 0; j < 16; j++) {
        uint32_t xh0 = ((qh >> j) << 4) & 0x10;
        uint32_t xh1 = (qh >> (j + 12)) & 0x10;
        float x0 = (float)((qs[j] & 0x0F) | xh0);
        float x1 = (float)((qs[j] >> 4) | xh1);
        o[j] = x0 * d + m;
        o[j + 16] = x1 * d + m;
    }
}

/* GGUF Q4_0 layout (absent from Quartz): [d f16][16 B]; v = (q - 8) * d */
static void blk_q4_0(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b));
    const uint8_t* qs = b + 2;
    for (int j = 0; j < 16; j++) {
        o[j] = (float)((int32_t)(qs[j] & 0x0F) - 8) * d;
        o[j + 16] = (float)((int32_t)(qs[j] >> 4) - 8) * d;
    }
}

/* GGUF Q4_1 layout (absent from Quartz): [d f16][m f16][16 B]; v = q * d + m */
static void blk_q4_1(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b)), m = o_f16_to_f32(rd16(b + 2));
    const uint8_t* qs = b + 4;
    for (int j = 0; j < 16; j++) {
        o[j] = (float)(qs[j] & 0x0F) * d + m;
        o[j + 16] = (float)(qs[j] >> 4) * d + m;
    }
}

/* src/dequant.rs:1527-1530, 1557-1574 */
static const float IQ4NL_TABLE[16] = {-127.0f, -104.0f, -83.0f, -65.0f, -49.0f, -35.0f,
                                      -22.0f,  -10.0f,  1.0f,   13.0f,  25.0f,  38.0f,
                                      53.0f,   69.0f,   89.0f,  113.0f};
static void blk_iq4nl(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b));
    const uint8_t* qs = b + 2;
    for (int k = 0; k < 16; k++) {
        o[k] = d * IQ4NL_TABLE[qs[k] & 0x0F];
        o[k + 16] = d * IQ4NL_TABLE[qs[k] >> 4];
    }
}

/* src/dequant.rs:1482-1519 */
static void blk_q4_k(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b)), dmin = o_f16_to_f32(rd16(b + 2));
    const uint8_t* scales = b + 4;
    const uint8_t* qs = b + 16;
    int q_off = 0, is = 0, n = 0;
    for (int it = 0; it < 4; it++) {
        uint8_t sc1, m1b, sc2, m2b;
        o_get_scale_min_k4(is, scales, &sc1, &m1b);
        o_get_scale_min_k4(is + 1, scales, &sc2, &m2b);
        float d1 = d * (float)sc1, m1 = dmin * (float)m1b;
        float d2 = d * (float)sc2, m2 = dmin * (float)m2b;
        for (int l = 0; l < 32; l++) o[n++] = d1 * (float)(qs[q_off + l] & 0x0F) - m1;
        for (int l = 0; l < 32; l++) o[n++] = d2 * (float)(qs[q_off + l] >> 4) - m2;
        q_off += 32;
        is += 2;
    }
}

/* src/dequant.rs:1146-1181 */
static void blk_q5_k(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b)), dmin = o_f16_to_f32(rd16(b + 2));
    const uint8_t* scales = b + 4;
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    int is = 0, n = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int jb = 0; jb < 4; jb++) {
        const uint8_t* ql = qs + jb * 32;
        uint8_t sc1, mm1, sc2, mm2;
        o_get_scale_min_k4(is, scales, &sc1, &mm1);
        float d1 = d * (float)sc1, m1 = dmin * (float)mm1;
        o_get_scale_min_k4(is + 1, scales, &sc2, &mm2);
        float d2 = d * (float)sc2, m2 = dmin * (float)mm2;
        for (int l = 0; l < 32; l++)
            o[n++] = d1 * ((float)(ql[l] & 0xF) + ((qh[l] & u1) ? 16.0f : 0.0f)) - m1;
        for (int l = 0; l < 32; l++)
            o[n++] = d2 * ((float)(ql[l] >> 4) + ((qh[l] & u2) ? 16.0f : 0.0f)) - m2;
        is += 2;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

/* src/dequant.rs:1583-1631 */
static void blk_q6_k(const uint8_t* b, float* o) {
    const uint8_t* ql_base = b;
    const uint8_t* qh_base = b + 128;
    const uint8_t* sc_base = b + 192;
    float d = o_f16_to_f32(rd16(b + 208));
    for (int h = 0; h < 2; h++) {
        const uint8_t* ql = ql_base + 64 * h;
        const uint8_t* qh = qh_base + 32 * h;
        const int8_t* sc = (const int8_t*)(sc_base + 8 * h);
        float* y = o + 128 * h;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l + 0] = d * (float)sc[is + 0] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

/* src/dequant.rs:1113-1144 */
static void blk_q2_k(const uint8_t* b, float* o) {
    const uint8_t* scales = b;
    const uint8_t* qs = b + 16;
    float d = o_f16_to_f32(rd16(b + 80)), dmin = o_f16_to_f32(rd16(b + 82));
    int is = 0, k = 0;
    for (int n = 0; n < 256; n += 128) {
        const uint8_t* q = qs + (n / 128) * 32;
        for (int j = 0; j < 4; j++) {
            int shift = 2 * j;
            uint8_t sc = scales[is++];
            float dl = d * (float)(sc & 0xf), ml = dmin * (float)(sc >> 4);
            for (int l = 0; l < 16; l++) o[k++] = dl * (float)((q[l] >> shift) & 3) - ml;
            sc = scales[is++];
            dl = d * (float)(sc & 0xf);
            ml = dmin * (float)(sc >> 4);
            for (int l = 0; l < 16; l++) o[k++] = dl * (float)((q[l + 16] >> shift) & 3) - ml;
        }
    }
}

/* src/dequant.rs:1011-1041 */
static void blk_iq2_xxs(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b));
    const uint8_t* qs = b + 2;
    int k = 0;
    for (int ib32 = 0; ib32 < 8; ib32++) {
        const uint8_t* a0 = qs + 8 * ib32;
        uint32_t a1 = rd32(qs + 8 * ib32 + 4);
        float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            uint64_t g = qh_iq2xxs_grid[a0[l]];
            uint8_t signs = ksigns((a1 >> (7 * l)) & 127);
            for (int j = 0; j < 8; j++) {
                float s = (signs & KMASK(j)) ? -1.0f : 1.0f;
                o[k++] = db * (float)(int8_t)(g >> (8 * j)) * s;
            }
        }
    }
}

/* src/dequant.rs:1043-1075 */
static void blk_iq2_xs(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b));
    const uint8_t* qs = b + 2;
    const uint8_t* scales = b + 66;
    int k = 0;
    for (int ib32 = 0; ib32 < 8; ib32++) {
        float db0 = d * (0.5f + (float)(scales[ib32] & 0xf)) * 0.25f;
        float db1 = d * (0.5f + (float)(scales[ib32] >> 4)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            uint16_t q = rd16(qs + 2 * (4 * ib32 + l));
            uint64_t g = qh_iq2xs_grid[q & 511];
            uint8_t signs = ksigns(q >> 9);
            float db = l < 2 ? db0 : db1;
            for (int j = 0; j < 8; j++) {
                float s = (signs & KMASK(j)) ? -1.0f : 1.0f;
                o[k++] = db * (float)(int8_t)(g >> (8 * j)) * s;
            }
        }
    }
}

/* src/dequant.rs:1077-1110 */
static void blk_iq2_s(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b));
    const uint8_t* qs = b + 2;
    const uint8_t* qh = b + 66;
    const uint8_t* scales = b + 74;
    int k = 0;
    for (int ib32 = 0; ib32 < 8; ib32++) {
        float db0 = d * (0.5f + (float)(scales[ib32] & 0xf)) * 0.25f;
        float db1 = d * (0.5f + (float)(scales[ib32] >> 4)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            float db = l < 2 ? db0 : db1;
            uint32_t idx = qs[4 * ib32 + l] | (((uint32_t)qh[ib32] << (8 - 2 * l)) & 0x300);
            uint64_t g = qh_iq2s_grid[idx];
            uint8_t signs = qs[32 + 4 * ib32 + l];
            for (int j = 0; j < 8; j++) {
                float s = (signs & KMASK(j)) ? -1.0f : 1.0f;
                o[k++] = db * (float)(int8_t)(g >> (8 * j)) * s;
            }
        }
    }
}

/* src/dequant.rs:1184-1237 */
static void blk_iq3_s(const uint8_t* b, float* o) {
    float d = o_f16_to_f32(rd16(b));
    const uint8_t* qs = b + 2;
    const uint8_t* qh = b + 66;
    const uint8_t* sg = b + 74;
    const uint8_t* scales = b + 106;
    int qo = 0, so = 0, ho = 0, k = 0;
    for (int ib32 = 0; ib32 < 8; ib32 += 2) {
        float db1 = d * (1.0f + 2.0f * (float)(scales[ib32 / 2] & 0xf));
        float db2 = d * (1.0f + 2.0f * (float)(scales[ib32 / 2] >> 4));
        for (int half = 0; half < 2; half++) {
            float db = half ? db2 : db1;
            uint32_t qhb = qh[ho + half];
            int qbase = qo + half * 8, sbase = so + half * 4;
            for (int l = 0; l < 4; l++) {
                uint32_t i0 = qs[qbase + 2 * l] | ((qhb << (8 - 2 * l)) & 256);
                uint32_t i1 = qs[qbase + 2 * l + 1] | ((qhb << (7 - 2 * l)) & 256);
                uint32_t g1 = qh_iq3s_grid[i0], g2 = qh_iq3s_grid[i1];
                uint8_t s = sg[sbase + l];
                for (int j = 0; j < 4; j++)
                    o[k++] = db * (float)(int8_t)(g1 >> (8 * j)) * ((s & KMASK(j)) ? -1.0f : 1.0f);
                for (int j = 0; j < 4; j++)
                    o[k++] = db * (float)(int8_t)(g2 >> (8 * j)) * ((s & KMASK(j + 4)) ? -1.0f : 1.0f);
            }
        }
        qo += 16;
        so += 8;
        ho += 2;
    }
}

typedef void (*blk_fn)(const uint8_t*, float*);

static blk_fn block_decoder(uint32_t t) {
    switch (t) {
        case 2: return blk_q4_0;
        case 3: return blk_q4_1;
        case 6: return blk_q5_0;
        case 7: return blk_q5_1;
        case 8: return blk_q8_0;
        case 10: return blk_q2_k;
        case 12: return blk_q4_k;
        case 13: return blk_q5_k;
        case 14: return blk_q6_k;
        case 16: return blk_iq2_xxs;
        case 17: return blk_iq2_xs;
        case 20: return blk_iq4nl;
        case 21: return blk_iq3_s;
        case 22: return blk_iq2_s;
        default: return NULL;
    }
}

/* src/dequant.rs:1239-1258 dequant (+ :1321-1371 f32/f16/bf16).  n must be a
 * multiple of the block size (the Rust drops a trailing partial block). */
int o_dequant(uint32_t t, const uint8_t* data, size_t n, float* out) {
    if (t == 0) { for (size_t i = 0; i < n; i++) out[i] = bits_f32(rd32(data + 4 * i)); return 0; }
    if (t == 1) { for (size_t i = 0; i < n; i++) out[i] = o_f16_to_f32(rd16(data + 2 * i)); return 0; }
    if (t == 30) { for (size_t i = 0; i < n; i++) out[i] = bits_f32((uint32_t)rd16(data + 2 * i) << 16); return 0; }
    blk_fn f = block_decoder(t);
    if (!f) return -1;
    int qk = o_block_elems(t);
    size_t bsz = o_type_size(t, (size_t)qk);
    size_t nb = n / (size_t)qk;
#pragma omp parallel for schedule(static) if (nb > 4096)
    for (size_t b = 0; b < nb; b++) f(data + b * bsz, out + b * qk);
    return 0;
}

/* ------------------------------------------------------------ fused rows -- */

/* src/dequant.rs:659-706 q4k_row: per sub-block sq=Σx·q, sx=Σx, acc += d1*sq - m1*sx */
static float row_q4_k(const float* x, const uint8_t* row, int bpr) {
    float acc = 0.0f;
    for (int b = 0; b < bpr; b++) {
        const uint8_t* blk = row + (size_t)b * 144;
        float d = o_f16_to_f32(rd16(blk)), dmin = o_f16_to_f32(rd16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        const float* xb = x + (size_t)b * 256;
        int q_off = 0, is = 0, o = 0;
        for (int it = 0; it < 4; it++) {
            uint8_t sc1, mb1, sc2, mb2;
            o_get_scale_min_k4(is, scales, &sc1, &mb1);
            o_get_scale_min_k4(is + 1, scales, &sc2, &mb2);
            float d1 = d * (float)sc1, m1 = dmin * (float)mb1;
            float d2 = d * (float)sc2, m2 = dmin * (float)mb2;
            float sq1 = 0.0f, sx1 = 0.0f;
            for (int l = 0; l < 32; l++) {
                float xv = xb[o + l];
                sq1 += xv * (float)(qs[q_off + l] & 0x0F);
                sx1 += xv;
            }
            acc += d1 * sq1 - m1 * sx1;
            o += 32;
            float sq2 = 0.0f, sx2 = 0.0f;
            for (int l = 0; l < 32; l++) {
                float xv = xb[o + l];
                sq2 += xv * (float)(qs[q_off + l] >> 4);
                sx2 += xv;
            }
            acc += d2 * sq2 - m2 * sx2;
            o += 32;
            q_off += 32;
            is += 2;
        }
    }
    return acc;
}

/* src/dequant.rs:710-752 q6k_row: decode the block, then acc += xb[i]*y[i] over the row */
static float row_q6_k(const float* x, const uint8_t* row, int bpr) {
    float acc = 0.0f, y[256];
    for (int b = 0; b < bpr; b++) {
        blk_q6_k(row + (size_t)b * 210, y);
        const float* xb = x + (size_t)b * 256;
        for (int i = 0; i < 256; i++) acc += xb[i] * y[i];
    }
    return acc;
}

/* src/dequant.rs:916-944 gemv_q5_1 row: acc += x[k]*(q0*d+m) + x[k+16]*(q1*d+m) */
static float row_q5_1(const float* x, const uint8_t* row, int bpr) {
    float acc = 0.0f;
    for (int b = 0; b < bpr; b++) {
        const uint8_t* blk = row + (size_t)b * 24;
        float d = o_f16_to_f32(rd16(blk)), m = o_f16_to_f32(rd16(blk + 2));
        uint32_t qh = rd32(blk + 4);
        const uint8_t* qs = blk + 8;
        const float* xi = x + (size_t)b * 32;
        for (int k = 0; k < 16; k++) {
            uint32_t xh0 = ((qh >> k) << 4) & 0x10;
            uint32_t xh1 = (qh >> (k + 12)) & 0x10;
            float q0 = (float)((qs[k] & 0x0F) | xh0);
            float q1 = (float)((qs[k] >> 4) | xh1);
            acc += xi[k] * (q0 * d + m) + xi[k + 16] * (q1 * d + m);
        }
    }
    return acc;
}

/* src/dequant.rs:1532-1555 gemv_iq4nl row: acc += x*d*T[lo]; acc += x*d*T[hi] */
static float row_iq4nl(const float* x, const uint8_t* row, int bpr) {
    float acc = 0.0f;
    for (int b = 0; b < bpr; b++) {
        const uint8_t* blk = row + (size_t)b * 18;
        float d = o_f16_to_f32(rd16(blk));
        const uint8_t* qs = blk + 2;
        const float* xi = x + (size_t)b * 32;
        for (int k = 0; k < 16; k++) {
            acc += xi[k] * d * IQ4NL_TABLE[qs[k] & 0x0F];
            acc += xi[k + 16] * d * IQ4NL_TABLE[qs[k] >> 4];
        }
    }
    return acc;
}

/* src/dequant.rs:946-962 gemv_bf16 row: Σ x*w via iterator sum (fold from -0.0) */
static float row_bf16(const float* x, const uint8_t* row, int in_dim) {
    float acc = -0.0f;
    for (int k = 0; k < in_dim; k++) acc += x[k] * bits_f32((uint32_t)rd16(row + 2 * k) << 16);
    return acc;
}

/* src/dequant.rs:964-981 gemv_f32_data row */
static float row_f32(const float* x, const uint8_t* row, int in_dim) {
    float acc = -0.0f;
    for (int k = 0; k < in_dim; k++) acc += x[k] * bits_f32(rd32(row + 4 * k));
    return acc;
}

/* src/main.rs:710-718 matmul row over a dequantized row: zip-map-sum (fold from -0.0) */
static float row_dot_iter(const float* x, const float* w, int in_dim) {
    float acc = -0.0f;
    for (int k = 0; k < in_dim; k++) acc += x[k] * w[k];
    return acc;
}

/* src/dequant.rs:617-623 dot (explicit 0.0 start, used by gemm's generic arm) */
static float row_dot(const float* a, const float* b, int n) {
    float s = 0.0f;
    for (int k = 0; k < n; k++) s += a[k] * b[k];
    return s;
}

static int dims_ok(uint32_t t, int in_dim, int out_dim) {
    int qk = o_block_elems(t);
    if (qk == 0) return -1;
    if (in_dim <= 0 || out_dim < 0 || in_dim % qk) return -2;
    return 0;
}

/* src/dequant.rs:18-31 gemv dispatch.  Types 7/12/14/20/30/0 use the fused rows;
 * every other type takes the `_` arm: dequantize W, then crate::matmul
 * (src/main.rs:710-718).  Dequantizing row by row gives the same values as the
 * whole-matrix dequant (blocks are independent); the sum order is unchanged. */
int o_gemv(uint32_t t, const float* x, const uint8_t* data, int in_dim, int out_dim, float* y) {
    int rc = dims_ok(t, in_dim, out_dim);
    if (rc) return rc;
    size_t rb = o_type_size(t, (size_t)in_dim);
    int qk = o_block_elems(t);
    int bpr = in_dim / qk;
    switch (t) {
        case 7: case 12: case 14: case 20: case 30: case 0: {
#pragma omp parallel for schedule(static)
            for (int j = 0; j < out_dim; j++) {
                const uint8_t* row = data + (size_t)j * rb;
                float v;
                if (t == 7) v = row_q5_1(x, row, bpr);
                else if (t == 12) v = row_q4_k(x, row, bpr);
                else if (t == 14) v = row_q6_k(x, row, bpr);
                else if (t == 20) v = row_iq4nl(x, row, bpr);
                else if (t == 30) v = row_bf16(x, row, in_dim);
                else v = row_f32(x, row, in_dim);
                y[j] = v;
            }
            return 0;
        }
        default: {
            int err = 0;
#pragma omp parallel
            {
                float* w = (float*)malloc(sizeof(float) * (size_t)in_dim);
                if (!w) {
#pragma omp atomic write
                    err = -3;
                }
#pragma omp for schedule(static)
                for (int j = 0; j < out_dim; j++) {
                    if (!w) continue;
                    o_dequant(t, data + (size_t)j * rb, (size_t)in_dim, w);
                    y[j] = row_dot_iter(x, w, in_dim);
                }
                free(w);
            }
            return err;
        }
    }
}

/* The `_` arm of src/dequant.rs:26-29 as the reference runs it: dequant() of
 * the WHOLE matrix into one f32 buffer (src/dequant.rs:1239-1258, w here,
 * out_dim * in_dim floats, caller-owned), then crate::matmul's row-parallel
 * zip-map-sum (src/main.rs:710-718).  Same values and sum order as o_gemv's
 * row-by-row form; timed as the CPU baseline of the types that take this arm. */
int o_gemv_dequant_matmul(uint32_t t, const float* x, const uint8_t* data, int in_dim, int out_dim, float* w,
                          float* y) {
    int rc = dims_ok(t, in_dim, out_dim);
    if (rc) return rc;
    size_t rb = o_type_size(t, (size_t)in_dim);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < out_dim; j++) o_dequant(t, data + (size_t)j * rb, (size_t)in_dim, w + (size_t)j * in_dim);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < out_dim; j++) y[j] = row_dot_iter(x, w + (size_t)j * in_dim, in_dim);
    return 0;
}

/* src/dequant.rs:38-77 q4k_row_batched / :81-122 q6k_row_batched: decode each
 * superblock once into wv[256], then acc[t] += Σ_i xt[i]*wv[i] (s from 0.0). */
static void rowb_k(uint32_t t, const float* x, int in_dim, int n, const uint8_t* row, float* acc) {
    int bpr = in_dim / 256;
    size_t bsz = t == 12 ? 144 : 210;
    float wv[256];
    for (int b = 0; b < bpr; b++) {
        if (t == 12) blk_q4_k(row + b * bsz, wv);
        else blk_q6_k(row + b * bsz, wv);
        size_t base = (size_t)b * 256;
        for (int tk = 0; tk < n; tk++) {
            const float* xt = x + (size_t)tk * in_dim + base;
            float s = 0.0f;
            for (int i = 0; i < 256; i++) s += xt[i] * wv[i];
            acc[tk] += s;
        }
    }
}

/* src/dequant.rs:143-200 gemm: X [n, in] token-major -> Y [n, out] token-major. */
int o_gemm(uint32_t t, const float* x, const uint8_t* data, int in_dim, int out_dim, int n, float* y) {
    if (n == 1) return o_gemv(t, x, data, in_dim, out_dim, y);
    int rc = dims_ok(t, in_dim, out_dim);
    if (rc) return rc;
    if (n <= 0) return -2;
    size_t rb = o_type_size(t, (size_t)in_dim);
    int err = 0;
#pragma omp parallel
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)n);
        float* w = (float*)malloc(sizeof(float) * (size_t)in_dim);
        if (!acc || !w) {
#pragma omp atomic write
            err = -3;
        }
#pragma omp for schedule(static)
        for (int j = 0; j < out_dim; j++) {
            if (!acc || !w) continue;
            const uint8_t* row = data + (size_t)j * rb;
            for (int tk = 0; tk < n; tk++) acc[tk] = 0.0f;
            if (t == 12 || t == 14) {
                rowb_k(t, x, in_dim, n, row, acc);
            } else {
                o_dequant(t, row, (size_t)in_dim, w);
                for (int tk = 0; tk < n; tk++) acc[tk] = row_dot(x + (size_t)tk * in_dim, w, in_dim);
            }
            for (int tk = 0; tk < n; tk++) y[(size_t)tk * out_dim + j] = acc[tk];
        }
        free(acc);
        free(w);
    }
    return err;
}

/* Threads used by the parallel loops (omp_set_num_threads wrapper). */
#ifdef _OPENMP
#include <omp.h>
void o_set_threads(int n) { if (n > 0) omp_set_num_threads(n); }
int o_get_threads(void) { return omp_get_max_threads(); }
#else
void o_set_threads(int n) { (void)n; }
int o_get_threads(void) { return 1; }
#endif

const char* o_grid_sha256(int which) {
    switch (which) {
        case 0: return QH_IQ2XXS_GRID_SHA256;
        case 1: return QH_IQ2XS_GRID_SHA256;
        case 2: return QH_IQ2S_GRID_SHA256;
        case 3: return QH_IQ3S_GRID_SHA256;
        default: return "";
    }
}

/* ------------------------------------------------ Q8_1 MMQ arithmetic mode -- */
/* The reference's CPU oracles of ggml-cuda's int8 MMQ path (src/dequant.rs:
 * 202-645): activations quantised to Q8_1 per 32 values, f16-rounded scales,
 * integer dots, f32 accumulation with explicit mul_add (fmaf here) in block /
 * group order, optional stream-K split of the accumulation. */

/* f32_to_f16_round_to_even (src/dequant.rs:604-645), restated. */
uint16_t o_f32_to_f16_rne(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const int exponent = (int)((bits >> 23) & 0xffu);
    const uint32_t mantissa = bits & 0x7fffffu;
    if (exponent == 0xff) return (uint16_t)(sign | (mantissa == 0 ? 0x7c00u : 0x7e00u));
    const int half_exponent = exponent - 127 + 15;
    if (half_exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    if (half_exponent <= 0) {
        if (half_exponent < -10) return sign;
        const uint32_t significand = mantissa | 0x800000u;
        const uint32_t shift = (uint32_t)(14 - half_exponent);
        uint32_t rounded = significand >> shift;
        const uint32_t remainder = significand & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        if (remainder > halfway || (remainder == halfway && (rounded & 1u))) rounded++;
        return (uint16_t)(sign | rounded);
    }
    uint32_t rounded = mantissa >> 13;
    const uint32_t remainder = mantissa & 0x1fffu;
    if (remainder > 0x1000u || (remainder == 0x1000u && (rounded & 1u))) rounded++;
    if (rounded == 0x400u) {
        const int e = half_exponent + 1;
        return (uint16_t)(sign | (e >= 31 ? 0x7c00u : (uint32_t)e << 10));
    }
    return (uint16_t)(sign | ((uint32_t)half_exponent << 10) | rounded);
}

static inline float round_to_f16(float v) { return o_f16_to_f32(o_f32_to_f16_rne(v)); } /* :600-602 */

/* quantize_q8_1_mmq (src/dequant.rs:515-556) and _d4 (:558-598): per 32 values,
 * partial max / sum over 8 lanes of 4, combined in XOR order 4, 2, 1; q =
 * round(x * 127/max) (half away from zero); scale 1/(127/max), rounded to f16
 * unless d4; sum f16-rounded (d4: 0). */
void o_quantize_q8_1_mmq(const float* x, int in_dim, int rows, int d4, int8_t* values, float* scale, float* sum) {
    const int nb = in_dim / 32;
    for (int row = 0; row < rows; row++)
        for (int b = 0; b < nb; b++) {
            const float* grp = x + (size_t)row * in_dim + 32 * b;
            float pm[8], ps[8];
            for (int lane = 0; lane < 8; lane++) {
                const float* v = grp + 4 * lane;
                float m = 0.0f;
                for (int i = 0; i < 4; i++) m = fmaxf(m, fabsf(v[i]));
                pm[lane] = m;
                ps[lane] = ((v[0] + v[1]) + v[2]) + v[3];
            }
            static const int offs[3] = {4, 2, 1};
            for (int o = 0; o < 3; o++) {
                float om[8], os[8];
                memcpy(om, pm, sizeof om);
                memcpy(os, ps, sizeof os);
                for (int lane = 0; lane < 8; lane++) {
                    pm[lane] = fmaxf(om[lane], om[lane ^ offs[o]]);
                    ps[lane] = os[lane] + os[lane ^ offs[o]];
                }
            }
            const float maximum = pm[0];
            const float inv = maximum == 0.0f ? 0.0f : 127.0f / maximum;
            int8_t* q = values + ((size_t)row * nb + b) * 32;
            for (int i = 0; i < 32; i++) {
                if (inv != 0.0f) {
                    float r = roundf(grp[i] * inv);
                    r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);  /* `as i8` saturates */
                    q[i] = (int8_t)r;
                } else {
                    q[i] = 0;
                }
            }
            const float sc = inv == 0.0f ? 0.0f : 1.0f / inv;
            scale[(size_t)row * nb + b] = d4 ? sc : round_to_f16(sc);
            sum[(size_t)row * nb + b] = d4 ? 0.0f : round_to_f16(ps[0]);
        }
}

/* cuda_stream_k_cut (src/dequant.rs:338-374): the superblock at which ggml-cuda's
 * stream-K partition splits output (row, column)'s accumulation, or -1. */
int o_stream_k_cut(int row, int column, int in_dim, int out_dim, int reference_rows, int multiprocessors) {
    const long MMQ_X = 128, MMQ_Y = 128, VPK = 256;
    if (multiprocessors == 0 || in_dim % VPK != 0) return -1;
    const long blocks_per_tile = in_dim / VPK;
    const long tiles_x = (reference_rows + MMQ_X - 1) / MMQ_X;
    const long tiles_y = (out_dim + MMQ_Y - 1) / MMQ_Y;
    const long tile_count = tiles_x * tiles_y;
    const long waves = (tile_count + multiprocessors - 1) / multiprocessors;
    const long efficiency = 100 * tile_count / (multiprocessors * waves);
    const long grid = efficiency >= 90 ? tile_count : multiprocessors;
    if (grid == 0 || tile_count % grid == 0) return -1;
    const long tile = (column / MMQ_Y) * tiles_x + row / MMQ_X;
    const long tile_start = tile * blocks_per_tile, tile_end = tile_start + blocks_per_tile;
    const long total = tile_count * blocks_per_tile;
    for (long block = 1; block < grid; block++) {
        const long boundary = block * total / grid;
        if (boundary > tile_start && boundary < tile_end) return (int)(boundary - tile_start);
    }
    return -1;
}

/* gemm_q4k_q8_1_mmq[_stream_k] (src/dequant.rs:216-336) and
 * gemm_q6k_q8_1_mmq[_stream_k] (:377-513).  x [rows][in_dim], y [rows][out_dim];
 * reference_rows = 0: no stream-K split. */
int o_gemm_q8_1_mmq(uint32_t ggml_type, const float* x, const uint8_t* data, int in_dim, int out_dim, int rows,
                    int reference_rows, int multiprocessors, float* y) {
    if ((ggml_type != 12 && ggml_type != 14) || in_dim % 256 || rows < 0 || out_dim < 0) return -1;
    const int q6 = ggml_type == 14;
    const int nb8 = in_dim / 32, nsb = in_dim / 256;
    const size_t bb = q6 ? 210 : 144;
    int8_t* qv = malloc((size_t)rows * in_dim + 1);
    float* qs = malloc(((size_t)rows * nb8 + 1) * sizeof(float));
    float* qm = malloc(((size_t)rows * nb8 + 1) * sizeof(float));
    if (!qv || !qs || !qm) { free(qv); free(qs); free(qm); return -2; }
    o_quantize_q8_1_mmq(x, in_dim, rows, q6, qv, qs, qm);
#pragma omp parallel for schedule(static)
    for (int column = 0; column < out_dim; column++) {
        const uint8_t* wrow = data + (size_t)column * nsb * bb;
        for (int row = 0; row < rows; row++) {
            float acc = 0.0f, prefix = 0.0f;
            const int cut = reference_rows > 0
                                ? o_stream_k_cut(row, column, in_dim, out_dim, reference_rows, multiprocessors)
                                : -1;
            for (int b = 0; b < nsb; b++) {
                if (b == cut) { prefix = acc; acc = 0.0f; }
                const uint8_t* blk = wrow + (size_t)b * bb;
                const size_t a0 = (size_t)row * nb8 + (size_t)b * 8;
                if (!q6) {
                    const float d = o_f16_to_f32(rd16(blk)), dmin = o_f16_to_f32(rd16(blk + 2));
                    for (int g = 0; g < 8; g++) {
                        uint8_t sc, m;
                        o_get_scale_min_k4(g, blk + 4, &sc, &m);
                        const float cs = round_to_f16(d * (float)sc);
                        const float cm = round_to_f16(-dmin * (float)m);
                        const int8_t* av = qv + (a0 + g) * 32;
                        const uint8_t* qq = blk + 16 + (g / 2) * 32;
                        int dot = 0;
                        for (int i = 0; i < 32; i++) {
                            const int w = (g & 1) ? (qq[i] >> 4) : (qq[i] & 0x0f);
                            dot += w * av[i];
                        }
                        const float ds = cs * qs[a0 + g];
                        acc = fmaf(ds, (float)dot, acc);
                        acc = fmaf(cm, qm[a0 + g], acc);
                    }
                } else {
                    int8_t q[256];
                    for (int half = 0; half < 2; half++)
                        for (int i = 0; i < 32; i++) {
                            const uint8_t l0 = blk[64 * half + i], l1 = blk[64 * half + i + 32];
                            const uint8_t h = blk[128 + 32 * half + i];
                            q[128 * half + i] = (int8_t)(((l0 & 0x0f) | ((h & 0x03) << 4)) - 32);
                            q[128 * half + i + 32] = (int8_t)(((l1 & 0x0f) | (((h >> 2) & 0x03) << 4)) - 32);
                            q[128 * half + i + 64] = (int8_t)(((l0 >> 4) | (((h >> 4) & 0x03) << 4)) - 32);
                            q[128 * half + i + 96] = (int8_t)(((l1 >> 4) | (((h >> 6) & 0x03) << 4)) - 32);
                        }
                    const float d6 = o_f16_to_f32(rd16(blk + 208));
                    for (int f = 0; f < 2; f++) {
                        float fs = 0.0f;
                        for (int g = 4 * f; g < 4 * f + 4; g++) {
                            const int8_t* av = qv + (a0 + g) * 32;
                            int d1 = 0, d2 = 0;
                            for (int i = 0; i < 16; i++) {
                                d1 += q[32 * g + i] * av[i];
                                d2 += q[32 * g + i + 16] * av[i + 16];
                            }
                            const int s1 = (int8_t)blk[192 + 2 * g], s2 = (int8_t)blk[192 + 2 * g + 1];
                            fs = fmaf(qs[a0 + g], (float)(s1 * d1 + s2 * d2), fs);
                        }
                        acc = fmaf(d6, fs, acc);
                    }
                }
            }
            if (cut >= 0) acc = acc + prefix;  /* tail + prefix, ggml's fixup order */
            y[(size_t)row * out_dim + column] = acc;
        }
    }
    free(qv);
    free(qs);
    free(qm);
    return 0;
}
