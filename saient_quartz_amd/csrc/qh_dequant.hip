// qh_dequant.hip -- bit-exact GGUF block decode on the GPU (hip_dequant).
//
// Each function restates the matching dequant_* of src/dequant.rs with the same
// f32 operations in the same order (contraction disabled), so every decoded value
// is bit-identical to Quartz's CPU decode.  The IQ codebooks live here as
// device globals initialised from iq_grids.h.
#define QH_GRIDS_NO_STATIC
#include "iq_grids.h"
#include "qh_formats.h"
#include "qh_internal.h"

__device__ uint64_t qh_g_iq2xxs[256] = {QH_IQ2XXS_GRID_VALUES};
__device__ uint64_t qh_g_iq2xs[512] = {QH_IQ2XS_GRID_VALUES};
__device__ uint64_t qh_g_iq2s[1024] = {QH_IQ2S_GRID_VALUES};
__device__ uint32_t qh_g_iq3s[512] = {QH_IQ3S_GRID_VALUES};

#pragma clang fp contract(off)

QH_DEV uint32_t qh_rd16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
QH_DEV uint32_t qh_rd32(const uint8_t* p) { return qh_rd16(p) | (qh_rd16(p + 2) << 16); }

QH_DEV void qh_gsm_k4(int j, const uint8_t* s, uint32_t& sc, uint32_t& m) {  // src/dequant.rs:1471-1480
    if (j < 4) {
        sc = s[j] & 63u;
        m = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 0x0Fu) | ((uint32_t)(s[j - 4] >> 6) << 4);
        m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
}

__device__ void qh_decode_block(uint32_t t, const uint8_t* b, float* o) {
    switch (t) {
        case QT_F32: o[0] = qh_bits(qh_rd32(b)); return;
        case QT_F16: o[0] = qh_f16(qh_rd16(b)); return;
        case QT_BF16: o[0] = qh_bits(qh_rd16(b) << 16); return;
        case QT_Q8_0: {  // :1450-1463
            const float d = qh_f16(qh_rd16(b));
            for (int i = 0; i < 32; i++) o[i] = d * (float)(int8_t)b[2 + i];
            return;
        }
        case QT_Q5_0: {  // :1381-1409
            const float d = qh_f16(qh_rd16(b));
            const uint32_t qh = qh_rd32(b + 2);
            for (int j = 0; j < 16; j++) {
                const uint32_t xh0 = ((qh >> j) << 4) & 0x10u, xh1 = (qh >> (j + 12)) & 0x10u;
                o[j] = (float)((int32_t)((b[6 + j] & 0x0Fu) | xh0) - 16) * d;
                o[j + 16] = (float)((int32_t)((uint32_t)(b[6 + j] >> 4) | xh1) - 16) * d;
            }
            return;
        }
        case QT_Q5_1: {  // :1419-1443
            const float d = qh_f16(qh_rd16(b)), m = qh_f16(qh_rd16(b + 2));
            const uint32_t qh = qh_rd32(b + 4);
            for (int j = 0; j < 16; j++) {
                const uint32_t xh0 = ((qh >> j) << 4) & 0x10u, xh1 = (qh >> (j + 12)) & 0x10u;
                o[j] = (float)((b[8 + j] & 0x0Fu) | xh0) * d + m;
                o[j + 16] = (float)((uint32_t)(b[8 + j] >> 4) | xh1) * d + m;
            }
            return;
        }
        case QT_Q4_0: {  // GGUF layout
            const float d = qh_f16(qh_rd16(b));
            for (int j = 0; j < 16; j++) {
                o[j] = (float)((int32_t)(b[2 + j] & 0x0Fu) - 8) * d;
                o[j + 16] = (float)((int32_t)(b[2 + j] >> 4) - 8) * d;
            }
            return;
        }
        case QT_Q4_1: {  // GGUF layout
            const float d = qh_f16(qh_rd16(b)), m = qh_f16(qh_rd16(b + 2));
            for (int j = 0; j < 16; j++) {
                o[j] = (float)(b[4 + j] & 0x0Fu) * d + m;
                o[j + 16] = (float)(b[4 + j] >> 4) * d + m;
            }
            return;
        }
        case QT_IQ4_NL: {  // :1557-1574
            const float T[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                 1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};
            const float d = qh_f16(qh_rd16(b));
            for (int k = 0; k < 16; k++) {
                o[k] = d * T[b[2 + k] & 0x0F];
                o[k + 16] = d * T[b[2 + k] >> 4];
            }
            return;
        }
        case QT_Q4_K: {  // :1482-1519
            const float d = qh_f16(qh_rd16(b)), dmin = qh_f16(qh_rd16(b + 2));
            const uint8_t* sc = b + 4;
            const uint8_t* qs = b + 16;
            for (int it = 0; it < 4; it++) {
                uint32_t s1, mb1, s2, mb2;
                qh_gsm_k4(2 * it, sc, s1, mb1);
                qh_gsm_k4(2 * it + 1, sc, s2, mb2);
                const float d1 = d * (float)s1, m1 = dmin * (float)mb1;
                const float d2 = d * (float)s2, m2 = dmin * (float)mb2;
                for (int l = 0; l < 32; l++) o[64 * it + l] = d1 * (float)(qs[32 * it + l] & 0x0F) - m1;
                for (int l = 0; l < 32; l++) o[64 * it + 32 + l] = d2 * (float)(qs[32 * it + l] >> 4) - m2;
            }
            return;
        }
        case QT_Q5_K: {  // :1146-1181
            const float d = qh_f16(qh_rd16(b)), dmin = qh_f16(qh_rd16(b + 2));
            const uint8_t* sc = b + 4;
            const uint8_t* qh = b + 16;
            const uint8_t* qs = b + 48;
            uint32_t u1 = 1, u2 = 2;
            for (int jb = 0; jb < 4; jb++) {
                const uint8_t* ql = qs + 32 * jb;
                uint32_t s1, mm1, s2, mm2;
                qh_gsm_k4(2 * jb, sc, s1, mm1);
                const float d1 = d * (float)s1, m1 = dmin * (float)mm1;
                qh_gsm_k4(2 * jb + 1, sc, s2, mm2);
                const float d2 = d * (float)s2, m2 = dmin * (float)mm2;
                for (int l = 0; l < 32; l++)
                    o[64 * jb + l] = d1 * ((float)(ql[l] & 0xF) + ((qh[l] & u1) ? 16.0f : 0.0f)) - m1;
                for (int l = 0; l < 32; l++)
                    o[64 * jb + 32 + l] = d2 * ((float)(ql[l] >> 4) + ((qh[l] & u2) ? 16.0f : 0.0f)) - m2;
                u1 <<= 2;
                u2 <<= 2;
            }
            return;
        }
        case QT_Q6_K: {  // :1583-1631
            const float d = qh_f16(qh_rd16(b + 208));
            for (int h = 0; h < 2; h++) {
                const uint8_t* ql = b + 64 * h;
                const uint8_t* qh = b + 128 + 32 * h;
                const int8_t* sc = (const int8_t*)(b + 192 + 8 * h);
                float* y = o + 128 * h;
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const int q1 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l] = d * (float)sc[is] * (float)q1;
                    y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    y[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
            return;
        }
        case QT_Q2_K: {  // :1113-1144
            const uint8_t* scales = b;
            const uint8_t* qs = b + 16;
            const float d = qh_f16(qh_rd16(b + 80)), dmin = qh_f16(qh_rd16(b + 82));
            int is = 0, k = 0;
            for (int n = 0; n < 2; n++) {
                const uint8_t* q = qs + 32 * n;
                for (int j = 0; j < 4; j++) {
                    const int shift = 2 * j;
                    uint32_t sc = scales[is++];
                    float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                    for (int l = 0; l < 16; l++) o[k++] = dl * (float)((q[l] >> shift) & 3) - ml;
                    sc = scales[is++];
                    dl = d * (float)(sc & 0xF);
                    ml = dmin * (float)(sc >> 4);
                    for (int l = 0; l < 16; l++) o[k++] = dl * (float)((q[l + 16] >> shift) & 3) - ml;
                }
            }
            return;
        }
        case QT_IQ2_XXS: {  // :1011-1041
            const float d = qh_f16(qh_rd16(b));
            const uint8_t* qs = b + 2;
            int k = 0;
            for (int ib32 = 0; ib32 < 8; ib32++) {
                const uint32_t a1 = qh_rd32(qs + 8 * ib32 + 4);
                const float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
                for (int l = 0; l < 4; l++) {
                    const uint64_t g = qh_g_iq2xxs[qs[8 * ib32 + l]];
                    const uint32_t signs = qh_ksigns((a1 >> (7 * l)) & 127u);
                    for (int j = 0; j < 8; j++) {
                        const float s = (signs & (1u << j)) ? -1.0f : 1.0f;
                        o[k++] = db * (float)(int8_t)(g >> (8 * j)) * s;
                    }
                }
            }
            return;
        }
        case QT_IQ2_XS: {  // :1043-1075
            const float d = qh_f16(qh_rd16(b));
            const uint8_t* qs = b + 2;
            const uint8_t* scales = b + 66;
            int k = 0;
            for (int ib32 = 0; ib32 < 8; ib32++) {
                const float db0 = d * (0.5f + (float)(scales[ib32] & 0xF)) * 0.25f;
                const float db1 = d * (0.5f + (float)(scales[ib32] >> 4)) * 0.25f;
                for (int l = 0; l < 4; l++) {
                    const uint32_t q = qh_rd16(qs + 2 * (4 * ib32 + l));
                    const uint64_t g = qh_g_iq2xs[q & 511u];
                    const uint32_t signs = qh_ksigns(q >> 9);
                    const float db = l < 2 ? db0 : db1;
                    for (int j = 0; j < 8; j++) {
                        const float s = (signs & (1u << j)) ? -1.0f : 1.0f;
                        o[k++] = db * (float)(int8_t)(g >> (8 * j)) * s;
                    }
                }
            }
            return;
        }
        case QT_IQ2_S: {  // :1077-1110
            const float d = qh_f16(qh_rd16(b));
            const uint8_t* qs = b + 2;
            const uint8_t* qh = b + 66;
            const uint8_t* scales = b + 74;
            int k = 0;
            for (int ib32 = 0; ib32 < 8; ib32++) {
                const float db0 = d * (0.5f + (float)(scales[ib32] & 0xF)) * 0.25f;
                const float db1 = d * (0.5f + (float)(scales[ib32] >> 4)) * 0.25f;
                for (int l = 0; l < 4; l++) {
                    const float db = l < 2 ? db0 : db1;
                    const uint32_t idx = qs[4 * ib32 + l] | (((uint32_t)qh[ib32] << (8 - 2 * l)) & 0x300u);
                    const uint64_t g = qh_g_iq2s[idx];
                    const uint32_t signs = qs[32 + 4 * ib32 + l];
                    for (int j = 0; j < 8; j++) {
                        const float s = (signs & (1u << j)) ? -1.0f : 1.0f;
                        o[k++] = db * (float)(int8_t)(g >> (8 * j)) * s;
                    }
                }
            }
            return;
        }
        case QT_IQ3_S: {  // :1184-1237
            const float d = qh_f16(qh_rd16(b));
            const uint8_t* qs = b + 2;
            const uint8_t* qh = b + 66;
            const uint8_t* sg = b + 74;
            const uint8_t* scales = b + 106;
            int k = 0;
            for (int it = 0; it < 4; it++) {
                const float db1 = d * (1.0f + 2.0f * (float)(scales[it] & 0xF));
                const float db2 = d * (1.0f + 2.0f * (float)(scales[it] >> 4));
                for (int half = 0; half < 2; half++) {
                    const float db = half ? db2 : db1;
                    const uint32_t qhb = qh[2 * it + half];
                    const int qbase = 16 * it + 8 * half, sbase = 8 * it + 4 * half;
                    for (int l = 0; l < 4; l++) {
                        const uint32_t i0 = qs[qbase + 2 * l] | ((qhb << (8 - 2 * l)) & 256u);
                        const uint32_t i1 = qs[qbase + 2 * l + 1] | ((qhb << (7 - 2 * l)) & 256u);
                        const uint32_t g1 = qh_g_iq3s[i0], g2 = qh_g_iq3s[i1];
                        const uint32_t s = sg[sbase + l];
                        for (int j = 0; j < 4; j++)
                            o[k++] = db * (float)(int8_t)(g1 >> (8 * j)) * ((s & (1u << j)) ? -1.0f : 1.0f);
                        for (int j = 0; j < 4; j++)
                            o[k++] = db * (float)(int8_t)(g2 >> (8 * j)) * ((s & (1u << (j + 4))) ? -1.0f : 1.0f);
                    }
                }
            }
            return;
        }
        default: return;
    }
}

// Elements 16u .. 16u + 15 of a Q4_K or Q6_K block (u < 16), with the same f32
// operations as qh_decode_block, so 16 threads decode a block bit-identically
// to one thread decoding all of it.  False for other types.
__device__ bool qh_decode_part16(uint32_t t, const uint8_t* b, int u, float* o) {
    if (t == QT_Q4_K) {  // sub-block j = u / 2, positions 16 (u % 2) ..
        const int j = u >> 1, l0 = 16 * (u & 1);
        const float d = qh_f16(qh_rd16(b)), dmin = qh_f16(qh_rd16(b + 2));
        uint32_t s, mb;
        qh_gsm_k4(j, b + 4, s, mb);
        const float d1 = d * (float)s, m1 = dmin * (float)mb;
        const uint8_t* qs = b + 16 + 32 * (j >> 1) + l0;
        for (int l = 0; l < 16; l++) o[l] = d1 * (float)((j & 1) ? (qs[l] >> 4) : (qs[l] & 0x0F)) - m1;
        return true;
    }
    if (t == QT_Q6_K) {  // half h = u / 8, quarter r = (u / 2) % 4, positions 16 (u % 2) ..
        const int h = u >> 3, r = (u >> 1) & 3, l0 = 16 * (u & 1), is = l0 / 16;
        const float d = qh_f16(qh_rd16(b + 208));
        const uint8_t* ql = b + 64 * h + (r & 1) * 32;
        const uint8_t* qh = b + 128 + 32 * h;
        const int8_t* sc = (const int8_t*)(b + 192 + 8 * h);
        for (int l = l0; l < l0 + 16; l++) {
            const int q = (int)(((r < 2) ? (ql[l] & 0x0F) : (ql[l] >> 4)) | (((qh[l] >> (2 * r)) & 3) << 4)) - 32;
            o[l - l0] = d * (float)sc[is + 2 * r] * (float)q;
        }
        return true;
    }
    return false;
}

#pragma clang fp contract(on)

// One thread per block.
__global__ __launch_bounds__(256) void qh_dequant_k(uint32_t type, const uint8_t* __restrict__ W,
                                                    float* __restrict__ out, size_t nblocks, int qk,
                                                    uint32_t blk_bytes) {
    const size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    float vals[256];
    qh_decode_block(type, W + b * blk_bytes, vals);
    float* o = out + b * (size_t)qk;
    for (int i = 0; i < qk; i++) o[i] = vals[i];
}

hipError_t qh_launch_dequant(uint32_t type, const uint8_t* W, float* out, size_t n_elems, hipStream_t st) {
    const int qk = qh_block_elems(type);
    const size_t nb = n_elems / (size_t)qk;
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(qh_dequant_k, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, type, W, out, nb, qk,
                       qh_block_bytes(type));
    return hipGetLastError();
}
