// qh_mmq81.hip -- the Q8_1 MMQ arithmetic mode (hip_gemm_q8_1_mmq): ggml-cuda's
// int8 MMQ rounding for Q4_K and Q6_K, bit-exact to the reference's CPU oracles
// gemm_q4k_q8_1_mmq[_stream_k] / gemm_q6k_q8_1_mmq[_stream_k]
// (src/dequant.rs:202-645):
//   * activations quantised per 32 values to Q8_1: max |x| and the sum over 8
//     lanes of 4 values, combined in XOR order 4, 2, 1; q = round(x * 127/max)
//     (half away from zero); scale 1 / (127/max), f16-rounded for Q4_K (with the
//     f16-rounded sum), kept in f32 for Q6_K (quantize_q8_1_mmq_d4);
//   * Q4_K: per 32-weight group, f16-rounded d*sc and -dmin*m, integer dot,
//     acc = fma(cs * scale, dot, acc); acc = fma(cm, sum, acc);
//   * Q6_K: per 128-value half, fragment = sum over 4 groups of fma(scale,
//     s1*dot1 + s2*dot2, .), acc = fma(d, fragment, acc);
//   * optional stream-K split (cuda_stream_k_cut): the accumulation restarts at
//     the cut superblock and the result is tail + prefix.
// One thread per output accumulates in exactly that order (the integer dots
// are exact, v_dot4_i32_i8); a workgroup (16 columns x 16 tokens) quantises
// each 256-value block of its tokens once into LDS.  This is a compatibility
// mode for ggml-identical results, not the fast batched path (qh_gemm.hip).
#include "qh_internal.h"

#define QM_T 16  // tokens per workgroup
#define QM_C 16  // columns per workgroup

QH_DEV float qm_f16r(float v) { return (float)(_Float16)v; }  // round to nearest even, as f32_to_f16_round_to_even

// Stream-K cut of output (row, column): cuda_stream_k_cut (src/dequant.rs:338-374).
QH_DEV int qm_cut(int row, int column, int in_dim, int out_dim, int ref_rows, int mps) {
    if (ref_rows <= 0 || mps <= 0 || in_dim % 256) return -1;
    const long long bpt = in_dim / 256, tx = (ref_rows + 127) / 128, ty = (out_dim + 127) / 128, tc = tx * ty;
    const long long waves = (tc + mps - 1) / mps, eff = 100 * tc / (mps * waves);
    const long long grid = eff >= 90 ? tc : mps;
    if (grid == 0 || tc % grid == 0) return -1;
    const long long tile = (long long)(column / 128) * tx + row / 128, ts = tile * bpt, te = ts + bpt,
                    tot = tc * bpt;
    // the first boundary block * tot / grid inside (ts, te)
    long long b = (ts * grid) / tot + 1;
    for (; b < grid; b++) {
        const long long bd = b * tot / grid;
        if (bd >= te) break;
        if (bd > ts) return (int)(bd - ts);
    }
    return -1;
}

template <bool Q6>
__global__ __launch_bounds__(256) void qh_mmq_q81(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                  float* __restrict__ y, int in_dim, int out_dim, int rows,
                                                  int ref_rows, int mps) {
    __shared__ __align__(16) int8_t qa[QM_T * 256];
    __shared__ float qs[QM_T * 8], qm[QM_T * 8];
    const int T = threadIdx.x, tok = T & (QM_T - 1), cl = T >> 4;
    const int row = blockIdx.y * QM_T + tok, column = blockIdx.x * QM_C + cl;
    const bool live = row < rows && column < out_dim;
    const int nsb = in_dim / 256;
    constexpr int BB = Q6 ? 210 : 144;
    const uint8_t* wrow = W + (size_t)(live ? column : 0) * nsb * BB;
    const int cut = live ? qm_cut(row, column, in_dim, out_dim, ref_rows, mps) : -1;
    float acc = 0.f, prefix = 0.f;
    for (int b = 0; b < nsb; b++) {
        // quantise: thread (t, g) < 128 takes token t's 32-value group g of block b
        if (T < QM_T * 8) {
            const int t = T >> 3, g = T & 7, r = blockIdx.y * QM_T + t;
            float v[32];
            if (r < rows) {
                const float4* src = reinterpret_cast<const float4*>(x + (size_t)r * in_dim + 256 * b + 32 * g);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float4 f = src[i];
                    v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 32; i++) v[i] = 0.f;
            }
            float pm[8], ps[8];
#pragma unroll
            for (int l = 0; l < 8; l++) {
                pm[l] = fmaxf(fmaxf(fmaxf(fmaxf(0.f, fabsf(v[4 * l])), fabsf(v[4 * l + 1])), fabsf(v[4 * l + 2])),
                              fabsf(v[4 * l + 3]));
                ps[l] = ((v[4 * l] + v[4 * l + 1]) + v[4 * l + 2]) + v[4 * l + 3];
            }
#pragma unroll
            for (int o = 4; o >= 1; o >>= 1) {
                float om[8], os[8];
#pragma unroll
                for (int l = 0; l < 8; l++) { om[l] = pm[l]; os[l] = ps[l]; }
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    pm[l] = fmaxf(om[l], om[l ^ o]);
                    ps[l] = os[l] + os[l ^ o];
                }
            }
            const float mx = pm[0];
            const float inv = mx == 0.f ? 0.f : __fdiv_rn(127.f, mx);
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                int8_t q4[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float rq = inv != 0.f ? roundf(v[i + j] * inv) : 0.f;
                    rq = fminf(fmaxf(rq, -128.f), 127.f);
                    q4[j] = (int8_t)rq;
                }
                *reinterpret_cast<uint32_t*>(qa + t * 256 + 32 * g + i) =
                    (uint32_t)(uint8_t)q4[0] | ((uint32_t)(uint8_t)q4[1] << 8) | ((uint32_t)(uint8_t)q4[2] << 16) |
                    ((uint32_t)(uint8_t)q4[3] << 24);
            }
            const float sc = inv == 0.f ? 0.f : __fdiv_rn(1.f, inv);
            qs[t * 8 + g] = Q6 ? sc : qm_f16r(sc);
            qm[t * 8 + g] = Q6 ? 0.f : qm_f16r(ps[0]);
        }
        __syncthreads();
        if (live) {
            if (b == cut) {
                prefix = acc;
                acc = 0.f;
            }
            const uint8_t* blk = wrow + (size_t)b * BB;
            const int* xa = reinterpret_cast<const int*>(qa + tok * 256);
            if constexpr (!Q6) {
                const float d = qh_f16(blk[0] | (blk[1] << 8)), dmin = qh_f16(blk[2] | (blk[3] << 8));
                uint8_t s[12];
#pragma unroll
                for (int i = 0; i < 12; i++) s[i] = blk[4 + i];
#pragma unroll
                for (int g = 0; g < 8; g++) {
                    uint32_t sc, m;  // get_scale_min_k4 (src/dequant.rs:1471-1480)
                    if (g < 4) {
                        sc = s[g] & 63u;
                        m = s[g + 4] & 63u;
                    } else {
                        sc = (s[g + 4] & 0x0Fu) | ((uint32_t)(s[g - 4] >> 6) << 4);
                        m = (uint32_t)(s[g + 4] >> 4) | ((uint32_t)(s[g] >> 6) << 4);
                    }
                    const float cs = qm_f16r(d * (float)sc), cm = qm_f16r(-dmin * (float)m);
                    const uint8_t* qq = blk + 16 + (g >> 1) * 32;
                    int dot = 0;
#pragma unroll
                    for (int i = 0; i < 32; i += 4) {
                        const uint32_t p = (uint32_t)qq[i] | ((uint32_t)qq[i + 1] << 8) | ((uint32_t)qq[i + 2] << 16) |
                                           ((uint32_t)qq[i + 3] << 24);
                        const uint32_t w4 = (g & 1) ? (p >> 4) & 0x0F0F0F0Fu : p & 0x0F0F0F0Fu;
                        dot = __builtin_amdgcn_sdot4((int)w4, xa[8 * g + i / 4], dot, false);
                    }
                    const float ds = cs * qs[tok * 8 + g];
                    acc = fmaf(ds, (float)dot, acc);
                    acc = fmaf(cm, qm[tok * 8 + g], acc);
                }
            } else {
                const float d6 = qh_f16(blk[208] | (blk[209] << 8));
#pragma unroll
                for (int f = 0; f < 2; f++) {
                    float fs = 0.f;
#pragma unroll
                    for (int g = 4 * f; g < 4 * f + 4; g++) {
                        // group g = values 32g .. 32g + 31: half h = g / 4, quarter k = g % 4
                        const int h = g >> 2, k = g & 3;
                        const uint8_t* ql = blk + 64 * h + 32 * (k & 1);
                        const uint8_t* qh = blk + 128 + 32 * h;
                        int d1 = 0, d2 = 0;
#pragma unroll
                        for (int i = 0; i < 32; i += 4) {
                            uint32_t w4 = 0;
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                const uint32_t lo = (k >> 1) ? (uint32_t)(ql[i + j] >> 4) : (uint32_t)(ql[i + j] & 15u);
                                const uint32_t hi = ((uint32_t)qh[i + j] >> (2 * k)) & 3u;
                                w4 |= (((lo | (hi << 4)) - 32u) & 0xFFu) << (8 * j);
                            }
                            if (i < 16) d1 = __builtin_amdgcn_sdot4((int)w4, xa[8 * g + i / 4], d1, false);
                            else d2 = __builtin_amdgcn_sdot4((int)w4, xa[8 * g + i / 4], d2, false);
                        }
                        const int s1 = (int8_t)blk[192 + 2 * g], s2 = (int8_t)blk[192 + 2 * g + 1];
                        fs = fmaf(qs[tok * 8 + g], (float)(s1 * d1 + s2 * d2), fs);
                    }
                    acc = fmaf(d6, fs, acc);
                }
            }
        }
        __syncthreads();
    }
    if (live) y[(size_t)row * out_dim + column] = cut >= 0 ? acc + prefix : acc;
}

hipError_t qh_launch_mmq_q81(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                             int rows, int ref_rows, int mps, hipStream_t st) {
    if ((type != QT_Q4_K && type != QT_Q6_K) || in_dim % 256 || ((uintptr_t)x & 15u)) return hipErrorNotSupported;
    if (rows == 0 || out_dim == 0) return hipSuccess;
    const dim3 grid((unsigned)((out_dim + QM_C - 1) / QM_C), (unsigned)((rows + QM_T - 1) / QM_T));
    if (type == QT_Q4_K)
        hipLaunchKernelGGL(qh_mmq_q81<false>, grid, dim3(256), 0, st, W, x, y, in_dim, out_dim, rows, ref_rows, mps);
    else
        hipLaunchKernelGGL(qh_mmq_q81<true>, grid, dim3(256), 0, st, W, x, y, in_dim, out_dim, rows, ref_rows, mps);
    return hipGetLastError();
}
