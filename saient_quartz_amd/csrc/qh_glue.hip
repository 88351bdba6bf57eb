// qh_glue.hip -- the decode step's kernels between the weight GEMVs.
//
// Counterparts of the reference's forward-pass helpers (src/cuda_kernels.cu:
// 545-750, launchers :1129-1290), used by forward_gpu_step
// (src/cuda.rs:507-851): vector add / scale-add / zero, RMS norm (eps 1e-5),
// RoPE with YaRN (NORM and NEOX pairings), KV-cache append, batched multi-head
// attention (scores, softmax with an optional sink, value sums; grouped-query
// head mapping kv_head = head * n_kv / n_heads), SwiGLU (SiLU and the clamped
// gpt-oss form) and the embedding row lookup.  Same formulas; the reductions
// are wave64 (DPP / cross-lane) trees instead of warp-of-32 shuffles, so f32
// results differ from the reference's only by summation order.
// hip_attention_decode fuses the three attention kernels into one launch per
// step (scores and probabilities stay in LDS).
#include "qh_internal.h"

// Sum / max over the 64 lanes of a wavefront (every lane gets the result).
QH_DEV float qg_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
QH_DEV float qg_wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Sum / max over a workgroup of up to 1024 threads (all threads get the result).
// `sm` holds one float per wavefront; the call ends with a barrier.
QH_DEV float qg_block_sum(float v, float* sm) {
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    v = qg_wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sm[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += sm[i];
    __syncthreads();
    return t;
}
QH_DEV float qg_block_max(float v, float* sm) {
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    v = qg_wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sm[w] = v;
    __syncthreads();
    float t = -1e30f;
    for (int i = 0; i < nw; i++) t = fmaxf(t, sm[i]);
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(256) void qg_vec_add(float* dst, const float* src, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] += src[i];
}
__global__ __launch_bounds__(256) void qg_vec_scale_add(float* dst, const float* src, float scale, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] += scale * src[i];
}
__global__ __launch_bounds__(256) void qg_vec_zero(float* dst, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = 0.f;
}

// out = x * rsqrt(mean(x^2) + 1e-5) * w, one workgroup (rms_norm_f32, :563-575).
// In-place (out == x) is safe: every read of x precedes the reduction's barriers.
__global__ __launch_bounds__(1024) void qg_rms_norm(float* out, const float* x, const float* w, int n) {
    __shared__ float sm[16];
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += x[i] * x[i];
    s = qg_block_sum(s, sm);
    const float r = rsqrtf(s / (float)n + 1e-5f);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * r * w[i];
}

// RoPE with YaRN on n_heads heads of head_dim (rope_yarn_f32, :577-605): pair i
// of a head rotates (i, i + head_dim/2) (NEOX) or (2i, 2i+1) (NORM) by pos *
// inv_freq(i), inv_freq ramped between theta^(-2i/d) and that / yarn_scale for
// YaRN (beta_fast 32, beta_slow 1).  One thread per pair.
__global__ __launch_bounds__(256) void qg_rope_yarn(float* x, int n_pairs, int head_dim, int pos, float theta,
                                                    float yarn_scale, int yarn_orig_ctx, int neox) {
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n_pairs) return;
    const int half = head_dim >> 1, head = p / half, i = p - head * half;
    float* xh = x + (size_t)head * head_dim;
    const float std_inv = 1.f / powf(theta, 2.f * (float)i / (float)head_dim);
    float eff_inv = std_inv;
    if (yarn_scale > 1.f && yarn_orig_ctx > 0) {
        const float hfw = (float)yarn_orig_ctx / 32.f, lfw = (float)yarn_orig_ctx / 1.f;
        const float wavelen = 2.f * 3.14159265358979f / std_inv;
        const float ramp = fmaxf(0.f, fminf(1.f, (lfw - wavelen) / (lfw - hfw)));
        eff_inv = ramp * std_inv + (1.f - ramp) * (std_inv / yarn_scale);
    }
    float s, c;
    sincosf((float)pos * eff_inv, &s, &c);
    const int i0 = neox ? i : 2 * i, i1 = neox ? i + half : 2 * i + 1;
    const float x0 = xh[i0], x1 = xh[i1];
    xh[i0] = x0 * c - x1 * s;
    xh[i1] = x0 * s + x1 * c;
}

__global__ __launch_bounds__(256) void qg_kv_append(float* kc, float* vc, const float* k, const float* v, int pos,
                                                    int kv_dim) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < kv_dim) {
        kc[(size_t)pos * kv_dim + i] = k[i];
        vc[(size_t)pos * kv_dim + i] = v[i];
    }
}

// scores[h * max_seq + t] = scale * dot(q[h], k_cache[t][kv_head(h)]): one
// wavefront per (head, t), four per workgroup (attn_score_all_f32, :1199-1214).
__global__ __launch_bounds__(256) void qg_attn_score_all(float* scores, const float* q, const float* kc, int n_heads,
                                                         int n_kv, int seq, int hd, int kv_dim, int max_seq,
                                                         float scale) {
    const int h = blockIdx.x, t = blockIdx.y * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= seq) return;
    const int kvh = h * n_kv / n_heads;
    const float* qh = q + (size_t)h * hd;
    const float* kt = kc + (size_t)t * kv_dim + (size_t)kvh * hd;
    float a = 0.f;
    for (int i = lane; i < hd; i += 64) a += qh[i] * kt[i];
    a = qg_wave_sum(a);
    if (lane == 0) scores[(size_t)h * max_seq + t] = a * scale;
}

// In-place softmax of each head's first seq scores; the sink (sinks[h], or sink0
// when sinks is NULL; <= -1e29: none) joins the normaliser only (softmax_sink_all_f32,
// :1216-1248).
__global__ __launch_bounds__(256) void qg_softmax_sink_all(float* scores, int seq, int max_seq, const float* sinks,
                                                           float sink0) {
    __shared__ float sm[16];
    float* x = scores + (size_t)blockIdx.x * max_seq;
    const float sink = sinks ? sinks[blockIdx.x] : sink0;
    float m = -1e30f;
    for (int i = threadIdx.x; i < seq; i += blockDim.x) m = fmaxf(m, x[i]);
    m = fmaxf(qg_block_max(m, sm), sink > -1e29f ? sink : -1e30f);
    float s = 0.f;
    for (int i = threadIdx.x; i < seq; i += blockDim.x) {
        const float e = expf(x[i] - m);
        x[i] = e;
        s += e;
    }
    const float tot = qg_block_sum(s, sm) + (sink > -1e29f ? expf(sink - m) : 0.f);
    for (int i = threadIdx.x; i < seq; i += blockDim.x) x[i] /= tot;
}

// out[h * hd + i] = sum_t scores[h][t] v_cache[t][kv_head(h)][i]: thread i of a
// head's workgroup, 4 slices of t reduced through LDS (attn_values_all_f32,
// :1250-1266).
__global__ __launch_bounds__(256) void qg_attn_values_all(float* out, const float* scores, const float* vc,
                                                          int n_heads, int n_kv, int seq, int hd, int kv_dim,
                                                          int max_seq) {
    __shared__ float part[4][256];
    const int h = blockIdx.x, kvh = h * n_kv / n_heads;
    const int i = blockIdx.y * 64 + (threadIdx.x & 63), q = threadIdx.x >> 6;
    const float* s = scores + (size_t)h * max_seq;
    float a = 0.f;
    if (i < hd)
        for (int t = q; t < seq; t += 4) a += s[t] * vc[(size_t)t * kv_dim + (size_t)kvh * hd + i];
    part[q][threadIdx.x & 63] = a;
    __syncthreads();
    if (q == 0 && i < hd) out[(size_t)h * hd + i] = (part[0][threadIdx.x] + part[1][threadIdx.x]) +
                                                    (part[2][threadIdx.x] + part[3][threadIdx.x]);
}

// The three attention kernels in one: a workgroup per head keeps its seq
// scores in LDS (seq <= QG_ATT_MAX), softmax with the sink, then the value sums.
#define QG_ATT_MAX 16384
__global__ __launch_bounds__(256) void qg_attention_decode(float* out, const float* q, const float* kc,
                                                           const float* vc, const float* sinks, int n_heads,
                                                           int n_kv, int seq, int hd, int kv_dim, float scale) {
    __shared__ float sc[QG_ATT_MAX];
    __shared__ float sm[16];
    __shared__ float part[4][256];
    const int h = blockIdx.x, kvh = h * n_kv / n_heads, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float* qh = q + (size_t)h * hd;
    for (int t = w; t < seq; t += 4) {
        const float* kt = kc + (size_t)t * kv_dim + (size_t)kvh * hd;
        float a = 0.f;
        for (int i = lane; i < hd; i += 64) a += qh[i] * kt[i];
        a = qg_wave_sum(a);
        if (lane == 0) sc[t] = a * scale;
    }
    __syncthreads();
    const float sink = sinks ? sinks[h] : -1e30f;
    float m = -1e30f;
    for (int i = threadIdx.x; i < seq; i += 256) m = fmaxf(m, sc[i]);
    m = fmaxf(qg_block_max(m, sm), sink > -1e29f ? sink : -1e30f);
    float s = 0.f;
    for (int i = threadIdx.x; i < seq; i += 256) {
        const float e = expf(sc[i] - m);
        sc[i] = e;
        s += e;
    }
    const float inv = 1.f / (qg_block_sum(s, sm) + (sink > -1e29f ? expf(sink - m) : 0.f));
    for (int i0 = 0; i0 < hd; i0 += 64) {
        const int i = i0 + lane;
        float a = 0.f;
        if (i < hd)
            for (int t = w; t < seq; t += 4) a += sc[t] * vc[(size_t)t * kv_dim + (size_t)kvh * hd + i];
        part[w][lane] = a;
        __syncthreads();
        if (w == 0 && i < hd)
            out[(size_t)h * hd + i] = ((part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane])) * inv;
        __syncthreads();
    }
}

// silu(gate) * up (swiglu_f32, :670-676) and the clamped gpt-oss form
// (swiglu_oai_f32, :660-668).
__global__ __launch_bounds__(256) void qg_swiglu(float* out, const float* gate, const float* up, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float g = gate[i];
    out[i] = (g / (1.f + expf(-g))) * up[i];
}
__global__ __launch_bounds__(256) void qg_swiglu_oai(float* out, const float* gate, const float* up, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float x = fminf(gate[i], 7.f), y = fmaxf(-7.f, fminf(7.f, up[i]));
    out[i] = (x / (1.f + expf(-1.702f * x))) * (y + 1.f);
}

// Row `token` of an embedding matrix of any supported type, decoded bit-exactly
// (embed_lookup_*, :678-731 handle Q5_1, IQ4_NL and BF16): one thread per block.
__global__ __launch_bounds__(256) void qg_embed_lookup(float* out, const uint8_t* data, uint32_t type, int token,
                                                       int embed_dim, int qk, uint32_t bb) {
    const int b = blockIdx.x * 256 + threadIdx.x, nb = embed_dim / qk;
    if (b >= nb) return;
    float v[256];
    qh_decode_block(type, data + ((size_t)token * nb + b) * bb, v);
    for (int i = 0; i < qk; i++) out[(size_t)b * qk + i] = v[i];
}

static unsigned qg_blocks(int n) { return (unsigned)((n + 255) / 256); }

hipError_t qh_glue_vec(int op, float* dst, const float* src, float scale, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (op == 0) hipLaunchKernelGGL(qg_vec_add, dim3(qg_blocks(n)), dim3(256), 0, st, dst, src, n);
    else if (op == 1) hipLaunchKernelGGL(qg_vec_scale_add, dim3(qg_blocks(n)), dim3(256), 0, st, dst, src, scale, n);
    else hipLaunchKernelGGL(qg_vec_zero, dim3(qg_blocks(n)), dim3(256), 0, st, dst, n);
    return hipGetLastError();
}

hipError_t qh_glue_rms_norm(float* out, const float* x, const float* w, int n, hipStream_t st) {
    const int blk = n >= 4096 ? 1024 : n >= 1024 ? 256 : 64;
    hipLaunchKernelGGL(qg_rms_norm, dim3(1), dim3(blk), 0, st, out, x, w, n);
    return hipGetLastError();
}

hipError_t qh_glue_rope(float* x, int n_heads, int head_dim, int pos, float theta, float yarn_scale, int orig_ctx,
                        int neox, hipStream_t st) {
    const int pairs = n_heads * (head_dim / 2);
    if (pairs <= 0) return hipSuccess;
    hipLaunchKernelGGL(qg_rope_yarn, dim3(qg_blocks(pairs)), dim3(256), 0, st, x, pairs, head_dim, pos, theta,
                       yarn_scale, orig_ctx, neox);
    return hipGetLastError();
}

hipError_t qh_glue_kv_append(float* kc, float* vc, const float* k, const float* v, int pos, int kv_dim,
                             hipStream_t st) {
    hipLaunchKernelGGL(qg_kv_append, dim3(qg_blocks(kv_dim)), dim3(256), 0, st, kc, vc, k, v, pos, kv_dim);
    return hipGetLastError();
}

hipError_t qh_glue_attn(int op, float* dst, const float* a, const float* b, const float* sinks, int n_heads,
                        int n_kv, int seq, int hd, int kv_dim, int max_seq, float scale, hipStream_t st) {
    // op 0: scores (scale), 1: softmax (sinks, or `scale` as the one sink when NULL), 2: value sums
    if (seq <= 0 || n_heads <= 0) return hipSuccess;
    if (op == 0)
        hipLaunchKernelGGL(qg_attn_score_all, dim3(n_heads, (seq + 3) / 4), dim3(256), 0, st, dst, a, b, n_heads,
                           n_kv, seq, hd, kv_dim, max_seq, scale);
    else if (op == 1)
        hipLaunchKernelGGL(qg_softmax_sink_all, dim3(n_heads), dim3(256), 0, st, dst, seq, max_seq, sinks, scale);
    else
        hipLaunchKernelGGL(qg_attn_values_all, dim3(n_heads, (hd + 63) / 64), dim3(256), 0, st, dst, a, b, n_heads,
                           n_kv, seq, hd, kv_dim, max_seq);
    return hipGetLastError();
}

hipError_t qh_glue_attention_decode(float* out, const float* q, const float* kc, const float* vc, const float* sinks,
                                    int n_heads, int n_kv, int seq, int hd, int kv_dim, float scale, hipStream_t st) {
    if (seq > QG_ATT_MAX) return hipErrorNotSupported;
    if (seq <= 0 || n_heads <= 0) return hipSuccess;
    hipLaunchKernelGGL(qg_attention_decode, dim3(n_heads), dim3(256), 0, st, out, q, kc, vc, sinks, n_heads, n_kv,
                       seq, hd, kv_dim, scale);
    return hipGetLastError();
}

hipError_t qh_glue_swiglu(int oai, float* out, const float* gate, const float* up, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (oai) hipLaunchKernelGGL(qg_swiglu_oai, dim3(qg_blocks(n)), dim3(256), 0, st, out, gate, up, n);
    else hipLaunchKernelGGL(qg_swiglu, dim3(qg_blocks(n)), dim3(256), 0, st, out, gate, up, n);
    return hipGetLastError();
}

hipError_t qh_glue_embed(float* out, const uint8_t* data, uint32_t type, int token, int embed_dim, hipStream_t st) {
    const int qk = qh_block_elems(type);
    const int nb = embed_dim / qk;
    hipLaunchKernelGGL(qg_embed_lookup, dim3(qg_blocks(nb)), dim3(256), 0, st, out, data, type, token, embed_dim, qk,
                       qh_block_bytes(type));
    return hipGetLastError();
}
