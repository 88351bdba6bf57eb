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
#include <climits>
#include <mutex>
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
    // row blockIdx.x of a token-major batch (one row: the reference's kernel)
    out += (size_t)blockIdx.x * n;
    x += (size_t)blockIdx.x * n;
    if (n <= 4 * (int)blockDim.x && (n & 3) == 0 &&
        !(((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15u)) {
        // x and w read once into registers: one round trip to memory, not two
        const int i = 4 * (int)threadIdx.x;
        float4 xv = {0.f, 0.f, 0.f, 0.f}, wv = xv;
        if (i < n) {
            xv = *reinterpret_cast<const float4*>(x + i);
            wv = *reinterpret_cast<const float4*>(w + i);
        }
        float s = (xv.x * xv.x + xv.y * xv.y) + (xv.z * xv.z + xv.w * xv.w);
        s = qg_block_sum(s, sm);
        const float r = rsqrtf(s / (float)n + 1e-5f);
        if (i < n) *reinterpret_cast<float4*>(out + i) = float4{xv.x * r * wv.x, xv.y * r * wv.y, xv.z * r * wv.z, xv.w * r * wv.w};
        return;
    }
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += x[i] * x[i];
    s = qg_block_sum(s, sm);
    const float r = rsqrtf(s / (float)n + 1e-5f);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * r * w[i];
}

// RMS norm of each token's row fused with the batched GEMM's x images: token
// t = blockIdx.x of a token-major batch (<= 32 tokens; 17-32 on two image
// halves, token t in half t / 16) is normalised exactly as
// qg_rms_norm's one-float4-per-thread path computes it (the same per-thread
// sums, block sum and products), and digitised straight into image slot 0
// (qg_digitise: one half-wavefront per 256-element group), so the GEMM reads
// the images (no normalised rows in memory, no image launch of its own).
// n % 256 == 0, n <= 4 blockDim.x, 16-byte aligned x and w.
__global__ __launch_bounds__(1024) void qg_norm_image(unsigned char* __restrict__ img, const float* x,
                                                      const float* w, int n, int halves) {
    __shared__ float sm[16];
    const int t = blockIdx.x;
    x += (size_t)t * n;
    const int i = 4 * (int)threadIdx.x;
    float4 xv = {0.f, 0.f, 0.f, 0.f};
    if (i < n) xv = *reinterpret_cast<const float4*>(x + i);
    float s = (xv.x * xv.x + xv.y * xv.y) + (xv.z * xv.z + xv.w * xv.w);
    s = qg_block_sum(s, sm);
    const float r = rsqrtf(s / (float)n + 1e-5f);
    const int lane = threadIdx.x & 63, xc = threadIdx.x & 31, ngroups = n >> 8, nh = (int)blockDim.x >> 5;
    // group loop uniform over each wavefront (both halves call qg_digitise)
    for (int g0 = 0; g0 < ngroups; g0 += nh) {
        const int g = g0 + ((int)threadIdx.x >> 5);
        const bool on = g < ngroups;
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (on) {
            const int e = 256 * g + 8 * xc;
            const float4 a = *reinterpret_cast<const float4*>(x + e), b = *reinterpret_cast<const float4*>(x + e + 4);
            const float4 wa = *reinterpret_cast<const float4*>(w + e), wb = *reinterpret_cast<const float4*>(w + e + 4);
            v[0] = a.x * r * wa.x;
            v[1] = a.y * r * wa.y;
            v[2] = a.z * r * wa.z;
            v[3] = a.w * r * wa.w;
            v[4] = b.x * r * wb.x;
            v[5] = b.y * r * wb.y;
            v[6] = b.z * r * wb.z;
            v[7] = b.w * r * wb.w;
        }
        qg_digitise(v, on, lane, t & 15, xc, img + ((size_t)(on ? g : 0) * halves + (t >> 4)) * XImg::BYTES);
    }
}

// RoPE with YaRN on n_heads heads of head_dim (rope_yarn_f32, :577-605): pair i
// of a head rotates (i, i + head_dim/2) (NEOX) or (2i, 2i+1) (NORM) by pos *
// inv_freq(i), inv_freq ramped between theta^(-2i/d) and that / yarn_scale for
// YaRN (beta_fast 32, beta_slow 1).  One thread per pair.
// Rotation of pair i of one head: (x[i0], x[i1]) -> by pos * inv_freq(i).
struct QgRot {
    int i0, i1;
    float c, s;
};
QH_DEV QgRot qg_rope_rot(int i, int head_dim, int pos, float theta, float yarn_scale, int yarn_orig_ctx, int neox) {
    const int half = head_dim >> 1;
    // base angular rate of pair i; with YaRN, pairs whose period lies between
    // orig_ctx / 32 and orig_ctx blend linearly towards rate / yarn_scale
    const float base_rate = 1.f / powf(theta, 2.f * (float)i / (float)head_dim);
    float rate = base_rate;
    if (yarn_scale > 1.f && yarn_orig_ctx > 0) {
        const float short_ctx = (float)yarn_orig_ctx / 32.f, long_ctx = (float)yarn_orig_ctx / 1.f;
        const float period = 2.f * 3.14159265358979f / base_rate;
        const float keep = fmaxf(0.f, fminf(1.f, (long_ctx - period) / (long_ctx - short_ctx)));
        rate = keep * base_rate + (1.f - keep) * (base_rate / yarn_scale);
    }
    QgRot r;
    sincosf((float)pos * rate, &r.s, &r.c);
    r.i0 = neox ? i : 2 * i;
    r.i1 = neox ? i + half : 2 * i + 1;
    return r;
}

__global__ __launch_bounds__(256) void qg_rope_yarn(float* x, int n_pairs, int head_dim, int pos, float theta,
                                                    float yarn_scale, int yarn_orig_ctx, int neox) {
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n_pairs) return;
    const int half = head_dim >> 1, head = p / half, i = p - head * half;
    float* xh = x + (size_t)head * head_dim;
    const QgRot r = qg_rope_rot(i, head_dim, pos, theta, yarn_scale, yarn_orig_ctx, neox);
    const float x0 = xh[r.i0], x1 = xh[r.i1];
    xh[r.i0] = x0 * r.c - x1 * r.s;
    xh[r.i1] = x0 * r.s + x1 * r.c;
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

// One decode step's attention block in one launch, split over the sequence
// (flash decoding).  Workgroup (g, c) takes kv head g with every q head that
// maps to it (kv_head(h) = h * n_kv / n_heads, a contiguous range of h) and the
// 32-row slices c, c + nch, ... of the pos + 1 cached rows:
//   * RoPE of its q heads (qg_rope_rot, as qg_rope_yarn) into LDS;
//   * the workgroup owning row pos rotates k, appends k and v to the cache at
//     row pos and takes that row from LDS (the others read rows < pos only, so
//     nobody waits for the append, and the first slice's K/V loads are issued
//     before the RoPE, sharing its round trip to memory);
//   * per slice: K and V rows into LDS once for all the group's heads, scores
//     (wavefront = q head, lane = row x half of head_dim), an online softmax
//     (running max m, sum l, output o; lane owns dims lane + 64 j);
//   * (m, l, o) per head go to the library's partial scratch with agent-scope
//     stores; the last workgroup of kv head g to arrive (per-g counter, back at
//     zero when it is done) merges them: M = max m_c, L = sum l_c e^(m_c - M)
//     (+ e^(sink - M)), out = sum o_c e^(m_c - M) / L.
// Same mathematics as cuda_attn_score_all + cuda_softmax_sink_all +
// cuda_attn_values_all (src/cuda_kernels.cu:1199-1266); the sums are grouped by
// slice, so f32 results differ from them by rounding only.
#define QA_ROWS 32       // rows per slice
#define QA_MAXCH 64      // slices in flight per kv head
#define QA_MAXHD 256     // head_dim
#define QA_MAXG 16       // q heads per kv head
#define QA_MAXKV 256     // kv heads (arrival counters)
#define QA_PART (1 << 20)  // partial scratch, floats
static __device__ __align__(256) float qa_part[QA_PART];
static __device__ __align__(256) unsigned int qa_cnt[QA_MAXKV];

// Workgroups per kv head (slices of 32 rows shared out) for a step at row pos:
// more workgroups until the merge of their partials costs more than the slices
// they take over (measured on MI355X: 1 slice each up to 16 slices, 2 up to 64,
// then 4).  Several sequences: at least two slices per workgroup and at most
// 512 workgroups in all (position 511: 16 sequences 4.73 -> 4.48 ms per step
// with 4 slices per workgroup, 4 sequences 2.98 -> 2.90 with 2).  per_force > 0
// fixes the slices per workgroup.  The host sizes a launch with it, and a launch
// that reads pos on the device recomputes it there, so both split alike.
__host__ __device__ inline int qa_nch(int pos, int n_seq, int n_kv, int n_heads, int hd, int per_force) {
    const int slices = (pos + QA_ROWS) / QA_ROWS;
    int per = per_force ? per_force : (slices <= 16 ? 1 : (slices <= 64 ? 2 : 4));
    if (!per_force && n_seq > 1) {
        if (per < 2 && slices > 1) per = 2;
        while (per < slices && (int64_t)n_kv * n_seq * ((slices + per - 1) / per) > 512) per *= 2;
    }
    int nch = (slices + per - 1) / per;
    nch = nch < QA_MAXCH ? nch : QA_MAXCH;
    const int cap = QA_PART / (n_seq * n_heads * (hd + 2));
    return nch < cap ? nch : cap;
}

// HD: head_dim capacity, 128 or QA_MAXHD (LDS, so occupancy, scales with it);
// GW: q heads per wavefront (1, 2 or 4: groups of up to 4, 8 or QA_MAXG heads).
// The attention of kv head g for one workgroup, slices c, c + nch, ... (the
// body of qg_attention_step).  Returns true in the workgroup that wrote the
// group's output rows (the only one when nch == 1, else the last to arrive,
// which merges the partials).
template <int HD, int GW>
QH_DEV bool qg_attn_group(float* out, const float* q, const float* k, const float* v, float* kc, float* vc,
                          const float* sinks, int n_heads, int n_kv, int hd, int kv_dim, int pos, float theta,
                          float yarn_scale, int orig_ctx, int neox, float scale, float* part, unsigned int* cnt,
                          const int g, const int c, int nch, float* kl, float* vl, float* qr, float* kr,
                          float* vr, int& last_flag, const int* pos_dev, int per_force, int n_seq, size_t z) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int h0 = (g * n_heads + n_kv - 1) / n_kv, h1 = ((g + 1) * n_heads + n_kv - 1) / n_kv, ng = h1 - h0;
    // pos_dev: the position comes from device memory (a step replayed from one
    // graph at consecutive positions) and `pos` is the launch's bound; the
    // reference clamps to the cache (src/cuda.rs:517-520).  Its load is issued
    // first and the first slice's K/V loads go out before it returns: they are
    // clamped to the bound, and rows past the position are either replaced by
    // row pos (the owner's slice) or never read.
    const int bound = pos;
    const int pos_ld = pos_dev ? *pos_dev : pos;
    const int half = hd >> 1;
    constexpr int kp = HD + 4;  // LDS row strides of K (padded) and V: the template capacity
    const float* kh = k + (size_t)g * hd;
    const float* vh = v + (size_t)g * hd;
    const int t_l = lane & 31, hsel = lane >> 5;
    // K and V rows of a slice: every thread's loads are issued before any is
    // stored, and the next slice's are in flight while this one is computed.
    constexpr int IT = QA_ROWS * (HD / 4) / 256;  // float4 per thread and slice
    const int q4 = hd >> 2;
    typedef float f4 __attribute__((ext_vector_type(4)));  // a native vector: promoted to registers
    f4 kk[IT], vv[IT];
    // Thread i of the slice covers row i / (HD/4), column chunk i % (HD/4).
    // Rows past the slice (or the sequence) read row pos again and columns past
    // hd a valid column; the compute reads neither, so loads and stores carry
    // no branches and stay in registers.
    auto fetch = [&](int sl) {
#pragma unroll
        for (int u = 0; u < IT; u++) {
            const int i = threadIdx.x + 256 * u, r = i / (HD / 4), c4 = min(i % (HD / 4), q4 - 1);
            const int t = min(sl * QA_ROWS + r, bound);
            kk[u] = *reinterpret_cast<const f4*>(kc + (size_t)t * kv_dim + (size_t)g * hd + 4 * c4);
            vv[u] = *reinterpret_cast<const f4*>(vc + (size_t)t * kv_dim + (size_t)g * hd + 4 * c4);
        }
    };
    fetch(c);
    if (pos_dev) {
        // workgroups past this position's split exit at once
        pos = min(max(pos_ld, 0), bound);
        nch = qa_nch(pos, n_seq, n_kv, n_heads, hd, per_force);
        if (c >= nch) return false;
    }
    part += z * (size_t)n_heads * nch * (hd + 2);
    const int seq = pos + 1;
    const bool owner = ((pos / QA_ROWS) % nch) == c;
    // q rows at stride HD, zero past hd: the score dot runs over HD (a constant)
    if (hd < HD)
        for (int p = threadIdx.x; p < ng * HD; p += 256)
            if (p % HD >= hd) qr[p] = 0.f;
    for (int p = threadIdx.x; p < ng * half; p += 256) {
        const int j = p / half, i = p - j * half;
        const QgRot r = qg_rope_rot(i, hd, pos, theta, yarn_scale, orig_ctx, neox);
        const float* qh = q + (size_t)(h0 + j) * hd;
        const float q0 = qh[r.i0], q1 = qh[r.i1];
        qr[j * HD + r.i0] = q0 * r.c - q1 * r.s;
        qr[j * HD + r.i1] = q0 * r.s + q1 * r.c;
        if (owner && j == 0) {
            const float k0 = kh[r.i0], k1 = kh[r.i1];
            kr[r.i0] = k0 * r.c - k1 * r.s;
            kr[r.i1] = k0 * r.s + k1 * r.c;
            vr[r.i0] = vh[r.i0];
            vr[r.i1] = vh[r.i1];
        }
    }
    __syncthreads();
    if (owner) {
        float* kd = kc + (size_t)pos * kv_dim + (size_t)g * hd;
        float* vd = vc + (size_t)pos * kv_dim + (size_t)g * hd;
        for (int i = threadIdx.x; i < hd; i += 256) {
            kd[i] = kr[i];
            vd[i] = vr[i];
        }
    }
    // running state of this wavefront's heads j = w, w + 4, ... (< ng)
    float m[GW], l[GW], o[GW][HD / 64];
#pragma unroll
    for (int a = 0; a < GW; a++) {
        m[a] = -1e30f;
        l[a] = 0.f;
#pragma unroll
        for (int d = 0; d < HD / 64; d++) o[a][d] = 0.f;
    }
    for (int sl = c; sl * QA_ROWS < seq; sl += nch) {
        const int t0 = sl * QA_ROWS, nv = min(QA_ROWS, seq - t0);
#pragma unroll
        for (int u = 0; u < IT; u++) {
            const int i = threadIdx.x + 256 * u, r = i / (HD / 4), c4 = i % (HD / 4);
            f4 ks = kk[u], vs = vv[u];
            if (owner && t0 + r >= pos) {  // row pos (and the rows past it, which read it again)
                const int cc = min(c4, q4 - 1);  // a valid column, as fetch reads (kr is unset past hd)
                ks = *reinterpret_cast<const f4*>(kr + 4 * cc);
                vs = *reinterpret_cast<const f4*>(vr + 4 * cc);
            }
            *reinterpret_cast<f4*>(kl + r * kp + 4 * c4) = ks;
            *reinterpret_cast<f4*>(vl + r * HD + 4 * c4) = vs;
        }
        __syncthreads();
        fetch(sl + nch);
#pragma unroll
        for (int a = 0; a < GW; a++) {
            const int j = w + 4 * a;
            if (j >= ng) break;  // uniform per wavefront
            // score of row t_l: half hsel of the dot (HD / 2 terms, the ones past hd
            // zero), then the two halves summed
            const float* qj = qr + j * HD + hsel * (HD / 2);
            const float* kt = kl + t_l * kp + hsel * (HD / 2);
            float sdot = 0.f;
#pragma unroll
            for (int i = 0; i < HD / 2; i += 4) {
                const float4 kk = *reinterpret_cast<const float4*>(kt + i);
                const float4 qq = *reinterpret_cast<const float4*>(qj + i);
                sdot += (qq.x * kk.x + qq.y * kk.y) + (qq.z * kk.z + qq.w * kk.w);
            }
            sdot += __shfl_xor(sdot, 32);
            const float sc = t_l < nv ? sdot * scale : -1e30f;
            float mx = sc;
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            const float mn = fmaxf(m[a], mx);
            const float corr = expf(m[a] - mn);
            const float p = t_l < nv ? expf(sc - mn) : 0.f;
            float ps = p;
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) ps += __shfl_xor(ps, off);
            l[a] = l[a] * corr + ps;
            m[a] = mn;
#pragma unroll
            for (int d = 0; d < HD / 64; d++) o[a][d] *= corr;
            // o += p_t v_t over the slice's rows in order (p is 0 past nv), eight
            // rows' V loads in flight at a time; p of row t sits in lane t and is
            // read as a scalar
#pragma unroll
            for (int t0 = 0; t0 < QA_ROWS; t0 += 8) {
                float vb[8][HD / 64];
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int d = 0; d < HD / 64; d++) vb[u][d] = vl[(t0 + u) * HD + lane + 64 * d];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const float pt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), t0 + u));
#pragma unroll
                    for (int d = 0; d < HD / 64; d++) o[a][d] = fmaf(pt, vb[u][d], o[a][d]);
                }
            }
        }
        __syncthreads();
    }
    auto finish = [&](int j, float mm, float ll, const float* oo, bool from_part) {
        (void)from_part;
        const int h = h0 + j;
        const float sink = sinks ? sinks[h] : -1e30f;
        float M = mm;
        if (sink > -1e29f) M = fmaxf(M, sink);
        const float L = ll * expf(mm - M) + (sink > -1e29f ? expf(sink - M) : 0.f);
        const float f = expf(mm - M) / L;
#pragma unroll
        for (int d = 0; d < HD / 64; d++) {
            const int dd = lane + 64 * d;
            if (dd < hd) out[(size_t)h * hd + dd] = oo[d] * f;
        }
    };
    if (nch == 1) {
#pragma unroll
        for (int a = 0; a < GW; a++) {
            const int j = w + 4 * a;
            if (j >= ng) break;
            finish(j, m[a], l[a], o[a], false);
        }
        return true;
    }
    // partial record of (head h, slice c): [m, l, o[0 .. hd)]
    const int rec = hd + 2;
#pragma unroll
    for (int a = 0; a < GW; a++) {
        const int j = w + 4 * a;
        if (j >= ng) break;
        float* pr = part + ((size_t)(h0 + j) * nch + c) * rec;
        if (lane == 0) {
            __hip_atomic_store(pr, m[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pr + 1, l[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int d = 0; d < HD / 64; d++) {
            const int dd = lane + 64 * d;
            if (dd < hd) __hip_atomic_store(pr + 2 + dd, o[a][d], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // Every thread's partial stores have completed before the counter moves.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0)
        last_flag = __hip_atomic_fetch_add(&cnt[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    (unsigned)(nch - 1);
    __syncthreads();
    if (!last_flag) return false;
    // Merge.  The partials are read with SC1 buffer loads (the coherence bit of
    // an agent-scope load, so no stale L2 line of another launch is seen), which
    // unlike atomic loads issue back to back: lane cc holds slice cc's (m, l).
    const QhBuf pb = qh_buf(part, 4u * QA_PART);
    for (int j = w; j < ng; j += 4) {
        const uint32_t base = 4u * (uint32_t)((size_t)(h0 + j) * nch * rec);
        const bool on = lane < nch;
        const float mc = on ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pb.rs, (int)(base + 4u * lane * rec), 0, 16)) : -1e30f;
        const float lc = on ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pb.rs, (int)(base + 4u * (lane * rec + 1)), 0, 16)) : 0.f;
        float M = mc;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float e = on ? expf(mc - M) : 0.f;
        float L = lc * e;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) L += __shfl_xor(L, off);
        float oo[HD / 64];
#pragma unroll
        for (int d = 0; d < HD / 64; d++) oo[d] = 0.f;
        for (int c0 = 0; c0 < nch; c0 += 8) {
            // eight slices' loads in flight before any of them is used
            float ov[8][HD / 64];
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int d = 0; d < HD / 64; d++) {
                    const int dd = lane + 64 * d, cc = c0 + u;
                    const uint32_t off = (cc < nch && dd < hd) ? base + 4u * (cc * rec + 2 + dd) : 0x80000000u;
                    ov[u][d] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pb.rs, (int)off, 0, 16));
                }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float ec = __shfl(e, (c0 + u) & 63);
#pragma unroll
                for (int d = 0; d < HD / 64; d++) oo[d] = fmaf(c0 + u < nch ? ov[u][d] : 0.f, ec, oo[d]);
            }
        }
        finish(j, M, L, oo, true);
    }
    if (threadIdx.x == 0) __hip_atomic_store(&cnt[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
    return true;
}

template <int HD, int GW>
__global__ __launch_bounds__(256) void qg_attention_step(float* out, const float* q, const float* k, const float* v,
                                                         float* kc, float* vc, const float* sinks, int n_heads,
                                                         int n_kv, int hd, int kv_dim, int pos, float theta,
                                                         float yarn_scale, int orig_ctx, int neox, float scale,
                                                         float* part, unsigned int* cnt, size_t cache_stride,
                                                         const int* pos_dev, int per_force) {
    __shared__ __align__(16) float kl[QA_ROWS * (HD + 4)];
    __shared__ __align__(16) float vl[QA_ROWS * HD];
    __shared__ __align__(16) float qr[QA_MAXG * HD];
    __shared__ __align__(16) float kr[HD];
    __shared__ __align__(16) float vr[HD];
    __shared__ int last_flag;
    const int g = blockIdx.x, c = blockIdx.y;
    // sequence blockIdx.z of a batch: its q/k/v/out rows and its own K/V cache
    // (its partials: offset once the split is known)
    const size_t z = blockIdx.z;
    q += z * (size_t)n_heads * hd;
    out += z * (size_t)n_heads * hd;
    k += z * (size_t)kv_dim;
    v += z * (size_t)kv_dim;
    kc += z * cache_stride;
    vc += z * cache_stride;
    cnt += z * (size_t)n_kv;
    return (void)qg_attn_group<HD, GW>(out, q, k, v, kc, vc, sinks, n_heads, n_kv, hd, kv_dim, pos, theta,
                                              yarn_scale, orig_ctx, neox, scale, part, cnt, g, c, (int)gridDim.y, kl,
                                              vl, qr, kr, vr, last_flag, pos_dev, per_force, (int)gridDim.z, z);
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
// (embed_lookup_*, :678-731 handle Q5_1, IQ4_NL and BF16).  A workgroup takes
// up to 4096 output values: it stages their blocks' bytes in LDS with coalesced
// loads, one thread per block decodes from LDS into LDS (qh_decode_block), and
// the values leave in coalesced stores.  Several rows (a batch's tokens) go in
// one launch, row blockIdx.y = toks.t[blockIdx.y] into out + blockIdx.y *
// out_stride, so the rows decode side by side.
#define QG_EMB_OUT 4096
#define QG_EMB_RAW 4608
#define QG_EMB_TOKS 64  // rows per launch
struct QgToks { int t[QG_EMB_TOKS]; };
__global__ __launch_bounds__(256) void qg_embed_lookup(float* out, const uint8_t* data, uint32_t type,
                                                       const QgToks toks, size_t out_stride, int embed_dim, int qk,
                                                       uint32_t bb, int bpw, const int* tok_dev, int vocab) {
    __shared__ __align__(16) uint8_t raw[QG_EMB_RAW];
    __shared__ __align__(16) float dec[QG_EMB_OUT];
    out += (size_t)blockIdx.y * out_stride;
    const int nb = embed_dim / qk, b0 = blockIdx.x * bpw;
    const int nbw = min(bpw, nb - b0);
    int token = toks.t[blockIdx.y];
    if (tok_dev) {
        // token ids from device memory (a step replayed from one graph): an id
        // outside the table gives a zero row instead of a read past it
        token = tok_dev[blockIdx.y];
        if (token < 0 || token >= vocab) {
            for (int i = threadIdx.x; i < nbw * qk; i += 256) out[(size_t)b0 * qk + i] = 0.f;
            return;
        }
    }
    const uint8_t* src = data + ((size_t)token * nb + b0) * bb;
    if ((type == QT_Q4_K || type == QT_Q6_K) && nbw <= 16) {
        // 16 threads per block, each decoding 16 values straight from memory:
        // one round trip and no serial decode of whole blocks
        const int blk = threadIdx.x >> 4, u = threadIdx.x & 15;
        if (blk < nbw) {
            float v[16];
            (void)qh_decode_part16(type, src + (size_t)blk * bb, u, v);
            float* o = out + (size_t)(b0 + blk) * qk + 16 * u;
            if ((reinterpret_cast<uintptr_t>(o) & 15u) == 0) {
#pragma unroll
                for (int i = 0; i < 16; i += 4)
                    *reinterpret_cast<float4*>(o + i) = float4{v[i], v[i + 1], v[i + 2], v[i + 3]};
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) o[i] = v[i];
            }
        }
        return;
    }
    for (int i = threadIdx.x; i < nbw * (int)bb; i += 256) raw[i] = src[i];
    __syncthreads();
    if ((int)threadIdx.x < nbw) qh_decode_block(type, raw + threadIdx.x * bb, dec + threadIdx.x * qk);
    __syncthreads();
    float* o = out + (size_t)b0 * qk;
    for (int i = threadIdx.x; i < nbw * qk; i += 256) o[i] = dec[i];
}

// Greedy next token of each of `rows` logit rows: the reference's temperature
// <= 0 arm (src/main.rs:1684-1692), max_by(total_cmp), which returns the last
// of equal maxima.  Key of a value: its bits with the magnitude flipped when
// negative (f32::total_cmp's order as a signed compare), joined with the index
// so one signed 64-bit max picks the largest key and, among equal keys, the
// largest index.  One workgroup per row; tokens[r] = the index, and pos (if
// non-null) advances by one, so a captured step can feed the next one.
__device__ __forceinline__ long long qg_greedy_key(float v, int i) {
    const int b = __float_as_int(v);
    const int key = b ^ ((b >> 31) & 0x7FFFFFFF);
    return ((long long)key << 32) | (unsigned)i;
}
// A row is split over QG_GP workgroups (a single workgroup reading a 128256-
// entry row is bound by one CU's bandwidth: 12 us); each writes its best key,
// and the last of a row's workgroups to arrive reduces them in order and
// writes the token (row 0's also advances pos).
#define QG_GP 32
#define QG_GROWS 256
static __device__ __align__(256) unsigned long long qg_gpart[QG_GROWS * QG_GP];
static __device__ __align__(256) unsigned int qg_gcnt[QG_GROWS];
__global__ __launch_bounds__(256) void qg_greedy(const float* logits, size_t stride, int n, int* tokens, int* pos,
                                                 unsigned long long* gpart, unsigned int* gcnt) {
    __shared__ long long best_w[4];
    __shared__ int last;
    const int p = blockIdx.x, r = blockIdx.y;
    const float* x = logits + (size_t)r * stride;
    // chunk [i0, i1) of the row, 4-element aligned in index
    const int per = ((n + QG_GP - 1) / QG_GP + 3) & ~3;
    const int i0 = min(p * per, n), i1 = min(i0 + per, n);
    long long best = LLONG_MIN;
    if ((((uintptr_t)(x + i0)) & 15u) == 0) {
        const int n4 = (i1 - i0) >> 2;
        const float4* x4 = reinterpret_cast<const float4*>(x + i0);
        for (int j0 = threadIdx.x; j0 < n4; j0 += 4 * 256) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = x4[min(j0 + u * 256, n4 - 1)];  // a repeat changes nothing
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = i0 + 4 * min(j0 + u * 256, n4 - 1);
                long long kk = qg_greedy_key(v[u].x, i);
                kk = max(kk, qg_greedy_key(v[u].y, i + 1));
                kk = max(kk, qg_greedy_key(v[u].z, i + 2));
                kk = max(kk, qg_greedy_key(v[u].w, i + 3));
                best = kk > best ? kk : best;
            }
        }
        for (int i = i0 + 4 * n4 + (int)threadIdx.x; i < i1; i += 256) best = max(best, qg_greedy_key(x[i], i));
    } else {
        for (int i = i0 + (int)threadIdx.x; i < i1; i += 256) best = max(best, qg_greedy_key(x[i], i));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const long long o = __shfl_xor(best, off);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) best_w[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) best = best_w[w] > best ? best_w[w] : best;
        // stored with the sign flipped: unsigned order = signed order
        __hip_atomic_store(gpart + (size_t)r * QG_GP + p, (unsigned long long)best ^ 0x8000000000000000ull,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        last = __hip_atomic_fetch_add(gcnt + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == QG_GP - 1;
    }
    __syncthreads();
    if (!last) return;
    if (threadIdx.x < 64) {
        unsigned long long v = threadIdx.x < QG_GP
                                   ? __hip_atomic_load(gpart + (size_t)r * QG_GP + threadIdx.x, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : 0ull;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const unsigned long long o = __shfl_xor(v, off);
            v = o > v ? o : v;
        }
        if (threadIdx.x == 0) {
            tokens[r] = (int)(unsigned)(v & 0xFFFFFFFFull);
            if (pos && r == 0) pos[0] += 1;
            __hip_atomic_store(gcnt + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
        }
    }
}

struct QgGreedyScratch { unsigned long long* part; unsigned int* cnt; };
static const QgGreedyScratch* qg_greedy_scratch() {
    static QgGreedyScratch ptrs[64] = {};
    static std::once_flag once[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::call_once(once[dev], [&] {
        void *a = nullptr, *b = nullptr;
        if (hipGetSymbolAddress(&a, HIP_SYMBOL(qg_gpart)) == hipSuccess &&
            hipGetSymbolAddress(&b, HIP_SYMBOL(qg_gcnt)) == hipSuccess)
            ptrs[dev] = QgGreedyScratch{static_cast<unsigned long long*>(a), static_cast<unsigned int*>(b)};
    });
    return ptrs[dev].part ? &ptrs[dev] : nullptr;
}

hipError_t qh_glue_greedy(const float* logits, size_t stride, int rows, int n, int* tokens, int* pos, hipStream_t st) {
    if (rows <= 0 || n <= 0) return hipSuccess;
    const QgGreedyScratch* sc = qg_greedy_scratch();
    if (!sc) return hipErrorInvalidDevice;
    for (int r0 = 0; r0 < rows; r0 += QG_GROWS) {
        const int c = rows - r0 < QG_GROWS ? rows - r0 : QG_GROWS;
        hipLaunchKernelGGL(qg_greedy, dim3(QG_GP, (unsigned)c), dim3(256), 0, st, logits + (size_t)r0 * stride,
                           stride, n, tokens + r0, r0 == 0 ? pos : nullptr, sc->part, sc->cnt);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

static unsigned qg_blocks(int n) { return (unsigned)((n + 255) / 256); }

hipError_t qh_glue_vec(int op, float* dst, const float* src, float scale, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (op == 0) hipLaunchKernelGGL(qg_vec_add, dim3(qg_blocks(n)), dim3(256), 0, st, dst, src, n);
    else if (op == 1) hipLaunchKernelGGL(qg_vec_scale_add, dim3(qg_blocks(n)), dim3(256), 0, st, dst, src, scale, n);
    else hipLaunchKernelGGL(qg_vec_zero, dim3(qg_blocks(n)), dim3(256), 0, st, dst, n);
    return hipGetLastError();
}

hipError_t qh_glue_rms_norm(float* out, const float* x, const float* w, int n, hipStream_t st, int rows) {
    int blk = n >= 4096 ? 1024 : n >= 1024 ? 256 : 64;
    if (n % 4 == 0 && n <= 4096) blk = (n / 4 + 63) / 64 * 64;  // one float4 per thread (the register path)
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(qg_rms_norm, dim3((unsigned)rows), dim3(blk), 0, st, out, x, w, n);
    return hipGetLastError();
}

hipError_t qh_glue_norm_image(unsigned char* img, const float* x, const float* w, int n_tok, int in_dim,
                              hipStream_t st) {
    // the launch shape of qh_glue_rms_norm's register path, so the norm is its
    if (n_tok < 1 || n_tok > 32 || in_dim % 256 || in_dim > 4096 || (((uintptr_t)x | (uintptr_t)w) & 15u))
        return hipErrorNotSupported;
    const int blk = (in_dim / 4 + 63) / 64 * 64;
    hipLaunchKernelGGL(qg_norm_image, dim3((unsigned)n_tok), dim3(blk), 0, st, img, x, w, in_dim, n_tok > 16 ? 2 : 1);
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

// Device addresses of the attention scratch, per device (hipGetSymbolAddress once).
struct QaScratch { float* part; unsigned int* cnt; };
static const QaScratch* qa_scratch_ptrs() {
    static QaScratch ptrs[64] = {};
    static std::once_flag once[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::call_once(once[dev], [&] {
        void *a = nullptr, *b = nullptr;
        if (hipGetSymbolAddress(&a, HIP_SYMBOL(qa_part)) == hipSuccess &&
            hipGetSymbolAddress(&b, HIP_SYMBOL(qa_cnt)) == hipSuccess)
            ptrs[dev] = QaScratch{static_cast<float*>(a), static_cast<unsigned int*>(b)};
    });
    return ptrs[dev].part ? &ptrs[dev] : nullptr;
}

hipError_t qh_glue_attention_step(float* out, const float* q, const float* k, const float* v, float* kc, float* vc,
                                  const float* sinks, int n_heads, int n_kv, int hd, int kv_dim, int pos, float theta,
                                  float yarn_scale, int orig_ctx, int neox, float scale, hipStream_t st, int n_seq,
                                  size_t cache_stride, const int* pos_dev) {
    if (pos < 0 || hd <= 0 || (hd & 3) || hd > QA_MAXHD || n_seq < 1 || n_kv * n_seq > QA_MAXKV || (kv_dim & 3) ||
        (cache_stride & 3) || ((uintptr_t)kc & 15) || ((uintptr_t)vc & 15))
        return hipErrorNotSupported;
    if (n_heads <= 0) return hipSuccess;
    // q heads per kv head (the largest group)
    if ((n_heads + n_kv - 1) / n_kv > QA_MAXG) return hipErrorNotSupported;
    const QaScratch* sc = qa_scratch_ptrs();
    if (!sc) return hipErrorInvalidDevice;
    // QUARTZ_HIP_ATTN_SLICES=k forces k slices per workgroup
    static const int env_per = [] {
        const int k = qh_env_int("QUARTZ_HIP_ATTN_SLICES", 0);
        return k > 0 ? k : 0;
    }();
    // pos_dev: the grid covers the largest split of any position up to pos
    int nch = 0;
    if (pos_dev) {
        for (int sl = 1; sl <= pos / QA_ROWS + 1; sl++) {
            const int c = qa_nch(sl * QA_ROWS - 1, n_seq, n_kv, n_heads, hd, env_per);
            nch = c > nch ? c : nch;
        }
    } else {
        nch = qa_nch(pos, n_seq, n_kv, n_heads, hd, env_per);
    }
    if (nch < 1) return hipErrorNotSupported;
    const int gmax = (n_heads + n_kv - 1) / n_kv;
    auto launch = [&](auto HDC, auto GWC) {
        constexpr int H = decltype(HDC)::value, G = decltype(GWC)::value;
        hipLaunchKernelGGL((qg_attention_step<H, G>), dim3(n_kv, nch, n_seq), dim3(256), 0, st, out, q, k, v, kc, vc,
                           sinks, n_heads, n_kv, hd, kv_dim, pos, theta, yarn_scale, orig_ctx, neox, scale, sc->part,
                           sc->cnt, cache_stride, pos_dev, env_per);
    };
    using I128 = std::integral_constant<int, 128>;
    using IMAX = std::integral_constant<int, QA_MAXHD>;
    using G1 = std::integral_constant<int, 1>;
    using G2 = std::integral_constant<int, 2>;
    using G4 = std::integral_constant<int, QA_MAXG / 4>;
    if (hd <= 128) {
        if (gmax <= 4) launch(I128{}, G1{});
        else if (gmax <= 8) launch(I128{}, G2{});
        else launch(I128{}, G4{});
    } else {
        if (gmax <= 4) launch(IMAX{}, G1{});
        else if (gmax <= 8) launch(IMAX{}, G2{});
        else launch(IMAX{}, G4{});
    }
    return hipGetLastError();
}

hipError_t qh_glue_swiglu(int oai, float* out, const float* gate, const float* up, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    if (oai) hipLaunchKernelGGL(qg_swiglu_oai, dim3(qg_blocks(n)), dim3(256), 0, st, out, gate, up, n);
    else hipLaunchKernelGGL(qg_swiglu, dim3(qg_blocks(n)), dim3(256), 0, st, out, gate, up, n);
    return hipGetLastError();
}

hipError_t qh_glue_embed(float* out, size_t out_stride, const uint8_t* data, uint32_t type, const int* tokens,
                         int n_tok, int embed_dim, hipStream_t st, const int* tok_dev, int vocab) {
    const int qk = qh_block_elems(type);
    const uint32_t bb = qh_block_bytes(type);
    const int nb = embed_dim / qk;
    int bpw = QG_EMB_OUT / qk;
    if (bpw > 256) bpw = 256;
    if ((uint32_t)bpw * bb > QG_EMB_RAW) bpw = QG_EMB_RAW / bb;
    for (int t0 = 0; t0 < n_tok; t0 += QG_EMB_TOKS) {
        const int c = n_tok - t0 < QG_EMB_TOKS ? n_tok - t0 : QG_EMB_TOKS;
        QgToks toks = {};
        if (!tok_dev)
            for (int i = 0; i < c; i++) toks.t[i] = tokens[t0 + i];
        hipLaunchKernelGGL(qg_embed_lookup, dim3((unsigned)((nb + bpw - 1) / bpw), (unsigned)c), dim3(256), 0, st,
                           out + (size_t)t0 * out_stride, data, type, toks, out_stride, embed_dim, qk, bb, bpw,
                           tok_dev ? tok_dev + t0 : nullptr, vocab);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
