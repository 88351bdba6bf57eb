// qh_moe.hip -- the mixture-of-experts glue around the expert GEMMs, on the device.
//
// The reference routes on the host: the router GEMV's logits are copied back
// (src/cuda.rs:670-700), sorted with sort_unstable_by(total_cmp) descending,
// the top k kept and weighted by a softmax over the top k (moe_renorm:
// Mixtral, Qwen-MoE, gpt-oss) or over all experts without renormalisation
// (OLMoE); each chosen expert then runs gate, up, (bias,) SwiGLU, down, (bias,)
// and is scale-added into the output (src/main.rs:952-1043, GPU twin
// src/cuda.rs:703-798).  Here the same steps run as five small kernels so a
// batch of tokens never leaves HBM:
//   route    logits (+ bias) -> top-k expert ids and weights per token
//   plan     ids -> per-expert token ranges (tok_off), the expert-ordered slot
//            of each (token, choice) and the token/expert of each slot
//   gather   x rows -> expert-ordered rows, the input of the grouped GEMMs
//   swiglu   (g + gate bias, u + up bias) of each slot -> SwiGLU, plain or OAI
//   combine  out[t] (+)= sum over choices j of w[t][j] * (down row + down bias)
// Ordering: the IEEE total order (total_cmp), so -0 < +0 and NaNs order by sign
// and payload; equal keys keep the lower expert index first (the reference's
// unstable sort leaves ties unspecified).
#include "qh_internal.h"

#define QM_MAXE 256  // experts
#define QM_MAXK 16   // experts per token

// total_cmp key: larger key = later in the total order.
QH_DEV uint32_t qm_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One wavefront per token; lane l holds experts l, l + 64, l + 128, l + 192.
__global__ __launch_bounds__(256) void qm_route(const float* __restrict__ logits, const float* __restrict__ bias,
                                                int n_tok, int ne, int k, int renorm, int* __restrict__ ids,
                                                float* __restrict__ wts) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n_tok) return;  // uniform per wavefront
    float v[4];
    bool taken[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int e = lane + 64 * s;
        v[s] = e < ne ? logits[(size_t)t * ne + e] : 0.f;
        if (e < ne && bias) v[s] = v[s] + bias[e];
        taken[s] = e >= ne;
    }
    float top_v = 0.f;
    int top_e = 0;
    float tv[QM_MAXK];
    int te[QM_MAXK];
    for (int r = 0; r < k; r++) {
        // best untaken entry of this lane: larger key, then lower index
        uint32_t bk = 0;
        int be = 0x7fffffff;
        bool any = false;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t kk = qm_key(v[s]);
            if (!taken[s] && (!any || kk > bk)) {
                bk = kk;
                be = lane + 64 * s;
                any = true;
            }
        }
        // wavefront arg-max over (key, -index); lanes with nothing left use key 0, index max
        if (!any) bk = 0;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const uint32_t ok = __shfl_xor(bk, o);
            const int oe = __shfl_xor(be, o);
            if (ok > bk || (ok == bk && oe < be)) {
                bk = ok;
                be = oe;
            }
        }
#pragma unroll
        for (int s = 0; s < 4; s++)
            if (lane + 64 * s == be) taken[s] = true;
        // the value itself, from the lane that owns it
        float mine = 0.f;
#pragma unroll
        for (int s = 0; s < 4; s++)
            if (lane + 64 * s == be) mine = v[s];
        top_v = __shfl(mine, be & 63);
        top_e = be;
        tv[r] = top_v;
        te[r] = top_e;
    }
    float ex[QM_MAXK];
    float denom = 0.f;
    if (renorm) {
        // softmax over the chosen k: max folded from -inf with f32::max semantics
        float mx = -INFINITY;
        for (int r = 0; r < k; r++) mx = fmaxf(mx, tv[r]);
        for (int r = 0; r < k; r++) {
            ex[r] = expf(tv[r] - mx);
            denom = denom + ex[r];
        }
    } else {
        // softmax over all experts, the chosen k not renormalised
        float mx = -INFINITY;
#pragma unroll
        for (int s = 0; s < 4; s++)
            if (lane + 64 * s < ne) mx = fmaxf(mx, v[s]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        float part = 0.f;
#pragma unroll
        for (int s = 0; s < 4; s++)
            if (lane + 64 * s < ne) part += expf(v[s] - mx);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o);
        denom = part;
        for (int r = 0; r < k; r++) ex[r] = expf(tv[r] - mx);
    }
    if (lane < k) {
        // lane r writes choice r (k <= 16 < 64)
        float er = 0.f;
        int eid = 0;
        for (int r = 0; r < k; r++)
            if (r == lane) {
                er = ex[r];
                eid = te[r];
            }
        ids[(size_t)t * k + lane] = eid;
        wts[(size_t)t * k + lane] = __fdiv_rn(er, denom);
    }
}

// One workgroup of 16 wavefronts; wavefront w takes experts w, w + 16, ...
// and walks the (token, choice) slots in order 64 at a time, so the slot order
// inside an expert is token order, then choice order: deterministic.
__global__ __launch_bounds__(1024) void qm_plan(const int* __restrict__ ids, int n_slots, int k, int ne,
                                                int* __restrict__ tok_off, int* __restrict__ slot_of,
                                                int* __restrict__ slot_tok, int* __restrict__ slot_exp) {
    __shared__ int cnt[QM_MAXE], off[QM_MAXE + 1];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int p = threadIdx.x; p < n_slots; p += 1024) slot_of[p] = -1;  // ids outside [0, ne) get no slot
    for (int e = w; e < ne; e += 16) {
        int c = 0;
        for (int p0 = 0; p0 < n_slots; p0 += 64) {
            const int p = p0 + lane;
            c += __popcll(__ballot(p < n_slots && ids[p] == e));
        }
        if (lane == 0) cnt[e] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int s = 0;
        for (int e = 0; e < ne; e++) {
            off[e] = s;
            s += cnt[e];
        }
        off[ne] = s;
    }
    __syncthreads();
    for (int e = threadIdx.x; e <= ne; e += 1024) tok_off[e] = off[e];
    for (int e = w; e < ne; e += 16) {
        int base = off[e];
        for (int p0 = 0; p0 < n_slots; p0 += 64) {
            const int p = p0 + lane;
            const bool hit = p < n_slots && ids[p] == e;
            const uint64_t m = __ballot(hit);
            if (hit) {
                const int q = base + (int)__popcll(m & ((1ull << lane) - 1ull));
                slot_of[p] = q;
                slot_tok[q] = p / k;
                slot_exp[q] = e;
            }
            base += (int)__popcll(m);
        }
    }
}

// xg[q][:] = x[slot_tok[q]][:]
__global__ __launch_bounds__(256) void qm_gather(float* __restrict__ xg, const float* __restrict__ x,
                                                 const int* __restrict__ slot_tok, int d) {
    const int q = blockIdx.x;
    const float* src = x + (size_t)slot_tok[q] * d;
    float* dst = xg + (size_t)q * d;
    for (int i = blockIdx.y * 256 + threadIdx.x; i < d; i += 256 * gridDim.y) dst[i] = src[i];
}

// act[q][i] = swiglu(g[q][i] + gb[e][i], u[q][i] + ub[e][i]), e = slot_exp[q]
__global__ __launch_bounds__(256) void qm_swiglu(float* __restrict__ act, const float* __restrict__ g,
                                                 const float* __restrict__ u, const float* __restrict__ gb,
                                                 const float* __restrict__ ub, const int* __restrict__ slot_exp, int f,
                                                 int oai) {
    const int q = blockIdx.x, e = slot_exp[q];
    const size_t r = (size_t)q * f;
    for (int i = blockIdx.y * 256 + threadIdx.x; i < f; i += 256 * gridDim.y) {
        float gv = g[r + i], uv = u[r + i];
        if (gb) gv = gv + gb[(size_t)e * f + i];
        if (ub) uv = uv + ub[(size_t)e * f + i];
        if (oai) {
            const float xx = fminf(gv, 7.f), yy = fmaxf(-7.f, fminf(7.f, uv));
            act[r + i] = (xx / (1.f + expf(-1.702f * xx))) * (yy + 1.f);
        } else {
            act[r + i] = (gv / (1.f + expf(-gv))) * uv;
        }
    }
}

// out[t][i] = (accumulate ? out[t][i] : 0) + (sum over j in order of w * (yg + db))
__global__ __launch_bounds__(256) void qm_combine(float* __restrict__ out, const float* __restrict__ yg,
                                                  const int* __restrict__ slot_of, const float* __restrict__ wts,
                                                  const int* __restrict__ ids, const float* __restrict__ db, int k,
                                                  int d, int accumulate) {
    // `*a += rw * b` rounds the product and the sum separately: no FMA contraction here
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    for (int i = blockIdx.y * 256 + threadIdx.x; i < d; i += 256 * gridDim.y) {
        float acc = 0.f;
        for (int j = 0; j < k; j++) {
            const int q = slot_of[(size_t)t * k + j];
            if (q < 0) continue;
            float v = yg[(size_t)q * d + i];
            if (db) v = v + db[(size_t)ids[(size_t)t * k + j] * d + i];
            acc = acc + wts[(size_t)t * k + j] * v;
        }
        float* o = out + (size_t)t * d + i;
        *o = accumulate ? *o + acc : acc;
    }
}

static unsigned qm_ysplit(int n) { return (unsigned)((n + 1023) / 1024 < 64 ? (n + 1023) / 1024 : 64); }

hipError_t qh_moe_route(const float* logits, const float* bias, int n_tok, int ne, int k, int renorm, int* ids,
                        float* wts, hipStream_t st) {
    if (ne < 1 || ne > QM_MAXE || k < 1 || k > QM_MAXK || k > ne) return hipErrorInvalidValue;
    if (n_tok == 0) return hipSuccess;
    hipLaunchKernelGGL(qm_route, dim3((unsigned)((n_tok + 3) / 4)), dim3(256), 0, st, logits, bias, n_tok, ne, k,
                       renorm, ids, wts);
    return hipGetLastError();
}

hipError_t qh_moe_plan(const int* ids, int n_tok, int k, int ne, int* tok_off, int* slot_of, int* slot_tok,
                       int* slot_exp, hipStream_t st) {
    if (ne < 1 || ne > QM_MAXE || k < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(qm_plan, dim3(1), dim3(1024), 0, st, ids, n_tok * k, k, ne, tok_off, slot_of, slot_tok,
                       slot_exp);
    return hipGetLastError();
}

hipError_t qh_moe_gather(float* xg, const float* x, const int* slot_tok, int n_slots, int d, hipStream_t st) {
    if (n_slots == 0 || d == 0) return hipSuccess;
    hipLaunchKernelGGL(qm_gather, dim3((unsigned)n_slots, qm_ysplit(d)), dim3(256), 0, st, xg, x, slot_tok, d);
    return hipGetLastError();
}

hipError_t qh_moe_swiglu(float* act, const float* g, const float* u, const float* gb, const float* ub,
                         const int* slot_exp, int n_slots, int f, int oai, hipStream_t st) {
    if (n_slots == 0 || f == 0) return hipSuccess;
    hipLaunchKernelGGL(qm_swiglu, dim3((unsigned)n_slots, qm_ysplit(f)), dim3(256), 0, st, act, g, u, gb, ub,
                       slot_exp, f, oai);
    return hipGetLastError();
}

hipError_t qh_moe_combine(float* out, const float* yg, const int* slot_of, const float* wts, const int* ids,
                          const float* db, int n_tok, int k, int d, int accumulate, hipStream_t st) {
    if (n_tok == 0 || d == 0) return hipSuccess;
    hipLaunchKernelGGL(qm_combine, dim3((unsigned)n_tok, qm_ysplit(d)), dim3(256), 0, st, out, yg, slot_of, wts,
                       ids, db, k, d, accumulate);
    return hipGetLastError();
}

// Y[t][j] = sum_i W[j][i] x[t][i] for f32 W (the router GEMV, src/cuda.rs:672,
// over a batch): one wavefront per (token, row), float4 loads when rows are
// 16-byte aligned, a wave64 tree for the sum.
__global__ __launch_bounds__(256) void qm_gemm_f32(const float* __restrict__ W, const float* __restrict__ x,
                                                   float* __restrict__ y, int in_dim, int out_dim, int n, int vec4) {
    const int lane = threadIdx.x & 63, item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= n * out_dim) return;  // uniform per wavefront
    const int t = item / out_dim, j = item - t * out_dim;
    const float* wr = W + (size_t)j * in_dim;
    const float* xr = x + (size_t)t * in_dim;
    float acc = 0.f;
    if (vec4) {
        const float4* w4 = reinterpret_cast<const float4*>(wr);
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        for (int i = lane; i < in_dim / 4; i += 64) {
            const float4 a = w4[i], b = x4[i];
            acc = fmaf(a.x, b.x, acc);
            acc = fmaf(a.y, b.y, acc);
            acc = fmaf(a.z, b.z, acc);
            acc = fmaf(a.w, b.w, acc);
        }
    } else {
        for (int i = lane; i < in_dim; i += 64) acc = fmaf(wr[i], xr[i], acc);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) y[(size_t)t * out_dim + j] = acc;
}

hipError_t qh_launch_gemm_f32(const float* W, const float* x, float* y, int in_dim, int out_dim, int n,
                              hipStream_t st) {
    const int64_t items = (int64_t)n * out_dim;
    if (items == 0) return hipSuccess;
    if (items > ((int64_t)1 << 31) - 4) return hipErrorNotSupported;
    const int vec4 = in_dim % 4 == 0 && ((uintptr_t)W & 15u) == 0 && ((uintptr_t)x & 15u) == 0;
    hipLaunchKernelGGL(qm_gemm_f32, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, st, W, x, y, in_dim, out_dim, n,
                       vec4);
    return hipGetLastError();
}
