// qh_internal.h -- declarations shared by the translation units of libquartz_hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

// Block geometry, src/gguf.rs:172-191 (Q4_0/Q4_1 from the GGUF layout).
__host__ __device__ inline int qh_block_elems(uint32_t t) {
    switch (t) {
        case 0: case 1: case 30: return 1;
        case 2: case 3: case 6: case 7: case 8: case 20: return 32;
        case 10: case 12: case 13: case 14: case 16: case 17: case 21: case 22: return 256;
        default: return 0;
    }
}
__host__ __device__ inline uint32_t qh_block_bytes(uint32_t t) {
    switch (t) {
        case 0: return 4;
        case 1: case 30: return 2;
        case 2: return 18;
        case 3: return 20;
        case 6: return 22;
        case 7: return 24;
        case 8: return 34;
        case 10: return 84;
        case 12: return 144;
        case 13: return 176;
        case 14: return 210;
        case 16: return 66;
        case 17: return 74;
        case 20: return 18;
        case 21: return 110;
        case 22: return 82;
        default: return 0;
    }
}
__host__ __device__ inline size_t qh_type_size(uint32_t t, size_t n) {
    const int qk = qh_block_elems(t);
    return qk ? (n / (size_t)qk) * qh_block_bytes(t) : 0;
}

// Bit-exact decode of one block (qk elements) -- qh_dequant.hip.
__device__ void qh_decode_block(uint32_t type, const uint8_t* blk, float* out);
__device__ bool qh_decode_part16(uint32_t type, const uint8_t* blk, int part, float* out);

hipError_t qh_launch_mmv16(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                           hipStream_t st);
hipError_t qh_launch_mmq(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                         int n, hipStream_t st);
hipError_t qh_launch_mmq_mixed(uint32_t t1, int c1, const uint8_t* const* W1, float* const* Y1, const int* o1,
                               uint32_t t2, int c2, const uint8_t* const* W2, float* const* Y2, const int* o2,
                               const float* x, int n, int in_dim, hipStream_t st, const float* nw = nullptr);
// n (2..32) tokens of x, RMS-normalised with nw, through count matrices of one
// type: the norm and the digitisation in one launch, then the batched kernel
// on those images.  img_done: the images already hold this x and nw (an
// earlier call of the same n, x and nw, on the same stream): no norm launch.
// hipErrorNotSupported when the shapes do not fit.
hipError_t qh_launch_mmq_norm(uint32_t type, int count, const uint8_t* const* W, float* const* Y, const int* out_dims,
                              const float* x, const float* nw, int n, int in_dim, hipStream_t st,
                              bool img_done = false);
hipError_t qh_launch_mmq_moe_dev(uint32_t type, int sets, const uint8_t* const* E, float* const* Y, int n_exp,
                                 const int* tok_off, int max_tokens, const float* X, const float* X2, int in_dim,
                                 int out_dim, int accum, hipStream_t st);
hipError_t qh_launch_mmq_grouped(uint32_t type, int count, const uint8_t* const* W, const float* const* X,
                                 float* const* Y, const int* n, const int* out_dims, int in_dim, hipStream_t st,
                                 const float* const* X2 = nullptr, int accum = 0, const float* nw = nullptr);
hipError_t qh_launch_mmv16_multi(uint32_t type, const uint8_t* const* Ws, float* const* ys, const int* outs, int nm,
                                 const float* x, int in_dim, hipStream_t st, const float* norm_w, int accum,
                                 bool swiglu_pair = false);
hipError_t qh_launch_mmv16_mix(uint32_t t1, const uint8_t* const* Ws1, float* const* ys1, const int* outs1, int n1,
                               uint32_t t2, const uint8_t* const* Ws2, float* const* ys2, const int* outs2, int n2,
                               const float* x, int in_dim, const float* nw, int accum, hipStream_t st);
hipError_t qh_launch_mmv16_mix_tokens(uint32_t t1, const uint8_t* const* Ws1, float* const* ys1, const int* outs1,
                                      const int* ldys1, int n1, uint32_t t2, const uint8_t* const* Ws2,
                                      float* const* ys2, const int* outs2, const int* ldys2, int n2, const float* x,
                                      int ldx, int ntok, int in_dim, const float* nw, int accum, hipStream_t st);
hipError_t qh_launch_mmv16_tokens(uint32_t type, int nm, const uint8_t* const* Ws, float* const* ys, const int* outs,
                                  const int* ldys, const float* x, int ldx, int ntok, int in_dim, int accum,
                                  hipStream_t st, const float* nw = nullptr);
hipError_t qh_launch_mmq_q81(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                             int rows, int ref_rows, int mps, hipStream_t st);
hipError_t qh_launch_mmv(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                         hipStream_t st);
// QUARTZ_HIP_KERNEL=valu selects the lane-per-unit VALU kernels instead of the
// matrix-core ones (for A/B measurement); read once per process.
bool qh_force_valu();
hipError_t qh_launch_gemv(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                          hipStream_t st);
hipError_t qh_launch_gemm(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                          int n, hipStream_t st);
void qh_set_error(const char* msg);
// Decode-step glue kernels (qh_glue.hip).
hipError_t qh_glue_vec(int op, float* dst, const float* src, float scale, int n, hipStream_t st);
hipError_t qh_glue_rms_norm(float* out, const float* x, const float* w, int n, hipStream_t st, int rows = 1);
// RMS norm of n_tok <= 32 token rows fused with the batched GEMM's x images
// (slot 0 of img; two halves past 16 tokens); in_dim % 256 == 0, in_dim <= 4096.
hipError_t qh_glue_norm_image(unsigned char* img, const float* x, const float* w, int n_tok, int in_dim,
                              hipStream_t st);
hipError_t qh_glue_rope(float* x, int n_heads, int head_dim, int pos, float theta, float yarn_scale, int orig_ctx,
                        int neox, hipStream_t st);
hipError_t qh_glue_kv_append(float* kc, float* vc, const float* k, const float* v, int pos, int kv_dim,
                             hipStream_t st);
hipError_t qh_glue_attn(int op, float* dst, const float* a, const float* b, const float* sinks, int n_heads,
                        int n_kv, int seq, int hd, int kv_dim, int max_seq, float scale, hipStream_t st);
hipError_t qh_glue_attention_decode(float* out, const float* q, const float* kc, const float* vc, const float* sinks,
                                    int n_heads, int n_kv, int seq, int hd, int kv_dim, float scale, hipStream_t st);
hipError_t qh_glue_attention_step(float* out, const float* q, const float* k, const float* v, float* kc, float* vc,
                                  const float* sinks, int n_heads, int n_kv, int hd, int kv_dim, int pos, float theta,
                                  float yarn_scale, int orig_ctx, int neox, float scale, hipStream_t st, int n_seq = 1,
                                  size_t cache_stride = 0, const int* pos_dev = nullptr);
hipError_t qh_glue_greedy(const float* logits, size_t stride, int rows, int n, int* tokens, int* pos, hipStream_t st);
hipError_t qh_launch_gemm_f32(const float* W, const float* x, float* y, int in_dim, int out_dim, int n,
                              hipStream_t st);
hipError_t qh_moe_route(const float* logits, const float* bias, int n_tok, int ne, int k, int renorm, int* ids,
                        float* wts, hipStream_t st);
hipError_t qh_moe_plan(const int* ids, int n_tok, int k, int ne, int* tok_off, int* slot_of, int* slot_tok,
                       int* slot_exp, hipStream_t st);
hipError_t qh_moe_gather(float* xg, const float* x, const int* slot_tok, int n_slots, int d, hipStream_t st);
hipError_t qh_moe_swiglu(float* act, const float* g, const float* u, const float* gb, const float* ub,
                         const int* slot_exp, int n_slots, int f, int oai, hipStream_t st);
hipError_t qh_moe_combine(float* out, const float* yg, const int* slot_of, const float* wts, const int* ids,
                          const float* db, int n_tok, int k, int d, int accumulate, hipStream_t st);
hipError_t qh_glue_swiglu(int oai, float* out, const float* gate, const float* up, int n, hipStream_t st);
hipError_t qh_glue_embed(float* out, size_t out_stride, const uint8_t* data, uint32_t type, const int* tokens,
                         int n_tok, int embed_dim, hipStream_t st, const int* tok_dev = nullptr,
                         int vocab = 0);
hipError_t qh_launch_dequant(uint32_t type, const uint8_t* W, float* out, size_t n_elems, hipStream_t st);

// Integer value of a tuning variable: dflt when it is unset, empty or not a
// whole decimal number.
static inline int qh_env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    if (!e || !*e) return dflt;
    char* end = nullptr;
    const long v = strtol(e, &end, 10);
    return (*end == '\0' && v >= -(1L << 30) && v <= (1L << 30)) ? (int)v : dflt;
}
