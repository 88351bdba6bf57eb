/*
 * quartz_hip.h -- C ABI of libquartz_hip.so, the MI355X (gfx950) quantized
 * dequant-GEMV backend for Quartz.
 *
 * Drop-in for the `cuda_*` extern block of Quartz's CUDA backend
 * (src/cuda.rs:6-55, defined in src/cuda_kernels.cu:1025-1125): every symbol
 * below with a `cuda_` twin takes the same arguments in the same order with the
 * same meaning, with `hip_` in place of `cuda_`.  Differences, all additive:
 *   - entry points return an int status (0 = ok, negative = error, see QH_ERR_*)
 *     where the reference returns void;
 *   - `_async` variants take a hipStream_t passed as `void*` (NULL = the legacy
 *     default stream, which is what the synchronous forms use);
 *   - hip_gemm / hip_gemm_async (batched tokens) and hip_dequant are new: the
 *     reference has them only on the CPU (src/dequant.rs:143, :1239).
 *
 * Layouts: d_data points at out_dim contiguous GGUF rows of in_dim/QK blocks (no
 * row padding; GGUF row j holds elements [j*in_dim, (j+1)*in_dim)).  x and y are
 * f32.  Batched activations are token-major: x[n][in_dim], y[n][out_dim].
 * y is overwritten, never accumulated.  Buffers are caller-owned device memory;
 * no entry point allocates device memory.  Calls on one stream are ordered; the
 * library keeps no per-call host state and is safe to call from several host
 * threads on distinct streams, with one exception: hip_gemm / hip_gemm_grouped /
 * hip_gemm_moe (and their _async forms) with n >= 2 on Q4_K, Q5_K, Q6_K, IQ3_S
 * or IQ2_XXS stage the digitised activations and split-K partials in static
 * device arrays (104.25 MiB: 64 MiB of split-K partials, 40 MiB of x images and
 * 256 KiB of counters, one set per device), so such calls that overlap on
 * one device must be serialised by the caller (e.g. one stream per device).
 */
#ifndef QUARTZ_HIP_H
#define QUARTZ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define QH_OK 0
#define QH_ERR_TYPE (-1)  /* unsupported ggml_type (y is zero-filled, as the reference does) */
#define QH_ERR_DIMS (-2)  /* in_dim <= 0, out_dim/n < 0, or in_dim not a multiple of the block size */
#define QH_ERR_NULL (-3)  /* null device pointer with non-empty dims */
#define QH_ERR_HIP (-4)   /* HIP runtime error; hip_last_error() has the message */
#define QH_ERR_RANGE (-5) /* argument outside a documented limit */
#define QH_ERR_FORMAT (-6) /* malformed or unsupported GGUF file (message in hip_last_error) */
#define QH_ERR_IO (-7)     /* file cannot be opened, mapped or written */

/* GGML type ids handled: 0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 6 Q5_0, 7 Q5_1, 8 Q8_0,
 * 10 Q2_K, 12 Q4_K, 13 Q5_K, 14 Q6_K, 16 IQ2_XXS, 17 IQ2_XS, 20 IQ4_NL,
 * 21 IQ3_S, 22 IQ2_S, 30 BF16  (src/gguf.rs:172-191; 2 and 3 are GGUF types the
 * reference lacks). */

/* y[j] = sum_k W[j,k] x[k].  Replaces cuda_gemv (src/cuda_kernels.cu:1046-1077,
 * Rust decl src/cuda.rs:7-8). */
int hip_gemv(uint32_t ggml_type, const uint8_t* d_data, const float* d_x, float* d_y, int in_dim, int out_dim);
int hip_gemv_async(uint32_t ggml_type, const uint8_t* d_data, const float* d_x, float* d_y, int in_dim,
                   int out_dim, void* stream);

/* y[k] = W[k] x for k < count (1..4): several GEMVs that share x, the type and
 * in_dim (a layer's q and k projections, or gate and up) in one launch.  W, y and
 * out_dims are host arrays of count device pointers / row counts.  Each y[k] is
 * bit-identical to hip_gemv(type, W[k], x, y[k], in_dim, out_dims[k]).  No
 * counterpart in the reference, which calls cuda_gemv once per matrix
 * (src/cuda.rs:556-562, :773-788); this is the decode-step launch fusion. */
int hip_gemv_multi(uint32_t ggml_type, int count, const uint8_t* const* W, float* const* y, const int* out_dims,
                   const float* d_x, int in_dim);
int hip_gemv_multi_async(uint32_t ggml_type, int count, const uint8_t* const* W, float* const* y,
                         const int* out_dims, const float* d_x, int in_dim, void* stream);

/* y[k] (op)= W[k] x' for k < count (1..4) matrices sharing x, type and in_dim,
 * with the decode step's neighbours of a GEMV fused in:
 *   norm_w != NULL: x' = rms_norm(x) * norm_w (eps 1e-5), the reference's
 *     cuda_rms_norm before the q/k/v, gate/up and lm_head GEMVs
 *     (src/cuda.rs:549-562, :729-733, :773-781, :824-833);
 *   accumulate != 0: y[k] += W[k] x' instead of =, the residual cuda_vec_add
 *     after the o and down GEMVs (src/cuda.rs:647-662, :782-799).
 * One launch for Q4_K/Q5_K/Q6_K when the norm's x fits one workgroup
 * (in_dim <= 4096) or without the norm; otherwise the separate kernels run on
 * `scratch` (device, in_dim + max(out_dims) floats; may be NULL when the fused
 * kernel applies, QH_ERR_NULL if it was needed).  x must not alias any y[k].
 * Results are within the GEMV tolerance of the separate-kernel sequence (the
 * row scale rsqrt(mean(x^2)+eps) is applied after the dot instead of before). */
int hip_gemv_fused_async(uint32_t ggml_type, int count, const uint8_t* const* W, float* const* y,
                         const int* out_dims, const float* d_x, const float* norm_w, int accumulate, int in_dim,
                         float* scratch, void* stream);

/* Y[t][j] = sum_k W[j,k] X[t][k] for t < n (token-major).  GPU counterpart of
 * dequant::gemm (src/dequant.rs:143-200); n == 1 is hip_gemv.  For n >= 2 the
 * matrix-core path reads the weights once per 32 tokens (see the note above on
 * its device scratch); x is kept to 23 bits below each token's largest |x| per
 * 256 elements, so results stay within 1e-3 relative L2 per token (observed
 * ~1e-6) with activation outliers up to thousands of times the RMS. */
int hip_gemm(uint32_t ggml_type, const uint8_t* d_data, const float* d_x, float* d_y, int in_dim, int out_dim,
             int n);
int hip_gemm_async(uint32_t ggml_type, const uint8_t* d_data, const float* d_x, float* d_y, int in_dim,
                   int out_dim, int n, void* stream);

/* Y[k] = X[k] W[k]^T for k < count: several batched GEMMs of one type and
 * in_dim in as few launches as the device scratch allows (one weight pass per 16
 * tokens of each matrix).  W, x, y, n and out_dims are host arrays of count
 * entries: device pointers, tokens n[k] >= 0 (x[k] is [n[k]][in_dim], y[k] is
 * [n[k]][out_dims[k]], token-major) and row counts.  Matrices that share an x
 * pointer (a layer's q/k/v, gate/up) share its digitisation.  No counterpart in
 * the reference, whose CPU gemm (src/dequant.rs:143-200) takes one matrix. */
int hip_gemm_grouped(uint32_t ggml_type, int count, const uint8_t* const* W, const float* const* x,
                     float* const* y, const int* n, const int* out_dims, int in_dim);
int hip_gemm_grouped_async(uint32_t ggml_type, int count, const uint8_t* const* W, const float* const* x,
                           float* const* y, const int* n, const int* out_dims, int in_dim, void* stream);

/* hip_gemm_grouped with the batched decode step's neighbours fused in:
 * x_up != NULL: the GEMM's input is silu(x[k]) * x_up[k] (x[k] the gate rows,
 *   x_up[k] the up rows, token-major [n[k]][in_dim]): cuda_swiglu before the down
 *   projection, applied while x is digitised (src/cuda.rs:785-792);
 * accumulate != 0: y[k] += product, the residual cuda_vec_add
 *   (src/cuda.rs:647-662, :797-799).
 * One prologue + one main launch on the matrix cores when every n[k] >= 2 and
 * the type has the batched kernel; otherwise separate kernels on scratch
 * (device, n*in_dim + n*max(out_dims) floats per matrix in turn; NULL is
 * QH_ERR_NULL then).  x / x_up must not alias y. */
int hip_gemm_grouped_ex_async(uint32_t ggml_type, int count, const uint8_t* const* W, const float* const* x,
                              const float* const* x_up, float* const* y, const int* n, const int* out_dims,
                              int in_dim, int accumulate, float* scratch, void* stream);

/* y[k][t][:] = W[k] (rms_norm(x[t]) * norm_w) for count matrices of one type
 * sharing the n token rows of x (token-major, in_dim each): the RMS norm
 * (eps 1e-5, cuda_rms_norm's formula, src/cuda_kernels.cu:563-575) fused into
 * the GEMMs that read it, as forward_gpu_step's norm + q/k/v and norm +
 * gate/up pairs (src/cuda.rs:549-562, :662-665, :773-788) for a batch.  The norm
 * fuses into the GEMV kernel for n <= 4 tokens (n = 3, 4 on matrices up to
 * 16 MB); otherwise the rows are normalised into scratch (n * in_dim floats)
 * and then multiplied, and a null scratch returns QH_ERR_NULL. */
int hip_gemm_grouped_norm_async(uint32_t ggml_type, int count, const uint8_t* const* d_data, const float* d_x,
                                const float* d_norm_w, float* const* d_y, int n, const int* out_dims, int in_dim,
                                float* d_scratch, void* stream);

/* hip_gemm_grouped_norm_async without the scratch argument: the normalised
 * rows go to a static device array of the library (4 MB, one per device, kept
 * until the process ends), so the call allocates nothing and needs no
 * workspace from the caller.  No counterpart in the reference; for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  n * in_dim must be <= 1048576
 * (QH_ERR_RANGE otherwise, with the limit in hip_last_error()).  Every call on
 * one device shares that array: calls that overlap on one device (different
 * streams) race and must be serialised by the caller. */
int hip_gemm_grouped_norm_static_async(uint32_t ggml_type, int count, const uint8_t* const* d_data, const float* d_x,
                                       const float* d_norm_w, float* const* d_y, int n, const int* out_dims,
                                       int in_dim, void* stream);

/* hip_gemm_grouped_norm_async over count (1..8) matrices of mixed types
 * (types[k] for W[k]): a batch's norm + q/k/v when v has its own type, as
 * Q4_K_M models have (src/cuda.rs:549-562).  For 2..4 tokens, two types among
 * Q4_K/Q5_K + Q6_K and in_dim <= 4096, one launch computes every matrix; each
 * token's result then equals the per-type call's bit for bit.  For 5..32
 * tokens of Q4_K + Q6_K, one launch normalises the rows straight into the
 * batched kernel's x images (in_dim <= 4096; otherwise, up to 16 tokens, into
 * d_scratch, n * in_dim floats) and both types run in one batched matrix-core
 * launch; each token's result equals the per-type batched call's within
 * rounding (the split of K may differ).  For 5..16 tokens of one matrix-core
 * type, and 17..32 tokens of any matrix-core types, with in_dim <= 4096, the
 * same fused norm feeds each type's batched launch, bit-identical to the
 * per-type call.  Otherwise one hip_gemm_grouped_norm_async per type, with its
 * scratch rule. */
int hip_gemm_group_norm_async(int count, const uint32_t* types, const uint8_t* const* d_data, const float* d_x,
                              const float* d_norm_w, float* const* d_y, int n, const int* out_dims, int in_dim,
                              float* d_scratch, void* stream);

/* Y[t][j] for t < rows with ggml-cuda's int8 MMQ rounding (Q4_K, Q6_K): the
 * GPU twin of the reference's CPU oracles gemm_q4k_q8_1_mmq / gemm_q6k_q8_1_mmq
 * and their _stream_k forms (src/dequant.rs:202-645), bit-exact to them: x is
 * quantised to Q8_1 per 32 values (f16 scale and sum for Q4_K, f32 scale for
 * Q6_K), weight scale pairs are rounded to f16, dots are integer, and the f32
 * accumulation runs in block order with fused multiply-adds.  reference_rows > 0
 * and multiprocessors > 0 reproduce ggml-cuda's stream-K split for a launch of
 * reference_rows rows on that many multiprocessors (cuda_stream_k_cut).  Token-
 * major X [rows][in_dim] (16-byte aligned), Y [rows][out_dim]; in_dim % 256 == 0.
 * A compatibility mode for ggml-identical results; hip_gemm is the fast path. */
int hip_gemm_q8_1_mmq(uint32_t ggml_type, const uint8_t* d_data, const float* d_x, float* d_y, int in_dim,
                      int out_dim, int rows, int reference_rows, int multiprocessors);
int hip_gemm_q8_1_mmq_async(uint32_t ggml_type, const uint8_t* d_data, const float* d_x, float* d_y, int in_dim,
                            int out_dim, int rows, int reference_rows, int multiprocessors, void* stream);

/* Mixture-of-experts layer GEMMs over gathered tokens: for i < n_sel, expert
 * e = expert_ids[i] (its weights at d_experts + e * hip_type_size(type,
 * in_dim*out_dim), the expert slicing of src/cuda.rs:250-258 / :723-725)
 * multiplies tokens tok_off[i] .. tok_off[i+1]-1 of d_x[.][in_dim] into the same
 * rows of d_y[.][out_dim].  expert_ids and tok_off (n_sel + 1 entries, non-
 * decreasing) are host arrays.  Generalises cuda_gemv_moe4
 * (src/cuda_kernels.cu:1085-1106: <= 4 experts, one token each) to any number
 * of experts and tokens, as the per-expert loop of src/cuda.rs:667-798 needs. */
int hip_gemm_moe(uint32_t ggml_type, const uint8_t* d_experts, int n_sel, const int* expert_ids, const int* tok_off,
                 const float* d_x, float* d_y, int in_dim, int out_dim);
int hip_gemm_moe_async(uint32_t ggml_type, const uint8_t* d_experts, int n_sel, const int* expert_ids,
                       const int* tok_off, const float* d_x, float* d_y, int in_dim, int out_dim, void* stream);

/* The same expert GEMMs with the token ranges on the device: for s < n_sets
 * (1, or 2 for a gate/up pair sharing x) and e < n_exp, the gathered rows
 * t = d_tok_off[e] .. d_tok_off[e+1]-1 of d_x (each expert's x digitised once
 * for both sets) multiply expert e of d_experts[s] (at + e * hip_type_size(type,
 * in_dim*out_dim)) into the same rows of d_y[s] (y += with accumulate).  With
 * d_x_up, x is silu(d_x) * d_x_up (a down projection after SwiGLU).  max_tokens
 * bounds any expert's token count (the launch holds ceil(max_tokens/16) token
 * chunks per expert, of 32 tokens when max_tokens > 16; the empty ones exit at
 * once), so nothing is read back to the host and the call can be captured in a
 * HIP graph.  An expert with more rows than the chunks cover (a max_tokens
 * below its count) gets only its first chunks' rows computed; its later rows
 * of d_y are left as they were (the bound is the caller's: n_tok * k, or the
 * batch size, always holds).  Replaces the host
 * round trip of the per-expert loop of src/cuda.rs:667-798 (the reference
 * copies the router logits back to build it).  Matrix-core types only (Q4_K,
 * Q5_K, Q6_K, IQ3_S, IQ2_XXS; QH_ERR_TYPE otherwise), in_dim % 256 == 0,
 * 16-byte aligned d_x. */
int hip_gemm_moe_dev_async(uint32_t ggml_type, int n_sets, const uint8_t* const* d_experts, float* const* d_y,
                           int n_exp, const int* d_tok_off, int max_tokens, const float* d_x, const float* d_x_up,
                           int in_dim, int out_dim, int accumulate, void* stream);

/* Up to 4 expert GEMVs in one call.  Replaces cuda_gemv_moe4
 * (src/cuda_kernels.cu:1085-1106, Rust decl src/cuda.rs:39-45); any type. */
int hip_gemv_moe4(uint32_t ggml_type, const uint8_t* w0, const uint8_t* w1, const uint8_t* w2,
                  const uint8_t* w3, const float* xi0, const float* xi1, const float* xi2, const float* xi3,
                  float* o0, float* o1, float* o2, float* o3, int n_act, int in_dim, int out_dim);

/* Bit-exact decode of n_elems elements to f32 on the GPU.  GPU counterpart of
 * dequant::dequant (src/dequant.rs:1239-1258); n_elems must be a multiple of
 * the block size. */
int hip_dequant(uint32_t ggml_type, const uint8_t* d_data, float* d_out, size_t n_elems);
int hip_dequant_async(uint32_t ggml_type, const uint8_t* d_data, float* d_out, size_t n_elems, void* stream);

/* Byte size of n_elems elements of ggml_type; 0 for an unsupported type.
 * Mirrors ggml_type_size (src/gguf.rs:172-191), which panics instead. */
size_t hip_type_size(uint32_t ggml_type, size_t n_elems);

/* Memory.  Replace cuda_alloc / cuda_drop / cuda_h2d / cuda_d2h / cuda_sync /
 * cuda_mem_info (src/cuda_kernels.cu:1042-1044, 1109-1125).  hip_alloc returns
 * NULL on failure (256-byte aligned otherwise); h2d/d2h are blocking. */
void* hip_alloc(size_t bytes);
void hip_drop(void* ptr);
int hip_h2d(void* dst, const void* src, size_t bytes);
int hip_d2h(void* dst, const void* src, size_t bytes);
int hip_sync(void);
int hip_mem_info(size_t* free_b, size_t* total_b);
/* Copies ordered on a stream (no counterpart in the reference, whose copies are
 * blocking); with pageable host memory they return once the source is read. */
int hip_h2d_async(void* dst, const void* src, size_t bytes, void* stream);
int hip_d2h_async(void* dst, const void* src, size_t bytes, void* stream);

/* Streams and HIP graphs through the C ABI (no counterpart in the reference,
 * which launches every kernel eagerly): a host that reaches HIP only through
 * this library records a decode step once and replays it per token.
 *   hip_stream_create: a new non-blocking stream at the default priority;
 *   hip_graph_begin: start capturing `stream` (not the null stream; thread-local
 *     capture mode); every _async call on it is recorded, not run;
 *   hip_graph_end: stop, instantiate, and return the executable graph in *exec;
 *   hip_graph_launch: replay it on a stream; hip_graph_destroy frees it.
 * A captured call keeps the argument values it was given.  To replay one step
 * at consecutive positions, capture the _dev entries (hip_attention_step_dev_async,
 * hip_embed_lookup_dev_async), which read the position and the token ids from
 * device memory at run time: write them (hip_h2d_async) before each replay, or
 * end the step with hip_greedy_next_async, which writes the next token and
 * advances the position on the device. */
int hip_stream_create(void** stream);
int hip_stream_sync(void* stream);
void hip_stream_destroy(void* stream);
int hip_graph_begin(void* stream);
int hip_graph_end(void* stream, void** exec);
int hip_graph_launch(void* exec, void* stream);
void hip_graph_destroy(void* exec);

/* IQ codebooks.  Replace cuda_set_iq3s_grid / _iq2s_grid / _iq2xxs_grid /
 * _iq2xs_grid / cuda_set_ksigns (src/cuda_kernels.cu:1027-1041).  The library is
 * built with ggml's codebooks already resident, so calling these is optional;
 * they overwrite the device tables (idempotent for the standard tables).
 * ksigns is a closed form (i | parity(i) << 7) in this library: hip_set_ksigns
 * only checks that the table it is given is that one (QH_ERR_RANGE if not). */
int hip_set_iq3s_grid(const uint32_t* host);
int hip_set_iq2s_grid(const uint64_t* host);
int hip_set_iq2xxs_grid(const uint64_t* host);
int hip_set_iq2xs_grid(const uint64_t* host);
int hip_set_ksigns(const uint8_t* host);

/* Diagnostics. */
const char* hip_status_string(int status);
/* Device timestamps for timing work inside captured HIP graphs (no counterpart in
 * the reference; for benchmarks): a one-thread kernel on `stream` writes the
 * device's constant-rate wall clock (s_memrealtime) to *dst when it runs, i.e.
 * after the stream's previous work completes.  hip_wallclock_khz gives that
 * clock's rate (0 on failure). */
int hip_timestamp_async(uint64_t* dst, void* stream);
int hip_wallclock_khz(void);
const char* hip_last_error(void); /* last HIP error seen on this host thread ("" if none) */

/* ---------------------------------------------------------------- decode-step glue
 * The kernels between the GEMVs of a decode step, twins of the reference's
 * forward-pass helpers (src/cuda_kernels.cu:1129-1290, Rust decls
 * src/cuda.rs:20-55), same arguments and formulas; f32 results differ only by
 * summation order (wave64 reductions).  Plain forms run on the default stream,
 * _async forms on the given one.  hip_attention_decode is new: the three
 * attention kernels fused into one launch (seq_len <= 16384; QH_ERR_RANGE past
 * it), sinks may be NULL (no sink).  hip_embed_lookup decodes any supported type
 * bit-exactly (the reference handles Q5_1, IQ4_NL and BF16). */
int hip_vec_add(float* dst, const float* src, int n);                                  /* dst += src */
int hip_vec_add_async(float* dst, const float* src, int n, void* stream);
int hip_vec_scale_add(float* dst, const float* src, float scale, int n);                /* dst += scale*src */
int hip_vec_scale_add_async(float* dst, const float* src, float scale, int n, void* stream);
int hip_vec_zero(float* dst, int n);
int hip_vec_zero_async(float* dst, int n, void* stream);
int hip_rms_norm(float* out, const float* x, const float* w, int n);                    /* eps 1e-5; out may be x */
int hip_rms_norm_async(float* out, const float* x, const float* w, int n, void* stream);
/* rows token-major rows of n: out[r] = rms_norm(x[r]) * w, one launch (batched decode). */
int hip_rms_norm_rows_async(float* out, const float* x, const float* w, int rows, int n, void* stream);
int hip_rope_yarn(float* x, int n_heads, int head_dim, int pos, float theta, float yarn_scale, int yarn_orig_ctx,
                  int neox);
int hip_rope_yarn_async(float* x, int n_heads, int head_dim, int pos, float theta, float yarn_scale,
                        int yarn_orig_ctx, int neox, void* stream);
int hip_kv_append(float* k_cache, float* v_cache, const float* k, const float* v, int pos, int kv_dim);
int hip_kv_append_async(float* k_cache, float* v_cache, const float* k, const float* v, int pos, int kv_dim,
                        void* stream);
int hip_attn_score(float* scores, const float* q, const float* k_cache, int seq_len, int head_dim, int kv_dim,
                   int kv_head_off, float scale);
int hip_softmax_sink(float* x, int n, float sink);                                     /* sink <= -1e29: none */
int hip_attn_values(float* out, const float* scores, const float* v_cache, int seq_len, int head_dim, int kv_dim,
                    int kv_head_off);
int hip_attn_score_all(float* scores, const float* q, const float* k_cache, int n_heads, int n_kv_heads, int seq_len,
                       int head_dim, int kv_dim, int max_seq, float scale);
int hip_attn_score_all_async(float* scores, const float* q, const float* k_cache, int n_heads, int n_kv_heads,
                             int seq_len, int head_dim, int kv_dim, int max_seq, float scale, void* stream);
int hip_softmax_sink_all(float* scores, int n_heads, int seq_len, int max_seq, const float* sinks);
int hip_softmax_sink_all_async(float* scores, int n_heads, int seq_len, int max_seq, const float* sinks,
                               void* stream);
int hip_attn_values_all(float* out, const float* scores, const float* v_cache, int n_heads, int n_kv_heads,
                        int seq_len, int head_dim, int kv_dim, int max_seq);
int hip_attn_values_all_async(float* out, const float* scores, const float* v_cache, int n_heads, int n_kv_heads,
                              int seq_len, int head_dim, int kv_dim, int max_seq, void* stream);
int hip_attention_decode(float* out, const float* q, const float* k_cache, const float* v_cache, const float* sinks,
                         int n_heads, int n_kv_heads, int seq_len, int head_dim, int kv_dim, float scale);
int hip_attention_decode_async(float* out, const float* q, const float* k_cache, const float* v_cache,
                               const float* sinks, int n_heads, int n_kv_heads, int seq_len, int head_dim, int kv_dim,
                               float scale, void* stream);
int hip_swiglu(float* out, const float* gate, const float* up, int n);
int hip_swiglu_async(float* out, const float* gate, const float* up, int n, void* stream);
int hip_swiglu_oai(float* out, const float* gate, const float* up, int n);
int hip_swiglu_oai_async(float* out, const float* gate, const float* up, int n, void* stream);

/* Mixture-of-experts routing and gather/scatter on the device, for a batch of
 * n_tok tokens (all arrays device memory, token-major).  The reference routes
 * on the host after copying the router logits back (src/cuda.rs:670-700,
 * src/main.rs:964-993) and scale-adds each chosen expert's output
 * (src/cuda.rs:703-798, src/main.rs:995-1040).  The layer is:
 *   hip_gemm(F32 router) -> hip_moe_route -> hip_moe_plan -> hip_moe_gather ->
 *   gate/up GEMMs per expert over its slot range -> hip_moe_swiglu ->
 *   hip_gemm_moe (down) -> hip_moe_combine.
 * route: logits[n_tok][n_exp] (+ router_bias[n_exp] if non-null) -> the top k
 *   experts per token in total_cmp descending order (equal keys: lower index
 *   first) in ids[n_tok][k], and weights[n_tok][k]: softmax over the chosen k
 *   (renorm != 0: Mixtral, Qwen-MoE, gpt-oss) or the chosen entries of a softmax
 *   over all n_exp logits (renorm == 0: OLMoE).  n_exp <= 256, k <= 16.
 * plan: ids -> tok_off[n_exp + 1] (expert e's slots are tok_off[e] ..
 *   tok_off[e+1]-1, in token then choice order), slot_of[n_tok][k] (the slot of
 *   each choice; -1 for an id outside [0, n_exp)), slot_tok[] and slot_exp[]
 *   (token and expert of each slot).  Copy tok_off to the host to size the
 *   expert GEMMs (the reference copies the logits at the same point).
 * gather: xg[q] = x[slot_tok[q]] for q < n_slots, rows of dim floats.
 * swiglu: act[q] = swiglu(gate[q] + gate_bias[e], up[q] + up_bias[e]),
 *   e = slot_exp[q]; biases may be null; oai != 0 is the clamped gpt-oss form.
 * combine: out[t] = (accumulate ? out[t] : 0) + sum over j = 0..k-1, in order,
 *   of weights[t][j] * (y_slots[slot_of[t][j]] + down_bias[ids[t][j]]), each
 *   product and sum rounded separately as the reference's `*a += rw * b`. */
int hip_moe_route_async(const float* logits, const float* router_bias, int n_tok, int n_exp, int k, int renorm,
                        int* ids, float* weights, void* stream);
int hip_moe_plan_async(const int* ids, int n_tok, int k, int n_exp, int* tok_off, int* slot_of, int* slot_tok,
                       int* slot_exp, void* stream);
int hip_moe_gather_async(float* xg, const float* x, const int* slot_tok, int n_slots, int dim, void* stream);
int hip_moe_swiglu_async(float* act, const float* gate, const float* up, const float* gate_bias, const float* up_bias,
                         const int* slot_exp, int n_slots, int ffn_dim, int oai, void* stream);
int hip_moe_combine_async(float* out, const float* y_slots, const int* slot_of, const float* weights, const int* ids,
                          const float* down_bias, int n_tok, int k, int dim, int accumulate, void* stream);
/* hip_gemv_fused over count (1..8) matrices of any types sharing x (per-matrix
 * types[k]): the projections of one input, e.g. a Q4_K_M layer's q and k
 * (Q4_K) with v (Q6_K).  Two matrix-core types (Q4_K, Q5_K, Q6_K; <= 4
 * matrices each) go out as one launch whose workgroups split between the two
 * formats; otherwise one hip_gemv_fused call per type.  No counterpart in the
 * reference (one cuda_gemv per matrix, src/cuda.rs:556-562); results equal
 * hip_gemv_fused's per type within the GEMV tolerance. */
int hip_gemv_group_async(int count, const uint32_t* types, const uint8_t* const* W, float* const* y,
                         const int* out_dims, const float* d_x, const float* norm_w, int accumulate, int in_dim,
                         float* scratch, void* stream);

/* act = silu(W_gate x') * (W_up x'), x' = rms_norm(x) * norm_w (norm_w NULL: x'
 * = x): the dense FFN's cuda_rms_norm + two cuda_gemv + cuda_swiglu
 * (src/cuda.rs:729-733, :773-792) in one launch for Q4_K/Q5_K/Q6_K (the gate
 * and up tiles of a row block go to one workgroup, which applies the SwiGLU
 * before writing).  Other types / shapes run the separate kernels on scratch
 * (in_dim + 2 * ffn_dim floats; NULL is QH_ERR_NULL then).  x must not alias
 * act. */
int hip_gemv_swiglu_async(uint32_t ggml_type, const uint8_t* W_gate, const uint8_t* W_up, float* act, int ffn_dim,
                          const float* d_x, const float* norm_w, int in_dim, float* scratch, void* stream);

/* The attention block of one decode step in one launch: RoPE (as hip_rope_yarn)
 * on q (n_heads heads) and k (n_kv_heads heads), the K/V-cache append of the
 * rotated k and of v at row pos (as hip_kv_append), then attention over pos + 1
 * cached positions (as hip_attention_decode; sinks may be NULL).  Replaces the
 * reference's cuda_rope_yarn x2 + cuda_kv_append + cuda_attn_score_all +
 * cuda_softmax_sink_all + cuda_attn_values_all (src/cuda.rs:614-645, no sliding
 * window).  q and k are not modified; out gets n_heads * head_dim floats.
 * The sequence is split into 32-row slices over up to 64 workgroups per kv
 * head whose partial softmax states are merged through the library's static
 * device scratch (4 MB, per device; calls that overlap on one device race).
 * Limits (else QH_ERR_RANGE): head_dim and kv_dim multiples of 4, head_dim <=
 * 256, <= 16 q heads per kv head, n_kv_heads <= 256, k_cache / v_cache 16-byte
 * aligned. */
int hip_attention_step_async(float* out, const float* q, const float* k, const float* v, float* k_cache,
                             float* v_cache, const float* sinks, int n_heads, int n_kv_heads, int head_dim,
                             int kv_dim, int pos, float theta, float yarn_scale, int yarn_orig_ctx, int neox,
                             float scale, void* stream);
/* hip_attention_step for n_seq sequences decoding in lockstep (all at row pos):
 * sequence z uses q + z*n_heads*head_dim, k/v + z*kv_dim, out + z*n_heads*head_dim
 * and its own caches k_cache/v_cache + z*cache_stride (floats, >= (pos+1)*kv_dim).
 * One launch; n_seq * n_kv_heads <= 256. */
int hip_attention_step_batched_async(float* out, const float* q, const float* k, const float* v, float* k_cache,
                                     float* v_cache, const float* sinks, int n_seq, size_t cache_stride, int n_heads,
                                     int n_kv_heads, int head_dim, int kv_dim, int pos, float theta, float yarn_scale,
                                     int yarn_orig_ctx, int neox, float scale, void* stream);
/* hip_attention_step_batched_async with the position read from device memory
 * when the kernel runs (*d_pos, clamped to [0, max_pos] as forward_gpu_step
 * clamps pos to max_seq - 1, src/cuda.rs:517-520), so one captured launch serves
 * every position.  The launch is sized for max_pos (cache_stride >= (max_pos+1)
 * * kv_dim when n_seq > 1); workgroups beyond the split of the actual position
 * exit at once, and the arithmetic equals the host-position call's bit for bit.
 * No counterpart in the reference (pos is a host argument there). */
int hip_attention_step_dev_async(float* out, const float* q, const float* k, const float* v, float* k_cache,
                                 float* v_cache, const float* sinks, int n_seq, size_t cache_stride, int n_heads,
                                 int n_kv_heads, int head_dim, int kv_dim, const int* d_pos, int max_pos, float theta,
                                 float yarn_scale, int yarn_orig_ctx, int neox, float scale, void* stream);
int hip_embed_lookup(float* out, const uint8_t* d_data, uint32_t ggml_type, int token, int embed_dim);
int hip_embed_lookup_async(float* out, const uint8_t* d_data, uint32_t ggml_type, int token, int embed_dim,
                           void* stream);
/* n_tok rows at once (a batch's tokens, host array): row i = tokens[i] into
 * out + i * out_stride floats (out_stride >= embed_dim when n_tok > 1), each
 * bit-identical to hip_embed_lookup; up to 64 rows per launch.  No counterpart
 * in the reference (one embed_lookup per token); for callers that step several
 * sequences together. */
int hip_embed_lookup_batched_async(float* out, size_t out_stride, const uint8_t* d_data, uint32_t ggml_type,
                                   const int* tokens, int n_tok, int embed_dim, void* stream);
/* hip_embed_lookup_batched_async with the n_tok token ids read from device
 * memory (d_tokens) when the kernel runs; an id outside [0, n_vocab) gives a row
 * of zeros.  No counterpart in the reference (the token is a host argument). */
int hip_embed_lookup_dev_async(float* out, size_t out_stride, const uint8_t* d_data, uint32_t ggml_type,
                               const int* d_tokens, int n_tok, int n_vocab, int embed_dim, void* stream);
/* Greedy sampling on the device: d_tokens[r] = the index of the largest of the
 * n logits of row r (rows at logits + r * row_stride) in f32::total_cmp order,
 * the last one among equal maxima -- the reference's temperature <= 0 arm
 * (src/main.rs:1684-1692, max_by over total_cmp).  If d_pos is non-null,
 * *d_pos += 1 after the rows are read, so a captured step feeds itself. */
int hip_greedy_next_async(const float* logits, size_t row_stride, int rows, int n, int* d_tokens, int* d_pos,
                          void* stream);

/* ---------------------------------------------------------------- GGUF
 * Reader for the weight container either side of the GEMV path: GgufFile
 * (src/gguf.rs:61-191).  hip_gguf_open memory-maps the file and parses the
 * header (magic 0x46554747, versions 1..3; v1 has u32 counts and dims), the
 * typed metadata and the tensor infos; the data section starts at the next
 * multiple of general.alignment (default 32).  Errors the reference reports with
 * bail! come back as QH_ERR_FORMAT / QH_ERR_IO with its message in
 * hip_last_error().  Metadata getters follow GgufValue::as_u32 / as_u64 / as_str
 * (src/gguf.rs:18-35).  hip_gguf_tensor_data is GgufFile::tensor_data
 * (src/gguf.rs:116-121), a view into the map; hip_gguf_upload copies a tensor to
 * a new device buffer (free with hip_drop), as GpuWeights::from_weights does per
 * tensor (src/cuda.rs:170-172).  Value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32,
 * 5 i32, 6 f32, 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64. */
typedef struct qh_gguf qh_gguf;
typedef struct qh_gguf_writer qh_gguf_writer;

int hip_gguf_open(const char* path, qh_gguf** out);
void hip_gguf_close(qh_gguf* f);
uint32_t hip_gguf_version(const qh_gguf* f);
uint64_t hip_gguf_data_offset(const qh_gguf* f);
uint64_t hip_gguf_alignment(const qh_gguf* f);
int64_t hip_gguf_kv_count(const qh_gguf* f);
const char* hip_gguf_kv_key(const qh_gguf* f, int64_t i);  /* file order */
int hip_gguf_kv_type(const qh_gguf* f, const char* key, uint32_t* elem_type, uint64_t* count); /* -1: absent */
int hip_gguf_get_u32(const qh_gguf* f, const char* key, uint32_t* v);  /* Uint32 or Int32 */
int hip_gguf_get_u64(const qh_gguf* f, const char* key, uint64_t* v);  /* Uint64 or Uint32 */
int hip_gguf_get_i64(const qh_gguf* f, const char* key, int64_t* v);   /* any integer or bool */
int hip_gguf_get_f32(const qh_gguf* f, const char* key, float* v);
int hip_gguf_get_f64(const qh_gguf* f, const char* key, double* v);    /* Float64 or Float32 */
const char* hip_gguf_get_str(const qh_gguf* f, const char* key, uint64_t* len);
const void* hip_gguf_get_array(const qh_gguf* f, const char* key, uint32_t* elem_type, uint64_t* count);
const char* hip_gguf_get_array_str(const qh_gguf* f, const char* key, uint64_t i, uint64_t* len);
int64_t hip_gguf_tensor_count(const qh_gguf* f);
int64_t hip_gguf_find_tensor(const qh_gguf* f, const char* name);  /* -1: absent */
int hip_gguf_tensor_info(const qh_gguf* f, int64_t i, const char** name, uint32_t* n_dims, uint64_t* dims8,
                         uint32_t* ggml_type, uint64_t* offset);
const void* hip_gguf_tensor_data(const qh_gguf* f, int64_t i, size_t* bytes);
int hip_gguf_upload(const qh_gguf* f, int64_t i, void** d_ptr, size_t* bytes);

/* Writer: the container make_test_model.py produces (version 3, tensors in
 * order, each padded to general.alignment, default 32), for any ggml type and
 * metadata type.  Tensor data pointers must stay valid until _write. */
qh_gguf_writer* hip_gguf_writer_new(void);
void hip_gguf_writer_free(qh_gguf_writer* w);
int hip_gguf_writer_kv_scalar(qh_gguf_writer* w, const char* key, uint32_t type, const void* le8);
int hip_gguf_writer_kv_str(qh_gguf_writer* w, const char* key, const char* s, uint64_t len);
int hip_gguf_writer_kv_array(qh_gguf_writer* w, const char* key, uint32_t elem_type, const void* data,
                             uint64_t count);
int hip_gguf_writer_kv_array_str(qh_gguf_writer* w, const char* key, const char* const* strs, const uint64_t* lens,
                                 uint64_t count);
int hip_gguf_writer_tensor(qh_gguf_writer* w, const char* name, uint32_t n_dims, const uint64_t* dims,
                           uint32_t ggml_type, const void* data);
int hip_gguf_writer_write(const qh_gguf_writer* w, const char* path);

#ifdef __cplusplus
}
#endif
#endif /* QUARTZ_HIP_H */
