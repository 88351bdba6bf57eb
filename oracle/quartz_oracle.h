/* quartz_oracle.h -- CPU restatement of Quartz's quantized GEMV path.
 * TEST INFRASTRUCTURE ONLY (the checker for the HIP library, never linked by it). */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float o_f16_to_f32(uint16_t bits);
void o_get_scale_min_k4(int j, const uint8_t* scales, uint8_t* sc, uint8_t* m);
size_t o_type_size(uint32_t ggml_type, size_t n_elems);   /* 0 = unsupported type */
int o_block_elems(uint32_t ggml_type);                     /* 0 = unsupported type */
int o_dequant(uint32_t ggml_type, const uint8_t* data, size_t n_elems, float* out);
int o_gemv(uint32_t ggml_type, const float* x, const uint8_t* data, int in_dim, int out_dim, float* y);
int o_gemv_dequant_matmul(uint32_t ggml_type, const float* x, const uint8_t* data, int in_dim, int out_dim,
                          float* w_scratch, float* y);
int o_gemm(uint32_t ggml_type, const float* x, const uint8_t* data, int in_dim, int out_dim, int n, float* y);
void o_set_threads(int n);
int o_get_threads(void);
const char* o_grid_sha256(int which);
/* Q8_1 MMQ arithmetic mode (src/dequant.rs:202-645) */
uint16_t o_f32_to_f16_rne(float value);
void o_quantize_q8_1_mmq(const float* x, int in_dim, int rows, int d4, int8_t* values, float* scale, float* sum);
int o_stream_k_cut(int row, int column, int in_dim, int out_dim, int reference_rows, int multiprocessors);
int o_gemm_q8_1_mmq(uint32_t ggml_type, const float* x, const uint8_t* data, int in_dim, int out_dim, int rows,
                    int reference_rows, int multiprocessors, float* y);

#ifdef __cplusplus
}
#endif
