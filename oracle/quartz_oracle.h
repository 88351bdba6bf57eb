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
int o_gemm(uint32_t ggml_type, const float* x, const uint8_t* data, int in_dim, int out_dim, int n, float* y);
void o_set_threads(int n);
int o_get_threads(void);
const char* o_grid_sha256(int which);

#ifdef __cplusplus
}
#endif
