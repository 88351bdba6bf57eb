// qh_lib.hip -- the single translation unit of libquartz_hip.so.
// The IQ codebooks are device globals shared by the decode and GEMV kernels;
// compiling everything as one unit keeps them visible without relocatable
// device code.
#include "qh_dequant.hip"
#include "qh_mmv.hip"
#include "qh_mmv16.hip"
#include "qh_gemm.hip"
#include "qh_mmq81.hip"
#include "qh_gemv.hip"
#include "qh_glue.hip"
#include "qh_moe.hip"
#include "qh_api.hip"
#include "qh_gguf.hip"
