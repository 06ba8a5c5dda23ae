// y [M, N] = x [M, K] * w [N, K]^T (bf16, float32 accumulation) -- placeholder until the
// hipBLASLt plan cache lands; returns hipErrorNotSupported.
#include <hip/hip_runtime.h>

#include "qwen3_5_ops.h"

extern "C" {

void* cs1_gemm_create(size_t) { return nullptr; }
void cs1_gemm_destroy(void*) {}
int cs1_gemm(void*, const void*, const void*, void*, int, int, int, int, void*) { return hipErrorNotSupported; }

}  // extern "C"
