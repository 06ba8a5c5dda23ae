// The reference's vision-tower entry points (ops.h:127-138). The vision tower is not on
// the text prefill path this library implements; the symbols exist so that a loader that
// resolves the whole reference symbol table (cuda.rs:33-46) can load the library, and
// each reports hipErrorNotSupported.
#include <hip/hip_runtime.h>

#include "qwen3_5_ops.h"

extern "C" {

int cs1_vision_linear(void*, const void*, const void*, const void*, void*, int, int, int, void*) {
    return hipErrorNotSupported;
}
int cs1_gemm_f32(void*, const float*, const float*, float*, int, int, int, void*) { return hipErrorNotSupported; }
int cs1_vision_norm(const void*, const void*, const void*, void*, int, int, void*) { return hipErrorNotSupported; }
int cs1_vision_position(void*, const void*, const int*, const float*, int, void*) { return hipErrorNotSupported; }
int cs1_vision_rope(const void*, const float*, const float*, void*, void*, int, void*) { return hipErrorNotSupported; }
int cs1_vision_attention(const void*, const void*, const void*, void*, int, void*) { return hipErrorNotSupported; }
int cs1_vision_bias(void*, const void*, size_t, int, void*) { return hipErrorNotSupported; }
int cs1_vision_gelu(void*, size_t, int, void*) { return hipErrorNotSupported; }
int cs1_vision_add(void*, const void*, size_t, void*) { return hipErrorNotSupported; }
int cs1_vision_to_float(const void*, float*, size_t, void*) { return hipErrorNotSupported; }
int cs1_vision_lora_add(void*, const float*, size_t, float, void*) { return hipErrorNotSupported; }

}  // extern "C"
