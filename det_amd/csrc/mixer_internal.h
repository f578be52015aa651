// Entry points of mixer.hip that the model runner calls and the C ABI does not export.
#pragma once
#include <stdint.h>
#include "../../include/det_hip.h"

namespace det {

// det_gdn, with the a|b projection optionally fused into the decode input stage: when ab != NULL (one token, a W8
// linear of 2 n_v rows: the a heads, then the b heads), a and b are not read; the kernel computes them from the
// token's quantized row (xq, sx, mx) with det_gemm_ex's integers and epilogue, bit for bit.
__attribute__((visibility("hidden")))
void gdn_run(const det_gdn_layer* L, det_gdn_state* S, const float* qkv, const float* z, const float* a, const float* b,
             const det_qlinear* ab, const int8_t* xq, const float* sx, const uint16_t* mx, float eps, int M, int n_k,
             int n_v, int dk, int dv, float* on, void* scratch, hipStream_t st);

} // namespace det
