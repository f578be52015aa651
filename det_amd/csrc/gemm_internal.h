// Entry points of gemm.hip and quant.hip that the model runner calls and the C ABI does not export.
#pragma once
#include <stdint.h>
#include "../../include/det_hip.h"

namespace det {

// det_gemm_ex for one token (M = 1) with Parts output, where the values of part 0 are stored as silu_f(v): the
// one-token gate|up projection hands silu(g) to mul_quant, which then needs no transcendental.
__attribute__((visibility("hidden")))
void gemm_parts_silu0(const det_qlinear* L, const int8_t* xq, const float* sx, const uint16_t* mx, int nparts,
                      const int* offs, float* const* dsts, hipStream_t st);

// det_silu_mul_quant with the silu already applied to a: h = a * b, quantized in group mode (n % 128 == 0,
// n <= 32768, 16-byte aligned rows); the same h, codes and scales as det_silu_mul_quant(g, u) when a = silu_f(g).
// Returns false, having launched nothing, when the row does not fit.
__attribute__((visibility("hidden")))
bool mul_quant(const float* a, const float* b, int M, int n, int8_t* xq, float* sx, uint16_t* mx, hipStream_t st);

} // namespace det
