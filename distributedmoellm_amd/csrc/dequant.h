#pragma once
#include "common.h"

namespace moe {
int run_dequant_q4(const uint8_t* raw, const void* s, int s_f16, int O, int I, int gs, uint32_t xor8, float* out,
                   hipStream_t st);
int run_dequant_q8(const int8_t* q, const void* s, int s_f16, int O, int I, int gs, float* out, hipStream_t st);
int run_dequant_gguf(const uint8_t* raw, int qtype, int O, int cols, float* out, hipStream_t st);
}  // namespace moe
