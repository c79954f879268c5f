// Activations on the wire (wire.hip): f32, f16, or int8 with f32 scales per
// group of 64 values (moelan/protocol.py:90-123).
#pragma once
#include "common.h"

#define MOE_WIRE_F32 0
#define MOE_WIRE_F16 1
#define MOE_WIRE_INT8 2

namespace moe {
// values per int8 scale of rows of d values: 64, or d when 64 does not divide it
int wire_group(int d);
// rows[r] (rows null: r) of a [*, lda], r < n, encoded into out [n, d] (f32,
// f16 or int8) and, for int8, scale [n, d / wire_group(d)]
int run_wire_encode(const float* a, int lda, const int* rows, int n, int d, int wire, void* out, float* scale,
                    hipStream_t st);
// row r of in [n, d] decoded into out[rows[r]] (rows null: out[r]), row stride ldo
int run_wire_decode(const void* in, const float* scale, int wire, int n, int d, const int* rows, float* out, int ldo,
                    hipStream_t st);
}  // namespace moe
