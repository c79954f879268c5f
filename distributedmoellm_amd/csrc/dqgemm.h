// Group-scaled int8 / int4 weights times many f32 rows on f32 MFMA
// (dqgemm.hip), used by the single-matrix entry points once a call has
// enough rows.
#pragma once
#include "common.h"

namespace moe {

enum { DQ_INT8 = 0, DQ_INT4 = 1, DQ_Q8_0 = 2, DQ_Q4_K = 3 };

struct DqArgs {
  const float* x;  // [n, ldx] f32 rows
  int ldx;
  int n;
  const void* w;   // int8 [O, K], int4 [O, K/2] (low nibble = even column) Q8_0 [O, K/32 x 34 B] or Q4_K blocks [O, K/256 x 144 B]
  const void* s;   // scales [O, K/gs], f16 or f32 (not used by Q8_0)
  int s_f16;
  uint32_t xor4;   // int4: XOR of each stored word (0x88888888: two's-complement nibbles)
  int O, K, gs;
  float* y;        // [n, ldy]
  int ldy;
};

// calls with at least this many rows take the MFMA product
constexpr int kDqRows = 16;

// the kernel takes the shape and pointers (K a multiple of 64 -- 128 for
// Q8_0, 256 for Q4_K -- gs of 16, x rows 16-byte aligned, int8 / Q4_K weights
// 16-byte, int4 8-byte, Q8_0 4-byte aligned)
bool dq_mfma_ok(int wf, const DqArgs& a);
int run_dq_mfma(int wf, const DqArgs& a, hipStream_t st);

}  // namespace moe
