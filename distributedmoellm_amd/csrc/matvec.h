// Internal interface of the decode mat-vec (matvec.hip), used by the exported
// entry points in abi.hip.
#pragma once
#include "common.h"

namespace moe {

// GGUF ids as ggml's; FMT_Q4 and FMT_Q8 are colibri's int4 and int8
enum {
  FMT_Q4 = 0,
  FMT_Q8 = 1,
  FMT_Q4_0 = 2,
  FMT_Q4_1 = 3,
  FMT_Q5_0 = 6,
  FMT_Q5_1 = 7,
  FMT_Q8_0 = 8,
  FMT_Q2_K = 10,
  FMT_Q3_K = 11,
  FMT_Q4_K = 12,
  FMT_Q5_K = 13,
  FMT_Q6_K = 14
};

// One int4 expert as the fused layer call reads it; the layout of
// moe_q4_expert in include/moehip.h.
struct ExpertDesc {
  const uint8_t* gu_w;  // gate|up bytes [2I, H/2]
  const void* gu_s;     // their scales [2I, H/gs]
  const uint8_t* dn_w;  // down bytes [H, I/2]
  const void* dn_s;     // their scales [H, I/gs]
  uint32_t xor8;        // 0x88: two's-complement nibbles as stored; 0: already XOR-ed
  int32_t s_f16;        // scales are f16 (else f32)
};

struct MatRef {
  const uint8_t* w;
  const void* s;
  uint32_t xor4;  // XOR for each 32-bit weight word
  int s_f16;
};

struct MVShape {
  int O, I;       // output rows, input columns
  int gs, G;      // group size, groups per row (Q4/Q8)
  int row_bytes;  // bytes per weight row
  int cpr, rpp;   // chunks per row, rows per pass of a block
  int pow2;       // cpr is a power of two <= 64 (cross-lane reduction)
};

struct MVJob {
  const float* x;
  int ldx;
  float* y;
  int ldy;
  const int* seg;   // [nmat+1]: pairs of matrix m are seg[m]..seg[m+1]; null: pairs 0..n-1
  const int* xrow;  // input row of each pair; null: the pair index itself
  int n;
  const ExpertDesc* experts;  // expert descriptors; null: `single`
  const int* eidx;            // matrix m reads experts[eidx[m]]; null: experts[m]
  MatRef single;
  int which;    // 0: gate|up of the descriptor, 1: down
  int half_in;  // > 0: input rows are h = gate|up (2*half_in wide), use silu(gate)*up
  int xrows;    // the int8 mat-vec: rows of q that xrow may name (xrow values are clamped to them)
};

// the matrix a launch's blockIdx.y reads
__device__ __forceinline__ MatRef resolve(const MVJob& job, int mat) {
  if (job.experts == nullptr) return job.single;
  const ExpertDesc& e = job.experts[job.eidx ? job.eidx[mat] : mat];
  MatRef m;
  m.w = job.which ? e.dn_w : e.gu_w;
  m.s = job.which ? e.dn_s : e.gu_s;
  m.xor4 = e.xor8 * 0x01010101u;
  m.s_f16 = e.s_f16;
  return m;
}

int plan_matvec(int fmt, int O, int I, int gs, MVShape* sh);
// grid.z slices of the input rows for a launch of `waves` waves taking NR rows
// a pass: 1 .. ceil(max_rows / NR), about 16K waves in all
int row_slices(int max_rows, int NR, long waves);
// rows xrow[p] (or p) of x, or silu(h[:, :half]) * h[:, half:] when half > 0,
// rounded to int8 per group of gs (a multiple of 64 up to 512): q [n, K] bytes,
// each 32-column chunk as its 16 even columns then its 16 odd ones; d, s8 [n, K/gs].
// pslot (optional): pslot[rpair[j]] = p for j in rptr[p] .. rptr[p + 1], the
// rounded row each pair of row p reads
int run_round_q8(const float* x, int ldx, const int* xrow, int n, int K, int half, int gs, int8_t* q, float* d, int* s8,
                 hipStream_t st, const int* rptr = nullptr, const int* rpair = nullptr, int* pslot = nullptr);
// y[pair] = int8 row job.xrow[pair] (xrow null: row `pair`) of q (with its d,
// s8) against W_m, for every int4 matrix m and its pairs (job.seg; job.x is not
// used)
int run_matvec_q4i8(const MVShape& sh, const MVJob& job, int nmat, const int8_t* q, const float* dq, const int* s8q,
                    hipStream_t st);
// y[pair] = x[xrow[pair]] @ W_m.T for every matrix m and its pairs
int run_matvec(int fmt, const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st);

}  // namespace moe
