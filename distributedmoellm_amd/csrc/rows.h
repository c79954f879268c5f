// Internal interface of the multi-row decode GEMM (rows.hip), used by the
// layer call (layer.hip) for experts that carry several input rows.
#pragma once
#include "common.h"
#include "matvec.h"

namespace moe {

// Whether the rows GEMM takes a layer of this shape: both matrices' rows are
// whole 256-column stages (H and I multiples of 256, at most 16384) and the
// group size is 32.
bool rows_gemm_ok(int H, int I, int gs);

// Workspace bytes the rows GEMM adds to the layer call for P pairs.
size_t rows_workspace(int P, int H, int I);

struct RowsSpace {
  int* qbase;    // [k] first quad of each expert
  float* fac;    // [P] 2^-sigma / 16 of each pair's activation row
  uint8_t* agu;  // [P quads][H/64][64][16] activation limbs for gate|up
  uint8_t* adn;  // [P quads][I/64][64][16] activation limbs for down
  size_t bytes;
};
RowsSpace rows_layout(void* base, int P, int H, int I);

// Activation limbs of every pair: half = 0 reads x[xrow[p]] (K values), half > 0
// reads silu(x[p, :K]) * x[p, half:half + K]. poff ascends from poff[0] = 0 to
// poff[k] = P.
int run_rows_prep(const float* x, int ldx, const int* xrow, const int* poff, int k, int P, int K, int half,
                  const RowsSpace& ws, uint8_t* limbs, hipStream_t st);
// y[p] = a(p) @ W_m.T for every expert m of the job (its gate|up matrix for
// which = 0, down for 1) and all its pairs (at most max_rows an expert), from
// the limbs of run_rows_prep.
int run_rows_gemm(const MVJob& job, int k, int O, int K, int max_rows, const RowsSpace& ws, const uint8_t* limbs,
                  hipStream_t st);

}  // namespace moe
