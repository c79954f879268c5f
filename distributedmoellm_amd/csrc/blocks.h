// GGUF block types (blocks.hip): the mat-vec of every quantized type (Q4_0,
// Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K); the dequant of all but
// Q8_0 and Q4_K (dequant.hip).
#pragma once
#include "common.h"
#include "matvec.h"

namespace moe {
// values and bytes per block, values per mat-vec chunk; false for other types
bool block_geometry(int qtype, int* per, int* size, int* vals);
// y[pair] = x[xrow[pair]] @ W_m.T for every matrix m and its pairs; rows of
// more than 8192 values take one launch per 8192-value segment; a matrix's
// blocks are read once per 1, 2 or 4 of its input rows (max_rows: the most
// rows any matrix has)
int run_matvec_blocks(int qtype, const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st);
int run_dequant_blocks(const uint8_t* raw, int qtype, int O, int cols, float* out, hipStream_t st);
}  // namespace moe
