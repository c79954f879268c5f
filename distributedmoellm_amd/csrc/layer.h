#pragma once
#include "common.h"
#include "matvec.h"

namespace moe {

struct Q4LayerArgs {
  const float* x;
  int ldx;
  const ExpertDesc* table;
  const int* eidx;
  int k;
  const int* poff;   // [k+1]
  const int* prow;   // [P] input row of each pair
  const float* pw;   // [P] gate weight of each pair
  int P;
  const int* rrow;   // [nr] touched rows, each once
  const int* rptr;   // [nr+1]
  const int* rpair;  // [P] pairs of each touched row, ascending
  int nr;
  float* out;
  int ldo;
  int H, I, gs, max_rows;
  void* workspace;
};

size_t q4_layer_workspace(int P, int H, int I);
// bytes of the library-held scratch the workspace-free layer call uses (per device)
constexpr size_t kLayerScratchBytes = (size_t)32 << 20;
// that scratch's device address on the current device (looked up once per device)
int layer_scratch(void** ptr);
int run_q4_layer(const Q4LayerArgs& a, hipStream_t st);
// the same call with activations rounded to int8 per group (gs a multiple of 64)
size_t q4i8_layer_workspace(int P, int H, int I, int gs);
int run_q4i8_layer(const Q4LayerArgs& a, hipStream_t st);
int run_silu_mul(const float* h, int ldh, int n, int I, float* a, int lda, hipStream_t st);
int run_combine(const float* y, int ldy, const float* pw, const int* rrow, const int* rptr, const int* rpair, int nr,
                float* out, int ldo, int H, hipStream_t st);
// the same sum in one launch: a block per (row, 16 columns), 64 pair lanes added by a fixed tree
// (P: the call's pairs; with at most 32 a touched row on average each row is
// summed by one thread per column quad in list order instead)
int run_combine_runs(float* y, int ldy, const float* pw, const int* rrow, const int* rptr, const int* rpair, int nr,
                     int max_pairs, float* out, int ldo, int H, hipStream_t st, int P = 0);

}  // namespace moe
