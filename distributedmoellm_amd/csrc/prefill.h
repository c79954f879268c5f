#pragma once
#include "common.h"
#include "matvec.h"

namespace moe {

enum { MODE_PLAIN = 0, MODE_GATE_UP = 1, MODE_DOWN = 2 };

struct GemmArgs {
  // Activations: f16 rows (8-column groups in MFMA order), each row scaled by
  // a power of two (GATE_UP: xfac[m] undoes it; DOWN: afac[m * ldaf + c]
  // undoes it for 16-column piece c), or
  // f32 rows X (PLAIN, rows32) scaled per row while staged.
  const _Float16* A;  // [P, K] (rows32 == 0); GATE_UP with `rows`: [*, lda] rows taken through `rows`
  int lda;
  const float* xfac;  // GATE_UP (with `rows`: per row of A)
  const float* afac;  // DOWN
  int ldaf;
  int rows32;          // activations are f32 rows of X gathered through `rows` (PLAIN only)
  const float* X;      // [*, ldx] f32
  int ldx;
  const int* rows;     // row of X (rows32) or of A (GATE_UP) for each grouped row (null: the grouped row itself)
  const int* eoff;           // [nexp + 1] rows of expert e: eoff[e] .. eoff[e+1]
  const ExpertDesc* table;   // expert e's matrices; null: `single` with rows 0 .. single_rows
  ExpertDesc single;
  int single_rows;
  int which;                 // 0: gate|up, 1: down
  int K;                     // reduction length (H for gate|up, I for down)
  int N;                     // output columns (PLAIN / DOWN)
  int I;                     // intermediate size (GATE_UP: up rows start at I)
  int gs;
  float* Y;  // PLAIN / DOWN output [P, N] f32
  int ldy;
  _Float16* act;  // GATE_UP output silu(gate) * up [P, I] f16, MFMA column order, each row and
  int ldact;      // 16 columns scaled by a power of two that act_fac[m * ldaf_out + c] undoes
  float* act_fac;
  int ldaf_out;
};

// picks per token the token combine takes (its ordering lives in LDS)
constexpr int kCombineMaxPicks = 4096;
// experts per grouped-GEMM launch (one grid row each)
constexpr int kMaxGridY = 65535;

int router_slices(int T, int E, int H);
int run_router_partials(const float* x, int ldx, const float* R, int T, int E, int H, int nz, float* part,
                        hipStream_t st);
// the f32 MFMA router applies: H a multiple of 64, rows 16-byte aligned
bool router_mfma_ok(const float* x, int ldx, const float* R, int H);
// K slices for the MFMA router (1 unless the tiles are few; at most max_slices)
int router_mfma_slices(int T, int E, int H, int max_slices);
// part: nz slices of T x E partial logits (nz = 1: the logits)
int run_router_mfma(const float* x, int ldx, const float* R, int T, int E, int H, int nz, float* part, hipStream_t st);
// MFMA when it applies, else split K: scratch router_slices(T, E, H) * T * E floats (null: one slice)
int run_router_logits(const float* x, int ldx, const float* R, int T, int E, int H, float* logits, float* scratch,
                      hipStream_t st);
// xs (optional): token t's row x[t] (H values) also goes out as its f16 copy
// xs[t] (as run_gather_f16) with factor xf[t]
int run_route(const float* logits, int nz, int T, int E, int k, int normalize, int* idx, float* w, hipStream_t st,
              const float* x = nullptr, int ldx = 0, int H = 0, _Float16* xs = nullptr, float* xf = nullptr);
// experts / offsets / n_used may be null (not produced)
int run_group(const int* idx, const float* w, int T, int k, int E, int* eoff, int* rows, float* wts, int* pos,
              int* experts, int* offsets, int* n_used, hipStream_t st);
// Xs[q] = f16(x[rows[q]] * 2^a_q) in MFMA column order, a_q putting the row's
// largest |value| in [2^13, 2^14); fac[q] = 2^-a_q (1 for a row of zeros or
// with non-finite values)
int run_gather_f16(const float* x, int ldx, const int* rows, int P, int K, _Float16* Xs, float* fac, hipStream_t st);
int run_gemm(int mode, const GemmArgs& a, int nexp, hipStream_t st);
int run_token_combine(const float* y, int ldy, const int* pos, const float* wts, int T, int k, int H, float* out,
                      int ldo, hipStream_t st);

}  // namespace moe
