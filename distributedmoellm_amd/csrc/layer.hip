// One MoE layer's int4 experts for a few rows each, in three launches
// (moelan/kernels.py:712-782, _moe_q4; wrapper 942-968):
//   1. gate|up of every (expert, row) pair      h[p]  = x[prow[p]] @ GU_e.T
//   2. down of silu(gate)*up, fused on load     y[p]  = a(h[p]) @ DN_e.T
//   3. weighted sum per touched row, in runs of 8 pairs in pair order
//      (expert order), then added to out: out[r] += sum_p pw[p] * y[p]
//      (deterministic)
#include "common.h"
#include "matvec.h"
#include "layer.h"

namespace moe {

// part = sum over the row's pairs of w * y; then out[row] += part. A block
// takes one touched row and 256 columns (64 threads x 4 columns); its 4 waves
// sum interleaved quarters of the row's pair list, which are then added in a
// fixed order: deterministic, and no atomics.
__global__ __launch_bounds__(256) void combine_kernel(const float* y, int ldy, const float* pw, const int* rrow,
                                                      const int* rptr, const int* rpair, float* out, int ldo, int H,
                                                      int vec4) {
  __shared__ float4 part[4][64];
  const int i = blockIdx.y;
  const int q0 = rptr[i], q1 = rptr[i + 1];
  const int seg = threadIdx.x >> 6, t = threadIdx.x & 63;
  const int c = blockIdx.x * 256 + 4 * t;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c < H) {
    for (int q = q0 + seg; q < q1; q += 4) {
      const int p = rpair[q];
      const float w = pw[p];
      const float* yp = y + (size_t)p * ldy + c;
      if (vec4) {
        const float4 v = *reinterpret_cast<const float4*>(yp);
        a.x += w * v.x;
        a.y += w * v.y;
        a.z += w * v.z;
        a.w += w * v.w;
      } else {
        a.x += w * yp[0];
        if (c + 1 < H) a.y += w * yp[1];
        if (c + 2 < H) a.z += w * yp[2];
        if (c + 3 < H) a.w += w * yp[3];
      }
    }
  }
  part[seg][t] = a;
  __syncthreads();
  if (seg == 0 && c < H) {
    float4 s = part[0][t];
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      const float4 v = part[k][t];
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
    float* dst = out + (size_t)rrow[i] * ldo + c;
    dst[0] += s.x;
    if (c + 1 < H) dst[1] += s.y;
    if (c + 2 < H) dst[2] += s.z;
    if (c + 3 < H) dst[3] += s.w;
  }
}

int run_combine(const float* y, int ldy, const float* pw, const int* rrow, const int* rptr, const int* rpair, int nr,
                float* out, int ldo, int H, hipStream_t st) {
  if (nr <= 0) return MOE_OK;
  const int vec4 = (H % 4 == 0 && ldy % 4 == 0 && aligned(y, 16)) ? 1 : 0;
  hipLaunchKernelGGL(combine_kernel, dim3((H + 255) / 256, nr), dim3(256), 0, st, y, ldy, pw, rrow, rptr, rpair, out,
                     ldo, H, vec4);
  return check_launch("weighted combine");
}

// The layer call's combine, in two launches, for rows with many pairs (one
// token's 384 experts): the pair list of a row is cut into runs of kRun pairs
// in list order. Launch 1: a block sums one run for 1024 columns (a thread
// takes 4 columns, its kRun loads issued together) and writes the partial sum
// over the y row of the run's first pair, which no other block reads (each
// pair belongs to one row and one run); a row with a single run is added to
// out at once. Launch 2: per row of more than one run, the partial sums in
// run order, added to out. Fixed order, no atomics. y is overwritten.
constexpr int kRun = 8;

__global__ __launch_bounds__(256) void combine_runs_kernel(float* y, int ldy, const float* pw, const int* rrow,
                                                           const int* rptr, const int* rpair, int nr, float* out,
                                                           int ldo, int H) {
  const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= H) return;
  for (int i = blockIdx.y; i < nr; i += gridDim.y) {
    const int r0 = rptr[i], r1 = rptr[i + 1];
    for (int q0 = r0 + blockIdx.z * kRun; q0 < r1; q0 += gridDim.z * kRun) {
      const int n = min(kRun, r1 - q0);
      int ps[kRun];
      float ws[kRun];
      float4 v[kRun];
#pragma unroll
      for (int j = 0; j < kRun; ++j) {
        ps[j] = rpair[q0 + (j < n ? j : 0)];
        ws[j] = j < n ? pw[ps[j]] : 0.f;
        v[j] = *reinterpret_cast<const float4*>(y + (size_t)ps[j] * ldy + c);
      }
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int j = 0; j < kRun; ++j) {
        if (j < n) {
          a.x += ws[j] * v[j].x;
          a.y += ws[j] * v[j].y;
          a.z += ws[j] * v[j].z;
          a.w += ws[j] * v[j].w;
        }
      }
      if (r1 - r0 <= kRun) {
        float4* dst = reinterpret_cast<float4*>(out + (size_t)rrow[i] * ldo + c);
        float4 o = *dst;
        o.x += a.x;
        o.y += a.y;
        o.z += a.z;
        o.w += a.w;
        *dst = o;
      } else {
        *reinterpret_cast<float4*>(y + (size_t)ps[0] * ldy + c) = a;
      }
    }
  }
}

__global__ __launch_bounds__(256) void combine_partials_kernel(const float* y, int ldy, const int* rrow,
                                                               const int* rptr, const int* rpair, int nr, float* out,
                                                               int ldo, int H) {
  const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= H) return;
  for (int i = blockIdx.y; i < nr; i += gridDim.y) {
    const int r0 = rptr[i], r1 = rptr[i + 1];
    if (r1 - r0 <= kRun) continue;
    const int runs = (r1 - r0 + kRun - 1) / kRun;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < runs; s0 += 8) {
      float4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int s = s0 + j < runs ? s0 + j : s0;
        v[j] = *reinterpret_cast<const float4*>(y + (size_t)rpair[r0 + s * kRun] * ldy + c);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (s0 + j < runs) {
          a.x += v[j].x;
          a.y += v[j].y;
          a.z += v[j].z;
          a.w += v[j].w;
        }
      }
    }
    float4* dst = reinterpret_cast<float4*>(out + (size_t)rrow[i] * ldo + c);
    float4 o = *dst;
    o.x += a.x;
    o.y += a.y;
    o.z += a.z;
    o.w += a.w;
    *dst = o;
  }
}

// max_pairs: an upper bound of the pairs of one row
int run_combine_runs(float* y, int ldy, const float* pw, const int* rrow, const int* rptr, const int* rpair,
                            int nr, int max_pairs, float* out, int ldo, int H, hipStream_t st) {
  if (nr <= 0) return MOE_OK;
  const bool vec4 = H % 4 == 0 && ldy % 4 == 0 && ldo % 4 == 0 && aligned(y, 16) && aligned(out, 16);
  if (!vec4) return run_combine(y, ldy, pw, rrow, rptr, rpair, nr, out, ldo, H, st);
  const int runs = (max_pairs + kRun - 1) / kRun;
  const dim3 grid((H + 1023) / 1024, nr < 65535 ? nr : 65535, runs < 1 ? 1 : (runs < 1024 ? runs : 1024));
  hipLaunchKernelGGL(combine_runs_kernel, grid, dim3(256), 0, st, y, ldy, pw, rrow, rptr, rpair, nr, out, ldo, H);
  if (runs > 1)
    hipLaunchKernelGGL(combine_partials_kernel, dim3(grid.x, grid.y), dim3(256), 0, st, y, ldy, rrow, rptr, rpair, nr,
                       out, ldo, H);
  return check_launch("weighted combine");
}

size_t q4_layer_workspace(int P, int H, int I) { return (size_t)P * (2 * (size_t)I + H) * sizeof(float); }

int run_q4_layer(const Q4LayerArgs& a, hipStream_t st) {
  float* h = reinterpret_cast<float*>(a.workspace);
  float* y = h + (size_t)a.P * 2 * a.I;
  MVShape s1, s2;
  plan_matvec(FMT_Q4, 2 * a.I, a.H, a.gs, &s1);
  plan_matvec(FMT_Q4, a.H, a.I, a.gs, &s2);

  MVJob j1{};
  j1.x = a.x;
  j1.ldx = a.ldx;
  j1.y = h;
  j1.ldy = 2 * a.I;
  j1.seg = a.poff;
  j1.xrow = a.prow;
  j1.experts = a.table;
  j1.eidx = a.eidx;
  j1.which = 0;
  j1.half_in = 0;
  int rc = run_matvec(FMT_Q4, s1, j1, a.k, a.max_rows, st);
  if (rc) return rc;

  MVJob j2{};
  j2.x = h;
  j2.ldx = 2 * a.I;
  j2.y = y;
  j2.ldy = a.H;
  j2.seg = a.poff;
  j2.xrow = nullptr;
  j2.experts = a.table;
  j2.eidx = a.eidx;
  j2.which = 1;
  j2.half_in = a.I;
  rc = run_matvec(FMT_Q4, s2, j2, a.k, a.max_rows, st);
  if (rc) return rc;

  // a row has at most one pair per expert of the call
  return run_combine_runs(y, a.H, a.pw, a.rrow, a.rptr, a.rpair, a.nr, a.k < a.P ? a.k : a.P, a.out, a.ldo, a.H, st);
}

// The workspace of the int8-activation call, each piece 256-byte aligned:
// h [P, 2I] f32, y [P, H] f32, the rounded inputs [P, H] bytes with d, s8
// [P, H/gs], the rounded SiLU outputs [P, I] bytes with d, s8 [P, I/gs].
struct Q4I8Space {
  float* h;
  float* y;
  int8_t* qx;
  float* dx;
  int* sx;
  int8_t* qa;
  float* da;
  int* sa;
  size_t bytes;
};

static Q4I8Space q4i8_layout(void* base, int P, int H, int I, int gs) {
  Q4I8Space w{};
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t o = off;
    off += (n + 255) / 256 * 256;
    return (char*)base + o;
  };
  const size_t p = (size_t)P;
  w.h = (float*)take(p * 2 * I * 4);
  w.y = (float*)take(p * H * 4);
  w.qx = (int8_t*)take(p * H);
  w.dx = (float*)take(p * (H / gs) * 4);
  w.sx = (int*)take(p * (H / gs) * 4);
  w.qa = (int8_t*)take(p * I);
  w.da = (float*)take(p * (I / gs) * 4);
  w.sa = (int*)take(p * (I / gs) * 4);
  w.bytes = off;
  return w;
}

size_t q4i8_layer_workspace(int P, int H, int I, int gs) { return q4i8_layout(nullptr, P, H, I, gs).bytes; }

// _moe_q4i (moelan/kernels.py:854-917): round the pairs' input rows, gate|up,
// SiLU * up rounded again, down, then the same weighted combine as the float call
int run_q4i8_layer(const Q4LayerArgs& a, hipStream_t st) {
  const Q4I8Space w = q4i8_layout(a.workspace, a.P, a.H, a.I, a.gs);
  MVShape s1, s2;
  plan_matvec(FMT_Q4, 2 * a.I, a.H, a.gs, &s1);
  plan_matvec(FMT_Q4, a.H, a.I, a.gs, &s2);
  int rc = run_round_q8(a.x, a.ldx, a.prow, a.P, a.H, 0, a.gs, w.qx, w.dx, w.sx, st);
  if (rc) return rc;

  MVJob j1{};
  j1.y = w.h;
  j1.ldy = 2 * a.I;
  j1.seg = a.poff;
  j1.n = a.P;
  j1.experts = a.table;
  j1.eidx = a.eidx;
  j1.which = 0;
  rc = run_matvec_q4i8(s1, j1, a.k, w.qx, w.dx, w.sx, st);
  if (rc) return rc;

  rc = run_round_q8(w.h, 2 * a.I, nullptr, a.P, a.I, a.I, a.gs, w.qa, w.da, w.sa, st);
  if (rc) return rc;

  MVJob j2{};
  j2.y = w.y;
  j2.ldy = a.H;
  j2.seg = a.poff;
  j2.n = a.P;
  j2.experts = a.table;
  j2.eidx = a.eidx;
  j2.which = 1;
  rc = run_matvec_q4i8(s2, j2, a.k, w.qa, w.da, w.sa, st);
  if (rc) return rc;

  return run_combine_runs(w.y, a.H, a.pw, a.rrow, a.rptr, a.rpair, a.nr, a.k < a.P ? a.k : a.P, a.out, a.ldo, a.H, st);
}

}  // namespace moe

namespace moe {

// a[r, c] = silu(h[r, c]) * h[r, I + c]  (moelan/experts.py:256-259, silu :62-63)
__global__ void silu_mul_kernel(const float* h, int ldh, int n, int I, float* a, int lda) {
  const long total = (long)n * I;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int r = (int)(i / I), c = (int)(i % I);
    const float* hr = h + (size_t)r * ldh;
    a[(size_t)r * lda + c] = silu(hr[c]) * hr[I + c];
  }
}

int run_silu_mul(const float* h, int ldh, int n, int I, float* a, int lda, hipStream_t st) {
  if (n <= 0) return MOE_OK;
  long blocks = ((long)n * I + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((int)blocks), dim3(256), 0, st, h, ldh, n, I, a, lda);
  return check_launch("silu(gate)*up");
}

}  // namespace moe
