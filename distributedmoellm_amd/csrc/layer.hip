// One MoE layer's int4 experts for a few rows each, in three launches
// (moelan/kernels.py:712-782, _moe_q4; wrapper 942-968):
//   1. gate|up of every (expert, row) pair      h[p]  = x[prow[p]] @ GU_e.T
//   2. down of silu(gate)*up, fused on load     y[p]  = a(h[p]) @ DN_e.T
//   3. weighted sum per touched row, in pair order (expert order), then
//      added to out:  out[r] += sum_p pw[p] * y[p]      (deterministic)
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

  return run_combine(y, a.H, a.pw, a.rrow, a.rptr, a.rpair, a.nr, a.out, a.ldo, a.H, st);
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
