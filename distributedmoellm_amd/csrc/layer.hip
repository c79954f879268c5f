// One MoE layer's int4 experts for a few rows each, in three launches
// (moelan/kernels.py:712-782, _moe_q4; wrapper 942-968):
//   1. gate|up of every (expert, row) pair      h[p]  = x[prow[p]] @ GU_e.T
//   2. down of silu(gate)*up, fused on load     y[p]  = a(h[p]) @ DN_e.T
//   3. weighted sum per touched row, in runs of 8 pairs in pair order
//      (expert order), then added to out: out[r] += sum_p pw[p] * y[p]
//      (deterministic)
#include <mutex>
#include <stdlib.h>

#include "common.h"
#include "matvec.h"
#include "layer.h"
#include "rows.h"

namespace moe {

// MOEHIP_ROWS=0 keeps experts with several rows on the mat-vec kernels (a
// measurement switch)
static bool rows_disabled() {
  static const bool off = [] {
    const char* e = getenv("MOEHIP_ROWS");
    return e && e[0] == '0';
  }();
  return off;
}

// ------------------------------------------------------------------ library-held scratch
//
// The workspace-free layer call (moe_q4_layer_noalloc) keeps its h and y in
// this array instead of a caller's workspace. Each device the library runs
// on holds its own copy from when the code object is loaded there until the
// process ends. In host code `scratch` names a host-side stand-in, not device
// memory: its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that address is
// used. Every call on a device shares that device's array, so calls that
// overlap on one device (other streams, other threads) race.
static __device__ __align__(256) uint8_t scratch[kLayerScratchBytes];

int layer_scratch(void** ptr) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(MOE_EHIP, "layer scratch: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(MOE_EUNSUPPORTED, "layer scratch: device %d", dev);
  std::lock_guard<std::mutex> g(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(MOE_EHIP, "layer scratch: hipGetSymbolAddress on device %d: %s", dev, hipGetErrorString(e));
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return MOE_OK;
}

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

// One launch: a block takes 16 columns of one row, 4 threads per column
// quad x 64 pair lanes; lane j sums the row's pairs j, j+64, j+128, ... in
// list order (their loads issued together), then the 64 lane sums are added
// by a fixed tree -- within each wave by lane swaps (16 sums), then the 4
// waves' in wave order through LDS -- and the total goes to out. Fixed
// order, no atomics; y is only read.
__global__ __launch_bounds__(256) void combine_tree_kernel(const float* y, int ldy, const float* pw, const int* rrow,
                                                           const int* rptr, const int* rpair, int nr, float* out,
                                                           int ldo, int H) {
  __shared__ float4 red[4][4];
  const int q = threadIdx.x & 3, j = threadIdx.x >> 2;
  const int c = blockIdx.x * 16 + q * 4;
  for (int i = blockIdx.y; i < nr; i += gridDim.y) {
    const int r0 = rptr[i], r1 = rptr[i + 1];
    // the writing lanes read out's row first: its latency overlaps the pairs'
    const bool writer = j == 0 && c < H;
    float4* const dst = reinterpret_cast<float4*>(out + (size_t)rrow[i] * ldo + c);
    float4 o = writer ? *dst : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c < H) {
      for (int t0 = r0 + j; t0 < r1; t0 += 64 * 8) {
        float4 v[8];
        float w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int t = t0 + 64 * u;
          const int p = rpair[t < r1 ? t : t0];
          w[u] = t < r1 ? pw[p] : 0.f;
          v[u] = *reinterpret_cast<const float4*>(y + (size_t)p * ldy + c);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (t0 + 64 * u < r1) {
            a.x += w[u] * v[u].x;
            a.y += w[u] * v[u].y;
            a.z += w[u] * v[u].z;
            a.w += w[u] * v[u].w;
          }
        }
      }
    }
    // lane 4 jw + q of wave w holds pair lane j = 16 w + jw: sum the 16 of
    // the wave (lane offsets 4, 8, 16, 32), then the waves in order
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) {
      a.x += __shfl_xor(a.x, o, 64);
      a.y += __shfl_xor(a.y, o, 64);
      a.z += __shfl_xor(a.z, o, 64);
      a.w += __shfl_xor(a.w, o, 64);
    }
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) < 4) red[wv][q] = a;
    __syncthreads();
    if (writer) {
      float4 t = red[0][q];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        t.x += red[w][q].x;
        t.y += red[w][q].y;
        t.z += red[w][q].z;
        t.w += red[w][q].w;
      }
      o.x += t.x;
      o.y += t.y;
      o.z += t.z;
      o.w += t.w;
      *dst = o;
    }
    __syncthreads();  // red is reused by the next row
  }
}

// Few pairs a row (a decode step's top-k): a thread takes 4 columns of one
// row and adds the row's pairs in list order (ascending), then adds the sum
// to out. Fixed order, no atomics; y is only read.
__global__ __launch_bounds__(256) void combine_rows_kernel(const float* y, int ldy, const float* pw, const int* rrow,
                                                           const int* rptr, const int* rpair, float* out, int ldo,
                                                           int H) {
  const int i = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= H) return;
  const int q0 = rptr[i], q1 = rptr[i + 1];
  // out's row is read before the pairs, so that its latency overlaps theirs
  // (the kernel is a chain of dependent loads at a decode step's sizes)
  float4* dst = reinterpret_cast<float4*>(out + (size_t)rrow[i] * ldo + c);
  float4 o = *dst;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  int q = q0;
  for (; q + 4 <= q1; q += 4) {  // four loads in flight, added in list order
    float4 v[4];
    float w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = rpair[q + u];
      w[u] = pw[p];
      v[u] = *reinterpret_cast<const float4*>(y + (size_t)p * ldy + c);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a.x += w[u] * v[u].x;
      a.y += w[u] * v[u].y;
      a.z += w[u] * v[u].z;
      a.w += w[u] * v[u].w;
    }
  }
  for (; q < q1; ++q) {
    const int p = rpair[q];
    const float w = pw[p];
    const float4 v = *reinterpret_cast<const float4*>(y + (size_t)p * ldy + c);
    a.x += w * v.x;
    a.y += w * v.y;
    a.z += w * v.z;
    a.w += w * v.w;
  }
  o.x += a.x;
  o.y += a.y;
  o.z += a.z;
  o.w += a.w;
  *dst = o;
}

// max_pairs: an upper bound of the pairs of one row; P: all pairs of the call
int run_combine_runs(float* y, int ldy, const float* pw, const int* rrow, const int* rptr, const int* rpair,
                            int nr, int max_pairs, float* out, int ldo, int H, hipStream_t st, int P) {
  if (nr <= 0) return MOE_OK;
  const bool vec4 = H % 4 == 0 && ldy % 4 == 0 && ldo % 4 == 0 && aligned(y, 16) && aligned(out, 16);
  if (!vec4) return run_combine(y, ldy, pw, rrow, rptr, rpair, nr, out, ldo, H, st);
  if (P > 0 && P <= 32 * nr && nr <= 65535) {  // few pairs a row on average: one thread a row's column quad
    hipLaunchKernelGGL(combine_rows_kernel, dim3((H / 4 + 255) / 256, nr), dim3(256), 0, st, y, ldy, pw, rrow, rptr,
                       rpair, out, ldo, H);
    return check_launch("weighted combine");
  }
  (void)max_pairs;  // the tree takes any number of pairs a row
  hipLaunchKernelGGL(combine_tree_kernel, dim3((H + 15) / 16, nr < 65535 ? nr : 65535), dim3(256), 0, st, y, ldy, pw,
                     rrow, rptr, rpair, nr, out, ldo, H);
  return check_launch("weighted combine");
}

// The workspace: h [P, 2I] f32, y [P, H] f32, then (for shapes the rows GEMM
// takes) its activation limbs, each piece 256-byte aligned.
static size_t hy_bytes(int P, int H, int I) {
  return ((size_t)P * (2 * (size_t)I + H) * sizeof(float) + 255) / 256 * 256;
}

size_t q4_layer_workspace(int P, int H, int I) {
  size_t n = hy_bytes(P, H, I);
  if (H % 256 == 0 && I % 256 == 0) n += rows_workspace(P, H, I);
  return n;
}

// Experts with several rows each: each weight row read once per pass of up to
// 8 rows, on integer MFMA (rows.hip); the same combine.
static int run_q4_layer_rows(const Q4LayerArgs& a, hipStream_t st) {
  float* h = reinterpret_cast<float*>(a.workspace);
  float* y = h + (size_t)a.P * 2 * a.I;
  const RowsSpace rs = rows_layout((char*)a.workspace + hy_bytes(a.P, a.H, a.I), a.P, a.H, a.I);
  int rc = run_rows_prep(a.x, a.ldx, a.prow, a.poff, a.k, a.P, a.H, 0, rs, rs.agu, st);
  if (rc) return rc;
  MVJob j1{};
  j1.y = h;
  j1.ldy = 2 * a.I;
  j1.seg = a.poff;
  j1.experts = a.table;
  j1.eidx = a.eidx;
  j1.which = 0;
  rc = run_rows_gemm(j1, a.k, 2 * a.I, a.H, a.max_rows, rs, rs.agu, st);
  if (rc) return rc;
  rc = run_rows_prep(h, 2 * a.I, nullptr, a.poff, a.k, a.P, a.I, a.I, rs, rs.adn, st);
  if (rc) return rc;
  MVJob j2{};
  j2.y = y;
  j2.ldy = a.H;
  j2.seg = a.poff;
  j2.experts = a.table;
  j2.eidx = a.eidx;
  j2.which = 1;
  rc = run_rows_gemm(j2, a.k, a.H, a.I, a.max_rows, rs, rs.adn, st);
  if (rc) return rc;
  return run_combine_runs(y, a.H, a.pw, a.rrow, a.rptr, a.rpair, a.nr, a.k < a.P ? a.k : a.P, a.out, a.ldo, a.H, st,
                          a.P);
}

int run_q4_layer(const Q4LayerArgs& a, hipStream_t st) {
  if (a.max_rows >= 2 && rows_gemm_ok(a.H, a.I, a.gs) && !rows_disabled()) return run_q4_layer_rows(a, st);
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
  return run_combine_runs(y, a.H, a.pw, a.rrow, a.rptr, a.rpair, a.nr, a.k < a.P ? a.k : a.P, a.out, a.ldo, a.H, st,
                          a.P);
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
  int* pslot;
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
  w.pslot = (int*)take(p * 4);
  w.bytes = off;
  return w;
}

size_t q4i8_layer_workspace(int P, int H, int I, int gs) { return q4i8_layout(nullptr, P, H, I, gs).bytes; }

// _moe_q4i (moelan/kernels.py:854-917): round the input rows, gate|up, SiLU *
// up rounded again, down, then the same weighted combine as the float call.
// Each touched input row is rounded once (the rows are rrow, a pair's slot
// goes to pslot), however many pairs read it: a token's 8 picks, or the 384
// evaluations of one row in a single call.
int run_q4i8_layer(const Q4LayerArgs& a, hipStream_t st) {
  if (a.nr <= 0) return MOE_OK;  // no row takes a sum: out is unchanged
  const Q4I8Space w = q4i8_layout(a.workspace, a.P, a.H, a.I, a.gs);
  MVShape s1, s2;
  plan_matvec(FMT_Q4, 2 * a.I, a.H, a.gs, &s1);
  plan_matvec(FMT_Q4, a.H, a.I, a.gs, &s2);
  int rc = run_round_q8(a.x, a.ldx, a.rrow, a.nr, a.H, 0, a.gs, w.qx, w.dx, w.sx, st, a.rptr, a.rpair, w.pslot);
  if (rc) return rc;

  MVJob j1{};
  j1.y = w.h;
  j1.ldy = 2 * a.I;
  j1.seg = a.poff;
  j1.xrow = w.pslot;
  j1.xrows = a.nr;
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

  return run_combine_runs(w.y, a.H, a.pw, a.rrow, a.rptr, a.rpair, a.nr, a.k < a.P ? a.k : a.P, a.out, a.ldo, a.H,
                          st, a.P);
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
