// Decode mat-vec y = x @ W.T straight from packed weight bytes, f32 accumulate.
//
// Replaces the numba kernels _q4 / _q4_rows / _q8 / _q8_rows / _mv_q8_0 /
// _mv_q4_k / _gguf_mm (moelan/kernels.py:85-168, 482-527, 678-691) and the
// gate|up and down sweeps of _moe_q4 (moelan/kernels.py:712-777).
//
// Work decomposition (one launch may cover many matrices, e.g. a layer's experts):
//   grid.y  = matrix (expert), grid.x = tile of output rows of that matrix
//   block   = rpp rows x cpr chunk columns; thread t owns chunk column t % cpr
//             and row slot t / cpr, so one pass of the block reads rpp whole
//             consecutive rows: contiguous, 16-byte loads per lane.
//   PASSES  passes per block, all loads issued before any math.
//   NR      input rows held in registers at once; more rows loop in batches
//           (the tile's weights are re-read from L2, not HBM).
// A lane computes sum(chunk of weights * chunk of x) * group scale; partial
// sums of a row are added across its cpr lanes with cross-lane shuffles when
// cpr is a power of two <= 64, else through LDS.
#include <map>
#include <mutex>
#include <tuple>
#include "common.h"
#include "formats.h"
#include "matvec.h"
#include "blocks.h"

#include <stdlib.h>

#include <type_traits>

namespace moe {

// 16 weight bytes of a row: one 128-bit load when the matrix is 16-byte
// aligned (the usual case: HBM buffers), byte loads otherwise.
__device__ __forceinline__ uint4 load16(const uint8_t* p, bool a16) {
  if (a16) return stream_load16(p);
  uint32_t v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    v[i] = p[4 * i] | (p[4 * i + 1] << 8) | (p[4 * i + 2] << 16) | ((uint32_t)p[4 * i + 3] << 24);
  return uint4{v[0], v[1], v[2], v[3]};
}


// Adds the partials of a pass and writes y; `acc` is [PASSES][NR].
template <int PASSES, int NR>
__device__ __forceinline__ void reduce_store(const MVShape& sh, const MVJob& job, float (&acc)[PASSES][NR],
                                             int row0, int rs, int c, int pb, int p1, float* red) {
  const int t = threadIdx.x;
  if (sh.pow2) {
#pragma unroll
    for (int k = 0; k < PASSES; ++k)
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const float v = group_sum(acc[k][r], sh.cpr);
        const int o = row0 + k * sh.rpp + rs;
        if (c == 0 && rs < sh.rpp && o < sh.O && pb + r < p1) job.y[(size_t)(pb + r) * job.ldy + o] = v;
      }
    return;
  }
  const int ld = sh.cpr + 1;
  if (rs < sh.rpp) {
#pragma unroll
    for (int k = 0; k < PASSES; ++k)
#pragma unroll
      for (int r = 0; r < NR; ++r) red[((k * NR + r) * sh.rpp + rs) * ld + c] = acc[k][r];
  }
  __syncthreads();
  const int nsum = PASSES * NR * sh.rpp;
  for (int i = t; i < nsum; i += blockDim.x) {
    const int rs2 = i % sh.rpp, kr = i / sh.rpp, r = kr % NR, k = kr / NR;
    const float* p = red + i * ld;
    float v = 0.f;
    for (int j = 0; j < sh.cpr; ++j) v += p[j];
    const int o = row0 + k * sh.rpp + rs2;
    if (o < sh.O && pb + r < p1) job.y[(size_t)(pb + r) * job.ldy + o] = v;
  }
  __syncthreads();
}

template <class F, int NR, int PASSES>
__global__ __launch_bounds__(256) void mv_kernel(MVShape sh, MVJob job) {
  extern __shared__ float red[];
  const int mat = blockIdx.y;
  int p0 = 0, p1 = job.n;
  if (job.seg) {
    p0 = job.seg[mat];
    p1 = job.seg[mat + 1];
  }
  if (p0 >= p1) return;
  const MatRef M = resolve(job, mat);
  const int t = threadIdx.x;
  const int c = t % sh.cpr, rs = t / sh.cpr;
  const bool lane_on = rs < sh.rpp;
  const int row0 = blockIdx.x * sh.rpp * PASSES;

  const bool a16 = aligned(M.w, 16);
  for (int pb = p0; pb < p1; pb += NR) {
    float xr[NR][F::XR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (lane_on && pb + r < p1) {
        const int p = pb + r;
        const int xrow = job.xrow ? job.xrow[p] : p;
        const XSrc xs = make_xsrc(job.x, job.ldx, xrow, job.half_in);
        F::load_x(xs, c, xr[r]);
      } else {
#pragma unroll
        for (int j = 0; j < F::XR; ++j) xr[r][j] = 0.f;
      }
    }
    uint4 w[PASSES];
#pragma unroll
    for (int k = 0; k < PASSES; ++k) {
      const int o = row0 + k * sh.rpp + rs;
      if (lane_on && o < sh.O) w[k] = load16(M.w + (size_t)o * sh.row_bytes + (size_t)c * 16, a16);
      else w[k] = uint4{};
    }
    float acc[PASSES][NR];
#pragma unroll
    for (int k = 0; k < PASSES; ++k) {
      const int o = row0 + k * sh.rpp + rs;
      const bool on = lane_on && o < sh.O;
      const float sc = on ? load_scale(M.s, (size_t)o * sh.G + (c * F::VALS) / sh.gs, M.s_f16) : 0.f;
#pragma unroll
      for (int r = 0; r < NR; ++r) acc[k][r] = on ? F::dot(w[k], M.xor4, xr[r]) * sc : 0.f;
    }
    reduce_store<PASSES, NR>(sh, job, acc, row0, rs, c, pb, p1, red);
  }
}

// ------------------------------------------------------------------ streaming kernel
//
// The decode kernel for rows whose chunk count is a multiple of 8 (every
// expert shape of interest): L lanes per row (8, 16, 32 or 64), CPL chunks per
// lane, so a wave covers 64/L rows per pass. Each wave owns a run of ng groups
// of G passes; its activations are prepared once into registers, weight loads
// for group g+1 are issued before group g is computed (two register buffers),
// and a row's partial sums are added across its L lanes with DPP row shifts /
// broadcasts (v_add_f32_dpp: no LDS, no barrier). Waves of a block are
// independent.

// passes per register buffer, by chunks per lane and input rows
template <int CPL, int NR>
constexpr int fast_group() {
  return (CPL * NR >= 6) ? 1 : (CPL * NR >= 2 ? 2 : 4);
}

// 16 weight bytes with the alignment known at compile time
template <bool A16>
__device__ __forceinline__ uint4 wload16(const uint8_t* p) {
  if constexpr (A16) {
    return stream_load16(p);
  } else {
    const MOE_GLOBAL uint8_t* q = gptr<uint8_t>(p);
    uint32_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[i] = q[4 * i] | (q[4 * i + 1] << 8) | (q[4 * i + 2] << 16) | ((uint32_t)q[4 * i + 3] << 24);
    return uint4{v[0], v[1], v[2], v[3]};
  }
}

// a scale's bits; converted when used, so that its load is not waited for early
template <bool SF16>
__device__ __forceinline__ uint32_t sload_bits(const void* s, uint32_t idx) {
  if constexpr (SF16) return gptr<uint16_t>(s)[idx];
  else return gptr<uint32_t>(s)[idx];
}

template <bool SF16>
__device__ __forceinline__ float scale_value(uint32_t bits) {
  if constexpr (SF16) return half_bits_to_float(bits);
  else return __builtin_bit_cast(float, bits);
}

// Lane (lg, lc) of a wave works on row lg of each pass of 64/L rows, chunks
// lc, lc + A, ... of it (A <= L lanes of a group are active). Everything a
// lane needs per row is a 24-bit multiply from a uniform base: the chunk
// offsets and scale indices are fixed per lane. Rows past the end of the
// matrix are read as its last row (in bounds) and not stored.
// SHARE (NR = 1): the workgroup's 256 lanes build each input row's chunks
// once into dynamic LDS ([cpr][XR] floats) and every wave reads its lanes'
// chunks from there, instead of each wave building them all; every wave of
// the workgroup then takes part in the set-up's barriers, rows or not.
template <class F, int L, int CPL, int NR, bool SF16, bool A16, bool SHARE>
__device__ __forceinline__ void mv_fast_body(const MVShape& sh, const MVJob& job, const MatRef& M, int A, int ng,
                                             int p0, int p1, int row_begin) {
  constexpr int G = fast_group<CPL, NR>();
  constexpr int RPP = 64 / L;
  const int lane = threadIdx.x & 63;
  const int lg = lane / L, lc = lane % L;
  const bool active = lc < A;  // the first A lanes of a group own the row's chunks
  const int gdiv = sh.gs / F::VALS;  // chunks per scale group (gs is a multiple of VALS here)
  uint32_t woff[CPL], soff[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int chunk = active ? lc + c * A : 0;
    woff[c] = (uint32_t)chunk * 16u;
    soff[c] = (uint32_t)(chunk / gdiv);
  }
  const uint32_t omax = (uint32_t)sh.O - 1u, rb = (uint32_t)sh.row_bytes, gpr = (uint32_t)sh.G;
  const uint8_t* const W = M.w;
  const void* const S = M.s;

  // grid.z splits the input rows: slice z takes batches z, z + gridDim.z, ...
  for (int pb = p0 + (int)blockIdx.z * NR; pb < p1; pb += NR * (int)gridDim.z) {
    float xr[NR][CPL][F::XR];
    uint4 wb[2][G][CPL];
    uint32_t sb[2][G][CPL];
    // buffers are named by compile-time constants only, so they stay in VGPRs
    auto issue = [&](auto buf, int grp) {
      constexpr int B = decltype(buf)::value;
      const uint32_t obase = (uint32_t)(row_begin + grp * (G * RPP) + lg);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t o = min(obase + (uint32_t)(g * RPP), omax);
        const uint32_t wrow = __umul24(o, rb), srow = __umul24(o, gpr);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          wb[B][g][c] = wload16<A16>(W + (wrow + woff[c]));
          sb[B][g][c] = sload_bits<SF16>(S, srow + soff[c]);
        }
      }
    };
    auto compute = [&](auto buf, int grp) {
      constexpr int B = decltype(buf)::value;
      const int obase = row_begin + grp * (G * RPP) + lg;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          float a = 0.f;
#pragma unroll
          for (int c = 0; c < CPL; ++c)
            a = fmaf(F::dot(wb[B][g][c], M.xor4, xr[r][c]), scale_value<SF16>(sb[B][g][c]), a);
          acc[r] = lane_group_sum<L>(a);
        }
        const int o = obase + g * RPP;
        if (lc == L - 1 && o < sh.O) {
#pragma unroll
          for (int r = 0; r < NR; ++r)
            if (pb + r < p1) job.y[(size_t)(pb + r) * job.ldy + o] = acc[r];
        }
      }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    // the first weights go out before the activations are read, so that their
    // latencies overlap; then the steady state with unconditional issues (the
    // compiler's wait counts leave one buffer in flight while the other is
    // used), then the last one or two groups
    issue(B0{}, 0);
    if constexpr (SHARE) {
      static_assert(NR == 1, "the shared set-up holds one input row");
      extern __shared__ float xlds[];  // [cpr][XR]
      const XSrc xs = make_xsrc(job.x, job.ldx, job.xrow ? job.xrow[pb] : pb, job.half_in);
      for (int ci = (int)threadIdx.x; ci < sh.cpr; ci += (int)blockDim.x) {
        float t[F::XR];
        F::load_x(xs, ci, t);
#pragma unroll
        for (int j = 0; j < F::XR; ++j) xlds[ci * F::XR + j] = t[j];
      }
      __syncthreads();
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int j = 0; j < F::XR; ++j) xr[0][c][j] = active ? xlds[(lc + c * A) * F::XR + j] : 0.f;
      if (row_begin >= sh.O) {  // past the matrix's rows: only the set-up is this wave's
        __syncthreads();
        continue;
      }
    } else {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (pb + r < p1) {
          const int p = pb + r;
          const int xrow = job.xrow ? job.xrow[p] : p;
          const XSrc xs = make_xsrc(job.x, job.ldx, xrow, job.half_in);
#pragma unroll
          for (int c = 0; c < CPL; ++c) {
            if (active) F::load_x(xs, lc + c * A, xr[r][c]);
            else
#pragma unroll
              for (int j = 0; j < F::XR; ++j) xr[r][c][j] = 0.f;
          }
        } else {
#pragma unroll
          for (int c = 0; c < CPL; ++c)
#pragma unroll
            for (int j = 0; j < F::XR; ++j) xr[r][c][j] = 0.f;
        }
      }
    }
    int grp = 0;
    for (; grp + 2 < ng; grp += 2) {
      issue(B1{}, grp + 1);
      compute(B0{}, grp);
      issue(B0{}, grp + 2);
      compute(B1{}, grp + 1);
    }
    if (grp + 1 < ng) {
      issue(B1{}, grp + 1);
      compute(B0{}, grp);
      compute(B1{}, grp + 1);
    } else {
      compute(B0{}, grp);
    }
    if constexpr (SHARE) __syncthreads();  // the next input row's set-up rewrites the LDS
  }
}

// ------------------------------------------------------------------ 24-byte int4 chunks
//
// Rows whose 16-byte chunk count is not a power of two leave lanes of every
// group idle (384-byte rows: 24 chunks, 24 of 32 lanes busy). Cut into
// 24-byte chunks (48 values) such rows can fill a group (384 bytes: 16
// chunks, 16 lanes). A chunk is three sub-chunks of 16 values, each inside
// one scale group (gs a multiple of 16), so each sub-chunk has its own scale.
struct Q4W24 {
  static constexpr int XR = 51;

  // xr[m] = x[2m] - x[2m+1]/16, xr[24+m] = x[2m+1]/16 (byte m of the chunk),
  // xr[48+k] = sum of sub-chunk k's 16 values
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {  // one sub-chunk at a time keeps the set-up's registers few
      float v[16];
      xs.run<16>(chunk * 48 + 16 * k, v);
      float sum = 0.f;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const float xe = v[2 * m], xo = v[2 * m + 1];
        xr[8 * k + m] = xe - xo * 0.0625f;
        xr[24 + 8 * k + m] = xo * 0.0625f;
        sum += xe + xo;
      }
      xr[48 + k] = sum;
    }
  }

  // sum over sub-chunk k (words 2k, 2k+1) of (u - 8) * x
  __device__ static float sub(const uint32_t (&w)[6], uint32_t xor4, const float* xr, int k) {
    float acc = 0.f;
#pragma unroll
    for (int i = 2 * k; i < 2 * k + 2; ++i) {
      const uint32_t a = w[i] ^ xor4;
      const uint32_t lo = opaque(a & 0x0F0F0F0Fu);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        acc = fmaf(ubyte(lo, b), xr[4 * i + b], acc);
        acc = fmaf(ubyte(a, b), xr[24 + 4 * i + b], acc);
      }
    }
    return fmaf(-8.0f, xr[48 + k], acc);
  }
};

// The integer dot for the same chunks (as FmtQ4D): each 16-value sub-chunk is
// exact fixed point from its own largest |x|, six 4-bit limb words per weight
// word (limb word 12 k + 6 h + l: digit l of word 2 k + h), xr[36 + k] its
// 2^-S. sub() returns the same sum as Q4W24::sub.
struct Q4W24D {
  static constexpr int XR = 39;

  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      float v[16];
      xs.run<16>(chunk * 48 + 16 * k, v);
      float m = 0.f, z = 0.f;  // z: 0, or NaN when a value is not finite (fmaxf drops NaN)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        m = fmaxf(m, fabsf(v[i]));
        z += v[i] - v[i];
      }
      const int S = 22 - (m > 0.f ? __builtin_amdgcn_frexp_expf(m) : 0);
      uint32_t xb[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) xb[i] = FmtQ4D::fixed_biased(v[i], S);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t w[6];
        FmtQ4D::limbs8(xb + 8 * h, w);
#pragma unroll
        for (int l = 0; l < 6; ++l) xr[12 * k + 6 * h + l] = __builtin_bit_cast(float, w[l]);
      }
      xr[36 + k] = __builtin_ldexpf(1.0f, -S) + z;  // NaN for a sub-chunk holding Inf or NaN
    }
  }

  // sum over sub-chunk k (words 2k, 2k+1) of (u - 8) * x
  __device__ static float sub(const uint32_t (&w)[6], uint32_t xor4, const float* xr, int k) {
    const uint32_t flip = xor4 ^ 0x88888888u;
    const uint32_t s0 = w[2 * k] ^ flip, s1 = w[2 * k + 1] ^ flip;
    int acc[6];
#pragma unroll
    for (int l = 0; l < 6; ++l) {
      acc[l] = __builtin_amdgcn_sdot8((int)s0, (int)__builtin_bit_cast(uint32_t, xr[12 * k + l]), 0, false);
      acc[l] = __builtin_amdgcn_sdot8((int)s1, (int)__builtin_bit_cast(uint32_t, xr[12 * k + 6 + l]), acc[l], false);
    }
    const int lo = acc[0] + 16 * acc[1] + 256 * acc[2];
    const int hi = acc[3] + 16 * acc[4] + 256 * acc[5];
    return fmaf((float)hi, 4096.0f, (float)lo) * xr[36 + k];
  }
};

// One input row for the whole workgroup: its first L lanes build the row's L
// chunks into xsh ([L][XR] floats), then every wave of the workgroup meets at
// one barrier. Every wave calls this exactly once, rows or not.
template <class F, int L>
__device__ __forceinline__ void w24_setup_shared(const MVJob& job, int p, float* xsh) {
  static_assert(F::XR <= 51, "the launch sizes the shared chunks for XR <= 51");
  if ((int)threadIdx.x < L) {
    const XSrc xs = make_xsrc(job.x, job.ldx, job.xrow ? job.xrow[p] : p, job.half_in);
    float t[F::XR];
    F::load_x(xs, (int)threadIdx.x, t);
#pragma unroll
    for (int j = 0; j < F::XR; ++j) xsh[threadIdx.x * F::XR + j] = t[j];
  }
  __syncthreads();
}

// As mv_fast_body with one 24-byte chunk per lane and one input row: L lanes
// per row (all busy), two passes of 64/L rows per register buffer, two
// buffers. Weights are read as three 8-byte words (24-byte offsets are
// 8-byte aligned when the matrix is).
template <class F, int L, int G, bool SF16>
__device__ __forceinline__ void mv_w24_body(const MVShape& sh, const MVJob& job, const MatRef& M, int ng, int p0,
                                            int p1, int row_begin, float* xsh) {
  constexpr int RPP = 64 / L;
  const int lane = threadIdx.x & 63;
  const int lg = lane / L, lc = lane % L;
  const uint32_t woff = (uint32_t)lc * 24u;
  uint32_t soff[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) soff[k] = (uint32_t)((48 * lc + 16 * k) / sh.gs);
  const uint32_t omax = (uint32_t)sh.O - 1u, rb = (uint32_t)sh.row_bytes, gpr = (uint32_t)sh.G;
  const uint8_t* const W = M.w;
  const void* const S = M.s;

  for (int p = p0; p < p1; ++p) {
    float xr[F::XR];
    uint32_t wb[2][G][6];
    uint32_t sb[2][G][3];
    auto issue = [&](auto buf, int grp) {
      constexpr int B = decltype(buf)::value;
      const uint32_t obase = (uint32_t)(row_begin + grp * (G * RPP) + lg);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t o = min(obase + (uint32_t)(g * RPP), omax);
        const uint32_t wrow = __umul24(o, rb), srow = __umul24(o, gpr);
        const MOE_GLOBAL u32x2* wp = gptr<u32x2>(W + (wrow + woff));
#pragma unroll
        for (int h = 0; h < 3; ++h) {
          const u32x2 v = __builtin_nontemporal_load(wp + h);
          wb[B][g][2 * h] = v.x;
          wb[B][g][2 * h + 1] = v.y;
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) sb[B][g][k] = sload_bits<SF16>(S, srow + soff[k]);
      }
    };
    auto compute = [&](auto buf, int grp) {
      constexpr int B = decltype(buf)::value;
      const int obase = row_begin + grp * (G * RPP) + lg;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float a = 0.f;
#pragma unroll
        for (int k = 0; k < 3; ++k) a = fmaf(F::sub(wb[B][g], M.xor4, xr, k), scale_value<SF16>(sb[B][g][k]), a);
        a = lane_group_sum<L>(a);
        const int o = obase + g * RPP;
        if (lc == L - 1 && o < sh.O) job.y[(size_t)p * job.ldy + o] = a;
      }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    issue(B0{}, 0);  // before the activations are read: the latencies overlap
    if (xsh) {  // one input row (p1 = p0 + 1)
      w24_setup_shared<F, L>(job, p, xsh);
#pragma unroll
      for (int j = 0; j < F::XR; ++j) xr[j] = xsh[lc * F::XR + j];
    } else {
      const XSrc xs = make_xsrc(job.x, job.ldx, job.xrow ? job.xrow[p] : p, job.half_in);
      F::load_x(xs, lc, xr);
    }
    int grp = 0;
    for (; grp + 2 < ng; grp += 2) {
      issue(B1{}, grp + 1);
      compute(B0{}, grp);
      issue(B0{}, grp + 2);
      compute(B1{}, grp + 1);
    }
    if (grp + 1 < ng) {
      issue(B1{}, grp + 1);
      compute(B0{}, grp);
      compute(B1{}, grp + 1);
    } else {
      compute(B0{}, grp);
    }
  }
}

// ------------------------------------------------------------------ 24-byte chunks through an LDS ring
//
// mv_w24_body holds its prefetched rows in VGPRs: two passes in flight per
// wave at 158 VGPRs, three waves a SIMD -- about 46 KB in flight per CU, less
// than HBM needs to stay busy. The ring variant streams a wave's run of rows
// (contiguous bytes) and their scales with direct-to-LDS loads
// (global_load_lds_dwordx4: 1 KB a wave per instruction, no VGPRs held) into
// a ring of NS stages of two passes, NS - 1 stages in flight, and computes
// from LDS. Waits are explicit: loads return in issue order, so before stage
// j is read, `s_waitcnt vmcnt(n * D)` (D loads a stage, n stages issued after
// j) leaves exactly the later stages in flight; stores of y issued in between
// count too and can only lengthen the wait. The ring is read by ds_read
// instructions in inline asm that end with their own lgkmcnt wait: the
// compiler tracks direct-to-LDS loads but cannot tell the ring's stages apart
// and would wait for every load in flight before any LDS read it sees.
//
// Stage layout: the weights of 2 * 64 / L rows (3072 bytes: 64 lanes x 24
// bytes a pass), then their scales (sst bytes, at most 1024). A matrix takes
// the ring when its weights and scales are 16-byte aligned and a stage's
// scales fill whole 16-byte loads; otherwise the wave runs mv_w24_body.

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes a lane into LDS at lds + 16 lane, nontemporal (the `nt` cache
// policy, as the register path's streaming loads: rows are read once)
__device__ __forceinline__ void dma16(const void* g, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds, 16, 0, 2);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// wait until at most min(n, NMAX) * D vector-memory operations are outstanding
template <int D, int NMAX>
__device__ __forceinline__ void wait_stages(int n) {
  static_assert(NMAX >= 1 && NMAX <= 3 && 3 * D <= 63, "vmcnt is 6 bits");
  if (n <= 0) wait_vmcnt<0>();
  else if (n == 1 || NMAX == 1) wait_vmcnt<D>();
  else if (n == 2 || NMAX == 2) wait_vmcnt<2 * D>();
  else wait_vmcnt<3 * D>();
}

// one stage's operands for this lane: the 24-byte chunk of two passes
// (addresses a0, a1) and the three scales of each (s0.., s1..), then the wait
template <bool SF16>
__device__ __forceinline__ void lds_stage24(uint32_t a0, uint32_t a1, const uint32_t (&sa)[2][3], uint32_t (&w)[2][6],
                                            uint32_t (&sc)[2][3]) {
  u32x2 v0, v1, v2, v3, v4, v5;
  if constexpr (SF16) {
    asm volatile(
        "ds_read_b64 %0, %12\n\tds_read_b64 %1, %12 offset:8\n\tds_read_b64 %2, %12 offset:16\n\t"
        "ds_read_b64 %3, %13\n\tds_read_b64 %4, %13 offset:8\n\tds_read_b64 %5, %13 offset:16\n\t"
        "ds_read_u16 %6, %14\n\tds_read_u16 %7, %15\n\tds_read_u16 %8, %16\n\t"
        "ds_read_u16 %9, %17\n\tds_read_u16 %10, %18\n\tds_read_u16 %11, %19\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3), "=&v"(v4), "=&v"(v5), "=&v"(sc[0][0]), "=&v"(sc[0][1]),
          "=&v"(sc[0][2]), "=&v"(sc[1][0]), "=&v"(sc[1][1]), "=&v"(sc[1][2])
        : "v"(a0), "v"(a1), "v"(sa[0][0]), "v"(sa[0][1]), "v"(sa[0][2]), "v"(sa[1][0]), "v"(sa[1][1]), "v"(sa[1][2])
        : "memory");
  } else {
    asm volatile(
        "ds_read_b64 %0, %12\n\tds_read_b64 %1, %12 offset:8\n\tds_read_b64 %2, %12 offset:16\n\t"
        "ds_read_b64 %3, %13\n\tds_read_b64 %4, %13 offset:8\n\tds_read_b64 %5, %13 offset:16\n\t"
        "ds_read_b32 %6, %14\n\tds_read_b32 %7, %15\n\tds_read_b32 %8, %16\n\t"
        "ds_read_b32 %9, %17\n\tds_read_b32 %10, %18\n\tds_read_b32 %11, %19\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3), "=&v"(v4), "=&v"(v5), "=&v"(sc[0][0]), "=&v"(sc[0][1]),
          "=&v"(sc[0][2]), "=&v"(sc[1][0]), "=&v"(sc[1][1]), "=&v"(sc[1][2])
        : "v"(a0), "v"(a1), "v"(sa[0][0]), "v"(sa[0][1]), "v"(sa[0][2]), "v"(sa[1][0]), "v"(sa[1][1]), "v"(sa[1][2])
        : "memory");
  }
  const u32x2 v[6] = {v0, v1, v2, v3, v4, v5};
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      w[q][2 * h] = v[3 * q + h].x;
      w[q][2 * h + 1] = v[3 * q + h].y;
    }
}

constexpr int kW24Stage = 2 * 1536;  // weight bytes of a ring stage (two passes)

// the ring's scale bytes a stage for rows of G groups (f16 or f32 scales)
__host__ __device__ inline uint32_t w24_ring_scales(int L, int G, bool f16) {
  return (uint32_t)(2 * (64 / L)) * (uint32_t)G * (f16 ? 2u : 4u);
}

template <class F, int L, int NS, bool SF16>
__device__ __forceinline__ void mv_w24_ring(const MVShape& sh, const MVJob& job, const MatRef& M, int ng, int p,
                                            int row_begin, uint8_t* ring, uint32_t stride, float* xsh) {
  constexpr int RPP = 64 / L, RPS = 2 * RPP;
  constexpr int kWI = kW24Stage / 1024;  // weight loads a stage
  constexpr int D = kWI + 1;              // and one for the scales
  const int lane = threadIdx.x & 63;
  const int lg = lane / L, lc = lane % L;
  const uint32_t rb = (uint32_t)sh.row_bytes, sbr = (uint32_t)sh.G * (SF16 ? 2u : 4u);
  const uint32_t wlast = (uint32_t)sh.O * rb - 16u, slast = ((uint32_t)sh.O * sbr - 16u) & ~15u;
  const uint8_t* const W = M.w;
  const uint8_t* const S = static_cast<const uint8_t*>(M.s);
  // this lane's LDS offsets inside a stage
  const uint32_t ring0 = (uint32_t)(uintptr_t)ring;  // the low 32 bits of a shared address are its LDS offset
  uint32_t wof[2], sof[2][3];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    wof[q] = (uint32_t)(q * RPP + lg) * rb + 24u * (uint32_t)lc;
#pragma unroll
    for (int k = 0; k < 3; ++k)
      sof[q][k] = (uint32_t)kW24Stage + (uint32_t)(q * RPP + lg) * sbr +
                  (uint32_t)((48 * lc + 16 * k) / sh.gs) * (SF16 ? 2u : 4u);
  }
  // stage j's rows into ring slot `slot`. Every lane loads 16 scale bytes,
  // so a stage is always D loads (the stage's scale area is 1024 bytes):
  // lanes past the stage's scales read its first 16 again (the cache line
  // lane 0 reads, so no extra traffic) into the unused part of the area.
  const uint32_t slane = (uint32_t)lane * 16u < RPS * sbr ? 16u * (uint32_t)lane : 0u;
  auto issue = [&](int j, int slot) {
    uint8_t* st = ring + slot * stride;
    const uint32_t r0 = (uint32_t)(row_begin + j * RPS);
    const uint32_t wb = r0 * rb + 16u * (uint32_t)lane;
#pragma unroll
    for (int i = 0; i < kWI; ++i) dma16(W + min(wb + 1024u * i, wlast), st + 1024 * i);
    dma16(S + min(r0 * sbr + slane, slast), st + kW24Stage);
  };
  // the input row's index, then the first stages (a wave of fewer stages
  // loads its last one again into the slots it does not use), then the
  // activations: the latencies overlap
  const int xrow = job.xrow ? job.xrow[p] : p;
#pragma unroll
  for (int j = 0; j < NS - 1; ++j) issue(min(j, ng - 1), j);
  float xr[F::XR];
  if (xsh) {
    w24_setup_shared<F, L>(job, p, xsh);
#pragma unroll
    for (int j = 0; j < F::XR; ++j) xr[j] = xsh[lc * F::XR + j];
  } else {
    const XSrc xs = make_xsrc(job.x, job.ldx, xrow, job.half_in);
    F::load_x(xs, lc, xr);
  }
  for (int j = 0; j < ng; ++j) {
    if (j + NS - 1 < ng) issue(j + NS - 1, (j + NS - 1) % NS);
    wait_stages<D, NS - 1>(min(ng - 1 - j, NS - 1));
    const uint32_t st = ring0 + (uint32_t)(j % NS) * stride;
    uint32_t sa[2][3];
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int k = 0; k < 3; ++k) sa[q][k] = st + sof[q][k];
    uint32_t w[2][6], sc[2][3];
    lds_stage24<SF16>(st + wof[0], st + wof[1], sa, w, sc);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < 3; ++k) a = fmaf(F::sub(w[q], M.xor4, xr, k), scale_value<SF16>(sc[q][k]), a);
      a = lane_group_sum<L>(a);
      const int o = row_begin + j * RPS + q * RPP + lg;
      if (lc == L - 1 && o < sh.O) job.y[(size_t)p * job.ldy + o] = a;
    }
  }
}

// ring_stride > 0: waves stream through LDS rings of NS stages of that many
// bytes (dynamic LDS, one ring a wave), ng stages a wave; 0: mv_w24_body, ng
// groups of G passes a wave
template <class F, int L, int G, int NS>
__global__ __launch_bounds__(256) void mv_q4w24_kernel(MVShape sh, MVJob job, int ng, int ring_stride) {
  extern __shared__ __attribute__((aligned(16))) uint8_t w24_ring[];
  const int mat = blockIdx.y;
  int p0 = 0, p1 = job.n;
  if (job.seg) {
    p0 = job.seg[mat];
    p1 = job.seg[mat + 1];
  }
  if (p0 >= p1) return;
  const int wave = threadIdx.x >> 6;
  const int wave_rows = ring_stride > 0 ? ng * 2 * (64 / L) : ng * G * (64 / L);
  const int row_begin = (blockIdx.x * (blockDim.x >> 6) + wave) * wave_rows;
  // one input row for the workgroup (uniform): its activation chunks are
  // built once, after the rings, and every wave takes part in that barrier
  float* const xsh = p1 - p0 == 1 ? reinterpret_cast<float*>(w24_ring + (size_t)4 * NS * ring_stride) : nullptr;
  if (row_begin >= sh.O) {
    if (xsh) w24_setup_shared<F, L>(job, p0, xsh);
    return;
  }
  const MatRef M = resolve(job, mat);
  if (ring_stride > 0 && p1 - p0 == 1 && aligned(M.w, 16) && aligned(M.s, 16)) {
    const uint32_t sst = w24_ring_scales(L, sh.G, M.s_f16 != 0);
    // the scale loads are whole 16-byte pieces clamped to the matrix's last
    // one: the matrix's scale bytes must end on a 16-byte boundary, or the
    // tail of its last row would be read from the wrong place
    const uint32_t sall = (uint32_t)sh.O * (uint32_t)sh.G * (M.s_f16 ? 2u : 4u);
    if (sst % 16 == 0 && (uint32_t)kW24Stage + sst <= (uint32_t)ring_stride && sall >= 16u && sall % 16u == 0) {
      uint8_t* ring = w24_ring + (size_t)wave * NS * ring_stride;
      if (M.s_f16) mv_w24_ring<F, L, NS, true>(sh, job, M, ng, p0, row_begin, ring, (uint32_t)ring_stride, xsh);
      else mv_w24_ring<F, L, NS, false>(sh, job, M, ng, p0, row_begin, ring, (uint32_t)ring_stride, xsh);
      return;
    }
  }
  // the register path covers the wave's rows in groups of G passes
  const int ngr = (wave_rows + G * (64 / L) - 1) / (G * (64 / L));
  if (M.s_f16) mv_w24_body<F, L, G, true>(sh, job, M, ngr, p0, p1, row_begin, xsh);
  else mv_w24_body<F, L, G, false>(sh, job, M, ngr, p0, p1, row_begin, xsh);
}

// One launch covers every matrix of the call (grid.y); the scale type and the
// weight alignment are uniform per matrix, so the specialised body is chosen
// once at the top.
template <class F, int L, int CPL, int NR, bool SHARE>
__global__ __launch_bounds__(256) void mv_fast_kernel(MVShape sh, MVJob job, int A, int ng) {
  constexpr int G = fast_group<CPL, NR>();
  const int mat = blockIdx.y;
  int p0 = 0, p1 = job.n;
  if (job.seg) {
    p0 = job.seg[mat];
    p1 = job.seg[mat + 1];
  }
  if (p0 >= p1) return;  // the whole workgroup
  const int wave = threadIdx.x >> 6;
  const int wave_rows = ng * G * (64 / L);
  const int row_begin = (blockIdx.x * (blockDim.x >> 6) + wave) * wave_rows;
  // without SHARE there is no block-level synchronisation below
  if (!SHARE && row_begin >= sh.O) return;
  const MatRef M = resolve(job, mat);
  const bool a16 = aligned(M.w, 16);
  if (M.s_f16) {
    if (a16) mv_fast_body<F, L, CPL, NR, true, true, SHARE>(sh, job, M, A, ng, p0, p1, row_begin);
    else mv_fast_body<F, L, CPL, NR, true, false, SHARE>(sh, job, M, A, ng, p0, p1, row_begin);
  } else {
    if (a16) mv_fast_body<F, L, CPL, NR, false, true, SHARE>(sh, job, M, A, ng, p0, p1, row_begin);
    else mv_fast_body<F, L, CPL, NR, false, false, SHARE>(sh, job, M, A, ng, p0, p1, row_begin);
  }
}

// Any int4 / int8 shape the chunked kernels do not take (group sizes that split
// a chunk, unaligned rows): one thread per (output row, input row), straight
// loops. (GGUF rows of any alignment go to blocks.hip.)
__global__ void mv_generic_kernel(MVShape sh, MVJob job, int fmt, int nmat) {
  const int mat = blockIdx.y;
  int p0 = 0, p1 = job.n;
  if (job.seg) {
    p0 = job.seg[mat];
    p1 = job.seg[mat + 1];
  }
  const MatRef M = resolve(job, mat);
  const int np = p1 - p0;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < (long)np * sh.O; i += (long)gridDim.x * blockDim.x) {
    const int p = p0 + (int)(i / sh.O), o = (int)(i % sh.O);
    const int xrow = job.xrow ? job.xrow[p] : p;
    const XSrc xs = make_xsrc(job.x, job.ldx, xrow, job.half_in);
    const uint8_t* row = M.w + (size_t)o * sh.row_bytes;
    float acc = 0.f;
    if (fmt == FMT_Q4) {
      for (int g = 0; g < sh.G; ++g) {
        float part = 0.f;
        for (int j = 0; j < sh.gs; ++j) {
          const int col = g * sh.gs + j;
          const uint32_t b = row[col >> 1] ^ (M.xor4 & 0xFFu);
          const int u = (col & 1) ? (int)(b >> 4) : (int)(b & 15u);
          part = fmaf((float)(u - 8), xs(col), part);
        }
        acc = fmaf(part, load_scale(M.s, (size_t)o * sh.G + g, M.s_f16), acc);
      }
    } else {  // Q8
      for (int g = 0; g < sh.G; ++g) {
        float part = 0.f;
        for (int j = 0; j < sh.gs; ++j) {
          const int col = g * sh.gs + j;
          part = fmaf((float)(int8_t)row[col], xs(col), part);
        }
        acc = fmaf(part, load_scale(M.s, (size_t)o * sh.G + g, M.s_f16), acc);
      }
    }
    job.y[(size_t)p * job.ldy + o] = acc;
  }
}

// ------------------------------------------------------------------ int8 activations
//
// The reference's int8-activation layer call (_moe_q4i, moelan/kernels.py:
// 854-917): each row of activations is rounded to int8 per group of gs
// (a multiple of 64) by _round_q8 (:833-852); a group's product with int4
// weights is an exact integer sum of unsigned nibble * int8 (_q4c64,
// :807-831), turned into f32 once: f32(isum - 8 * sum q) * (s_w * d).
// Rounded rows are stored per 32-column chunk as the 16 even columns' bytes
// then the 16 odd ones', so that one nibble dword meets its activations in
// two v_dot4_i32_i8: low nibbles with the even bytes, high with the odd.

// One wave per (row, group): the group's largest |v|, the scale m / 127 (1 if
// m is 0), q = floor(v * (1 / scale) + 0.5) with the product and the sum
// rounded separately, as the reference writes them. PER = gs / 64 values a lane.
template <int PER>
__global__ __launch_bounds__(256) void round_q8_kernel(const float* x, int ldx, const int* xrow, int n, int K, int half,
                                                       int gs, int8_t* q, float* d, int* s8, const int* rptr,
                                                       const int* rpair, int* pslot) {
  const int G = K / gs;
  const long wid = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wid >= (long)n * G) return;  // the whole wave: no barrier below
  const int p = (int)(wid / G), g = (int)(wid % G);
  // pslot: row p's pairs rpair[rptr[p] .. rptr[p + 1]) read rounded row p
  if (pslot && g == 0)
    for (int j = rptr[p] + lane; j < rptr[p + 1]; j += 64) pslot[rpair[j]] = p;
  const float* row = x + (size_t)(xrow ? xrow[p] : p) * ldx;
  float v[PER];
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = g * gs + 64 * i + lane;
    float t = row[c];
    if (half > 0) t = silu(t) * row[half + c];
    v[i] = t;
    m = fmaxf(m, fabsf(t));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  const float sc = m > 0.f ? m / 127.0f : 1.0f;
  const float inv = 1.0f / sc;
  int sum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int qi = (int)floorf(__fadd_rn(__fmul_rn(v[i], inv), 0.5f));
    sum += qi;
    const int c = g * gs + 64 * i + lane, k = c & 31;
    q[(size_t)p * K + (c - k) + (k & 1) * 16 + (k >> 1)] = (int8_t)qi;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
  if (lane == 0) {
    d[(size_t)p * G + g] = sc;
    s8[(size_t)p * G + g] = 8 * sum;
  }
}

// the sum over aligned groups of GD lanes (GD = 2, 4), in every lane of the group
template <int GD>
__device__ __forceinline__ int lane_group_isum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true);  // quad_perm [1,0,3,2]
  if constexpr (GD >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true);  // quad_perm [2,3,0,1]
  return v;
}

// As mv_fast_body (L lanes per row, CPL chunks per lane, two register buffers
// of G passes) with int8 activations: per chunk two v_dot4 per nibble dword,
// the group's integer sum gathered over its GD lanes, and one f32 term per group
// added by the group's last lane.
template <int L, int CPL, int GD, bool SF16>
__device__ __forceinline__ void mv_q4i8_body(const MVShape& sh, const MVJob& job, const MatRef& M, const int8_t* q,
                                             const float* dq, const int* s8q, int A, int ng, int p0, int p1,
                                             int row_begin) {
  constexpr int G = CPL >= 2 ? 2 : 4;
  constexpr int RPP = 64 / L;
  const int lane = threadIdx.x & 63;
  const int lg = lane / L, lc = lane % L;
  const bool active = lc < A;
  const int gx = sh.I / sh.gs;  // groups of an activation row
  uint32_t woff[CPL], soff[CPL];
  bool tail[CPL];  // the chunk is its group's last: its lane adds the group's term
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int chunk = active ? lc + c * A : 0;
    woff[c] = (uint32_t)chunk * 16u;
    soff[c] = (uint32_t)(chunk / GD);
    tail[c] = active && (chunk % GD) == GD - 1;
  }
  const uint32_t omax = (uint32_t)sh.O - 1u, rb = (uint32_t)sh.row_bytes, gpr = (uint32_t)sh.G;
  const uint8_t* const W = M.w;
  const void* const S = M.s;

  for (int p = p0; p < p1; ++p) {
    // the pair's rounded row (clamped: a pair missing from the row lists
    // reads a wrong row, never past the buffer)
    const int qp = job.xrow ? (int)min((unsigned)job.xrow[p], (unsigned)job.xrows - 1u) : p;
    uint32_t xe[CPL][4], xo[CPL][4];
    float dx[CPL];
    int sx[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int chunk = active ? lc + c * A : 0;
      const uint4 e = *reinterpret_cast<const uint4*>(q + (size_t)qp * sh.I + 32 * chunk);
      const uint4 o = *reinterpret_cast<const uint4*>(q + (size_t)qp * sh.I + 32 * chunk + 16);
      xe[c][0] = e.x; xe[c][1] = e.y; xe[c][2] = e.z; xe[c][3] = e.w;
      xo[c][0] = o.x; xo[c][1] = o.y; xo[c][2] = o.z; xo[c][3] = o.w;
      dx[c] = dq[(size_t)qp * gx + chunk / GD];
      sx[c] = s8q[(size_t)qp * gx + chunk / GD];
    }
    uint4 wb[2][G][CPL];
    uint32_t sb[2][G][CPL];
    auto issue = [&](auto buf, int grp) {
      constexpr int B = decltype(buf)::value;
      const uint32_t obase = (uint32_t)(row_begin + grp * (G * RPP) + lg);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const uint32_t o = min(obase + (uint32_t)(g * RPP), omax);
        const uint32_t wrow = __umul24(o, rb), srow = __umul24(o, gpr);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          wb[B][g][c] = stream_load16(W + (wrow + woff[c]));
          sb[B][g][c] = sload_bits<SF16>(S, srow + soff[c]);
        }
      }
    };
    auto compute = [&](auto buf, int grp) {
      constexpr int B = decltype(buf)::value;
      const int obase = row_begin + grp * (G * RPP) + lg;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float a = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const uint32_t w[4] = {wb[B][g][c].x ^ M.xor4, wb[B][g][c].y ^ M.xor4, wb[B][g][c].z ^ M.xor4,
                                 wb[B][g][c].w ^ M.xor4};
          int isum = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            isum = __builtin_amdgcn_sdot4((int)(w[i] & 0x0F0F0F0Fu), (int)xe[c][i], isum, false);
            isum = __builtin_amdgcn_sdot4((int)((w[i] >> 4) & 0x0F0F0F0Fu), (int)xo[c][i], isum, false);
          }
          isum = lane_group_isum<GD>(isum);
          if (tail[c]) a += (float)(isum - sx[c]) * (scale_value<SF16>(sb[B][g][c]) * dx[c]);
        }
        const float acc = lane_group_sum<L>(a);
        const int o = obase + g * RPP;
        if (lc == L - 1 && o < sh.O) job.y[(size_t)p * job.ldy + o] = acc;
      }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    issue(B0{}, 0);
    int grp = 0;
    for (; grp + 2 < ng; grp += 2) {
      issue(B1{}, grp + 1);
      compute(B0{}, grp);
      issue(B0{}, grp + 2);
      compute(B1{}, grp + 1);
    }
    if (grp + 1 < ng) {
      issue(B1{}, grp + 1);
      compute(B0{}, grp);
      compute(B1{}, grp + 1);
    } else {
      compute(B0{}, grp);
    }
  }
}

template <int L, int CPL, int GD>
__global__ __launch_bounds__(256) void mv_q4i8_kernel(MVShape sh, MVJob job, const int8_t* q, const float* dq,
                                                      const int* s8q, int A, int ng) {
  constexpr int G = CPL >= 2 ? 2 : 4;
  const int mat = blockIdx.y;
  int p0 = 0, p1 = job.n;
  if (job.seg) {
    p0 = job.seg[mat];
    p1 = job.seg[mat + 1];
  }
  if (p0 >= p1) return;
  const int wave = threadIdx.x >> 6;
  const int wave_rows = ng * G * (64 / L);
  const int row_begin = (blockIdx.x * (blockDim.x >> 6) + wave) * wave_rows;
  if (row_begin >= sh.O) return;  // the whole wave: no block-level synchronisation below
  const MatRef M = resolve(job, mat);
  if (M.s_f16) mv_q4i8_body<L, CPL, GD, true>(sh, job, M, q, dq, s8q, A, ng, p0, p1, row_begin);
  else mv_q4i8_body<L, CPL, GD, false>(sh, job, M, q, dq, s8q, A, ng, p0, p1, row_begin);
}

// Any other shape with gs a multiple of 64: one thread per (pair, output row),
// the same sums in the same f32 order as the reference (groups in order).
__global__ void mv_q4i8_generic_kernel(MVShape sh, MVJob job, int nmat, const int8_t* q, const float* dq,
                                       const int* s8q) {
  const int mat = blockIdx.y;
  int p0 = 0, p1 = job.n;
  if (job.seg) {
    p0 = job.seg[mat];
    p1 = job.seg[mat + 1];
  }
  const MatRef M = resolve(job, mat);
  const int np = p1 - p0, gx = sh.I / sh.gs;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < (long)np * sh.O; i += (long)gridDim.x * blockDim.x) {
    const int p = p0 + (int)(i / sh.O), o = (int)(i % sh.O);
    const uint8_t* row = M.w + (size_t)o * sh.row_bytes;
    // the pair's rounded row (clamped: a pair missing from the row lists
    // reads a wrong row, never past the buffer)
    const int qp = job.xrow ? (int)min((unsigned)job.xrow[p], (unsigned)job.xrows - 1u) : p;
    const int8_t* qr = q + (size_t)qp * sh.I;
    float acc = 0.f;
    for (int g = 0; g < gx; ++g) {
      int isum = 0;
      for (int c = g * sh.gs; c < (g + 1) * sh.gs; c += 2) {
        const uint32_t b = row[c >> 1] ^ (M.xor4 & 0xFFu);
        const int k = c & 31, base = c - k;
        isum += (int)(b & 15u) * qr[base + k / 2] + (int)(b >> 4) * qr[base + 16 + k / 2];
      }
      acc += (float)(isum - s8q[(size_t)qp * gx + g]) *
             (load_scale(M.s, (size_t)o * sh.G + g, M.s_f16) * dq[(size_t)qp * gx + g]);
    }
    job.y[(size_t)p * job.ldy + o] = acc;
  }
}

// ------------------------------------------------------------------ host side

static int bytes_per_row(int fmt, int I) {
  switch (fmt) {
    case FMT_Q4: return I / 2;
    case FMT_Q8: return I;
  }
  int per, size, vals;
  return block_geometry(fmt, &per, &size, &vals) ? I / per * size : 0;
}

static int vals_per_chunk(int fmt) {
  switch (fmt) {
    case FMT_Q4: return 32;
    case FMT_Q8: return 16;
  }
  int per, size, vals;
  return block_geometry(fmt, &per, &size, &vals) ? vals : 0;
}

int plan_matvec(int fmt, int O, int I, int gs, MVShape* sh) {
  sh->O = O;
  sh->I = I;
  sh->gs = gs;
  sh->G = (fmt == FMT_Q4 || fmt == FMT_Q8) ? I / gs : 0;
  sh->row_bytes = bytes_per_row(fmt, I);
  const int v = vals_per_chunk(fmt);
  sh->cpr = I / v;  // 0 when a row is narrower than one chunk: generic kernel
  sh->rpp = sh->cpr >= 256 || sh->cpr < 1 ? 1 : 256 / sh->cpr;
  sh->pow2 = (sh->cpr <= 64 && (sh->cpr & (sh->cpr - 1)) == 0) ? 1 : 0;
  return MOE_OK;
}

// Whether the chunked kernels take this shape (pointer alignment is handled
// inside them).
static bool chunked_ok(int fmt, const MVShape& sh) {
  if (sh.cpr < 1 || sh.cpr > 256) return false;
  switch (fmt) {
    case FMT_Q4: return sh.I % 32 == 0 && sh.gs % 32 == 0 && sh.row_bytes % 16 == 0;
    case FMT_Q8: return sh.I % 16 == 0 && sh.gs % 16 == 0 && sh.row_bytes % 16 == 0;
  }
  return false;
}

template <class F, int NR, int PASSES>
static void launch_nr(const MVShape& sh, const MVJob& job, int nmat, hipStream_t st) {
  const int rows_per_block = sh.rpp * PASSES;
  dim3 grid((sh.O + rows_per_block - 1) / rows_per_block, nmat);
  dim3 block(sh.rpp * sh.cpr);
  const size_t lds = sh.pow2 ? 0 : (size_t)PASSES * NR * sh.rpp * (sh.cpr + 1) * sizeof(float);
  hipLaunchKernelGGL((mv_kernel<F, NR, PASSES>), grid, block, lds, st, sh, job);
}

template <class F>
static void launch_fmt(const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st) {
  constexpr int P = 4;
  if (max_rows <= 1) launch_nr<F, 1, P>(sh, job, nmat, st);
  else if (max_rows <= 2) launch_nr<F, 2, P>(sh, job, nmat, st);
  else launch_nr<F, 4, P>(sh, job, nmat, st);
}

// Slices of the input rows (grid.z) for a launch of `waves` waves: with few
// waves and many row batches of NR, each wave would stream its weights once
// per batch in sequence; slices run the batches side by side (the weights are
// read again from L2 or the MALL), up to ~16K waves in all.
int row_slices(int max_rows, int NR, long waves) {
  const long batches = (max_rows + NR - 1) / NR;
  long z = 16384 / (waves > 0 ? waves : 1);
  z = z < 1 ? 1 : (z > batches ? batches : z);
  return (int)(z > 65535 ? 65535 : z);
}

// Stages a wave must stream for the down mat-vec to take its LDS ring: a
// launch of a few experts gives each resident wave only a few stages, and
// then the register path is faster (8 experts x [4096 x 1536]: 13.8 against
// 17.1 us; at 384 experts each wave streams 32 stages and the ring wins).
// MOEHIP_MV_RING_MIN=n overrides it (a measurement switch).
static int ring_min_stages() {
  static const int v = [] {
    const char* e = getenv("MOEHIP_MV_RING_MIN");
    const int n = e ? atoi(e) : 0;
    return n >= 1 && n <= 4096 ? n : 8;
  }();
  return v;
}

template <class F, int L, int CPL>
static void launch_fast_l(const MVShape& sh, const MVJob& job, int nmat, int nr, int max_rows, int A, hipStream_t st) {
  constexpr int rpp = 64 / L;
  // groups of G * rpp rows a wave runs: runs of several groups per wave
  // amortise the activation set-up; keep at least ~8 waves per CU of the 256
  // in flight (longer runs when the activations are SiLU(gate) * up, computed
  // per wave)
  auto runs = [&](int G) {
    const long groups = (long)nmat * ((sh.O + G * rpp - 1) / (G * rpp));  // wave groups in the launch
    static const int ng_env = [] {
      const char* e = getenv("MOEHIP_MV_NGMAX");  // tuning override
      const int v = e ? atoi(e) : 0;
      return v >= 1 && v <= 64 ? v : 0;
    }();
    const int ng_max = ng_env ? ng_env : (job.half_in > 0 ? 32 : 16);
    const int ng = (int)(groups / 2048);
    return ng < 1 ? 1 : (ng > ng_max ? ng_max : ng);
  };
  auto go = [&](auto kernel, int G, int NR) {
    const int ng = runs(G);
    const int wave_rows = ng * G * rpp;
    const int waves = (sh.O + wave_rows - 1) / wave_rows;
    dim3 grid((waves + 3) / 4, nmat, row_slices(max_rows, NR, (long)waves * nmat));
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, st, sh, job, A, ng);
  };
  // One input row a matrix: the workgroup's 4 waves share the activation
  // set-up through LDS (the integer-dot format only)
  static const bool share_env = [] {
    const char* e = getenv("MOEHIP_MV_SHARE");  // measurement switch: 0 keeps a set-up per wave
    return !(e && e[0] == '0');
  }();
  if (std::is_same<F, FmtQ4D>::value && nr == 1 && max_rows == 1 && share_env) {
    constexpr int G = fast_group<CPL, 1>();
    const int ng = runs(G);
    const int wave_rows = ng * G * rpp;
    const int waves = (sh.O + wave_rows - 1) / wave_rows;
    const size_t lds = (size_t)sh.cpr * F::XR * sizeof(float);
    if (lds <= 32768) {
      hipLaunchKernelGGL((mv_fast_kernel<F, L, CPL, 1, true>), dim3((waves + 3) / 4, nmat, 1), dim3(256), lds, st,
                         sh, job, A, ng);
      return;
    }
  }
  if (nr == 1) go(mv_fast_kernel<F, L, CPL, 1, false>, fast_group<CPL, 1>(), 1);
  else if (nr == 2 || CPL > 1) go(mv_fast_kernel<F, L, CPL, 2, false>, fast_group<CPL, 2>(), 2);
  else go(mv_fast_kernel<F, L, 1, 4, false>, fast_group<1, 4>(), 4);
}

// Lanes per row: by default one chunk per lane whenever a row has at most 64
// chunks (idle lanes fill a power-of-two group if it stays >= 3/4 busy),
// otherwise power-of-two groups with several chunks per lane. MOEHIP_MV_DENSE=1
// always takes the latter (for measurements).
static void lanes_for(int cpr, int* L, int* A, int* cpl) {
  static const int dense = [] {
    const char* e = getenv("MOEHIP_MV_DENSE");
    return e && e[0] == '1';
  }();
  if (!dense && cpr <= 64) {
    int l = 8;
    while (l < cpr) l <<= 1;
    if (4 * cpr >= 3 * l) {
      *L = l;
      *A = cpr;
      *cpl = 1;
      return;
    }
  }
  int l = 64;
  while (cpr % l) l >>= 1;
  *L = l;
  *A = l;
  *cpl = cpr / l;
}

// false: the shape goes to the general kernels
// The fast kernels form row offsets with 24-bit multiplies into 32 bits.
static bool offsets_fit(const MVShape& sh) {
  return sh.O < (1 << 24) && (uint64_t)sh.O * (uint64_t)sh.row_bytes < (1ull << 32);
}

template <class F>
static bool launch_fast(const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st) {
  if (sh.cpr % 8 != 0 || !offsets_fit(sh)) return false;
  int L, A, cpl;
  lanes_for(sh.cpr, &L, &A, &cpl);
  const int nr = max_rows <= 1 ? 1 : (max_rows <= 2 ? 2 : 4);
  if (L == 64) {
    switch (cpl) {
      case 1: launch_fast_l<F, 64, 1>(sh, job, nmat, nr, max_rows, A, st); return true;
      case 2: launch_fast_l<F, 64, 2>(sh, job, nmat, nr, max_rows, A, st); return true;
      case 3: launch_fast_l<F, 64, 3>(sh, job, nmat, nr, max_rows, A, st); return true;
      case 4: launch_fast_l<F, 64, 4>(sh, job, nmat, nr, max_rows, A, st); return true;
    }
    return false;
  }
  if (L == 32 && cpl == 1) { launch_fast_l<F, 32, 1>(sh, job, nmat, nr, max_rows, A, st); return true; }
  if (L == 32 && cpl == 2) { launch_fast_l<F, 32, 2>(sh, job, nmat, nr, max_rows, A, st); return true; }
  if (L == 16 && cpl == 1) { launch_fast_l<F, 16, 1>(sh, job, nmat, nr, max_rows, A, st); return true; }
  if (L == 8 && cpl == 1) { launch_fast_l<F, 8, 1>(sh, job, nmat, nr, max_rows, A, st); return true; }
  return false;
}

// Waves of a ring kernel resident on the current device at once for a block
// size and LDS size (0 when unknown), cached per device, kernel and sizes.
static long ring_slots(const void* kernel, int threads, size_t lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, const void*, int, size_t>, long> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const auto key = std::make_tuple(dev, kernel, threads, lds);
  {
    std::lock_guard<std::mutex> g(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int per_cu = 0, cus = 0;
  long slots = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) == hipSuccess && per_cu > 0 &&
      cus > 0)
    slots = (long)per_cu * (threads / 64) * cus;
  std::lock_guard<std::mutex> g(mu);
  cache[key] = slots;
  return slots;
}

// MOEHIP_MV_FLOATDOT=1 keeps the int4 float dot (FmtQ4, Q4W24) in place of
// the integer dot (FmtQ4D, Q4W24D): a measurement switch
static bool float_dot() {
  static const bool on = [] {
    const char* e = getenv("MOEHIP_MV_FLOATDOT");
    return e && e[0] == '1';
  }();
  return on;
}

// MOEHIP_MV_RING=0 keeps the register paths (a measurement switch)
static bool ring_disabled() {
  static const bool off = [] {
    const char* e = getenv("MOEHIP_MV_RING");
    return e && e[0] == '0';
  }();
  return off;
}

// 24-byte chunks for int4 rows whose 16-byte chunks do not fill a lane group
// but whose 24-byte chunks do (8, 16, 32 or 64 of them); one input row a pair
static bool launch_w24(const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st) {
  static const int off = [] {
    const char* e = getenv("MOEHIP_MV_NO24");  // measurement switch: keep 16-byte chunks
    return e && e[0] == '1';
  }();
  if (off || max_rows != 1 || sh.row_bytes % 24 != 0 || sh.gs % 16 != 0 || !offsets_fit(sh)) return false;
  const int c16 = sh.row_bytes / 16, c24 = sh.row_bytes / 24;
  if (sh.row_bytes % 16 == 0 && (c16 & (c16 - 1)) == 0) return false;  // 16-byte chunks fill their groups
  int L = 0;
  if (c24 == 8 || c24 == 16 || c24 == 32 || c24 == 64) L = c24;
  if (L == 0) return false;
  constexpr int G = 2;   // passes per register buffer (1: 126 VGPRs, 4 waves a SIMD, measured no faster)
  constexpr int NS = 3;  // ring stages a wave
  const bool ring_off = ring_disabled();
  const int rpp = 64 / L;
  auto go = [&](auto kernel) {
    int ng, wave_rows, stride = 0;
    size_t lds = 0;
    // the ring's stage: the weights of 2 rpp rows and a 1024-byte scale area
    // (wider scale rows take the register path)
    const int ring_stride = kW24Stage + 1024;
    const size_t xsh_lds = (size_t)L * 51 * sizeof(float);  // the shared chunks ([L][XR], XR <= 51)
    const size_t ring_lds = (size_t)4 * NS * ring_stride + xsh_lds;
    // waves resident at once (LDS-bound), spread evenly over the matrices
    const long slots = ring_off ? 0 : ring_slots(reinterpret_cast<const void*>(kernel), 256, ring_lds);
    if (slots > 0) {
      stride = ring_stride;
      static const int rounds = [] {
        const char* e = getenv("MOEHIP_MV_RING_ROUNDS");  // tuning override
        const int v = e ? atoi(e) : 0;
        return v >= 1 && v <= 64 ? v : 1;
      }();
      const int spm = (sh.O + 2 * rpp - 1) / (2 * rpp);  // stages a matrix
      long wpm = rounds * slots / nmat;
      wpm = wpm < 1 ? 1 : (wpm > spm ? spm : wpm);
      ng = (int)((spm + wpm - 1) / wpm);
      wave_rows = ng * 2 * rpp;
      if (ng < ring_min_stages()) stride = 0;
    }
    if (stride > 0) {
      lds = ring_lds;
    } else {
      lds = xsh_lds;
      const long groups = (long)nmat * ((sh.O + G * rpp - 1) / (G * rpp));
      const int ng_max = job.half_in > 0 ? 32 : 16;
      ng = (int)(groups / 2048);
      ng = ng < 1 ? 1 : (ng > ng_max ? ng_max : ng);
      wave_rows = ng * G * rpp;
    }
    const int waves = (sh.O + wave_rows - 1) / wave_rows;
    const dim3 grid((waves + 3) / 4, nmat);
    hipLaunchKernelGGL(kernel, grid, dim3(256), lds, st, sh, job, ng, stride);
    return true;
  };
  if (float_dot()) {
    switch (L) {
      case 8: return go(mv_q4w24_kernel<Q4W24, 8, G, NS>);
      case 16: return go(mv_q4w24_kernel<Q4W24, 16, G, NS>);
      case 32: return go(mv_q4w24_kernel<Q4W24, 32, G, NS>);
      default: return go(mv_q4w24_kernel<Q4W24, 64, G, NS>);
    }
  }
  switch (L) {
    case 8: return go(mv_q4w24_kernel<Q4W24D, 8, G, NS>);
    case 16: return go(mv_q4w24_kernel<Q4W24D, 16, G, NS>);
    case 32: return go(mv_q4w24_kernel<Q4W24D, 32, G, NS>);
    default: return go(mv_q4w24_kernel<Q4W24D, 64, G, NS>);
  }
}

int run_matvec(int fmt, const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st) {
  if (max_rows <= 0 || nmat <= 0 || sh.O <= 0) return MOE_OK;
  int per, size, vals;
  if (block_geometry(fmt, &per, &size, &vals)) return run_matvec_blocks(fmt, sh, job, nmat, max_rows, st);  // GGUF
  if (chunked_ok(fmt, sh)) {
    if (fmt == FMT_Q4 && launch_w24(sh, job, nmat, max_rows, st)) return check_launch("int4 mat-vec (24-byte chunks)");
    if (fmt == FMT_Q4 &&
        (float_dot() ? launch_fast<FmtQ4>(sh, job, nmat, max_rows, st) : launch_fast<FmtQ4D>(sh, job, nmat, max_rows, st)))
      return check_launch("int4 mat-vec");
    if (fmt == FMT_Q8 && launch_fast<FmtQ8>(sh, job, nmat, max_rows, st)) return check_launch("int8 mat-vec");
    const int nr = max_rows <= 1 ? 1 : (max_rows <= 2 ? 2 : 4);
    const size_t lds = sh.pow2 ? 0 : (size_t)4 * nr * sh.rpp * (sh.cpr + 1) * sizeof(float);
    if (lds <= 64 * 1024) {
      switch (fmt) {
        case FMT_Q4: launch_fmt<FmtQ4>(sh, job, nmat, max_rows, st); break;
        case FMT_Q8: launch_fmt<FmtQ8>(sh, job, nmat, max_rows, st); break;
      }
      return check_launch("decode mat-vec");
    }
  }
  const long work = (long)max_rows * sh.O;
  const int threads = 256;
  const int blocks = (int)((work + threads - 1) / threads > 4096 ? 4096 : (work + threads - 1) / threads);
  hipLaunchKernelGGL(mv_generic_kernel, dim3(blocks, nmat), dim3(threads), 0, st, sh, job, fmt, nmat);
  return check_launch("decode mat-vec (generic)");
}

int run_round_q8(const float* x, int ldx, const int* xrow, int n, int K, int half, int gs, int8_t* q, float* d, int* s8,
                 hipStream_t st, const int* rptr, const int* rpair, int* pslot) {
  if (n <= 0) return MOE_OK;
  if (gs % 64 != 0 || K % gs != 0)
    return set_error(MOE_EUNSUPPORTED, "int8 activations: group size %d must be a multiple of 64 dividing %d", gs, K);
  const long waves = (long)n * (K / gs);
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, block, 0, st, x, ldx, xrow, n, K, half, gs, q, d, s8, rptr, rpair, pslot);
  };
  switch (gs / 64) {
    case 1: go(round_q8_kernel<1>); break;
    case 2: go(round_q8_kernel<2>); break;
    case 3: go(round_q8_kernel<3>); break;
    case 4: go(round_q8_kernel<4>); break;
    case 5: go(round_q8_kernel<5>); break;
    case 6: go(round_q8_kernel<6>); break;
    case 7: go(round_q8_kernel<7>); break;
    case 8: go(round_q8_kernel<8>); break;
    default: return set_error(MOE_EUNSUPPORTED, "int8 activations: group size %d (a multiple of 64 up to 512)", gs);
  }
  return check_launch("round activations to int8");
}

template <int L, int CPL, int GD>
static void launch_q4i8(const MVShape& sh, const MVJob& job, int nmat, const int8_t* q, const float* dq,
                        const int* s8q, int A, hipStream_t st) {
  constexpr int G = CPL >= 2 ? 2 : 4;
  constexpr int rpp = 64 / L;
  const long groups = (long)nmat * ((sh.O + G * rpp - 1) / (G * rpp));
  int ng = (int)(groups / 2048);
  ng = ng < 1 ? 1 : (ng > 16 ? 16 : ng);
  const int wave_rows = ng * G * rpp;
  const int waves = (sh.O + wave_rows - 1) / wave_rows;
  hipLaunchKernelGGL((mv_q4i8_kernel<L, CPL, GD>), dim3((waves + 3) / 4, nmat), dim3(256), 0, st, sh, job, q, dq, s8q,
                     A, ng);
}

template <int GD>
static bool launch_q4i8_gd(const MVShape& sh, const MVJob& job, int nmat, const int8_t* q, const float* dq,
                           const int* s8q, hipStream_t st) {
  if (sh.cpr % 8 != 0 || !offsets_fit(sh)) return false;
  int L, A, cpl;
  lanes_for(sh.cpr, &L, &A, &cpl);
  if (A % GD != 0) return false;
  if (L == 64 && cpl == 1) launch_q4i8<64, 1, GD>(sh, job, nmat, q, dq, s8q, A, st);
  else if (L == 64 && cpl == 2) launch_q4i8<64, 2, GD>(sh, job, nmat, q, dq, s8q, A, st);
  else if (L == 64 && cpl == 4) launch_q4i8<64, 4, GD>(sh, job, nmat, q, dq, s8q, A, st);
  else if (L == 32 && cpl == 1) launch_q4i8<32, 1, GD>(sh, job, nmat, q, dq, s8q, A, st);
  else if (L == 16 && cpl == 1) launch_q4i8<16, 1, GD>(sh, job, nmat, q, dq, s8q, A, st);
  else if (L == 8 && cpl == 1) launch_q4i8<8, 1, GD>(sh, job, nmat, q, dq, s8q, A, st);
  else return false;
  return true;
}

int run_matvec_q4i8(const MVShape& sh, const MVJob& job, int nmat, const int8_t* q, const float* dq, const int* s8q,
                    hipStream_t st) {
  if (nmat <= 0) return MOE_OK;
  bool done = false;  // the rounded activations are the layer's own 256-byte aligned buffers
  if (sh.row_bytes % 16 == 0) {
    if (sh.gs == 64) done = launch_q4i8_gd<2>(sh, job, nmat, q, dq, s8q, st);
    else if (sh.gs == 128) done = launch_q4i8_gd<4>(sh, job, nmat, q, dq, s8q, st);
  }
  if (!done) {
    const long work = (long)job.n * sh.O;
    long blocks = (work + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(mv_q4i8_generic_kernel, dim3((unsigned)blocks, nmat), dim3(256), 0, st, sh, job, nmat, q, dq,
                       s8q);
  }
  return check_launch("int4 mat-vec, int8 activations");
}

}  // namespace moe
