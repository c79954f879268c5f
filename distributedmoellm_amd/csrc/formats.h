// Weight formats of the routed-expert path, as seen by the decode mat-vec.
//
// A weight row is cut into "chunks": the unit one lane owns. A lane keeps the
// activations its chunk multiplies in registers (prepared once per input row)
// and streams the same chunk column through many weight rows, so activations
// are never re-read while weights stream from HBM.
//
//   Q4   colibri int4 (moelan/experts.py:170-236): 16 bytes = 32 columns, byte j
//        holds column 2j in the low and 2j+1 in the high nibble; nibbles become
//        unsigned with XOR 0x88 (u = v + 8); one scale per gs columns.
//   Q8   group-scaled int8 (moelan/experts.py:125-167): 16 bytes = 16 columns.
//   Q4_K GGUF superblock of 144 bytes (moelan/kernels.py:310-336): a chunk is
//        16 bytes of its nibbles (16 low + 16 high values) plus the header; the
//        GGUF mat-vec itself is in blocks.hip.
#pragma once
#include "common.h"

namespace moe {

// Where the activations of one input row come from: a plain f32 row, or the
// gate|up output h of an expert (2*I values) turned into silu(gate) * up.
// A chunk's activations are runs of consecutive columns, read with 16-byte
// loads when the row allows it; the silu/plain choice is made once per run.
struct XSrc {
  const float* row;
  int half;  // > 0: silu input, h[c] is gate, h[half + c] is up
  bool a16;  // row (and, for silu, row + half) 16-byte aligned

  template <int N>
  __device__ __forceinline__ void raw(const float* p, float* v) const {
    if (a16) {
#pragma unroll
      for (int i = 0; i < N / 4; ++i) {
        const float4 q = reinterpret_cast<const float4*>(p)[i];
        v[4 * i] = q.x;
        v[4 * i + 1] = q.y;
        v[4 * i + 2] = q.z;
        v[4 * i + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) v[i] = p[i];
    }
  }

  // v[0..N) = activations of columns c0 .. c0+N-1 (N a multiple of 4, c0 of 4)
  template <int N>
  __device__ __forceinline__ void run(int c0, float* v) const {
    if (half > 0) {
      float u[N];
      raw<N>(row + c0, v);
      raw<N>(row + half + c0, u);
#pragma unroll
      for (int i = 0; i < N; ++i) v[i] = silu(v[i]) * u[i];
    } else {
      raw<N>(row + c0, v);
    }
  }

  // one column (generic kernels)
  __device__ __forceinline__ float operator()(int c) const {
    if (half > 0) return silu(row[c]) * row[half + c];
    return row[c];
  }
};

__device__ __forceinline__ XSrc make_xsrc(const float* x, int ldx, int xrow, int half) {
  const float* row = x + (size_t)xrow * ldx;
  const bool a = aligned(row, 16) && (half % 4) == 0;
  return XSrc{row, half, a};
}

// ------------------------------------------------------------------ Q4
struct FmtQ4 {
  static constexpr int VALS = 32;   // columns per chunk
  static constexpr int XR = 33;     // activation registers per chunk and row
  static constexpr int BYTES = 16;

  // xr[m] = x[2m] - x[2m+1]/16, xr[16+m] = x[2m+1]/16, xr[32] = sum of the 32.
  // With u-nibbles lo, hi and the byte b = lo + 16 hi of byte m:
  //   lo*x[2m] + hi*x[2m+1] = lo*xr[m] + b*xr[16+m]
  // so one masked word and the raw word feed v_cvt_f32_ubyteK directly.
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) {
    float v[32];
    xs.run<32>(chunk * 32, v);
    float sum = 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const float xe = v[2 * m], xo = v[2 * m + 1];
      xr[m] = xe - xo * 0.0625f;
      xr[16 + m] = xo * 0.0625f;
      sum += xe + xo;
    }
    xr[32] = sum;
  }

  // sum over the chunk of (u - 8) * x, u the unsigned nibble
  __device__ static float dot(const uint4 w, uint32_t xor4, const float* xr) {
    const uint32_t a[4] = {w.x ^ xor4, w.y ^ xor4, w.z ^ xor4, w.w ^ xor4};
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = opaque(a[i] & 0x0F0F0F0Fu);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc = fmaf(ubyte(lo, k), xr[4 * i + k], acc);
        acc = fmaf(ubyte(a[i], k), xr[16 + 4 * i + k], acc);
      }
    }
    return fmaf(-8.0f, xr[32], acc);
  }
};

// ------------------------------------------------------------------ Q4, integer dot
// The same 32-value chunk as FmtQ4, multiplied with v_dot8c_i32_i4 (8 signed
// nibbles x 8 signed nibbles, exact) instead of 32 converts and 32 FMAs.
//  * Activations: the chunk's 32 values as exact fixed point x_int =
//    rint(x * 2^S), |x_int| <= 2^22, S from the chunk's largest |x|. Each is
//    the sum of six balanced 4-bit digits d_k * 16^k, d_k in [-8, 7]: the
//    hex digits of x_int + 0x888888, minus 8. Limb word 6 j + k holds digit
//    k of the 8 values of weight word j, value i in nibble i, as two's
//    complement. xr[24] = 2^-S (NaN when the chunk holds a non-finite value).
//  * Weights: u ^ 8 is the signed nibble u - 8 (u = stored ^ xor4).
//  * Dot: acc_k = sum over the 4 words of dot8(w, limb k), exact; the chunk's
//    sum (u - 8) * x_int = sum acc_k 16^k, formed as two exact 3-limb
//    integers joined by one rounding, then scaled by 2^-S.
// Each product term is off by at most |u - 8| * 2^-(S+1) <= 8 * 2^-22 of the
// chunk's largest |x| m (2^-(S+1) <= 2^-22 m, as m >= 2^(21-S)), and a
// one-hot x is exact.
struct FmtQ4D {
  static constexpr int VALS = 32;
  static constexpr int XR = 25;
  static constexpr int BYTES = 16;

  // rint(v * 2^S) + 0x888888 as 24 bits. The clamp to +-2^22 only acts on
  // non-finite values (finite ones are within it by the choice of S) and
  // keeps the conversion defined; NaN clamps to -2^22.
  __device__ static uint32_t fixed_biased(float v, int S) {
    const float t = fminf(fmaxf(__builtin_rintf(__builtin_ldexpf(v, S)), -4194304.0f), 4194304.0f);
    return (uint32_t)((int)t + 0x888888);
  }

  // limb words of 8 biased values xb (24 bits each): six words, digit k of
  // value i in nibble i of word k, XOR 8 per nibble (two's complement digit)
  __device__ static void limbs8(const uint32_t* xb, uint32_t* out) {
    uint32_t E[4], O[4];  // byte n of E[p]: digit 2n of values 2p (low nibble) and 2p+1; O: digit 2n+1
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      E[p] = (xb[2 * p] & 0x0F0F0F0Fu) | ((xb[2 * p + 1] << 4) & 0xF0F0F0F0u);
      O[p] = ((xb[2 * p] >> 4) & 0x0F0F0F0Fu) | (xb[2 * p + 1] & 0xF0F0F0F0u);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t* src = h ? O : E;
      // byte gathers: perm(hi, lo, sel) picks bytes 0-3 of lo, 4-7 of hi.
      // p01 = [src0.b0, src1.b0, src0.b1, src1.b1], p45 the same of src2, src3;
      // q01 = [src0.b2, src1.b2, ...]; digit word n takes byte n of each pair
      const uint32_t p01 = __builtin_amdgcn_perm(src[1], src[0], 0x05010400u);
      const uint32_t p45 = __builtin_amdgcn_perm(src[3], src[2], 0x05010400u);
      const uint32_t q01 = __builtin_amdgcn_perm(src[1], src[0], 0x06020602u);
      const uint32_t q45 = __builtin_amdgcn_perm(src[3], src[2], 0x06020602u);
      out[h + 0] = __builtin_amdgcn_perm(p45, p01, 0x05040100u) ^ 0x88888888u;
      out[h + 2] = __builtin_amdgcn_perm(p45, p01, 0x07060302u) ^ 0x88888888u;
      out[h + 4] = __builtin_amdgcn_perm(q45, q01, 0x05040100u) ^ 0x88888888u;
    }
  }

  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) {
    float v[32];
    xs.run<32>(chunk * 32, v);
    // m: the largest |x| (fmaxf drops NaN); z: 0, or NaN when a value is not finite
    float m = 0.f, z = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      m = fmaxf(m, fabsf(v[i]));
      z += v[i] - v[i];
    }
    const int S = 22 - (m > 0.f ? __builtin_amdgcn_frexp_expf(m) : 0);
    uint32_t xb[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) xb[i] = fixed_biased(v[i], S);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t w[6];
      limbs8(xb + 8 * j, w);
#pragma unroll
      for (int k = 0; k < 6; ++k) xr[6 * j + k] = __builtin_bit_cast(float, w[k]);
    }
    xr[24] = __builtin_ldexpf(1.0f, -S) + z;  // NaN for a chunk holding Inf or NaN
  }

  // sum over the chunk of (u - 8) * x, u the unsigned nibble
  __device__ static float dot(const uint4 w, uint32_t xor4, const float* xr) {
    const uint32_t flip = xor4 ^ 0x88888888u;
    const uint32_t s[4] = {w.x ^ flip, w.y ^ flip, w.z ^ flip, w.w ^ flip};
    int acc[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      acc[k] = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[k] = __builtin_amdgcn_sdot8((int)s[j], (int)__builtin_bit_cast(uint32_t, xr[6 * j + k]), acc[k], false);
    }
    const int lo = acc[0] + 16 * acc[1] + 256 * acc[2];
    const int hi = acc[3] + 16 * acc[4] + 256 * acc[5];
    return fmaf((float)hi, 4096.0f, (float)lo) * xr[24];
  }
};

// ------------------------------------------------------------------ Q8
struct FmtQ8 {
  static constexpr int VALS = 16;
  static constexpr int XR = 16;
  static constexpr int BYTES = 16;

  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { xs.run<16>(chunk * 16, xr); }

  __device__ static float dot(const uint4 w, uint32_t, const float* xr) {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) acc = fmaf((float)(int8_t)(a[i] >> (8 * k)), xr[4 * i + k], acc);
    return acc;
  }
};

// ------------------------------------------------------------------ GGUF Q4_K
// Q4_K helpers shared by the block mat-vec (blocks.hip) and the dequant
struct FmtQ4K {
  // chunk c: superblock c/8, nibble group kk = (c%8)/2, half = c%2. Its 16
  // bytes give values 64kk + 16half + l (low nibble, sub-block 2kk) and
  // 64kk + 32 + 16half + l (high nibble, sub-block 2kk+1), l = 0..15.
  __device__ static int col_lo(int chunk) {
    const int sb = chunk >> 3, j = chunk & 7;
    return sb * 256 + (j >> 1) * 64 + (j & 1) * 16;
  }

  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) {
    const int c0 = col_lo(chunk);
    xs.run<16>(c0, xr);
    xs.run<16>(c0 + 32, xr + 16);
    float slo = 0.f, shi = 0.f;
#pragma unroll
    for (int l = 0; l < 16; ++l) {
      slo += xr[l];
      shi += xr[16 + l];
    }
    xr[32] = slo;
    xr[33] = shi;
  }

  // scale / min of sub-block j from the 12 packed bytes (moelan/kernels.py:310-316);
  // `s(i)` returns packed byte i
  template <class B>
  __device__ static void scale_min(int j, const B& s, int& sc, int& m) {
    if (j < 4) {
      sc = s(j) & 63;
      m = s(j + 4) & 63;
    } else {
      sc = (s(j + 4) & 0xF) | ((s(j - 4) >> 6) << 4);
      m = (s(j + 4) >> 4) | ((s(j) >> 6) << 4);
    }
  }

  // the 12 packed bytes held in the header's last three words (selects, no
  // private-memory array)
  struct HdrBytes {
    uint32_t w0, w1, w2;
    __device__ int operator()(int i) const {
      const uint32_t w = i < 4 ? w0 : (i < 8 ? w1 : w2);
      return (int)((w >> (8 * (i & 3))) & 0xFFu);
    }
  };
  struct MemBytes {
    const uint8_t* p;
    __device__ int operator()(int i) const { return p[i]; }
  };
};

}  // namespace moe
