// GGUF block types: the decode mat-vec of every quantized type, and the
// bit-exact dequant of all but Q8_0 / Q4_K (dequant.hip has those)
// (moelan/kernels.py:262-453 decoders, 482-676 fused mat-vecs, 981-1003
// dispatch).
//
//   Q8_0  34 B / 32 values: f16 d, 32 int8; w = d * q
//   Q4_K  144 B / 256: d, dmin, 12 bytes of 6-bit scale/min, 128 nibble bytes;
//         w = (d*sc) * q - dmin*m
//   Q4_0  18 B / 32 values: f16 d, 16 bytes; byte j = value j (low nibble) and
//         j+16 (high); w = d * (q - 8)
//   Q4_1  20 B: d, f16 min, 16 bytes; w = d * q + min
//   Q5_0  22 B: d, 32-bit qh (bit j = bit 4 of value j), 16 bytes; w = d * (q - 16) + 0
//   Q5_1  24 B: d, min, qh, 16 bytes; w = d * q + min
//   Q2_K  84 B / 256: 16 bytes of (scale | min << 4) per 16 values, 64 bytes of
//         2-bit values, f16 d, f16 dmin; w = (d*sc) * q - dmin*m
//   Q3_K  110 B: 32 hmask bytes, 64 bytes of 2-bit values, 12 bytes of 6-bit
//         scales, f16 d; w = (d*sc) * (q - 4 unless the hmask bit is set)
//   Q5_K  176 B: d, dmin, 12 bytes of 6-bit scale/min (as Q4_K), 32 qh bytes,
//         128 nibble bytes; w = (d*sc) * (q + 16h) - dmin*m
//   Q6_K  210 B: 128 ql bytes, 64 qh bytes, 16 int8 scales, f16 d;
//         w = d * (sc * (q - 32))
//
// Mat-vec layout. A lane owns a "chunk" of a row cut where the bytes are: a
// whole block for the 32-value types; for the K types a run of 16 (Q2_K,
// Q3_K, Q6_K) or 16+16 (Q5_K) storage bytes together with every value those
// bytes hold (64 or 32 values), so that each byte a lane reads is used by
// that lane, and neighbouring lanes read neighbouring bytes. The chunk's
// activations (and their sums per scale) are prepared once per input row in
// registers; the lane then streams the chunk column down ng * 64/L rows, two
// rows' bytes in flight. Rows need no alignment: a lane reads the aligned
// words that overlap its bytes and realigns them with v_alignbyte.
#include "common.h"
#include "formats.h"
#include "matvec.h"
#include "blocks.h"

#include <type_traits>

namespace moe {

namespace {

// Bytes [p, p + N) as ceil(N/4) little-endian words. Only the aligned words
// that overlap the span are read: each holds at least one of its bytes, so
// none lies on a page the buffer does not touch.
template <int N>
__device__ __forceinline__ void load_span(const uint8_t* p, uint32_t (&w)[(N + 3) / 4]) {
  constexpr int NW = (N + 3) / 4;
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t sh = (uint32_t)(a & 3u);
  const uintptr_t base = a - sh;
  uint32_t d[NW + 1];
#pragma unroll
  for (int i = 0; i < NW; ++i) d[i] = __builtin_nontemporal_load(gptr<uint32_t>((const void*)(base + 4 * i)));
  d[NW] = (sh + N > 4u * NW) ? __builtin_nontemporal_load(gptr<uint32_t>((const void*)(base + 4 * NW))) : 0u;
#pragma unroll
  for (int i = 0; i < NW; ++i) w[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}

// bit k of x (k < 4) moved to bit 8k: four 1-bit fields spread to the bytes
__device__ __forceinline__ uint32_t spread4(uint32_t x) { return __umul24(x & 0xFu, 0x00204081u) & 0x01010101u; }

// sum over a word's four bytes b_k of b_k * v[k]
__device__ __forceinline__ float dot4(uint32_t w, const float* v, float acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k) acc = fmaf(ubyte(w, k), v[k], acc);
  return acc;
}

// 16 activations at c0 into v, their sum returned
__device__ __forceinline__ float run16(const XSrc& xs, int c0, float* v) {
  xs.run<16>(c0, v);
  float s = 0.f;
#pragma unroll
  for (int l = 0; l < 16; ++l) s += v[l];
  return s;
}

// ---------------------------------------------------------------- 32-value blocks

// xr[j] = x[j] - x[j+16]/16, xr[16+j] = x[j+16]/16, xr[32] = sum: with the byte
// b = lo + 16 hi of byte j, lo*x[j] + hi*x[j+16] = lo*xr[j] + b*xr[16+j]
__device__ __forceinline__ void load_x_nibble_pairs(const XSrc& xs, int chunk, float* xr) {
  float v[32];
  xs.run<32>(chunk * 32, v);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    xr[j] = v[j] - v[16 + j] * 0.0625f;
    xr[16 + j] = v[16 + j] * 0.0625f;
    s += v[j] + v[16 + j];
  }
  xr[32] = s;
}

// sum of q * x over a block from its 16 nibble bytes (four words)
__device__ __forceinline__ float nibble_pairs_dot(const uint32_t (&q)[4], const float* xr) {
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = opaque(q[i] & 0x0F0F0F0Fu);
    acc = dot4(lo, xr + 4 * i, acc);
    acc = dot4(q[i], xr + 16 + 4 * i, acc);
  }
  return acc;
}

struct BQ4_0 {
  static constexpr int QT = FMT_Q4_0, PER = 32, SIZE = 18, VALS = 32, XR = 33, NW = 5;
  struct Blk {
    uint32_t w[NW];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { load_x_nibble_pairs(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) { load_span<18>(row + 18 * chunk, b.w); }
  __device__ static float dot(const Blk& b, int, const float* xr) {
    const uint32_t q[4] = {__builtin_amdgcn_alignbyte(b.w[1], b.w[0], 2), __builtin_amdgcn_alignbyte(b.w[2], b.w[1], 2),
                           __builtin_amdgcn_alignbyte(b.w[3], b.w[2], 2), __builtin_amdgcn_alignbyte(b.w[4], b.w[3], 2)};
    return gguf_half(b.w[0] & 0xFFFFu) * fmaf(-8.0f, xr[32], nibble_pairs_dot(q, xr));
  }
};

struct BQ4_1 {
  static constexpr int QT = FMT_Q4_1, PER = 32, SIZE = 20, VALS = 32, XR = 33, NW = 5;
  struct Blk {
    uint32_t w[NW];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { load_x_nibble_pairs(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) { load_span<20>(row + 20 * chunk, b.w); }
  __device__ static float dot(const Blk& b, int, const float* xr) {
    const uint32_t q[4] = {b.w[1], b.w[2], b.w[3], b.w[4]};
    return fmaf(gguf_half(b.w[0] & 0xFFFFu), nibble_pairs_dot(q, xr), gguf_half(b.w[0] >> 16) * xr[32]);
  }
};

// Q5_0 / Q5_1: 5-bit values q = nibble | (qh bit << 4), against plain x
__device__ __forceinline__ void load_x_plain32(const XSrc& xs, int chunk, float* xr) {
  xs.run<32>(chunk * 32, xr);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 32; ++j) s += xr[j];
  xr[32] = s;
}

__device__ __forceinline__ float five_bit_dot(const uint32_t (&q)[4], uint32_t qh, const float* xr) {
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (spread4(qh >> (4 * i)) << 4);
    const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (spread4(qh >> (16 + 4 * i)) << 4);
    acc = dot4(lo, xr + 4 * i, acc);
    acc = dot4(hi, xr + 16 + 4 * i, acc);
  }
  return acc;
}

struct BQ5_0 {
  static constexpr int QT = FMT_Q5_0, PER = 32, SIZE = 22, VALS = 32, XR = 33, NW = 6;
  struct Blk {
    uint32_t w[NW];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { load_x_plain32(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) { load_span<22>(row + 22 * chunk, b.w); }
  __device__ static float dot(const Blk& b, int, const float* xr) {
    const uint32_t qh = __builtin_amdgcn_alignbyte(b.w[1], b.w[0], 2);
    const uint32_t q[4] = {__builtin_amdgcn_alignbyte(b.w[2], b.w[1], 2), __builtin_amdgcn_alignbyte(b.w[3], b.w[2], 2),
                           __builtin_amdgcn_alignbyte(b.w[4], b.w[3], 2), __builtin_amdgcn_alignbyte(b.w[5], b.w[4], 2)};
    return gguf_half(b.w[0] & 0xFFFFu) * fmaf(-16.0f, xr[32], five_bit_dot(q, qh, xr));
  }
};

struct BQ5_1 {
  static constexpr int QT = FMT_Q5_1, PER = 32, SIZE = 24, VALS = 32, XR = 33, NW = 6;
  struct Blk {
    uint32_t w[NW];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { load_x_plain32(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) { load_span<24>(row + 24 * chunk, b.w); }
  __device__ static float dot(const Blk& b, int, const float* xr) {
    const uint32_t q[4] = {b.w[2], b.w[3], b.w[4], b.w[5]};
    return fmaf(gguf_half(b.w[0] & 0xFFFFu), five_bit_dot(q, b.w[1], xr), gguf_half(b.w[0] >> 16) * xr[32]);
  }
};

// Q8_0: 34-byte blocks of f16 d and 32 int8. Signed bytes b read as unsigned
// u = b ^ 0x80 = b + 128: sum b*x = sum u*x - 128 * sum x.
struct BQ8_0 {
  static constexpr int QT = FMT_Q8_0, PER = 32, SIZE = 34, VALS = 32, XR = 33, NW = 9;
  struct Blk {
    uint32_t w[NW];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { load_x_plain32(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) { load_span<34>(row + 34 * chunk, b.w); }
  __device__ static float dot(const Blk& b, int, const float* xr) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = dot4(__builtin_amdgcn_alignbyte(b.w[i + 1], b.w[i], 2) ^ 0x80808080u, xr + 4 * i, acc);
    return gguf_half(b.w[0] & 0xFFFFu) * fmaf(-128.0f, xr[32], acc);
  }
};

// ---------------------------------------------------------------- superblocks

// Q2_K / Q3_K / Q6_K chunks: four per superblock, ci = chunk % 4 = 2n + s
// (n the 128-value half, s the 16-byte half of its 32 storage bytes). The
// chunk's values are n*128 + 32t + 16s + l, t = 0..3, l = 0..15: xr[16t + l],
// and xr[64 + t] their sums.
__device__ __forceinline__ void load_x_quarters(const XSrc& xs, int chunk, float* xr) {
  const int c0 = (chunk >> 2) * 256 + ((chunk >> 1) & 1) * 128 + (chunk & 1) * 16;
#pragma unroll
  for (int t = 0; t < 4; ++t) xr[64 + t] = run16(xs, c0 + 32 * t, xr + 16 * t);
}

struct BQ2_K {
  static constexpr int QT = FMT_Q2_K, PER = 256, SIZE = 84, VALS = 64, XR = 68;
  struct Blk {
    uint32_t q[4], sc[2], dd[1];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { load_x_quarters(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) {
    const uint8_t* blk = row + (size_t)(chunk >> 2) * 84;
    const int n = (chunk >> 1) & 1, s = chunk & 1;
    load_span<16>(blk + 16 + 32 * n + 16 * s, b.q);
    load_span<8>(blk + 8 * n, b.sc);
    load_span<4>(blk + 80, b.dd);
  }
  // sum over t of d * sc_t * S_t - dmin * m_t * X_t (moelan/kernels.py:597-632)
  __device__ static float dot(const Blk& b, int chunk, const float* xr) {
    const int s = chunk & 1;
    const float d = gguf_half(b.dd[0] & 0xFFFFu), dmin = gguf_half(b.dd[0] >> 16);
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float S = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) S = dot4((b.q[i] >> (2 * t)) & 0x03030303u, xr + 16 * t + 4 * i, S);
      // scale byte 2t + s of the half's eight
      const uint32_t scb = (b.sc[t >> 1] >> (8 * (2 * (t & 1) + s))) & 0xFFu;
      acc += d * (float)(scb & 15u) * S - dmin * (float)(scb >> 4) * xr[64 + t];
    }
    return acc;
  }
};

struct BQ3_K {
  static constexpr int QT = FMT_Q3_K, PER = 256, SIZE = 110, VALS = 64, XR = 68;
  struct Blk {
    uint32_t q[4], hm[4], sd[4];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { load_x_quarters(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) {
    const uint8_t* blk = row + (size_t)(chunk >> 2) * 110;
    const int n = (chunk >> 1) & 1, s = chunk & 1;
    load_span<16>(blk + 32 + 32 * n + 16 * s, b.q);
    load_span<16>(blk + 16 * s, b.hm);
    load_span<14>(blk + 96, b.sd);
  }
  // scale i of the 16 (moelan/kernels.py:634-641): byte (i & 7)'s low (i < 8) or
  // high nibble, and bits 2 * (i / 4) of byte 8 + i % 4, minus 32
  __device__ static int scale(const Blk& b, int i) {
    const int w = i >> 2, k = i & 3;
    uint32_t lo = (b.sd[w & 1] >> (8 * k)) & 0xFFu;
    lo = w < 2 ? (lo & 15u) : (lo >> 4);
    const uint32_t hi = (b.sd[2] >> (8 * k + 2 * w)) & 3u;
    return (int)(lo | (hi << 4)) - 32;
  }
  __device__ static float dot(const Blk& b, int chunk, const float* xr) {
    const int n = (chunk >> 1) & 1, s = chunk & 1;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float S = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t u = ((b.q[i] >> (2 * t)) & 0x03030303u) | (((b.hm[i] >> (4 * n + t)) & 0x01010101u) << 2);
        S = dot4(u, xr + 16 * t + 4 * i, S);
      }
      acc = fmaf((float)scale(b, 8 * n + 2 * t + s), fmaf(-4.0f, xr[64 + t], S), acc);
    }
    return gguf_half(b.sd[3] & 0xFFFFu) * acc;
  }
};

// Q4_K: eight chunks per superblock (kk = (chunk % 8) / 2 the 64-value group,
// h = chunk % 2 the 16-byte half): nibble bytes 16 + 32kk + 16h + l give values
// 64kk + 16h + l (low) and 64kk + 32 + 16h + l (high);
// d*(sc1*S1 + sc2*S2) - dmin*(m1*X1 + m2*X2) (moelan/kernels.py:499-527)
struct BQ4_K {
  static constexpr int QT = FMT_Q4_K, PER = 256, SIZE = 144, VALS = 32, XR = 34;
  struct Blk {
    uint32_t hdr[4], q[4];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { FmtQ4K::load_x(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) {
    const uint8_t* blk = row + (size_t)(chunk >> 3) * 144;
    load_span<16>(blk, b.hdr);
    load_span<16>(blk + 16 + 16 * (chunk & 7), b.q);
  }
  __device__ static float dot(const Blk& b, int chunk, const float* xr) {
    const int kk = (chunk & 7) >> 1;
    const float d = gguf_half(b.hdr[0] & 0xFFFFu), dmin = gguf_half(b.hdr[0] >> 16);
    const FmtQ4K::HdrBytes sb{b.hdr[1], b.hdr[2], b.hdr[3]};
    int sc1, m1, sc2, m2;
    FmtQ4K::scale_min(2 * kk, sb, sc1, m1);
    FmtQ4K::scale_min(2 * kk + 1, sb, sc2, m2);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s1 = dot4(opaque(b.q[i] & 0x0F0F0F0Fu), xr + 4 * i, s1);
      s2 = dot4(opaque((b.q[i] >> 4) & 0x0F0F0F0Fu), xr + 16 + 4 * i, s2);
    }
    return d * ((float)sc1 * s1 + (float)sc2 * s2) - dmin * ((float)m1 * xr[32] + (float)m2 * xr[33]);
  }
};

// Q5_K: eight chunks per superblock as Q4_K's (kk = (chunk % 8) / 2 the 64-value
// group, h = chunk % 2 the 16-byte half): 16 nibble bytes at 48 + 32kk + 16h give
// values 64kk + 16h + l (low, qh bit 2kk) and 64kk + 32 + 16h + l (high, bit 2kk+1)
// of qh byte 16h + l.
struct BQ5_K {
  static constexpr int QT = FMT_Q5_K, PER = 256, SIZE = 176, VALS = 32, XR = 34;
  struct Blk {
    uint32_t hdr[4], q[4], qh[4];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { FmtQ4K::load_x(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) {
    const uint8_t* blk = row + (size_t)(chunk >> 3) * 176;
    const int kk = (chunk & 7) >> 1, h = chunk & 1;
    load_span<16>(blk, b.hdr);
    load_span<16>(blk + 48 + 32 * kk + 16 * h, b.q);
    load_span<16>(blk + 16 + 16 * h, b.qh);
  }
  __device__ static float dot(const Blk& b, int chunk, const float* xr) {
    const int kk = (chunk & 7) >> 1;
    const float d = gguf_half(b.hdr[0] & 0xFFFFu), dmin = gguf_half(b.hdr[0] >> 16);
    const FmtQ4K::HdrBytes sb{b.hdr[1], b.hdr[2], b.hdr[3]};
    int sc1, m1, sc2, m2;
    FmtQ4K::scale_min(2 * kk, sb, sc1, m1);
    FmtQ4K::scale_min(2 * kk + 1, sb, sc2, m2);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (b.q[i] & 0x0F0F0F0Fu) | (((b.qh[i] >> (2 * kk)) & 0x01010101u) << 4);
      const uint32_t hi = ((b.q[i] >> 4) & 0x0F0F0F0Fu) | (((b.qh[i] >> (2 * kk + 1)) & 0x01010101u) << 4);
      s1 = dot4(lo, xr + 4 * i, s1);
      s2 = dot4(hi, xr + 16 + 4 * i, s2);
    }
    return d * ((float)sc1 * s1 + (float)sc2 * s2) - dmin * ((float)m1 * xr[32] + (float)m2 * xr[33]);
  }
};

// Q6_K: four chunks per superblock, ci = 2n + c: ql bytes 64n + 16c + l and
// 64n + 32 + 16c + l and qh byte 128 + 32n + 16c + l hold values
// n*128 + 16c + l + 32t, t = 0..3, with scale 8n + c + 2t.
struct BQ6_K {
  static constexpr int QT = FMT_Q6_K, PER = 256, SIZE = 210, VALS = 64, XR = 68;
  struct Blk {
    uint32_t qa[4], qc[4], qh[4], sc[2], dd[1];
  };
  __device__ static void load_x(const XSrc& xs, int chunk, float* xr) { load_x_quarters(xs, chunk, xr); }
  __device__ static void load(const uint8_t* row, int chunk, Blk& b) {
    const uint8_t* blk = row + (size_t)(chunk >> 2) * 210;
    const int n = (chunk >> 1) & 1, c = chunk & 1;
    load_span<16>(blk + 64 * n + 16 * c, b.qa);
    load_span<16>(blk + 64 * n + 32 + 16 * c, b.qc);
    load_span<16>(blk + 128 + 32 * n + 16 * c, b.qh);
    load_span<8>(blk + 192 + 8 * n, b.sc);
    load_span<2>(blk + 208, b.dd);
  }
  // d * sum over t of sc_t * (S_t - 32 X_t) (moelan/kernels.py:562-596)
  __device__ static float dot(const Blk& b, int chunk, const float* xr) {
    const int c = chunk & 1;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float S = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t ql = (t & 1) ? b.qc[i] : b.qa[i];
        const uint32_t u = ((ql >> (4 * (t >> 1))) & 0x0F0F0F0Fu) | (((b.qh[i] >> (2 * t)) & 0x03030303u) << 4);
        S = dot4(u, xr + 16 * t + 4 * i, S);
      }
      const int sc = (int)(int8_t)((b.sc[t >> 1] >> (8 * (c + 2 * (t & 1)))) & 0xFFu);
      acc = fmaf((float)sc, fmaf(-32.0f, xr[64 + t], S), acc);
    }
    return gguf_half(b.dd[0] & 0xFFFFu) * acc;
  }
};

// ---------------------------------------------------------------- the mat-vec kernel

// L lanes per row (8..64), CPL chunks per lane; a wave covers 64/L rows a step
// and ng steps. Waves are independent (no barrier). The launch takes chunks
// c0 .. c0+cn of every row (rows longer than L*CPL chunks take several
// launches); acc: add to y instead of writing it. NR input rows share each
// pass over the weights (their activations held together), so a matrix's
// blocks are read once per NR rows. SHARE (NR = 1): the workgroup's 256 lanes
// build each input row's cn chunks once into dynamic LDS ([cn][XR] floats)
// and every wave reads its lanes' chunks from there; every wave then takes
// part in the set-up's barriers, rows or not.
template <class F, int L, int CPL, int NR, bool SHARE>
__global__ __launch_bounds__(256) void mv_blocks_kernel(MVShape sh, MVJob job, int ng, int c0, int cn, int acc) {
  constexpr int RPW = 64 / L;
  const int mat = blockIdx.y;
  int p0 = 0, p1 = job.n;
  if (job.seg) {
    p0 = job.seg[mat];
    p1 = job.seg[mat + 1];
  }
  if (p0 >= p1) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lg = lane / L, lc = lane % L;
  const int row_begin = (blockIdx.x * (blockDim.x >> 6) + wave) * ng * RPW;
  if (!SHARE && row_begin >= sh.O) return;  // the whole wave: no block-level synchronisation below
  const MatRef M = resolve(job, mat);
  int ch[CPL];
  bool on[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    ch[c] = c0 + lc + c * L;
    on[c] = lc + c * L < cn;
  }
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // grid.z splits the input rows: slice z takes batches z, z + gridDim.z, ...
  for (int pb = p0 + (int)blockIdx.z * NR; pb < p1; pb += NR * (int)gridDim.z) {
    float xr[NR][CPL][F::XR];
    if constexpr (SHARE) {
      static_assert(NR == 1, "the shared set-up holds one input row");
      extern __shared__ float xlds[];  // [cn][XR]
      const XSrc xs = make_xsrc(job.x, job.ldx, job.xrow ? job.xrow[pb] : pb, job.half_in);
      for (int ci = (int)threadIdx.x; ci < cn; ci += (int)blockDim.x) {
        float t[F::XR];
        F::load_x(xs, c0 + ci, t);
#pragma unroll
        for (int j = 0; j < F::XR; ++j) xlds[ci * F::XR + j] = t[j];
      }
      __syncthreads();
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int j = 0; j < F::XR; ++j) xr[0][c][j] = on[c] ? xlds[(lc + c * L) * F::XR + j] : 0.f;
      if (row_begin >= sh.O) {  // past the matrix's rows: only the set-up is this wave's
        __syncthreads();
        continue;
      }
    } else {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int p = pb + r < p1 ? pb + r : p1 - 1;  // rows past the end repeat the last (not stored)
        const XSrc xs = make_xsrc(job.x, job.ldx, job.xrow ? job.xrow[p] : p, job.half_in);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          if (on[c]) {
            F::load_x(xs, ch[c], xr[r][c]);
          } else {
#pragma unroll
            for (int j = 0; j < F::XR; ++j) xr[r][c][j] = 0.f;
          }
        }
      }
    }
    typename F::Blk b[2][CPL];
    auto issue = [&](auto buf, int it) {
      constexpr int B = decltype(buf)::value;
      const int o = min(row_begin + it * RPW + lg, sh.O - 1);
      const uint8_t* row = M.w + (size_t)o * sh.row_bytes;
#pragma unroll
      for (int c = 0; c < CPL; ++c)
        if (on[c]) F::load(row, ch[c], b[B][c]);
    };
    auto compute = [&](auto buf, int it) {
      constexpr int B = decltype(buf)::value;
      const int o = row_begin + it * RPW + lg;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float a = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c)
          if (on[c]) a += F::dot(b[B][c], ch[c], xr[r][c]);
        a = lane_group_sum<L>(a);
        if (lc == L - 1 && o < sh.O && pb + r < p1) {
          float* yo = job.y + (size_t)(pb + r) * job.ldy + o;
          *yo = acc ? *yo + a : a;
        }
      }
    };
    issue(B0{}, 0);
    int it = 0;
    for (; it + 2 < ng; it += 2) {
      issue(B1{}, it + 1);
      compute(B0{}, it);
      issue(B0{}, it + 2);
      compute(B1{}, it + 1);
    }
    if (it + 1 < ng) {
      issue(B1{}, it + 1);
      compute(B0{}, it);
      compute(B1{}, it + 1);
    } else {
      compute(B0{}, it);
    }
    if constexpr (SHARE) __syncthreads();  // the next input row's set-up rewrites the LDS
  }
}

// ---------------------------------------------------------------- dequant (bit-exact)

__device__ __forceinline__ uint32_t le16(const uint8_t* p) { return p[0] | ((uint32_t)p[1] << 8); }

// one block / superblock into out, in the reference's f32 operation order
// (separate roundings: no contraction into FMA)
template <int QT>
__device__ void dq_block(const uint8_t* b, float* out) {
  if constexpr (QT == FMT_Q4_0 || QT == FMT_Q4_1) {  // moelan/kernels.py:270-289
    const float d = gguf_half(le16(b));
    const int q0 = QT == FMT_Q4_0 ? 2 : 4;
    for (int j = 0; j < 16; ++j) {
      const int q = b[q0 + j];
      if constexpr (QT == FMT_Q4_0) {
        out[j] = __fmul_rn(d, (float)((q & 15) - 8));
        out[j + 16] = __fmul_rn(d, (float)((q >> 4) - 8));
      } else {
        const float mn = gguf_half(le16(b + 2));
        out[j] = __fadd_rn(__fmul_rn(d, (float)(q & 15)), mn);
        out[j + 16] = __fadd_rn(__fmul_rn(d, (float)(q >> 4)), mn);
      }
    }
  } else if constexpr (QT == FMT_Q5_0 || QT == FMT_Q5_1) {  // :291-308
    constexpr bool with_min = QT == FMT_Q5_1;
    const float d = gguf_half(le16(b));
    const float mn = with_min ? gguf_half(le16(b + 2)) : 0.0f;
    const uint8_t* h = b + (with_min ? 4 : 2);
    const uint32_t qh = h[0] | ((uint32_t)h[1] << 8) | ((uint32_t)h[2] << 16) | ((uint32_t)h[3] << 24);
    const int off = with_min ? 0 : 16;
    for (int j = 0; j < 16; ++j) {
      const uint32_t q = h[4 + j];
      const int x0 = (int)((q & 15u) | (((qh >> j) << 4) & 0x10u)) - off;
      const int x1 = (int)((q >> 4) | ((qh >> (j + 12)) & 0x10u)) - off;
      out[j] = __fadd_rn(__fmul_rn(d, (float)x0), mn);
      out[j + 16] = __fadd_rn(__fmul_rn(d, (float)x1), mn);
    }
  } else if constexpr (QT == FMT_Q2_K) {  // :389-415
    const float d = gguf_half(le16(b + 80)), dmin = gguf_half(le16(b + 82));
    for (int n = 0; n < 2; ++n)
      for (int t = 0; t < 4; ++t)
        for (int s = 0; s < 2; ++s) {
          const uint32_t sc = b[8 * n + 2 * t + s];
          const float dl = __fmul_rn(d, (float)(sc & 15u)), ml = __fmul_rn(dmin, (float)(sc >> 4));
          for (int l = 0; l < 16; ++l) {
            const uint32_t q = (b[16 + 32 * n + 16 * s + l] >> (2 * t)) & 3u;
            out[128 * n + 32 * t + 16 * s + l] = __fsub_rn(__fmul_rn(dl, (float)q), ml);
          }
        }
  } else if constexpr (QT == FMT_Q3_K) {  // :416-454
    const float d = gguf_half(le16(b + 108));
    for (int n = 0; n < 2; ++n)
      for (int t = 0; t < 4; ++t)
        for (int s = 0; s < 2; ++s) {
          const int i = 8 * n + 2 * t + s, w = i >> 2, k = i & 3;
          uint32_t lo = b[96 + (w & 1) * 4 + k];
          lo = w < 2 ? (lo & 15u) : (lo >> 4);
          const int sc = (int)(lo | (((uint32_t)(b[104 + k] >> (2 * w)) & 3u) << 4)) - 32;
          const float dl = __fmul_rn(d, (float)sc);
          for (int l = 0; l < 16; ++l) {
            const int q = (int)((b[32 + 32 * n + 16 * s + l] >> (2 * t)) & 3u);
            const int v = q - ((b[16 * s + l] >> (4 * n + t)) & 1u ? 0 : 4);
            out[128 * n + 32 * t + 16 * s + l] = __fmul_rn(dl, (float)v);
          }
        }
  } else if constexpr (QT == FMT_Q5_K) {  // :338-362
    const float d = gguf_half(le16(b)), dmin = gguf_half(le16(b + 2));
    const FmtQ4K::MemBytes sb{b + 4};
    for (int k = 0; k < 4; ++k) {
      int sc, m;
      FmtQ4K::scale_min(2 * k, sb, sc, m);
      const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)m);
      FmtQ4K::scale_min(2 * k + 1, sb, sc, m);
      const float d2 = __fmul_rn(d, (float)sc), m2 = __fmul_rn(dmin, (float)m);
      for (int l = 0; l < 32; ++l) {
        const uint32_t v = b[48 + 32 * k + l], h = b[16 + l];
        const int lo = (int)(v & 15u) + ((h >> (2 * k)) & 1u ? 16 : 0);
        const int hi = (int)(v >> 4) + ((h >> (2 * k + 1)) & 1u ? 16 : 0);
        out[64 * k + l] = __fsub_rn(__fmul_rn(d1, (float)lo), m1);
        out[64 * k + 32 + l] = __fsub_rn(__fmul_rn(d2, (float)hi), m2);
      }
    }
  } else {  // Q6_K :363-388
    const float d = gguf_half(le16(b + 208));
    for (int n = 0; n < 2; ++n)
      for (int l = 0; l < 32; ++l) {
        const uint32_t a = b[64 * n + l], c = b[64 * n + 32 + l], h = b[128 + 32 * n + l];
        const int q[4] = {(int)((a & 15u) | ((h & 3u) << 4)) - 32, (int)((c & 15u) | (((h >> 2) & 3u) << 4)) - 32,
                          (int)((a >> 4) | (((h >> 4) & 3u) << 4)) - 32, (int)((c >> 4) | (((h >> 6) & 3u) << 4)) - 32};
        for (int t = 0; t < 4; ++t) {
          const int sc = (int)(int8_t)b[192 + 8 * n + l / 16 + 2 * t];
          out[128 * n + l + 32 * t] = __fmul_rn(d, (float)(sc * q[t]));
        }
      }
  }
}

template <class F>
__global__ void dq_blocks_kernel(const uint8_t* raw, int O, int cols, float* out) {
  const int nb = cols / F::PER;
  const long n = (long)O * nb;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const int o = (int)(i / nb), b = (int)(i % nb);
    dq_block<F::QT>(raw + (size_t)o * nb * F::SIZE + (size_t)b * F::SIZE, out + (size_t)o * cols + (size_t)b * F::PER);
  }
}

// ---------------------------------------------------------------- host side

template <class F, int L, int CPL, int NR = 1>
void launch_blocks(const MVShape& sh, const MVJob& job, int nmat, hipStream_t st, int c0 = 0, int cn = -1,
                   int acc = 0, int max_rows = 1) {
  constexpr int RPW = 64 / L;
  const long steps = (long)nmat * ((sh.O + RPW - 1) / RPW);
  int ng = (int)(steps / 2048);  // keep >= ~2048 waves in flight, amortise the activations
  ng = ng < 1 ? 1 : (ng > 16 ? 16 : ng);
  const int wave_rows = ng * RPW;
  const int waves = (sh.O + wave_rows - 1) / wave_rows;
  const int n = cn < 0 ? sh.cpr : cn;
  // One input row a matrix, 32-value kinds: the workgroup's 4 waves share the
  // activation set-up through LDS (the 64-value kinds measured no faster, Q2_K
  // slower, and keep a set-up per wave)
  static const bool share_env = [] {
    const char* e = getenv("MOEHIP_MV_SHARE");  // measurement switch: 0 keeps a set-up per wave
    return !(e && e[0] == '0');
  }();
  if constexpr (NR == 1 && F::XR <= 40) {
    const size_t lds = (size_t)n * F::XR * sizeof(float);
    if (share_env && max_rows == 1 && lds <= 48 * 1024) {
      hipLaunchKernelGGL((mv_blocks_kernel<F, L, CPL, 1, true>), dim3((waves + 3) / 4, nmat, 1), dim3(256), lds, st,
                         sh, job, ng, c0, n, acc);
      return;
    }
  }
  hipLaunchKernelGGL((mv_blocks_kernel<F, L, CPL, NR, false>),
                     dim3((waves + 3) / 4, nmat, row_slices(max_rows, NR, (long)waves * nmat)), dim3(256), 0, st, sh,
                     job, ng, c0, n, acc);
}

// chunks a lane can hold activations for: 4 of the 32-value kinds, 2 of the 64-value
template <class F>
constexpr int max_cpl() {
  return F::XR > 40 ? 2 : 4;
}

// input rows a pass holds: 4 with one chunk of a 32-value kind per lane, 2
// with one 64-value chunk or two 32-value ones, else 1
template <class F, int CPL>
constexpr int rows_per_pass() {
  return F::XR * CPL <= 40 ? 4 : (F::XR * CPL <= 80 ? 2 : 1);
}

template <class F, int L, int CPL>
void launch_rows(const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st, int c0 = 0, int cn = -1,
                 int acc = 0) {
  constexpr int NR = rows_per_pass<F, CPL>();
  if (NR >= 4 && max_rows >= 3) launch_blocks<F, L, CPL, NR>(sh, job, nmat, st, c0, cn, acc, max_rows);
  else if (NR >= 2 && max_rows >= 2)
    launch_blocks<F, L, CPL, (NR >= 2 ? 2 : 1)>(sh, job, nmat, st, c0, cn, acc, max_rows);
  else launch_blocks<F, L, CPL, 1>(sh, job, nmat, st, c0, cn, acc, max_rows);
}

template <class F>
int launch_fmt_blocks(const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st) {
  const int cpr = sh.cpr;
  if (cpr < 1) return set_error(MOE_EUNSUPPORTED, "GGUF mat-vec: rows of %d values", sh.I);
  constexpr int seg = 64 * max_cpl<F>();  // chunks a lane group holds activations for
  if (cpr > seg) {                        // long rows: one launch per segment, the later ones adding
    for (int c0 = 0; c0 < cpr; c0 += seg) {
      launch_rows<F, 64, max_cpl<F>()>(sh, job, nmat, max_rows, st, c0, cpr - c0 < seg ? cpr - c0 : seg, c0 > 0);
      if (int rc = check_launch("GGUF block mat-vec (row segment)")) return rc;
    }
    return MOE_OK;
  }
  if (cpr <= 8) launch_rows<F, 8, 1>(sh, job, nmat, max_rows, st);
  else if (cpr <= 16) launch_rows<F, 16, 1>(sh, job, nmat, max_rows, st);
  else if (cpr <= 32) launch_rows<F, 32, 1>(sh, job, nmat, max_rows, st);
  else if (cpr <= 64) launch_rows<F, 64, 1>(sh, job, nmat, max_rows, st);
  else if (cpr <= 128) launch_rows<F, 64, 2>(sh, job, nmat, max_rows, st);
  else if constexpr (max_cpl<F>() >= 4) launch_rows<F, 64, 4>(sh, job, nmat, max_rows, st);
  return check_launch("GGUF block mat-vec");
}

template <class F>
int launch_dq(const uint8_t* raw, int O, int cols, float* out, hipStream_t st) {
  const long n = (long)O * (cols / F::PER);
  long blocks = (n + 255) / 256;
  blocks = blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks);
  hipLaunchKernelGGL(dq_blocks_kernel<F>, dim3((unsigned)blocks), dim3(256), 0, st, raw, O, cols, out);
  return check_launch("GGUF dequant");
}

}  // namespace

bool block_geometry(int qtype, int* per, int* size, int* vals) {
  switch (qtype) {
#define MOE_GEOM(F) \
  case F::QT:       \
    *per = F::PER;  \
    *size = F::SIZE; \
    *vals = F::VALS; \
    return true;
    MOE_GEOM(BQ8_0)
    MOE_GEOM(BQ4_K)
    MOE_GEOM(BQ4_0)
    MOE_GEOM(BQ4_1)
    MOE_GEOM(BQ5_0)
    MOE_GEOM(BQ5_1)
    MOE_GEOM(BQ2_K)
    MOE_GEOM(BQ3_K)
    MOE_GEOM(BQ5_K)
    MOE_GEOM(BQ6_K)
#undef MOE_GEOM
  }
  return false;
}

int run_matvec_blocks(int qtype, const MVShape& sh, const MVJob& job, int nmat, int max_rows, hipStream_t st) {
  if (nmat <= 0 || sh.O <= 0) return MOE_OK;
  switch (qtype) {
    case FMT_Q8_0: return launch_fmt_blocks<BQ8_0>(sh, job, nmat, max_rows, st);
    case FMT_Q4_K: return launch_fmt_blocks<BQ4_K>(sh, job, nmat, max_rows, st);
    case FMT_Q4_0: return launch_fmt_blocks<BQ4_0>(sh, job, nmat, max_rows, st);
    case FMT_Q4_1: return launch_fmt_blocks<BQ4_1>(sh, job, nmat, max_rows, st);
    case FMT_Q5_0: return launch_fmt_blocks<BQ5_0>(sh, job, nmat, max_rows, st);
    case FMT_Q5_1: return launch_fmt_blocks<BQ5_1>(sh, job, nmat, max_rows, st);
    case FMT_Q2_K: return launch_fmt_blocks<BQ2_K>(sh, job, nmat, max_rows, st);
    case FMT_Q3_K: return launch_fmt_blocks<BQ3_K>(sh, job, nmat, max_rows, st);
    case FMT_Q5_K: return launch_fmt_blocks<BQ5_K>(sh, job, nmat, max_rows, st);
    case FMT_Q6_K: return launch_fmt_blocks<BQ6_K>(sh, job, nmat, max_rows, st);
  }
  return set_error(MOE_EUNSUPPORTED, "GGUF mat-vec: qtype %d", qtype);
}

int run_dequant_blocks(const uint8_t* raw, int qtype, int O, int cols, float* out, hipStream_t st) {
  switch (qtype) {
    case FMT_Q4_0: return launch_dq<BQ4_0>(raw, O, cols, out, st);
    case FMT_Q4_1: return launch_dq<BQ4_1>(raw, O, cols, out, st);
    case FMT_Q5_0: return launch_dq<BQ5_0>(raw, O, cols, out, st);
    case FMT_Q5_1: return launch_dq<BQ5_1>(raw, O, cols, out, st);
    case FMT_Q2_K: return launch_dq<BQ2_K>(raw, O, cols, out, st);
    case FMT_Q3_K: return launch_dq<BQ3_K>(raw, O, cols, out, st);
    case FMT_Q5_K: return launch_dq<BQ5_K>(raw, O, cols, out, st);
    case FMT_Q6_K: return launch_dq<BQ6_K>(raw, O, cols, out, st);
  }
  return set_error(MOE_EUNSUPPORTED, "GGUF dequant: qtype %d (Q8_0 and Q4_K: dequant.hip)", qtype);
}

}  // namespace moe
