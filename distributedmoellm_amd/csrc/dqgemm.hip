// Group-scaled int8 / int4 and GGUF Q8_0 / Q4_K weights times many f32 rows on
// f32 MFMA.
//
// The reference widens a matrix to f32 and uses BLAS once a call has enough
// rows (Packed4 / GroupQuant matmul_t, moelan/experts.py:152, 216-219; from 8
// rows). Here the widening happens in registers: each value becomes
// q * s (int8) or (u - 8) * s (int4) in f32 -- exact, the product of a
// small integer and an f16 or f32 scale (GGUF Q8_0 and Q4_K: the block
// dequant's own f32 operations, so the same values) -- and feeds
// v_mfma_f32_16x16x4_f32
// with f32 rows, f32 accumulation. Nothing is written but y.
//
// Tiles: a workgroup takes 16 weight rows (N) x MT tiles of 16 input rows (M)
// and the whole reduction, its W waves a slice of the 64-column chunks each;
// the slices' sums meet in LDS and are added in wave order (fixed order, no
// atomics). Each widened weight feeds the MT tiles' MFMAs. MFMA step s of chunk c gives lane (r, j) -- r = lane %
// 16 the weight (B) or input (A) row, j = lane / 16 -- column 64 c + 16 j + s,
// so a lane's operands over a chunk are 16 consecutive columns: one 16-byte
// (int8) or 8-byte (int4) load of weights, four float4 of activations, and
// one scale (16 columns never straddle a group: gs is a multiple of 16).
// Rows past the end read the last row and are not stored.
#include "common.h"
#include "dqgemm.h"
#include "formats.h"

#include <cstdlib>
#include <type_traits>

namespace moe {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int WF>
struct WSlice;

template <>
struct WSlice<DQ_INT8> {
  u32x4 v;
  __device__ void load(const uint8_t* w, uint32_t off) { v = *gptr<u32x4>(w + off); }
  // column s of the slice, times its scale
  __device__ float at(int s, float sc, uint32_t) const {
    const uint32_t d = s < 4 ? v.x : (s < 8 ? v.y : (s < 12 ? v.z : v.w));
    return (float)(int8_t)(d >> (8 * (s & 3))) * sc;
  }
  static constexpr uint32_t kBytes = 16;  // a lane's 16 columns
  static constexpr int kCols = 16;
};

template <>
struct WSlice<DQ_INT4> {
  u32x2 v;
  __device__ void load(const uint8_t* w, uint32_t off) { v = *gptr<u32x2>(w + off); }
  // u = the stored nibble ^ its XOR (8 for two's-complement storage); value u - 8
  __device__ float at(int s, float sc, uint32_t xor4) const {
    const uint32_t d = (s < 8 ? v.x : v.y) ^ xor4;
    const int u = (int)((d >> (4 * (s & 7))) & 15u);
    return (float)(u - 8) * sc;
  }
  static constexpr uint32_t kBytes = 8;
  static constexpr int kCols = 16;
};

// GGUF Q8_0: a lane's 32 columns are one block, an f16 d then 32 int8 q at
// byte 34 b of the row (2-byte aligned): the dwords overlapping it, realigned
template <>
struct WSlice<DQ_Q8_0> {
  uint32_t v[9];  // d in the low half of v[0], q from byte 2
  // Rows are whole dwords (K/32 x 34 bytes, K a multiple of 64) from a
  // 4-byte aligned base, so a block starts at 0 or 2 mod 4 and the 9 dwords
  // from the one below it stay in the row: a block at 2 mod 4 ends on a dword
  // boundary, and one at 0 mod 4 is never a row's last block.
  __device__ void load(const uint8_t* w, uint32_t off) {
    const uint32_t sh = off & 3u;
    const uint8_t* base = w + (off - sh);
    uint32_t d[10];
#pragma unroll
    for (int i = 0; i < 9; ++i) d[i] = *gptr<uint32_t>(base + 4 * i);
    d[9] = 0u;  // v[8] needs bytes 32 and 33 of the span only
#pragma unroll
    for (int i = 0; i < 9; ++i) v[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
  }
  __device__ float2 params() const { return make_float2(gguf_half(v[0] & 0xFFFFu), 0.f); }
  __device__ float at(int s, float2 p) const {
    const int b = s + 2;
    return (float)(int8_t)(v[b >> 2] >> (8 * (b & 3))) * p.x;
  }
  static constexpr int kCols = 32;
};

// GGUF Q4_K: a lane's 32 columns are one sub-block j of a 256-value superblock
// (144 bytes: f16 d, f16 dmin, 12 packed 6-bit scale / min bytes, 128 nibble
// bytes; sub-block j = 2 kk + h is nibble h of bytes 16 + 32 kk .. + 32).
// Value (d * sc) * q - dmin * m, rounded as the block dequant rounds it.
template <>
struct WSlice<DQ_Q4_K> {
  u32x4 hdr, q0, q1;
  int j;
  __device__ void load(const uint8_t* w, uint32_t col) {
    const uint32_t sb = col >> 8;
    j = (int)((col >> 5) & 7u);
    const uint8_t* blk = w + sb * 144u;
    hdr = *gptr<u32x4>(blk);
    q0 = *gptr<u32x4>(blk + 16 + 32 * (j >> 1));
    q1 = *gptr<u32x4>(blk + 32 + 32 * (j >> 1));
  }
  __device__ float2 params() const {
    int sc, m;
    FmtQ4K::scale_min(j, FmtQ4K::HdrBytes{hdr.y, hdr.z, hdr.w}, sc, m);
    return make_float2(__fmul_rn(gguf_half(hdr.x & 0xFFFFu), (float)sc), __fmul_rn(gguf_half(hdr.x >> 16), (float)m));
  }
  __device__ float at(int s, float2 p) const {
    const uint32_t wd = s < 16 ? (s < 4 ? q0.x : s < 8 ? q0.y : s < 12 ? q0.z : q0.w)
                               : (s < 20 ? q1.x : s < 24 ? q1.y : s < 28 ? q1.z : q1.w);
    const uint32_t q = (wd >> (8 * (s & 3) + 4 * (j & 1))) & 15u;
    return __fsub_rn(__fmul_rn(p.x, (float)q), p.y);
  }
  static constexpr int kCols = 32;
};

template <int WF, bool SF16, int MT, int W>
__global__ __launch_bounds__(64 * W) void dq_mfma_kernel(DqArgs a) {
  __shared__ f32x4 part[W - 1][MT][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, j = lane >> 4;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16 * MT;
  const int wrow = min(n0 + r, a.O - 1);
  constexpr int SW = WSlice<WF>::kCols, CW = 4 * SW;  // a lane's columns a chunk, a chunk's columns
  const uint32_t rb = WF == DQ_INT8    ? (uint32_t)a.K
                      : WF == DQ_INT4  ? (uint32_t)a.K / 2u
                      : WF == DQ_Q8_0  ? (uint32_t)a.K / 32u * 34u
                                       : (uint32_t)a.K / 256u * 144u;
  const uint32_t G = WF >= DQ_Q8_0 ? 1u : (uint32_t)(a.K / a.gs);
  const uint8_t* w = static_cast<const uint8_t*>(a.w) + (size_t)wrow * rb;
  const float* x[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) x[t] = a.x + (size_t)min(m0 + 16 * t + r, a.n - 1) * a.ldx;
  const int chunks = a.K / CW, gs = a.gs;
  const uint32_t xor4 = a.xor4;
  const void* const sp = a.s;
  const int c0 = wave * chunks / W, c1 = (wave + 1) * chunks / W;
  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  WSlice<WF> ws[2];
  uint32_t sbits[2];
  f32x4 xv[2][MT][SW / 4];
  auto issue = [&](int c, auto bc) {
    constexpr int B = decltype(bc)::value;
    const uint32_t col = (uint32_t)(CW * c + SW * j);
    if constexpr (WF == DQ_Q8_0) {
      ws[B].load(w, col / 32u * 34u);
    } else if constexpr (WF == DQ_Q4_K) {
      ws[B].load(w, col);
    } else {
      ws[B].load(w, col * WSlice<WF>::kBytes / 16u);
      const uint32_t si = (uint32_t)wrow * G + col / (uint32_t)gs;
      sbits[B] = SF16 ? (uint32_t)gptr<uint16_t>(sp)[si] : gptr<uint32_t>(sp)[si];
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < SW / 4; ++q) xv[B][t][q] = *gptr<f32x4>(x[t] + col + 4 * q);
  };
  auto compute = [&](auto bc) {
    constexpr int B = decltype(bc)::value;
    float2 gp = make_float2(0.f, 0.f);
    float sc = 0.f;
    if constexpr (WF >= DQ_Q8_0) gp = ws[B].params();
    else sc = SF16 ? half_bits_to_float(sbits[B]) : __builtin_bit_cast(float, sbits[B]);
#pragma unroll
    for (int s = 0; s < SW; ++s) {
      float wv;  // one widened weight feeds the MT tiles
      if constexpr (WF >= DQ_Q8_0) wv = ws[B].at(s, gp);
      else wv = ws[B].at(s, sc, xor4);
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[B][t][s >> 2][s & 3], wv, acc[t], 0, 0, 0);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  if (c0 < c1) {
    // unconditional issues (the last chunk again past the end) keep one chunk in flight
    issue(c0, I0{});
    int c = c0;
    for (; c + 1 < c1; c += 2) {
      issue(c + 1, I1{});
      compute(I0{});
      issue(min(c + 2, c1 - 1), I0{});
      compute(I1{});
    }
    if (c < c1) compute(I0{});
  }
  // the K slices' sums, added in wave order
  if (wave > 0)
#pragma unroll
    for (int t = 0; t < MT; ++t) part[wave - 1][t][lane] = acc[t];
  __syncthreads();
  if (wave == 0) {
    const int col = n0 + r;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int v = 0; v < W - 1; ++v) acc[t] += part[v][t][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * t + 4 * j + i;
        if (m < a.n && col < a.O) a.y[(size_t)m * a.ldy + col] = acc[t][i];
      }
    }
  }
}

template <int WF, bool SF16>
int launch_dq(const DqArgs& a, hipStream_t st) {
  // M tiles a block (one widened weight feeds them) and waves a block (K
  // slices), as measured on the 256-expert int8 pool at B = 16 / 64: large
  // products share each widened weight over 4 M tiles; small ones (a single
  // expert matrix) are bound by latency and take more, shorter waves
  struct Cfg {
    int mt, w;
  };
  constexpr Cfg cfgs[] = {{4, 4}, {2, 8}, {2, 4}, {1, 16}, {1, 8}, {1, 4}};
  const int chunks = a.K / (4 * WSlice<WF>::kCols), mtiles = (a.n + 15) / 16, ntiles = (a.O + 15) / 16;
  // (GGUF chunks are twice as wide: a small GGUF product wants 16 slices)
  int pick;
  if ((long)ntiles * mtiles >= 4096) pick = mtiles >= 4 ? 0 : (mtiles >= 2 ? 2 : 5);
  else if (WSlice<WF>::kCols == 32) pick = chunks >= 16 ? 3 : (chunks >= 8 ? 4 : 5);
  else pick = mtiles >= 2 ? 2 : (chunks >= 8 ? 4 : 5);
  static const int env = [] {
    const char* e = getenv("MOEHIP_DQ_CFG");  // tuning override: index into cfgs
    const int v = e ? atoi(e) : -1;
    return v >= 0 && v < 6 ? v : -1;
  }();
  if (env >= 0 && cfgs[env].w <= chunks) pick = env;
  const Cfg c = cfgs[pick];
  const dim3 grid(ntiles, (mtiles + c.mt - 1) / c.mt);
  if ((long)grid.y > 65535)
    return set_error(MOE_EUNSUPPORTED, "int8/int4 MFMA product: %d rows (at most %d)", a.n, 65535 * 16);
  switch (c.mt * 100 + c.w) {
    case 404: hipLaunchKernelGGL((dq_mfma_kernel<WF, SF16, 4, 4>), grid, dim3(256), 0, st, a); break;
    case 208: hipLaunchKernelGGL((dq_mfma_kernel<WF, SF16, 2, 8>), grid, dim3(512), 0, st, a); break;
    case 204: hipLaunchKernelGGL((dq_mfma_kernel<WF, SF16, 2, 4>), grid, dim3(256), 0, st, a); break;
    case 116: hipLaunchKernelGGL((dq_mfma_kernel<WF, SF16, 1, 16>), grid, dim3(1024), 0, st, a); break;
    case 108: hipLaunchKernelGGL((dq_mfma_kernel<WF, SF16, 1, 8>), grid, dim3(512), 0, st, a); break;
    default: hipLaunchKernelGGL((dq_mfma_kernel<WF, SF16, 1, 4>), grid, dim3(256), 0, st, a); break;
  }
  return check_launch("int8/int4 MFMA product");
}

}  // namespace

bool dq_mfma_ok(int wf, const DqArgs& a) {
  if (a.ldx % 4 != 0 || !aligned(a.x, 16)) return false;
  if (wf == DQ_Q8_0) return a.K % 128 == 0 && aligned(a.w, 4);
  if (wf == DQ_Q4_K) return a.K % 256 == 0 && aligned(a.w, 16);
  if (a.K % 64 != 0 || a.gs <= 0 || a.gs % 16 != 0 || a.K % a.gs != 0) return false;
  return wf == DQ_INT8 ? aligned(a.w, 16) : aligned(a.w, 8);
}

int run_dq_mfma(int wf, const DqArgs& a, hipStream_t st) {
  if (a.n <= 0 || a.O <= 0) return MOE_OK;
  if (wf == DQ_Q8_0) return launch_dq<DQ_Q8_0, true>(a, st);
  if (wf == DQ_Q4_K) return launch_dq<DQ_Q4_K, true>(a, st);
  if (wf == DQ_INT8) return a.s_f16 ? launch_dq<DQ_INT8, true>(a, st) : launch_dq<DQ_INT8, false>(a, st);
  return a.s_f16 ? launch_dq<DQ_INT4, true>(a, st) : launch_dq<DQ_INT4, false>(a, st);
}

}  // namespace moe
