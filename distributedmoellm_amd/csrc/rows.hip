// Decode GEMM for experts that carry several input rows in one layer call.
//
// The reference decodes each weight row once and multiplies it with every
// row routed to the expert (_q4_rows, moelan/kernels.py:108-131; from 8 rows it
// widens the matrix and uses BLAS, moelan/experts.py:216-219). Here each weight
// row is read from HBM once per pass of up to 4 input rows and multiplied on
// MFMA in exact integer arithmetic:
//  * Weights: a nibble placed in the high half of a byte is the int8 16 v, so a
//    weight dword becomes two int8 words with two masks.
//  * Activations: an input row is scaled by the power of two 2^sigma that puts
//    its largest |x| in [2^29, 2^30), rounded to the integer x_int, and split
//    into four balanced base-256 digits ("limbs") d_0..d_3 in [-128, 127] with
//    x_int = sum d_i 256^i. The 16 rows of an MFMA A operand are 4 input rows x
//    4 limbs (a "quad").
//  * Product: v_mfma_i32_16x16x32_i8 sums the 32 columns of one scale group of
//    limb x 16 v exactly in int32. Lane (j, n) receives the four limbs of input
//    row j of the quad for weight row n and joins them as
//    f32(T0 + 256 T1) + 65536 f32(T2 + 256 T3) (one rounding of each part),
//    then adds that times the group scale in f32.
//  * The row's 2^-sigma / 16 is applied once, when the output is stored.
// Each product term is off by at most 8 * 2^-30 of its input row's largest |x|;
// an input row holding Inf or NaN gives NaN outputs.
//
// Layout of the activation limbs of one quad: [K/64][64 lanes][16 B]; for the
// group pair (2h, 2h+1) and MFMA lane (j, m) the 16 bytes are 8 for group 2h
// then 8 for group 2h+1: input row m/4 of the quad, limb m%4, of columns
// 32g + 8j + {0, 2, 4, 6, 1, 3, 5, 7} (the low nibbles of the weight dword j of
// the group come first, then its high nibbles).
//
// Weight loads: each load instruction reads whole 128-byte lines -- 8 rows x
// the stage's 128 bytes (8 groups), lane (r8, c8) the 16 bytes of group c8 of
// row r8 -- and a pass through the wave's own LDS area leaves dword j of
// group q of row n in register q of lane (j, n), the MFMA B layout. (Lanes
// reading 16-byte halves of lines across 16 rows, transposed with permlanes,
// streamed about a fifth slower.)
// Scale loads: lane (j, n) reads the 8 scales of stage 4b + j of row n, and
// stage 4b + u takes them from lane (u, n) with ds_bpermute (one load per row
// and 4 stages instead of 16 lines per load).
#include <type_traits>
#include <utility>

#include "common.h"
#include "matvec.h"
#include "rows.h"

namespace moe {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kRowsR = 2;            // 16-row blocks of weight rows per wave and row group
constexpr int kGroupRows = 16 * kRowsR;  // weight rows a wave takes per row group
constexpr int kRowsMaxK = 16384;         // longest row the limb kernel holds in registers (8 chunks a thread)

__device__ __forceinline__ u32x4 wload(const uint8_t* p) {
  return __builtin_nontemporal_load(gptr<u32x4>(p));
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace

// ------------------------------------------------------------------ activation limbs

// One block per pair p: its expert m, the expert's first quad (the ceil(n / 4)
// of the experts before it), the row's scale 2^sigma, and its limbs into slot
// i % 4 of quad qbase[m] + i / 4, i = p - poff[m].
//  * The row is loaded once, first, into registers: chunk c of thread t holds
//    columns 8 (t + 256 c) .. 8 (t + 256 c) + 7, NC chunks a thread (K <= 2048 NC).
//  * poff is ascending from poff[0] = 0, so expert e lies wholly before p
//    exactly when poff[e + 1] <= p: m is the count of such experts, poff[m] the
//    sum of their rows and qbase[m] the sum of their quads -- one pass of
//    independent loads in place of a search of dependent ones.
template <int NC, bool V4>
__global__ __launch_bounds__(256) void rows_prep_kernel(const float* x, int ldx, const int* xrow, const int* poff,
                                                        int k, int K, int half, int* qbase, float* fac,
                                                        uint8_t* limbs) {
  __shared__ float red[2][4];
  __shared__ int ired[3][4];
  const int p = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const float* row = x + (size_t)(xrow ? xrow[p] : p) * ldx;
  const int nch = K / 8;
  auto load8 = [&](const float* src, float* d) {
    if constexpr (V4) {
      const f32x4 a = gptr<f32x4>(src)[0], b = gptr<f32x4>(src)[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d[e] = a[e];
        d[4 + e] = b[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = src[e];
    }
  };
  float v[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int cb = t + 256 * c;
    if (cb < nch) {
      load8(row + 8 * cb, v[c]);
      if (half > 0) {
        float u[8];
        load8(row + half + 8 * cb, u);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[c][e] = silu(v[c][e]) * u[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[c][e] = 0.f;
    }
  }
  int m = 0, q = 0, before = 0;
  for (int e = t; e < k; e += 256) {
    const int a = poff[e], b = poff[e + 1];
    if (b <= p) {
      ++m;
      q += (b - a + 3) >> 2;
      before += b - a;
    }
  }
  // the largest |v|; z is 0, or NaN when a value is not finite (fmaxf drops NaN)
  float mx = 0.f, z = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      mx = fmaxf(mx, fabsf(v[c][e]));
      z += v[c][e] - v[c][e];
    }
  mx = wave_max_f(mx);
  z = wave_sum_f(z);
  m = wave_sum_i(m);
  q = wave_sum_i(q);
  before = wave_sum_i(before);
  if (lane == 0) {
    red[0][wv] = mx;
    red[1][wv] = z;
    ired[0][wv] = m;
    ired[1][wv] = q;
    ired[2][wv] = before;
  }
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  z = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  m = (ired[0][0] + ired[0][1]) + (ired[0][2] + ired[0][3]);
  q = (ired[1][0] + ired[1][1]) + (ired[1][2] + ired[1][3]);
  before = (ired[2][0] + ired[2][1]) + (ired[2][2] + ired[2][3]);
  const int i = p - before;
  if (i == 0 && t == 0) qbase[m] = q;
  const int quad = q + (i >> 2), slot = i & 3;
  const int sigma = 30 - (mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) : 0);
  if (t == 0) fac[p] = __builtin_ldexpf(0.0625f, -sigma) + z;
  const int G2 = K / 64;
  uint8_t* blk = limbs + (size_t)quad * G2 * 1024;
  // chunk cb is (group g, K slot j) = (cb / 4, cb % 4): its 8 values go out in
  // the column order 32 g + 8 j + {0, 2, 4, 6, 1, 3, 5, 7}
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int cb = t + 256 * c;
    if (cb >= nch) continue;
    const int g = cb >> 2, j = cb & 3;
    uint32_t u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // |v| 2^sigma < 2^30 for finite values; the clamp keeps Inf and NaN defined
      const float r = fminf(fmaxf(__builtin_rintf(__builtin_ldexpf(v[c][e < 4 ? 2 * e : 2 * (e - 4) + 1], sigma)),
                                  -1073741824.0f),
                            1073741824.0f);
      u[e] = (uint32_t)(int)r + 0x80808080u;  // bytes minus 128 are the balanced digits
    }
#pragma unroll
    for (int L = 0; L < 4; ++L) {
      uint32_t d0 = 0, d1 = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d0 |= ((u[e] >> (8 * L)) & 0xFFu) << (8 * e);
        d1 |= ((u[e + 4] >> (8 * L)) & 0xFFu) << (8 * e);
      }
      const int mrow = 4 * slot + L;
      uint2* dst = reinterpret_cast<uint2*>(blk + ((size_t)(g >> 1) * 64 + (j * 16 + mrow)) * 16 + (g & 1) * 8);
      *dst = make_uint2(d0 ^ 0x80808080u, d1 ^ 0x80808080u);
    }
  }
}

// ------------------------------------------------------------------ the GEMM

// One wave: weight rows [row0, row0 + kGroupRows * ng) of matrix M (O rows, K columns),
// Q quads of input rows (quad q0 + qq, pairs pq + 4 qq + j), all K.
template <int Q, bool SF16>
__device__ __forceinline__ void rows_wave(const MVJob& job, const MatRef& M, int O, int K, int row0, int ng,
                                          const uint8_t* limbs, int q0, int pq, int p1, const float* fac,
                                          uint32_t* tw, u32x4 (*act)[4][64]) {
  static_assert(Q == 1, "the workgroup shares one quad's limbs");
  constexpr int R = kRowsR;
  const int wv = threadIdx.x >> 6;
  constexpr uint32_t SB = SF16 ? 16u : 32u;  // scale bytes of a row per stage
  const int lane = threadIdx.x & 63, n = lane & 15, j = lane >> 4;
  const uint32_t rb = (uint32_t)K / 2, G = (uint32_t)K / 32;
  const int T = K / 256, nstage = ng * T;
  const uint32_t flip = M.xor4 ^ 0x88888888u;  // stored bytes are two's complement nibbles after this XOR
  const uint8_t* const W = M.w;
  const uint8_t* const S = static_cast<const uint8_t*>(M.s);
  const uint8_t* const A = limbs + (size_t)q0 * (K / 64) * 1024 + 16 * lane;

  u32x4 wb[2][R][2], ap[2];
  u32x4 sbn[R][SF16 ? 1 : 2], sbc[R][SF16 ? 1 : 2];
  // the weight row of this lane in row block r of row group rg (rows past O read row O - 1)
  auto wrow = [&](int rg, int r) {
    const int o = row0 + kGroupRows * rg + 16 * r + n;
    return (uint32_t)(o < O ? o : O - 1);
  };
  // whole 128-byte lines: lane (r8, c8) = (lane / 8, lane % 8) reads group c8
  // of the stage (16 bytes) of rows r8 and r8 + 8 of each 16-row block
  const int r8 = lane >> 3, c8 = lane & 7;
  auto lrow = [&](int rg, int r, int h) {
    const int o = row0 + kGroupRows * rg + 16 * r + 8 * h + r8;
    return (uint32_t)(o < O ? o : O - 1);
  };
  // The 4 waves of a workgroup take the same quad: wave wv loads the stage's
  // limb block wv (1 KB) and puts it in the workgroup's LDS slot s % 2; each
  // wave reads all 4 from there after the stage's barrier. The block load is
  // issued first, so that waiting for it leaves the stage's weights in flight.
  auto issue = [&](int s, auto bc, auto uc) {
    constexpr int B = decltype(bc)::value, U = decltype(uc)::value;  // U = s % 4
    const int rg = s / T, t = s - rg * T;
    ap[B] = *gptr<u32x4>(A + ((size_t)(4 * t + wv)) * 1024);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      wb[B][r][0] = wload(W + (lrow(rg, r, 0) * rb + 128u * t + 16u * c8));
      wb[B][r][1] = wload(W + (lrow(rg, r, 1) * rb + 128u * t + 16u * c8));
    }
    if constexpr (U == 0) {  // scales of stages s .. s + 3: stage s + j in lane (j, n)
      const int sj = s + j < nstage ? s + j : nstage - 1;
      const int rgj = sj / T, tj = sj - rgj * T;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint8_t* p = S + (wrow(rgj, r) * (G * (SF16 ? 2u : 4u)) + SB * tj);
#pragma unroll
        for (int h = 0; h < (SF16 ? 1 : 2); ++h) sbn[r][h] = *gptr<u32x4>(p + 16 * h);
      }
    }
  };
  auto put = [&](auto bc) {  // this wave's limb block of the stage in slot B
    constexpr int B = decltype(bc)::value;
    act[B][wv][lane] = ap[B];
  };
  float acc[Q][R];
#pragma unroll
  for (int qq = 0; qq < Q; ++qq)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[qq][r] = 0.f;
  float f[Q];
#pragma unroll
  for (int qq = 0; qq < Q; ++qq) {
    const int p = pq + 4 * qq + j;
    f[qq] = p < p1 ? fac[p] : 0.f;
  }
  auto compute = [&](auto bc, auto uc) {
    constexpr int B = decltype(bc)::value, U = decltype(uc)::value;
    __syncthreads();  // every wave's limb block of this stage is in slot B; slot B ^ 1 is free
    u32x4 ab[Q][4];
#pragma unroll
    for (int h = 0; h < 4; ++h) ab[0][h] = act[B][h][lane];
    put(std::integral_constant<int, B ^ 1>{});  // the next stage's block (issued before this compute)
    if constexpr (U == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int h = 0; h < (SF16 ? 1 : 2); ++h) sbc[r][h] = sbn[r][h];
    }
    const int src = (U * 16 + n) * 4;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // to the MFMA B layout through this wave's LDS area: dword d of group
      // c8 of row m goes to word 36 m + 8 d + c8 (rows 144 bytes apart: the
      // writes of a row's 8 lanes spread over the banks), and lane (n, j)
      // reads words 36 n + 8 j .. + 8: dword j of groups 0..7 of row n
      uint32_t* const area = tw + r * (16 * 36);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int d = 0; d < 4; ++d) area[36 * (r8 + 8 * h) + 8 * d + c8] = wb[B][r][h][d];
      __builtin_amdgcn_wave_barrier();
      const u32x4 w0 = *reinterpret_cast<const u32x4*>(area + 36 * n + 8 * j);
      const u32x4 w1 = *reinterpret_cast<const u32x4*>(area + 36 * n + 8 * j + 4);
      __builtin_amdgcn_wave_barrier();
      const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      uint32_t sw[SF16 ? 4 : 8];
#pragma unroll
      for (int h = 0; h < (SF16 ? 1 : 2); ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) sw[4 * h + e] = __builtin_amdgcn_ds_bpermute(src, sbc[r][h][e]);
#pragma unroll
      for (int qq = 0; qq < Q; ++qq) {
        i32x4 tm[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          const uint32_t wd = w[g] ^ flip;
          const long b = (long)(((uint64_t)(wd & 0xF0F0F0F0u) << 32) | ((wd << 4) & 0xF0F0F0F0u));
          const u32x4 a2 = ab[qq][g >> 1];
          const long a = (g & 1) ? (long)(((uint64_t)a2.w << 32) | a2.z) : (long)(((uint64_t)a2.y << 32) | a2.x);
          tm[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, i32x4{0, 0, 0, 0}, 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          float sc;
          if constexpr (SF16) sc = half_bits_to_float((g & 1) ? (sw[g >> 1] >> 16) : (sw[g >> 1] & 0xFFFFu));
          else sc = __builtin_bit_cast(float, sw[g]);
          const int lo = tm[g][0] + (tm[g][1] << 8), hi = tm[g][2] + (tm[g][3] << 8);
          acc[qq][r] = fmaf(fmaf((float)hi, 65536.0f, (float)lo), sc, acc[qq][r]);
        }
      }
    }
  };
  auto finish = [&](int s) {
    if ((s + 1) % T != 0) return;
    const int rg = s / T;
#pragma unroll
    for (int qq = 0; qq < Q; ++qq) {
      const int p = pq + 4 * qq + j;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int o = row0 + kGroupRows * rg + 16 * r + n;
        if (p < p1 && o < O) job.y[(size_t)p * job.ldy + o] = acc[qq][r] * f[qq];
        acc[qq][r] = 0.f;
      }
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  // every issue is unconditional (past the last stage it loads the last stage
  // again, from L2), so the compiler's wait before a compute leaves the one
  // stage issued after it in flight; a conditional issue makes it wait for all
  const int last = nstage - 1;
  issue(0, I0{}, I0{});
  __syncthreads();  // a previous quad's last stage may still be read from slot 0
  put(I0{});
  for (int s = 0; s < nstage; s += 4) {
    issue(min(s + 1, last), I1{}, I1{});
    compute(I0{}, I0{});
    finish(s);
    if (s + 1 >= nstage) break;
    issue(min(s + 2, last), I0{}, I2{});
    compute(I1{}, I1{});
    finish(s + 1);
    if (s + 2 >= nstage) break;
    issue(min(s + 3, last), I1{}, I3{});
    compute(I0{}, I2{});
    finish(s + 2);
    if (s + 3 >= nstage) break;
    issue(min(s + 4, last), I0{}, I0{});
    compute(I1{}, I3{});
    finish(s + 3);
  }
}

// grid.y = expert of the call, grid.x = (quad of its input rows, group of 4
// waves over its weight rows); each wave takes ng row groups of kGroupRows rows for
// one quad, so the quads of an expert with many rows run side by side
__global__ __launch_bounds__(256) void rows_gemm_kernel(MVJob job, int O, int K, int ng, int tiles,
                                                        const int* qbase, const float* fac, const uint8_t* limbs) {
  __shared__ __attribute__((aligned(16))) uint32_t tw[4][kRowsR * 16 * 36];  // each wave's weight transpose area
  __shared__ u32x4 act[2][4][64];  // the quad's limb blocks of two stages
  const int mat = blockIdx.y;
  const int p0 = job.seg[mat], p1 = job.seg[mat + 1];
  const int quads = gridDim.x / tiles, tile = blockIdx.x % tiles;
  const int wave = tile * 4 + (threadIdx.x >> 6);
  // a wave past the last row still runs the stage loop (its barriers): it
  // reads the last row and stores nothing
  const int row0 = wave * kGroupRows * ng;
  const MatRef M = resolve(job, mat);
  // one quad a wave (two quads a pass held about 230 VGPRs, one wave a SIMD);
  // quads past the grid's (a max_rows below the true count) loop here
  for (int qp = blockIdx.x / tiles; p0 + 4 * qp < p1; qp += quads) {
    const int pq = p0 + 4 * qp;
    if (!aligned(M.w, 16) || !aligned(M.s, 16)) {
      // the 16-byte loads need 16-byte aligned arrays (device allocations are):
      // other arrays give NaN rather than a wrong product
      const int lane = threadIdx.x & 63, pe = min(pq + 4, p1);
      for (int p = pq; p < pe; ++p)
        for (int o = row0 + lane; o < row0 + kGroupRows * ng && o < O; o += 64)
          job.y[(size_t)p * job.ldy + o] = __builtin_nanf("");
      continue;
    }
    const int q = qbase[mat] + qp;
    uint32_t* const area = tw[threadIdx.x >> 6];
    if (M.s_f16) rows_wave<1, true>(job, M, O, K, row0, ng, limbs, q, pq, p1, fac, area, act);
    else rows_wave<1, false>(job, M, O, K, row0, ng, limbs, q, pq, p1, fac, area, act);
  }
}

// ------------------------------------------------------------------ host side

bool rows_gemm_ok(int H, int I, int gs) {
  return gs == 32 && H % 256 == 0 && I % 256 == 0 && H <= kRowsMaxK && I <= kRowsMaxK;
}

RowsSpace rows_layout(void* base, int P, int H, int I) {
  RowsSpace w{};
  size_t off = 0;
  auto take = [&](size_t nb) {
    const size_t o = off;
    off += (nb + 255) / 256 * 256;
    return (char*)base + o;
  };
  // at most one quad a pair (ceil(n / 4) <= n)
  w.qbase = (int*)take((size_t)(P + 1) * 4);
  w.fac = (float*)take((size_t)P * 4);
  w.agu = (uint8_t*)take((size_t)P * (H / 64) * 1024);
  w.adn = (uint8_t*)take((size_t)P * (I / 64) * 1024);
  w.bytes = off;
  return w;
}

size_t rows_workspace(int P, int H, int I) { return rows_layout(nullptr, P, H, I).bytes; }

int run_rows_prep(const float* x, int ldx, const int* xrow, const int* poff, int k, int P, int K, int half,
                  const RowsSpace& ws, uint8_t* limbs, hipStream_t st) {
  if (P <= 0 || k <= 0) return MOE_OK;
  const bool v4 = aligned(x, 16) && ldx % 4 == 0 && half % 4 == 0;
  auto go = [&](auto nc) {
    constexpr int NC = decltype(nc)::value;
    if (v4)
      hipLaunchKernelGGL((rows_prep_kernel<NC, true>), dim3(P), dim3(256), 0, st, x, ldx, xrow, poff, k, K, half,
                         ws.qbase, ws.fac, limbs);
    else
      hipLaunchKernelGGL((rows_prep_kernel<NC, false>), dim3(P), dim3(256), 0, st, x, ldx, xrow, poff, k, K, half,
                         ws.qbase, ws.fac, limbs);
  };
  if (K <= 2048) go(std::integral_constant<int, 1>{});
  else if (K <= 4096) go(std::integral_constant<int, 2>{});
  else if (K <= 8192) go(std::integral_constant<int, 4>{});
  else if (K <= kRowsMaxK) go(std::integral_constant<int, 8>{});
  else return set_error(MOE_EUNSUPPORTED, "multi-row int4 GEMM: rows of %d values", K);
  return check_launch("activation limbs");
}

int run_rows_gemm(const MVJob& job, int k, int O, int K, int max_rows, const RowsSpace& ws, const uint8_t* limbs,
                  hipStream_t st) {
  if (k <= 0 || O <= 0 || max_rows <= 0) return MOE_OK;
  const int groups = (O + kGroupRows - 1) / kGroupRows;  // row groups per matrix
  const int quads = (max_rows + 3) / 4;
  // one row group a wave: most experts have one quad, and a wave streams its
  // rows at a few GB/s, so the work is spread over as many waves as it allows
  const int ng = 1;
  const int tiles = ((groups + ng - 1) / ng + 3) / 4;
  if ((long)tiles * quads > 0x7fffffffL)
    return set_error(MOE_EUNSUPPORTED, "multi-row int4 GEMM: %d rows an expert", max_rows);
  hipLaunchKernelGGL(rows_gemm_kernel, dim3(tiles * quads, k), dim3(256), 0, st, job, O, K, ng, tiles, ws.qbase,
                     ws.fac, limbs);
  return check_launch("multi-row int4 GEMM");
}

}  // namespace moe
