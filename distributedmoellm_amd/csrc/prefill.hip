// Prompt reading (prefill): one MoE layer over T tokens on the device.
//
//   logits = x @ R.T                       (f32)        moelan/model.py:597
//   idx, w = route(logits, k, normalize)                moelan/model.py:154-167
//   groups = group_by_expert(idx, w)                    moelan/model.py:226-236
//   act    = silu(X_e @ GATE_e.T) * (X_e @ UP_e.T)      moelan/experts.py:256-259
//   y      = act @ DOWN_e.T
//   out[t] = sum over t's experts, ascending, of w*y    moelan/experts.py:707-727
//
// The expert products are a grouped GEMM over the expert-sorted rows: int4
// weights are read straight from their packed bytes, widened in registers to
// f16 with their group scale ((u - 8) * s, one f16 rounding), and fed to
// v_mfma_f32_16x16x32_f16 with f32 accumulation. Activations enter as f16
// (written by the gather kernel, and by the gate|up epilogue for the down
// product). f16 operands keep 11 significand bits against bf16's 8 at the same
// MFMA rate; the chained gate|up -> SiLU -> down stays within 2e-3.
//
// K order inside an 8-column group: a dword of 8 nibbles widens to four f16
// pairs holding columns (0,4) (1,5) (2,6) (3,7) (one v_and_or each), so the f16
// activation buffers store every 8 columns in that order: position p holds
// column (p % 2) * 4 + p / 2.
#include "common.h"
#include "matvec.h"
#include "prefill.h"

namespace moe {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__host__ __device__ inline int perm_pos(int c) { return (c & ~7) | (2 * (c & 3) + ((c >> 2) & 1)); }

// ------------------------------------------------------------------ router logits

// logits[t, e] = sum_k x[t, k] * R[e, k], f32; 64x64 tiles, K through LDS.
__global__ __launch_bounds__(256) void router_logits_kernel(const float* x, int ldx, const float* R, int T, int E, int H,
                                                            float* logits) {
  __shared__ float xs[32][65];
  __shared__ float rs[32][65];
  const int t0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  for (int k0 = 0; k0 < H; k0 += 32) {
    for (int i = threadIdx.x; i < 64 * 32; i += 256) {
      const int r = i / 32, kk = i % 32, k = k0 + kk;
      xs[kk][r] = (t0 + r < T && k < H) ? x[(size_t)(t0 + r) * ldx + k] : 0.f;
      rs[kk][r] = (e0 + r < E && k < H) ? R[(size_t)(e0 + r) * H + k] : 0.f;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = xs[kk][ty * 4 + i];
        b[i] = rs[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = t0 + ty * 4 + i, e = e0 + tx * 4 + j;
      if (t < T && e < E) logits[(size_t)t * E + e] = acc[i][j];
    }
}

// ------------------------------------------------------------------ routing

__device__ __forceinline__ void better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// One wave per token: softmax over E <= 256 logits (f32: x - max, exp, / sum),
// k picks by repeated arg-max (ties to the lower expert id, as a stable
// descending sort), then w / sum(w) when normalising.
__global__ __launch_bounds__(256) void route_kernel(const float* logits, int T, int E, int k, int normalize, int* idx,
                                                    float* w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* lg = logits + (size_t)t * E;
  float v[4];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? lg[e] : -INFINITY;
    m = fmaxf(m, v[j]);
  }
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? expf(v[j] - m) : 0.f;
    s += v[j];
  }
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = v[j] / s;  // probabilities, f32
  bool taken[4] = {false, false, false, false};
  float wsum = 0.f, picked = 0.f;
  int mine = -1;  // lane r keeps pick r
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      if (e < E && !taken[j]) better(bv, bi, v[j], e);
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      better(bv, bi, ov, oi);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (lane + 64 * j == bi) taken[j] = true;
    wsum += bv;
    if (lane == r) {
      mine = bi;
      picked = bv;
    }
  }
  if (lane < k) {
    idx[(size_t)t * k + lane] = mine;
    w[(size_t)t * k + lane] = normalize ? picked / wsum : picked;
  }
}

// ------------------------------------------------------------------ grouping

// Stable grouping of the (token, pick) pairs by expert in one workgroup:
// per-expert token bitsets (atomicOr: order-free), per-word prefix counts, a
// scan over experts; a pair's place is its expert's offset plus the number of
// earlier tokens in the bitset. Invalid expert ids are dropped (pos = -1).
__global__ __launch_bounds__(1024) void group_kernel(const int* idx, const float* w, int T, int k, int E, int W,
                                                     int* eoff, int* rows, float* wts, int* pos, int* experts,
                                                     int* offsets, int* n_used) {
  extern __shared__ uint32_t sh[];
  uint32_t* bits = sh;          // [E][W]
  uint32_t* pre = sh + E * W;   // [E][W]
  __shared__ int tot[1025];
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int i = tid; i < E * W; i += nt) bits[i] = 0u;
  __syncthreads();
  const int P = T * k;
  for (int p = tid; p < P; p += nt) {
    const int e = idx[p], t = p / k;
    if (e >= 0 && e < E) atomicOr(&bits[e * W + (t >> 5)], 1u << (t & 31));
  }
  __syncthreads();
  for (int e = tid; e < E; e += nt) {
    int run = 0;
    for (int wd = 0; wd < W; ++wd) {
      pre[e * W + wd] = run;
      run += __popc(bits[e * W + wd]);
    }
    tot[e] = run;
  }
  __syncthreads();
  if (tid == 0) {  // E <= 1024 counts: a serial scan, plus the compact list
    int run = 0, nu = 0;
    for (int e = 0; e < E; ++e) {
      const int c = tot[e];
      eoff[e] = run;
      if (c > 0) {
        experts[nu] = e;
        offsets[nu] = run;
        ++nu;
      }
      run += c;
    }
    eoff[E] = run;
    offsets[nu] = run;
    *n_used = nu;
  }
  __syncthreads();
  for (int p = tid; p < P; p += nt) {
    const int e = idx[p], t = p / k;
    if (e < 0 || e >= E) {
      pos[p] = -1;
      continue;
    }
    const int wd = t >> 5, b = t & 31;
    const int r = pre[e * W + wd] + __popc(bits[e * W + wd] & ((1u << b) - 1u));
    const int q = eoff[e] + r;
    rows[q] = t;
    wts[q] = w[p];
    pos[p] = q;
  }
}

// ------------------------------------------------------------------ gather

// Xs[q, :] = f16(x[rows[q], :]) with each 8 columns in MFMA order.
__global__ void gather_f16_kernel(const float* x, int ldx, const int* rows, int P, int K, _Float16* Xs, int ldxs) {
  const int groups = K / 8;
  const long total = (long)P * groups;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int q = (int)(i / groups), g = (int)(i % groups);
    const float* src = x + (size_t)(rows ? rows[q] : q) * ldx + 8 * g;
    float v[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = src[c];
    half8 h;
#pragma unroll
    for (int p = 0; p < 8; ++p) h[p] = (_Float16)v[(p & 1) * 4 + (p >> 1)];
    *reinterpret_cast<half8*>(Xs + (size_t)q * ldxs + 8 * g) = h;
  }
}

// ------------------------------------------------------------------ grouped GEMM

// 8 nibbles (one dword, columns 0..7 of a 32-column run) -> four f16 pairs
// (0,4) (1,5) (2,6) (3,7), each (u - 8) * s rounded once to f16.
__device__ __forceinline__ half8 widen8(uint32_t w, __half2 s2) {
  const uint32_t m = 0x000F000Fu, magic = 0x64006400u;  // f16 1024 + u
  const __half2 off = __halves2half2(__float2half(1032.f), __float2half(1032.f));
  uint32_t r[4];
  r[0] = (w & m) | magic;
  r[1] = ((w >> 4) & m) | magic;
  r[2] = ((w >> 8) & m) | magic;
  r[3] = ((w >> 12) & m) | magic;
  half8 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    __half2 h = __builtin_bit_cast(__half2, r[i]);
    h = __hmul2(__hsub2(h, off), s2);  // exact (u - 8), then one rounding
    const uint32_t b = __builtin_bit_cast(uint32_t, h);
    out[2 * i] = __builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu));
    out[2 * i + 1] = __builtin_bit_cast(_Float16, (uint16_t)(b >> 16));
  }
  return out;
}

template <bool SF16>
__device__ __forceinline__ float gscale(const void* s, size_t i) {
  if constexpr (SF16) return half_bits_to_float(gptr<uint16_t>(s)[i]);
  else return gptr<float>(s)[i];
}

// One wave: 32 rows (2 x 16) of an expert's token block against 4 weight
// sub-tiles of 16 rows; per 128-wide K step a lane reads 16 bytes (32 nibbles)
// of each weight row and 4 x 16 bytes of each activation row it covers, and
// issues 4 x 2 x 4 MFMAs.
//   MODE_PLAIN / MODE_DOWN: sub-tile s = weight rows n0 + 16 s .. ; y f32
//   MODE_GATE_UP: sub-tiles 0,1 gate rows j0 .. j0+31, 2,3 up rows I + j0 ..;
//                 act = silu(gate) * up as f16, columns in MFMA order
template <int MODE, bool SF16>
__device__ __forceinline__ void gemm_body(const GemmArgs& a, const uint8_t* Wt, const void* S, uint32_t xor4, int m0,
                                          int m1, int nbase) {
  const int lane = threadIdx.x & 63, ln = lane & 15, q = lane >> 4;
  const int row_bytes = a.K / 2, G = a.K / a.gs;
  int wrow[4];
  bool wok[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (MODE == MODE_GATE_UP) {
      const int j = nbase + 16 * (s & 1) + ln;
      wok[s] = j < a.I;
      wrow[s] = (s < 2 ? 0 : a.I) + (wok[s] ? j : 0);
    } else {
      const int n = nbase + 16 * s + ln;
      wok[s] = n < a.N;
      wrow[s] = wok[s] ? n : 0;
    }
  }
  for (int mb = m0; mb < m1; mb += 32) {
    f32x4 acc[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[h][s] = f32x4{0.f, 0.f, 0.f, 0.f};
    int arow[2];
    bool aok[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = mb + 16 * h + ln;
      aok[h] = m < m1;
      arow[h] = aok[h] ? m : m0;
    }
    for (int k0 = 0; k0 < a.K; k0 += 128) {
      const int kc = k0 + 32 * q;  // this lane's 32-column run
      uint4 braw[4];
      float bsc[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        braw[s] = stream_load16(Wt + (size_t)wrow[s] * row_bytes + kc / 2);
        bsc[s] = gscale<SF16>(S, (size_t)wrow[s] * G + kc / a.gs);
      }
      half8 av[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const half8* src = reinterpret_cast<const half8*>(a.A + (size_t)arow[h] * a.lda + kc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          av[h][i] = src[i];
          if (!aok[h]) av[h][i] = half8{};
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const __half2 s2 = __float2half2_rn(bsc[s]);
        const uint32_t wd[4] = {braw[s].x ^ xor4, braw[s].y ^ xor4, braw[s].z ^ xor4, braw[s].w ^ xor4};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const half8 bv = widen8(wd[i], s2);
#pragma unroll
          for (int h = 0; h < 2; ++h) acc[h][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[h][i], bv, acc[h][s], 0, 0, 0);
        }
      }
    }
    // D layout: lane holds rows 4q .. 4q+3 of column ln of each 16x16 tile
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = mb + 16 * h + 4 * q + j;
        if (m >= m1) continue;
        if (MODE == MODE_GATE_UP) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            if (!wok[s]) continue;
            const float g = acc[h][s][j], u = acc[h][s + 2][j];
            const int col = nbase + 16 * s + ln;
            a.act[(size_t)m * a.ldact + perm_pos(col)] = (_Float16)(silu(g) * u);
          }
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s)
            if (wok[s]) a.Y[(size_t)m * a.ldy + nbase + 16 * s + ln] = acc[h][s][j];
        }
      }
  }
}

template <int MODE>
__global__ __launch_bounds__(256) void gemm_q4_kernel(GemmArgs a) {
  const int e = blockIdx.y;
  const int m0 = a.table ? a.eoff[e] : 0, m1 = a.table ? a.eoff[e + 1] : a.single_rows;
  if (m0 >= m1) return;
  const int wave = threadIdx.x >> 6;
  const int per_wave = MODE == MODE_GATE_UP ? 32 : 64;
  const int nbase = (blockIdx.x * 4 + wave) * per_wave;
  if (nbase >= (MODE == MODE_GATE_UP ? a.I : a.N)) return;
  const ExpertDesc d = a.table ? a.table[e] : a.single;
  const uint8_t* Wt = a.which ? d.dn_w : d.gu_w;
  const void* S = a.which ? d.dn_s : d.gu_s;
  const uint32_t xor4 = d.xor8 * 0x01010101u;
  if (d.s_f16) gemm_body<MODE, true>(a, Wt, S, xor4, m0, m1, nbase);
  else gemm_body<MODE, false>(a, Wt, S, xor4, m0, m1, nbase);
}

// ------------------------------------------------------------------ combine

// out[t] = sum over t's picks in ascending expert order (= ascending pair
// position) of w * y[pos]; overwrites out (the layer output starts at zero).
__global__ __launch_bounds__(256) void token_combine_kernel(const float* y, int ldy, const int* pos, const float* wts,
                                                            int k, int H, float* out, int ldo) {
  const int t = blockIdx.y;
  int pp[16];
  int n = 0;
  for (int j = 0; j < k && j < 16; ++j) {
    const int p = pos[(size_t)t * k + j];
    if (p < 0) continue;
    int i = n++;
    while (i > 0 && pp[i - 1] > p) {
      pp[i] = pp[i - 1];
      --i;
    }
    pp[i] = p;
  }
  for (int c = (blockIdx.x * blockDim.x + threadIdx.x) * 4; c < H; c += gridDim.x * blockDim.x * 4) {
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = 0; i < n; ++i) {
      const float w = wts[pp[i]];
      const float* yp = y + (size_t)pp[i] * ldy + c;
      a.x += w * yp[0];
      if (c + 1 < H) a.y += w * yp[1];
      if (c + 2 < H) a.z += w * yp[2];
      if (c + 3 < H) a.w += w * yp[3];
    }
    float* dst = out + (size_t)t * ldo + c;
    dst[0] = a.x;
    if (c + 1 < H) dst[1] = a.y;
    if (c + 2 < H) dst[2] = a.z;
    if (c + 3 < H) dst[3] = a.w;
  }
}

// ------------------------------------------------------------------ host side

static int blocks_for(long n, int per = 256, int cap = 8192) {
  long b = (n + per - 1) / per;
  return (int)(b < 1 ? 1 : (b > cap ? cap : b));
}

int run_router_logits(const float* x, int ldx, const float* R, int T, int E, int H, float* logits, hipStream_t st) {
  hipLaunchKernelGGL(router_logits_kernel, dim3((T + 63) / 64, (E + 63) / 64), dim3(256), 0, st, x, ldx, R, T, E, H,
                     logits);
  return check_launch("router logits");
}

int run_route(const float* logits, int T, int E, int k, int normalize, int* idx, float* w, hipStream_t st) {
  hipLaunchKernelGGL(route_kernel, dim3((T + 3) / 4), dim3(256), 0, st, logits, T, E, k, normalize, idx, w);
  return check_launch("softmax top-k");
}

size_t group_lds_bytes(int T, int E) { return (size_t)2 * E * ((T + 31) / 32) * sizeof(uint32_t); }

int run_group(const int* idx, const float* w, int T, int k, int E, int* eoff, int* rows, float* wts, int* pos,
              int* experts, int* offsets, int* n_used, hipStream_t st) {
  const int W = (T + 31) / 32;
  hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), group_lds_bytes(T, E), st, idx, w, T, k, E, W, eoff, rows, wts,
                     pos, experts, offsets, n_used);
  return check_launch("group by expert");
}

int run_gather_f16(const float* x, int ldx, const int* rows, int P, int K, _Float16* Xs, hipStream_t st) {
  if (P <= 0) return MOE_OK;
  hipLaunchKernelGGL(gather_f16_kernel, dim3(blocks_for((long)P * K / 8)), dim3(256), 0, st, x, ldx, rows, P, K, Xs,
                     K);
  return check_launch("gather rows (f16)");
}

int run_gemm(int mode, const GemmArgs& a, int nexp, hipStream_t st) {
  if (nexp <= 0) return MOE_OK;
  const int per_wave = mode == MODE_GATE_UP ? 32 : 64;
  const int n = mode == MODE_GATE_UP ? a.I : a.N;
  const int waves = (n + per_wave - 1) / per_wave;
  dim3 grid((waves + 3) / 4, nexp);
  switch (mode) {
    case MODE_PLAIN: hipLaunchKernelGGL(gemm_q4_kernel<MODE_PLAIN>, grid, dim3(256), 0, st, a); break;
    case MODE_GATE_UP: hipLaunchKernelGGL(gemm_q4_kernel<MODE_GATE_UP>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(gemm_q4_kernel<MODE_DOWN>, grid, dim3(256), 0, st, a); break;
  }
  return check_launch("int4 grouped GEMM");
}

int run_token_combine(const float* y, int ldy, const int* pos, const float* wts, int T, int k, int H, float* out,
                      int ldo, hipStream_t st) {
  if (T <= 0) return MOE_OK;
  const int gx = (H + 1023) / 1024;
  hipLaunchKernelGGL(token_combine_kernel, dim3(gx, T), dim3(256), 0, st, y, ldy, pos, wts, k, H, out, ldo);
  return check_launch("token combine");
}

}  // namespace moe
