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

// Partial logits over one K slice: part[z][t][e] = sum over k in slice z of
// x[t, k] * R[e, k], f32; 32x32 tiles, 2x2 outputs per thread, K through LDS.
// Slices are summed in slice order afterwards (deterministic).
__global__ __launch_bounds__(256) void router_logits_kernel(const float* x, int ldx, const float* R, int T, int E, int H,
                                                            int kslice, float* part) {
  __shared__ float xs[32][33];
  __shared__ float rs[32][33];
  const int t0 = blockIdx.x * 32, e0 = blockIdx.y * 32, z = blockIdx.z;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int kb = z * kslice, ke = min(H, kb + kslice);
  float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  for (int k0 = kb; k0 < ke; k0 += 32) {
    for (int i = threadIdx.x; i < 32 * 32; i += 256) {
      const int r = i / 32, kk = i % 32, k = k0 + kk;
      xs[kk][r] = (t0 + r < T && k < ke) ? x[(size_t)(t0 + r) * ldx + k] : 0.f;
      rs[kk][r] = (e0 + r < E && k < ke) ? R[(size_t)(e0 + r) * H + k] : 0.f;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      const float a0 = xs[kk][ty * 2], a1 = xs[kk][ty * 2 + 1];
      const float b0 = rs[kk][tx * 2], b1 = rs[kk][tx * 2 + 1];
      acc[0][0] = fmaf(a0, b0, acc[0][0]);
      acc[0][1] = fmaf(a0, b1, acc[0][1]);
      acc[1][0] = fmaf(a1, b0, acc[1][0]);
      acc[1][1] = fmaf(a1, b1, acc[1][1]);
    }
    __syncthreads();
  }
  float* dst = part + (size_t)z * T * E;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = t0 + ty * 2 + i, e = e0 + tx * 2 + j;
      if (t < T && e < E) dst[(size_t)t * E + e] = acc[i][j];
    }
}

__global__ void sum_slices_kernel(const float* part, int nz, long n, float* out) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    float v = part[i];
    for (int z = 1; z < nz; ++z) v += part[(size_t)z * n + i];
    out[i] = v;
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
__global__ __launch_bounds__(256) void route_kernel(const float* logits, int nz, int T, int E, int k, int normalize,
                                                    int* idx, float* w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* lg = logits + (size_t)t * E;
  float v[4];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    float l = -INFINITY;
    if (e < E) {
      l = lg[e];
      for (int z = 1; z < nz; ++z) l += lg[(size_t)z * T * E + e];  // K slices, in order
    }
    v[j] = l;
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

// A workgroup computes an output tile of one expert: up to 64 of its rows
// (NB = 1 or 2 blocks of 32 = 2 x 16) against 32 weight rows (2 sub-tiles of
// 16); its 4 waves split K: wave w takes the 128-wide K steps w, w+4, ...,
// and the partial tiles are added through LDS in wave order at the end
// (deterministic). There is no barrier in the K loop. Per step a lane reads
// 16 bytes (32 nibbles) of each of its 2 weight rows, widens them to f16 with
// the group scale once, and uses them for every row block: 2 x 4 x NB x 2
// MFMAs. An expert with more rows than one pass holds is done in passes
// (its weight tile is then read again, from L2).
//   MODE_PLAIN / MODE_DOWN: sub-tile s = weight rows n0 + 16 s .. ; y f32
//   MODE_GATE_UP: sub-tile 0 = gate rows j0 .. j0+15, 1 = up rows I + j0 ..;
//                 act = silu(gate) * up as f16, columns in MFMA order
// Activations: f16 rows (8-column groups in MFMA order), or f32 rows of X
// gathered through `rows` and rounded to f16 on load.

template <int MODE, bool SF16, bool ROWS32, int NB>
__device__ __forceinline__ void gemm_body(const GemmArgs& a, const uint8_t* Wt, const void* S, uint32_t xor4, int m0,
                                          int m1, int nbase, f32x4* red) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, ln = lane & 15, q = lane >> 4;
  const int row_bytes = a.K / 2, G = a.K / a.gs;
  int wrow[2];
  bool wok[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (MODE == MODE_GATE_UP) {
      const int j = nbase + ln;
      wok[s] = j < a.I;
      wrow[s] = (s == 0 ? 0 : a.I) + (wok[s] ? j : 0);
    } else {
      const int n = nbase + 16 * s + ln;
      wok[s] = n < a.N;
      wrow[s] = wok[s] ? n : 0;
    }
  }
  const int nsteps = a.K / 128;
  constexpr int RB = 32 * NB;  // rows per pass

  for (int mb = m0; mb < m1; mb += RB) {
    int arow[NB][2];
    bool aok[NB][2];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int m = mb + 32 * b + 16 * h + ln;
        aok[b][h] = m < m1;
        const int mm = aok[b][h] ? m : m0;
        arow[b][h] = ROWS32 ? (a.rows ? a.rows[mm] : mm) : mm;
      }
    f32x4 acc[NB][2][2];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int s = 0; s < 2; ++s) acc[b][h][s] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int st = wave; st < nsteps; st += 4) {
      const int kc = st * 128 + 32 * q;  // this lane's 32-column run
      uint4 braw[2];
      float bsc[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        braw[s] = stream_load16(Wt + (size_t)wrow[s] * row_bytes + kc / 2);
        bsc[s] = gscale<SF16>(S, (size_t)wrow[s] * G + kc / a.gs);
      }
      half8 av[NB][2][4];
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if constexpr (ROWS32) {
            const float4* src = reinterpret_cast<const float4*>(a.X + (size_t)arow[b][h] * a.ldx + kc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float4 lo = src[2 * i], hi = src[2 * i + 1];
              const float c[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
              for (int p = 0; p < 8; ++p) av[b][h][i][p] = (_Float16)c[(p & 1) * 4 + (p >> 1)];
              if (!aok[b][h]) av[b][h][i] = half8{};
            }
          } else {
            const half8* src = reinterpret_cast<const half8*>(a.A + (size_t)arow[b][h] * a.lda + kc);
#pragma unroll
            for (int i = 0; i < 4; ++i) av[b][h][i] = aok[b][h] ? src[i] : half8{};
          }
        }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const __half2 s2 = __float2half2_rn(bsc[s]);
        const uint32_t wd[4] = {braw[s].x ^ xor4, braw[s].y ^ xor4, braw[s].z ^ xor4, braw[s].w ^ xor4};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const half8 bv = widen8(wd[i], s2);
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int h = 0; h < 2; ++h)
              acc[b][h][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[b][h][i], bv, acc[b][h][s], 0, 0, 0);
        }
      }
    }
    // per row block: the waves' partial tiles added in wave order, then stored
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int s = 0; s < 2; ++s) red[((wave * 2 + h) * 2 + s) * 64 + lane] = acc[b][h][s];
      __syncthreads();
      // wave w finishes row half h = w & 1 of sub-tile pair / sub-tile (w >> 1)
      const int h = wave & 1, s = wave >> 1;
      auto sum_red = [&](int ss) {
        f32x4 v = red[((0 * 2 + h) * 2 + ss) * 64 + lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) v += red[((w * 2 + h) * 2 + ss) * 64 + lane];
        return v;
      };
      // D layout: lane holds rows 4q .. 4q+3 of column ln of each 16x16 tile
      if (MODE == MODE_GATE_UP) {
        if (s == 0) {
          const f32x4 g = sum_red(0), u = sum_red(1);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int m = mb + 32 * b + 16 * h + 4 * q + j;
            if (m < m1 && wok[0]) a.act[(size_t)m * a.ldact + perm_pos(nbase + ln)] = (_Float16)(silu(g[j]) * u[j]);
          }
        }
      } else {
        const f32x4 v = sum_red(s);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = mb + 32 * b + 16 * h + 4 * q + j;
          if (m < m1 && wok[s]) a.Y[(size_t)m * a.ldy + nbase + 16 * s + ln] = v[j];
        }
      }
      __syncthreads();  // red is reused by the next block / pass
    }
  }
}

// NBMAX 2: an expert with more than 32 rows is done 64 rows per pass (its
// weight tile read once for up to 64 rows); the others 32 rows per pass.
template <int MODE, bool ROWS32, int NBMAX>
__global__ __launch_bounds__(256) void gemm_q4_kernel(GemmArgs a) {
  __shared__ f32x4 red[4 * 2 * 2 * 64];  // 16 KB: per wave, row half, sub-tile, lane
  // all column tiles of one expert on one XCD: its activation rows stay in that L2
  const int L = xcd_contiguous(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
  const int e = L / gridDim.x, tile = L % gridDim.x;
  const int m0 = a.table ? a.eoff[e] : 0, m1 = a.table ? a.eoff[e + 1] : a.single_rows;
  if (m0 >= m1) return;
  const int per_tile = MODE == MODE_GATE_UP ? 16 : 32;
  const int nbase = tile * per_tile;
  const ExpertDesc d = a.table ? a.table[e] : a.single;
  const uint8_t* Wt = a.which ? d.dn_w : d.gu_w;
  const void* S = a.which ? d.dn_s : d.gu_s;
  const uint32_t xor4 = d.xor8 * 0x01010101u;
  if (NBMAX == 2 && m1 - m0 > 32) {
    if (d.s_f16) gemm_body<MODE, true, ROWS32, 2>(a, Wt, S, xor4, m0, m1, nbase, red);
    else gemm_body<MODE, false, ROWS32, 2>(a, Wt, S, xor4, m0, m1, nbase, red);
  } else {
    if (d.s_f16) gemm_body<MODE, true, ROWS32, 1>(a, Wt, S, xor4, m0, m1, nbase, red);
    else gemm_body<MODE, false, ROWS32, 1>(a, Wt, S, xor4, m0, m1, nbase, red);
  }
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

int router_slices(int T, int E, int H) {
  const long tiles = (long)((T + 31) / 32) * ((E + 31) / 32);
  int nz = (int)((512 + tiles - 1) / tiles);  // ~512 workgroups
  const int maxz = (H + 127) / 128;           // slices of at least 128 columns
  nz = nz < 1 ? 1 : (nz > maxz ? maxz : nz);
  return nz > 16 ? 16 : nz;
}

int run_router_partials(const float* x, int ldx, const float* R, int T, int E, int H, int nz, float* part,
                        hipStream_t st) {
  const int kslice = ((H + nz - 1) / nz + 31) / 32 * 32;
  hipLaunchKernelGGL(router_logits_kernel, dim3((T + 31) / 32, (E + 31) / 32, nz), dim3(256), 0, st, x, ldx, R, T, E,
                     H, kslice, part);
  return check_launch("router logits");
}

int run_router_logits(const float* x, int ldx, const float* R, int T, int E, int H, float* logits, float* scratch,
                      hipStream_t st) {
  const int nz = scratch ? router_slices(T, E, H) : 1;
  int rc = run_router_partials(x, ldx, R, T, E, H, nz, nz > 1 ? scratch : logits, st);
  if (rc || nz == 1) return rc;
  const long n = (long)T * E;
  hipLaunchKernelGGL(sum_slices_kernel, dim3(blocks_for(n)), dim3(256), 0, st, scratch, nz, n, logits);
  return check_launch("router logits (slice sum)");
}

int run_route(const float* logits, int nz, int T, int E, int k, int normalize, int* idx, float* w, hipStream_t st) {
  hipLaunchKernelGGL(route_kernel, dim3((T + 3) / 4), dim3(256), 0, st, logits, nz, T, E, k, normalize, idx, w);
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

int run_gemm(int mode, const GemmArgs& a, int nexp, hipStream_t st, int rows_hint) {
  if (nexp <= 0) return MOE_OK;
  const int per_tile = mode == MODE_GATE_UP ? 16 : 32;
  const int n = mode == MODE_GATE_UP ? a.I : a.N;
  dim3 grid((n + per_tile - 1) / per_tile, nexp);
  // 64-row passes cost occupancy: only when some experts may hold > 32 rows
  const bool two = rows_hint > 16;
  auto go = [&](auto k) { hipLaunchKernelGGL(k, grid, dim3(256), 0, st, a); };
  if (a.rows32) {
    if (mode == MODE_PLAIN) two ? go(gemm_q4_kernel<MODE_PLAIN, true, 2>) : go(gemm_q4_kernel<MODE_PLAIN, true, 1>);
    else if (mode == MODE_GATE_UP)
      two ? go(gemm_q4_kernel<MODE_GATE_UP, true, 2>) : go(gemm_q4_kernel<MODE_GATE_UP, true, 1>);
    else return set_error(MOE_EINVAL, "int4 grouped GEMM: the down product takes f16 activations");
  } else {
    if (mode == MODE_PLAIN) two ? go(gemm_q4_kernel<MODE_PLAIN, false, 2>) : go(gemm_q4_kernel<MODE_PLAIN, false, 1>);
    else if (mode == MODE_GATE_UP)
      two ? go(gemm_q4_kernel<MODE_GATE_UP, false, 2>) : go(gemm_q4_kernel<MODE_GATE_UP, false, 1>);
    else two ? go(gemm_q4_kernel<MODE_DOWN, false, 2>) : go(gemm_q4_kernel<MODE_DOWN, false, 1>);
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
