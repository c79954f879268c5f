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

#include <type_traits>

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

// Router logits on the f32 matrix cores: block (t0, e0, z) computes the
// 16 x 16 tile (tokens x experts) of x . R^T over K slice z (kslice columns);
// its W waves take equal parts of the slice and their partial tiles are added
// through LDS in wave order; several slices are summed in slice order by the
// consumer (deterministic). Per 16 columns a lane loads a float4 of its token
// row and of its expert row and feeds them to 4 MFMAs (v_mfma_f32_16x16x4_f32;
// MFMA j takes column 4q + j of each 16, for A and B alike). kslice a multiple
// of 16 W, rows 16-byte aligned. Rows / experts past T / E repeat the last
// one and are not stored.
template <int W, int CH>
__global__ __launch_bounds__(64 * W) void router_mfma_kernel(const float* x, int ldx, const float* R, int T, int E,
                                                             int H, int kslice, float* part) {
  __shared__ f32x4 red[W][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ln = lane & 15, q = lane >> 4;
  // the expert tiles (and slices) of one token tile on one XCD: its rows of x
  // come from HBM once and then from that XCD's L2
  const int L = xcd_contiguous(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z),
                               gridDim.x * gridDim.y * gridDim.z);
  const int z = L % gridDim.z, e0 = (L / gridDim.z) % gridDim.y * 16, t0 = L / (gridDim.z * gridDim.y) * 16;
  const int t = min(t0 + ln, T - 1), e = min(e0 + ln, E - 1);
  const int kw = kslice / W, kb = z * kslice + wave * kw;
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)t * ldx + kb) + q;
  const float4* rr = reinterpret_cast<const float4*>(R + (size_t)e * H + kb) + q;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // chunks of CH x 16 columns (kw is a multiple): all of a chunk's loads first
  for (int k0 = 0; k0 < kw; k0 += 16 * CH) {
    float4 a[CH], b[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      a[j] = xr[(k0 + 16 * j) / 4];
      b[j] = rr[(k0 + 16 * j) / 4];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load of the chunk ahead of its MFMAs
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].x, b[j].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].y, b[j].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].z, b[j].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j].w, b[j].w, acc, 0, 0, 0);
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4 v = red[0][lane];
#pragma unroll
  for (int w = 1; w < W; ++w) v += red[w][lane];
  float* dst = part + (size_t)z * T * E;
  // D layout: lane (ln, q) holds tokens 4q .. 4q+3 of expert column ln
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tt = t0 + 4 * q + j, ee = e0 + ln;
    if (tt < T && ee < E) dst[(size_t)tt * E + ee] = v[j];
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

// one step of a DPP reduction: the (value, index) of the lane CTRL names, or
// (sv, si) where that lane is out of the row (the lanes ROWMASK leaves out keep
// (sv, si) too)
template <int CTRL, int ROWMASK>
__device__ __forceinline__ void dpp_better(float& v, int& i, float sv, int si) {
  const float ov = __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, sv), __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xf, false));
  const int oi = __builtin_amdgcn_update_dpp(si, i, CTRL, ROWMASK, 0xf, false);
  better(v, i, ov, oi);
}

// the wave's best (value, index) -- larger value, then lower index -- in every
// lane: DPP row shifts and broadcasts into lane 63, then read out of it
__device__ __forceinline__ void wave_best(float& v, int& i) {
  const float sv = -INFINITY;
  const int si = 0x7fffffff;
  dpp_better<0x111, 0xf>(v, i, sv, si);  // row_shr:1
  dpp_better<0x112, 0xf>(v, i, sv, si);  // row_shr:2
  dpp_better<0x114, 0xf>(v, i, sv, si);  // row_shr:4
  dpp_better<0x118, 0xf>(v, i, sv, si);  // row_shr:8
  dpp_better<0x142, 0xa>(v, i, sv, si);  // row_bcast:15 into rows 1, 3
  dpp_better<0x143, 0xc>(v, i, sv, si);  // row_bcast:31 into rows 2, 3
  v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
  i = __builtin_amdgcn_readlane(i, 63);
}

// numpy's pairwise float32 sum of a[0..n) (the order of w.sum(-1) in the
// reference's route): fewer than 8 values in sequence; up to 128 in 8 strided
// partial sums, combined as ((0+1)+(2+3))+((4+5)+(6+7)), then the tail; longer
// runs split at half (rounded down to a multiple of 8) and the halves added.
// Explicit stack: eval entries push a value, combine entries add the last two.
__device__ float pairwise_leaf(const float* a, int n) {
  if (n < 8) {
    float r = 0.f;
    for (int i = 0; i < n; ++i) r += a[i];
    return r;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = a[j];
  int i = 8;
  for (; i < n - n % 8; i += 8)
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] += a[i + j];
  float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res += a[i];
  return res;
}

__device__ __noinline__ float pairwise_sum(const float* a, int n) {
  int todo_off[64], todo_n[64];  // n < 0: combine
  float val[32];
  int nt = 0, nv = 0;
  todo_off[nt] = 0;
  todo_n[nt++] = n;
  while (nt > 0) {
    --nt;
    const int o = todo_off[nt], m = todo_n[nt];
    if (m < 0) {
      const float r = val[--nv];
      val[nv - 1] = val[nv - 1] + r;
    } else if (m <= 128) {
      val[nv++] = pairwise_leaf(a + o, m);
    } else {
      int h = m / 2;
      h -= h % 8;
      todo_n[nt++] = -1;  // runs after both halves
      todo_off[nt] = o + h;
      todo_n[nt++] = m - h;
      todo_off[nt] = o;
      todo_n[nt++] = h;  // left half first
    }
  }
  return val[0];
}

// Order of the picks: larger probability first, then lower expert id (a
// stable descending argsort); a NaN probability sorts after every number, as
// numpy's argsort puts NaN last. key = p, or -1 for NaN (p >= 0 otherwise).
__device__ __forceinline__ float pick_key(float p) { return p == p ? p : -1.f; }

// ------------------------------------------------------------------ gather

// 2^(t - e) for m = f * 2^e, f in [0.5, 1): m times it lands in [2^(t-1), 2^t);
// 1 for m = 0 or non-finite m
__device__ __forceinline__ float pow2_into(float m, int t) {
  if (!(m > 0.f && m < INFINITY)) return 1.f;
  return ldexpf(1.f, t - __builtin_amdgcn_frexp_expf(m));
}

// One wave's f16 copy of a row of K floats: dst = f16(src * 2^a) with each 8
// columns in MFMA order, the power chosen from the row's largest |value| (so no
// value overflows f16); *fac = 2^-a. Up to 2048 values stay in registers
// between the load (issued early, so its latency overlaps other work) and the
// store; longer rows read their tail twice.
struct HeldRow {
  static constexpr int kHeld = 4;  // 8-column groups a lane holds
  float4 v[kHeld][2];

  __device__ __forceinline__ void load(const float* src, int K, int lane) {
#pragma unroll
    for (int k = 0; k < kHeld; ++k) {
      const int c = 8 * lane + 512 * k;
      if (c < K) {
        v[k][0] = *reinterpret_cast<const float4*>(src + c);
        v[k][1] = *reinterpret_cast<const float4*>(src + c + 4);
      }
    }
  }

  __device__ __forceinline__ void store_f16(const float* src, int K, _Float16* dst, float* fac, int lane) const {
    float m = 0.f;
#pragma unroll
    for (int k = 0; k < kHeld; ++k) {
      if (8 * lane + 512 * k < K) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
          m = fmaxf(m, fmaxf(fmaxf(fabsf(v[k][h].x), fabsf(v[k][h].y)), fmaxf(fabsf(v[k][h].z), fabsf(v[k][h].w))));
      }
    }
    for (int c = 8 * lane + 512 * kHeld; c < K; c += 512) {
      const float4 lo = *reinterpret_cast<const float4*>(src + c), hi = *reinterpret_cast<const float4*>(src + c + 4);
      m = fmaxf(m, fmaxf(fmaxf(fmaxf(fabsf(lo.x), fabsf(lo.y)), fmaxf(fabsf(lo.z), fabsf(lo.w))),
                         fmaxf(fmaxf(fabsf(hi.x), fabsf(hi.y)), fmaxf(fabsf(hi.z), fabsf(hi.w)))));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const float f = pow2_into(m, 14);
    auto put = [&](int c, float4 lo, float4 hi) {
      const float w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      half8 h;
#pragma unroll
      for (int p = 0; p < 8; ++p) h[p] = (_Float16)(w[(p & 1) * 4 + (p >> 1)] * f);
      *reinterpret_cast<half8*>(dst + c) = h;
    };
#pragma unroll
    for (int k = 0; k < kHeld; ++k) {
      const int c = 8 * lane + 512 * k;
      if (c < K) put(c, v[k][0], v[k][1]);
    }
    for (int c = 8 * lane + 512 * kHeld; c < K; c += 512)
      put(c, *reinterpret_cast<const float4*>(src + c), *reinterpret_cast<const float4*>(src + c + 4));
    if (lane == 0) *fac = 1.f / f;
  }
};

// Xs[q, :] = the f16 copy of x[rows[q], :], fac[q] its factor. One wave a row.
__global__ __launch_bounds__(256) void gather_f16_kernel(const float* x, int ldx, const int* rows, int P, int K,
                                                         _Float16* Xs, int ldxs, float* fac) {
  const int q = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (q >= P) return;
  const float* src = x + (size_t)(rows ? rows[q] : q) * ldx;
  HeldRow row;
  row.load(src, K, lane);
  row.store_f16(src, K, Xs + (size_t)q * ldxs, fac + q, lane);
}

// One wave per token: softmax over the E logits (f32: x - max, exp, / sum),
// then k picks, each the best (key, id) after the previous pick in that order
// (no per-expert state, so E and k are not bounded), then w / sum(w) when
// normalising, the sum in the reference's order. J > 0: the probabilities of
// E <= 64 J experts stay in registers; J = 0: they are recomputed from the
// logits in each pick round (the same operations, so the same values).
// Picks r < 64 are kept by lane r and written together; with k > 64 lane 0
// writes every pick as it is found and normalises them afterwards, reading
// back its own writes.
template <int J>
__global__ __launch_bounds__(256) void route_kernel(const float* logits, int nz, int T, int E, int k, int normalize,
                                                    int* idx, float* w, const float* x, int ldx, int H, _Float16* xs,
                                                    float* xf) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  // xs: the token's row also goes out as its f16 copy (as gather_f16_kernel),
  // loaded first so that its latency overlaps the routing
  HeldRow row;
  if (xs) row.load(x + (size_t)t * ldx, H, lane);
  const float* lg = logits + (size_t)t * E;
  auto logit = [&](int e) {
    float l = lg[e];
    for (int z = 1; z < nz; ++z) l += lg[(size_t)z * T * E + e];  // K slices, in order
    return l;
  };
  constexpr int JR = J > 0 ? J : 1;
  float v[JR];
  float m = -INFINITY;
  if constexpr (J > 0) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e = lane + 64 * j;
      v[j] = e < E ? logit(e) : -INFINITY;
      m = fmaxf(m, v[j]);
    }
  } else {
    for (int e = lane; e < E; e += 64) m = fmaxf(m, logit(e));
  }
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  float s = 0.f;
  if constexpr (J > 0) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int e = lane + 64 * j;
      v[j] = e < E ? expf(v[j] - m) : 0.f;
      s += v[j];
    }
  } else {
    for (int e = lane; e < E; e += 64) s += expf(logit(e) - m);
  }
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if constexpr (J > 0) {
#pragma unroll
    for (int j = 0; j < J; ++j) v[j] = v[j] / s;  // probabilities, f32
  }
  // numpy's pairwise order for k <= 128, accumulated as the picks come:
  // acc[0] takes pick r < k - k % 8 and the eight rotate (8 steps restore them)
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  const int nb = k < 8 ? 0 : k - k % 8;
  float pk = INFINITY;  // the previous pick: key, id
  int pi = -1;
  float picked = 0.f;
  int mine = -1;
  for (int r = 0; r < k; ++r) {
    float bk = -INFINITY;
    int bi = 0x7fffffff;
    auto consider = [&](float p, int e) {
      const float key = pick_key(p);
      if (key < pk || (key == pk && e > pi)) better(bk, bi, key, e);
    };
    if constexpr (J > 0) {
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int e = lane + 64 * j;
        if (e < E) consider(v[j], e);
      }
    } else {
      for (int e = lane; e < E; e += 64) consider(expf(logit(e) - m) / s, e);
    }
    wave_best(bk, bi);
    pk = bk;
    pi = bi;
    const float p = bk < 0.f ? __builtin_nanf("") : bk;
    if (r < nb) {
      acc[0] += p;
      const float a0 = acc[0];
#pragma unroll
      for (int j = 0; j < 7; ++j) acc[j] = acc[j + 1];
      acc[7] = a0;
      if (r == nb - 1) wsum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    } else {
      wsum += p;
    }
    if (k <= 64) {
      if (lane == r) {
        mine = bi;
        picked = p;
      }
    } else if (lane == 0) {
      idx[(size_t)t * k + r] = bi;
      w[(size_t)t * k + r] = p;
    }
  }
  if (k <= 64) {
    if (lane < k) {
      idx[(size_t)t * k + lane] = mine;
      w[(size_t)t * k + lane] = normalize ? picked / wsum : picked;
    }
  } else if (normalize && lane == 0) {
    float* wt = w + (size_t)t * k;
    if (k > 128) wsum = pairwise_sum(wt, k);
    for (int r = 0; r < k; ++r) wt[r] = wt[r] / wsum;
  }
  if (xs) row.store_f16(x + (size_t)t * ldx, H, xs + (size_t)t * H, xf + t, lane);
}

// ------------------------------------------------------------------ grouping

// Stable grouping of the P = T*k picks by expert, one block per expert: a
// pick's place is its expert's offset (the number of picks of lower expert
// ids) plus the number of earlier picks of the same expert -- exactly
// argsort(idx.ravel(), kind="stable"). The block stages the pick ids and
// weights in LDS in chunks; its 4 waves take quarters of each chunk, count
// (per lane, then summed), add the earlier quarters' counts (LDS, in order)
// and write the places in pick order with ballots. Invalid expert ids are
// dropped (pos = -1, written by the block of expert 0).
constexpr int kGroupChunk = 4096;  // picks staged at once (ids and weights: 32 KB)

__global__ __launch_bounds__(256) void group_kernel(const int* idx, const float* w, int P, int k, int E, int* eoff,
                                                    int* rows, float* wts, int* pos) {
  __shared__ int ids[kGroupChunk];
  __shared__ float wv[kGroupChunk];
  __shared__ int cnt[2][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x;
  const uint64_t below = (1ull << lane) - 1ull;
  // chunk c0 .. c0+n into LDS, padded with id -1 up to a multiple of 1024; each
  // thread's loads are issued together (16 picks per thread)
  auto stage = [&](int c0, int n) {
    __syncthreads();
    int iv[16];
    float fv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int i = threadIdx.x + 256 * j, p = c0 + i;
      const bool in = i < n;
      iv[j] = in ? idx[p] : -1;
      fv[j] = in ? w[p] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      ids[threadIdx.x + 256 * j] = iv[j];
      wv[threadIdx.x + 256 * j] = fv[j];
    }
    __syncthreads();
  };
  // wave quarters of a chunk of n picks: [wave * q, (wave + 1) * q), q a multiple of 64
  auto quarter = [&](int n) { return ((n + 255) / 256) * 64; };
  // pass 1: per-wave counts of lower ids and of e over all chunks
  int lt = 0, eq = 0;
  for (int c0 = 0; c0 < P; c0 += kGroupChunk) {
    const int n = min(kGroupChunk, P - c0), qn = quarter(n);
    stage(c0, n);
    for (int i0 = wave * qn; i0 < (wave + 1) * qn; i0 += 64) {
      const int id = ids[i0 + lane];
      lt += (id >= 0 && id < e) ? 1 : 0;
      eq += id == e ? 1 : 0;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    lt += __shfl_xor(lt, off, 64);
    eq += __shfl_xor(eq, off, 64);
  }
  if (lane == 0) {
    cnt[0][wave] = lt;
    cnt[1][wave] = eq;
  }
  __syncthreads();
  const int below_e = cnt[0][0] + cnt[0][1] + cnt[0][2] + cnt[0][3];
  if (threadIdx.x == 0) {
    eoff[e] = below_e;
    if (e == E - 1) eoff[E] = below_e + cnt[1][0] + cnt[1][1] + cnt[1][2] + cnt[1][3];
  }
  // pass 2: places in pick order. Within a chunk, wave w starts after the
  // earlier waves' picks of e in that chunk: counted again per chunk
  int run = below_e;
  for (int c0 = 0; c0 < P; c0 += kGroupChunk) {
    const int n = min(kGroupChunk, P - c0), qn = quarter(n);
    if (P > kGroupChunk) stage(c0, n);  // one chunk: still in LDS
    int mine_n = 0;
    for (int i0 = wave * qn; i0 < (wave + 1) * qn; i0 += 64) mine_n += ids[i0 + lane] == e ? 1 : 0;
    for (int off = 32; off > 0; off >>= 1) mine_n += __shfl_xor(mine_n, off, 64);
    __syncthreads();
    if (lane == 0) cnt[1][wave] = mine_n;
    __syncthreads();
    int r = run;
    for (int v = 0; v < wave; ++v) r += cnt[1][v];
    for (int i0 = wave * qn; i0 < (wave + 1) * qn; i0 += 64) {
      const int i = i0 + lane, p = c0 + i;
      const int id = ids[i];
      const bool mine = id == e;
      const uint64_t m = __ballot(mine);
      if (mine) {
        const int q = r + __popcll(m & below);
        rows[q] = p / k;
        wts[q] = wv[i];
        pos[p] = q;
      }
      if (e == 0 && i < n && (id < 0 || id >= E)) pos[p] = -1;
      r += __popcll(m);
    }
    run += cnt[1][0] + cnt[1][1] + cnt[1][2] + cnt[1][3];
  }
}

// The experts that received picks, ascending, with their ranges: one block
// walks the experts 1024 at a time, carrying the count so far.
__global__ __launch_bounds__(1024) void used_experts_kernel(const int* eoff, int E, int* experts, int* offsets,
                                                            int* n_used) {
  __shared__ int wave_used[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int base = 0;
  for (int e0 = 0; e0 < E; e0 += 1024) {
    const int e = e0 + threadIdx.x;
    const bool used = e < E && eoff[e + 1] > eoff[e];
    const uint64_t m = __ballot(used);
    if (lane == 0) wave_used[wave] = __popcll(m);
    __syncthreads();
    int before = base, all = base;
    for (int i = 0; i < 16; ++i) {
      before += i < wave ? wave_used[i] : 0;
      all += wave_used[i];
    }
    if (used) {
      const int slot = before + __popcll(m & ((1ull << lane) - 1ull));
      experts[slot] = e;
      offsets[slot] = eoff[e];
    }
    base = all;
    __syncthreads();  // wave_used is rewritten by the next round
  }
  if (threadIdx.x == 0) {
    *n_used = base;
    offsets[base] = eoff[E];
  }
}

// ------------------------------------------------------------------ grouped GEMM

// 8 nibbles (one dword, columns 0..7 of a 32-column run) -> four f16 pairs
// (0,4) (1,5) (2,6) (3,7), each (u - 8) * s rounded once to f16. A nibble in
// bits 0..3 of a half under exponent 2^10 (0x6400) reads 1024 + u; one in bits
// 4..7 under exponent 2^6 (0x5400, mantissa unit 1/16) reads 64 + u, so one
// shift serves all four pairs. c0 / c1 = (xor & mask) | exponent: the XOR that
// turns stored nibbles v into u = v + 8 rides along with the exponent bits.
__device__ __forceinline__ uint32_t widen_c0(uint32_t xor4) { return (xor4 & 0x000F000Fu) | 0x64006400u; }
__device__ __forceinline__ uint32_t widen_c1(uint32_t xor4) { return (xor4 & 0x00F000F0u) | 0x54005400u; }

__device__ __forceinline__ half8 widen8(uint32_t w, __half2 s2, uint32_t c0, uint32_t c1) {
  const uint32_t w8 = w >> 8;
  const uint32_t r[4] = {(w & 0x000F000Fu) ^ c0, (w & 0x00F000F0u) ^ c1, (w8 & 0x000F000Fu) ^ c0,
                         (w8 & 0x00F000F0u) ^ c1};
  const __half2 off_lo = __halves2half2(__float2half(1032.f), __float2half(1032.f));
  const __half2 off_hi = __halves2half2(__float2half(72.f), __float2half(72.f));
  half8 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    __half2 h = __builtin_bit_cast(__half2, r[i]);
    h = __hmul2(__hsub2(h, (i & 1) ? off_hi : off_lo), s2);  // exact (u - 8), then one rounding
    const uint32_t bits = __builtin_bit_cast(uint32_t, h);
    out[2 * i] = __builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
    out[2 * i + 1] = __builtin_bit_cast(_Float16, (uint16_t)(bits >> 16));
  }
  return out;
}

// A workgroup computes the output tile of one expert for up to 64 of its rows
// and 128 weight rows: wave w owns weight rows 32w .. 32w+31 of the tile as
// two 16-row sub-tiles.
//   MODE_PLAIN / MODE_DOWN: sub-tile s = weight rows n0 + 32w + 16s ..; y f32
//   MODE_GATE_UP: sub-tile 0 = gate rows j0 + 16w .., 1 = the up rows I + j0 +
//                 16w ..; act = silu(gate) * up as f16, columns in MFMA order
// K advances in steps of 128 columns.
//  * Activations: the step's tile (16 RT rows x 128 f16) is staged in LDS once
//    and read by all four waves (double buffered, one barrier per step, loaded
//    two steps ahead; 16 threads read one row's 256 contiguous bytes). RT, the
//    row tiles of the pass, is a compile-time constant of the pass's code, so
//    the MFMAs of rows the pass does not have are not issued.
//  * Weights: a wave reads its 32 rows a pair of steps at a time, 128 bytes
//    (a cache line) per row, 8 rows per instruction -- the pattern HBM serves
//    at full rate -- two pairs ahead, and passes them through a wave-private
//    LDS area to the MFMA operand layout. Each lane's 16 bytes (32 nibbles)
//    of a row per step are widened to f16 with the group scale once and fed
//    to every row tile: 2 x 4 x RT MFMAs per step.
// A pass's last row tile may hold rows past the expert's last row: they
// repeat its last row and are not stored. An expert with more than 64 rows
// (32 for f32 rows) is done in passes (its weight tile read again).
// Activations: f16 rows (8-column groups in MFMA order), or f32 rows of X
// gathered through `rows` and rounded to f16 when staged.
// Range: every f16 activation is its value times a power of two, undone on
// the f32 sums in the epilogue, so no activation overflows f16 where f32
// stays finite:
//   GATE_UP: per row, chosen by the gather from the row's largest |value|;
//   DOWN: silu(gate) * up is written per row and 16 columns with the power
//         that puts the piece's largest |value| in [2^13, 2^14); staging
//         brings every piece of a row to its largest piece's power;
//   PLAIN (f32 rows): per row, chosen when the pass starts.
// Weights are (u - 8) * s rounded once to f16: scales above 8188 overflow and
// scales below 2^-14 / 8 lose precision (f16 subnormals); int4 group scales
// are far inside that range.

constexpr int kGK = 128;                   // K per step
constexpr int kGRows = 48;                 // expert rows per pass (f16 activations)
constexpr int kARow = kGK * 2 + 16;        // LDS bytes per activation row (16 B of padding: conflict-free)
constexpr int kABuf = kGRows * kARow;      // one step's activation tile
constexpr int kBRow = 128 + 16;            // LDS bytes per weight row of a pair of steps (padded)
constexpr int kBWave = 32 * kBRow;         // a wave's weight rows
constexpr int kSRow = 144;                 // LDS bytes per row of a wave's scale window (16-byte aligned)
constexpr int kSWave = 32 * kSRow;         // a wave's scale rows
constexpr int kFacOff = 2 * kABuf + 4 * kBWave + 4 * kSWave;  // per row of the pass: the factor undoing its scaling
constexpr int kGemmLds = kFacOff + kGRows * 4;

template <bool SF16>
__device__ __forceinline__ uint32_t gscale_bits(const void* s, uint32_t i) {
  if constexpr (SF16) return gptr<uint16_t>(s)[i];
  else return gptr<uint32_t>(s)[i];
}

template <bool SF16>
__device__ __forceinline__ float gscale_value(uint32_t bits) {
  if constexpr (SF16) return half_bits_to_float(bits);
  else return __builtin_bit_cast(float, bits);
}

template <int N>
using IC = std::integral_constant<int, N>;

// SWIN: the rows' scales (at most 128 bytes a row, 16-byte aligned) are read
// once per tile into a wave-private LDS window instead of per pair from HBM.
// C: the workgroup takes C adjacent column tiles of the expert as one
// pipeline -- pair v is pair v % npairs of tile v / npairs -- so the loads of
// a tile's first pairs are in flight while the previous tile's last pairs are
// computed and its outputs stored (each tile's accumulators start at zero;
// its scales come per pair, SWIN off).
template <int MODE, bool SF16, bool ROWS32, bool SWIN, int C>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, const uint8_t* Wt, const void* S, uint32_t xor4, int m0,
                                          int m1, int nbase0, uint8_t* lds) {
  static_assert(C == 1 || !SWIN, "chained tiles read their scales per pair");
  constexpr int kTileCols = MODE == MODE_GATE_UP ? 64 : 128;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, ln = lane & 15, q = lane >> 4;
  const uint32_t row_bytes = (uint32_t)a.K / 2, G = (uint32_t)(a.K / a.gs);
  const int nsteps = a.K / kGK, last = nsteps - 1, npairs = (nsteps + 1) / 2;
  const int nv = C * npairs, lastv = nv - 1;  // pairs of all C tiles, in one pipeline
  const int nbase = nbase0;
  // weight row of sub-tile s, row r of it in the tile at nb (rows past the matrix: row 0, not stored)
  auto weight_row = [&](int s, int r, bool* ok, int nb) -> uint32_t {
    if (MODE == MODE_GATE_UP) {
      const int j = nb + 16 * wave + r;
      *ok = j < a.I;
      return (s == 0 ? 0u : (uint32_t)a.I) + (uint32_t)(*ok ? j : 0);
    } else {
      const int n = nb + 32 * wave + 16 * s + r;
      *ok = n < a.N;
      return (uint32_t)(*ok ? n : 0);
    }
  };
  auto tile_of = [&](int v) { return C == 1 ? 0 : v / npairs; };
  // MFMA layout: lane (ln, q) works on row ln of each sub-tile
  bool wok0[2];
  uint32_t wrow[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) wrow[s] = weight_row(s, ln, &wok0[s], nbase);
  // load layout: load j of a pair reads row 8 j + lane / 8 of the wave's 32
  // (sub-tile j / 2), bytes 16 (lane % 8) of the pair's 128
  uint32_t lrowb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bool ok;
    lrowb[j] = weight_row(j >> 1, 8 * (j & 1) + (lane >> 3), &ok, nbase) * row_bytes;
  }
  auto lrow_of = [&](int j, int c) {
    if (C == 1) return lrowb[j];
    bool ok;
    return weight_row(j >> 1, 8 * (j & 1) + (lane >> 3), &ok, nbase + kTileCols * c) * row_bytes;
  };
  // the lane's 32-column run of step st starts at column 128 st + 32 q; its
  // group is x / d with x = 4 st + q, d = gs / 32, as the high word of
  // 2x * ceil(2^31 / d) (the multiplier fits 32 bits for d = 1 too): exact
  // while x * d < 2^31, i.e. for K below 2^20
  const uint32_t g32 = (uint32_t)(a.gs / 32), gmul = (uint32_t)((0x80000000ull + g32 - 1) / g32);
  auto group_of = [&](int st) -> uint32_t { return __umulhi((uint32_t)(8 * st + 2 * q), gmul); };
  // two pairs in flight: slot B holds pair p with p % 2 == B. The compute of
  // pair p reads its scales from the slot, so a slot's scales are reloaded
  // after that compute, its weights before.
  uint4 breg[2][4];
  uint32_t sreg[2][2][2];  // [slot][sub-tile][step of the pair]
  auto load_w = [&](int v, auto slot) {
    constexpr int B = decltype(slot)::value;
    const int c = tile_of(v), p = v - c * npairs;
    // a last pair of one step reads its 64 bytes twice (within the row)
    const uint32_t cb = 128u * p + 16u * (2 * p + 1 < nsteps ? (lane & 7) : (lane & 3));
#pragma unroll
    for (int j = 0; j < 4; ++j) breg[B][j] = stream_load16(Wt + (lrow_of(j, c) + cb));
  };
  auto load_s = [&](int p, auto slot) {
    if constexpr (!SWIN) {
      constexpr int B = decltype(slot)::value;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int c = tile_of(p), pp = p - c * npairs;
          bool ok;
          const uint32_t wr = C == 1 ? wrow[s] : weight_row(s, ln, &ok, nbase + kTileCols * c);
          sreg[B][s][h] = gscale_bits<SF16>(S, wr * G + group_of(min(2 * pp + h, last)));
        }
    }
  };
  // the scale window: row r of the wave's 32 at r * kSRow, its scales as stored
  uint8_t* const swin = lds + 2 * kABuf + 4 * kBWave + wave * kSWave;
  if constexpr (SWIN) {
    // load j: row 8 j + lane / 8 (as the weights), bytes 16 (lane % 8) of the
    // row's scales; lanes past the row's end read its start (not used)
    const uint32_t sb = SF16 ? 2u : 4u, srow_bytes = G * sb;
    const uint32_t b = 16u * (lane & 7) < srow_bytes ? 16u * (lane & 7) : 0u;
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = *gptr<u32x4>(static_cast<const uint8_t*>(S) + (lrow_of(j, 0) / row_bytes) * srow_bytes + b);
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(swin + (8 * j + (lane >> 3)) * kSRow + b) = v[j];
    // read by this wave's lanes only (LDS serves a wave in order)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  uint8_t* const bw = lds + 2 * kABuf + wave * kBWave;
  auto take_pair = [&](auto slot) {
    constexpr int B = decltype(slot)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<uint4*>(bw + (8 * j + (lane >> 3)) * kBRow + 16 * (lane & 7)) = breg[B][j];
    // other lanes of this wave read what it wrote: keep the compiler from
    // moving the reads above the writes (LDS serves a wave in order)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  const uint32_t c0 = widen_c0(xor4), c1 = widen_c1(xor4);
  const int srow = tid >> 4, aseg = tid & 15;  // staging: row 16 i + srow, 16 bytes at 16 aseg

  // f32 rows take twice the registers per staged row: passes of 32 rows; f16
  // rows: passes of 48 (a fourth row tile would not fit the registers beside
  // the scaling of silu(gate) * up)
  constexpr int kPassRows = ROWS32 ? 32 : kGRows;
  for (int mb = m0; mb < m1; mb += kPassRows) {
    const int rows = min(kPassRows, m1 - mb);
    auto pass = [&](auto rt_c) {
      constexpr int RT = decltype(rt_c)::value;
      int arow[RT];
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        const int am = mb + min(16 * i + srow, rows - 1);
        arow[i] = (ROWS32 || MODE == MODE_GATE_UP) && a.rows ? a.rows[am] : am;
      }
      float* const fbuf = reinterpret_cast<float*>(lds + kFacOff);
      // Each staged row's undoing factor, for the epilogue (row 16 i + srow of
      // the pass, in LDS), and what staging multiplies by:
      //   GATE_UP: the gathered row's factor;
      //   DOWN: silu(gate) * up comes scaled per row and 16 columns (af: its
      //         undoing factors); staging rescales every piece to the row's
      //         largest factor (the piece with the largest values), so one
      //         factor per row remains;
      //   PLAIN: f32 rows, scaled while staged by the power of two that puts
      //         the row's largest |value| in [2^13, 2^14) (found here first).
      // The factors are read before the pipeline's first loads (oldest, so that
      // waiting for them waits for nothing newer) and committed after them.
      float rowf[RT];
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        rowf[i] = 1.f;
        if constexpr (MODE == MODE_GATE_UP) {
          rowf[i] = a.xfac ? a.xfac[arow[i]] : 1.f;
        } else if constexpr (MODE == MODE_DOWN) {  // the row's factors, 16 threads a row
          const float* af = a.afac + (size_t)arow[i] * a.ldaf;
          const int n = a.K / 16;
          float v[4];  // independent loads, all in flight at once (rows of up to 1024 values)
#pragma unroll
          for (int k = 0; k < 4; ++k) v[k] = aseg + 16 * k < n ? af[aseg + 16 * k] : 0.f;
          rowf[i] = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
          for (int c = aseg + 64; c < n; c += 16) rowf[i] = fmaxf(rowf[i], af[c]);
        }
      }
      auto stage_factors = [&]() {
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          const int r = 16 * i + srow;
          if constexpr (MODE == MODE_GATE_UP) {
            if (aseg == 0) fbuf[r] = rowf[i];
          } else if constexpr (MODE == MODE_DOWN) {
            // the largest over the row's 16 threads
            float m = rowf[i];
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
            m = m > 0.f ? m : 1.f;
            rowf[i] = m;
            if (aseg == 0) fbuf[r] = m;
          } else if constexpr (ROWS32) {
            const float* xr = a.X + (size_t)arow[i] * a.ldx;
            float m = 0.f;
            for (int c = 4 * aseg; c < a.K; c += 64) {
              const float4 v = *reinterpret_cast<const float4*>(xr + c);
              m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
            rowf[i] = pow2_into(m, 14);
            if (aseg == 0) fbuf[r] = 1.f / rowf[i];
          }
        }
      };
      // a step's share of the tile: RT x 16 bytes of f16, or RT x 8 floats;
      // two sets, named by compile-time constants only (so that they stay in
      // registers)
      using AVec = std::conditional_t<ROWS32, float4, u32x4>;
      constexpr int kAV = ROWS32 ? 2 * RT : RT;
      AVec areg[2][kAV];
      float pfac[2][RT];  // DOWN: the undoing factor of the staged piece's 16 columns
      auto load_a = [&](int st, auto set) {
        constexpr int R = decltype(set)::value;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          if constexpr (ROWS32) {
            const float4* src = reinterpret_cast<const float4*>(a.X + (size_t)arow[i] * a.ldx + st * kGK + 8 * aseg);
            areg[R][2 * i] = src[0];
            areg[R][2 * i + 1] = src[1];
          } else {
            areg[R][i] = *reinterpret_cast<const u32x4*>(a.A + (size_t)arow[i] * a.lda + st * kGK + 8 * aseg);
            if constexpr (MODE == MODE_DOWN)
              pfac[R][i] = *gptr<float>(a.afac + (size_t)arow[i] * a.ldaf + 8 * st + (aseg >> 1));
          }
        }
      };
      auto stage_a = [&](auto set, int buf) {
        constexpr int R = decltype(set)::value;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          uint8_t* dst = lds + buf * kABuf + (16 * i + srow) * kARow + 16 * aseg;
          if constexpr (ROWS32) {
            // 8 floats -> 8 f16 in MFMA order: position p holds column (p % 2) * 4 + p / 2
            const float4 lo = areg[R][2 * i], hi = areg[R][2 * i + 1];
            const float c[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            half8 h;
#pragma unroll
            for (int p = 0; p < 8; ++p) h[p] = (_Float16)(c[(p & 1) * 4 + (p >> 1)] * rowf[i]);
            *reinterpret_cast<half8*>(dst) = h;
          } else if constexpr (MODE == MODE_DOWN) {
            // to the row's scaling: times a power of two at most 1, exact but
            // where it reaches f16's subnormals
            const float ratio = pfac[R][i] * __builtin_amdgcn_rcpf(rowf[i]);
            const half8 v = __builtin_bit_cast(half8, areg[R][i]) * (_Float16)ratio;
            *reinterpret_cast<half8*>(dst) = v;
          } else {
            *reinterpret_cast<u32x4*>(dst) = areg[R][i];
          }
        }
      };

      f32x4 acc[RT][2];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int s = 0; s < 2; ++s) acc[rt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

      // step h of the current pair, activations from LDS buffer buf; the
      // fragments of slice i + 1 are read while slice i is widened and multiplied
      auto compute = [&](int h, int buf, auto slot, int p_cur) {
        constexpr int B = decltype(slot)::value;
        const uint8_t* A = lds + buf * kABuf + ln * kARow + 64 * q;
        uint4 w[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) w[s] = *reinterpret_cast<const uint4*>(bw + (16 * s + ln) * kBRow + 64 * h + 16 * q);
        half8 av[2][RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) av[0][rt] = *reinterpret_cast<const half8*>(A + rt * 16 * kARow);
        __half2 s2[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          uint32_t bits;
          if constexpr (SWIN) {
            const uint8_t* sp = swin + (16 * s + ln) * kSRow + group_of(2 * (p_cur) + h) * (SF16 ? 2 : 4);
            if constexpr (SF16) bits = *reinterpret_cast<const uint16_t*>(sp);
            else bits = *reinterpret_cast<const uint32_t*>(sp);
          } else {
            bits = sreg[B][s][h];
          }
          s2[s] = __float2half2_rn(gscale_value<SF16>(bits));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i < 3) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
              av[(i + 1) & 1][rt] = *reinterpret_cast<const half8*>(A + rt * 16 * kARow + 16 * (i + 1));
          }
          const uint32_t w0 = i == 0 ? w[0].x : i == 1 ? w[0].y : i == 2 ? w[0].z : w[0].w;
          const uint32_t w1 = i == 0 ? w[1].x : i == 1 ? w[1].y : i == 2 ? w[1].z : w[1].w;
          const half8 b0 = widen8(w0, s2[0], c0, c1), b1 = widen8(w1, s2[1], c0, c1);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            acc[rt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i & 1][rt], b0, acc[rt][0], 0, 0, 0);
            acc[rt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i & 1][rt], b1, acc[rt][1], 0, 0, 0);
          }
        }
      };

      // Pair p: its weights (slot B) and both of its steps' activation tiles
      // go to LDS first; then the next pair's activations and the weights of
      // pair p + 2 are issued, both steps computed, and the scales of pair
      // p + 2 issued. Loads return in issue order for the wait counts, so
      // each wait here is for loads older than the last weights issued: two
      // pairs stay in flight while a pair is computed. Every load is
      // unconditional (indices past the end repeat the last pair or step, in
      // L2), so the compiler's wait counts stay exact.
      // D layout: lane (ln, q) holds rows 4q .. 4q+3 of column ln of each 16x16 tile;
      // tile c's outputs, then its accumulators start again at zero
      auto epilogue = [&](int c) {
      const int nbase = nbase0 + kTileCols * c;
      bool wok[2] = {wok0[0], wok0[1]};
      if constexpr (C > 1) {
#pragma unroll
        for (int s = 0; s < 2; ++s) (void)weight_row(s, ln, &wok[s], nbase);
      }
      if constexpr (MODE == MODE_GATE_UP) {
        // silu(gate) * up of the wave's 16 columns, scaled per row by the power
        // of two that puts their largest |value| in [2^13, 2^14)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 16 * rt + 4 * q + j, m = mb + r;
            const float fx = fbuf[r];
            const float av = silu(acc[rt][0][j] * fx) * (acc[rt][1][j] * fx);
            float mx = wok[0] ? fabsf(av) : 0.f;
            // every lane of the 16 gets their largest (rotations within the row)
            mx = fmaxf(mx, dpp_read<0x128, 0xf, false>(mx));  // row_ror:8
            mx = fmaxf(mx, dpp_read<0x124, 0xf, false>(mx));  // row_ror:4
            mx = fmaxf(mx, dpp_read<0x4E, 0xf, false>(mx));   // quad_perm [2,3,0,1]
            mx = fmaxf(mx, dpp_read<0xB1, 0xf, false>(mx));   // quad_perm [1,0,3,2]
            const float f = pow2_into(mx, 14);
            if (m < m1) {
              if (wok[0]) a.act[(size_t)m * a.ldact + perm_pos(nbase + 16 * wave + ln)] = (_Float16)(av * f);
              if (ln == 0) a.act_fac[(size_t)m * a.ldaf_out + nbase / 16 + wave] = 1.f / f;
            }
          }
        }
      } else {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int m = mb + 16 * rt + 4 * q + j;
            if (m >= m1) continue;
            const float f = fbuf[16 * rt + 4 * q + j];
#pragma unroll
            for (int s = 0; s < 2; ++s)
              if (wok[s]) a.Y[(size_t)m * a.ldy + nbase + 32 * wave + 16 * s + ln] = acc[rt][s][j] * f;
          }
        }
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int s = 0; s < 2; ++s) acc[rt][s] = f32x4{0.f, 0.f, 0.f, 0.f};
      };
      auto body = [&](int v, auto slot, bool more) {
        const int c = tile_of(v), p = v - c * npairs;
        __syncthreads();  // every wave is done with the previous pair's tiles
        take_pair(slot);
        stage_a(IC<0>{}, 0);
        stage_a(IC<1>{}, 1);
        __syncthreads();
        if (more) {
          // the next pair's steps: this tile's next, or the next tile's first
          const int pn = p + 1 < npairs ? p + 1 : (v + 1 < nv ? 0 : p + 1);
          load_a(min(2 * pn, last), IC<0>{});
          load_a(min(2 * pn + 1, last), IC<1>{});
          load_w(min(v + 2, lastv), slot);
        }
        __builtin_amdgcn_sched_barrier(0);
        compute(0, 0, slot, p);
        if (2 * p + 1 < nsteps) compute(1, 1, slot, p);
        if (more) load_s(min(v + 2, lastv), slot);
        if (p == npairs - 1) epilogue(c);
      };

      // the same issue order as the loop's (weights and scales of a slot, the
      // activations, the other slot): the compiler's wait counts at the loop
      // head merge the prologue's order with the loop's
      load_w(0, IC<0>{});
      load_s(0, IC<0>{});
      __builtin_amdgcn_sched_barrier(0);
      load_a(0, IC<0>{});
      load_a(min(1, last), IC<1>{});
      load_w(min(1, lastv), IC<1>{});
      __builtin_amdgcn_sched_barrier(0);
      load_s(min(1, lastv), IC<1>{});
      __builtin_amdgcn_sched_barrier(0);
      stage_factors();
      int v = 0;
      for (; v + 2 < nv; v += 2) {
        body(v, IC<0>{}, true);
        body(v + 1, IC<1>{}, true);
      }
      if (v + 2 == nv) {
        body(v, IC<0>{}, true);
        body(v + 1, IC<1>{}, false);
      } else {
        body(v, IC<0>{}, false);
      }

    };
    // the same on every thread of the workgroup: no thread skips a barrier
    if constexpr (ROWS32) {
      if (rows <= 16) pass(IC<1>{});
      else pass(IC<2>{});
    } else {
      switch ((rows + 15) >> 4) {
        case 1: pass(IC<1>{}); break;
        case 2: pass(IC<2>{}); break;
        default: pass(IC<3>{}); break;
      }
    }
    __syncthreads();  // the LDS tiles are refilled by the next pass
  }
}

template <int MODE, bool ROWS32, int C>
__global__ __launch_bounds__(256, 2) void gemm_q4_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kGemmLds];
  // all column tiles of one expert on one XCD: its activation rows stay in that L2
  const int L = xcd_contiguous(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
  const int e = L / gridDim.x, tile = L % gridDim.x;
  const int m0 = a.table ? a.eoff[e] : 0, m1 = a.table ? a.eoff[e + 1] : a.single_rows;
  if (m0 >= m1) return;  // the whole workgroup: before any barrier
  const int nbase = tile * C * (MODE == MODE_GATE_UP ? 64 : 128);
  const ExpertDesc d = a.table ? a.table[e] : a.single;
  const uint8_t* Wt = a.which ? d.dn_w : d.gu_w;
  const void* S = a.which ? d.dn_s : d.gu_s;
  const uint32_t xor4 = d.xor8 * 0x01010101u;
  // scale rows of at most 128 bytes, 16-byte aligned: read once into LDS
  const uint32_t srow_bytes = (uint32_t)(a.K / a.gs) * (d.s_f16 ? 2u : 4u);
  const bool swin = srow_bytes <= 128 && srow_bytes % 16 == 0 && ((uintptr_t)S & 15) == 0;
  if constexpr (C > 1) {
    (void)swin;
    if (d.s_f16) gemm_tile<MODE, true, ROWS32, false, C>(a, Wt, S, xor4, m0, m1, nbase, lds);
    else gemm_tile<MODE, false, ROWS32, false, C>(a, Wt, S, xor4, m0, m1, nbase, lds);
  } else if (d.s_f16) {
    if (swin) gemm_tile<MODE, true, ROWS32, true, 1>(a, Wt, S, xor4, m0, m1, nbase, lds);
    else gemm_tile<MODE, true, ROWS32, false, 1>(a, Wt, S, xor4, m0, m1, nbase, lds);
  } else {
    if (swin) gemm_tile<MODE, false, ROWS32, true, 1>(a, Wt, S, xor4, m0, m1, nbase, lds);
    else gemm_tile<MODE, false, ROWS32, false, 1>(a, Wt, S, xor4, m0, m1, nbase, lds);
  }
}

// ------------------------------------------------------------------ combine

// out[t] = sum over t's picks in ascending expert order (= ascending pair
// position) of w * y[pos]; overwrites out (the layer output starts at zero).
// One block per token. The picks are put in LDS in position order -- a pick's
// rank is the number of smaller positions, positions being distinct: for
// k <= 64 the first wave ranks them with shuffles; for more, the block stages
// the positions in dynamic LDS (12 bytes a pick) and every thread ranks its
// picks against them. Then each thread sums float4 columns over the picks in
// order.
__global__ __launch_bounds__(256) void token_combine_kernel(const float* y, int ldy, const int* pos, const float* wts,
                                                            int k, int H, float* out, int ldo, int vec4) {
  __shared__ int sp64[64];
  __shared__ float sw64[64];
  __shared__ int sn;
  extern __shared__ int dyn[];  // k > 64: raw positions [k], ordered positions [k], weights [k]
  const int t = blockIdx.x;
  const int* prow = pos + (size_t)t * k;
  int* sp = sp64;
  float* sw = sw64;
  if (k <= 64) {
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      const bool mine = lane < k;
      const int p = mine ? prow[lane] : -1;
      int rank = 0;
      for (int i = 0; i < k; ++i) {
        const int pi = __shfl(p, i, 64);
        rank += (pi >= 0 && pi < p) ? 1 : 0;
      }
      const uint64_t valid = __ballot(mine && p >= 0);
      if (mine && p >= 0) {
        sp[rank] = p;
        sw[rank] = wts[p];
      }
      if (lane == 0) sn = __popcll(valid);
    }
  } else {
    int* raw = dyn;
    sp = dyn + k;
    sw = reinterpret_cast<float*>(dyn + 2 * k);
    if (threadIdx.x == 0) sn = 0;
    for (int i = threadIdx.x; i < k; i += 256) raw[i] = prow[i];
    __syncthreads();
    int valid = 0;
    for (int i = threadIdx.x; i < k; i += 256) {
      const int p = raw[i];
      if (p < 0) continue;
      int rank = 0;
      for (int j = 0; j < k; ++j) rank += (raw[j] >= 0 && raw[j] < p) ? 1 : 0;
      sp[rank] = p;
      sw[rank] = wts[p];
      ++valid;
    }
    for (int off = 32; off > 0; off >>= 1) valid += __shfl_xor(valid, off, 64);
    if ((threadIdx.x & 63) == 0) atomicAdd(&sn, valid);
  }
  __syncthreads();
  const int n = sn;
  float* dst = out + (size_t)t * ldo;
  if (vec4) {
    for (int c = threadIdx.x * 4; c < H; c += 1024) {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
      for (int i = 0; i < n; ++i) {
        const float w = sw[i];
        const float4 v = *reinterpret_cast<const float4*>(y + (size_t)sp[i] * ldy + c);
        a.x += w * v.x;
        a.y += w * v.y;
        a.z += w * v.z;
        a.w += w * v.w;
      }
      *reinterpret_cast<float4*>(dst + c) = a;
    }
  } else {
    for (int c = threadIdx.x; c < H; c += 256) {
      float a = 0.f;
      for (int i = 0; i < n; ++i) a += sw[i] * y[(size_t)sp[i] * ldy + c];
      dst[c] = a;
    }
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

bool router_mfma_ok(const float* x, int ldx, const float* R, int H) {
  return H % 64 == 0 && ldx % 4 == 0 && aligned(x, 16) && aligned(R, 16);
}

// K slices of the MFMA router: one, unless the token x expert tiles are too
// few to fill the chip (then up to max_slices, each of at least 1024 columns)
int router_mfma_slices(int T, int E, int H, int max_slices) {
  const long tiles = (long)((T + 15) / 16) * ((E + 15) / 16);
  int z = 1;
  while (2 * z <= max_slices && tiles * z < 256 && H % (512 * z) == 0 && H / (2 * z) >= 1024) z *= 2;
  return z;
}

int run_router_mfma(const float* x, int ldx, const float* R, int T, int E, int H, int nz, float* part, hipStream_t st) {
  if (T <= 0) return MOE_OK;
  const dim3 grid((T + 15) / 16, (E + 15) / 16, nz);
  const int kslice = H / nz;
  // W waves per block, each kslice / W columns in chunks of CH x 16
  if (kslice % (16 * 128) == 0)
    hipLaunchKernelGGL((router_mfma_kernel<16, 8>), grid, dim3(1024), 0, st, x, ldx, R, T, E, H, kslice, part);
  else if (kslice % (4 * 128) == 0)
    hipLaunchKernelGGL((router_mfma_kernel<4, 8>), grid, dim3(256), 0, st, x, ldx, R, T, E, H, kslice, part);
  else
    hipLaunchKernelGGL((router_mfma_kernel<4, 1>), grid, dim3(256), 0, st, x, ldx, R, T, E, H, kslice, part);
  return check_launch("router logits (MFMA)");
}

int run_router_logits(const float* x, int ldx, const float* R, int T, int E, int H, float* logits, float* scratch,
                      hipStream_t st) {
  if (router_mfma_ok(x, ldx, R, H)) {
    const int nz = scratch ? router_mfma_slices(T, E, H, router_slices(T, E, H)) : 1;
    int rc = run_router_mfma(x, ldx, R, T, E, H, nz, nz > 1 ? scratch : logits, st);
    if (rc || nz == 1) return rc;
    const long n = (long)T * E;
    hipLaunchKernelGGL(sum_slices_kernel, dim3(blocks_for(n)), dim3(256), 0, st, scratch, nz, n, logits);
    return check_launch("router logits (slice sum)");
  }
  const int nz = scratch ? router_slices(T, E, H) : 1;
  int rc = run_router_partials(x, ldx, R, T, E, H, nz, nz > 1 ? scratch : logits, st);
  if (rc || nz == 1) return rc;
  const long n = (long)T * E;
  hipLaunchKernelGGL(sum_slices_kernel, dim3(blocks_for(n)), dim3(256), 0, st, scratch, nz, n, logits);
  return check_launch("router logits (slice sum)");
}

int run_route(const float* logits, int nz, int T, int E, int k, int normalize, int* idx, float* w, hipStream_t st,
              const float* x, int ldx, int H, _Float16* xs, float* xf) {
  if (T <= 0) return MOE_OK;
  const dim3 grid((T + 3) / 4), block(256);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, block, 0, st, logits, nz, T, E, k, normalize, idx, w, x, ldx, H, xs, xf);
  };
  if (E <= 256) go(route_kernel<4>);
  else if (E <= 1024) go(route_kernel<16>);
  else go(route_kernel<0>);
  return check_launch("softmax top-k");
}

int run_group(const int* idx, const float* w, int T, int k, int E, int* eoff, int* rows, float* wts, int* pos,
              int* experts, int* offsets, int* n_used, hipStream_t st) {
  hipLaunchKernelGGL(group_kernel, dim3(E), dim3(256), 0, st, idx, w, T * k, k, E, eoff, rows, wts, pos);
  if (int rc = check_launch("group by expert")) return rc;
  if (!experts) return MOE_OK;
  hipLaunchKernelGGL(used_experts_kernel, dim3(1), dim3(1024), 0, st, eoff, E, experts, offsets, n_used);
  return check_launch("group by expert (used experts)");
}

int run_gather_f16(const float* x, int ldx, const int* rows, int P, int K, _Float16* Xs, float* fac, hipStream_t st) {
  if (P <= 0) return MOE_OK;
  hipLaunchKernelGGL(gather_f16_kernel, dim3((P + 3) / 4), dim3(256), 0, st, x, ldx, rows, P, K, Xs, K, fac);
  return check_launch("gather rows (f16)");
}

int run_gemm(int mode, const GemmArgs& a, int nexp, hipStream_t st) {
  if (nexp <= 0) return MOE_OK;
  if (nexp > kMaxGridY)
    return set_error(MOE_EUNSUPPORTED, "int4 grouped GEMM: %d experts (at most %d a launch)", nexp, kMaxGridY);
  const int per_tile = mode == MODE_GATE_UP ? 64 : 128;
  const int n = mode == MODE_GATE_UP ? a.I : a.N;
  const int ntiles = (n + per_tile - 1) / per_tile;
  // The down product (K = I, a few pairs a tile) chains 4 column tiles a
  // workgroup while the launch still fills the chip's 512 workgroup slots:
  // a tile's first loads then overlap the previous tile's last pairs and
  // stores. MOEHIP_GEMM_CHAIN=1, 2 or 4 sets it (a measurement switch).
  static const int chain_env = [] {
    const char* e = getenv("MOEHIP_GEMM_CHAIN");
    const int v = e ? atoi(e) : 0;
    return v == 1 || v == 2 || v == 4 ? v : 0;
  }();
  int C = 1;
  if (mode == MODE_DOWN && !a.rows32) {
    if (chain_env) C = chain_env;
    else if ((long)(ntiles / 4) * nexp >= 512) C = 4;
    if (ntiles % C != 0) C = 1;
  }
  dim3 grid(ntiles / C, nexp);
  auto go = [&](auto k) { hipLaunchKernelGGL(k, grid, dim3(256), 0, st, a); };
  if (a.rows32) {
    if (mode == MODE_PLAIN) go(gemm_q4_kernel<MODE_PLAIN, true, 1>);
    else return set_error(MOE_EINVAL, "int4 grouped GEMM: only the plain product takes f32 rows");
  } else if (mode == MODE_PLAIN) {
    go(gemm_q4_kernel<MODE_PLAIN, false, 1>);
  } else if (mode == MODE_GATE_UP) {
    go(gemm_q4_kernel<MODE_GATE_UP, false, 1>);
  } else {
    if (C == 4) go(gemm_q4_kernel<MODE_DOWN, false, 4>);
    else if (C == 2) go(gemm_q4_kernel<MODE_DOWN, false, 2>);
    else go(gemm_q4_kernel<MODE_DOWN, false, 1>);
  }
  return check_launch("int4 grouped GEMM");
}

int run_token_combine(const float* y, int ldy, const int* pos, const float* wts, int T, int k, int H, float* out,
                      int ldo, hipStream_t st) {
  if (T <= 0) return MOE_OK;
  if (k > kCombineMaxPicks)
    return set_error(MOE_EUNSUPPORTED, "token combine: k=%d (at most %d picks per token)", k, kCombineMaxPicks);
  const int vec4 = H % 4 == 0 && ldy % 4 == 0 && ldo % 4 == 0 && aligned(y, 16) && aligned(out, 16);
  const size_t lds = k > 64 ? (size_t)12 * k : 0;
  hipLaunchKernelGGL(token_combine_kernel, dim3(T), dim3(256), lds, st, y, ldy, pos, wts, k, H, out, ldo, vec4);
  return check_launch("token combine");
}

}  // namespace moe
