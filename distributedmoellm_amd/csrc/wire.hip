// Activations on the wire between a coordinator and its workers
// (moelan/protocol.py:90-123): encoded and decoded on the device, so a worker
// sends y[touched] straight from HBM and reads x into HBM without host passes.
//
//   f16   each value rounded to half (round to nearest even, overflow to inf):
//         numpy's astype(float16)
//   int8  per row, groups of 64 values (the whole row when 64 does not divide
//         it): s = max|g| / 127 (1 for a zero group), q = clip(rint(g / s),
//         -127, 127) with an IEEE divide and round-half-to-even; s kept as f32
//
// Encoding gathers rows (the touched rows of y); decoding scatters them into
// a strided f32 output. Bit-exact with the reference for finite inputs.
#include "common.h"
#include "wire.h"

namespace moe {

namespace {

// one wave per (row, group of 64): lane j holds value j of the group
__global__ __launch_bounds__(256) void wire_i8_enc64_kernel(const float* a, int lda, const int* rows, int n, int d,
                                                            int8_t* q, float* s) {
  const int G = d / 64;
  const long wid = ((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wid >= (long)n * G) return;  // the whole wave
  const int r = (int)(wid / G), g = (int)(wid % G);
  const float v = a[(size_t)(rows ? rows[r] : r) * lda + g * 64 + lane];
  float m = fabsf(v);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  float sc = __fdiv_rn(m, 127.0f);
  if (sc == 0.0f) sc = 1.0f;
  const float t = rintf(__fdiv_rn(v, sc));
  q[(size_t)r * d + g * 64 + lane] = (int8_t)fminf(fmaxf(t, -127.0f), 127.0f);
  if (lane == 0) s[(size_t)r * G + g] = sc;
}

// the whole row one group (d not a multiple of 64): one block per row
__global__ __launch_bounds__(256) void wire_i8_enc_row_kernel(const float* a, int lda, const int* rows, int d,
                                                              int8_t* q, float* s) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const float* src = a + (size_t)(rows ? rows[r] : r) * lda;
  float m = 0.0f;
  for (int c = threadIdx.x; c < d; c += blockDim.x) m = fmaxf(m, fabsf(src[c]));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sc = __fdiv_rn(m, 127.0f);
  if (sc == 0.0f) sc = 1.0f;
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    const float t = rintf(__fdiv_rn(src[c], sc));
    q[(size_t)r * d + c] = (int8_t)fminf(fmaxf(t, -127.0f), 127.0f);
  }
  if (threadIdx.x == 0) s[r] = sc;
}

// f16 (round to nearest even) or f32 (a gathered copy)
template <class T>
__global__ void wire_cast_kernel(const float* a, int lda, const int* rows, int n, int d, T* out) {
  const long total = (long)n * d;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int r = (int)(i / d), c = (int)(i % d);
    const float v = a[(size_t)(rows ? rows[r] : r) * lda + c];
    if constexpr (sizeof(T) == 2) out[i] = __float2half_rn(v);
    else out[i] = v;
  }
}

// out[rows[r]] (or out[r]) = decoded row r
__global__ void wire_dec_kernel(const void* in, const float* s, int wire, int n, int d, int gs, const int* rows,
                                float* out, int ldo) {
  const long total = (long)n * d;
  const int G = d / gs;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int r = (int)(i / d), c = (int)(i % d);
    float v;
    if (wire == MOE_WIRE_INT8) v = __fmul_rn((float)reinterpret_cast<const int8_t*>(in)[i], s[(size_t)r * G + c / gs]);
    else if (wire == MOE_WIRE_F16) v = __half2float(reinterpret_cast<const __half*>(in)[i]);
    else v = reinterpret_cast<const float*>(in)[i];
    out[(size_t)(rows ? rows[r] : r) * ldo + c] = v;
  }
}

// 16-byte vectors: 4 values a lane, rows a multiple of 4 values apart

// one wave per 4 groups of 64: 16 lanes a group, each with 4 consecutive values
__global__ __launch_bounds__(256) void wire_i8_enc64x4_kernel(const float* a, int lda, const int* rows, int n, int d,
                                                              int8_t* q, float* s) {
  const int G = d / 64;
  const long total = (long)n * G;
  const long gid = (((long)blockIdx.x * blockDim.x + threadIdx.x) >> 6) * 4 + ((threadIdx.x & 63) >> 4);
  const int l16 = threadIdx.x & 15;
  const bool on = gid < total;  // every lane takes part in the shuffles below
  const int r = on ? (int)(gid / G) : 0, g = on ? (int)(gid % G) : 0;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (on) v = *reinterpret_cast<const float4*>(a + (size_t)(rows ? rows[r] : r) * lda + g * 64 + 4 * l16);
  float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));  // within the 16 lanes
  if (!on) return;
  float sc = __fdiv_rn(m, 127.0f);
  if (sc == 0.0f) sc = 1.0f;
  const float e[4] = {v.x, v.y, v.z, v.w};
  uint32_t packed = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float t = fminf(fmaxf(rintf(__fdiv_rn(e[k], sc)), -127.0f), 127.0f);
    packed |= ((uint32_t)(int)t & 0xFFu) << (8 * k);
  }
  *reinterpret_cast<uint32_t*>(q + (size_t)r * d + g * 64 + 4 * l16) = packed;
  if (l16 == 0) s[(size_t)r * G + g] = sc;
}

template <class T>
__global__ void wire_cast4_kernel(const float* a, int lda, const int* rows, int n, int d, T* out) {
  const int d4 = d / 4;
  const long total = (long)n * d4;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int r = (int)(i / d4), c = (int)(i % d4) * 4;
    const float4 v = *reinterpret_cast<const float4*>(a + (size_t)(rows ? rows[r] : r) * lda + c);
    if constexpr (sizeof(T) == 2) {
      const __half2 lo = __floats2half2_rn(v.x, v.y), hi = __floats2half2_rn(v.z, v.w);
      uint2 u;
      u.x = *reinterpret_cast<const uint32_t*>(&lo);
      u.y = *reinterpret_cast<const uint32_t*>(&hi);
      *reinterpret_cast<uint2*>(out + (size_t)r * d + c) = u;
    } else {
      *reinterpret_cast<float4*>(out + (size_t)r * d + c) = v;
    }
  }
}

__global__ void wire_dec4_kernel(const void* in, const float* s, int wire, int n, int d, int gs, const int* rows,
                                 float* out, int ldo) {
  const int d4 = d / 4, G = d / gs;
  const long total = (long)n * d4;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    const int r = (int)(i / d4), c = (int)(i % d4) * 4;
    const size_t at = (size_t)r * d + c;
    float4 v;
    if (wire == MOE_WIRE_INT8) {
      const uint32_t b = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const int8_t*>(in) + at);
      const float sc = s[(size_t)r * G + c / gs];  // 4 values never straddle a group (gs % 4 == 0)
      v.x = __fmul_rn((float)(int8_t)(b & 0xFFu), sc);
      v.y = __fmul_rn((float)(int8_t)((b >> 8) & 0xFFu), sc);
      v.z = __fmul_rn((float)(int8_t)((b >> 16) & 0xFFu), sc);
      v.w = __fmul_rn((float)(int8_t)(b >> 24), sc);
    } else if (wire == MOE_WIRE_F16) {
      const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const __half*>(in) + at);
      const float2 lo = __half22float2(*reinterpret_cast<const __half2*>(&u.x));
      const float2 hi = __half22float2(*reinterpret_cast<const __half2*>(&u.y));
      v = make_float4(lo.x, lo.y, hi.x, hi.y);
    } else {
      v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(in) + at);
    }
    *reinterpret_cast<float4*>(out + (size_t)(rows ? rows[r] : r) * ldo + c) = v;
  }
}

int grid_of(long n, int per_block) {
  long b = (n + per_block - 1) / per_block;
  return (int)(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

}  // namespace

int wire_group(int d) { return d % 64 == 0 ? 64 : d; }

int run_wire_encode(const float* a, int lda, const int* rows, int n, int d, int wire, void* out, float* scale,
                    hipStream_t st) {
  if (n <= 0) return MOE_OK;
  // 16-byte loads of the source rows, 4-value stores
  const bool v4 = d % 4 == 0 && lda % 4 == 0 && aligned(a, 16) && aligned(out, 8);
  if (v4 && wire == MOE_WIRE_INT8 && d % 64 == 0) {
    const long waves = ((long)n * (d / 64) + 3) / 4;
    hipLaunchKernelGGL(wire_i8_enc64x4_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a, lda, rows, n,
                       d, static_cast<int8_t*>(out), scale);
    return check_launch("wire encode");
  }
  if (v4 && wire == MOE_WIRE_F16) {
    hipLaunchKernelGGL(wire_cast4_kernel<__half>, dim3(grid_of((long)n * d / 4, 256)), dim3(256), 0, st, a, lda, rows,
                       n, d, static_cast<__half*>(out));
    return check_launch("wire encode");
  }
  if (v4 && wire == MOE_WIRE_F32 && aligned(out, 16)) {
    hipLaunchKernelGGL(wire_cast4_kernel<float>, dim3(grid_of((long)n * d / 4, 256)), dim3(256), 0, st, a, lda, rows,
                       n, d, static_cast<float*>(out));
    return check_launch("wire encode");
  }
  if (wire == MOE_WIRE_INT8) {
    if (d % 64 == 0) {
      const long waves = (long)n * (d / 64);
      hipLaunchKernelGGL(wire_i8_enc64_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a, lda, rows, n,
                         d, static_cast<int8_t*>(out), scale);
    } else {
      hipLaunchKernelGGL(wire_i8_enc_row_kernel, dim3((unsigned)n), dim3(256), 0, st, a, lda, rows, d,
                         static_cast<int8_t*>(out), scale);
    }
  } else if (wire == MOE_WIRE_F16) {
    hipLaunchKernelGGL(wire_cast_kernel<__half>, dim3(grid_of((long)n * d, 256)), dim3(256), 0, st, a, lda, rows, n,
                       d, static_cast<__half*>(out));
  } else {
    hipLaunchKernelGGL(wire_cast_kernel<float>, dim3(grid_of((long)n * d, 256)), dim3(256), 0, st, a, lda, rows, n,
                       d, static_cast<float*>(out));
  }
  return check_launch("wire encode");
}

int run_wire_decode(const void* in, const float* scale, int wire, int n, int d, const int* rows, float* out, int ldo,
                    hipStream_t st) {
  if (n <= 0) return MOE_OK;
  const int gs = wire_group(d);
  if (d % 4 == 0 && gs % 4 == 0 && ldo % 4 == 0 && aligned(out, 16) && aligned(in, 16)) {
    hipLaunchKernelGGL(wire_dec4_kernel, dim3(grid_of((long)n * d / 4, 256)), dim3(256), 0, st, in, scale, wire, n, d,
                       gs, rows, out, ldo);
    return check_launch("wire decode");
  }
  hipLaunchKernelGGL(wire_dec_kernel, dim3(grid_of((long)n * d, 256)), dim3(256), 0, st, in, scale, wire, n, d, gs,
                     rows, out, ldo);
  return check_launch("wire decode");
}

}  // namespace moe
