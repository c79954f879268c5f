// Widen packed weights to f32, bit-exact with moelan's decoders:
//   int4   (u - 8) * s          moelan/kernels.py:215-228
//   int8   q * s                moelan/kernels.py:230-237
//   Q8_0   d * q                moelan/kernels.py:262-268
//   Q4_K   (d*sc) * q - dmin*m  moelan/kernels.py:318-336 (no FMA contraction)
//   the other GGUF block types: blocks.hip
// Not on the hot path (the mat-vec and the grouped GEMM never materialise
// f32 weights); used by the matrix objects' dequant() and by tests.
#include "common.h"
#include "formats.h"
#include "dequant.h"
#include "matvec.h"
#include "blocks.h"

namespace moe {

__global__ void dq_q4_kernel(const uint8_t* raw, const void* s, int s_f16, int O, int I, int gs, uint32_t xor8,
                             float* out) {
  const long nbytes = (long)O * (I / 2);
  const int G = I / gs;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < nbytes; i += (long)gridDim.x * blockDim.x) {
    const int o = (int)(i / (I / 2)), j = (int)(i % (I / 2));
    const uint32_t b = raw[i] ^ xor8;
    const int c = 2 * j;
    const float sc0 = load_scale(s, (size_t)o * G + c / gs, s_f16);
    const float sc1 = load_scale(s, (size_t)o * G + (c + 1) / gs, s_f16);
    out[(size_t)o * I + c] = __fmul_rn((float)((int)(b & 15u) - 8), sc0);
    out[(size_t)o * I + c + 1] = __fmul_rn((float)((int)(b >> 4) - 8), sc1);
  }
}

__global__ void dq_q8_kernel(const int8_t* q, const void* s, int s_f16, int O, int I, int gs, float* out) {
  const long n = (long)O * I;
  const int G = I / gs;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const int o = (int)(i / I), c = (int)(i % I);
    out[i] = __fmul_rn((float)q[i], load_scale(s, (size_t)o * G + c / gs, s_f16));
  }
}

__global__ void dq_q8_0_kernel(const uint8_t* raw, int O, int cols, float* out) {
  const int nb = cols / 32;
  const long n = (long)O * nb;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const int o = (int)(i / nb), b = (int)(i % nb);
    const uint8_t* blk = raw + (size_t)o * nb * 34 + (size_t)b * 34;
    const float d = gguf_half(blk[0] | (blk[1] << 8));
    float* dst = out + (size_t)o * cols + (size_t)b * 32;
    for (int j = 0; j < 32; ++j) dst[j] = __fmul_rn(d, (float)(int8_t)blk[2 + j]);
  }
}

__global__ void dq_q4_k_kernel(const uint8_t* raw, int O, int cols, float* out) {
  const int nb = cols / 256;
  const long n = (long)O * nb * 4;  // one thread per 64 values
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const int kk = (int)(i % 4);
    const long ob = i / 4;
    const int o = (int)(ob / nb), b = (int)(ob % nb);
    const uint8_t* blk = raw + (size_t)o * nb * 144 + (size_t)b * 144;
    const float d = gguf_half(blk[0] | (blk[1] << 8)), dmin = gguf_half(blk[2] | (blk[3] << 8));
    const FmtQ4K::MemBytes sb{blk + 4};
    int sc, m;
    FmtQ4K::scale_min(2 * kk, sb, sc, m);
    const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)m);
    FmtQ4K::scale_min(2 * kk + 1, sb, sc, m);
    const float d2 = __fmul_rn(d, (float)sc), m2 = __fmul_rn(dmin, (float)m);
    float* dst = out + (size_t)o * cols + (size_t)b * 256 + kk * 64;
    const uint8_t* q = blk + 16 + 32 * kk;
    for (int l = 0; l < 32; ++l) {
      const uint32_t v = q[l];
      dst[l] = __fsub_rn(__fmul_rn(d1, (float)(v & 15u)), m1);
      dst[32 + l] = __fsub_rn(__fmul_rn(d2, (float)(v >> 4)), m2);
    }
  }
}

static int grid_for(long n) {
  long b = (n + 255) / 256;
  return (int)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

int run_dequant_q4(const uint8_t* raw, const void* s, int s_f16, int O, int I, int gs, uint32_t xor8, float* out,
                   hipStream_t st) {
  hipLaunchKernelGGL(dq_q4_kernel, dim3(grid_for((long)O * I / 2)), dim3(256), 0, st, raw, s, s_f16, O, I, gs, xor8,
                     out);
  return check_launch("int4 dequant");
}

int run_dequant_q8(const int8_t* q, const void* s, int s_f16, int O, int I, int gs, float* out, hipStream_t st) {
  hipLaunchKernelGGL(dq_q8_kernel, dim3(grid_for((long)O * I)), dim3(256), 0, st, q, s, s_f16, O, I, gs, out);
  return check_launch("int8 dequant");
}

int run_dequant_gguf(const uint8_t* raw, int qtype, int O, int cols, float* out, hipStream_t st) {
  if (qtype == FMT_Q8_0)
    hipLaunchKernelGGL(dq_q8_0_kernel, dim3(grid_for((long)O * cols / 32)), dim3(256), 0, st, raw, O, cols, out);
  else if (qtype == FMT_Q4_K)
    hipLaunchKernelGGL(dq_q4_k_kernel, dim3(grid_for((long)O * cols / 64)), dim3(256), 0, st, raw, O, cols, out);
  else
    return run_dequant_blocks(raw, qtype, O, cols, out, st);
  return check_launch("GGUF dequant");
}

}  // namespace moe
