// Shared helpers for the routed-expert HIP kernels (gfx950, wave64).
//
// Every exported entry point validates its arguments on the host, records a
// readable message with set_error() on failure and returns a non-zero status;
// moe_last_error() hands the message to the caller (thread-local, like errno).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#define MOE_API extern "C" __attribute__((visibility("default")))

// status codes shared with include/moehip.h
#define MOE_OK 0
#define MOE_EINVAL 1      // bad argument (shape, pointer, size)
#define MOE_EHIP 2        // a HIP runtime call failed
#define MOE_EWORKSPACE 3  // caller's workspace too small
#define MOE_EUNSUPPORTED 4

namespace moe {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// hipGetLastError() after a launch; returns MOE_OK or MOE_EHIP with the message set
int check_launch(const char* what);

__host__ __device__ inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Pointers in the global address space: loads through them are global_load_*
// (counted by vmcnt only), not flat loads, even when the address came from memory.
#define MOE_GLOBAL __attribute__((address_space(1)))

template <class T>
__device__ __forceinline__ const MOE_GLOBAL T* gptr(const void* p) {
  return (const MOE_GLOBAL T*)(uintptr_t)p;
}

// 16 bytes that are read once: a non-temporal 128-bit global load
__device__ __forceinline__ uint4 stream_load16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(gptr<u32x4>(p));
  return uint4{v.x, v.y, v.z, v.w};
}

// ---------------------------------------------------------------- device helpers

// An empty asm that hides a value's known bits from the optimiser, so
// (v >> 8k) & 0xFF on a nibble-masked word maps to one v_cvt_f32_ubyteK.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ float ubyte(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return __half2float(__ushort_as_half((unsigned short)h));
}

// Group scales are f16 or f32, chosen per call.
__device__ __forceinline__ float load_scale(const void* s, size_t idx, int f16) {
  return f16 ? half_bits_to_float(reinterpret_cast<const uint16_t*>(s)[idx])
             : reinterpret_cast<const float*>(s)[idx];
}

// GGUF f16 fields: llama.cpp-style decode, except that exponent 31 (Inf and NaN)
// reads as a signed infinity (moelan/kernels.py:244-255).
__device__ __forceinline__ float gguf_half(uint32_t h) {
  if ((h & 0x7C00u) == 0x7C00u) return (h & 0x8000u) ? -INFINITY : INFINITY;
  return half_bits_to_float(h);
}

// g / (1 + e^-g) with the hardware exp and reciprocal (a few ulp; no IEEE divide)
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

template <int CTRL, int ROWMASK, bool BC>
__device__ __forceinline__ float dpp_read(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xf, BC));
}

// lane L-1 of every aligned group of L lanes (L = 8, 16, 32, 64) receives the group's sum
template <int L>
__device__ __forceinline__ float lane_group_sum(float v) {
  v += dpp_read<0x111, 0xf, true>(v);  // row_shr:1
  v += dpp_read<0x112, 0xf, true>(v);  // row_shr:2
  v += dpp_read<0x114, 0xf, true>(v);  // row_shr:4
  if constexpr (L >= 16) v += dpp_read<0x118, 0xf, true>(v);   // row_shr:8
  if constexpr (L >= 32) v += dpp_read<0x142, 0xa, false>(v);  // row_bcast:15 into rows 1, 3
  if constexpr (L >= 64) v += dpp_read<0x143, 0xc, false>(v);  // row_bcast:31 into rows 2, 3
  return v;
}

// sum over aligned groups of `width` lanes (width a power of two <= 64)
__device__ __forceinline__ float group_sum(float v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Workgroups are dispatched round-robin over the chip's 8 XCDs (each with its
// own L2): workgroup b runs on XCD b % 8. Returns the logical index for b so
// that each XCD receives one contiguous range of logical indices (work that
// shares operands then shares an L2). A bijection on [0, total).
__device__ __forceinline__ int xcd_contiguous(int b, int total) {
  constexpr int kXcds = 8;
  const int x = b % kXcds, slot = b / kXcds, base = total / kXcds, rem = total % kXcds;
  return x * base + (x < rem ? x : rem) + slot;
}

}  // namespace moe
