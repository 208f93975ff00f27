// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rmoe.h"

namespace rmoe {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 bits
__device__ __forceinline__ float bf16_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __uint_as_float(packed & 0xFFFF0000u);
}
// Round-to-nearest-even; NaN/Inf truncated (same rule as the host oracle).
__device__ __forceinline__ uint32_t f32_to_bf16(float v) {
  const uint32_t u = __float_as_uint(v);
  if (((u >> 23) & 0xFFu) == 0xFFu) return u >> 16;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float round_bf16(float v) {
  return bf16_to_f32(f32_to_bf16(v));
}

// ------------------------------------------------------- wave reductions
// Butterfly p <- p + p[lane ^ d], d = 32..1: every lane ends with the same
// value, and the order of additions is fixed (the router relies on it).
__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}
// Sum within aligned segments of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float segment_sum(float v, int width) {
  for (int d = width >> 1; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const uint32_t o = __shfl_xor(v, d, kWave);
    v = o > v ? o : v;
  }
  return v;
}

// ------------------------------------------------------- packed dot chunks
// One 16-byte chunk of a packed row against the matching activations.
// 8-bit: 16 codes; 4-bit: 32 codes.  Returns sum_i q_i * v_i in fp32.
__device__ __forceinline__ float qdot_word8(uint32_t w, float a0, float a1,
                                            float a2, float a3, float acc) {
  acc = fmaf((float)(w & 0xFFu), a0, acc);
  acc = fmaf((float)((w >> 8) & 0xFFu), a1, acc);
  acc = fmaf((float)((w >> 16) & 0xFFu), a2, acc);
  acc = fmaf((float)(w >> 24), a3, acc);
  return acc;
}

template <int BITS>
__device__ __forceinline__ float qdot_chunk(const uint4 w, const float* v) {
  float acc = 0.0f;
  if constexpr (BITS == 8) {
    acc = qdot_word8(w.x, v[0], v[1], v[2], v[3], acc);
    acc = qdot_word8(w.y, v[4], v[5], v[6], v[7], acc);
    acc = qdot_word8(w.z, v[8], v[9], v[10], v[11], acc);
    acc = qdot_word8(w.w, v[12], v[13], v[14], v[15], acc);
  } else {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // Even nibbles land in the low nibble of each byte, odd ones in the
      // high nibble: two masks give byte-aligned codes for v_cvt_f32_ubyteN.
      const uint32_t lo = words[i] & 0x0F0F0F0Fu;
      const uint32_t hi = (words[i] >> 4) & 0x0F0F0F0Fu;
      const float* a = v + 8 * i;
      acc = fmaf((float)(lo & 0xFFu), a[0], acc);
      acc = fmaf((float)(hi & 0xFFu), a[1], acc);
      acc = fmaf((float)((lo >> 8) & 0xFFu), a[2], acc);
      acc = fmaf((float)((hi >> 8) & 0xFFu), a[3], acc);
      acc = fmaf((float)((lo >> 16) & 0xFFu), a[4], acc);
      acc = fmaf((float)((hi >> 16) & 0xFFu), a[5], acc);
      acc = fmaf((float)(lo >> 24), a[6], acc);
      acc = fmaf((float)(hi >> 24), a[7], acc);
    }
  }
  return acc;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
// Streaming load for weights read exactly once per call: non-temporal hint
// keeps them from evicting the activations and small tables from L2.
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }
__device__ __forceinline__ float sigmoid(float g) { return 1.0f / (1.0f + __expf(-g)); }

// Order-preserving 16-bit key of a bf16 value (-0 folded onto +0, so equal
// values compare equal exactly as float comparison does).
__device__ __forceinline__ uint32_t bf16_order_key(uint32_t b) {
  b &= 0xFFFFu;
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}
__device__ __forceinline__ uint32_t bf16_from_order_key(uint32_t k) {
  k &= 0xFFFFu;
  return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
}

// Agent-scope release / acquire around workgroup hand-offs (the L2 of each
// XCD is private, so plain stores need the release before a counter bump and
// readers need the acquire after observing it).
__device__ __forceinline__ void fence_release() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}
__device__ __forceinline__ void fence_acquire() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}
__device__ __forceinline__ uint32_t atomic_add_acq_rel(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace rmoe
