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
// Butterfly p <- p + p[lane ^ d], d = 1, 2, 4, 8, 16, 32: every lane ends
// with the same value, and the order of additions is fixed (the router's
// bit-exact contract relies on it).  Reference form; wave_sum below is the
// fast equivalent.
__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int d = 1; d <= 32; d <<= 1) v += __shfl_xor(v, d, kWave);
  return v;
}
// Sum within aligned segments of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float segment_sum(float v, int width) {
  for (int d = 1; d < width; d <<= 1) v += __shfl_xor(v, d, kWave);
  return v;
}
// The same butterfly with cheap cross-lane operations.  After each level
// every lane of a block holds the same value, so adding the mirrored
// partner (DPP row_half_mirror / row_mirror) or the swizzled one gives the
// exact value the xor partner would: the results equal wave_sum_butterfly
// bit for bit.
__device__ __forceinline__ float dpp_f(float v, int ctrl) {
  int r;
  switch (ctrl) {  // the control must be a compile-time constant
    case 0xB1: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false); break;
    case 0x4E: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false); break;
    case 0x141: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false); break;
    default: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false); break;
  }
  return __int_as_float(r);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f(v, 0xB1);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp_f(v, 0x4E);   // quad_perm [2,3,0,1]: lane ^ 2
  v += dpp_f(v, 0x141);  // row_half_mirror: the other quad of the 8
  v += dpp_f(v, 0x140);  // row_mirror: the other 8 of the row
  // ds_swizzle bit mode, xor 16 within each 32 lanes
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}
// Sum within aligned segments of `width` lanes (a power of two, 1..64) with
// the same butterfly order; every lane of a segment gets the segment sum.
__device__ __forceinline__ float segment_sum_fast(float v, int width) {
  if (width >= 2) v += dpp_f(v, 0xB1);
  if (width >= 4) v += dpp_f(v, 0x4E);
  if (width >= 8) v += dpp_f(v, 0x141);
  if (width >= 16) v += dpp_f(v, 0x140);
  if (width >= 32)
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  if (width >= 64)
    v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return v;
}

// Wave maximum of unsigned keys: rows of 16 by DPP, then across row pairs
// and halves with the gfx950 permlane swaps (VALU, no LDS round trip);
// every lane ends with the maximum.
__device__ __forceinline__ uint32_t dpp_u(uint32_t v, int ctrl) {
  switch (ctrl) {
    case 0xB1: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
    case 0x4E: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
    case 0x141: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false);
    default: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false);
  }
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u(v, 0xB1));
  v = max(v, dpp_u(v, 0x4E));
  v = max(v, dpp_u(v, 0x141));
  v = max(v, dpp_u(v, 0x140));
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(a[0], a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(b[0], b[1]);
}

// Each lane's P keys in descending order (odd-even transposition network).
template <int P>
__device__ __forceinline__ void sort_desc(uint32_t (&k)[P]) {
#pragma unroll
  for (int r = 0; r < P; ++r)
#pragma unroll
    for (int i = r & 1; i + 1 < P; i += 2) {
      const uint32_t hi = k[i] > k[i + 1] ? k[i] : k[i + 1];
      const uint32_t lo = k[i] > k[i + 1] ? k[i + 1] : k[i];
      k[i] = hi;
      k[i + 1] = lo;
    }
}

// The lanes whose largest remaining key equals `best` drop it.
template <int P>
__device__ __forceinline__ void pop_head(uint32_t (&k)[P], uint32_t best) {
  if (k[0] == best) {
#pragma unroll
    for (int i = 0; i + 1 < P; ++i) k[i] = k[i + 1];
    k[P - 1] = 0;
  }
}

// ------------------------------------------------------------ top-k keys
// Keys are unique and nonzero: (bf16 order key << 16) | (0xFFFF - index), so
// "larger key" = larger logit, then lower index.  The k largest of the P
// keys per lane (absent keys are 0): each lane sorts its keys, then k
// rounds of a wave maximum over the lanes' largest remaining keys.  Must be
// called by a whole wave; returns, in lane j < k, the key of rank j
// (descending).  (A 32-step ballot search for the k-th key took about
// three times as long: every step waits for a compare, a ballot and a
// scalar count in turn.)
template <int P>
__device__ __forceinline__ uint32_t wave_topk(uint32_t (&keys)[P], int k) {
  const int lane = threadIdx.x & 63;
  sort_desc<P>(keys);
  uint32_t mine = 0;
  for (int j = 0; j < k; ++j) {
    const uint32_t best = wave_max_u32(keys[0]);
    if (lane == j) mine = best;
    pop_head<P>(keys, best);
  }
  return mine;
}

// The k-th largest of the P keys per lane counted with multiplicity (keys
// may repeat; absent keys are 0): rounds of a wave maximum over the lanes'
// largest remaining keys, every lane holding that maximum dropping it,
// until k keys have been dropped (at most k rounds).
template <int P>
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t (&keys)[P], int k) {
  sort_desc<P>(keys);
  int taken = 0;
  uint32_t best = 0;
  while (taken < k) {
    best = wave_max_u32(keys[0]);
    taken += __popcll(__ballot(keys[0] == best));
    pop_head<P>(keys, best);
  }
  return best;
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

// Keep the compiler from moving loads or their uses across this point, so
// that every load of a batch is issued before the first wait on any of them.
__device__ __forceinline__ void issue_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// One 16-byte chunk (16 codes) of an 8-bit MLX-affine gate row folded into
// a router lane's partial, in the fixed order of the quantized router
// contract: qa = sum q_i v_i and xs = sum v_i, each sequential from +0 (the
// products are exact), then acc = fma(qa, s, acc), acc = fma(xs, b, acc)
// with the chunk's group scale and bias.
__device__ __forceinline__ float qgate_chunk(float acc, const uint4 w, const float* v, float s,
                                             float b) {
  const float qa = qdot_chunk<8>(w, v);
  float xs = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) xs += v[i];
  acc = fmaf(qa, s, acc);
  return fmaf(xs, b, acc);
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

// Cross-workgroup hand-off without whole-cache maintenance.  Each XCD has a
// private L2, and an agent-scope release/acquire fence writes back or
// invalidates that entire L2 (microseconds per wave).  Instead, the few
// values handed over are stored and loaded with agent-scope atomics, which
// are coherent on their own (write-through / bypassing stale lines); the
// producer waits for its stores to be acknowledged before bumping the
// counter.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }
__device__ __forceinline__ uint32_t atomic_add_agent(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace rmoe
