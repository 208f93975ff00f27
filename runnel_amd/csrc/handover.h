// Hand-overs between workgroups of one launch through tagged words, with
// bounded waits (the single-launch decode, the few-token router): a word is
// (bf16 value << 16) | tag, the tag of the call's phase, so a word holds
// either the value of the current phase or something a reader can tell
// apart; every wait gives up after a round limit, or once another workgroup
// of the call has given up, and records the call's failure in the scratch's
// status word.
#pragma once

#include "kernels.h"

namespace rmoe {

constexpr int kSpinLimit = 1 << 20;
constexpr int kAbortCheck = 64;  // rounds between reads of the abort word

__device__ __forceinline__ void store_coherent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_coherent_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t tagged(uint32_t bf16_bits, uint32_t tag) {
  return (bf16_bits << 16) | (tag & 0xFFFFu);
}
__device__ __forceinline__ bool tag_ok(uint32_t word, uint32_t tag) {
  return (word & 0xFFFFu) == (tag & 0xFFFFu);
}
// Tag of a phase: 1 .. 65535 (0 is the tag of zero-filled scratch).
__device__ __forceinline__ uint32_t phase_tag(uint32_t phase) { return phase % 65535u + 1u; }

// State of one wave's bounded waits in one call: the call's abort key (its
// first phase, never 0) and whether the wave has given up.
struct WaitState {
  FusedScratch* sc;
  uint32_t key;
  bool gave_up;
};
__device__ __forceinline__ void publish_failure(FusedScratch* sc, uint32_t key, uint32_t status) {
  __hip_atomic_fetch_max(&sc->err, status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&sc->abort, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Called after a round that left words pending: true when the wave stops
// waiting (round limit, or another workgroup gave up a wait of this call).
__device__ __forceinline__ bool give_up(WaitState& w, int spin) {
  const bool stop =
      spin >= kSpinLimit ||
      ((spin & (kAbortCheck - 1)) == kAbortCheck - 1 &&
       __hip_atomic_load(&w.sc->abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == w.key);
  if (stop) {
    if (!w.gave_up) publish_failure(w.sc, w.key, 1u);
    w.gave_up = true;
  }
  return stop;
}

}  // namespace rmoe
