// Decode-shaped kernels of the MoE block for gfx950 (wave64).
//
//   router_kernel   one wave per router row (fixed-order bf16 dot), then the
//                   last workgroup of each token ranks the logits with wave
//                   ballots/maxima: top-k, softmax, renormalisation, shared
//                   sigmoid gate.
//   gate_up_kernel  one wave per (up row c, gate row c + I) pair of one
//                   selected expert: 16-byte streaming loads, dequantised in
//                   registers, SwiGLU in the epilogue.  The shared expert is
//                   the (k+1)-th unit of every token.
//   down_kernel     one wave per group of output rows, all units of a token:
//                   the router-weighted combine and the gated shared expert
//                   are summed in registers, bf16 written once.
//   qmv_kernel      plain gather-QMV (mx.gather_qmm at M rows).
#include "common.h"
#include "handover.h"
#include "kernels.h"

namespace rmoe {

// --------------------------------------------------------------- few tokens
// Calls of 2..8 tokens below the expert-sorted threshold (T K < 64) at the
// single-launch shapes (hidden 2048, intermediate 512, 8-bit experts).  The
// waves of each launch are resident at once (one round at up to 4 tokens):
// a wave issues the loads of all its rows first and computes each row as
// it lands, so the dequantisation runs under the stream instead of after
// it.  The router launch also computes the shared expert's gate/up (which
// does not depend on the routing), every pair for every token; the
// activations go to the down kernel as bf16 (they are bf16-valued).
namespace few {
constexpr int H = kFusedH;
constexpr int I = kFusedI;
constexpr int G = H / 64;                 // groups per gate/up row (32)
// gate/up pairs per wave: small waves, many per SIMD (4 tokens through 40
// layers from HBM, us per layer call: 8 pairs 42.0, 4 pairs 34.7, 2 pairs 30.5)
constexpr int NP = 2;
constexpr int kWavesPerUnit = I / NP;
constexpr int kSharedPairs = 1;           // router launch: shared pairs per wave
constexpr int kSharedBlocks = I / (4 * kSharedPairs);  // 128

template <int BITS>
struct Shape {
  static constexpr int VPC = BITS == 8 ? 16 : 32;   // values per 16-byte chunk
  static constexpr int CPL = H / VPC / 64;          // chunks per lane: 2 | 1
  static constexpr int WPR = H * BITS / 32;         // words per gate/up row
};
}  // namespace few

// N (up, gate) pairs of a bank: per pair one 4-byte word per lane that,
// over the wave, holds every scale and bias of both rows (lanes 0-15 up
// scales, 16-31 gate scales, 32-47 up biases, 48-63 gate biases: 16 words
// = a row's 32 groups), and the packed chunks lane + 64 i of both rows.
template <int BITS, int N>
struct FewPairs {
  uint4 wu[N][few::Shape<BITS>::CPL], wg[N][few::Shape<BITS>::CPL];
  uint32_t pw[N];
};

// The parameter words first (small), then the packed rows in pair order.
template <int BITS, int N>
__device__ __forceinline__ void few_load_pairs(FewPairs<BITS, N>& r, const QW& q, size_t up0,
                                               int lane) {
  using S = few::Shape<BITS>;
#pragma unroll
  for (int pp = 0; pp < N; ++pp) {
    const size_t row = up0 + pp + ((lane >> 4) & 1) * few::I;
    const uint16_t* base = (lane < 32 ? q.s : q.b) + row * few::G;
    r.pw[pp] = reinterpret_cast<const uint32_t*>(base)[lane & 15];
  }
#pragma unroll
  for (int pp = 0; pp < N; ++pp) {
#pragma unroll
    for (int i = 0; i < S::CPL; ++i) {
      const int ch = lane + 64 * i;
      r.wu[pp][i] = load16_stream(q.w + (up0 + pp) * S::WPR + ch * 4);
      r.wg[pp][i] = load16_stream(q.w + (up0 + pp + few::I) * S::WPR + ch * 4);
    }
  }
}

// Keeps the optimiser from converting the codes of every pair once, ahead
// of a loop over tokens (which held them all as floats and spilled).
template <int BITS, int N>
__device__ __forceinline__ void few_opaque(FewPairs<BITS, N>& r) {
#pragma unroll
  for (int pp = 0; pp < N; ++pp)
#pragma unroll
    for (int i = 0; i < few::Shape<BITS>::CPL; ++i)
      asm volatile("" : "+v"(r.wu[pp][i].x), "+v"(r.wu[pp][i].y), "+v"(r.wu[pp][i].z),
                   "+v"(r.wu[pp][i].w), "+v"(r.wg[pp][i].x), "+v"(r.wg[pp][i].y),
                   "+v"(r.wg[pp][i].z), "+v"(r.wg[pp][i].w));
}

// One token's x for the gate/up dot: chunks lane + 64 i as loaded (raw),
// then as floats with the chunk sums.
template <int BITS>
struct FewX {
  uint4 raw[few::Shape<BITS>::CPL][few::Shape<BITS>::VPC / 8];
  float v[few::Shape<BITS>::CPL][few::Shape<BITS>::VPC];
  float sum[few::Shape<BITS>::CPL];
};

template <int BITS>
__device__ __forceinline__ void few_load_x(uint4 (&raw)[few::Shape<BITS>::CPL]
                                                      [few::Shape<BITS>::VPC / 8],
                                           const uint16_t* xt, int lane) {
  using S = few::Shape<BITS>;
#pragma unroll
  for (int i = 0; i < S::CPL; ++i)
#pragma unroll
    for (int h = 0; h < S::VPC / 8; ++h) raw[i][h] = load16(xt + (lane + 64 * i) * S::VPC + h * 8);
}

template <int BITS>
__device__ __forceinline__ void few_unpack_x(FewX<BITS>& x,
                                             const uint4 (&raw)[few::Shape<BITS>::CPL]
                                                               [few::Shape<BITS>::VPC / 8]) {
  using S = few::Shape<BITS>;
#pragma unroll
  for (int i = 0; i < S::CPL; ++i) {
#pragma unroll
    for (int h = 0; h < S::VPC / 8; ++h) {
      const uint4 b = raw[i][h];
      x.v[i][h * 8 + 0] = bf16_lo(b.x);
      x.v[i][h * 8 + 1] = bf16_hi(b.x);
      x.v[i][h * 8 + 2] = bf16_lo(b.y);
      x.v[i][h * 8 + 3] = bf16_hi(b.y);
      x.v[i][h * 8 + 4] = bf16_lo(b.z);
      x.v[i][h * 8 + 5] = bf16_hi(b.z);
      x.v[i][h * 8 + 6] = bf16_lo(b.w);
      x.v[i][h * 8 + 7] = bf16_hi(b.w);
    }
    x.sum[i] = 0.0f;
#pragma unroll
    for (int v = 0; v < S::VPC; ++v) x.sum[i] += x.v[i][v];
  }
}

// bf16 value of group g from the parameter word spread over lanes
// [first, first + 16): word g / 2, half g % 2.
__device__ __forceinline__ float few_param(uint32_t word, int first, int g) {
  const uint32_t w = (uint32_t)__shfl((int)word, first + (g >> 1), 64);
  return __uint_as_float((g & 1) ? (w & 0xFFFF0000u) : (w << 16));
}

// One (up, gate) pair's packed chunks.
template <int BITS>
struct FewPair {
  uint4 wu[few::Shape<BITS>::CPL], wg[few::Shape<BITS>::CPL];
};

template <int BITS>
__device__ __forceinline__ void few_load_pair(FewPair<BITS>& r, const QW& q, size_t up_row,
                                              int lane) {
  using S = few::Shape<BITS>;
#pragma unroll
  for (int i = 0; i < S::CPL; ++i) {
    const int ch = lane + 64 * i;
    r.wu[i] = load16_stream(q.w + up_row * S::WPR + ch * 4);
    r.wg[i] = load16_stream(q.w + (up_row + few::I) * S::WPR + ch * 4);
  }
}

// bf16 bits of bf16(silu(bf16(gate)) * bf16(up)) of one pair (every lane).
template <int BITS>
__device__ __forceinline__ uint32_t few_pair_act(const FewPair<BITS>& r, uint32_t pw,
                                                 const FewX<BITS>& x, int lane) {
  using S = few::Shape<BITS>;
  float au = 0.0f, ag = 0.0f;
#pragma unroll
  for (int i = 0; i < S::CPL; ++i) {
    const int g = ((lane + 64 * i) * S::VPC) >> 6;
    au += few_param(pw, 0, g) * qdot_chunk<BITS>(r.wu[i], x.v[i]) + few_param(pw, 32, g) * x.sum[i];
    ag += few_param(pw, 16, g) * qdot_chunk<BITS>(r.wg[i], x.v[i]) + few_param(pw, 48, g) * x.sum[i];
  }
  au = wave_sum(au);
  ag = wave_sum(ag);
  return f32_to_bf16(silu(round_bf16(ag)) * round_bf16(au));
}

// SwiGLU activations of N pairs against one token: lane pp < N returns the
// bf16 bits of pair pp's bf16(silu(bf16(gate)) * bf16(up)).
template <int BITS, int N>
__device__ __forceinline__ uint32_t few_pair_acts(const FewPairs<BITS, N>& r,
                                                  const FewX<BITS>& x, int lane) {
  using S = few::Shape<BITS>;
  uint32_t res = 0;
#pragma unroll
  for (int pp = 0; pp < N; ++pp) {
    float au = 0.0f, ag = 0.0f;
#pragma unroll
    for (int i = 0; i < S::CPL; ++i) {
      const int g = ((lane + 64 * i) * S::VPC) >> 6;
      au += few_param(r.pw[pp], 0, g) * qdot_chunk<BITS>(r.wu[pp][i], x.v[i]) +
            few_param(r.pw[pp], 32, g) * x.sum[i];
      ag += few_param(r.pw[pp], 16, g) * qdot_chunk<BITS>(r.wg[pp][i], x.v[i]) +
            few_param(r.pw[pp], 48, g) * x.sum[i];
    }
    au = wave_sum(au);
    ag = wave_sum(ag);
    const uint32_t a = f32_to_bf16(silu(round_bf16(ag)) * round_bf16(au));
    res = lane == pp ? a : res;
    // one pair at a time: the unpacked codes of later pairs are not hoisted
    __builtin_amdgcn_sched_barrier(0);
  }
  return res;
}

// The router launch's shared-expert role: pairs c0 .. c0 + kSharedPairs - 1
// for every token (x of all tokens in flight at once).
template <int BITS>
__device__ __forceinline__ void few_shared_gate_up(const DecodeArgs& p, int c0, int lane) {
  using S = few::Shape<BITS>;
  constexpr int NS = few::kSharedPairs;
  const int U1 = p.K + 1;
  uint4 xr[kFewMaxTokens][S::CPL][S::VPC / 8];
#pragma unroll
  for (int t = 0; t < kFewMaxTokens; ++t)
    if (t < p.T) few_load_x<BITS>(xr[t], p.x + (size_t)t * few::H, lane);
  FewPairs<BITS, NS> pr;
  few_load_pairs<BITS, NS>(pr, p.sgu, (size_t)c0, lane);
  uint16_t* act = reinterpret_cast<uint16_t*>(p.act);
#pragma unroll
  for (int t = 0; t < kFewMaxTokens; ++t) {
    if (t < p.T) {
      FewX<BITS> x;
      few_unpack_x<BITS>(x, xr[t]);
      few_opaque(pr);
      const uint32_t a = few_pair_acts<BITS, NS>(pr, x, lane);
      if (lane < NS) act[((size_t)t * U1 + p.K) * few::I + c0 + lane] = (uint16_t)a;
    }
  }
}

// ------------------------------------------------------------------ router
// Ranking, softmax and scores of one token from its bf16-valued logits
// (lane + 64 i holds expert lane + 64 i; experts >= E are ignored) and the
// shared-expert gate's fp32 logit.  One wave.
template <int P>
__device__ __forceinline__ void finish_route(const DecodeArgs& p, int t, const float (&lv)[P],
                                             float sg_logit) {
  const int lane = threadIdx.x & 63;
  uint32_t keys[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int e = lane + 64 * i;
    keys[i] = e < p.E ? (bf16_order_key(f32_to_bf16(lv[i])) << 16) | (0xFFFFu - (uint32_t)e)
                      : 0u;
  }
  const uint32_t my_key = wave_topk<P>(keys, p.K);
  const uint32_t top_key = __builtin_amdgcn_readfirstlane(my_key);
  const float m = bf16_to_f32(bf16_from_order_key(top_key >> 16));
  float z = 0.0f;
#pragma unroll
  for (int i = 0; i < P; ++i)
    if (lane + 64 * i < p.E) z += __expf(lv[i] - m);
  z = wave_sum(z);
  const int my_sel = (int)(0xFFFFu - (my_key & 0xFFFFu));
  const float my_logit = bf16_to_f32(bf16_from_order_key(my_key >> 16));
  float pb = 0.0f;
  if (lane < p.K) pb = round_bf16(__expf(my_logit - m) / z);
  float total = 0.0f;
  for (int j = 0; j < p.K; ++j)
    total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pb), j));
  // the denominator is bf16, as mlx-lm's scores.sum(-1) of bf16 scores
  const float score = p.norm ? round_bf16(pb / round_bf16(total)) : pb;
  if (lane < p.K) {
    p.idx[t * p.K + lane] = my_sel;
    p.scores[t * (p.K + 1) + lane] = score;
    if (p.idx_out) p.idx_out[t * p.K + lane] = my_sel;
    if (p.scores_out) p.scores_out[t * p.K + lane] = score;
  }
  if (lane == 0) {
    float sg = 1.0f;
    if (p.has_sg) sg = round_bf16(sigmoid(round_bf16(sg_logit)));
    p.scores[t * (p.K + 1) + p.K] = sg;
  }
}

// One lane's partials of a bf16 gate row (the router contract) for TB
// tokens (rows x, x + xs, ...; tokens >= nt are skipped): chunks lane + 64 i
// of 8 values, element by element.  The row is loaded once for all tokens;
// all loads of a batch are issued before the first multiply (one memory
// round trip per batch).
template <int TB>
__device__ __forceinline__ void bf16_gate_partials(const uint16_t* wr, const uint16_t* x,
                                                   size_t xs, int nt, int H, int lane,
                                                   float (&acc)[TB]) {
#pragma unroll
  for (int k = 0; k < TB; ++k) acc[k] = 0.0f;
  const int chunks = H >> 3;
  for (int c0 = lane; c0 < chunks; c0 += 64 * kRouterBatch) {
    uint4 wv[kRouterBatch], xv[TB][kRouterBatch];
#pragma unroll
    for (int i = 0; i < kRouterBatch; ++i) {
      const int c = c0 + 64 * i;
      wv[i] = make_uint4(0, 0, 0, 0);
      // (the default cache policy: a layer's router rows are read every
      // call, and the memory-side cache keeps some of them between calls;
      // 4 tokens through the 40-layer stack 28.45 -> 28.22 us per layer call)
      if (c < chunks) wv[i] = load16(wr + c * 8);
#pragma unroll
      for (int k = 0; k < TB; ++k) {
        xv[k][i] = make_uint4(0, 0, 0, 0);
        if (c < chunks && k < nt) xv[k][i] = load16(x + k * xs + c * 8);
      }
    }
#pragma unroll
    for (int k = 0; k < TB; ++k) {
#pragma unroll
      for (int i = 0; i < kRouterBatch; ++i) {
        if (c0 + 64 * i < chunks) {
          float a = acc[k];
          const uint4 v = xv[k][i], w = wv[i];
          a = fmaf(bf16_lo(v.x), bf16_lo(w.x), a);
          a = fmaf(bf16_hi(v.x), bf16_hi(w.x), a);
          a = fmaf(bf16_lo(v.y), bf16_lo(w.y), a);
          a = fmaf(bf16_hi(v.y), bf16_hi(w.y), a);
          a = fmaf(bf16_lo(v.z), bf16_lo(w.z), a);
          a = fmaf(bf16_hi(v.z), bf16_hi(w.z), a);
          a = fmaf(bf16_lo(v.w), bf16_lo(w.w), a);
          a = fmaf(bf16_hi(v.w), bf16_hi(w.w), a);
          acc[k] = a;
        }
      }
    }
  }
}

// 16 bf16 inputs (two 16-byte pieces) as floats.
__device__ __forceinline__ void unpack_x16(const uint4 a, const uint4 b, float (&v)[16]) {
  const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[2 * i] = bf16_lo(u[i]);
    v[2 * i + 1] = bf16_hi(u[i]);
  }
}

// One lane's partials of row `row` of an 8-bit MLX-affine gate bank (the
// quantized router contract) for TB tokens: chunks lane + 64 i of 16 codes.
template <int TB>
__device__ __forceinline__ void q8_gate_partials(const QW& bank, size_t row, const uint16_t* x,
                                                 size_t xs, int nt, int H, int lane,
                                                 float (&acc)[TB]) {
#pragma unroll
  for (int k = 0; k < TB; ++k) acc[k] = 0.0f;
  const int chunks = H >> 4;
  const uint32_t* wr = bank.w + row * (size_t)(H >> 2);
  const uint16_t* sr = bank.s + row * (size_t)(H >> 6);
  const uint16_t* br = bank.b + row * (size_t)(H >> 6);
  for (int c0 = lane; c0 < chunks; c0 += 64 * kRouterBatch) {
    uint4 wv[kRouterBatch], xa[TB][kRouterBatch], xb[TB][kRouterBatch];
    uint32_t sv[kRouterBatch], bv[kRouterBatch];
#pragma unroll
    for (int i = 0; i < kRouterBatch; ++i) {
      const int c = c0 + 64 * i;
      wv[i] = make_uint4(0, 0, 0, 0);
      sv[i] = bv[i] = 0;
      if (c < chunks) {
        wv[i] = load16(wr + c * 4);  // (default cache policy, as above)
        sv[i] = sr[c >> 2];
        bv[i] = br[c >> 2];
      }
#pragma unroll
      for (int k = 0; k < TB; ++k) {
        xa[k][i] = xb[k][i] = make_uint4(0, 0, 0, 0);
        if (c < chunks && k < nt) {
          xa[k][i] = load16(x + k * xs + c * 16);
          xb[k][i] = load16(x + k * xs + c * 16 + 8);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < TB; ++k) {
#pragma unroll
      for (int i = 0; i < kRouterBatch; ++i) {
        if (c0 + 64 * i < chunks) {
          float v[16];
          unpack_x16(xa[k][i], xb[k][i], v);
          acc[k] = qgate_chunk(acc[k], wv[i], v, bf16_to_f32(sv[i]), bf16_to_f32(bv[i]));
        }
      }
    }
  }
}

// One wave per router row and group of TB tokens (grid.y): the row is
// streamed once for the group.  The last workgroup of a group ranks its
// tokens, one wave per token.  With the few-token kernels (SB != 0) the
// logits go over as tagged words instead (bf16 | tag of the call, read from
// the epoch word, which the gate/up launch after this one advances): each
// row's wave stores its words without waiting for them to land, and
// workgroup 0 of the group polls its tokens' words (bounded, like every
// wait of the single-launch decode; a failed wait sets the status word) and
// ranks them as soon as they are in, one wave per token: no acknowledged
// stores, no counter.
template <int P, int TB, int SB>
__global__ __launch_bounds__(256) void router_kernel(const DecodeArgs p) {
  static_assert(TB >= 1 && TB <= 4, "one ranking wave per token");
  const int n_row_blocks = (p.E + p.has_sg + 3) / 4;
  if constexpr (SB != 0) {
    // workgroups past the router rows (token group 0 only): the shared
    // expert's gate/up of every token
    if ((int)blockIdx.x >= n_row_blocks) {
      if (blockIdx.y == 0)
        few_shared_gate_up<SB>(p, ((blockIdx.x - n_row_blocks) * 4 + (threadIdx.x >> 6)) *
                                      few::kSharedPairs,
                               threadIdx.x & 63);
      return;
    }
  }
  const int g = blockIdx.y;
  const int t0 = g * TB;
  const int nt = p.T - t0 < TB ? p.T - t0 : TB;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int has_sg = p.has_sg;
  const int R = p.E + has_sg;
  const int row = blockIdx.x * 4 + wave;
  const size_t ls = (size_t)(p.E + 1);
  // (the few-token path's words: their own area of the single-launch
  // scratch, never written by the other routers, whose fp32 logits could
  // carry any low half)
  uint32_t* const words = SB != 0 ? &p.fs->few[0][0] : reinterpret_cast<uint32_t*>(p.logits);
  uint32_t base = 0;
  if constexpr (SB != 0) base = load_coherent_u32(&p.fs->epoch);
  const uint32_t tag = phase_tag(base + 1);
  if (row < R) {
    float acc[TB];
    const uint16_t* xt = p.x + (size_t)t0 * p.H;
    if (p.rq8)
      q8_gate_partials<TB>(row < p.E ? p.rq : p.sgq, row < p.E ? (size_t)row : 0, xt,
                           (size_t)p.H, nt, p.H, lane, acc);
    else
      bf16_gate_partials<TB>(row < p.E ? p.router_w + (size_t)row * p.H : p.sgate_w, xt,
                             (size_t)p.H, nt, p.H, lane, acc);
#pragma unroll
    for (int k = 0; k < TB; ++k) {
      if (k < nt) {
        const float v = wave_sum(acc[k]);
        if (lane == 0) {
          if constexpr (SB != 0)
            store_coherent_u32(words + (t0 + k) * ls + row, tagged(f32_to_bf16(v), tag));
          else
            store_coherent(p.logits + (t0 + k) * ls + row, v);
        }
      }
    }
  }

  if constexpr (SB != 0) {
    // Workgroup 0 of the group: wave w ranks token t0 + w.
    if (blockIdx.x != 0 || wave >= nt) return;
    const int t = t0 + wave;
    const uint32_t* lw = words + t * ls;
    WaitState ws{p.fs, base + 1, false};
    // a call whose key the host has written into the abort word beforehand
    // waits for nothing (status 1)
    if (load_coherent_u32(&p.fs->abort) == ws.key) {
      ws.gave_up = true;
      if (lane == 0) publish_failure(p.fs, ws.key, 1u);
    }
    uint32_t w[P], wsg = 0;
    uint32_t pend = 0;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      w[i] = 0;
      if (lane + 64 * i < p.E) pend |= 1u << i;
    }
    if (lane == 0 && has_sg) pend |= 1u << P;
    if (ws.gave_up) pend = 0;
    for (int spin = 0;; ++spin) {
#pragma unroll
      for (int i = 0; i < P; ++i)
        if ((pend >> i) & 1u) w[i] = load_coherent_u32(lw + lane + 64 * i);
      if ((pend >> P) & 1u) wsg = load_coherent_u32(lw + p.E);
#pragma unroll
      for (int i = 0; i < P; ++i)
        if (((pend >> i) & 1u) && tag_ok(w[i], tag)) pend &= ~(1u << i);
      if (((pend >> P) & 1u) && tag_ok(wsg, tag)) pend &= ~(1u << P);
      if (!__any(pend != 0u)) break;
      if (give_up(ws, spin)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    float lv[P];
#pragma unroll
    for (int i = 0; i < P; ++i)
      lv[i] = lane + 64 * i < p.E ? __uint_as_float(w[i] & 0xFFFF0000u) : 0.0f;
    // Every word seen is cleared (tag 0 is never current), so a later call
    // can only find 0 or its own words there, whatever its tag; a word
    // still pending after a failed wait stays (the epoch moves on).
    if (!ws.gave_up) {
#pragma unroll
      for (int i = 0; i < P; ++i)
        if (lane + 64 * i < p.E) store_coherent_u32(words + t * ls + lane + 64 * i, 0u);
      if (lane == 0 && has_sg) store_coherent_u32(words + t * ls + p.E, 0u);
    }
    // (lane 0 holds the shared gate's word; only lane 0 uses it)
    finish_route<P>(p, t, lv, __uint_as_float(wsg & 0xFFFF0000u));
    return;
  }

  // Last workgroup of this token group ranks the logits.
  __shared__ uint32_t s_last;
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomic_add_agent(&p.ctr[g], 1u);
    s_last = (prev == (uint32_t)n_row_blocks - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (s_last == 0u || wave >= nt) return;

  const int t = t0 + wave;
  const float* lg = p.logits + t * ls;
  float lv[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int e = lane + 64 * i;
    lv[i] = e < p.E ? round_bf16(load_coherent(lg + e)) : 0.0f;
  }
  const float sg_logit = has_sg ? load_coherent(lg + p.E) : 0.0f;
  finish_route<P>(p, t, lv, sg_logit);
  if (wave == 0 && lane == 0)
    __hip_atomic_store(&p.ctr[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------ prefill router (MFMA)
// For many tokens the router is a [T, H] x [H, E] product.  The logits are
// computed on the matrix cores in fp32 (order of the hardware's choosing),
// then every token's selection is settled exactly.  For a bf16 gate:
//
//   |L - exact| <= (H - 1) 2^-23 S   any order of fp32 sums of the exact
//                                    bf16 products (round to nearest or
//                                    toward zero)
//   |c - exact| <= (H/64 + 8) 2^-24 S  the router contract's order
//   S = sum |x_k w_k| <= |x|_2 max_e |w_e|_2
//
// An 8-bit gate is first split into two bf16 planes, hi = bf16(w) and
// lo = bf16(w - hi) with w = fl32(q s + b), so |w - hi - lo| <= 2^-18 |w|;
// L sums the 2H products of x with both planes, and with
// S = sum |x_k| (|q_k s| + |b|) <= |x|_2 max_e || |q s| + |b| ||_2:
//
//   |L - exact| <= ((2H - 1) 2^-23 (1 + 2^-7) + 2^-17) S
//   |c - exact| <= (15 + 2 ceil(H / 1024) + 8) 2^-24 S   (quantized contract)
//
// so with delta the sum of both bounds (plus a denormal allowance), an
// expert whose L is more than margin = 2 delta + one bf16 ulp (at the
// largest logit's magnitude, padded) below the k-th largest L rounds to a
// bf16 logit strictly below those of k other experts and cannot be
// selected.  Every expert within the margin is recomputed in the contract
// order (the decode router's exact fp32 value); the ranking then runs on
// exact bf16 logits for all candidates.  Experts outside the margin keep
// bf16(L) (they only enter the softmax denominator).

// 8-bit gate rows as two bf16 planes hi = bf16(w), lo = bf16(w - hi) of
// w = fl32(q s + b) (w - hi is exact), and the row bound
// || |q s| + |b| ||_2.  One wave per row, 16 codes per lane and step.
__global__ __launch_bounds__(256) void router_split_kernel(const DecodeArgs p, uint16_t* hi,
                                                           uint16_t* lo, float* wnorm) {
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (e >= p.E) return;
  const int H = p.H;
  const uint32_t* wr = p.rq.w + (size_t)e * (H >> 2);
  const uint16_t* sr = p.rq.s + (size_t)e * (H >> 6);
  const uint16_t* br = p.rq.b + (size_t)e * (H >> 6);
  uint16_t* hr = hi + (size_t)e * H;
  uint16_t* lr = lo + (size_t)e * H;
  float n2 = 0.0f;
  for (int c = lane; c < (H >> 4); c += 64) {
    const uint4 w = load16(wr + c * 4);
    const float sc = bf16_to_f32(sr[c >> 2]);
    const float bi = bf16_to_f32(br[c >> 2]);
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    uint32_t ph[8], pl[8];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float q = (float)((words[j >> 2] >> (8 * (j & 3))) & 0xFFu);
      const float v = fmaf(q, sc, bi);                 // q s exact: one rounding
      const uint32_t h = f32_to_bf16(v);
      const uint32_t l = f32_to_bf16(v - bf16_to_f32(h));
      const float m = fabsf(q * sc) + fabsf(bi);
      n2 = fmaf(m, m, n2);
      if (j & 1) {
        ph[j >> 1] |= h << 16;
        pl[j >> 1] |= l << 16;
      } else {
        ph[j >> 1] = h;
        pl[j >> 1] = l;
      }
    }
    *reinterpret_cast<uint4*>(hr + c * 16) = make_uint4(ph[0], ph[1], ph[2], ph[3]);
    *reinterpret_cast<uint4*>(hr + c * 16 + 8) = make_uint4(ph[4], ph[5], ph[6], ph[7]);
    *reinterpret_cast<uint4*>(lr + c * 16) = make_uint4(pl[0], pl[1], pl[2], pl[3]);
    *reinterpret_cast<uint4*>(lr + c * 16 + 8) = make_uint4(pl[4], pl[5], pl[6], pl[7]);
  }
  n2 = wave_sum(n2);
  if (lane == 0) wnorm[e] = sqrtf(n2) * (1.0f + 1.0f / 1024.0f);
}

typedef __bf16 bf16x8_r __attribute__((ext_vector_type(8)));
typedef float f32x4_r __attribute__((ext_vector_type(4)));

// Matrix-core router logits: a workgroup computes BT tokens x BE experts over
// the whole of K.  Each stage of 64 k values of its BT token rows and BE
// router rows (128 bytes of each) arrives in LDS by LDS-DMA, eight lanes per
// row so that every load instruction fetches whole 128-byte lines; NB stage
// buffers, NB - 1 stages in flight.  Wave (wm, wn) of the WM x WN grid
// multiplies its (BT / WM) x (BE / WN) block from LDS fragments.  Loading
// the fragments straight into registers (16 rows x 64 bytes per instruction)
// took 35 us at 8192 tokens against 21 us for this kernel (13.5 against 11.7
// at 512 tokens; event-timed, 5.5 us of launch included).
//
// Stage layout (as the grouped GEMM's): row r holds 8 slots of 16 bytes,
// slot sl at position 8 r + (sl ^ f(r)), f(r) = (r & 7) ^ ((r >> 3) & 1), so
// the 16-row operand reads fall on distinct bank groups.  Slot 2 kg + j holds
// the 8 k values lane group kg feeds to k-step j; A and B share the layout,
// so the products pair equal k.  The waits are counted: every stage issues
// the same ND DMAs per wave (stages past the end reload the last one into a
// buffer nobody reads), so NB - 2 stages' loads may stay in flight when a
// stage's own copy is needed.
//
// ACC adds the sums already in `logits` (the second plane of a split gate).
// WNORM: the first token tile's workgroups also write the bound
// ||w_e||_2 (1 + 2^-10) of their router rows into wnorm from the fragments
// they read (the padding covers any order of the fp32 sum of squares).
__device__ __forceinline__ int stage_swizzle(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <int BT, int BE, int WM, int WN>
struct LogitsTile {
  static constexpr int WAVES = WM * WN, ROWS = BT + BE, NI = ROWS / 8, ND = NI / WAVES;
  static constexpr int MBW = BT / WM / 16, CBW = BE / WN / 16;
  static_assert(NI % WAVES == 0 && MBW >= 1 && CBW >= 1, "tile shape");
  static constexpr int vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
};

template <int BT, int BE, int WM, int WN, bool WNORM>
__device__ __forceinline__ void logits_stage(
    const uint16_t* __restrict__ buf, const int (&rd)[2], int arow0, int brow0,
    f32x4_r (&acc)[LogitsTile<BT, BE, WM, WN>::MBW][LogitsTile<BT, BE, WM, WN>::CBW],
    float (&ss)[LogitsTile<BT, BE, WM, WN>::CBW], bool norms) {
  using C = LogitsTile<BT, BE, WM, WN>;
  const char* b = reinterpret_cast<const char*>(buf);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    u32x4 bf[C::CBW];
#pragma unroll
    for (int cb = 0; cb < C::CBW; ++cb)
      bf[cb] = *reinterpret_cast<const u32x4*>(b + (brow0 + cb * 16) * 128 + rd[j]);
    if (WNORM && norms) {
#pragma unroll
      for (int cb = 0; cb < C::CBW; ++cb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ss[cb] = fmaf(bf16_lo(bf[cb][i]), bf16_lo(bf[cb][i]), ss[cb]);
          ss[cb] = fmaf(bf16_hi(bf[cb][i]), bf16_hi(bf[cb][i]), ss[cb]);
        }
    }
#pragma unroll
    for (int mb = 0; mb < C::MBW; ++mb) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(b + (arow0 + mb * 16) * 128 + rd[j]);
#pragma unroll
      for (int cb = 0; cb < C::CBW; ++cb)
        acc[mb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_r, a), __builtin_bit_cast(bf16x8_r, bf[cb]), acc[mb][cb], 0,
            0, 0);
    }
  }
}

template <int BT, int BE, int WM, int WN, int NB, bool ACC, bool WNORM>
__device__ __forceinline__ void router_logits_body(const DecodeArgs& p, float* wnorm,
                                                   uint16_t* __restrict__ s0,
                                                   uint16_t* __restrict__ s1,
                                                   uint16_t* __restrict__ s2,
                                                   uint16_t* __restrict__ s3) {
  using C = LogitsTile<BT, BE, WM, WN>;
  uint16_t* const sb[4] = {s0, s1, s2, s3};
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int kg = lane >> 4;
  const int t0 = blockIdx.x * BT, e0 = blockIdx.y * BE;
  const int trows = min(BT, p.T - t0);
  const int H = p.H;
  // resources based at the tile's first token / router row (offsets stay 32-bit)
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + (size_t)t0 * H), (short)0, trows * H * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.router_w + (size_t)e0 * H), (short)0, BE * H * 2, 0x00020000);
  // DMA ii of this wave covers stage rows 8 i .. 8 i + 7, i = wave + WAVES ii:
  // lane l fetches the slot that belongs at position l & 7 of row 8 i + l / 8
  uint32_t src[C::ND];
#pragma unroll
  for (int ii = 0; ii < C::ND; ++ii) {
    const int i = wave + C::WAVES * ii;
    const int r = 8 * i + (lane >> 3);
    const int sl = (lane & 7) ^ stage_swizzle(r);
    const int row = 8 * i >= BT ? r - BT : min(r, trows - 1);  // tokens past the end: the last
    src[ii] = ((uint32_t)row * H + sl * 8) * 2;
  }
  const int wm = wave % WM, wn = wave / WM;
  const int arow0 = wm * (BT / WM), brow0 = BT + wn * (BE / WN);
  int rd[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    rd[j] = ((lane & 15) * 8 + ((2 * kg + j) ^ stage_swizzle(lane & 15))) * 16;
  f32x4_r acc[C::MBW][C::CBW];
#pragma unroll
  for (int mb = 0; mb < C::MBW; ++mb)
#pragma unroll
    for (int cb = 0; cb < C::CBW; ++cb) acc[mb][cb] = f32x4_r{0.f, 0.f, 0.f, 0.f};
  float ss[C::CBW];
#pragma unroll
  for (int cb = 0; cb < C::CBW; ++cb) ss[cb] = 0.f;
  const bool norms = WNORM && blockIdx.x == 0 && wm == 0;
  // this workgroup's share of H (blockIdx.z of gridDim.z): stages c0 .. c0 + nst - 1
  const int nst = H / 64 / (int)gridDim.z;
  const int c0 = (int)blockIdx.z * nst;
  auto dma = [&](uint16_t* buf, int c) {
#pragma unroll
    for (int ii = 0; ii < C::ND; ++ii) {
      const int i = wave + C::WAVES * ii;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          8 * i >= BT ? rb : ra, (__attribute__((address_space(3))) void*)(buf + i * 512), 16,
          src[ii], (c0 + c) * 128, 0, 0);
    }
  };
#pragma unroll
  for (int q = 0; q < NB - 1; ++q) {
    __builtin_amdgcn_sched_barrier(0);
    dma(sb[q], min(q, nst - 1));
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(C::vmcnt((NB - 2) * C::ND));
  __builtin_amdgcn_s_barrier();
  for (int c = 0; c < nst; c += NB) {
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      if (c + q < nst) {
        __builtin_amdgcn_sched_barrier(0);
        dma(sb[(q + NB - 1) % NB], min(c + q + NB - 1, nst - 1));
        __builtin_amdgcn_sched_barrier(0);
        logits_stage<BT, BE, WM, WN, WNORM>(sb[q], rd, arow0, brow0, acc, ss, norms);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(C::vmcnt((NB - 2) * C::ND));
        __builtin_amdgcn_s_barrier();
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(C::vmcnt(0));  // the DMAs past the end have landed
  if (WNORM && norms) {
#pragma unroll
    for (int cb = 0; cb < C::CBW; ++cb) {
      float v = ss[cb];
      v += __shfl_xor(v, 16, kWave);
      v += __shfl_xor(v, 32, kWave);
      // this share's sum of squares (the selection adds the shares)
      if (kg == 0) wnorm[(size_t)blockIdx.z * p.E + e0 + brow0 - BT + cb * 16 + (lane & 15)] = v;
    }
  }
  // lane (col, kg) of block (mb, cb) holds tokens 4 kg + [0, 4) of expert col
#pragma unroll
  for (int mb = 0; mb < C::MBW; ++mb)
#pragma unroll
    for (int cb = 0; cb < C::CBW; ++cb) {
      const int e = e0 + brow0 - BT + cb * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + arow0 + mb * 16 + 4 * kg + i;
        if (t < p.T) {
          float* o = p.logits + ((size_t)blockIdx.z * p.T + t) * (p.E + 1) + e;
          *o = ACC ? *o + acc[mb][cb][i] : acc[mb][cb][i];
        }
      }
    }
}

template <int BT, int BE, int WM, int WN, int NB, bool ACC, bool WNORM>
__global__ __launch_bounds__(64 * WM * WN) void router_logits_kernel(const DecodeArgs p,
                                                                     float* wnorm) {
  static_assert(NB >= 3 && NB <= 4, "stage buffers");
  using C = LogitsTile<BT, BE, WM, WN>;
  __shared__ __attribute__((aligned(16))) uint16_t s0[C::ROWS * 64];
  __shared__ __attribute__((aligned(16))) uint16_t s1[C::ROWS * 64];
  __shared__ __attribute__((aligned(16))) uint16_t s2[C::ROWS * 64];
  __shared__ __attribute__((aligned(16))) uint16_t s3[NB > 3 ? C::ROWS * 64 : 8];
  router_logits_body<BT, BE, WM, WN, NB, ACC, WNORM>(p, wnorm, s0, s1, s2, s3);
}

__device__ __forceinline__ uint32_t f32_order_key(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float f32_from_order_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// One gate row re-checked in the router contract's order, as this lane
// walks it: bf16 gate, 16-byte piece c = chunk lane + 64 c (8 values);
// 8-bit gate, chunk lane + 64 i (16 codes) with its group's scale and bias.
// The token row xv has the same layout (8-bit: chunk i in xv[2 i],
// xv[2 i + 1]).  XC pieces of the token row cover H <= 512 XC.
template <int RQ, int XC>
struct CheckRow {
  static constexpr int NW = RQ ? XC / 2 : XC;
  uint4 w[NW];
  uint32_t s[RQ ? NW : 1], b[RQ ? NW : 1];
};

// The loads of one row, none of them conditional (pieces past the row's end
// reload its first piece and the dot skips them), so that the compiler
// can count the loads in flight and wait for this row alone.
template <int RQ, int XC>
__device__ __forceinline__ void check_load(CheckRow<RQ, XC>& r, const uint16_t* wrow,
                                           const QW& bank, size_t row, int H, int lane) {
  if constexpr (RQ) {
    const int chunks = H >> 4;
#pragma unroll
    for (int i = 0; i < CheckRow<RQ, XC>::NW; ++i) {
      const int ch = lane + 64 * i < chunks ? lane + 64 * i : 0;
      r.w[i] = load16(bank.w + row * (size_t)(H >> 2) + ch * 4);
      r.s[i] = bank.s[row * (size_t)(H >> 6) + (ch >> 2)];
      r.b[i] = bank.b[row * (size_t)(H >> 6) + (ch >> 2)];
    }
  } else {
    const int nxc = H >> 9;
#pragma unroll
    for (int c = 0; c < XC; ++c) r.w[c] = load16(wrow + (lane + 64 * (c < nxc ? c : 0)) * 8);
  }
}

template <int RQ, int XC>
__device__ __forceinline__ float check_dot(const uint4 (&xv)[XC], const CheckRow<RQ, XC>& r,
                                           int H, int lane) {
  float acc = 0.0f;
  if constexpr (RQ) {
    const int chunks = H >> 4;
#pragma unroll
    for (int i = 0; i < CheckRow<RQ, XC>::NW; ++i) {
      if (lane + 64 * i < chunks) {
        uint4 x0 = xv[2 * i], x1 = xv[2 * i + 1];  // opaque: unpacked per row
        asm volatile("" : "+v"(x0.x), "+v"(x0.y), "+v"(x0.z), "+v"(x0.w));
        asm volatile("" : "+v"(x1.x), "+v"(x1.y), "+v"(x1.z), "+v"(x1.w));
        float v[16];
        unpack_x16(x0, x1, v);
        acc = qgate_chunk(acc, r.w[i], v, bf16_to_f32(r.s[i]), bf16_to_f32(r.b[i]));
      }
    }
  } else {
    const int nxc = H >> 9;
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      if (c < nxc) {
        // opaque copies: unpacked per row, so that the token row stays in
        // 16 registers rather than being kept as 32 floats
        const uint32_t xx[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
        const uint32_t ww[4] = {r.w[c].x, r.w[c].y, r.w[c].z, r.w[c].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc = fmaf(bf16_lo(xx[i]), bf16_lo(ww[i]), acc);
          acc = fmaf(bf16_hi(xx[i]), bf16_hi(ww[i]), acc);
        }
      }
    }
  }
  // every loaded register counts as used on every path, so that no load of
  // this row is still pending where the next row's loads reuse registers
  // (the compiler would then wait for all loads in flight)
#pragma unroll
  for (int i = 0; i < CheckRow<RQ, XC>::NW; ++i) {
    asm volatile("" ::"v"(r.w[i].x), "v"(r.w[i].y), "v"(r.w[i].z), "v"(r.w[i].w));
    if constexpr (RQ) asm volatile("" ::"v"(r.s[i]), "v"(r.b[i]));
  }
  return wave_sum(acc);
}

// One wave per token (E <= 256, H a multiple of 512 up to 512 XC).  RQ: the
// gates are 8-bit banks (the logits came from their split planes).
//
// The re-checks form one list per wave in LDS: the shared gate's row first
// (its loads go out with the token row's, before the threshold is known),
// then every expert within the margin; the rows stream two deep (the next
// row's loads in flight while this one is dotted), where one row at a time
// waited for a memory round trip per row.  At 8192 tokens the kernel is
// bound by VALU issue (about 2000 instructions per wave, 9 re-checked rows
// per token): the token row stays unpacked as floats, which costs
// occupancy (5 waves per SIMD) but 32 fewer instructions per row
// (8192 tokens 32.4 -> 27.8 us, 512 tokens 13.3 -> 11.2).
// WPT = 4 (fewer tokens than the device has SIMDs): one workgroup per
// token; wave 0 finds the threshold and the list, the four waves re-check
// every fourth listed row each (the dots go to LDS), wave 0 ranks.
template <int RQ, int XC, int WPT>
__global__ __launch_bounds__(256) 
void router_select_kernel(const DecodeArgs p, const float* wnorm) {
  static_assert(WPT == 1 || WPT == 4, "a wave per token, or a workgroup");
  constexpr int P = 4;
  __shared__ int s_list[WPT == 1 ? 4 : 1][P * 64 + 1];
  __shared__ float s_c[WPT == 1 ? 1 : P * 64 + 1];
  __shared__ int s_n;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = WPT == 1 ? blockIdx.x * 4 + wave : blockIdx.x;
  if (t >= p.T) return;
  const bool lead = WPT == 1 || wave == 0;  // finds the list and ranks
  const int H = p.H;
  const float* lg = p.logits + (size_t)t * (p.E + 1);
  const uint16_t* xt = p.x + (size_t)t * H;
  // code of a listed row: an expert, or E for the shared gate
  auto row_ptr = [&](int code) {
    return code < p.E ? p.router_w + (size_t)code * H : p.sgate_w;
  };
  auto row_bank = [&](int code) -> const QW& { return code < p.E ? p.rq : p.sgq; };
  auto row_index = [&](int code) { return code < p.E ? (size_t)code : (size_t)0; };
  CheckRow<RQ, XC> ra, rb;
  uint4 xv[XC];
  float nx2 = 0.0f;
#pragma unroll
  for (int c = 0; c < XC; ++c) {
    if constexpr (RQ) {
      const int ch = lane + 64 * (c >> 1);
      xv[c] = load16(xt + (ch < (H >> 4) ? ch : 0) * 16 + (c & 1) * 8);
    } else {
      xv[c] = load16(xt + (lane + 64 * (c < (H >> 9) ? c : 0)) * 8);
    }
  }
  if (p.has_sg && lead) check_load<RQ, XC>(ra, row_ptr(p.E), row_bank(p.E), 0, H, lane);
  int n = 0;
  float out[P];
  int* const list = s_list[WPT == 1 ? wave : 0];
  if (lead) {
    // logits and row bounds: unconditional loads (lanes past E read expert
    // E - 1), so that all of them are in flight together
    // (the matrix-core logits as partial planes, added in plane order; for a
    // bf16 gate the row bounds as planes of partial sums of squares)
    const int NP = max(p.logit_planes, 1);
    const size_t plane = (size_t)p.T * (p.E + 1);
    float lraw[P], wraw[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int e = min(lane + 64 * i, p.E - 1);
      lraw[i] = lg[e];
      wraw[i] = wnorm[e];
    }
    for (int z = 1; z < NP; ++z) {
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int e = min(lane + 64 * i, p.E - 1);
        lraw[i] += lg[z * plane + e];
        if constexpr (!RQ) wraw[i] += wnorm[(size_t)z * p.E + e];
      }
    }
    if constexpr (!RQ) {
#pragma unroll
      for (int i = 0; i < P; ++i) wraw[i] = sqrtf(wraw[i]) * (1.0f + 1.0f / 1024.0f);
    }
    issue_fence();  // keeps these loads from being sunk into per-lane branches
    float lv[P], wn = 0.0f, amax = 0.0f;
    uint32_t key[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const bool on = lane + 64 * i < p.E;
      lv[i] = on ? lraw[i] : 0.0f;
      key[i] = on ? f32_order_key(lraw[i]) : 0u;
      wn = fmaxf(wn, on ? wraw[i] : 0.0f);
      amax = fmaxf(amax, fabsf(lv[i]));
    }
    // pieces past the row's end were loaded as the first piece: zero them
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      const bool live = RQ ? lane + 64 * (c >> 1) < (H >> 4) : c < (H >> 9);
      if (!live) xv[c] = make_uint4(0, 0, 0, 0);
      const uint32_t vv[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        nx2 = fmaf(bf16_lo(vv[i]), bf16_lo(vv[i]), nx2);
        nx2 = fmaf(bf16_hi(vv[i]), bf16_hi(vv[i]), nx2);
      }
    }
    const float nx = sqrtf(wave_sum(nx2)) * (1.0f + 1.0f / 1024.0f);
    wn = __uint_as_float(wave_max_u32(__float_as_uint(wn)));      // non-negative
    amax = __uint_as_float(wave_max_u32(__float_as_uint(amax)));
    // k-th largest L (with multiplicity)
    const uint32_t thr = wave_kth_largest<P>(key, p.K);
    const float tk = f32_from_order_key(thr);
    const float gam =
        RQ ? (float)(2 * H - 1) * 0x1p-23f * (1.0f + 0x1p-7f) + 0x1p-17f +
                 (float)(15 + 2 * ((H + 1023) / 1024) + 8) * 0x1p-24f
           : (float)(H - 1) * 0x1p-23f + (float)(H / 64 + 8) * 0x1p-24f;
    const float delta = gam * nx * wn + 0x1p-100f * (1.0f + nx + wn);
    const float mag = amax + 2.0f * delta + 1.0f;
    const int ex = (int)((__float_as_uint(mag) >> 23) & 0xFFu);
    const float ulp = __uint_as_float((uint32_t)max(ex - 7, 1) << 23);
    const float margin = (2.0f * delta + 1.25f * ulp) * (1.0f + 0x1p-20f);
    const float lo = tk - margin;
#pragma unroll
    for (int i = 0; i < P; ++i) out[i] = lane + 64 * i < p.E ? round_bf16(lv[i]) : 0.0f;
    // the list: the shared gate, then the experts within the margin in index order
    n = p.has_sg ? 1 : 0;
    if (p.has_sg && lane == 0) list[0] = p.E;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const bool in = lane + 64 * i < p.E && lv[i] >= lo;
      const uint64_t m = __ballot(in);
      if (in) list[n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0))] =
          lane + 64 * i;
      n += __popcll(m);
    }
    if (WPT > 1 && lane == 0) s_n = n;
  } else {
    // the other waves only re-check: zero the pieces past the row's end
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      const bool live = RQ ? lane + 64 * (c >> 1) < (H >> 4) : c < (H >> 9);
      if (!live) xv[c] = make_uint4(0, 0, 0, 0);
    }
  }
  if constexpr (WPT > 1) {
    __syncthreads();
    n = s_n;
  } else {
    __builtin_amdgcn_wave_barrier();
  }
  float sg_logit = 0.0f;
  auto record = [&](int code, float c) {
    if (code >= p.E) {
      sg_logit = c;
    } else {
#pragma unroll
      for (int i = 0; i < P; ++i)
        if ((code >> 6) == i && lane == (code & 63)) out[i] = round_bf16(c);
    }
  };
  // this wave's rows: list[j] for j = first, first + WPT, ... (n = 0 only
  // for NaN logits); the lead wave's ra holds the shared gate's row,
  // list[0], already
  const int first = WPT == 1 ? 0 : wave;
  auto emit = [&](int j, int code, float c) {
    if constexpr (WPT == 1)
      record(code, c);
    else if (lane == 0)
      s_c[j] = c;
  };
  int ca = p.E;
  if (!(p.has_sg && lead) && first < n) {
    ca = __builtin_amdgcn_readfirstlane(list[first]);
    check_load<RQ, XC>(ra, row_ptr(ca), row_bank(ca), row_index(ca), H, lane);
  }
  for (int j = first; j < n; j += 2 * WPT) {
    const int cb = __builtin_amdgcn_readfirstlane(list[min(j + WPT, n - 1)]);
    check_load<RQ, XC>(rb, row_ptr(cb), row_bank(cb), row_index(cb), H, lane);
    emit(j, ca, check_dot<RQ, XC>(xv, ra, H, lane));
    if (j + WPT >= n) break;
    const int cn = __builtin_amdgcn_readfirstlane(list[min(j + 2 * WPT, n - 1)]);
    check_load<RQ, XC>(ra, row_ptr(cn), row_bank(cn), row_index(cn), H, lane);
    emit(j + WPT, cb, check_dot<RQ, XC>(xv, rb, H, lane));
    ca = cn;
  }
  if constexpr (WPT > 1) {
    __syncthreads();
    if (!lead) return;
    for (int j = 0; j < n; ++j) record(list[j], s_c[j]);
  }
  finish_route<P>(p, t, out, sg_logit);
}

// ----------------------------------------------------------------- RMSNorm
// out[t] = bf16(bf16(x[t] r) w), r = 1 / sqrt(sum(x^2) / H + eps): the sum in
// the router contract's order (8-value chunks, lane l takes chunks l, l+64,
// ..., then the butterfly), ms, v, r correctly rounded in fp32 (the library is
// built with correctly rounded fp32 division and square root).  One wave
// per token.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, const uint16_t* w,
                                                      int T, int H, float eps, uint16_t* out) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= T) return;
  const uint16_t* xt = x + (size_t)t * H;
  const int chunks = H >> 3;
  float acc = 0.0f;
  for (int c = lane; c < chunks; c += 64) {
    const uint4 v = load16(xt + c * 8);
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc = fmaf(bf16_lo(vv[i]), bf16_lo(vv[i]), acc);
      acc = fmaf(bf16_hi(vv[i]), bf16_hi(vv[i]), acc);
    }
  }
  const float ms = wave_sum(acc) / (float)H;
  const float r = 1.0f / sqrtf(ms + eps);
  for (int c = lane; c < chunks; c += 64) {
    const uint4 v = load16(xt + c * 8);
    const uint4 g = load16(w + c * 8);
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
    const uint32_t gg[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = round_bf16(bf16_lo(vv[i]) * r) * bf16_lo(gg[i]);
      const float hi = round_bf16(bf16_hi(vv[i]) * r) * bf16_hi(gg[i]);
      o[i] = f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
    }
    *reinterpret_cast<uint4*>(out + (size_t)t * H + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ----------------------------------------------------------------- gate/up
template <int BITS>
struct Packing {
  static constexpr int kValuesPerChunk = BITS == 8 ? 16 : 32;  // per 16 B
  static constexpr int kValuesPerWord = 32 / BITS;
};

template <int BITS, int CPL, int PPW>
__global__ __launch_bounds__(256) void gate_up_kernel(const DecodeArgs p,
                                                      const int blocks_per_unit) {
  constexpr int VPC = Packing<BITS>::kValuesPerChunk;
  const int U1 = p.K + p.has_shared;
  const int unit = blockIdx.x / blocks_per_unit;
  const int blk = blockIdx.x - unit * blocks_per_unit;
  const int t = unit / U1;
  const int j = unit - t * U1;
  const bool shared = j >= p.K;
  const QW q = shared ? p.sgu : p.gu;
  const int I = p.I;
  const int e = shared ? 0 : p.idx[t * p.K + j];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int c0 = (blk * 4 + wave) * PPW;
  if (c0 >= I) return;
  if (!shared && (unsigned)e >= (unsigned)p.E) {
    // Caller index outside the bank: the slot contributes zeros and no
    // weight memory is touched.
    if (lane < PPW && c0 + lane < I) p.act[(size_t)unit * I + c0 + lane] = 0.0f;
    return;
  }
  const int H = p.H;
  const int CH = H / VPC;
  const int WPR = H / Packing<BITS>::kValuesPerWord;
  const int G = H >> 6;

  float xv[CPL][VPC];
  float xs[CPL];
  const uint16_t* xt = p.x + (size_t)t * H;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int ch = lane + 64 * i;
    xs[i] = 0.0f;
#pragma unroll
    for (int v = 0; v < VPC; ++v) xv[i][v] = 0.0f;
    if (ch < CH) {
#pragma unroll
      for (int h = 0; h < VPC / 8; ++h) {
        const uint4 b = load16(xt + ch * VPC + h * 8);
        xv[i][h * 8 + 0] = bf16_lo(b.x);
        xv[i][h * 8 + 1] = bf16_hi(b.x);
        xv[i][h * 8 + 2] = bf16_lo(b.y);
        xv[i][h * 8 + 3] = bf16_hi(b.y);
        xv[i][h * 8 + 4] = bf16_lo(b.z);
        xv[i][h * 8 + 5] = bf16_hi(b.z);
        xv[i][h * 8 + 6] = bf16_lo(b.w);
        xv[i][h * 8 + 7] = bf16_hi(b.w);
      }
#pragma unroll
      for (int v = 0; v < VPC; ++v) xs[i] += xv[i][v];
    }
  }

  uint4 wu[PPW][CPL], wg[PPW][CPL];
  float su[PPW][CPL], bu[PPW][CPL], sg[PPW][CPL], bg[PPW][CPL];
#pragma unroll
  for (int pp = 0; pp < PPW; ++pp) {
    const int c = c0 + pp;
    const size_t up_row = (size_t)e * 2 * I + (c < I ? c : 0);
    const size_t gate_row = up_row + I;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int ch = lane + 64 * i;
      wu[pp][i] = make_uint4(0, 0, 0, 0);
      wg[pp][i] = make_uint4(0, 0, 0, 0);
      su[pp][i] = bu[pp][i] = sg[pp][i] = bg[pp][i] = 0.0f;
      if (c < I && ch < CH) {
        wu[pp][i] = load16_stream(q.w + up_row * WPR + ch * 4);
        wg[pp][i] = load16_stream(q.w + gate_row * WPR + ch * 4);
        const int grp = (ch * VPC) >> 6;
        su[pp][i] = bf16_to_f32(q.s[up_row * G + grp]);
        bu[pp][i] = bf16_to_f32(q.b[up_row * G + grp]);
        sg[pp][i] = bf16_to_f32(q.s[gate_row * G + grp]);
        bg[pp][i] = bf16_to_f32(q.b[gate_row * G + grp]);
      }
    }
  }
#pragma unroll
  for (int pp = 0; pp < PPW; ++pp) {
    const int c = c0 + pp;
    if (c >= I) continue;  // wave-uniform
    float au = 0.0f, ag = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      au += su[pp][i] * qdot_chunk<BITS>(wu[pp][i], xv[i]) + bu[pp][i] * xs[i];
      ag += sg[pp][i] * qdot_chunk<BITS>(wg[pp][i], xv[i]) + bg[pp][i] * xs[i];
    }
    au = wave_sum(au);
    ag = wave_sum(ag);
    if (lane == 0) {
      const float up = round_bf16(au);
      const float gate = round_bf16(ag);
      p.act[(size_t)unit * I + c] = round_bf16(silu(gate) * up);
    }
  }
}

// -------------------------------------------------------------------- down
// act of the token's units is staged in LDS; every wave owns 64/CHR output
// rows and loops over the units.  COMBINE: weighted sum + shared expert +
// optional residual -> out[t, h]; otherwise per-slot rows y[t, j, h].
template <int BITS, bool COMBINE>
__global__ __launch_bounds__(256) void down_kernel(const DecodeArgs p,
                                                   const int blocks_per_token) {
  constexpr int VPC = Packing<BITS>::kValuesPerChunk;
  extern __shared__ float s_act[];
  const int t = blockIdx.x / blocks_per_token;
  const int blk = blockIdx.x - t * blocks_per_token;
  const int U1 = p.K + p.has_shared;
  const int units = COMBINE ? U1 : p.K;
  const int I = p.I;
  const int H = p.H;
  const float* act_t = p.act + (size_t)t * U1 * I;
  const int CHR = I / VPC;  // chunks per row: power of two <= 64

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int RPL = 64 / CHR;
  const int r = lane / CHR;
  const int ch = lane - r * CHR;
  const int h0 = (blk * 4 + wave) * RPL;
  const int h = h0 + r;
  const bool valid = h0 < H && h < H;
  const int WPR = I / Packing<BITS>::kValuesPerWord;
  const int G = I >> 6;
  const int grp = (ch * VPC) >> 6;

  // The weights of a batch of units depend on the routing only: they are
  // issued before the activations are staged, so the two round trips
  // overlap.
  uint4 wv[kUnitBatch];
  float sv[kUnitBatch], bv[kUnitBatch];
  auto load_batch = [&](int u0) {
#pragma unroll
    for (int b = 0; b < kUnitBatch; ++b) {
      const int u = u0 + b;
      wv[b] = make_uint4(0, 0, 0, 0);
      sv[b] = bv[b] = 0.0f;
      const bool sh = u >= p.K;
      const int e = (u < units && !sh) ? p.idx[t * p.K + u] : 0;
      if (u < units && valid && (unsigned)e < (unsigned)p.E) {
        const QW q = sh ? p.sdn : p.dn;
        const size_t row = (size_t)e * H + h;
        wv[b] = load16_stream(q.w + row * WPR + ch * 4);
        sv[b] = bf16_to_f32(q.s[row * G + grp]);
        bv[b] = bf16_to_f32(q.b[row * G + grp]);
      }
    }
  };
  load_batch(0);

  // Transposed staging: value v of chunk ch of unit u at u*I + v*CHR + ch,
  // so the lanes of a row (consecutive ch) read consecutive banks.
  {
    // 16-byte loads, all issued before the LDS stores (one round trip).
    const int n4 = units * I / 4;
    const float4* src4 = reinterpret_cast<const float4*>(act_t);
    for (int i0 = threadIdx.x; i0 < n4; i0 += 256 * kStageBatch) {
      float4 v[kStageBatch];
#pragma unroll
      for (int b = 0; b < kStageBatch; ++b) {
        const int i = i0 + 256 * b;
        if (i < n4) v[b] = src4[i];
      }
#pragma unroll
      for (int b = 0; b < kStageBatch; ++b) {
        const int i = i0 + 256 * b;
        if (i < n4) {
          const float vals[4] = {v[b].x, v[b].y, v[b].z, v[b].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int e = 4 * i + q;
            const int u = e / I;
            const int k = e - u * I;
            const int c = k / VPC;
            s_act[u * I + (k - c * VPC) * CHR + c] = vals[q];
          }
        }
      }
    }
  }
  // the LDS stores of every wave are done; the weight loads stay in flight
  // (a fenced __syncthreads would wait for them too)
  __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));
  __builtin_amdgcn_s_barrier();
  if (h0 >= H) return;

  float acc = 0.0f;
  for (int u0 = 0; u0 < units; u0 += kUnitBatch) {
    if (u0 > 0) load_batch(u0);  // top_k + shared above the batch size
#pragma unroll
    for (int b = 0; b < kUnitBatch; ++b) {
      const int u = u0 + b;
      if (u >= units) continue;  // wave-uniform
      float a[VPC];
      float asum = 0.0f;
      // the unit's LDS offset is opaque to the optimiser: hoisting the
      // read addresses of every unit out of the batch loop took 200+
      // registers and left two waves per SIMD
      int off = u * I + ch;
      asm volatile("" : "+v"(off));
      const float* src = s_act + off;
#pragma unroll
      for (int v = 0; v < VPC; ++v) {
        a[v] = src[v * CHR];
        asum += a[v];
      }
      float y = sv[b] * qdot_chunk<BITS>(wv[b], a) + bv[b] * asum;
      y = round_bf16(segment_sum_fast(y, CHR));
      if constexpr (COMBINE) {
        acc += p.scores[t * p.score_stride + u] * y;
      } else {
        if (ch == 0 && valid)
          p.out[((size_t)t * p.K + u) * H + h] = (uint16_t)f32_to_bf16(y);
      }
    }
  }
  if constexpr (COMBINE) {
    if (ch == 0 && valid) {
      float o = round_bf16(acc);
      if (p.residual) o = round_bf16(bf16_to_f32(p.residual[(size_t)t * H + h]) + o);
      p.out[(size_t)t * H + h] = (uint16_t)f32_to_bf16(o);
    }
  }
}

// ------------------------------------------------- few tokens: gate/up, down
// Every wave of the gate/up kernel is resident at once, but a wave keeps
// only a window of its rows in flight (kWindow pairs beyond the one it
// computes) and issues the next as it consumes one.  With all rows requested
// at once the memory system served every wave's first row late (measured:
// the first of 8 pairs landed a median 7.8 us into a 16 us kernel) and the
// dequantisation ran after the stream instead of under it.
namespace few {
constexpr int kWindow = 1;
}

// One wave per NP pairs of one routed (token, slot) unit: I / NP waves per
// unit.  Units of the call that chose the same expert share its rows: the
// first (in token-major order) streams them and computes every member.
template <int BITS>
__global__ __launch_bounds__(256) void gate_up_few_kernel(const DecodeArgs p) {
  constexpr int NP = few::NP;
  constexpr int D = few::kWindow;
  const int K = p.K;
  const int U1 = K + p.has_shared;
  const int TK = p.T * K;
  // wave-uniform in the compiler's view: the expert ids and scores become
  // scalar loads, outside the vector-memory counter the rows are waited on
  // with (a vector load of them issued behind a window of rows made every
  // wait on it a wait for the whole window)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  // the router launch before this one has finished with the call's tag
  if (blockIdx.x == 0 && threadIdx.x == 0)
    store_coherent_u32(&p.fs->epoch, load_coherent_u32(&p.fs->epoch) + 1);
  const int gw = blockIdx.x * 4 + wave;
  const int m = gw / few::kWavesPerUnit;
  if (m >= TK) return;
  const int c0 = (gw - m * few::kWavesPerUnit) * NP;
  const int e = p.idx[m];
  const int el = lane < TK ? p.idx[lane] : -1;
  const uint64_t members = __ballot(el == e && lane < TK);
  if (__builtin_ctzll(members) != m) return;  // an earlier unit streams the rows
  uint16_t* act = reinterpret_cast<uint16_t*>(p.act);
  auto act_at = [&](int b) { return ((size_t)(b / K) * U1 + (b % K)) * few::I + c0; };
  if ((unsigned)e >= (unsigned)p.E) {
    // caller index outside the bank: zeros, no weight memory touched
    for (uint64_t mm = members; mm; mm &= mm - 1)
      if (lane < NP) act[act_at(__builtin_ctzll(mm)) + lane] = 0;
    return;
  }
  const size_t up0 = (size_t)e * 2 * few::I + c0;
  // every pair's scale/bias word (lanes 0-15 up scales, 16-31 gate scales,
  // 32-47 up biases, 48-63 gate biases)
  uint32_t pw[NP];
#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
    const size_t row = up0 + pp + ((lane >> 4) & 1) * few::I;
    pw[pp] = reinterpret_cast<const uint32_t*>((lane < 32 ? p.gu.s : p.gu.b) +
                                               row * few::G)[lane & 15];
  }
  uint4 xr[few::Shape<BITS>::CPL][few::Shape<BITS>::VPC / 8];
  for (uint64_t mm = members; mm; mm &= mm - 1) {
    const int b = __builtin_ctzll(mm);
    few_load_x<BITS>(xr, p.x + (size_t)(b / K) * few::H, lane);  // an L2 hit, first
    FewPair<BITS> w[NP];
#pragma unroll
    for (int pp = 0; pp < D; ++pp) few_load_pair<BITS>(w[pp], p.gu, up0 + pp, lane);
    FewX<BITS> x;
    few_unpack_x<BITS>(x, xr);
    uint32_t res = 0;
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      if (pp + D < NP) few_load_pair<BITS>(w[pp + D], p.gu, up0 + pp + D, lane);
      issue_fence();
      const uint32_t a = few_pair_act<BITS>(w[pp], pw[pp], x, lane);
      res = lane == pp ? a : res;
      issue_fence();
    }
    if (lane < NP) act[act_at(b) + lane] = (uint16_t)res;
  }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two bf16 of 8-bit codes q0, q1 (exact: a code has 8 significant bits),
// packed (q1 << 16 | q0) for v_dot2_f32_bf16.
__device__ __forceinline__ uint32_t codes_bf16x2(uint32_t w, int pair) {
  // (v_cvt_f32_ubyte0..3)
  const float f0 = (float)((w >> (16 * pair)) & 0xFFu);
  const float f1 = (float)((w >> (16 * pair + 8)) & 0xFFu);
  return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}
// The same for 4-bit codes 2 j and 2 j + 1 of a word, from its even nibbles
// (lo = w & 0x0F0F0F0F: codes 0, 2, 4, 6 as bytes) and odd ones (hi).
__device__ __forceinline__ uint32_t nibbles_bf16x2(uint32_t lo, uint32_t hi, int j) {
  const float f0 = (float)((lo >> (8 * j)) & 0xFFu);
  const float f1 = (float)((hi >> (8 * j)) & 0xFFu);
  return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// One workgroup per R output rows of one token, one wave per unit (slot,
// then the shared expert): wave u issues every load of unit u's
// rows at once and reduces them (8-bit: 32 lanes a row, 16 codes a lane,
// two rows per pass; 4-bit: 16 lanes a row, 32 codes a lane, four rows per
// pass), the codes as bf16 pairs (`v_cvt_f32_ubyte*` and one `v_perm_b32`
// per two codes: a code has 8 significant bits, so bf16 holds it exactly)
// for v_dot2_f32_bf16 against the packed bf16 activations; a row's value is
// fma(bias, sum a, scale * sum q a), rounded to bf16.  COMBINE: the units'
// rows meet in LDS and lanes 0 .. R - 1 sum them in slot order (weighted),
// then the residual; otherwise each wave writes its per-slot rows y[t, j, h].
// R = 16 rows up to 4 tokens, 8 beyond (more, shorter workgroups).
template <int BITS, bool COMBINE, int R>
__global__ __launch_bounds__(64 * kMaxFusedUnits) void down_few_kernel(const DecodeArgs p) {
  constexpr int H = few::H;
  constexpr int I = few::I;
  constexpr int NU = kMaxFusedUnits;
  constexpr int LPR = BITS == 8 ? 32 : 16;  // lanes per row
  constexpr int RPW = 64 / LPR;             // rows per pass: 2 | 4
  constexpr int RP = R / RPW;               // passes
  constexpr int VPL = BITS == 8 ? 16 : 32;  // values per lane
  constexpr int WPR = I * BITS / 32;        // words per down row
  constexpr int GD = I / 64;                // groups per down row
  constexpr int AV = VPL / 8;               // 16-byte activation pieces per lane
  const int K = p.K;
  const int U1 = K + p.has_shared;
  const int units = COMBINE ? U1 : K;
  const int u = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // this wave's unit
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x / (H / R);
  const int h0 = (blockIdx.x - t * (H / R)) * R;
  const int r = lane / LPR;
  const int ch = lane & (LPR - 1);
  __shared__ float s_y[NU][R];
  // the combine weights of the combining lanes, loaded first
  float score[NU];
  if (COMBINE && threadIdx.x < R) {
#pragma unroll
    for (int v = 0; v < NU; ++v) score[v] = p.scores[t * p.score_stride + min(v, units - 1)];
  }
  if (u < units) {
    // an index outside the bank (a caller's) reads expert 0 and gives zeros
    int e = 0;
    bool bad = false;
    if (u < K) {
      e = p.idx[t * K + u];
      bad = (unsigned)e >= (unsigned)p.E;
      e = bad ? 0 : e;
    }
    const QW q = u < K ? p.dn : p.sdn;
    const uint16_t* act =
        reinterpret_cast<const uint16_t*>(p.act) + ((size_t)t * U1 + u) * I + ch * VPL;
    uint4 av[AV], wv[RP];
    uint32_t sv[RP], bv[RP];
#pragma unroll
    for (int i = 0; i < AV; ++i) av[i] = load16(act + 8 * i);
#pragma unroll
    for (int rp = 0; rp < RP; ++rp) {
      const size_t row = (size_t)e * H + h0 + RPW * rp + r;
      wv[rp] = load16_stream(q.w + row * WPR + ch * 4);
      sv[rp] = q.s[row * GD + (ch * VPL >> 6)];
      bv[rp] = q.b[row * GD + (ch * VPL >> 6)];
    }
    constexpr uint32_t kOnes = 0x3F803F80u;  // bf16 (1, 1)
    uint32_t aw[VPL / 2];
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      aw[4 * i] = av[i].x;
      aw[4 * i + 1] = av[i].y;
      aw[4 * i + 2] = av[i].z;
      aw[4 * i + 3] = av[i].w;
    }
    float asum = 0.0f;
#pragma unroll
    for (int k = 0; k < VPL / 2; ++k) asum = dot2_bf16(aw[k], kOnes, asum);
#pragma unroll
    for (int rp = 0; rp < RP; ++rp) {
      const uint32_t ww[4] = {wv[rp].x, wv[rp].y, wv[rp].z, wv[rp].w};
      float dot = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (BITS == 8) {
          dot = dot2_bf16(codes_bf16x2(ww[k], 0), aw[2 * k], dot);
          dot = dot2_bf16(codes_bf16x2(ww[k], 1), aw[2 * k + 1], dot);
        } else {
          const uint32_t lo = ww[k] & 0x0F0F0F0Fu, hi = (ww[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
          for (int j = 0; j < 4; ++j) dot = dot2_bf16(nibbles_bf16x2(lo, hi, j), aw[4 * k + j], dot);
        }
      }
      float y = fmaf(bf16_to_f32(bv[rp]), asum, bf16_to_f32(sv[rp]) * dot);
      y = round_bf16(segment_sum_fast(y, LPR));
      y = bad ? 0.0f : y;
      if (ch == 0) {
        if constexpr (COMBINE)
          s_y[u][RPW * rp + r] = y;
        else
          p.out[((size_t)t * K + u) * H + h0 + RPW * rp + r] = (uint16_t)f32_to_bf16(y);
      }
    }
  }
  if constexpr (COMBINE) {
    __syncthreads();
    if (threadIdx.x < R) {
      const int h = h0 + threadIdx.x;
      float acc = 0.0f;
#pragma unroll
      for (int v = 0; v < NU; ++v)
        if (v < units) acc = fmaf(score[v], s_y[v][threadIdx.x], acc);
      float o = round_bf16(acc);
      if (p.residual) o = round_bf16(bf16_to_f32(p.residual[(size_t)t * H + h]) + o);
      p.out[(size_t)t * H + h] = (uint16_t)f32_to_bf16(o);
    }
  }
}

// --------------------------------------------------------------------- qmv
// y[m, n] = x[lhs[m]] . deq(w[rhs[m], n])^T.  Rows of 64/LPR outputs per wave
// load, where LPR = min(64, chunks per row); CPL chunks per lane.
template <int BITS, int CPL>
__global__ __launch_bounds__(256) void qmv_kernel(const QmvArgs p,
                                                  const int blocks_per_row) {
  constexpr int VPC = Packing<BITS>::kValuesPerChunk;
  const int m = blockIdx.x / blocks_per_row;
  const int blk = blockIdx.x - m * blocks_per_row;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int K = p.K;
  const int CH = K / VPC;
  const int LPR = CH >= 64 ? 64 : CH;
  const int RPL = 64 / LPR;
  const int r = lane / LPR;
  const int cl = lane - r * LPR;
  const int n = (blk * 4 + wave) * RPL + r;
  if ((blk * 4 + wave) * RPL >= p.N) return;
  const bool valid = n < p.N;
  int xrow = p.lhs ? p.lhs[m] : m;
  int e = p.rhs ? p.rhs[m] : 0;
  const bool in_range =
      (unsigned)xrow < (unsigned)p.x_rows && (unsigned)e < (unsigned)p.experts;
  if (!in_range) xrow = e = 0;  // row of zeros, no out-of-range access
  const uint16_t* xr = p.x + (size_t)xrow * K;
  const size_t row = (size_t)e * p.N + (valid ? n : 0);
  const int WPR = K / Packing<BITS>::kValuesPerWord;
  const int G = K >> 6;
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int ch = cl + LPR * i;
    if (ch < CH && valid && in_range) {
      const uint4 wv = load16_stream(p.w.w + row * WPR + ch * 4);
      float a[VPC];
      float asum = 0.0f;
#pragma unroll
      for (int h = 0; h < VPC / 8; ++h) {
        const uint4 b = load16(xr + ch * VPC + h * 8);
        a[h * 8 + 0] = bf16_lo(b.x);
        a[h * 8 + 1] = bf16_hi(b.x);
        a[h * 8 + 2] = bf16_lo(b.y);
        a[h * 8 + 3] = bf16_hi(b.y);
        a[h * 8 + 4] = bf16_lo(b.z);
        a[h * 8 + 5] = bf16_hi(b.z);
        a[h * 8 + 6] = bf16_lo(b.w);
        a[h * 8 + 7] = bf16_hi(b.w);
      }
#pragma unroll
      for (int v = 0; v < VPC; ++v) asum += a[v];
      const int grp = (ch * VPC) >> 6;
      acc += bf16_to_f32(p.w.s[row * G + grp]) * qdot_chunk<BITS>(wv, a) +
             bf16_to_f32(p.w.b[row * G + grp]) * asum;
    }
  }
  acc = segment_sum(acc, LPR);
  if (cl == 0 && valid) {
    if (p.y_f32)
      p.y_f32[(size_t)m * p.N + n] = acc;
    else
      p.y_bf16[(size_t)m * p.N + n] = (uint16_t)f32_to_bf16(acc);
  }
}

// ------------------------------------------------------------------ launch
#define RMOE_CHECK_LAUNCH()                  \
  do {                                       \
    hipError_t _e = hipGetLastError();       \
    if (_e != hipSuccess) return _e;         \
  } while (0)

bool router_mfma_eligible(int E, int H) {
  return E % 64 == 0 && E <= 256 && H % 512 == 0 && H <= 4096;
}

// 64 x 64 tiles (two workgroups of four waves per CU) from 4096 tokens on,
// 32 x 32 below, where 64-token tiles leave most CUs idle: at 512 tokens
// 11.7 against 17.3 us, at 8192 tokens 21.2 against 32.2 (event-timed).
// The selection: a workgroup per token while the tokens number at most the
// device's 1024 SIMDs (the re-checks of a token then run on four waves),
// else a wave per token.
template <int RQ, int XC>
static void select_launch(const DecodeArgs& a, const void* wnorm, hipStream_t s) {
  if (a.T <= 1024)
    hipLaunchKernelGGL((router_select_kernel<RQ, XC, 4>), dim3(a.T), dim3(256), 0, s, a,
                       (const float*)wnorm);
  else
    hipLaunchKernelGGL((router_select_kernel<RQ, XC, 1>), dim3((a.T + 3) / 4), dim3(256), 0, s,
                       a, (const float*)wnorm);
}

template <bool ACC, bool WNORM>
static void launch_logits(const DecodeArgs& a, float* wnorm, hipStream_t s) {
  const unsigned z = (unsigned)max(a.logit_planes, 1);
  if (a.T >= 4096)
    hipLaunchKernelGGL((router_logits_kernel<64, 64, 2, 2, 3, ACC, WNORM>),
                       dim3((a.T + 63) / 64, a.E / 64, z), dim3(256), 0, s, a, wnorm);
  else
    hipLaunchKernelGGL((router_logits_kernel<32, 32, 2, 2, 4, ACC, WNORM>),
                       dim3((a.T + 31) / 32, a.E / 32, z), dim3(256), 0, s, a, wnorm);
}

// Shares of H over which the logits kernel splits each tile (each share
// its own partial plane): a few hundred tokens leave most CUs idle with one
// workgroup per tile, and the shorter chain of stages ends sooner (512
// tokens: 245 -> 241 us per block call); from 4096 tokens on the 64 x 64
// tiles fill the device and the extra planes' traffic cost more (8192
// tokens: +8 us with two).
int router_logit_planes(int T) {
  return T <= 1024 ? 4 : T < 4096 ? 2 : 1;
}

hipError_t launch_router_mfma(const DecodeArgs& a, float* wnorm, uint16_t* split,
                              hipStream_t s) {
  if (a.rq8) {
    // logits over the hi plane, then continued over the lo plane
    hipLaunchKernelGGL(router_split_kernel, dim3((a.E + 3) / 4), dim3(256), 0, s, a, split,
                       split + (size_t)a.E * a.H, wnorm);
    DecodeArgs hi = a, lo = a;
    hi.router_w = split;
    lo.router_w = split + (size_t)a.E * a.H;
    launch_logits<false, false>(hi, nullptr, s);
    launch_logits<true, false>(lo, nullptr, s);
    if (a.H <= 2048)
      select_launch<1, 4>(a, wnorm, s);
    else
      select_launch<1, 8>(a, wnorm, s);
  } else {
    // the row norms come from the first token tile's workgroups
    launch_logits<false, true>(a, wnorm, s);
    if (a.H <= 2048)
      select_launch<0, 4>(a, wnorm, s);
    else
      select_launch<0, 8>(a, wnorm, s);
  }
  RMOE_CHECK_LAUNCH();
  return hipSuccess;
}

hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* w, int T, int H, float eps,
                          uint16_t* out, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x, w, T, H, eps, out);
  RMOE_CHECK_LAUNCH();
  return hipSuccess;
}

template <int TB>
static void router_tb(const DecodeArgs& a, hipStream_t s) {
  const int rows = a.E + a.has_sg;
  dim3 grid((rows + 3) / 4, (a.T + TB - 1) / TB);
  if (a.few_bits != 0 && a.has_shared) {
    // plus the shared expert's gate/up (E <= 256 on the few-token path)
    grid.x += few::kSharedBlocks;
    if (a.few_bits == 8)
      hipLaunchKernelGGL((router_kernel<4, TB, 8>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((router_kernel<4, TB, 4>), grid, dim3(256), 0, s, a);
  } else if (a.E <= 256) {
    hipLaunchKernelGGL((router_kernel<4, TB, 0>), grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((router_kernel<kMaxExperts / 64, TB, 0>), grid, dim3(256), 0, s, a);
  }
}

hipError_t launch_router(const DecodeArgs& a, hipStream_t s) {
  // tokens per group: each row is streamed once per group
  if (a.T == 1)
    router_tb<1>(a, s);
  else if (a.T == 2)
    router_tb<2>(a, s);
  else
    router_tb<4>(a, s);
  RMOE_CHECK_LAUNCH();
  return hipSuccess;
}

template <int BITS, int CPL>
static hipError_t gate_up_cpl(const DecodeArgs& a, hipStream_t s) {
  constexpr int PPW = 2;
  const int U1 = a.K + a.has_shared;
  const int bpu = (a.I + 4 * PPW - 1) / (4 * PPW);
  const long long blocks = (long long)bpu * U1 * a.T;
  hipLaunchKernelGGL((gate_up_kernel<BITS, CPL, PPW>), dim3((unsigned)blocks),
                     dim3(256), 0, s, a, bpu);
  RMOE_CHECK_LAUNCH();
  return hipSuccess;
}

hipError_t launch_gate_up(const DecodeArgs& a, int bits, hipStream_t s) {
  if (a.few_bits != 0) {
    const int waves = a.T * a.K * few::kWavesPerUnit;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (a.few_bits == 8)
      hipLaunchKernelGGL(gate_up_few_kernel<8>, grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(gate_up_few_kernel<4>, grid, dim3(256), 0, s, a);
    RMOE_CHECK_LAUNCH();
    return hipSuccess;
  }
  const int vpc = bits == 8 ? 16 : 32;
  const int cpl = (a.H / vpc + 63) / 64;
  if (bits == 8) {
    if (cpl <= 1) return gate_up_cpl<8, 1>(a, s);
    if (cpl <= 2) return gate_up_cpl<8, 2>(a, s);
    return gate_up_cpl<8, 4>(a, s);
  }
  if (cpl <= 1) return gate_up_cpl<4, 1>(a, s);
  if (cpl <= 2) return gate_up_cpl<4, 2>(a, s);
  return gate_up_cpl<4, 4>(a, s);
}

hipError_t launch_down(const DecodeArgs& a, int bits, bool combine, hipStream_t s) {
  if (a.few_bits != 0) {
    // rows per workgroup: 16 up to 4 tokens, 8 beyond
    const dim3 block(64 * kMaxFusedUnits);
    auto go = [&](auto bits_c, auto combine_c, auto r_c) {
      constexpr int B = decltype(bits_c)::value;
      constexpr bool C = decltype(combine_c)::value;
      constexpr int R = decltype(r_c)::value;
      hipLaunchKernelGGL((down_few_kernel<B, C, R>), dim3((unsigned)(a.T * (few::H / R))), block,
                         0, s, a);
    };
    using B8 = std::integral_constant<int, 8>;
    using B4 = std::integral_constant<int, 4>;
    using CT = std::true_type;
    using CF = std::false_type;
    using R16 = std::integral_constant<int, 16>;
    using R8 = std::integral_constant<int, 8>;
    const bool wide = a.T <= 4;
    if (a.few_bits == 8) {
      if (combine) wide ? go(B8{}, CT{}, R16{}) : go(B8{}, CT{}, R8{});
      else wide ? go(B8{}, CF{}, R16{}) : go(B8{}, CF{}, R8{});
    } else {
      if (combine) wide ? go(B4{}, CT{}, R16{}) : go(B4{}, CT{}, R8{});
      else wide ? go(B4{}, CF{}, R16{}) : go(B4{}, CF{}, R8{});
    }
    RMOE_CHECK_LAUNCH();
    return hipSuccess;
  }
  const int vpc = bits == 8 ? 16 : 32;
  const int rpl = 64 / (a.I / vpc);
  const int bpt = (a.H + 4 * rpl - 1) / (4 * rpl);
  const int units = combine ? a.K + a.has_shared : a.K;
  const size_t lds = (size_t)units * a.I * sizeof(float);
  dim3 grid((unsigned)((long long)bpt * a.T));
  if (bits == 8) {
    if (combine)
      hipLaunchKernelGGL((down_kernel<8, true>), grid, dim3(256), lds, s, a, bpt);
    else
      hipLaunchKernelGGL((down_kernel<8, false>), grid, dim3(256), lds, s, a, bpt);
  } else {
    if (combine)
      hipLaunchKernelGGL((down_kernel<4, true>), grid, dim3(256), lds, s, a, bpt);
    else
      hipLaunchKernelGGL((down_kernel<4, false>), grid, dim3(256), lds, s, a, bpt);
  }
  RMOE_CHECK_LAUNCH();
  return hipSuccess;
}

template <int BITS, int CPL>
static hipError_t qmv_cpl(const QmvArgs& a, hipStream_t s) {
  const int vpc = BITS == 8 ? 16 : 32;
  const int ch = a.K / vpc;
  const int lpr = ch >= 64 ? 64 : ch;
  const int rows_per_block = 4 * (64 / lpr);
  const int bpr = (a.N + rows_per_block - 1) / rows_per_block;
  const long long blocks = (long long)bpr * a.M;
  hipLaunchKernelGGL((qmv_kernel<BITS, CPL>), dim3((unsigned)blocks), dim3(256),
                     0, s, a, bpr);
  RMOE_CHECK_LAUNCH();
  return hipSuccess;
}

hipError_t launch_qmv(const QmvArgs& a, int bits, hipStream_t s) {
  const int vpc = bits == 8 ? 16 : 32;
  const int cpl = (a.K / vpc + 63) / 64;
  if (bits == 8) {
    if (cpl <= 1) return qmv_cpl<8, 1>(a, s);
    if (cpl <= 2) return qmv_cpl<8, 2>(a, s);
    return qmv_cpl<8, 4>(a, s);
  }
  if (cpl <= 1) return qmv_cpl<4, 1>(a, s);
  if (cpl <= 2) return qmv_cpl<4, 2>(a, s);
  return qmv_cpl<4, 4>(a, s);
}

}  // namespace rmoe
