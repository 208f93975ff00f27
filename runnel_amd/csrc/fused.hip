// Single-launch batch-1 decode of one or more MoE layers (gfx950).
//
// 256 workgroups of 8 waves, one per CU and 32 on each of the 8 XCDs,
// launched cooperatively so that every workgroup is resident (inside a
// captured graph: a plain launch of the same grid, see launch_fused_decode).
// A workgroup takes its XCD from the hardware (HW_REG_XCC_ID): the
// dispatcher deals the workgroups of a launch to the XCDs in turn, but the
// XCD that receives workgroup 0 follows the launches before it (a plain
// launch right behind a 7-workgroup kernel on the same queue started on
// XCD 7), so workgroup i is the (i / 8)-th of its XCD, not necessarily on
// XCD i % 8.  Routed slot u (u < K <= 8) is computed
// whole by XCD u: its gate/up pairs, the SwiGLU activations (handed over
// inside that XCD's L2) and all of its down rows, one bf16 output word per
// row.  The shared expert does not depend on the routing: XCD x computes its
// pairs 64 x .. 64 x + 63 right after the router rows (handed over
// device-wide, off the routed critical path) and its down rows
// 256 x .. 256 x + 255.  A layer therefore has one device-wide hand-over on
// its critical path: every XCD combines the unit outputs of its own 2048
// rows (each workgroup 64 rows), and the combined layer input is handed
// over inside the XCD.  Per layer:
//
//   C  the layer input.  Waves 0-3 ("pollers", no prefetched loads in their
//      queue, so a poll is not served behind them) collect the unit outputs
//      of their workgroup's rows, sum them in slot order with the previous
//      layer's scores, add the residual, publish the rows in the XCD's L2 and
//      collect all of x.  Waves 4-7 ("loaders") load the layer's
//      routing-independent rows (router rows, the shared gate's row, the
//      shared pairs, RMSNorm weights) and move the router rows to LDS
//   R  every wave dots one router row (the router contract's fixed order)
//      from LDS against x; logits go to the XCD's L2
//   S  waves 6 and 7: one shared pair each; its activation is published
//      device-wide after the routed loads are out
//   K  wave 0 ranks the XCD's logits: 4 keys per lane sorted locally, then
//      rounds of a DPP wave maximum up to this XCD's slot (the rest of the
//      top_k rounds once the routed loads are out)
//   G  this XCD's routed expert: two pairs per wave and, right behind
//      their rows, eight down rows per wave are loaded; activations to the
//      XCD's L2
//   D  the routed rows' dots, and (8-bit) two shared rows per loader wave;
//      4-bit layers reduce the shared rows on wave 1 before D, while the
//      routed activations are on their way.  The results go to LDS and one
//      wave stores them after the layer's last barrier
//   O  (after the last layer) every workgroup combines 8 output rows
//
// Values handed between workgroups are tagged words, (bf16 value << 16) |
// tag, where the tag of phase epoch + layer + 1 (the epoch word is read at
// start) is phase % 65535 + 1: never 0, the tag of zero-filled scratch.  A
// consumer polls the data itself until every tag it needs shows the current
// phase: no separate flag round trip, no same-address atomics (which
// serialise across CUs), no resets.  Every hand-over word is written by its
// producer in every layer whatever the call's shape (zeros where a slot is
// unused), so a word is never older than the previous call and an old word
// cannot carry the current tag.  XCD-local words are stored with sc0 (to the
// XCD's L2) and read with sc0 nt; device-wide words with sc1 stores and
// loads.
//
// Every wait is bounded.  A wait gives up after kSpinLimit rounds, or when
// the call's abort word shows that another workgroup gave up a wait (read
// every kAbortCheck rounds); the workgroup that gives up publishes the
// abort word and the status word (1) at once, and a wave that gave up skips
// its later waits, so a failed call ends promptly and still runs to
// completion.  A workgroup whose hardware XCC id is not below 8 sets the
// status word to 2 and the abort word.  A call whose key the host has
// written into the abort word beforehand waits for nothing and sets the
// status word to 1 (a cancelled call).
#include "common.h"
#include "handover.h"
#include "kernels.h"

namespace rmoe {

namespace {

constexpr int kThreads = kFusedThreads;
constexpr int kWaves = kThreads / 64;
constexpr int kPollWave = 0;  // ranks the logits and computes the scores
constexpr int kShDownWave = 1;  // 4-bit: the workgroup's shared down rows

// XCD-local hand-over (between workgroups on one XCD): stores reach the
// XCD's L2 (the vector L1 writes through); loads with sc0 nt skip the L1
// and are served by that L2.  Only valid between workgroups of one XCD.
constexpr int kXcdLoadAux = 3;   // sc0 | nt
constexpr int kXcdStoreAux = 1;  // sc0

// One wave collects n_words tagged words written by other workgroups: 16-byte
// loads at agent coherence (sc1, the bits agent-scope atomic loads use; each
// 4-byte word is as one store left it), repeated only for the pieces whose
// tags are not yet current, and the values (bf16 in the high half) go to
// LDS as floats.  Polling from one wave that has no prefetch outstanding
// keeps each round trip short (a wave's loads return in order) and the
// polling traffic to one stream per workgroup.
template <int NL, int AUX = 16>
__device__ __forceinline__ void poll_tagged(const uint32_t* src, int n_words, uint32_t tag,
                                            float* dst, int lane, int part, WaitState& ws) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(src), (short)0, n_words * 4, 0x00020000);
  // this wave's pieces: j0 + j, j < NL (16 bytes per lane each)
  const int j0 = part * NL;
  uint32_t pend = 0;
#pragma unroll
  for (int j = 0; j < NL; ++j)
    if ((lane + 64 * (j0 + j)) * 4 < n_words) pend |= 1u << j;
  if (ws.gave_up) pend = 0;
  for (int spin = 0;; ++spin) {
    u32x4 v[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j)
      if ((pend >> j) & 1u)
        v[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane + 64 * (j0 + j)) * 16, 0, AUX);
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      if ((pend >> j) & 1u) {
        if (tag_ok(v[j].x, tag) && tag_ok(v[j].y, tag) && tag_ok(v[j].z, tag) &&
            tag_ok(v[j].w, tag)) {
          *reinterpret_cast<float4*>(dst + (lane + 64 * (j0 + j)) * 4) =
              make_float4(__uint_as_float(v[j].x & 0xFFFF0000u),
                          __uint_as_float(v[j].y & 0xFFFF0000u),
                          __uint_as_float(v[j].z & 0xFFFF0000u),
                          __uint_as_float(v[j].w & 0xFFFF0000u));
          pend &= ~(1u << j);
        }
      }
    }
    if (!__any(pend != 0u)) break;
    if (give_up(ws, spin)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}


__device__ __forceinline__ void cswap_desc(uint32_t& a, uint32_t& b) {
  const uint32_t hi = a > b ? a : b;
  const uint32_t lo = a > b ? b : a;
  a = hi;
  b = lo;
}

template <int BITS>
struct Shape {
  static constexpr int H = kFusedH;
  static constexpr int I = kFusedI;
  static constexpr int GU_CPL = H * BITS / 8 / (64 * 16);  // 16-B chunks per lane: 2 | 1
  static constexpr int VPC = BITS == 8 ? 16 : 32;          // values per chunk
  static constexpr int GU_WPR = H * BITS / 32;             // words per gate/up row
  static constexpr int DN_WPL = 8 * BITS / 32;             // down words per lane: 2 | 1
  static constexpr int DN_WPR = I * BITS / 32;             // words per down row
};

}  // namespace

// Loads of one gate/up pair (up row c and gate row c + I of one unit): the
// packed chunks of this lane, and one 4-byte word per lane that together
// cover every scale and bias of both rows (lanes 0-15: up scales, 16-31:
// gate scales, 32-47: up biases, 48-63: gate biases; 16 words = 32 bf16 =
// one row's groups).  A lane's own group values come from `param_of`.
template <int CPL>
struct PairRegs {
  uint4 wu[CPL], wg[CPL];
  uint32_t pw;
};

template <int BITS, int CPL>
__device__ __forceinline__ void load_pair_params(PairRegs<CPL>& r, const QW& bank,
                                                 size_t up_row, int lane) {
  using S = Shape<BITS>;
  static_assert(S::H / 64 == 32, "16 words of bf16 per row");
  const size_t row = up_row + ((lane >> 4) & 1) * S::I;
  const uint16_t* base = (lane < 32 ? bank.s : bank.b) + row * (S::H / 64);
  r.pw = reinterpret_cast<const uint32_t*>(base)[lane & 15];
}

template <int BITS, int CPL>
__device__ __forceinline__ void load_pair_words(PairRegs<CPL>& r, const QW& bank,
                                                size_t up_row, int lane) {
  using S = Shape<BITS>;
  const size_t gate_row = up_row + S::I;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int ch = lane + 64 * i;
    r.wu[i] = load16_stream(bank.w + up_row * S::GU_WPR + ch * 4);
    r.wg[i] = load16_stream(bank.w + gate_row * S::GU_WPR + ch * 4);
  }
}

// bf16 value of group g held in the word array spread over lanes
// [first, first + 16): word g / 2, half g % 2.
__device__ __forceinline__ float param_of(uint32_t word, int first, int g) {
  const uint32_t w = (uint32_t)__shfl((int)word, first + (g >> 1), 64);
  return __uint_as_float((g & 1) ? (w & 0xFFFF0000u) : (w << 16));
}

// Down row h of one unit: lane l holds values [8l, 8l + 8).  Scales and
// biases of up to 8 units' rows come in one word per lane (lane 8u + j:
// unit u, j < 4 scale words, j >= 4 bias words).
template <int WPL>
struct DownRegs {
  uint32_t w[WPL];
};



// One gate row held in registers by a wave: bf16 (RQ 0: lane chunks
// lane + 64 i of 8 values) or 8-bit MLX-affine (RQ 1: lane chunks of 16
// codes with their group's scale and bias as raw bf16 bits).
template <int RQ>
struct GateRow;
template <>
struct GateRow<0> {
  static constexpr int C = kFusedH / 8 / 64;
  uint4 w[C];
};
template <>
struct GateRow<1> {
  static constexpr int C = kFusedH / 16 / 64;
  uint4 w[C];
  uint32_t s[C], b[C];
};


// This lane's partial of the router contract's dot (x as floats in LDS).
__device__ __forceinline__ float gate_partial(const GateRow<0>& r, const float* s_x, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < GateRow<0>::C; ++i) {
    const float* xv = s_x + (lane + 64 * i) * 8;
    acc = fmaf(xv[0], bf16_lo(r.w[i].x), acc);
    acc = fmaf(xv[1], bf16_hi(r.w[i].x), acc);
    acc = fmaf(xv[2], bf16_lo(r.w[i].y), acc);
    acc = fmaf(xv[3], bf16_hi(r.w[i].y), acc);
    acc = fmaf(xv[4], bf16_lo(r.w[i].z), acc);
    acc = fmaf(xv[5], bf16_hi(r.w[i].z), acc);
    acc = fmaf(xv[6], bf16_lo(r.w[i].w), acc);
    acc = fmaf(xv[7], bf16_hi(r.w[i].w), acc);
  }
  return acc;
}
__device__ __forceinline__ float gate_partial(const GateRow<1>& r, const float* s_x, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < GateRow<1>::C; ++i) {
    const float* xp = s_x + (lane + 64 * i) * 16;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
      const float4 f = *reinterpret_cast<const float4*>(xp + j);
      v[j] = f.x;
      v[j + 1] = f.y;
      v[j + 2] = f.z;
      v[j + 3] = f.w;
    }
    acc = qgate_chunk(acc, r.w[i], v, bf16_to_f32(r.s[i]), bf16_to_f32(r.b[i]));
  }
  return acc;
}

// Descriptor of layer l.  The table is read through the constant address
// space so the loads are scalar (uniform, read-only for the whole launch):
// waiting for them does not wait for the vector loads in flight, which a
// generic (flat) load of the descriptor would.
typedef const FusedLayer __attribute__((address_space(4)))* ConstLayerPtr;
__device__ __forceinline__ FusedLayer layer_desc(const FusedArgs& p, int l) {
  if (!p.table) return p.layer0;
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only parses device code
  return reinterpret_cast<ConstLayerPtr>(reinterpret_cast<uintptr_t>(p.table))[l];
#else
  return p.table[l];
#endif
}

// Whether the layer's shared expert has a sigmoid gate (its row pointer is
// set).  Taken from the layer descriptor rather than a launch-wide flag: the
// per-layer test keeps the compiler's schedule of the layer loop (a uniform
// kernel-argument flag here cost about 1 us per layer).
template <int RQ>
__device__ __forceinline__ bool shared_gated(const FusedLayer& L, bool has_shared) {
  return has_shared && (RQ ? L.sgq.w != nullptr : L.sgate_w != nullptr);
}




// Buffering.  Single-buffered XCD-local words (logits, act) are safe
// because every workgroup of the XCD reads the whole combined x of layer
// L + 1, written by each of them after it finished layer L.  The unit
// outputs, the combined x and the shared activations are double-buffered by
// layer parity: a workgroup writes layer L's unit outputs only after it has
// read every workgroup's shared activations of layer L, which each wrote
// after reading layer L - 1's combine inputs.  The shared activations are
// written (as zeros) even without a shared expert, so that workgroup 0, which
// reads them all, has consumed a word from every workgroup before it
// advances the epoch at the end.

constexpr int kXcds = 8;
constexpr int kXcdWgs = kFusedXcdGrid / kXcds;           // 32 workgroups per XCD
constexpr int kXcdWaves = kXcdWgs * kWaves;              // 256 waves per XCD
constexpr int kXcdRows = kFusedH / kXcdWaves;            // 8 rows per wave
constexpr int kSharedPairsPerXcd = kFusedI / kXcds;      // 64
constexpr int kSharedPairWave = kWaves - kSharedPairsPerXcd / kXcdWgs;  // waves 6, 7
static_assert(kXcdRows == 8 && kSharedPairsPerXcd % kXcdWgs == 0, "layout");
static_assert(kFusedH / kXcds == kXcdWaves, "one shared down row per wave");

__device__ __forceinline__ void store_xcd_u32(uint32_t* base, int n_words, int idx,
                                              uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(
      v, __builtin_amdgcn_make_buffer_rsrc(base, (short)0, n_words * 4, 0x00020000), idx * 4,
      0, kXcdStoreAux);
}

// Eight down rows of one unit, contiguous in memory: 16 bytes per lane per
// load (8-bit: two rows per load, 32 lanes each; 4-bit: four rows, 16 lanes
// each), and one word per lane of the rows' scales (lanes 0-31) and biases
// (lanes 32-63), 8 groups per row.
template <int BITS>
struct RowsRegs {
  static constexpr int N = BITS == 8 ? 4 : 2;
  uint4 w[N];
  uint32_t pw;
};

template <int BITS>
__device__ __forceinline__ void load_rows_params(RowsRegs<BITS>& r, const QW& bank, size_t row0,
                                                 int lane) {
  constexpr int I = kFusedI;
  const uint16_t* base = (lane < 32 ? bank.s : bank.b) + row0 * (I / 64);
  r.pw = reinterpret_cast<const uint32_t*>(base)[lane & 31];
}
template <int BITS>
__device__ __forceinline__ void load_rows_words(RowsRegs<BITS>& r, const QW& bank, size_t row0,
                                                int lane) {
  constexpr int WPR = kFusedI * BITS / 32;
  const uint32_t* src = bank.w + row0 * WPR;
#pragma unroll
  for (int i = 0; i < RowsRegs<BITS>::N; ++i) r.w[i] = load16_stream(src + (i * 64 + lane) * 4);
}

// One 8-value chunk of a down row at the lane's activations, in the order
// of the one-row-per-wave down dot: qa = sum q a and asum = sum a from +0,
// then fma(b, asum, s * qa).  Written with explicit fmaf so that the
// compiler cannot fuse the chunk sums of rows_dot into these products.
__device__ __forceinline__ float down_chunk8(uint32_t w0, uint32_t w1, const float* a,
                                             float dsc, float dbi) {
  const float asum = ((((((a[0] + a[1]) + a[2]) + a[3]) + a[4]) + a[5]) + a[6]) + a[7];
  float qa = 0.0f;
  qa = qdot_word8(w0, a[0], a[1], a[2], a[3], qa);
  qa = qdot_word8(w1, a[4], a[5], a[6], a[7], qa);
  return fmaf(dbi, asum, dsc * qa);
}
__device__ __forceinline__ float down_chunk4(uint32_t wd, const float* a, float dsc,
                                             float dbi) {
  const float asum = ((((((a[0] + a[1]) + a[2]) + a[3]) + a[4]) + a[5]) + a[6]) + a[7];
  const uint32_t lo = wd & 0x0F0F0F0Fu;
  const uint32_t hi = (wd >> 4) & 0x0F0F0F0Fu;
  float qa = 0.0f;
  qa = fmaf((float)(lo & 0xFFu), a[0], qa);
  qa = fmaf((float)(hi & 0xFFu), a[1], qa);
  qa = fmaf((float)((lo >> 8) & 0xFFu), a[2], qa);
  qa = fmaf((float)((hi >> 8) & 0xFFu), a[3], qa);
  qa = fmaf((float)((lo >> 16) & 0xFFu), a[4], qa);
  qa = fmaf((float)((hi >> 16) & 0xFFu), a[5], qa);
  qa = fmaf((float)(lo >> 24), a[6], qa);
  qa = fmaf((float)(hi >> 24), a[7], qa);
  return fmaf(dbi, asum, dsc * qa);
}

// The eight rows' dots.  The reduction tree is the one-row-per-wave one
// (chunks of 8 values paired 1, 2, 4, ... apart), so every row's fp32 sum is
// bit-identical to it: 8-bit rows hold two chunks per lane (level 1 inside
// the lane, levels 2-6 across 32 lanes), 4-bit rows four (levels 1-2 inside
// the lane, 3-6 across 16 lanes).  Returns in lane 32 b (8-bit) or 16 b
// (4-bit) of y[i] the sum of row (8-bit) 2 i + b or (4-bit) 4 i + b.
template <int BITS>
__device__ __forceinline__ void rows_dot(const RowsRegs<BITS>& r, const float* s_act, int lane,
                                         float (&y)[RowsRegs<BITS>::N]) {
  constexpr int N = RowsRegs<BITS>::N;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if constexpr (BITS == 8) {
      const int row = 2 * i + (lane >> 5);
      const int pi = row * 8 + ((lane & 31) >> 2);
      const float dsc = param_of(r.pw, 0, pi);
      const float dbi = param_of(r.pw, 32, pi);
      const float* a = s_act + (lane & 31) * 16;
      float av[16];
#pragma unroll
      for (int k = 0; k < 16; k += 4) {
        const float4 f = *reinterpret_cast<const float4*>(a + k);
        av[k] = f.x;
        av[k + 1] = f.y;
        av[k + 2] = f.z;
        av[k + 3] = f.w;
      }
      y[i] = down_chunk8(r.w[i].x, r.w[i].y, av, dsc, dbi) +
             down_chunk8(r.w[i].z, r.w[i].w, av + 8, dsc, dbi);
    } else {
      const int row = 4 * i + (lane >> 4);
      const int pi = row * 8 + ((lane & 15) >> 1);
      const float dsc = param_of(r.pw, 0, pi);
      const float dbi = param_of(r.pw, 32, pi);
      const float* a = s_act + (lane & 15) * 32;
      float av[32];
#pragma unroll
      for (int k = 0; k < 32; k += 4) {
        const float4 f = *reinterpret_cast<const float4*>(a + k);
        av[k] = f.x;
        av[k + 1] = f.y;
        av[k + 2] = f.z;
        av[k + 3] = f.w;
      }
      y[i] = (down_chunk4(r.w[i].x, av, dsc, dbi) + down_chunk4(r.w[i].y, av + 8, dsc, dbi)) +
             (down_chunk4(r.w[i].z, av + 16, dsc, dbi) + down_chunk4(r.w[i].w, av + 24, dsc, dbi));
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) y[i] += dpp_f(y[i], 0xB1);
#pragma unroll
  for (int i = 0; i < N; ++i) y[i] += dpp_f(y[i], 0x4E);
#pragma unroll
  for (int i = 0; i < N; ++i) y[i] += dpp_f(y[i], 0x141);
#pragma unroll
  for (int i = 0; i < N; ++i) y[i] += dpp_f(y[i], 0x140);
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      y[i] += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(y[i]), 0x401F));
  }
}

// The one-row-per-wave down dot of a full row (lane l: values 8 l .. 8 l + 7).
template <int BITS>
__device__ __forceinline__ float row_dot(const DownRegs<Shape<BITS>::DN_WPL>& d, uint32_t pw,
                                         const float* s_act, int lane) {
  const int gd = lane >> 3;
  const float dsc = param_of(pw, 0, gd);
  const float dbi = param_of(pw, 4, gd);
  const float4 a0 = *reinterpret_cast<const float4*>(s_act + lane * 8);
  const float4 a1 = *reinterpret_cast<const float4*>(s_act + lane * 8 + 4);
  const float a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  float c;
  if constexpr (BITS == 8)
    c = down_chunk8(d.w[0], d.w[1], a, dsc, dbi);
  else
    c = down_chunk4(d.w[0], a, dsc, dbi);
  return wave_sum(c);
}

// This lane's x values of its gate/up chunks (lane + 64 i) and their sums.
template <int BITS>
__device__ __forceinline__ void load_xv(const float* s_in, int lane,
                                        float (&xv)[Shape<BITS>::GU_CPL][Shape<BITS>::VPC],
                                        float (&xs)[Shape<BITS>::GU_CPL]) {
  using S = Shape<BITS>;
#pragma unroll
  for (int i = 0; i < S::GU_CPL; ++i) {
    const int ch = lane + 64 * i;
    xs[i] = 0.0f;
#pragma unroll
    for (int v = 0; v < S::VPC; v += 4) {
      const float4 f = *reinterpret_cast<const float4*>(s_in + ch * S::VPC + v);
      xv[i][v] = f.x;
      xv[i][v + 1] = f.y;
      xv[i][v + 2] = f.z;
      xv[i][v + 3] = f.w;
    }
#pragma unroll
    for (int v = 0; v < S::VPC; ++v) xs[i] += xv[i][v];
  }
}

// SwiGLU activation (bf16 bits) of one gate/up pair held in registers.
// Per 16-byte chunk: acc += fma(s, sum q x, b * sum x) (explicit, so every
// chunk rounds the same way), then the butterfly.
template <int BITS>
__device__ __forceinline__ uint32_t pair_act(const PairRegs<Shape<BITS>::GU_CPL>& pr,
                                             const float (&xv)[Shape<BITS>::GU_CPL][Shape<BITS>::VPC],
                                             const float (&xs)[Shape<BITS>::GU_CPL], int lane) {
  using S = Shape<BITS>;
  float au = 0.0f, ag = 0.0f;
#pragma unroll
  for (int i = 0; i < S::GU_CPL; ++i) {
    const int ch = lane + 64 * i;
    const int g = (ch * S::VPC) >> 6;
    au += fmaf(param_of(pr.pw, 0, g), qdot_chunk<BITS>(pr.wu[i], xv[i]),
               param_of(pr.pw, 32, g) * xs[i]);
    ag += fmaf(param_of(pr.pw, 16, g), qdot_chunk<BITS>(pr.wg[i], xv[i]),
               param_of(pr.pw, 48, g) * xs[i]);
  }
  au = wave_sum(au);
  ag = wave_sum(ag);
  const float up = round_bf16(au);
  const float gate = round_bf16(ag);
  return f32_to_bf16(silu(gate) * up);
}


// out = bf16(sum_u coef[u] * y[u]) in slot order (the shared unit, slot K,
// last), then the residual: the combine of the one-row-per-wave kernel.
__device__ __forceinline__ uint32_t combine_row(const float* y, int yst, const float* coef,
                                                int K, bool has_shared, int residual_mode,
                                                float x_in, const uint16_t* residual, int h) {
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kMaxFusedRouted; ++u)
    if (u < K) acc += coef[u] * y[u * yst];
  if (has_shared) acc += coef[K] * y[K * yst];
  float o = round_bf16(acc);
  if (residual_mode == 1)
    o = round_bf16(x_in + o);
  else if (residual_mode == 2)
    o = round_bf16(bf16_to_f32(residual[h]) + o);
  return f32_to_bf16(o);
}

// Buffer resource over [p, p + bytes): loads past the end return zero
// without touching memory, so a load of a part a layer does not have (no
// shared expert, a router row past E) is issued like any other.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
constexpr int kNt = 2;   // non-temporal (weights read once)
// Gate rows (router, shared gate): every XCD reads every row of a layer, so
// they are loaded with the default policy and the memory-side cache serves
// seven of the eight reads (the 40-layer 8-bit chain ran 12.59 -> 12.18 us
// per layer, 4-bit 12.21 -> 11.57, against non-temporal loads).
constexpr int kShared = 0;
constexpr int kSc1 = 16; // agent coherence

// Routing-independent loads of one layer held by a loader wave (waves 4-7,
// q = wave - 4) until it writes them to LDS at the start of the layer:
// router rows 2 q and 2 q + 1 of the workgroup (row j + 32 w), wave 5 the
// shared gate's row, wave 4 the RMSNorm weights.  bf16 rows: four 16-byte
// chunks per lane; 8-bit rows: two code chunks per lane and, in lanes 0-7,
// the row's 32 scales (lanes 0-3) and 32 biases (lanes 4-7).
struct LoaderRegs {
  uint4 g[3][4];
  uint4 nwv[4];
};

template <int RQ>
__device__ __forceinline__ void load_gate_rows(uint4 (&g)[4], const uint16_t* w16, const QW& q,
                                               int row, int rows, int lane) {
  constexpr int H = kFusedH;
  if constexpr (RQ == 0) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(w16, (uint32_t)rows * H * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
          rs, (row * H + (lane + 64 * i) * 8) * 2, 0, kShared);
      g[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
  } else {
    const __amdgpu_buffer_rsrc_t rw = rsrc(q.w, (uint32_t)rows * H);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, row * H + (lane + 64 * i) * 16,
                                                            0, kShared);
      g[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
    // lanes 0-3: scales, 4-7: biases (16 bytes each); other lanes past the end
    const __amdgpu_buffer_rsrc_t rp =
        rsrc(lane < 4 ? (const void*)q.s : (const void*)q.b, (uint32_t)rows * (H / 64) * 2);
    const int off = lane < 8 ? row * (H / 64) * 2 + (lane & 3) * 16 : rows * (H / 64) * 2;
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, 0);
    g[2] = make_uint4(v.x, v.y, v.z, v.w);
  }
}

// LDS image of one gate row (4096 bytes): bf16 [H], or 8-bit codes [H] then
// 32 bf16 scales and 32 bf16 biases.
template <int RQ>
__device__ __forceinline__ void store_gate_row_lds(char* slot, const uint4 (&g)[4], int lane) {
  if constexpr (RQ == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(slot + (lane + 64 * i) * 16) = g[i];
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<uint4*>(slot + (lane + 64 * i) * 16) = g[i];
    if (lane < 8) *reinterpret_cast<uint4*>(slot + kFusedH + lane * 16) = g[2];
  }
}
template <int RQ>
__device__ __forceinline__ void gate_row_from_lds(GateRow<RQ>& r, const char* slot, int lane) {
  if constexpr (RQ == 0) {
#pragma unroll
    for (int i = 0; i < GateRow<0>::C; ++i)
      r.w[i] = *reinterpret_cast<const uint4*>(slot + (lane + 64 * i) * 16);
  } else {
    const uint16_t* sb = reinterpret_cast<const uint16_t*>(slot + kFusedH);
#pragma unroll
    for (int i = 0; i < GateRow<1>::C; ++i) {
      const int ch = lane + 64 * i;
      r.w[i] = *reinterpret_cast<const uint4*>(slot + ch * 16);
      r.s[i] = sb[ch >> 2];
      r.b[i] = sb[32 + (ch >> 2)];
    }
  }
}

// Eight down rows through a buffer resource (rows past `rows` read as zero).
template <int BITS>
__device__ __forceinline__ void load_rows_buf(RowsRegs<BITS>& r, const QW& bank, uint32_t rows,
                                              uint32_t row0, int lane) {
  constexpr int I = kFusedI;
  constexpr int WPR = I * BITS / 32;
  const __amdgpu_buffer_rsrc_t rp =
      rsrc(lane < 32 ? (const void*)bank.s : (const void*)bank.b, rows * (I / 64) * 2);
  r.pw = __builtin_amdgcn_raw_buffer_load_b32(rp, row0 * (I / 64) * 2 + (lane & 31) * 4, 0, 0);
  const __amdgpu_buffer_rsrc_t rw = rsrc(bank.w, rows * WPR * 4);
#pragma unroll
  for (int i = 0; i < RowsRegs<BITS>::N; ++i) {
    const u32x4 v =
        __builtin_amdgcn_raw_buffer_load_b128(rw, (row0 * WPR + (i * 64 + lane) * 4) * 4, 0, kNt);
    r.w[i] = make_uint4(v.x, v.y, v.z, v.w);
  }
}

// Gate/up pair (up row c, gate row c + I of bank row base) through buffer
// loads: the same registers and lane layout as load_pair_params/words.
template <int BITS, int CPL>
__device__ __forceinline__ void load_pair_buf(PairRegs<CPL>& r, const QW& bank, uint32_t rows,
                                              int up_row, int lane) {
  using S = Shape<BITS>;
  const int prow = up_row + ((lane >> 4) & 1) * S::I;
  const __amdgpu_buffer_rsrc_t rp = rsrc(lane < 32 ? (const void*)bank.s : (const void*)bank.b,
                                         rows * (S::H / 64) * 2);
  r.pw = __builtin_amdgcn_raw_buffer_load_b32(rp, (prow * (S::H / 64) + (lane & 15) * 2) * 2, 0,
                                              0);
  issue_fence();
  const __amdgpu_buffer_rsrc_t rw = rsrc(bank.w, rows * (S::H * BITS / 8));
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int ch = lane + 64 * i;
    const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rw, up_row * S::GU_WPR * 4 + ch * 16,
                                                          0, kNt);
    const u32x4 g = __builtin_amdgcn_raw_buffer_load_b128(
        rw, (up_row + S::I) * S::GU_WPR * 4 + ch * 16, 0, kNt);
    r.wu[i] = make_uint4(u.x, u.y, u.z, u.w);
    r.wg[i] = make_uint4(g.x, g.y, g.z, g.w);
  }
}

// Full down row h (lane l: values 8 l .. 8 l + 7) and its scale/bias word
// (lanes 0-7) through buffer loads.
template <int BITS>
__device__ __forceinline__ void load_down_row_buf(DownRegs<Shape<BITS>::DN_WPL>& d, uint32_t& pw,
                                                  const QW& bank, uint32_t rows, int h,
                                                  int lane) {
  using S = Shape<BITS>;
  const __amdgpu_buffer_rsrc_t rp =
      rsrc(lane < 4 ? (const void*)bank.s : (const void*)bank.b, rows * (S::I / 64) * 2);
  pw = __builtin_amdgcn_raw_buffer_load_b32(
      rp, lane < 8 ? (h * (S::I / 64) + (lane & 3) * 2) * 2 : rows * (S::I / 64) * 2, 0, 0);
  const __amdgpu_buffer_rsrc_t rw = rsrc(bank.w, rows * (S::I * BITS / 8));
  if constexpr (S::DN_WPL == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rw, (h * S::DN_WPR + lane * 2) * 4, 0, 0);
    d.w[0] = v[0];
    d.w[1] = v[1];
  } else {
    d.w[0] = __builtin_amdgcn_raw_buffer_load_b32(rw, (h * S::DN_WPR + lane) * 4, 0, 0);
  }
}

template <int BITS, int RQ, bool NORM>
__global__ __launch_bounds__(kThreads) void fused_decode_kernel(const FusedArgs p) {
  using S = Shape<BITS>;
  constexpr int H = S::H;
  constexpr int I = S::I;
  constexpr int VPC = S::VPC;
  constexpr int CPL = S::GU_CPL;
  constexpr int NU = kMaxFusedUnits;
  constexpr int kStageX = H / kThreads;        // 4
  constexpr int kPer = kFusedMaxExperts / 64;  // keys per lane (4)
  constexpr int NR = RowsRegs<BITS>::N;
  constexpr int kRoutedPairs = I / kXcdWaves;  // 2
  constexpr int kPollers = 4;                  // waves 0-3: hand-overs, no prefetch
  constexpr int kCombRows = kXcdRows * kWaves / kPollers;  // 16 rows per polling wave
  constexpr int kRowSlot = 4096;               // bytes per gate row image in LDS
  static_assert(kPer == 4 && kRoutedPairs == 2, "layout");
  static_assert(H / 256 / kPollers == 2, "x hand-over: two 16-byte pieces per lane");
  const int wg = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane0 = threadIdx.x & 63;
  // this workgroup's XCD (HW_REG_XCC_ID, hardware register 20, bits 3:0)
  const uint32_t hw_xcc = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_s_getreg((3 << 11) | 20));
  const int xcd = (int)(hw_xcc & 7u);
  const int j = wg >> 3;   // workgroup within the XCD (the XCDs are dealt in turn)
  const int K = p.K;
  const int E = p.E;
  const bool has_shared = p.has_shared != 0;
  const int U = K + (has_shared ? 1 : 0);
  const bool routed = xcd < K;            // workgroup-uniform
  const bool loader = wave >= kPollers;   // wave-uniform
  const int q = wave - kPollers;          // loader index (0-3)
  const int row = j + kXcdWgs * wave;     // router row of this wave (< 256)
  const int vg = j + kXcdWgs * wave;      // routed pairs vg, vg + 256
  const int rrow0 = (j * kWaves + wave) * kXcdRows;  // routed down rows (8)
  // shared: pair of waves 6 and 7; the workgroup's eight down rows hsr0 ..
  // hsr0 + 7 (8-bit: rows 2 q, 2 q + 1 of them on loader q; 4-bit: all on
  // wave kShDownWave)
  const bool sp_wave = wave >= kSharedPairWave;
  const int spair = xcd * kSharedPairsPerXcd + (j + kXcdWgs * (wave - kSharedPairWave));
  const int hsr0 = xcd * kXcdWaves + j * kXcdRows;
  const int c_own = j * (kWaves * kXcdRows) + wave * kCombRows;  // combine rows (pollers)
  FusedScratch* sc = p.scratch;

  __shared__ float s_x[2][H];
  __shared__ float s_n[NORM ? H : 4];
  __shared__ __align__(16) char s_rw[9][kRowSlot];  // router rows 0-7, shared gate row
  __shared__ uint16_t s_nw[NORM ? H : 8];
  __shared__ float s_act[I];
  __shared__ float s_ash[I];
  __shared__ float s_y[kPollers][NU][kCombRows];
  __shared__ uint32_t s_yo[kWaves * kXcdRows + kXcdRows];  // this layer's unit outputs
  __shared__ int s_idx[NU];
  __shared__ float s_coef[NU];
  __shared__ uint32_t s_base, s_abort;

  uint32_t xin[kStageX];
#pragma unroll
  for (int jj = 0; jj < kStageX; ++jj)
    xin[jj] = (uint32_t)p.x[threadIdx.x + jj * kThreads] << 16;
  if (threadIdx.x == 0) {
    s_base = load_coherent_u32(&sc->epoch);
    s_abort = load_coherent_u32(&sc->abort);
  }

  PairRegs<CPL> pr[kRoutedPairs];
  PairRegs<CPL> spr;
  RowsRegs<BITS> dr;
  RowsRegs<BITS> shr;
  DownRegs<S::DN_WPL> sdr[2];
  uint32_t sdpw[2] = {0, 0};
  const int hs0 = hsr0 + 2 * q;
  LoaderRegs ld;

  // Loader waves: every routing-independent load of layer L (unconditional,
  // sized to zero where a part is absent).
  auto fetch_router = [&](const FusedLayer& L, int lane) {
    const int r0 = j + kXcdWgs * (2 * q), r1 = j + kXcdWgs * (2 * q + 1);
    load_gate_rows<RQ>(ld.g[0], L.router_w, L.rq, r0 < E ? r0 : E - 1, E, lane);
    load_gate_rows<RQ>(ld.g[1], L.router_w, L.rq, r1 < E ? r1 : E - 1, E, lane);
    issue_fence();
  };
  auto prefetch = [&](const FusedLayer& L, int lane) {
    if (q == 1) {
      const bool sg = shared_gated<RQ>(L, has_shared);
      load_gate_rows<RQ>(ld.g[2], L.sgate_w, L.sgq, 0, sg ? 1 : 0, lane);
    }
    if constexpr (NORM) {
      if (q == 0) {
        const __amdgpu_buffer_rsrc_t rn = rsrc(L.norm_w, H * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rn, (lane + 64 * i) * 16, 0, 0);
          ld.nwv[i] = make_uint4(v.x, v.y, v.z, v.w);
        }
      }
    }
    if constexpr (BITS == 8) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
        load_down_row_buf<BITS>(sdr[t], sdpw[t], L.sdn, has_shared ? H : 0, hs0 + t, lane);
    }
    if (q >= 2)
      load_pair_buf<BITS, CPL>(spr, L.sgu, sp_wave && has_shared ? 2 * I : 0,
                               sp_wave ? spair : 0, lane);
    issue_fence();
  };
  __syncthreads();
  const uint32_t base = s_base;
  WaitState wst{sc, base + 1, false};
  if (hw_xcc >= (uint32_t)kXcds) {
    wst.gave_up = true;
    if (threadIdx.x == 0) publish_failure(sc, wst.key, 2u);
  }
  // A call whose key is already in the abort word (set by the host to cancel
  // the call before it runs) waits for nothing and reports status 1.
  if (s_abort == wst.key) {
    wst.gave_up = true;
    if (threadIdx.x == 0) publish_failure(sc, wst.key, 1u);
  }

  for (int layer = 0; layer < p.n_layers; ++layer) {
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const FusedLayer L = layer_desc(p, layer);
    const bool last = layer == p.n_layers - 1;
    const int cur = layer & 1;
    const uint32_t tag = phase_tag(base + 1 + layer);
    const uint32_t prev_tag = phase_tag(base + layer);
    const bool sg_row = shared_gated<RQ>(L, has_shared);

    // ---- C: the layer input.  Pollers combine their rows of the previous
    // layer's unit outputs and collect x; loaders move their loads to LDS.
    if (layer == 0) {
#pragma unroll
      for (int jj = 0; jj < kStageX; ++jj)
        s_x[0][threadIdx.x + jj * kThreads] = __uint_as_float(xin[jj] & 0xFFFF0000u);
    }
    if (loader) {
      if (layer == 0) fetch_router(L, lane);
      prefetch(L, lane);
      store_gate_row_lds<RQ>(s_rw[2 * q], ld.g[0], lane);
      store_gate_row_lds<RQ>(s_rw[2 * q + 1], ld.g[1], lane);
      if (q == 1) store_gate_row_lds<RQ>(s_rw[8], ld.g[2], lane);
      if constexpr (NORM) {
        if (q == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(s_nw + (lane + 64 * i) * 8) = ld.nwv[i];
        }
      }
    } else if (layer > 0) {
      // unit outputs of rows c_own .. c_own + 15: lane 4 u + k loads rows
      // 4 k .. 4 k + 3 of unit u
      {
        const __amdgpu_buffer_rsrc_t rs = rsrc(sc->ys[cur ^ 1][0], NU * H * 4);
        const int u = lane >> 2, pc = lane & 3;
        bool pend = lane < 4 * U && !wst.gave_up;
        // unit u of the combine: routed slot u, or the shared expert's slot
        const int slot = u < K ? u : kMaxFusedRouted;
        const int off = (slot * H + c_own + 4 * pc) * 4;
        for (int spin = 0;; ++spin) {
          if (pend) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kSc1);
            if (tag_ok(v.x, prev_tag) && tag_ok(v.y, prev_tag) && tag_ok(v.z, prev_tag) &&
                tag_ok(v.w, prev_tag)) {
              *reinterpret_cast<float4*>(&s_y[wave][u][4 * pc]) = make_float4(
                  __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y & 0xFFFF0000u),
                  __uint_as_float(v.z & 0xFFFF0000u), __uint_as_float(v.w & 0xFFFF0000u));
              pend = false;
            }
          }
          if (!__any(pend)) break;
          if (give_up(wst, spin)) break;
          __builtin_amdgcn_s_sleep(1);
        }
      }
      __builtin_amdgcn_wave_barrier();
      if (lane < kCombRows) {
        const int h = c_own + lane;
        const uint32_t ob = combine_row(&s_y[wave][0][lane], kCombRows, s_coef, K, has_shared,
                                        p.residual_mode, s_x[cur ^ 1][h], p.residual, h);
        store_xcd_u32(sc->xl[xcd][cur], H, h, tagged(ob, tag));
      }
      poll_tagged<2, kXcdLoadAux>(sc->xl[xcd][cur], H, tag, s_x[cur], lane, wave, wst);
    }
    __syncthreads();
    float* const s_xc = s_x[cur];

    if constexpr (NORM) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < H / 512; ++i) {
        const float4 a = *reinterpret_cast<const float4*>(s_xc + (lane + 64 * i) * 8);
        const float4 b = *reinterpret_cast<const float4*>(s_xc + (lane + 64 * i) * 8 + 4);
        acc = fmaf(a.x, a.x, acc);
        acc = fmaf(a.y, a.y, acc);
        acc = fmaf(a.z, a.z, acc);
        acc = fmaf(a.w, a.w, acc);
        acc = fmaf(b.x, b.x, acc);
        acc = fmaf(b.y, b.y, acc);
        acc = fmaf(b.z, b.z, acc);
        acc = fmaf(b.w, b.w, acc);
      }
      const float ms = wave_sum(acc) / (float)H;
      const float r = 1.0f / sqrtf(ms + L.norm_eps);
      const float4 xv4 = *reinterpret_cast<const float4*>(s_xc + 4 * threadIdx.x);
      const uint2 nw = *reinterpret_cast<const uint2*>(s_nw + 4 * threadIdx.x);
      *reinterpret_cast<float4*>(s_n + 4 * threadIdx.x) =
          make_float4(round_bf16(round_bf16(xv4.x * r) * bf16_lo(nw.x)),
                      round_bf16(round_bf16(xv4.y * r) * bf16_hi(nw.x)),
                      round_bf16(round_bf16(xv4.z * r) * bf16_lo(nw.y)),
                      round_bf16(round_bf16(xv4.w * r) * bf16_hi(nw.y)));
      __syncthreads();
    }
    const float* const s_in = NORM ? s_n : s_xc;

    // ---- R: this wave's router row (from LDS).
    {
      GateRow<RQ> rw;
      gate_row_from_lds<RQ>(rw, s_rw[wave], lane);
      const float acc = wave_sum(gate_partial(rw, s_in, lane));
      if (lane == 0)
        store_xcd_u32(sc->logits[xcd], kFusedMaxExperts, row,
                      tagged(row < E ? f32_to_bf16(acc) : 0u, tag));
    }

    // ---- S: the shared pair of waves 6 and 7 (stored after the routed
    // loads are out).
    uint32_t s_a = 0;
    if (sp_wave && has_shared) {
      float xv[CPL][VPC], xs[CPL];
      load_xv<BITS>(s_in, lane, xv, xs);
      s_a = pair_act<BITS>(spr, xv, xs, lane);
    }

    // ---- K: rank the XCD's logits (wave 0).
    float lv[kPer];
    float m_top = 0.0f;
    uint32_t my = 0;
    uint32_t k[kPer] = {0u, 0u, 0u, 0u};
    uint32_t sel[NU - 1];
    if (wave == kPollWave) {
      const __amdgpu_buffer_rsrc_t rs = rsrc(sc->logits[xcd], E * 4);
      uint32_t w[kPer] = {0u, 0u, 0u, 0u};
      for (int spin = 0; !wst.gave_up; ++spin) {
        bool ok = true;
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, 0, kXcdLoadAux);
        w[0] = v.x;
        w[1] = v.y;
        w[2] = v.z;
        w[3] = v.w;
#pragma unroll
        for (int i = 0; i < kPer; ++i) ok &= 4 * lane + i >= E || tag_ok(w[i], tag);
        if (__all(ok)) break;
        if (give_up(wst, spin)) break;
        __builtin_amdgcn_s_sleep(1);
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int e = 4 * lane + i;
        const uint32_t b = w[i] >> 16;
        lv[i] = bf16_to_f32(b);
        k[i] = e < E ? ((bf16_order_key(b) << 16) | (0xFFFFu - (uint32_t)e)) : 0u;
      }
      cswap_desc(k[0], k[1]);
      cswap_desc(k[2], k[3]);
      cswap_desc(k[0], k[2]);
      cswap_desc(k[1], k[3]);
      cswap_desc(k[1], k[2]);
#pragma unroll
      for (int jj = 0; jj < NU - 1; ++jj) {
        sel[jj] = 0;
        if (jj < K && jj <= xcd) {
          const uint32_t best = wave_max_u32(k[0]);
          sel[jj] = best;
          if (k[0] == best) {
            k[0] = k[1];
            k[1] = k[2];
            k[2] = k[3];
            k[3] = 0;
          }
        }
      }
      m_top = bf16_to_f32(bf16_from_order_key(sel[0] >> 16));
      uint32_t mine = 0;
#pragma unroll
      for (int jj = 0; jj < NU - 1; ++jj)
        if (jj == xcd) mine = sel[jj];
      if (routed && lane == 0) s_idx[xcd] = (int)(0xFFFFu - (mine & 0xFFFFu));
    }
    __syncthreads();

    // ---- G: this XCD's routed expert (workgroup-uniform branch).
    const size_t e = routed ? (size_t)s_idx[xcd] : 0;
    if (routed) {
#pragma unroll
      for (int pp = 0; pp < kRoutedPairs; ++pp)
        load_pair_params<BITS, CPL>(pr[pp], L.gu, e * 2 * I + vg + kXcdWaves * pp, lane);
      load_rows_params<BITS>(dr, L.dn, e * H + (size_t)rrow0, lane);
      issue_fence();
#pragma unroll
      for (int pp = 0; pp < kRoutedPairs; ++pp)
        load_pair_words<BITS, CPL>(pr[pp], L.gu, e * 2 * I + vg + kXcdWaves * pp, lane);
      issue_fence();
      // the down rows right behind the gate/up rows (issued after the gate/up
      // math instead: 12.18 against 12.13 us per layer at 8 bits, 11.56
      // against 11.32 at 4 bits, once the gate rows came from the
      // memory-side cache)
      load_rows_words<BITS>(dr, L.dn, e * H + (size_t)rrow0, lane);
      issue_fence();
    }
    if (BITS == 4 && wave == kShDownWave) {
      // the shared down rows behind this wave's routed rows
      load_rows_buf<BITS>(shr, L.sdn, has_shared ? H : 0, hsr0, lane);
      issue_fence();
    }
    if (wave == kPollWave) {
      // the ranking rounds past this XCD's slot, now that the routed loads
      // are out (the K barrier waited only for the rounds up to it: 4-bit
      // chain 11.12 -> 11.03 us per layer, 8-bit 12.31 -> 12.27)
#pragma unroll
      for (int jj = 0; jj < NU - 1; ++jj) {
        if (jj < K && jj > xcd) {
          const uint32_t best = wave_max_u32(k[0]);
          sel[jj] = best;
          if (k[0] == best) {
            k[0] = k[1];
            k[1] = k[2];
            k[2] = k[3];
            k[3] = 0;
          }
        }
      }
#pragma unroll
      for (int jj = 0; jj < NU - 1; ++jj)
        if (lane == jj) my = sel[jj];
    }
    if (sp_wave && lane == 0) store_coherent_u32(sc->sact[cur] + spair, tagged(s_a, tag));
    if (routed) {
      float xv[CPL][VPC], xs[CPL];
      load_xv<BITS>(s_in, lane, xv, xs);
#pragma unroll
      for (int pp = 0; pp < kRoutedPairs; ++pp) {
        const uint32_t a = pair_act<BITS>(pr[pp], xv, xs, lane);
        if (lane == 0) store_xcd_u32(sc->xact[xcd], I, vg + kXcdWaves * pp, tagged(a, tag));
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if (lane == 0) {
      // an XCD without a routed slot in this call still tags its words
#pragma unroll
      for (int pp = 0; pp < kRoutedPairs; ++pp)
        store_xcd_u32(sc->xact[xcd], I, vg + kXcdWaves * pp, tagged(0u, tag));
    }

    // The next layer's router rows: issued inside the routed stream rather
    // than at the next layer's start, where they would queue in front of
    // the device-wide unit-output poll (13.45 -> 13.09 us per layer).
    if (loader && !last) fetch_router(layer_desc(p, layer + 1), lane);

    // ---- scores (wave 0), as in the one-row-per-wave kernel; the shared
    // gate's row comes from LDS.
    if (wave == kPollWave) {
      uint32_t wsg = 0;
      if (sg_row) {
        GateRow<RQ> sw;
        gate_row_from_lds<RQ>(sw, s_rw[8], lane);
        wsg = f32_to_bf16(wave_sum(gate_partial(sw, s_in, lane))) << 16;
      }
      float z = 0.0f;
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        if (4 * lane + i < E) z += __expf(lv[i] - m_top);
      z = wave_sum(z);
      const float pb =
          lane < K ? round_bf16(__expf(bf16_to_f32(bf16_from_order_key(my >> 16)) - m_top) / z)
                   : 0.0f;
      float total = 0.0f;
#pragma unroll
      for (int jj = 0; jj < NU - 1; ++jj)
        if (jj < K) total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pb), jj));
      if (lane < K) {
        const float score = p.norm ? round_bf16(pb / round_bf16(total)) : pb;
        s_coef[lane] = score;
        if (wg == 0 && last && p.idx_out) {
          p.idx_out[lane] = (int)(0xFFFFu - (my & 0xFFFFu));
          p.scores_out[lane] = score;
        }
      }
      if (lane == 0 && has_shared)
        s_coef[K] = sg_row ? round_bf16(sigmoid(bf16_to_f32(wsg >> 16))) : 1.0f;
    }

    // ---- the shared activations.  4-bit: wave kShDownWave collects them
    // and reduces the workgroup's eight shared down rows while the routed
    // activations are on their way (40-layer chain 11.42 -> 11.12 us per
    // layer; the same at 8 bits measured 12.3 -> 15.2 us, so 8-bit layers
    // keep two shared rows on each loader wave in D).
    if (BITS == 8 && (wave == 4 || wave == 5))
      poll_tagged<1, kSc1>(sc->sact[cur], I, tag, s_ash, lane, wave - 4, wst);
    if (BITS == 4 && wave == kShDownWave) {
      poll_tagged<2, kSc1>(sc->sact[cur], I, tag, s_ash, lane, 0, wst);
      float ysh[NR];
      rows_dot<BITS>(shr, s_ash, lane, ysh);
      constexpr int kLanesPerRow = BITS == 8 ? 32 : 16;
      if ((lane & (kLanesPerRow - 1)) == 0) {
#pragma unroll
        for (int i = 0; i < NR; ++i)
          s_yo[kWaves * kXcdRows + i * (64 / kLanesPerRow) + lane / kLanesPerRow] =
              tagged(has_shared ? f32_to_bf16(ysh[i]) : 0u, tag);
      }
    }

    // ---- collect the routed activations (XCD-local).
    if (routed && (wave == 2 || wave == 3))
      poll_tagged<1, kXcdLoadAux>(sc->xact[xcd], I, tag, s_act, lane, wave - 2, wst);
    __syncthreads();

    // ---- D: eight routed down rows per wave (8-bit: two shared rows per
    // loader wave as well); results to LDS.
    if (routed) {
      float y[NR];
      rows_dot<BITS>(dr, s_act, lane, y);
      constexpr int kLanesPerRow = BITS == 8 ? 32 : 16;
      if ((lane & (kLanesPerRow - 1)) == 0) {
#pragma unroll
        for (int i = 0; i < NR; ++i)
          s_yo[wave * kXcdRows + i * (64 / kLanesPerRow) + lane / kLanesPerRow] =
              tagged(f32_to_bf16(y[i]), tag);
      }
    } else if (lane < kXcdRows) {
      s_yo[wave * kXcdRows + lane] = tagged(0u, tag);
    }
    if (BITS == 8 && loader) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float y = has_shared ? row_dot<BITS>(sdr[t], sdpw[t], s_ash, lane) : 0.0f;
        if (lane == 0) s_yo[kWaves * kXcdRows + 2 * q + t] = tagged(f32_to_bf16(y), tag);
      }
    }
    __syncthreads();
    // ---- the workgroup's unit outputs, from one wave: 64 rows of this
    // XCD's routed slot (16-byte stores, lanes 0-15; zeros when the call
    // has no such slot) and 8 rows of the shared expert's slot (16-17).
    if (wave == kWaves - 1) {
      if (lane < 18) {
        const uint4 v = *reinterpret_cast<const uint4*>(s_yo + 4 * lane);
        const int dst = lane < 16 ? xcd * H + j * (kWaves * kXcdRows) + 4 * lane
                                  : kMaxFusedRouted * H + xcd * kXcdWaves + j * kXcdRows +
                                        4 * (lane - 16);
        u32x4 w;
        w.x = v.x;
        w.y = v.y;
        w.z = v.z;
        w.w = v.w;
        __builtin_amdgcn_raw_buffer_store_b128(w, rsrc(sc->ys[cur][0], NU * H * 4), dst * 4, 0,
                                               kSc1);
      }
    }
  }

  // ---- O: this wave's output row (8 per workgroup, all XCDs).
  {
    const int lane = lane0;
    const int last = p.n_layers - 1;
    const uint32_t tag = phase_tag(base + 1 + last);
    const int h = wg * kWaves + wave;
    const __amdgpu_buffer_rsrc_t rs = rsrc(sc->ys[last & 1][0], NU * H * 4);
    bool pend = lane < U && !wst.gave_up;
    const int slot = lane < K ? lane : kMaxFusedRouted;  // unit lane's slot
    uint32_t wv = 0;
    for (int spin = 0;; ++spin) {
      if (pend) {
        wv = __builtin_amdgcn_raw_buffer_load_b32(rs, (slot * H + h) * 4, 0, kSc1);
        pend = !tag_ok(wv, tag);
      }
      if (!__any(pend)) break;
      if (give_up(wst, spin)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    float y[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u)
      y[u] = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)wv, u) & 0xFFFF0000u);
    if (lane == 0)
      p.out[h] = (uint16_t)combine_row(y, 1, s_coef, K, has_shared, p.residual_mode,
                                       s_x[last & 1][h], p.residual, h);
  }
  // Workgroup 0 has read every workgroup's shared activations of the last
  // layer, each written after that workgroup read the epoch.
  if (wg == 0 && threadIdx.x == 0) store_coherent_u32(&sc->epoch, base + p.n_layers);
}

namespace {
template <int BITS, int RQ>
const void* fused_fn_n(int norm) {
  return norm ? (const void*)fused_decode_kernel<BITS, RQ, true>
              : (const void*)fused_decode_kernel<BITS, RQ, false>;
}
const void* fused_fn(int bits, int rq8, int norm) {
  if (bits == 8) return rq8 ? fused_fn_n<8, 1>(norm) : fused_fn_n<8, 0>(norm);
  return rq8 ? fused_fn_n<4, 1>(norm) : fused_fn_n<4, 0>(norm);
}
}  // namespace

hipError_t fused_grid(int bits, int rq8, int norm, int* grid) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  // Occupancy does not change for a device: cache it (grid + 1, 0 = unknown).
  static int cache[64][8];
  const int slot = (bits == 8 ? 0 : 4) + (rq8 ? 2 : 0) + (norm ? 1 : 0);
  if (dev >= 0 && dev < 64) {
    const int c = __atomic_load_n(&cache[dev][slot], __ATOMIC_RELAXED);
    if (c > 0) {
      *grid = c - 1;
      return hipSuccess;
    }
  }
  int cus = 0;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fused_fn(bits, rq8, norm),
                                                   kThreads, 0);
  if (e != hipSuccess) return e;
  // one workgroup per CU, 32 on each of the 8 XCDs (0: not this device)
  *grid = per_cu >= 1 && cus >= kFusedXcdGrid ? kFusedXcdGrid : 0;
  if (dev >= 0 && dev < 64) __atomic_store_n(&cache[dev][slot], *grid + 1, __ATOMIC_RELAXED);
  return hipSuccess;
}

hipError_t launch_fused_decode(const FusedArgs& a, int bits, int grid, hipStream_t s) {
  if (grid != kFusedXcdGrid) return hipErrorInvalidValue;
  FusedArgs args = a;
  void* kargs[] = {&args};
  const void* fn = fused_fn(bits, a.rq8, a.rms_norm);
  // A cooperative launch guarantees every workgroup is resident.  Under
  // stream capture, or when the caller has turned cooperative launches off,
  // a plain launch of the same grid is made instead (every workgroup fits at
  // once on an otherwise idle device; the bounded waits turn anything else
  // into a status error).
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (!cooperative_launch_enabled() ||
      (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone))
    return hipLaunchKernel(fn, dim3(grid), dim3(kThreads), kargs, 0, s);
  return hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kThreads), kargs, 0, s);
}

}  // namespace rmoe
