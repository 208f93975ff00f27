// Launch-side view of the kernels: argument blocks and launchers.  Host code
// (abi.cpp) validates every shape before calling a launcher.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rmoe {

constexpr int kMaxExperts = 1024;  // router ranks at most this many experts
constexpr int kMaxTopK = 64;       // one slot per lane in the ranking wave
constexpr int kUnitBatch = 9;      // down kernel: loads in flight per lane
constexpr int kMaxTokens = 65535;  // grid.y of the router; counters reserved
constexpr int kRouterBatch = 4;    // router: 16-byte loads in flight per lane
constexpr int kStageBatch = 8;     // down: float4 act loads in flight per lane
constexpr int kMaxGateUpChunksPerLane = 4;  // gate_up_kernel: 256 chunks per row

struct QW {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
};

struct FusedScratch;

// One decode-shaped call: T tokens, K routed slots, an optional shared
// expert (unit K of every token).
struct DecodeArgs {
  int T, H, I, E, K, has_shared, norm;
  int switch_mode;   // 1: idx are caller indices, range-checked per use
  int rq8;           // 1: the gates are 8-bit MLX-affine banks (rq, sgq)
  int has_sg;        // the shared expert has a sigmoid gate (sgate_w or sgq)
  const uint16_t* x;
  const uint16_t* router_w;   // bf16 gates (rq8 == 0)
  const uint16_t* sgate_w;
  QW rq, sgq;                 // quantized gates [E, H] / [1, H] (rq8 == 1)
  QW gu, dn, sgu, sdn;
  float* logits;     // [T, E + 1]
  int32_t* idx;      // [T, K]   (switch path: caller's indices)
  float* scores;     // [T, score_stride] (router: K + 1, slot K = shared gate)
  int score_stride;  // K + 1 (the router's scores) or K (caller weights)
  float* act;        // [T, K + has_shared, I]
  uint32_t* ctr;     // [T] zero between calls
  int few_bits;      // 8 | 4: the few-token kernels at these bits (act is
                     // bf16; the router launch also computes the shared
                     // expert's gate/up); 0: the general kernels
  uint16_t* out;     // [T, H] (block) or [T, K, H] (switch)
  const uint16_t* residual;
  int32_t* idx_out;
  float* scores_out;
  FusedScratch* fs;  // epoch and status words (the few-token router's tagged hand-over)
  // matrix-core router: its logits come in logit_planes partial planes of
  // [T, E + 1] (one per share of H, summed in plane order), and for a bf16
  // gate the row bounds as that many planes of partial sums of squares
  int logit_planes;
};

struct QmvArgs {
  int M, N, K;
  int x_rows, experts;  // lhs / rhs outside [0, x_rows) / [0, experts) -> zero row
  const uint16_t* x;
  const int32_t* lhs;
  const int32_t* rhs;
  QW w;
  uint16_t* y_bf16;
  float* y_f32;
};

// ---- single-launch decode (fused.hip): one token, one or more layers.
constexpr int kFusedThreads = 512;          // 8 waves, one workgroup per CU
constexpr int kFusedXcdGrid = 256;          // workgroups: 32 on each of the 8 XCDs
constexpr int kMaxFusedRouted = 8;          // routed slots (one per XCD)
constexpr int kMaxFusedUnits = kMaxFusedRouted + 1;  // plus the shared expert
constexpr int kFusedMaxExperts = 256;       // one router row per wave of an XCD
constexpr int kFusedH = 2048;
constexpr int kFusedI = 512;
// ---- few-token decode (decode.hip): 2..8 tokens at the shapes above.
constexpr int kFewMaxTokens = 8;

struct FusedLayer {
  const uint16_t* router_w;
  const uint16_t* sgate_w;
  QW gu, dn, sgu, sdn;
  QW rq, sgq;                 // 8-bit gates when the call's rq8 is set
  const uint16_t* norm_w;     // RMSNorm weights [H] when the call's norm is set
  float norm_eps;
};

// Device scratch of the fused kernel: lives at a fixed workspace offset so
// the epoch persists across calls of any shape.  Values handed between
// workgroups are tagged words: (bf16 value << 16) | (phase % 65535 + 1).
// Rows indexed by XCD are written and read inside that XCD only (its L2).
// err is the status word (0 ok, 1 a wait gave up, 2 a workgroup did not run
// on XCD i % 8); abort holds the first phase of a call in which a workgroup
// gave up, so that the other workgroups of that call stop waiting.
struct FusedScratch {
  uint32_t epoch;
  uint32_t err;
  uint32_t abort;
  uint32_t pad[61];
  uint32_t logits[8][kFusedMaxExperts];       // router logits of XCD x
  uint32_t xact[8][kFusedI];                  // routed activations of XCD x
  uint32_t sact[2][kFusedI];                  // shared activations, by layer parity
  uint32_t ys[2][kMaxFusedUnits][kFusedH];    // unit outputs, by layer parity
  uint32_t xl[8][2][kFusedH];                 // combined layer input of XCD x, by parity
  // the few-token router's logits, as tagged words (token t, expert e; the
  // shared gate's at e = E): only that router writes here, and its ranking
  // workgroup clears every word it has read
  uint32_t few[kFewMaxTokens][kFusedMaxExperts + 1];
};

struct FusedArgs {
  int n_layers, E, K, norm, has_shared;
  int rq8;                    // gates are 8-bit MLX-affine (every layer)
  int rms_norm;               // RMSNorm of the layer input (every layer)
  int residual_mode;          // 0 none, 1 the layer input, 2 `residual`
  FusedLayer layer0;          // used when table == nullptr
  const FusedLayer* table;    // device array of n_layers descriptors
  const uint16_t* x;
  uint16_t* out;
  const uint16_t* residual;
  FusedScratch* scratch;
  int32_t* idx_out;
  float* scores_out;
};

hipError_t fused_grid(int bits, int rq8, int rms_norm, int* grid);
hipError_t launch_fused_decode(const FusedArgs& a, int bits, int grid, hipStream_t s);
// rmoe_set_cooperative_launch's process-wide mode (abi.cpp).
bool cooperative_launch_enabled();

hipError_t launch_router(const DecodeArgs& a, hipStream_t s);
// RMSNorm of T rows of H bf16 values (H a multiple of 8; x, w, out 16-byte aligned).
hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* w, int T, int H, float eps,
                          uint16_t* out, hipStream_t s);
// Many-token router on the matrix cores with exact selection (prefill).
bool router_mfma_eligible(int E, int H);
int router_logit_planes(int T);
// wnorm: [E] floats; split: [2, E, H] bf16 (quantized gates only)
hipError_t launch_router_mfma(const DecodeArgs& a, float* wnorm, uint16_t* split,
                              hipStream_t s);
hipError_t launch_gate_up(const DecodeArgs& a, int bits, hipStream_t s);
hipError_t launch_down(const DecodeArgs& a, int bits, bool combine, hipStream_t s);
hipError_t launch_qmv(const QmvArgs& a, int bits, hipStream_t s);

hipError_t launch_quantize(const float* w, int64_t rows, int cols, int bits,
                           uint32_t* wq, uint16_t* s, uint16_t* b, hipStream_t st);
hipError_t launch_dequantize(const QW& q, int cols, int bits, int64_t row_begin,
                             int64_t rows, float* out_f32, uint16_t* out_bf16,
                             hipStream_t st);
hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* partials,
                              int blocks, hipStream_t st);

// ---- prefill (prefill.hip): expert-sorted grouped dequant-GEMM on MFMA.
constexpr int kPrefillMaxExperts = 512;  // buckets of the one-workgroup sort
constexpr int kPrefillBM = 128;          // sorted rows per m-tile (long prefill)
constexpr int kPrefillMaxSlices = 64;   // sorting workgroups at most
constexpr int kPrefillTileN = 128;       // [up; gate] pairs per gate/up tile
constexpr int kPrefillMinRows = 64;      // (token, slot) rows that select it

struct PrefillArgs {
  int T, H, I, E, K, has_shared;
  int bm;                  // rows per m-tile (set by launch_prefill)
  int dense;               // 1: rows 0..T-1 of expert 0 in order (no sort; tiles from T)
  const uint16_t* x;       // [T, H]
  const int32_t* idx;      // [T, K] expert ids (out of range -> zero rows)
  QW gu, dn, sgu, sdn;
  int32_t* rows;           // [T K + T] source row of each sorted row
  int32_t* offs;           // [E + 3] rows per bucket (E: shared, E + 1: bad ids)
  int32_t* tile_offs;      // [E + 3]: [E + 1] = full m-tiles, [E + 2] = all m-tiles
  int32_t* tile_desc;      // [m-tiles][4]: bucket, first sorted row, rows, 0
  int32_t* hist;           // [sort slices][E + 2] rows per bucket of each slice
  uint16_t* act;           // [T K + T, I] bf16, sorted order
  uint16_t* y;             // [T K (+ T), H] bf16 at row t K + j (shared: T K + t)
  const float* scores;     // [T, score_stride] router scores, slot K = shared gate
  int score_stride;        // K + 1 (the router's) or K (caller weights, no shared)
  const uint16_t* residual;
  uint16_t* out;           // [T, H]
};

// ---- the static scratch of rmoe_moe_block_noalloc (noalloc.hip).
constexpr size_t kStaticScratchBytes = size_t(16) << 20;
// Device address of this device's copy (looked up once per device).
// Device address of the static scratch on the device `stream` runs on.
hipError_t static_scratch(hipStream_t stream, void** out);
// *out = *word, then *word = 0 (one tiny kernel on `s`).
hipError_t launch_take_status(uint32_t* word, uint32_t* out, hipStream_t s);

int prefill_tile_rows(int T, int K, int E);
int prefill_max_mtiles(int T, int K, int E, int bm);
int prefill_sort_slices(int T, int K);
hipError_t launch_prefill(const PrefillArgs& a, int bits, bool combine, hipStream_t s);
// y[m] = x[m] . deq(w)^T on the matrix cores for M >= kDenseQmmMinRows rows
// (mx.quantized_matmul at prefill sizes): every dequantised weight rounded
// to bf16, fp32 accumulation, bf16 out.  Shapes: K % 128 == 0, N % 256 == 0.
constexpr int kDenseQmmMinRows = 64;
bool dense_qmm_eligible(int M, int N, int K);
hipError_t launch_dense_qmm(const uint16_t* x, int M, const QW& w, int N, int K, int bits,
                            uint16_t* y, hipStream_t s);

}  // namespace rmoe
