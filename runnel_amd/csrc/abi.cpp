// C ABI: host-side validation and dispatch.  Every argument is checked
// before anything is launched; failures return a negative RMOE_E* code and
// leave a message for rmoe_last_error().  Nothing here allocates device
// memory.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <string>

#include "kernels.h"
#include "rmoe.h"

static_assert(RMOE_NOALLOC_SCRATCH_BYTES == rmoe::kStaticScratchBytes,
              "the header states the static scratch size");

namespace {

thread_local std::string g_error;
std::atomic<int> g_cooperative{0};  // rmoe_set_cooperative_launch (plain by default)

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int ok() {
  g_error.clear();
  return RMOE_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(RMOE_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

int values_per_chunk(int bits) { return bits == 8 ? 16 : 32; }

int check_qweight(const rmoe_qweight* q, const char* name) {
  if (!q) return fail(RMOE_ENULL, "%s: descriptor is NULL", name);
  if (!q->w || !q->scales || !q->biases)
    return fail(RMOE_ENULL, "%s: weight, scales and biases are required", name);
  if (q->bits != 4 && q->bits != 8)
    return fail(RMOE_EBITS, "%s: bits must be 4 or 8 (got %d)", name, q->bits);
  if (q->group_size != 64)
    return fail(RMOE_EBITS, "%s: group_size must be 64 (got %d)", name,
                q->group_size);
  if (q->experts < 1 || q->rows < 1 || q->cols < 64 || q->cols % 64)
    return fail(RMOE_EINVAL,
                "%s: need experts >= 1, rows >= 1, cols a positive multiple of "
                "64 (got %d, %d, %d)",
                name, q->experts, q->rows, q->cols);
  if (!aligned(q->w, 16))
    return fail(RMOE_EALIGN, "%s: packed weight must be 16-byte aligned", name);
  if (!aligned(q->scales, 2) || !aligned(q->biases, 2))
    return fail(RMOE_EALIGN, "%s: scales/biases must be 2-byte aligned", name);
  return RMOE_OK;
}

// A quantized gate: one 8-bit group-64 bank [1, rows, hidden] (the format of
// the checkpoints' mlp.gate / mlp.shared_expert_gate).
int check_gate_q(const rmoe_qweight* q, int rows, int hidden, const char* name) {
  int rc;
  if ((rc = check_qweight(q, name))) return rc;
  if (q->bits != 8)
    return fail(RMOE_EBITS, "%s: quantized gates must be 8-bit (got %d)", name, q->bits);
  if (q->experts != 1 || q->rows != rows || q->cols != hidden)
    return fail(RMOE_EINVAL, "%s must be [1, %d, %d] (got [%d, %d, %d])", name, rows, hidden,
                q->experts, q->rows, q->cols);
  return RMOE_OK;
}

// The down-projection kernel maps one row onto inter/values_per_chunk lanes.
int check_down_width(int inter, int bits, const char* name) {
  const int chunks = inter / values_per_chunk(bits);
  if (inter % values_per_chunk(bits) || !pow2(chunks) || chunks > 64)
    return fail(RMOE_EINVAL,
                "%s: intermediate size %d unsupported at %d bits (needs "
                "inter/%d a power of two <= 64)",
                name, inter, bits, values_per_chunk(bits));
  return RMOE_OK;
}

// The few-token gate/up kernel gives each lane at most kMaxGateUpChunksPerLane
// 16-byte chunks of a row: hidden <= 256 chunks (4096 at 8 bits, 8192 at 4).
int check_hidden_width(int hidden, int bits, const char* name) {
  const int max_h = 64 * rmoe::kMaxGateUpChunksPerLane * values_per_chunk(bits);
  if (hidden > max_h)
    return fail(RMOE_EINVAL, "%s: hidden %d too large at %d bits (at most %d)", name, hidden,
                bits, max_h);
  return RMOE_OK;
}

int check_layer(const rmoe_layer* L) {
  if (!L) return fail(RMOE_ENULL, "layer is NULL");
  if (L->hidden < 64 || L->hidden % 64)
    return fail(RMOE_EINVAL, "hidden must be a positive multiple of 64 (got %d)",
                L->hidden);
  if (L->inter < 64 || L->inter % 64)
    return fail(RMOE_EINVAL, "inter must be a positive multiple of 64 (got %d)",
                L->inter);
  if (L->experts < 1 || L->experts > rmoe::kMaxExperts)
    return fail(RMOE_EINVAL, "experts must be in [1, %d] (got %d)",
                rmoe::kMaxExperts, L->experts);
  if (L->top_k < 1 || L->top_k > rmoe::kMaxTopK || L->top_k > L->experts)
    return fail(RMOE_EINVAL, "top_k must be in [1, min(%d, experts)] (got %d)",
                rmoe::kMaxTopK, L->top_k);
  int rc;
  const bool rq = L->router_q.w != nullptr;
  if (rq == (L->router_w != nullptr))
    return fail(rq ? RMOE_EINVAL : RMOE_ENULL,
                "exactly one of router_w (bf16) and router_q (8-bit) must be given");
  if (rq) {
    if ((rc = check_gate_q(&L->router_q, L->experts, L->hidden, "router_q"))) return rc;
  } else if (!aligned(L->router_w, 16)) {
    return fail(RMOE_EALIGN, "router_w must be 16-byte aligned");
  }
  if ((rc = check_qweight(&L->gate_up, "gate_up"))) return rc;
  if ((rc = check_qweight(&L->down, "down"))) return rc;
  if (L->gate_up.experts != L->experts || L->gate_up.rows != 2 * L->inter ||
      L->gate_up.cols != L->hidden)
    return fail(RMOE_EINVAL, "gate_up must be [experts, 2*inter, hidden]");
  if (L->down.experts != L->experts || L->down.rows != L->hidden ||
      L->down.cols != L->inter)
    return fail(RMOE_EINVAL, "down must be [experts, hidden, inter]");
  if (L->gate_up.bits != L->down.bits)
    return fail(RMOE_EBITS, "gate_up and down must share one bit width");
  if ((rc = check_down_width(L->inter, L->down.bits, "down"))) return rc;
  if ((rc = check_hidden_width(L->hidden, L->gate_up.bits, "gate_up"))) return rc;
  const bool has_shared = L->shared_gate_up.w != nullptr;
  if (has_shared) {
    if ((rc = check_qweight(&L->shared_gate_up, "shared_gate_up"))) return rc;
    if ((rc = check_qweight(&L->shared_down, "shared_down"))) return rc;
    if (L->shared_inter != L->inter)
      return fail(RMOE_EINVAL,
                  "shared_inter must equal inter (got %d vs %d)",
                  L->shared_inter, L->inter);
    if (L->shared_gate_up.experts != 1 ||
        L->shared_gate_up.rows != 2 * L->shared_inter ||
        L->shared_gate_up.cols != L->hidden)
      return fail(RMOE_EINVAL, "shared_gate_up must be [1, 2*shared_inter, hidden]");
    if (L->shared_down.experts != 1 || L->shared_down.rows != L->hidden ||
        L->shared_down.cols != L->shared_inter)
      return fail(RMOE_EINVAL, "shared_down must be [1, hidden, shared_inter]");
    if (L->shared_gate_up.bits != L->gate_up.bits ||
        L->shared_down.bits != L->gate_up.bits)
      return fail(RMOE_EBITS, "shared expert must use the routed bit width");
  } else if (L->shared_gate_w || L->shared_gate_q.w) {
    return fail(RMOE_EINVAL, "shared gate given without a shared expert");
  }
  if (L->shared_gate_w && L->shared_gate_q.w)
    return fail(RMOE_EINVAL, "give at most one of shared_gate_w and shared_gate_q");
  if ((rq && L->shared_gate_w) || (!rq && L->shared_gate_q.w))
    return fail(RMOE_EINVAL,
                "the shared gate must use the router's format (both bf16 or both 8-bit)");
  if (L->shared_gate_q.w &&
      (rc = check_gate_q(&L->shared_gate_q, 1, L->hidden, "shared_gate_q")))
    return rc;
  if (L->shared_gate_w && !aligned(L->shared_gate_w, 16))
    return fail(RMOE_EALIGN, "shared_gate_w must be 16-byte aligned");
  if (L->post_norm_w) {
    if (!aligned(L->post_norm_w, 16))
      return fail(RMOE_EALIGN, "post_norm_w must be 16-byte aligned");
    if (!(L->norm_eps >= 0.0f) || L->norm_eps > 1.0f)
      return fail(RMOE_EINVAL, "norm_eps must be in [0, 1] (got %g)", (double)L->norm_eps);
  }
  return RMOE_OK;
}

bool router_quantized(const rmoe_layer* L) { return L->router_q.w != nullptr; }
bool shared_gated(const rmoe_layer* L) {
  return L->shared_gate_up.w != nullptr && (L->shared_gate_w || L->shared_gate_q.w);
}

size_t align_up(size_t v) { return (v + 255) & ~size_t(255); }

// Workspace carve-up shared by the router, switch and block calls.
struct Layout {
  size_t ctr, fused, logits, idx, scores, act, total;
  // expert-sorted (prefill) path
  size_t rows, offs, tile_offs, tile_desc, hist, act16, y16, wnorm;
  size_t split;  // bf16 planes of a quantized gate (matrix-core router)
  size_t xn;     // RMSNorm of x [T, H] bf16 (layers with post_norm_w)
};

// Calls that route at least kPrefillMinRows (token, slot) rows take the
// expert-sorted grouped GEMM (the packed module sorts from 64 indices on,
// src/runnel/mlx.py:59); its tiles need these shapes.
bool prefill_path(int T, int K, int E, int H, int I) {
  return (long)T * K >= rmoe::kPrefillMinRows && E <= rmoe::kPrefillMaxExperts &&
         H % 256 == 0 && I % rmoe::kPrefillTileN == 0;
}

// The per-token counters sit at a fixed offset with room for the largest
// token count, so a workspace reused by calls of different shapes always
// finds them at zero (every kernel leaves them at zero when it finishes).
// The router's logits / indices / scores come next in both paths.
Layout layout(int T, int E, int K, int I, int H = 0, bool sorted = false,
              bool combine = false, bool split = false) {
  Layout l{};
  size_t off = 0;
  l.ctr = off;
  off = align_up(off + (size_t)(rmoe::kMaxTokens + 1) * sizeof(uint32_t));
  l.fused = off;
  off = align_up(off + sizeof(rmoe::FusedScratch));
  l.logits = off;
  // (as many partial planes as the matrix-core router would use at T, in
  // both paths, so that the offsets that follow do not depend on the path)
  const size_t planes = (size_t)rmoe::router_logit_planes(T);
  off = align_up(off + planes * (size_t)T * (E + 1) * sizeof(float));
  l.idx = off;
  off = align_up(off + (size_t)T * K * sizeof(int32_t));
  l.scores = off;
  off = align_up(off + (size_t)T * (K + 1) * sizeof(float));
  if (!sorted) {
    l.act = off;
    off = align_up(off + (size_t)T * (K + 1) * I * sizeof(float));
  } else {
    const size_t R = (size_t)T * K + T;
    l.rows = off;
    off = align_up(off + R * sizeof(int32_t));
    l.offs = off;
    off = align_up(off + (size_t)(E + 3) * sizeof(int32_t));
    l.tile_offs = off;
    off = align_up(off + (size_t)(E + 3) * sizeof(int32_t));
    l.tile_desc = off;  // sized for the smaller tile height (more tiles)
    off = align_up(off + (size_t)rmoe::prefill_max_mtiles(T, K, E, 32) * 4 * sizeof(int32_t));
    l.hist = off;
    off = align_up(off + (size_t)rmoe::prefill_sort_slices(T, K) * (E + 2) * sizeof(int32_t));
    l.wnorm = off;
    off = align_up(off + planes * (size_t)E * sizeof(float));
    if (split) {
      l.split = off;
      off = align_up(off + 2 * (size_t)E * H * sizeof(uint16_t));
    }
    l.act16 = off;
    off = align_up(off + R * I * sizeof(uint16_t));
    if (combine) {
      l.y16 = off;
      off = align_up(off + R * H * sizeof(uint16_t));
    }
  }
  l.total = off;
  return l;
}

Layout block_layout(const rmoe_layer* L, int T) {
  const bool sorted = prefill_path(T, L->top_k, L->experts, L->hidden, L->inter);
  const bool split = sorted && router_quantized(L) &&
                     rmoe::router_mfma_eligible(L->experts, L->hidden);
  Layout l = layout(T, L->experts, L->top_k, L->inter, L->hidden, sorted, true, split);
  if (L->post_norm_w) {
    l.xn = l.total;
    l.total = align_up(l.total + (size_t)T * L->hidden * sizeof(uint16_t));
  }
  return l;
}

rmoe::PrefillArgs prefill_args(const Layout& l, void* ws, int T, int H, int I, int E, int K,
                               const uint16_t* x, const int32_t* idx) {
  char* base = static_cast<char*>(ws);
  rmoe::PrefillArgs a{};
  a.T = T;
  a.H = H;
  a.I = I;
  a.E = E;
  a.K = K;
  a.x = x;
  a.idx = idx;
  a.rows = reinterpret_cast<int32_t*>(base + l.rows);
  a.offs = reinterpret_cast<int32_t*>(base + l.offs);
  a.tile_offs = reinterpret_cast<int32_t*>(base + l.tile_offs);
  a.tile_desc = reinterpret_cast<int32_t*>(base + l.tile_desc);
  a.hist = reinterpret_cast<int32_t*>(base + l.hist);
  a.act = reinterpret_cast<uint16_t*>(base + l.act16);
  a.y = l.y16 ? reinterpret_cast<uint16_t*>(base + l.y16) : nullptr;
  a.scores = reinterpret_cast<const float*>(base + l.scores);
  a.score_stride = K + 1;
  return a;
}

rmoe::QW qw(const rmoe_qweight& q) { return rmoe::QW{q.w, q.scales, q.biases}; }

int check_tokens(int32_t tokens) {
  if (tokens < 0 || tokens > rmoe::kMaxTokens)
    return fail(RMOE_EINVAL, "tokens must be in [0, %d] (got %d)", rmoe::kMaxTokens, tokens);
  return RMOE_OK;
}

int check_ws(void* ws, size_t have, size_t need) {
  if (need == 0) return RMOE_OK;
  if (!ws) return fail(RMOE_EWS, "workspace is NULL (%zu bytes needed)", need);
  if (have < need)
    return fail(RMOE_EWS, "workspace too small: %zu bytes given, %zu needed", have,
                need);
  if (!aligned(ws, 256)) return fail(RMOE_EALIGN, "workspace must be 256-byte aligned");
  return RMOE_OK;
}

rmoe::DecodeArgs decode_args(const rmoe_layer* L, const uint16_t* x, int T,
                             void* ws) {
  const Layout l = layout(T, L->experts, L->top_k, L->inter);
  char* base = static_cast<char*>(ws);
  rmoe::DecodeArgs a{};
  a.T = T;
  a.H = L->hidden;
  a.I = L->inter;
  a.E = L->experts;
  a.K = L->top_k;
  a.has_shared = L->shared_gate_up.w != nullptr;
  a.norm = L->norm_topk_prob != 0;
  a.switch_mode = 0;
  a.x = x;
  a.rq8 = router_quantized(L);
  a.has_sg = shared_gated(L);
  a.router_w = L->router_w;
  a.sgate_w = a.has_shared ? L->shared_gate_w : nullptr;
  a.rq = qw(L->router_q);
  a.sgq = qw(L->shared_gate_q);
  a.gu = qw(L->gate_up);
  a.dn = qw(L->down);
  a.sgu = qw(L->shared_gate_up);
  a.sdn = qw(L->shared_down);
  a.logits = reinterpret_cast<float*>(base + l.logits);
  a.idx = reinterpret_cast<int32_t*>(base + l.idx);
  a.scores = reinterpret_cast<float*>(base + l.scores);
  a.score_stride = a.K + 1;
  a.act = reinterpret_cast<float*>(base + l.act);
  a.ctr = reinterpret_cast<uint32_t*>(base + l.ctr);
  a.fs = reinterpret_cast<rmoe::FusedScratch*>(base + l.fused);
  return a;
}

// Shape part of the single-launch decode kernel's eligibility (host only):
// the block's native shape, at most kMaxFusedRouted routed slots (the
// kernel ranks that many) plus the shared expert, and at most
// kFusedMaxExperts experts (four ranking keys per lane).
bool fused_shape_ok(const rmoe_layer* L) {
  return L->hidden == rmoe::kFusedH && L->inter == rmoe::kFusedI &&
         L->top_k <= rmoe::kMaxFusedRouted && L->experts <= rmoe::kFusedMaxExperts;
}

// The single-launch decode kernel also needs its grid: one resident
// workgroup on each of 256 CUs, 32 on each of the 8 XCDs.
bool fused_eligible(const rmoe_layer* L, int* grid) {
  if (!fused_shape_ok(L)) return false;
  int g = 0;
  if (rmoe::fused_grid(L->gate_up.bits, router_quantized(L), L->post_norm_w != nullptr, &g) !=
      hipSuccess)
    return false;
  if (g != rmoe::kFusedXcdGrid) return false;
  *grid = g;
  return true;
}

// The few-token decode kernels (decode.hip): 2..kFewMaxTokens tokens below
// the expert-sorted path, at the single-launch shapes with 8- or 4-bit
// experts; their gate/up reads each row's scales and biases as 4-byte words.
bool few_eligible(const rmoe_layer* L, int T, bool sorted) {
  auto words = [](const rmoe_qweight& q) {
    return aligned(q.scales, 4) && aligned(q.biases, 4);
  };
  const bool shared = L->shared_gate_up.w != nullptr;
  return T >= 2 && T <= rmoe::kFewMaxTokens && !sorted && fused_shape_ok(L) &&
         words(L->gate_up) && (!shared || words(L->shared_gate_up));
}

rmoe::FusedLayer fused_layer(const rmoe_layer* L) {
  rmoe::FusedLayer f{};
  f.router_w = L->router_w;
  f.sgate_w = L->shared_gate_up.w ? L->shared_gate_w : nullptr;
  f.gu = qw(L->gate_up);
  f.dn = qw(L->down);
  f.sgu = qw(L->shared_gate_up);
  f.sdn = qw(L->shared_down);
  f.rq = qw(L->router_q);
  f.sgq = qw(L->shared_gate_q);
  f.norm_w = L->post_norm_w;
  f.norm_eps = L->norm_eps;
  return f;
}

rmoe::FusedArgs fused_args(const rmoe_layer* L, const uint16_t* x, uint16_t* out, void* ws) {
  const Layout l = layout(1, L->experts, L->top_k, L->inter);
  rmoe::FusedArgs f{};
  f.n_layers = 1;
  f.E = L->experts;
  f.K = L->top_k;
  f.norm = L->norm_topk_prob != 0;
  f.has_shared = L->shared_gate_up.w != nullptr;
  f.rq8 = router_quantized(L);
  f.rms_norm = L->post_norm_w != nullptr;
  f.layer0 = fused_layer(L);
  f.table = nullptr;
  f.x = x;
  f.out = out;
  f.scratch = reinterpret_cast<rmoe::FusedScratch*>(static_cast<char*>(ws) + l.fused);
  return f;
}

// Shapes shared by the switch calls: gate_up [E, 2I, H], down [E, H, I].
int check_switch(const rmoe_qweight* gate_up, const rmoe_qweight* down, int32_t tokens,
                 int32_t top_k) {
  int rc;
  if ((rc = check_qweight(gate_up, "gate_up"))) return rc;
  if ((rc = check_qweight(down, "down"))) return rc;
  if ((rc = check_tokens(tokens))) return rc;
  if (gate_up->rows % 2) return fail(RMOE_EINVAL, "gate_up rows must be 2*inter");
  const int I = gate_up->rows / 2;
  const int H = gate_up->cols;
  if (down->experts != gate_up->experts || down->rows != H || down->cols != I)
    return fail(RMOE_EINVAL, "down must be [experts, hidden, inter] of gate_up");
  if (down->bits != gate_up->bits)
    return fail(RMOE_EBITS, "gate_up and down must share one bit width");
  if ((rc = check_down_width(I, down->bits, "down"))) return rc;
  if ((rc = check_hidden_width(H, gate_up->bits, "gate_up"))) return rc;
  if (top_k < 1 || top_k > rmoe::kMaxTopK)
    return fail(RMOE_EINVAL, "top_k must be in [1, %d] (got %d)", rmoe::kMaxTopK, top_k);
  return RMOE_OK;
}

// The routed experts for caller indices; `weights` == nullptr: per-slot
// outputs into y [T, K, H]; otherwise out[t] = bf16(sum_j w[t, j] y[t, j])
// (+ residual) into y [T, H].
int switch_call(const rmoe_qweight* gate_up, const rmoe_qweight* down, const uint16_t* x,
                int32_t tokens, const int32_t* indices, const float* weights, int32_t top_k,
                const uint16_t* residual, uint16_t* y, void* ws, size_t ws_bytes,
                void* stream) {
  int rc;
  if ((rc = check_switch(gate_up, down, tokens, top_k))) return rc;
  if (tokens == 0) return ok();
  const bool combine = weights != nullptr;
  if (!x || !indices || !y) return fail(RMOE_ENULL, "x, indices and the output are required");
  if (!aligned(x, 16)) return fail(RMOE_EALIGN, "x must be 16-byte aligned");
  const int I = gate_up->rows / 2;
  const int H = gate_up->cols;
  const bool sorted = prefill_path(tokens, top_k, gate_up->experts, H, I);
  // the sorted path moves output and residual rows in 16-byte pieces
  const size_t row_align = sorted ? 16 : 2;
  if (!aligned(indices, 4) || (combine && !aligned(weights, 4)))
    return fail(RMOE_EALIGN, "indices/weights must be 4-byte aligned");
  if (!aligned(y, row_align) || (residual && !aligned(residual, row_align)))
    return fail(RMOE_EALIGN, "output/residual must be %zu-byte aligned", row_align);
  if (combine && static_cast<const void*>(y) == static_cast<const void*>(x))
    return fail(RMOE_EINVAL, "out must not alias x");
  const Layout lay = layout(tokens, gate_up->experts, top_k, I, H, sorted, combine);
  if ((rc = check_ws(ws, ws_bytes, lay.total))) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (sorted) {
    rmoe::PrefillArgs pa = prefill_args(lay, ws, tokens, H, I, gate_up->experts, top_k, x,
                                        indices);
    pa.gu = qw(*gate_up);
    pa.dn = qw(*down);
    if (combine) {
      pa.scores = weights;
      pa.score_stride = top_k;
      pa.residual = residual;
      pa.out = y;
    } else {
      pa.y = y;
    }
    const hipError_t e = rmoe::launch_prefill(pa, gate_up->bits, combine, s);
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
    return ok();
  }
  rmoe_layer L{};
  L.hidden = H;
  L.inter = I;
  L.experts = gate_up->experts;
  L.top_k = top_k;
  L.gate_up = *gate_up;
  L.down = *down;
  rmoe::DecodeArgs a = decode_args(&L, x, tokens, ws);
  a.idx = const_cast<int32_t*>(indices);
  a.switch_mode = 1;
  a.out = y;
  if (combine) {
    a.scores = const_cast<float*>(weights);
    a.score_stride = top_k;
    a.residual = residual;
  }
  hipError_t e = rmoe::launch_gate_up(a, gate_up->bits, s);
  if (e != hipSuccess) return hip_fail(e, "gate/up launch");
  e = rmoe::launch_down(a, gate_up->bits, combine, s);
  if (e != hipSuccess) return hip_fail(e, "down launch");
  return ok();
}

}  // namespace

extern "C" {

int rmoe_abi_version(void) { return RMOE_ABI_VERSION; }

const char* rmoe_last_error(void) { return g_error.c_str(); }

const char* rmoe_status_string(int status) {
  switch (status) {
    case RMOE_OK: return "ok";
    case RMOE_EINVAL: return "invalid argument";
    case RMOE_EBITS: return "unsupported quantization format";
    case RMOE_EALIGN: return "misaligned pointer";
    case RMOE_EWS: return "workspace too small";
    case RMOE_EHIP: return "HIP runtime error";
    case RMOE_ENULL: return "NULL pointer";
    case RMOE_ETIMEOUT: return "single-launch decode timed out (outputs not valid)";
    case RMOE_EPLACEMENT:
      return "single-launch decode: XCC id outside 0-7 (outputs not valid)";
    default: return "unknown status";
  }
}

int rmoe_validate_layer(const rmoe_layer* layer) {
  const int rc = check_layer(layer);
  return rc ? rc : ok();
}

size_t rmoe_workspace_bytes(const rmoe_layer* L, int32_t tokens) {
  if (check_layer(L) || tokens < 0) return 0;
  return block_layout(L, tokens).total;
}

size_t rmoe_switch_workspace_bytes(const rmoe_qweight* gate_up,
                                   const rmoe_qweight* down, int32_t tokens,
                                   int32_t top_k) {
  if (!gate_up || !down || tokens < 0 || top_k < 1) return 0;
  const int I = gate_up->rows / 2;
  const int H = gate_up->cols;
  const bool sorted = prefill_path(tokens, top_k, gate_up->experts, H, I);
  return layout(tokens, gate_up->experts, top_k, I, H, sorted, false).total;
}

size_t rmoe_switch_combine_workspace_bytes(const rmoe_qweight* gate_up,
                                           const rmoe_qweight* down, int32_t tokens,
                                           int32_t top_k) {
  if (!gate_up || !down || tokens < 0 || top_k < 1) return 0;
  const int I = gate_up->rows / 2;
  const int H = gate_up->cols;
  const bool sorted = prefill_path(tokens, top_k, gate_up->experts, H, I);
  return layout(tokens, gate_up->experts, top_k, I, H, sorted, true).total;
}

size_t rmoe_router_workspace_bytes(int32_t experts, int32_t top_k, int32_t tokens) {
  if (experts < 1 || top_k < 1 || tokens < 0) return 0;
  return layout(tokens, experts, top_k, 0).total;
}

int rmoe_router(const uint16_t* router_w, int32_t experts, int32_t hidden,
                int32_t top_k, int32_t norm_topk_prob, const uint16_t* x,
                int32_t tokens, int32_t* indices, float* scores, void* ws,
                size_t ws_bytes, void* stream) {
  int rc;
  if (hidden < 64 || hidden % 64)
    return fail(RMOE_EINVAL, "hidden must be a positive multiple of 64 (got %d)", hidden);
  if (experts < 1 || experts > rmoe::kMaxExperts)
    return fail(RMOE_EINVAL, "experts must be in [1, %d] (got %d)", rmoe::kMaxExperts,
                experts);
  if (top_k < 1 || top_k > rmoe::kMaxTopK || top_k > experts)
    return fail(RMOE_EINVAL, "top_k must be in [1, min(%d, experts)] (got %d)",
                rmoe::kMaxTopK, top_k);
  if ((rc = check_tokens(tokens))) return rc;
  if (!router_w) return fail(RMOE_ENULL, "router_w is NULL");
  if (!aligned(router_w, 16)) return fail(RMOE_EALIGN, "router_w must be 16-byte aligned");
  if (tokens == 0) return ok();
  if (!x || !indices || !scores) return fail(RMOE_ENULL, "x, indices and scores are required");
  if (!aligned(x, 16)) return fail(RMOE_EALIGN, "x must be 16-byte aligned");
  const size_t need = layout(tokens, experts, top_k, 0).total;
  if ((rc = check_ws(ws, ws_bytes, need))) return rc;
  rmoe_layer L{};
  L.hidden = hidden;
  L.inter = 0;
  L.experts = experts;
  L.top_k = top_k;
  L.norm_topk_prob = norm_topk_prob;
  L.router_w = router_w;
  rmoe::DecodeArgs a = decode_args(&L, x, tokens, ws);
  a.idx_out = indices;
  a.scores_out = scores;
  const hipError_t e = rmoe::launch_router(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "router launch");
  return ok();
}

int rmoe_rms_norm(const uint16_t* x, const uint16_t* weight, int32_t tokens, int32_t hidden,
                  float eps, uint16_t* out, void* stream) {
  int rc;
  if ((rc = check_tokens(tokens))) return rc;
  if (hidden < 8 || hidden % 8)
    return fail(RMOE_EINVAL, "hidden must be a positive multiple of 8 (got %d)", hidden);
  if (!(eps >= 0.0f) || eps > 1.0f)
    return fail(RMOE_EINVAL, "eps must be in [0, 1] (got %g)", (double)eps);
  if (tokens == 0) return ok();
  if (!x || !weight || !out) return fail(RMOE_ENULL, "x, weight and out are required");
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(out, 16))
    return fail(RMOE_EALIGN, "x, weight and out must be 16-byte aligned");
  const hipError_t e = rmoe::launch_rmsnorm(x, weight, tokens, hidden, eps, out,
                                            static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "rmsnorm launch");
  return ok();
}

int rmoe_router_q(const rmoe_qweight* router, int32_t top_k, int32_t norm_topk_prob,
                  const uint16_t* x, int32_t tokens, int32_t* indices, float* scores,
                  void* ws, size_t ws_bytes, void* stream) {
  int rc;
  if (!router) return fail(RMOE_ENULL, "router is NULL");
  const int experts = router->rows;
  const int hidden = router->cols;
  if ((rc = check_gate_q(router, experts, hidden, "router"))) return rc;
  if (experts > rmoe::kMaxExperts)
    return fail(RMOE_EINVAL, "experts must be in [1, %d] (got %d)", rmoe::kMaxExperts,
                experts);
  if (top_k < 1 || top_k > rmoe::kMaxTopK || top_k > experts)
    return fail(RMOE_EINVAL, "top_k must be in [1, min(%d, experts)] (got %d)",
                rmoe::kMaxTopK, top_k);
  if ((rc = check_tokens(tokens))) return rc;
  if (tokens == 0) return ok();
  if (!x || !indices || !scores) return fail(RMOE_ENULL, "x, indices and scores are required");
  if (!aligned(x, 16)) return fail(RMOE_EALIGN, "x must be 16-byte aligned");
  const size_t need = layout(tokens, experts, top_k, 0).total;
  if ((rc = check_ws(ws, ws_bytes, need))) return rc;
  rmoe_layer L{};
  L.hidden = hidden;
  L.experts = experts;
  L.top_k = top_k;
  L.norm_topk_prob = norm_topk_prob;
  L.router_q = *router;
  rmoe::DecodeArgs a = decode_args(&L, x, tokens, ws);
  a.idx_out = indices;
  a.scores_out = scores;
  const hipError_t e = rmoe::launch_router(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "router launch");
  return ok();
}

}  // extern "C"

namespace {

// Argument checks of a block call (everything but the workspace).
int check_block(const rmoe_layer* L, const uint16_t* x, int32_t tokens,
                const uint16_t* residual, const uint16_t* out) {
  int rc;
  if ((rc = check_layer(L))) return rc;
  if ((rc = check_tokens(tokens))) return rc;
  if (tokens == 0) return RMOE_OK;
  if (!x || !out) return fail(RMOE_ENULL, "x and out are required");
  if (!aligned(x, 16)) return fail(RMOE_EALIGN, "x must be 16-byte aligned");
  if (!aligned(out, 2) || (residual && !aligned(residual, 2)))
    return fail(RMOE_EALIGN, "out/residual must be 2-byte aligned");
  if (static_cast<const void*>(out) == static_cast<const void*>(x))
    return fail(RMOE_EINVAL, "out must not alias x");
  const Layout lay = block_layout(L, tokens);
  if (lay.rows && (!aligned(out, 16) || (residual && !aligned(residual, 16))))
    return fail(RMOE_EALIGN,
                "out/residual must be 16-byte aligned for calls that route %d or more "
                "(token, slot) rows", rmoe::kPrefillMinRows);
  return RMOE_OK;
}

// The block's launches on a checked call and a workspace of lay.total bytes.
int block_launch(const rmoe_layer* L, const uint16_t* x, int32_t tokens,
                 const uint16_t* residual, uint16_t* out, int32_t* indices_out,
                 float* scores_out, void* ws, void* stream) {
  const Layout lay = block_layout(L, tokens);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int bits = L->gate_up.bits;
  int grid = 0;
  if (tokens == 1 && fused_eligible(L, &grid)) {
    rmoe::FusedArgs f = fused_args(L, x, out, ws);
    f.n_layers = 1;
    f.residual_mode = residual == nullptr ? 0 : (residual == x ? 1 : 2);
    f.residual = residual;
    f.idx_out = indices_out;
    f.scores_out = scores_out;
    const hipError_t e = rmoe::launch_fused_decode(f, bits, grid, s);
    if (e != hipSuccess) return hip_fail(e, "fused decode launch");
    return ok();
  }
  hipError_t e;
  if (L->post_norm_w) {
    // the block's input is RMSNorm(x); the residual stays the caller's
    uint16_t* xn = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + lay.xn);
    e = rmoe::launch_rmsnorm(x, L->post_norm_w, tokens, L->hidden, L->norm_eps, xn, s);
    if (e != hipSuccess) return hip_fail(e, "rmsnorm launch");
    x = xn;
  }
  rmoe::DecodeArgs a = decode_args(L, x, tokens, ws);
  a.out = out;
  a.residual = residual;
  a.idx_out = indices_out;
  a.scores_out = scores_out;
  if (few_eligible(L, tokens, lay.rows != 0)) a.few_bits = L->gate_up.bits;
  a.logit_planes = lay.rows ? rmoe::router_logit_planes(tokens) : 1;
  if (lay.rows && rmoe::router_mfma_eligible(L->experts, L->hidden))
    e = rmoe::launch_router_mfma(
        a, reinterpret_cast<float*>(static_cast<char*>(ws) + lay.wnorm),
        lay.split ? reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + lay.split) : nullptr,
        s);
  else
    e = rmoe::launch_router(a, s);
  if (e != hipSuccess) return hip_fail(e, "router launch");
  if (lay.rows) {
    rmoe::PrefillArgs pa = prefill_args(lay, ws, tokens, L->hidden, L->inter, L->experts,
                                        L->top_k, x, a.idx);
    pa.has_shared = a.has_shared;
    pa.gu = a.gu;
    pa.dn = a.dn;
    pa.sgu = a.sgu;
    pa.sdn = a.sdn;
    pa.residual = residual;
    pa.out = out;
    e = rmoe::launch_prefill(pa, bits, true, s);
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
    return ok();
  }
  e = rmoe::launch_gate_up(a, bits, s);
  if (e != hipSuccess) return hip_fail(e, "gate/up launch");
  e = rmoe::launch_down(a, bits, true, s);
  if (e != hipSuccess) return hip_fail(e, "down launch");
  return ok();
}

}  // namespace

extern "C" {

int rmoe_moe_block(const rmoe_layer* L, const uint16_t* x, int32_t tokens,
                   const uint16_t* residual, uint16_t* out, int32_t* indices_out,
                   float* scores_out, void* ws, size_t ws_bytes, void* stream) {
  int rc;
  if ((rc = check_block(L, x, tokens, residual, out))) return rc;
  if (tokens == 0) return ok();
  if ((rc = check_ws(ws, ws_bytes, block_layout(L, tokens).total))) return rc;
  return block_launch(L, x, tokens, residual, out, indices_out, scores_out, ws, stream);
}

int rmoe_moe_block_noalloc(const rmoe_layer* L, const uint16_t* x, int32_t tokens,
                           const uint16_t* residual, uint16_t* out, int32_t* indices_out,
                           float* scores_out, uint32_t* status_out, void* stream) {
  int rc;
  if ((rc = check_block(L, x, tokens, residual, out))) return rc;
  if (status_out && !aligned(status_out, 4))
    return fail(RMOE_EALIGN, "status_out must be 4-byte aligned");
  if (tokens == 0) return ok();
  const size_t need = block_layout(L, tokens).total;
  if (need > rmoe::kStaticScratchBytes)
    return fail(RMOE_EWS,
                "this call needs %zu bytes of scratch, more than the %zu bytes of the "
                "library's static scratch; use rmoe_moe_block with a workspace",
                need, rmoe::kStaticScratchBytes);
  void* ws = nullptr;
  hipError_t e = rmoe::static_scratch(static_cast<hipStream_t>(stream), &ws);
  if (e != hipSuccess) return hip_fail(e, "static scratch address");
  if ((rc = block_launch(L, x, tokens, residual, out, indices_out, scores_out, ws, stream)))
    return rc;
  // the status word is taken (and cleared) after every call, so that a
  // later call never reports an earlier call's status as its own
  e = rmoe::launch_take_status(
      reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + rmoe_workspace_status_offset()),
      status_out, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "status launch");
  return ok();
}

int rmoe_switch_glu(const rmoe_qweight* gate_up, const rmoe_qweight* down,
                    const uint16_t* x, int32_t tokens, const int32_t* indices,
                    int32_t top_k, uint16_t* y, void* ws, size_t ws_bytes,
                    void* stream) {
  return switch_call(gate_up, down, x, tokens, indices, nullptr, top_k, nullptr, y, ws,
                     ws_bytes, stream);
}

int rmoe_switch_combine(const rmoe_qweight* gate_up, const rmoe_qweight* down,
                        const uint16_t* x, int32_t tokens, const int32_t* indices,
                        const float* weights, int32_t top_k, const uint16_t* residual,
                        uint16_t* out, void* ws, size_t ws_bytes, void* stream) {
  if (tokens > 0 && !weights) return fail(RMOE_ENULL, "weights are required");
  return switch_call(gate_up, down, x, tokens, indices, weights, top_k, residual, out, ws,
                     ws_bytes, stream);
}

int rmoe_gather_qmm(const uint16_t* x, int32_t x_rows, const int32_t* lhs,
                    const int32_t* rhs, int32_t rows, const rmoe_qweight* w,
                    uint16_t* y_bf16, float* y_f32, void* stream) {
  int rc;
  if ((rc = check_qweight(w, "w"))) return rc;
  if (rows < 0 || x_rows < 0) return fail(RMOE_EINVAL, "rows must be >= 0");
  if ((y_bf16 == nullptr) == (y_f32 == nullptr))
    return fail(RMOE_EINVAL, "exactly one of y_bf16 / y_f32 must be given");
  const bool dense = !lhs && !rhs && y_bf16 && aligned(y_bf16, 16) &&
                     rmoe::dense_qmm_eligible(rows, w->rows, w->cols);
  const int vpc = values_per_chunk(w->bits);
  const int chunks = w->cols / vpc;
  if (!dense && chunks < 64 && !pow2(chunks))
    return fail(RMOE_EINVAL, "cols %d unsupported at %d bits", w->cols, w->bits);
  if (!dense && chunks > 256)
    return fail(RMOE_EINVAL, "cols %d too large (max %d at %d bits)", w->cols,
                256 * vpc, w->bits);
  if (rows == 0) return ok();
  if (!x) return fail(RMOE_ENULL, "x is required");
  if (!aligned(x, 16)) return fail(RMOE_EALIGN, "x must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dense) {
    // a dense product at prefill sizes: the grouped GEMM on the matrix cores
    const hipError_t e =
        rmoe::launch_dense_qmm(x, rows, qw(*w), w->rows, w->cols, w->bits, y_bf16, s);
    if (e != hipSuccess) return hip_fail(e, "dense qmm launch");
    return ok();
  }
  rmoe::QmvArgs a{};
  a.M = rows;
  a.N = w->rows;
  a.K = w->cols;
  a.x_rows = lhs ? x_rows : rows;
  a.experts = w->experts;
  a.x = x;
  a.lhs = lhs;
  a.rhs = rhs;
  a.w = qw(*w);
  a.y_bf16 = y_bf16;
  a.y_f32 = y_f32;
  const hipError_t e = rmoe::launch_qmv(a, w->bits, s);
  if (e != hipSuccess) return hip_fail(e, "qmv launch");
  return ok();
}

int rmoe_quantize(const float* w, int64_t rows, int32_t cols, int32_t bits,
                  int32_t group_size, uint32_t* wq, uint16_t* scales,
                  uint16_t* biases, void* stream) {
  if (bits != 4 && bits != 8) return fail(RMOE_EBITS, "bits must be 4 or 8");
  if (group_size != 64) return fail(RMOE_EBITS, "group_size must be 64");
  if (rows < 0 || cols < 64 || cols % 64)
    return fail(RMOE_EINVAL, "cols must be a positive multiple of 64");
  if (rows == 0) return ok();
  if (!w || !wq || !scales || !biases) return fail(RMOE_ENULL, "all buffers are required");
  if (!aligned(w, 16) || !aligned(wq, 4))
    return fail(RMOE_EALIGN, "w must be 16-byte aligned");
  const hipError_t e = rmoe::launch_quantize(w, rows, cols, bits, wq, scales, biases,
                                             static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "quantize launch");
  return ok();
}

int rmoe_dequantize(const rmoe_qweight* w, int64_t row_begin, int64_t rows,
                    float* out_f32, uint16_t* out_bf16, void* stream) {
  int rc;
  if ((rc = check_qweight(w, "w"))) return rc;
  const int64_t total = (int64_t)w->experts * w->rows;
  if (row_begin < 0 || rows < 0 || row_begin + rows > total)
    return fail(RMOE_EINVAL, "row range [%lld, %lld) outside the bank of %lld rows",
                (long long)row_begin, (long long)(row_begin + rows), (long long)total);
  if (rows == 0 || (!out_f32 && !out_bf16)) return ok();
  const hipError_t e =
      rmoe::launch_dequantize(qw(*w), w->cols, w->bits, row_begin, rows, out_f32,
                              out_bf16, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "dequantize launch");
  return ok();
}

size_t rmoe_chain_table_bytes(int32_t n_layers) {
  return n_layers > 0 ? (size_t)n_layers * sizeof(rmoe::FusedLayer) : 0;
}

int rmoe_chain_table_pack(const rmoe_layer* layers, int32_t n_layers, void* host_table) {
  int rc;
  if (!layers || !host_table) return fail(RMOE_ENULL, "layers and host_table are required");
  if (n_layers < 1) return fail(RMOE_EINVAL, "n_layers must be >= 1");
  int grid = 0;
  for (int i = 0; i < n_layers; ++i) {
    if ((rc = check_layer(&layers[i]))) return rc;
    const rmoe_layer& a = layers[0];
    const rmoe_layer& b = layers[i];
    if (b.hidden != a.hidden || b.inter != a.inter || b.experts != a.experts ||
        b.top_k != a.top_k || b.norm_topk_prob != a.norm_topk_prob ||
        b.gate_up.bits != a.gate_up.bits ||
        (b.shared_gate_up.w == nullptr) != (a.shared_gate_up.w == nullptr) ||
        (b.shared_gate_w == nullptr) != (a.shared_gate_w == nullptr) ||
        (b.router_q.w == nullptr) != (a.router_q.w == nullptr) ||
        (b.shared_gate_q.w == nullptr) != (a.shared_gate_q.w == nullptr) ||
        (b.post_norm_w == nullptr) != (a.post_norm_w == nullptr))
      return fail(RMOE_EINVAL, "layer %d differs in shape or format from layer 0", i);
  }
  // the shape first: it needs no device, so argument errors never depend on one
  if (!fused_shape_ok(&layers[0]))
    return fail(RMOE_EINVAL,
                "chained decode needs hidden %d, inter %d, top_k <= %d (plus the shared "
                "expert) and experts <= %d (got %d, %d, %d, %d)",
                rmoe::kFusedH, rmoe::kFusedI, rmoe::kMaxFusedRouted, rmoe::kFusedMaxExperts,
                layers[0].hidden, layers[0].inter, layers[0].top_k, layers[0].experts);
  if (!fused_eligible(&layers[0], &grid))
    return fail(RMOE_EINVAL, "chained decode needs a device of at least %d CUs in 8 XCDs",
                rmoe::kFusedXcdGrid);
  for (int i = 0; i < n_layers; ++i)
    static_cast<rmoe::FusedLayer*>(host_table)[i] = fused_layer(&layers[i]);
  return ok();
}

int rmoe_moe_chain(const rmoe_layer* layer0, const void* device_table, int32_t n_layers,
                   const uint16_t* x, uint16_t* out, void* ws, size_t ws_bytes,
                   void* stream) {
  int rc;
  if ((rc = check_layer(layer0))) return rc;
  if (!device_table || !x || !out) return fail(RMOE_ENULL, "table, x and out are required");
  if (n_layers < 1) return fail(RMOE_EINVAL, "n_layers must be >= 1");
  if (!aligned(x, 16) || !aligned(device_table, 8))
    return fail(RMOE_EALIGN, "x must be 16-byte and the table 8-byte aligned");
  if (static_cast<const void*>(out) == static_cast<const void*>(x))
    return fail(RMOE_EINVAL, "out must not alias x");
  int grid = 0;
  if (!fused_eligible(layer0, &grid))
    return fail(RMOE_EINVAL, "layer shape is not supported by the chained decode kernel");
  const size_t need = layout(1, layer0->experts, layer0->top_k, layer0->inter).total;
  if ((rc = check_ws(ws, ws_bytes, need))) return rc;
  rmoe::FusedArgs f = fused_args(layer0, x, out, ws);
  f.n_layers = n_layers;
  f.table = static_cast<const rmoe::FusedLayer*>(device_table);
  f.residual_mode = 1;
  const hipError_t e = rmoe::launch_fused_decode(f, layer0->gate_up.bits, grid,
                                                 static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "chained decode launch");
  return ok();
}

size_t rmoe_workspace_status_offset(void) {
  return layout(0, 1, 1, 0).fused + offsetof(rmoe::FusedScratch, err);
}

int rmoe_set_cooperative_launch(int32_t enabled) {
  const int prev = g_cooperative.exchange(enabled ? 1 : 0);
  ok();
  return prev;
}

int rmoe_stream_read(const void* buffer, size_t bytes, uint32_t* partials,
                     int32_t blocks, void* stream) {
  if (!buffer || !partials) return fail(RMOE_ENULL, "buffer and partials are required");
  if (bytes % 16 || !aligned(buffer, 16))
    return fail(RMOE_EALIGN, "buffer must be 16-byte aligned and a multiple of 16 bytes");
  if (blocks < 1 || blocks > (1 << 20))
    return fail(RMOE_EINVAL, "blocks must be in [1, 2^20]");
  const hipError_t e = rmoe::launch_stream_read(buffer, bytes, partials, blocks,
                                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "stream launch");
  return ok();
}

}  // extern "C"

namespace rmoe {
bool cooperative_launch_enabled() { return g_cooperative.load(std::memory_order_relaxed) != 0; }
}  // namespace rmoe
