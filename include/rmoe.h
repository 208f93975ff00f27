/*
 * rmoe.h - C ABI of the MI355X-native quantized sparse-MoE block.
 *
 * All tensor pointers are caller-owned DEVICE pointers (for instance the
 * data_ptr() of torch tensors on the GPU); every compute call is enqueued on
 * `stream` (a hipStream_t passed as void*, NULL = the default stream) and
 * returns without waiting for the GPU.  Every call returns RMOE_OK (0) or a
 * negative RMOE_E* code; the message for the last failure on the calling
 * thread is rmoe_last_error().  Arguments are validated on the host before
 * anything is launched, so argument errors never reach the GPU.  No call
 * allocates device memory: scratch space is the caller's `workspace`,
 * which must be zero-filled once when it is first allocated (the library
 * keeps its counters at a fixed offset and leaves them at zero when each
 * call completes, so one workspace serves calls of any shape) and must not
 * be shared by calls that may run concurrently.
 *
 * Weight format (MLX "affine", transpose=True): a matrix W[out, in] of
 * `bits`-bit codes is stored as uint32 words [out, in * bits / 32], element
 * k of a row in word k / (32/bits) at bit offset bits * (k % (32/bits)),
 * least-significant first; scales and biases are bf16 [out, in / group];
 * W[r, k] = q * scale + bias.  Expert banks add a leading [experts] axis.
 * bf16 values travel as uint16_t bit patterns.
 *
 * Reference interfaces replaced (paths relative to the waylake/runnel tree):
 *   rmoe_switch_glu   FusedQuantizedSwitchGLU.__call__   src/runnel/mlx.py:57-82
 *   rmoe_gather_qmm   mx.gather_qmm / QuantizedSwitchLinear, called at
 *                     src/runnel/mlx.py:64-75 and :77-79
 *   rmoe_moe_block    mlx-lm SparseMoeBlock.__call__ (the caller of the
 *                     module, invoked as layer.mlp(x) at
 *                     bench/mlx_component_profile.py:130)
 *   rmoe_router       the router half of that block (gate -> softmax ->
 *                     top-k -> renormalise)
 *   rmoe_router_q     the same with the 8-bit QuantizedLinear gate of real
 *                     checkpoints (bench/runnel_bench/checkpoint.py:200-208)
 *   rmoe_quantize / rmoe_dequantize
 *                     mx.quantize / mx.dequantize (affine, group 64), the
 *                     format produced for the banks that
 *                     src/runnel/mlx.py:38-48 concatenates
 *   rmoe_stream_read  the HBM stream calibrator that replaces
 *                     native/shaders/persistent_stream.metal:12-79
 */
#ifndef RMOE_H
#define RMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RMOE_ABI_VERSION 5

#define RMOE_OK 0
#define RMOE_EINVAL (-1) /* inconsistent or unsupported shape / argument */
#define RMOE_EBITS (-2)  /* bits not in {4, 8} or group size not 64 */
#define RMOE_EALIGN (-3) /* a pointer is not 16-byte aligned */
#define RMOE_EWS (-4)    /* workspace missing or too small */
#define RMOE_EHIP (-5)   /* the HIP runtime reported an error */
#define RMOE_ENULL (-6)  /* a required pointer is NULL */
/* Not returned by any call (the calls do not wait for the GPU): the codes
 * callers report when a workspace's status word (rmoe_workspace_status_offset)
 * is 1 (a single-launch decode gave up a cross-workgroup wait, or the call
 * was cancelled) or 2 (a workgroup read an XCC id outside 0-7, so it could
 * not take part in the XCD-local hand-overs). */
#define RMOE_ETIMEOUT (-7)
#define RMOE_EPLACEMENT (-8)

/* One MLX-affine quantized bank: w [experts, rows, cols*bits/32] u32,
 * scales / biases [experts, rows, cols/group_size] bf16. */
typedef struct rmoe_qweight {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
  int32_t experts;
  int32_t rows;
  int32_t cols;
  int32_t bits;
  int32_t group_size;
} rmoe_qweight;

/* One MoE layer's resident weights.  gate_up rows are [up; gate]
 * (src/runnel/mlx.py:38-48).  The shared expert is present when
 * shared_gate_up.w != NULL; shared_gate_w (bf16 [hidden]) is its sigmoid
 * gate.  norm_topk_prob != 0 renormalises the selected probabilities.
 *
 * The router gate is either bf16 (router_w) or an 8-bit group-64 MLX-affine
 * bank (router_q, [1, experts, hidden]; router_w NULL), the format real
 * checkpoints give mlp.gate and mlp.shared_expert_gate
 * (bench/runnel_bench/checkpoint.py:200-208,
 * bench/results/m0/checkpoint-ornith-mlx-8bit.json:163-175).  The shared
 * gate then uses the same format: shared_gate_q [1, 1, hidden] instead of
 * shared_gate_w.  Quantized gate logits follow a fixed fp32 order of their
 * own: 16-code chunks lane + 64 i of a 64-lane wave, per chunk
 * acc = fma(sum q x, s, acc), acc = fma(sum x, b, acc), then a butterfly.
 *
 * post_norm_w != NULL puts the decoder layer's post-attention RMSNorm in
 * front of the block (appended in ABI version 3): the block's input is
 * rmoe_rms_norm(x, post_norm_w, norm_eps), the residual stays what the
 * caller passes, so a decoder computes h' = h + MoE(RMSNorm(h)) with
 * residual = x = h (the layer sequence of docs/architecture.md:31-37).
 *
 * Shapes: hidden and inter multiples of 64; hidden at most 4096 at 8 bits
 * (8192 at 4 bits); inter / (16 at 8 bits, 32 at 4 bits) a power of two
 * <= 64; experts <= 1024; top_k <= min(64, experts). */
typedef struct rmoe_layer {
  int32_t hidden;
  int32_t inter;
  int32_t shared_inter;
  int32_t experts;
  int32_t top_k;
  int32_t norm_topk_prob;
  const uint16_t* router_w;      /* bf16 [experts, hidden] */
  const uint16_t* shared_gate_w; /* bf16 [hidden], or NULL */
  rmoe_qweight gate_up;          /* [experts, 2*inter, hidden] */
  rmoe_qweight down;             /* [experts, hidden, inter] */
  rmoe_qweight shared_gate_up;   /* [1, 2*shared_inter, hidden] */
  rmoe_qweight shared_down;      /* [1, hidden, shared_inter] */
  rmoe_qweight router_q;         /* 8-bit gate [1, experts, hidden], or w NULL */
  rmoe_qweight shared_gate_q;    /* 8-bit shared gate [1, 1, hidden], or w NULL */
  const uint16_t* post_norm_w;   /* bf16 [hidden] RMSNorm weights, or NULL */
  float norm_eps;                /* its epsilon, in [0, 1] */
} rmoe_layer;

int rmoe_abi_version(void);

/* RMSNorm of `tokens` rows (mx.fast.rms_norm(x, weight, eps); checkpoints
 * store the effective weight): out = bf16(bf16(x r) w) with r = 1 /
 * sqrt(sum(x^2) / hidden + eps), the sum in the router's fixed fp32 order,
 * r correctly rounded.  hidden a multiple of 8; x, weight, out bf16, 16-byte
 * aligned. */
int rmoe_rms_norm(const uint16_t* x, const uint16_t* weight, int32_t tokens, int32_t hidden,
                  float eps, uint16_t* out, void* stream);
const char* rmoe_last_error(void);
const char* rmoe_status_string(int status);

/* Host-only validation of a layer description (no GPU access). */
int rmoe_validate_layer(const rmoe_layer* layer);

/* Bytes of workspace the block / router / switch calls need for `tokens`. */
size_t rmoe_workspace_bytes(const rmoe_layer* layer, int32_t tokens);

/* Router of mlx-lm's SparseMoeBlock: bf16 logits x . router_w^T (fixed fp32
 * reduction order), top_k experts by (logit desc, index asc), softmax over
 * all experts, probabilities rounded to bf16, renormalised when
 * norm_topk_prob.  indices int32 [tokens, top_k] in rank order, scores
 * fp32 [tokens, top_k] (bf16-valued). */
int rmoe_router(const uint16_t* router_w, int32_t experts, int32_t hidden,
                int32_t top_k, int32_t norm_topk_prob, const uint16_t* x,
                int32_t tokens, int32_t* indices, float* scores,
                void* workspace, size_t workspace_bytes, void* stream);
size_t rmoe_router_workspace_bytes(int32_t experts, int32_t top_k,
                                   int32_t tokens);

/* The same router with an 8-bit group-64 quantized gate (mlx-lm's
 * QuantizedLinear gate, x @ dequantize(W)^T): router [1, experts, hidden]
 * (experts = router->rows, hidden = router->cols), logits in the quantized
 * gate's fixed fp32 order.  Workspace: rmoe_router_workspace_bytes. */
int rmoe_router_q(const rmoe_qweight* router, int32_t top_k, int32_t norm_topk_prob,
                  const uint16_t* x, int32_t tokens, int32_t* indices, float* scores,
                  void* workspace, size_t workspace_bytes, void* stream);

/* FusedQuantizedSwitchGLU.__call__ (src/runnel/mlx.py:57-82): for every
 * (token, slot) the packed [up; gate] projection of expert indices[t, j],
 * SwiGLU, then the expert's down projection.  y bf16 [tokens, top_k,
 * hidden], per slot and not combined.  A slot whose index is outside
 * [0, experts) yields a zero row and touches no weight memory.  From 64
 * (token, slot) rows on (the expert-sorted path) y must be 16-byte
 * aligned. */
int rmoe_switch_glu(const rmoe_qweight* gate_up, const rmoe_qweight* down,
                    const uint16_t* x, int32_t tokens, const int32_t* indices,
                    int32_t top_k, uint16_t* y, void* workspace,
                    size_t workspace_bytes, void* stream);
size_t rmoe_switch_workspace_bytes(const rmoe_qweight* gate_up,
                                   const rmoe_qweight* down, int32_t tokens,
                                   int32_t top_k);

/* The routed half of the block for a caller's routing: the experts of
 * rmoe_switch_glu, then out[t] = bf16(sum_j weights[t, j] * y[t, j]) in slot
 * order, with residual != NULL out[t] = bf16(residual[t] + out[t]).  mlx-lm's
 * `(switch_mlp(x, inds) * scores[..., None]).sum(-2)` (the caller of
 * src/runnel/mlx.py:57-82), and the reference's native two-stage MoE with
 * given router weights (native/src/fused_moe_probe.mm:494-537, the
 * RNLMOE01 datasets of bench/export_ornith_moe_layer.py).  weights fp32
 * [tokens, top_k]; a slot with an out-of-range index adds nothing; out bf16
 * [tokens, hidden], not aliasing x. */
int rmoe_switch_combine(const rmoe_qweight* gate_up, const rmoe_qweight* down,
                        const uint16_t* x, int32_t tokens, const int32_t* indices,
                        const float* weights, int32_t top_k, const uint16_t* residual,
                        uint16_t* out, void* workspace, size_t workspace_bytes,
                        void* stream);
size_t rmoe_switch_combine_workspace_bytes(const rmoe_qweight* gate_up,
                                           const rmoe_qweight* down, int32_t tokens,
                                           int32_t top_k);

/* gather_qmm(x, w, scales, biases, rhs_indices, transpose=True):
 * y[m] = x[lhs[m]] . deq(w[rhs[m]])^T for m < rows.  lhs_indices == NULL
 * means row m reads x[m]; rhs_indices == NULL means expert 0; a row whose
 * index is out of range is written as zeros.  x bf16 [x_rows, w->cols];
 * exactly one of y_bf16 / y_f32 ([rows, w->rows]) is non-NULL.  Each row
 * is a group-affine dot over fp32 weights fl32(q*s + b), except a dense
 * product (no index arrays) of 64 or more rows into a 16-byte aligned
 * y_bf16 with w->rows a multiple of 256 and w->cols a multiple of 128
 * (mx.quantized_matmul at prefill sizes, the reference's qmm_4d_tile,
 * native/shaders/quantized_qmm.metal:68-151): that one runs on the matrix
 * cores with every dequantised weight rounded to bf16 and fp32
 * accumulation. */
int rmoe_gather_qmm(const uint16_t* x, int32_t x_rows,
                    const int32_t* lhs_indices, const int32_t* rhs_indices,
                    int32_t rows, const rmoe_qweight* w, uint16_t* y_bf16,
                    float* y_f32, void* stream);

/* Whole block (mlx-lm SparseMoeBlock.__call__): out[t] = bf16(sum_j
 * score_j * y_j + bf16(sigmoid(x . shared_gate_w)) * y_shared); with
 * residual != NULL, out[t] = bf16(residual[t] + out[t]).  indices_out /
 * scores_out may be NULL.  x, residual, out bf16 [tokens, hidden]; out may
 * alias residual but not x.  One token of a layer with hidden 2048, inter
 * 512, top_k <= 8 and experts <= 256 runs as one single-launch kernel on a
 * device of at least 256 CUs in 8 XCDs, such as MI355X (see
 * rmoe_workspace_status_offset); other calls that route fewer than 64
 * (token, slot) rows take the router, gate/up and down kernels; calls that
 * route 64 or more take the expert-sorted path, which needs out and
 * residual 16-byte aligned (2 bytes otherwise). */
int rmoe_moe_block(const rmoe_layer* layer, const uint16_t* x, int32_t tokens,
                   const uint16_t* residual, uint16_t* out,
                   int32_t* indices_out, float* scores_out, void* workspace,
                   size_t workspace_bytes, void* stream);

/* rmoe_moe_block without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference (its
 * probes own every buffer).  The call allocates nothing: its scratch is a
 * static device array of RMOE_NOALLOC_SCRATCH_BYTES held by each GPU the
 * library runs on until the process ends; a call that needs more
 * (rmoe_workspace_bytes(layer, tokens) > RMOE_NOALLOC_SCRATCH_BYTES, e.g.
 * long prefills) is refused with RMOE_EWS before anything is launched.
 * Every call on one GPU shares that array: calls that may overlap on one
 * GPU (different streams, different host threads) race and must be
 * serialised by the caller.  Arguments and outputs as rmoe_moe_block;
 * status_out (device uint32, may be NULL) receives this call's status word
 * (nonzero: a single-launch decode gave up a cross-workgroup wait and the
 * outputs are not valid), which the call then clears. */
#define RMOE_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int rmoe_moe_block_noalloc(const rmoe_layer* layer, const uint16_t* x, int32_t tokens,
                           const uint16_t* residual, uint16_t* out,
                           int32_t* indices_out, float* scores_out, uint32_t* status_out,
                           void* stream);

/* Batch-1 decode of one token through a stack of MoE layers with a residual
 * add between them: x_{l+1} = bf16(x_l + block_l(x_l)), one launch for the
 * whole stack (the chained decode of the reference's 40-layer model,
 * docs/architecture.md:31-37; there is no single reference entry point).
 * The layer descriptors are packed once on the host with
 * rmoe_chain_table_pack into rmoe_chain_table_bytes(n) bytes, copied by the
 * caller to device memory, and passed as device_table; layer0 describes the
 * common shape.  Needs hidden 2048, inter 512, top_k <= 8 (plus an optional
 * shared expert), experts <= 256 and a device of at least 256 CUs in 8 XCDs
 * (RMOE_EINVAL otherwise); rmoe_chain_table_pack checks the shape without
 * touching the device.  x, out bf16 [hidden]. */
size_t rmoe_chain_table_bytes(int32_t n_layers);
int rmoe_chain_table_pack(const rmoe_layer* layers, int32_t n_layers,
                          void* host_table);
int rmoe_moe_chain(const rmoe_layer* layer0, const void* device_table,
                   int32_t n_layers, const uint16_t* x, uint16_t* out,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Byte offset inside a workspace of a uint32 status word: nonzero when a
 * single-launch decode or a few-token call (2-8 tokens at the single-launch
 * shapes, whose router hands its logits over between workgroups) failed
 * (the call still completes; its outputs are then not valid): 1 when a
 * workgroup gave up a cross-workgroup wait (every wait is bounded, and the
 * other workgroups of the call stop waiting as soon as one gives up), 2 when
 * a workgroup read an XCC id outside 0-7.  The word is sticky: later calls
 * leave it set until the caller clears it.  The uint32 before it holds the
 * workspace's phase epoch and the one after it the abort word: a caller
 * cancels the next such call on the workspace before it runs by writing
 * epoch + 1 there (the call then waits for nothing and sets the status word
 * to 1). */
size_t rmoe_workspace_status_offset(void);

/* Launch mode of the single-launch decode kernel (rmoe_moe_block with one
 * token of the decode shape, rmoe_moe_chain) outside stream capture.
 * enabled = 0 (the default): a plain launch, as stream capture records it
 * (a one-token layer call takes about 14 us back to back on MI355X);
 * workgroups that wait for others that are not yet resident (kernels of
 * other streams holding CUs) wait until those run, and two single-launch
 * calls that overlap on different streams can each hold CUs the other
 * needs: their waits then give up and set the status word above.
 * enabled = 1: a cooperative launch, which guarantees every workgroup is
 * resident whatever else runs on the device, but does not overlap the
 * previous call (about 18 us more per call), for callers that run such
 * calls on several streams at once.  Process-wide; returns the previous
 * mode.  No counterpart in the reference (its probes submit one Metal
 * command buffer per call). */
int rmoe_set_cooperative_launch(int32_t enabled);

/* Affine quantization of fp32 rows [rows, cols] (group_size 64, bits 4|8):
 * per group, the larger-magnitude edge value is kept exact, scale and bias
 * are rounded to bf16 and the codes are round-half-even((w - b) / s)
 * clipped to [0, 2^bits - 1]. */
int rmoe_quantize(const float* w, int64_t rows, int32_t cols, int32_t bits,
                  int32_t group_size, uint32_t* wq, uint16_t* scales,
                  uint16_t* biases, void* stream);

/* Dequantize rows [row_begin, row_begin + rows) of the flattened bank
 * (experts * rows) to fp32 fl32(q*s + b) (out_f32) and/or to bf16 of that
 * value (out_bf16); either output may be NULL. */
int rmoe_dequantize(const rmoe_qweight* w, int64_t row_begin, int64_t rows,
                    float* out_f32, uint16_t* out_bf16, void* stream);

/* Reads `bytes` (a multiple of 16) once with 16-byte loads using `blocks`
 * workgroups of 256 lanes; workgroup i folds what it read into partials[i]
 * (device uint32 [blocks], overwritten).  Measures achievable HBM read
 * bandwidth for a given launch shape. */
int rmoe_stream_read(const void* buffer, size_t bytes, uint32_t* partials,
                     int32_t blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RMOE_H */
