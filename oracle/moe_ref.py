"""numpy oracle for the quantized sparse-MoE block.

TEST INFRASTRUCTURE ONLY.  The shipped package (runnel_amd/) never imports
this module; tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
use it to check the HIP path, never as the path itself.

What it restates, and where from:

* MLX affine packing: element k of a row sits in word k // (32/bits) at bit
  offset bits * (k % (32/bits)), LSB first; scales/biases are bf16
  ``[rows, K/group]``.  native/shaders/quantized_qmv.metal:35-44,60-64,
  native/src/fused_moe_probe.mm:649-654, bench/mlx_qmv_adapter.py:109-115,
  bench/export_ornith_moe_layer.py:119-124.
* Group-affine dot ``sum_g s_g * sum_{k in g} q_k v_k + b_g * sum_{k in g} v_k``
  (native/shaders/fused_moe.metal:20-67, bench/mlx_qmv_adapter.py:86-122),
  evaluated here in float64, which is exact for these operands to far below
  one bf16 ulp.
* The packed ``[up; gate]`` bank and SwiGLU ``silu(gate) * up``:
  src/runnel/mlx.py:38-48,76-78, native/shaders/fused_moe.metal:448-449,534-541.
* The caller's block (mlx-lm SparseMoeBlock, third-party, not present here):
  router ``x @ W_r.T`` -> softmax -> top-k -> renormalise -> switch_mlp ->
  ``sum_j score_j y_j`` + ``sigmoid(x . w_sg) * shared(x)``, whose call into
  the packed module is src/runnel/mlx.py:57-82.
* The prefill permutation ``_gather_sort`` / ``_scatter_unsort`` used at
  src/runnel/mlx.py:59-63,80-81 (mlx-lm): stable sort of the flattened
  (token, slot) expert ids.

Definitions that are this library's own (mlx / mlx-lm cannot run here, so the
exact bf16 rounding points inside ``gather_qmm`` and the tie order of
``argpartition`` are unpinned):

* Router logits use a fixed fp32 reduction order (``router_logits``) so the
  GPU and this oracle produce identical bf16 logits; top-k orders by
  (bf16 logit descending, expert index ascending).  Because softmax and bf16
  rounding are monotone, that selection is always one valid top-k of
  mlx-lm's bf16 probabilities.
* A quantized gate (8-bit group-64 ``QuantizedLinear``, the format real
  checkpoints give ``mlp.gate`` / ``mlp.shared_expert_gate``,
  bench/runnel_bench/checkpoint.py:200-208) has its own fixed order
  (``qrouter_logits``: 16-code chunks per lane, per chunk
  ``fma(sum q x, s, acc)`` then ``fma(sum x, b, acc)``, then the butterfly).
  Its fp32 FMA is emulated exactly (``fma32``, rounding to odd).  Pinned by
  the C restatement with libm's fmaf (bit-equal), by a closed form on
  integer data (every partial sum exact), by the rounding-error bound
  against the float64 dot, and by constructed double-rounding cases for
  ``fma32`` itself (tests/test_oracle.py).  mlx's quantized_matmul order is
  third-party and unpinned; the mlx-lm-style evaluation is held to the
  end-to-end tolerance (max-abs <= 2e-2, cosine >= 0.9999) instead.
* ``block_forward(mode="contract")`` is the HIP kernels' contract: fp32/f64
  arithmetic with bf16 rounding of x_up, x_gate, the SwiGLU activation, each
  expert's down output, the router probabilities, the renormalisation
  denominator (mlx-lm's ``scores.sum(-1)`` of bf16 scores is bf16), the
  scores, the shared gate and the block output.  ``mode="mlx"`` adds the extra bf16 roundings an
  op-by-op mlx-lm evaluation performs (silu output, score products, the
  routed sum, the gated shared term); the end-to-end tolerance
  (max-abs <= 2e-2, cosine >= 0.9999) is checked against it.
  ``mode="prefill"`` is the contract of the expert-sorted grouped GEMM used
  when a call routes at least 64 (token, slot) rows (the reference's sort
  threshold, src/runnel/mlx.py:59): the same rounding points, with each
  dequantised weight rounded to bf16 before the product (the operand of a
  bf16 matrix-core tile); this rounding point is the build's own choice.
* ``quantize`` restates MLX's documented affine quantizer (edge value kept
  exact, scale sign chosen by the larger-magnitude edge).  It only produces
  test weights; parity of the block never depends on it.  Parity unpinned
  against ``mx.quantize`` itself; pinned by invariants (|deq - w| <= |s|/2
  plus bf16 slack, codes in range) in tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

# --------------------------------------------------------------------------
# bf16
# --------------------------------------------------------------------------


def f32_to_bf16(a) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even; NaN/Inf are truncated
    (native/src/fused_moe_probe.mm:89-97)."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    bits = a.view(np.uint32).astype(np.uint64)
    special = ((bits >> 23) & 0xFF) == 0xFF
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    out = np.where(special, bits >> 16, rounded)
    return out.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(a))


# --------------------------------------------------------------------------
# MLX affine format
# --------------------------------------------------------------------------


def values_per_word(bits: int) -> int:
    if bits not in (4, 8):
        raise ValueError(f"unsupported bits {bits}")
    return 32 // bits


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """Integer codes [..., K] -> uint32 words [..., K / (32/bits)], LSB first."""
    vpp = values_per_word(bits)
    q = np.asarray(q, dtype=np.uint32)
    if q.shape[-1] % vpp:
        raise ValueError("K must be a multiple of the values per word")
    if q.size and int(q.max()) >= (1 << bits):
        raise ValueError("code out of range")
    q = q.reshape(*q.shape[:-1], q.shape[-1] // vpp, vpp)
    shifts = (np.arange(vpp, dtype=np.uint32) * bits)
    return np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)


def unpack(w: np.ndarray, bits: int) -> np.ndarray:
    """uint32 words [..., W] -> codes [..., W * (32/bits)] (uint32)."""
    vpp = values_per_word(bits)
    w = np.asarray(w, dtype=np.uint32)
    shifts = (np.arange(vpp, dtype=np.uint32) * bits)
    q = (w[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return q.reshape(*w.shape[:-1], w.shape[-1] * vpp)


def quantize(w: np.ndarray, bits: int, group: int = 64):
    """Affine quantization of float rows [..., K] -> (u32 words, bf16 scales
    bits, bf16 biases bits).  Computed in float32; the codes are chosen
    against the bf16-rounded scale and bias, so dequantization reproduces the
    nearest representable grid point."""
    w = np.asarray(w, dtype=np.float32)
    lead = w.shape[:-1]
    K = w.shape[-1]
    if K % group:
        raise ValueError("K must be a multiple of group")
    g = w.reshape(-1, K // group, group)
    n_bins = np.float32((1 << bits) - 1)
    w_max = g.max(axis=-1)
    w_min = g.min(axis=-1)
    mask = np.abs(w_min) > np.abs(w_max)
    scales = np.maximum((w_max - w_min) / n_bins, np.float32(1e-7)).astype(np.float32)
    scales = np.where(mask, scales, -scales).astype(np.float32)
    edge = np.where(mask, w_min, w_max).astype(np.float32)
    q0 = np.rint(edge / scales).astype(np.float32)
    safe_q0 = np.where(q0 != 0, q0, np.float32(1))
    scales = np.where(q0 != 0, edge / safe_q0, scales).astype(np.float32)
    biases = np.where(q0 == 0, np.float32(0), edge).astype(np.float32)
    s_bits = f32_to_bf16(scales)
    b_bits = f32_to_bf16(biases)
    s = bf16_to_f32(s_bits)[..., None]
    b = bf16_to_f32(b_bits)[..., None]
    q = np.clip(np.rint((g - b) / s), 0, n_bins).astype(np.uint32)
    words = pack(q.reshape(-1, K), bits)
    return (words.reshape(*lead, K // values_per_word(bits)),
            s_bits.reshape(*lead, K // group),
            b_bits.reshape(*lead, K // group))


def dequantize(words, scales, biases, bits: int, group: int = 64,
               dtype=np.float32) -> np.ndarray:
    """Closed form w = q*s + b.  q*s is exact in fp32 (<= 8 + 8 significant
    bits), so the float32 result is fl32(q*s + b), one rounding, whether or
    not the multiply-add is fused."""
    q = unpack(words, bits).astype(np.float64)
    s = bf16_to_f32(scales).astype(np.float64)
    b = bf16_to_f32(biases).astype(np.float64)
    K = q.shape[-1]
    s = np.repeat(s, group, axis=-1)[..., :K]
    b = np.repeat(b, group, axis=-1)[..., :K]
    exact = q * s + b  # exact in float64
    return exact.astype(dtype)


# --------------------------------------------------------------------------
# Router
# --------------------------------------------------------------------------


def router_logits(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """fp32 logits in the GPU router's fixed reduction order.

    x_bits [T, H], w_bits [E, H] (bf16 bits) -> float32 [T, E] (not rounded).
    The reduction axis is cut into 8-element chunks; lane l of 64 sums chunks
    l, l+64, ... element by element from +0.0; the lane sums are combined by
    the butterfly p_l <- p_l + p_(l xor d), d = 1, 2, 4, 8, 16, 32.  The
    products of two bf16 values are exact in float32.
    """
    x = bf16_to_f32(x_bits)
    w = bf16_to_f32(w_bits)
    T, H = x.shape
    E = w.shape[0]
    if H % 8:
        raise ValueError("hidden size must be a multiple of 8")
    chunks = H // 8
    rounds = (chunks + 63) // 64
    p = np.zeros((T, E, 64), dtype=np.float32)
    lanes = np.arange(64)
    for i in range(rounds):
        c = i * 64 + lanes
        valid = c < chunks
        cv = np.where(valid, c, 0)
        for j in range(8):
            k = cv * 8 + j
            prod = x[:, None, k] * w[None, :, k]  # [T, E, 64], exact
            p = np.where(valid[None, None, :], p + prod, p).astype(np.float32)
    for d in (1, 2, 4, 8, 16, 32):
        p = (p + p[:, :, lanes ^ d]).astype(np.float32)
    return p[:, :, 0]


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded float32 fused multiply-add fl32(a * b + c), the
    operation of C's fmaf and of the GPU's v_fma_f32.

    a * b is exact in float64 (two 24-bit significands).  The sum is rounded
    to odd at float64 precision: rounded to nearest, then, when the TwoSum
    error is nonzero and the result's last bit is even, moved one float64 ulp
    towards the exact value.  Rounding to odd at 53 bits followed by rounding
    to nearest at 24 bits equals a single rounding to nearest (Boldo and
    Melquiond, "Emulation of FMA and correctly rounded sums: proved
    algorithms using rounding to odd", IEEE Trans. Computers 57(4), 2008;
    it needs 53 >= 24 + 2)."""
    a = np.asarray(a, dtype=np.float32).astype(np.float64)
    b = np.asarray(b, dtype=np.float32).astype(np.float64)
    c = np.asarray(c, dtype=np.float32).astype(np.float64)
    p = a * b
    s = p + c
    pv = s - c                          # TwoSum: s + err == p + c exactly
    cv = s - pv
    err = (c - cv) + (p - pv)
    even = (np.asarray(s).view(np.int64) & 1) == 0
    toward = np.where(err > 0, np.inf, -np.inf)
    s = np.where((err != 0) & even, np.nextafter(s, toward), s)
    return np.asarray(s).astype(np.float32)


def qrouter_logits(x_bits: np.ndarray, qw: "QWeight") -> np.ndarray:
    """fp32 logits [T, rows] of an MLX-affine quantized gate (the 8-bit
    group-64 ``QuantizedLinear`` that real checkpoints carry for
    ``mlp.gate`` and ``mlp.shared_expert_gate``, counted at
    bench/runnel_bench/checkpoint.py:200-208 and overridden to 8 bits in
    bench/results/m0/checkpoint-ornith-mlx-8bit.json:163-175), in the GPU
    router's fixed order.  Not rounded.

    The codes of a row are cut into 16-byte chunks of V = 128 / bits values
    (a group of 64 spans 64 / V chunks); lane l of 64 takes chunks l, l+64,
    ... in order, from acc = +0.  For a chunk with inputs x_i, codes q_i and
    its group's scale s and bias b:

        qa  = q_0 x_0 + q_1 x_1 + ...   sequentially from +0 (products exact)
        xs  = x_0 + x_1 + ...           sequentially from +0
        acc = fma(qa, s, acc);  acc = fma(xs, b, acc)

    and the 64 lane sums are combined by the same butterfly as
    ``router_logits``.  ``qw`` is a one-expert bank [1, rows, H]."""
    x = bf16_to_f32(x_bits)
    T, H = x.shape
    if qw.experts != 1 or qw.cols != H or qw.group != 64:
        raise ValueError("quantized gate must be a [1, rows, hidden] bank with group 64")
    V = 128 // qw.bits
    q = unpack(qw.w[0], qw.bits).astype(np.float32)       # [E, H]
    s = bf16_to_f32(qw.scales[0])                          # [E, H / 64]
    b = bf16_to_f32(qw.biases[0])
    E = q.shape[0]
    chunks = H // V
    lanes = np.arange(64)
    acc = np.zeros((T, E, 64), dtype=np.float32)
    for i in range((chunks + 63) // 64):
        c = i * 64 + lanes
        valid = c < chunks
        cv = np.where(valid, c, 0)
        qa = np.zeros((T, E, 64), dtype=np.float32)
        xs = np.zeros((T, 64), dtype=np.float32)
        for j in range(V):
            k = cv * V + j
            qa = (qa + q[None, :, k] * x[:, None, k]).astype(np.float32)
            xs = (xs + x[:, k]).astype(np.float32)
        g = (cv * V) // 64
        new = fma32(qa, s[None, :, g], acc)
        new = fma32(np.broadcast_to(xs[:, None, :], new.shape), b[None, :, g], new)
        acc = np.where(valid[None, None, :], new, acc)
    for d in (1, 2, 4, 8, 16, 32):
        acc = (acc + acc[:, :, lanes ^ d]).astype(np.float32)
    return acc[:, :, 0]


def gate_logits(x_bits: np.ndarray, gate) -> np.ndarray:
    """fp32 router logits [T, rows] for a bf16 gate (bits [rows, H]) or a
    quantized one (QWeight [1, rows, H])."""
    if isinstance(gate, QWeight):
        return qrouter_logits(x_bits, gate)
    return router_logits(x_bits, gate)


def rms_norm(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """The decoder layer's post-attention RMSNorm in front of the block
    (``mx.fast.rms_norm(x, w, eps)``; the checkpoints store the effective
    weight): bf16 bits [T, H] -> bf16 bits [T, H].

    This library's fixed order: s = sum x_k^2 in the router contract's order
    (8-element chunks, lane l of 64 takes chunks l, l+64, ... from +0, then
    the butterfly; the squares of bf16 values are exact in fp32), then in
    fp32 with correct rounding ms = s / H, v = ms + eps, r = 1 / sqrt(v), and
    per element n = bf16(x r), y = bf16(n w)."""
    x_bits = np.asarray(x_bits, np.uint16)
    T, H = x_bits.shape
    s = np.empty(T, np.float32)
    for t in range(T):
        s[t] = router_logits(x_bits[t:t + 1], x_bits[t:t + 1])[0, 0]
    ms = (s / np.float32(H)).astype(np.float32)
    v = (ms + np.float32(eps)).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt(v)).astype(np.float32)
    n = round_bf16(bf16_to_f32(x_bits) * r[:, None])
    return f32_to_bf16(n * bf16_to_f32(np.asarray(w_bits, np.uint16))[None, :])


def topk_rank(logits_bf16: np.ndarray, k: int) -> np.ndarray:
    """Indices [T, k] ordered by (logit desc, index asc)."""
    order = np.argsort(-logits_bf16, axis=-1, kind="stable")
    return order[:, :k].astype(np.int32)


def boundary_ties(logits_bf16: np.ndarray, k: int) -> np.ndarray:
    """True where the k-th and (k+1)-th largest bf16 logits are equal, i.e.
    where another valid top-k selection exists."""
    s = -np.sort(-logits_bf16, axis=-1)
    if s.shape[-1] <= k:
        return np.zeros(s.shape[0], dtype=bool)
    return s[:, k - 1] == s[:, k]


def _sigmoid32(v):
    v = np.asarray(v, dtype=np.float32)
    return (np.float32(1) / (np.float32(1) + np.exp(-v))).astype(np.float32)


def _silu32(v):
    v = np.asarray(v, dtype=np.float32)
    return (v / (np.float32(1) + np.exp(-v))).astype(np.float32)


def route(x_bits, router_w_bits, top_k, norm_topk_prob=True):
    """-> (idx [T,k] int32, scores [T,k] float32, logits bf16-valued [T,E]).
    ``router_w_bits`` is a bf16 gate [E, H] or a quantized one (QWeight
    [1, E, H])."""
    logits = round_bf16(gate_logits(x_bits, router_w_bits))
    idx = topk_rank(logits, top_k)
    return idx, selected_scores(logits, idx, norm_topk_prob), logits


def selected_scores(logits, idx, norm_topk_prob=True):
    """Scores of the selected experts ``idx`` [T, k] from bf16-valued logits
    [T, E]: softmax in fp32 over every expert (sequential sum), probabilities
    rounded to bf16 (mlx's softmax of bf16 logits returns bf16), and with
    ``norm_topk_prob`` divided by ``scores.sum(-1)``, which mlx-lm computes on
    bf16 scores and so rounds to bf16 (fp32 sum in slot order, then bf16);
    the quotient is bf16."""
    m = logits.max(axis=-1, keepdims=True)
    e = np.exp((logits - m).astype(np.float32)).astype(np.float32)
    z = np.zeros(e.shape[0], dtype=np.float32)
    for i in range(e.shape[1]):
        z = (z + e[:, i]).astype(np.float32)
    p = (e / z[:, None]).astype(np.float32)
    pb = round_bf16(np.take_along_axis(p, idx, axis=-1))
    if not norm_topk_prob:
        return pb.astype(np.float32)
    tot = np.zeros(pb.shape[0], dtype=np.float32)
    for j in range(idx.shape[1]):
        tot = (tot + pb[:, j]).astype(np.float32)
    return round_bf16(pb / round_bf16(tot)[:, None]).astype(np.float32)


# --------------------------------------------------------------------------
# Layer container and the block
# --------------------------------------------------------------------------


@dataclass
class QWeight:
    """One MLX-affine bank: words [E, rows, K/vpp] u32, scales/biases
    [E, rows, K/group] bf16 bits."""
    w: np.ndarray
    scales: np.ndarray
    biases: np.ndarray
    bits: int
    group: int = 64

    @property
    def experts(self):
        return self.w.shape[0]

    @property
    def rows(self):
        return self.w.shape[1]

    @property
    def cols(self):
        return self.w.shape[2] * values_per_word(self.bits)

    def dequant(self, e: int) -> np.ndarray:
        return dequantize(self.w[e], self.scales[e], self.biases[e], self.bits,
                          self.group, dtype=np.float64)


@dataclass
class Layer:
    hidden: int
    inter: int
    experts: int
    top_k: int
    router_w: "np.ndarray | QWeight"   # bf16 bits [E, H], or an 8-bit bank [1, E, H]
    gate_up: QWeight               # [E, 2I, H], rows [up; gate]
    down: QWeight                  # [E, H, I]
    shared_gate_w: "np.ndarray | QWeight | None" = None  # bf16 bits [H], or [1, 1, H]
    shared_gate_up: QWeight | None = None     # [1, 2Is, H]
    shared_down: QWeight | None = None        # [1, H, Is]
    norm_topk_prob: bool = True
    post_norm_w: np.ndarray | None = None     # bf16 bits [H]: RMSNorm before the block
    norm_eps: float = 1e-6

    @property
    def shared_inter(self):
        return 0 if self.shared_gate_up is None else self.shared_gate_up.rows // 2


def _bf16_weights(w64: np.ndarray) -> np.ndarray:
    """Prefill weight tile: fl32(q*s + b) rounded to bf16 (RNE), the operand
    a bf16 matrix-core product consumes."""
    return round_bf16(w64.astype(np.float32)).astype(np.float64)


def expert_ffn(gate_up: QWeight, down: QWeight, e: int, xf: np.ndarray,
               mode: str = "contract") -> np.ndarray:
    """Rows of xf (float32 [n, H], bf16-valued) through expert e.
    Returns y [n, H] float32 (bf16-valued).  ``mode="prefill"`` is the
    contract with every dequantised weight rounded to bf16 first (the
    expert-sorted grouped GEMM's operand); the rest is the same."""
    I = gate_up.rows // 2
    wgu = gate_up.dequant(e)  # [2I, H] float64
    if mode == "prefill":
        wgu = _bf16_weights(wgu)
    gu = xf.astype(np.float64) @ wgu.T
    up = round_bf16(gu[:, :I].astype(np.float32))
    gate = round_bf16(gu[:, I:].astype(np.float32))
    if mode == "mlx":
        act = round_bf16(round_bf16(_silu32(gate)) * up)
    else:
        act = round_bf16(_silu32(gate) * up)
    wdn = down.dequant(e)  # [H, I]
    if mode == "prefill":
        wdn = _bf16_weights(wdn)
    y = act.astype(np.float64) @ wdn.T
    return round_bf16(y.astype(np.float32))


def switch_glu(layer: Layer, x_bits: np.ndarray, idx: np.ndarray,
               mode: str = "contract") -> np.ndarray:
    """FusedQuantizedSwitchGLU.__call__ (src/runnel/mlx.py:57-82): per-slot,
    uncombined expert outputs [T, k, H] (bf16-valued float32)."""
    xf = bf16_to_f32(x_bits)
    T, k = idx.shape
    y = np.zeros((T, k, layer.hidden), dtype=np.float32)
    flat = idx.reshape(-1)
    for e in np.unique(flat):
        rows = np.nonzero(flat == e)[0]
        t = rows // k
        y.reshape(-1, layer.hidden)[rows] = expert_ffn(
            layer.gate_up, layer.down, int(e), xf[t], mode)
    return y


def block_forward(layer: Layer, x_bits: np.ndarray, residual_bits=None,
                  mode: str = "contract", idx: np.ndarray | None = None):
    """Whole block.  x_bits [T, H] bf16 bits -> (out bf16 bits [T, H], idx,
    scores).  ``idx`` forces the routing (used to compare outputs when a
    boundary tie leaves more than one valid selection).  With
    ``layer.post_norm_w`` the block's input is ``rms_norm(x)`` (the residual
    stays what the caller passes)."""
    if layer.post_norm_w is not None:
        x_bits = rms_norm(x_bits, layer.post_norm_w, layer.norm_eps)
    r_idx, scores, logits = route(x_bits, layer.router_w, layer.top_k,
                                  layer.norm_topk_prob)
    if idx is None:
        idx = r_idx
    else:
        # scores of the forced selection
        scores = selected_scores(logits, idx, layer.norm_topk_prob)
    y = switch_glu(layer, x_bits, idx, mode)
    T = x_bits.shape[0]
    if mode == "mlx":
        acc = np.zeros((T, layer.hidden), dtype=np.float32)
        for j in range(layer.top_k):
            acc = acc + round_bf16(y[:, j, :] * scores[:, j:j + 1])
        acc = round_bf16(acc)
    else:
        acc = np.zeros((T, layer.hidden), dtype=np.float32)
        for j in range(layer.top_k):
            acc = (acc + scores[:, j:j + 1] * y[:, j, :]).astype(np.float32)
    if layer.shared_gate_up is not None:
        xf = bf16_to_f32(x_bits)
        ysh = expert_ffn(layer.shared_gate_up, layer.shared_down, 0, xf, mode)
        if layer.shared_gate_w is not None:
            sgw = layer.shared_gate_w
            sl = round_bf16(gate_logits(x_bits, sgw if isinstance(sgw, QWeight)
                                        else sgw[None, :])[:, 0])
            sg = round_bf16(_sigmoid32(sl))[:, None]
        else:
            sg = np.ones((T, 1), dtype=np.float32)
        if mode == "mlx":
            acc = acc + round_bf16(sg * ysh)
        else:
            acc = (acc + sg * ysh).astype(np.float32)
    out = round_bf16(acc)
    if residual_bits is not None:
        out = round_bf16(bf16_to_f32(residual_bits) + out)
    return f32_to_bf16(out), idx, scores


def gather_sort(indices: np.ndarray):
    """mlx-lm ``_gather_sort`` semantics: stable order of the flattened
    (token, slot) rows by expert id.  Returns (order, sorted expert ids,
    inverse order); row r of the sorted problem is token order[r] // k."""
    flat = indices.reshape(-1)
    order = np.argsort(flat, kind="stable")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    return order, flat[order], inv


# --------------------------------------------------------------------------
# Synthetic layers (numpy; small sizes for tests)
# --------------------------------------------------------------------------


def make_layer(seed: int, hidden=2048, inter=512, experts=256, top_k=8,
               bits=8, group=64, shared=True, w_std=0.02, router_std=0.02,
               shared_inter=None, router_bits=None) -> Layer:
    """Weights ~ N(0, w_std) quantized with ``quantize``; router and shared
    gate ~ N(0, router_std) in bf16, or quantized to ``router_bits`` (one-
    expert banks [1, E, H] and [1, 1, H]) when it is given."""
    rng = np.random.default_rng(seed)
    shared_inter = inter if shared_inter is None else shared_inter

    def qbank(e, rows, cols):
        w = rng.standard_normal((e, rows, cols), dtype=np.float32) * np.float32(w_std)
        words, s, b = quantize(w.reshape(e * rows, cols), bits, group)
        return QWeight(words.reshape(e, rows, -1), s.reshape(e, rows, -1),
                       b.reshape(e, rows, -1), bits, group)

    def gate(rows):
        w = rng.standard_normal((rows, hidden), dtype=np.float32) * np.float32(router_std)
        if router_bits is None:
            return f32_to_bf16(w if rows > 1 else w[0])
        words, s, b = quantize(w, router_bits, group)
        return QWeight(words[None], s[None], b[None], router_bits, group)

    router = gate(experts)
    gu = qbank(experts, 2 * inter, hidden)
    dn = qbank(experts, hidden, inter)
    layer = Layer(hidden, inter, experts, top_k, router, gu, dn)
    if shared:
        layer.shared_gate_w = gate(1)
        layer.shared_gate_up = qbank(1, 2 * shared_inter, hidden)
        layer.shared_down = qbank(1, hidden, shared_inter)
    return layer


def make_x(seed: int, T: int, hidden: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return f32_to_bf16(rng.standard_normal((T, hidden), dtype=np.float32))


# --------------------------------------------------------------------------
# C oracle (oracle/cpu_moe.c) through ctypes
# --------------------------------------------------------------------------

_LIB = None


def c_oracle():
    """Load oracle/_build/libmoe_oracle.so, building it first when the
    sources are present and the library is not."""
    global _LIB
    if _LIB is not None:
        return _LIB
    so = HERE / "_build" / "libmoe_oracle.so"
    if not so.exists():
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    lib = ctypes.CDLL(str(so))
    P = ctypes.c_void_p
    S = ctypes.c_size_t
    lib.orc_qmv_build.argtypes = [ctypes.c_int, S, S, S, S, S, P, S, P, P, P, P, P]
    lib.orc_fused_build.argtypes = [ctypes.c_int, S, P, P, P, P, P, P, P, P]
    lib.orc_fused_reference.argtypes = [ctypes.c_int, P, P, P, P, P, P, P, P, P, P, P]
    lib.orc_qmm_build.argtypes = [ctypes.c_int, S, S, S, P, P, P, P, P]
    lib.orc_router_dot.argtypes = [P, P, ctypes.c_int]
    lib.orc_router_dot.restype = ctypes.c_float
    lib.orc_qrouter_dot.argtypes = [P, ctypes.c_int, P]
    lib.orc_qrouter_dot.restype = ctypes.c_float
    lib.orc_fmaf_array.argtypes = [P, P, P, P, S]
    lib.orc_rms_norm.argtypes = [P, P, ctypes.c_int, ctypes.c_float, P]
    lib.orc_moe_block.argtypes = [P, P, ctypes.c_int, P, P, P, P, ctypes.c_int]
    lib.orc_random_sequence.argtypes = [ctypes.c_uint64, S, P]
    lib.orc_random_sequence.restype = ctypes.c_uint32
    lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.orc_f32_to_bf16.restype = ctypes.c_uint16
    lib.orc_max_threads.restype = ctypes.c_int
    _LIB = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def qmv_dataset(bits, output_size, reduction_size, group=64, bank_rows=0,
                rows_per_expert=0, selected=()):
    """The reference QMV probe's synthetic dataset and its CPU-oracle output
    (native/src/quantized_qmv_probe.mm:355-433)."""
    lib = c_oracle()
    vpp = values_per_word(bits)
    rows = bank_rows or output_size
    w = np.zeros(rows * reduction_size // vpp, np.uint32)
    s = np.zeros(rows * reduction_size // group, np.uint16)
    b = np.zeros_like(s)
    x = np.zeros(reduction_size, np.uint16)
    e = np.zeros(output_size, np.float32)
    sel = np.asarray(list(selected), dtype=np.uint32)
    rc = lib.orc_qmv_build(bits, output_size, reduction_size, group, bank_rows,
                           rows_per_expert, _p(sel) if sel.size else None,
                           sel.size, _p(w), _p(s), _p(b), _p(x), _p(e))
    if rc != 0:
        raise ValueError("invalid QMV dataset parameters")
    return {"w": w.reshape(rows, -1), "scales": s.reshape(rows, -1),
            "biases": b.reshape(rows, -1), "x": x, "expected": e,
            "selected": sel if sel.size else np.zeros(1, np.uint32)}


def write_rnlqmv02(path, ds, bits, output_size, reduction_size, group,
                   bank_rows, rows_per_expert):
    """RNLQMV02 writer (native/src/quantized_qmv_probe.mm:310-340;
    header layout bench/mlx_qmv_adapter.py:18-19)."""
    import struct
    rows = bank_rows or output_size
    rpe = rows_per_expert or output_size
    sel = ds["selected"]
    with open(path, "wb") as f:
        f.write(struct.pack("<8sIIIIIIII", b"RNLQMV02", 2, bits, output_size,
                            rows, rpe, reduction_size, group, sel.size))
        for a, dt in ((ds["w"], "<u4"), (ds["scales"], "<u2"),
                      (ds["biases"], "<u2"), (ds["x"], "<u2"), (sel, "<u4")):
            f.write(np.asarray(a, dtype=dt).tobytes(order="C"))


def fused_dataset(bits, total_experts=64):
    """The reference fused probe's synthetic dataset
    (native/src/fused_moe_probe.mm:449-492)."""
    lib = c_oracle()
    vpp = values_per_word(bits)
    gu_w = np.zeros(total_experts * 1024 * 2048 // vpp, np.uint32)
    gu_s = np.zeros(total_experts * 1024 * 32, np.uint16)
    gu_b = np.zeros_like(gu_s)
    dn_w = np.zeros(total_experts * 2048 * 512 // vpp, np.uint32)
    dn_s = np.zeros(total_experts * 2048 * 8, np.uint16)
    dn_b = np.zeros_like(dn_s)
    x = np.zeros(2048, np.uint16)
    router = np.zeros(8, np.float32)
    rc = lib.orc_fused_build(bits, total_experts, _p(gu_w), _p(gu_s), _p(gu_b),
                             _p(dn_w), _p(dn_s), _p(dn_b), _p(x), _p(router))
    if rc != 0:
        raise ValueError("invalid fused dataset parameters")
    E = total_experts
    return {
        "gate_up": QWeight(gu_w.reshape(E, 1024, -1), gu_s.reshape(E, 1024, -1),
                           gu_b.reshape(E, 1024, -1), bits),
        "down": QWeight(dn_w.reshape(E, 2048, -1), dn_s.reshape(E, 2048, -1),
                        dn_b.reshape(E, 2048, -1), bits),
        "x": x, "router": router,
    }


def fused_reference(bits, ds, selected):
    lib = c_oracle()
    sel = np.asarray(selected, dtype=np.uint32)
    out = np.zeros(2048, np.float32)
    inter = np.zeros(8 * 512, np.float32)
    gu, dn = ds["gate_up"], ds["down"]
    lib.orc_fused_reference(bits, _p(sel), _p(gu.w), _p(gu.scales), _p(gu.biases),
                            _p(dn.w), _p(dn.scales), _p(dn.biases), _p(ds["x"]),
                            _p(ds["router"]), _p(out), _p(inter))
    return out, inter.reshape(8, 512)


def qmm_dataset(bits, tokens, outputs, reduction):
    """The reference QMM probe's dataset (native/src/quantized_qmm_probe.mm:243-307)."""
    lib = c_oracle()
    vpp = values_per_word(bits)
    w = np.zeros(outputs * reduction // vpp, np.uint32)
    s = np.zeros(outputs * reduction // 64, np.uint16)
    b = np.zeros_like(s)
    x = np.zeros(tokens * reduction, np.uint16)
    e = np.zeros(tokens * outputs, np.float32)
    rc = lib.orc_qmm_build(bits, tokens, outputs, reduction, _p(w), _p(s), _p(b),
                           _p(x), _p(e))
    if rc != 0:
        raise ValueError("invalid QMM dataset parameters")
    return {"w": w.reshape(outputs, -1), "scales": s.reshape(outputs, -1),
            "biases": b.reshape(outputs, -1), "x": x.reshape(tokens, reduction),
            "expected": e.reshape(tokens, outputs)}


class _CQW(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("biases", ctypes.c_void_p), ("experts", ctypes.c_int32),
                ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
                ("bits", ctypes.c_int32), ("group", ctypes.c_int32)]


class _CLayer(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("inter", ctypes.c_int32),
                ("shared_inter", ctypes.c_int32), ("experts", ctypes.c_int32),
                ("top_k", ctypes.c_int32), ("norm_topk_prob", ctypes.c_int32),
                ("router_w", ctypes.c_void_p), ("shared_gate_w", ctypes.c_void_p),
                ("gate_up", _CQW), ("down", _CQW), ("shared_gate_up", _CQW),
                ("shared_down", _CQW), ("router_q", _CQW), ("shared_gate_q", _CQW),
                ("post_norm_w", ctypes.c_void_p), ("norm_eps", ctypes.c_float)]


def _cqw(q: QWeight | None, keep):
    if q is None:
        return _CQW()
    arrs = [np.ascontiguousarray(q.w), np.ascontiguousarray(q.scales),
            np.ascontiguousarray(q.biases)]
    keep.extend(arrs)
    return _CQW(_p(arrs[0]).value, _p(arrs[1]).value, _p(arrs[2]).value,
                q.experts, q.rows, q.cols, q.bits, q.group)


def c_block_forward(layer: Layer, x_bits: np.ndarray, residual_bits=None,
                    nthreads: int = 0):
    """The same block contract through oracle/cpu_moe.c (fp32, OpenMP)."""
    lib = c_oracle()
    keep: list = []
    rq = layer.router_w if isinstance(layer.router_w, QWeight) else None
    sgq = layer.shared_gate_w if isinstance(layer.shared_gate_w, QWeight) else None
    router = None if rq is not None else np.ascontiguousarray(layer.router_w)
    sg = (None if layer.shared_gate_w is None or sgq is not None
          else np.ascontiguousarray(layer.shared_gate_w))
    pnw = None if layer.post_norm_w is None else np.ascontiguousarray(layer.post_norm_w,
                                                                        dtype=np.uint16)
    keep += [router, sg, pnw]
    cl = _CLayer(layer.hidden, layer.inter, layer.shared_inter, layer.experts,
                 layer.top_k, int(layer.norm_topk_prob),
                 None if router is None else _p(router).value,
                 None if sg is None else _p(sg).value,
                 _cqw(layer.gate_up, keep), _cqw(layer.down, keep),
                 _cqw(layer.shared_gate_up, keep), _cqw(layer.shared_down, keep),
                 _cqw(rq, keep), _cqw(sgq, keep),
                 None if layer.post_norm_w is None else _p(pnw).value, layer.norm_eps)
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    T = x.shape[0]
    out = np.zeros((T, layer.hidden), np.uint16)
    idx = np.zeros((T, layer.top_k), np.int32)
    scores = np.zeros((T, layer.top_k), np.float32)
    res = None if residual_bits is None else np.ascontiguousarray(residual_bits, dtype=np.uint16)
    rc = lib.orc_moe_block(ctypes.byref(cl), _p(x), T, _p(res), _p(out), _p(idx),
                           _p(scores), nthreads)
    if rc != 0:
        raise ValueError("C oracle rejected the layer")
    return out, idx, scores


def cpu_count() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
