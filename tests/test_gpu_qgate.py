"""GPU parity with an 8-bit group-64 quantized router and shared-expert gate
(the format real checkpoints carry for mlp.gate / mlp.shared_expert_gate):
routing bit-exact against the oracle's quantized-gate contract on every path
that ranks experts (the per-token router, the single-launch decode, the
chained decode and the matrix-core prefill router), outputs within a bf16
rounding step of the contract and within the end-to-end tolerance (max-abs 2e-2, cosine 0.9999) of the
mlx-lm-style evaluation."""

import numpy as np
import pytest

from helpers import (cosine, dev_bf16, gate_to_dev, host_bf16, layer_from_dev,
                     layer_to_dev)
from oracle import moe_ref as M

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9999


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runnel_amd import _lib
    _lib.load()
    return torch


def _mismatches(got_bits, ref_bits):
    g = M.bf16_to_f32(got_bits).astype(np.float64)
    r = M.bf16_to_f32(ref_bits).astype(np.float64)
    tol = np.maximum(np.abs(r), 1e-3) * 2.0 ** -6 + 1e-6
    return int((np.abs(g - r) > tol).sum())


def _check_outputs(got_bits, L, xb, mode="contract", residual=None):
    # An activation whose fp32 value sits within accumulation error of a bf16
    # rounding midpoint rounds differently from the float64 oracle; the flip
    # moves every output of its token by ~1e-4, which exceeds the relative
    # bound on the few outputs near zero (a few dozen of one token's 2048).
    ref, _, _ = M.block_forward(L, xb, residual_bits=residual, mode=mode)
    assert _mismatches(got_bits, ref) <= max(2, got_bits.size // 200)
    mlx, _, _ = M.block_forward(L, xb, residual_bits=residual, mode="mlx")
    g, m = M.bf16_to_f32(got_bits), M.bf16_to_f32(mlx)
    assert np.abs(g - m).max() <= MAX_ABS
    assert cosine(g, m) >= MIN_COS


@pytest.mark.parametrize("T,H,E,K", [(1, 2048, 256, 8), (7, 2048, 256, 8), (40, 512, 64, 6),
                                     (3, 320, 16, 4)])
def test_quantized_router_exact(torch_cuda, T, H, E, K):
    """rmoe_router_q: indices bit for bit, scores within a bf16 step, for
    full rows, short rows (fewer than 64 chunks) and a partial lane round."""
    torch = torch_cuda
    from runnel_amd import native
    L = M.make_layer(300 + T, hidden=H, inter=64, experts=E, top_k=K, router_bits=8,
                     shared=False)
    x = M.make_x(301 + T, T, H)
    idx, scores = native.router(gate_to_dev(L.router_w), dev_bf16(x), K)
    torch.cuda.synchronize()
    ref_idx, ref_scores, _ = M.route(x, L.router_w, K)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.abs(scores.cpu().numpy() - ref_scores).max() <= 2.0 ** -8


def test_quantized_router_ties_break_by_index(torch_cuda):
    """Identical gate rows give exactly tied logits; the lower index wins."""
    torch = torch_cuda
    from runnel_amd import native
    L = M.make_layer(310, hidden=1024, inter=64, experts=64, top_k=6, router_bits=8,
                     shared=False)
    q = L.router_w
    for a in (q.w, q.scales, q.biases):
        a[0, 1::2] = a[0, 0::2]
    x = M.make_x(311, 24, 1024)
    idx, _ = native.router(gate_to_dev(q), dev_bf16(x), 6)
    torch.cuda.synchronize()
    ref_idx, _, logits = M.route(x, q, 6)
    assert M.boundary_ties(logits, 6).any()
    assert np.array_equal(idx.cpu().numpy(), ref_idx)


@pytest.fixture(scope="module", params=[8, 4])
def qgate_layer(request, torch_cuda):
    """Full-size layer (hidden 2048, 256 experts, top-8 + shared, inter 512)
    with 8-bit gates; experts at 8 or 4 bits (a 4-bit checkpoint keeps its
    gates at 8 bits)."""
    from runnel_amd import synthetic
    bits = request.param
    lw = synthetic.make_layer(5200 + bits, bits=bits, gate_bits=8)
    return bits, lw, lw.handle(), layer_from_dev(lw)


def test_single_launch_decode_token_sequence(torch_cuda, qgate_layer):
    """Consecutive one-token calls through the single-launch decode."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    bits, lw, h, L = qgate_layer
    assert isinstance(L.router_w, M.QWeight) and isinstance(L.shared_gate_w, M.QWeight)
    ws = torch.zeros(h.workspace_bytes(1), dtype=torch.uint8, device="cuda")
    xs = synthetic.make_x(5210 + bits, 6, 2048)
    outs, idxs = [], []
    for t in range(6):
        o, i, _ = native.moe_block(h, xs[t:t + 1], return_routing=True, workspace=ws)
        outs.append(o)
        idxs.append(i)
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0
    xb = host_bf16(xs)
    _, ref_idx, _ = M.block_forward(L, xb)
    assert np.array_equal(np.concatenate([i.cpu().numpy() for i in idxs]), ref_idx)
    _check_outputs(np.concatenate([host_bf16(o) for o in outs]), L, xb)


def test_multi_token_decode(torch_cuda, qgate_layer):
    """A few tokens: the per-token router kernel, gate/up and down kernels."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    bits, lw, h, L = qgate_layer
    x = synthetic.make_x(5220 + bits, 5, 2048)
    out, idx, _ = native.moe_block(h, x, return_routing=True)
    torch.cuda.synchronize()
    xb = host_bf16(x)
    _, ref_idx, _ = M.block_forward(L, xb)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    _check_outputs(host_bf16(out), L, xb)


def test_prefill_matrix_core_router(torch_cuda, qgate_layer):
    """200 tokens: the split-plane matrix-core logits with the exact
    re-check select the same experts as the oracle; the sorted grouped GEMM
    is held to its prefill contract."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    bits, lw, h, L = qgate_layer
    x = synthetic.make_x(5230 + bits, 200, 2048)
    out, idx, scores = native.moe_block(h, x, return_routing=True)
    torch.cuda.synchronize()
    xb = host_bf16(x)
    sample = np.random.default_rng(bits).choice(200, 64, replace=False)
    ref_idx, ref_scores, _ = M.route(xb[sample], L.router_w, 8)
    assert np.array_equal(idx.cpu().numpy()[sample], ref_idx)
    assert np.abs(scores.cpu().numpy()[sample] - ref_scores).max() <= 2.0 ** -8
    few = sample[:12]
    _check_outputs(host_bf16(out)[few], L, xb[few], mode="prefill")


def test_prefill_router_ties_and_wide_tiles(torch_cuda):
    """4096 tokens take the 64-token logits tiles; tied gate rows must still
    resolve to the lower index."""
    torch = torch_cuda
    from runnel_amd import native
    L = M.make_layer(320, hidden=512, inter=128, experts=64, top_k=4, router_bits=8)
    q = L.router_w
    for a in (q.w, q.scales, q.biases):
        a[0, 1::2] = a[0, 0::2]
    x = M.make_x(321, 4096, 512)
    h = layer_to_dev(L)
    _, idx, _ = native.moe_block(h, dev_bf16(x), return_routing=True)
    torch.cuda.synchronize()
    sample = np.random.default_rng(3).choice(4096, 192, replace=False)
    ref_idx, _, logits = M.route(x[sample], q, 4)
    assert M.boundary_ties(logits, 4).any()
    assert np.array_equal(idx.cpu().numpy()[sample], ref_idx)


def test_chain_with_quantized_gates(torch_cuda):
    """Two chained layers with 8-bit gates equal per-layer single-launch
    calls exactly and match the sequential oracle."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lws = [synthetic.make_layer(5300 + l, bits=8, gate_bits=8) for l in range(2)]
    hs = [lw.handle() for lw in lws]
    chain = native.Chain(hs)
    x = synthetic.make_x(5310, 1, 2048)
    ws = torch.zeros(chain.workspace_bytes(), dtype=torch.uint8, device="cuda")
    y_chain = native.moe_chain(chain, x, workspace=ws)
    y = x
    for h in hs:
        y = native.moe_block(h, y, residual=y)
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0
    assert torch.equal(y_chain, y)
    cur = host_bf16(x)
    for lw in lws:
        L = layer_from_dev(lw)
        cur, _, _ = M.block_forward(L, cur, residual_bits=cur)
    g, r = M.bf16_to_f32(host_bf16(y_chain)), M.bf16_to_f32(cur)
    assert np.abs(g - r).max() <= MAX_ABS
    assert cosine(g, r) >= MIN_COS


def test_sparse_moe_block_module_with_quantized_gate(torch_cuda):
    """The module surface: SparseMoeBlock(gate_bits=8) after the packed
    gate/up transform runs the fused path and routes like the oracle."""
    torch = torch_cuda
    from runnel_amd import SparseMoeBlock, native
    from runnel_amd.moe import FusedQuantizedSwitchGLU
    L = M.make_layer(330, hidden=512, inter=128, experts=32, top_k=4, router_bits=8)
    blk = SparseMoeBlock(512, 128, 32, 4, shared_expert_intermediate_size=128, bits=8,
                         device="cuda", gate_bits=8)
    w, s, b = gate_to_dev(L.router_w)
    blk.gate.weight, blk.gate.scales, blk.gate.biases = w, s, b
    w, s, b = gate_to_dev(L.shared_gate_w)
    g = blk.shared_expert_gate
    g.weight, g.scales, g.biases = w, s, b
    from helpers import bank_to_dev
    gu = bank_to_dev(L.gate_up)
    dn = bank_to_dev(L.down)
    I = 128
    sm = blk.switch_mlp
    sm.up_proj.weight, sm.up_proj.scales, sm.up_proj.biases = (t[:, :I].contiguous() for t in gu)
    sm.gate_proj.weight, sm.gate_proj.scales, sm.gate_proj.biases = (
        t[:, I:].contiguous() for t in gu)
    sm.down_proj.weight, sm.down_proj.scales, sm.down_proj.biases = dn
    sgu = bank_to_dev(L.shared_gate_up, squeeze=True)
    sdn = bank_to_dev(L.shared_down, squeeze=True)
    se = blk.shared_expert
    se.up_proj.weight, se.up_proj.scales, se.up_proj.biases = (t[:I].contiguous() for t in sgu)
    se.gate_proj.weight, se.gate_proj.scales, se.gate_proj.biases = (
        t[I:].contiguous() for t in sgu)
    se.down_proj.weight, se.down_proj.scales, se.down_proj.biases = sdn
    blk.switch_mlp = FusedQuantizedSwitchGLU(blk.switch_mlp)
    assert blk.layer_handle() is not None
    x = M.make_x(331, 9, 512)
    out = blk(dev_bf16(x))
    torch.cuda.synchronize()
    _check_outputs(host_bf16(out), L, x)
    inds, _ = native.router((blk.gate.weight, blk.gate.scales, blk.gate.biases), dev_bf16(x), 4)
    torch.cuda.synchronize()
    assert np.array_equal(inds.cpu().numpy(), M.route(x, L.router_w, 4)[0])


def test_prefill_router_widest_rows(torch_cuda):
    """Hidden 4096 with an 8-bit gate, 160 tokens: both split planes
    through the matrix-core logits (two passes over K per wave, the second
    continuing the first's sums) and the 8-piece re-check select exactly the
    oracle's experts."""
    torch = torch_cuda
    from runnel_amd import native
    L = M.make_layer(340, hidden=4096, inter=128, experts=64, top_k=4, router_bits=8)
    x = M.make_x(341, 160, 4096)
    h = layer_to_dev(L)
    _, idx, scores = native.moe_block(h, dev_bf16(x), return_routing=True)
    torch.cuda.synchronize()
    ref_idx, ref_scores, _ = M.route(x, L.router_w, 4)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.abs(scores.cpu().numpy() - ref_scores).max() <= 2.0 ** -8
