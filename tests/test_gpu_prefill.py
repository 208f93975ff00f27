"""GPU parity of the expert-sorted grouped GEMM (calls that route at least 64
(token, slot) rows) against the oracle's prefill contract: every dequantised
weight rounded to bf16, then the decode contract's rounding points.  Outputs
are held to a bf16 rounding step of that contract (a few mismatches allowed
for accumulation order) and to the end-to-end tolerance (max-abs 2e-2, cosine 0.9999) of the mlx-lm-style
evaluation; routing is bit-exact."""

import numpy as np
import pytest

from helpers import (bank_to_dev, cosine, dev_bf16, dev_i32, host_bf16, layer_from_dev,
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


def _mismatches(got, ref):
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    tol = np.maximum(np.abs(r), 1e-3) * 2.0 ** -6 + 1e-6
    return int((np.abs(g - r) > tol).sum())


def _switch(torch, L, x, idx):
    from runnel_amd import native
    keep = (bank_to_dev(L.gate_up), bank_to_dev(L.down))
    gu = native.qweight_struct(*keep[0], L.gate_up.bits)
    dn = native.qweight_struct(*keep[1], L.down.bits)
    y = native.switch_glu(dev_bf16(x), dev_i32(idx), gu, dn)
    torch.cuda.synchronize()
    return M.bf16_to_f32(host_bf16(y))


@pytest.mark.parametrize("bits", [8, 4])
def test_switch_glu_sorted_matches_prefill_contract(torch_cuda, bits):
    L = M.make_layer(31 + bits, hidden=512, inter=256, experts=16, top_k=4, bits=bits,
                     shared=False)
    x = M.make_x(7, 40, 512)
    idx = np.random.default_rng(bits).integers(0, 16, size=(40, 4)).astype(np.int32)
    got = _switch(torch_cuda, L, x, idx)
    ref = M.switch_glu(L, x, idx, mode="prefill")
    assert _mismatches(got, ref) <= got.size // 500
    exact = M.switch_glu(L, x, idx, mode="mlx")
    assert np.abs(got - exact).max() <= MAX_ABS
    assert cosine(got.reshape(-1), exact.reshape(-1)) >= MIN_COS


def test_switch_glu_sorted_skewed_and_bad_ids(torch_cuda):
    """One expert receives 300 rows (three m-tiles, the last partial), most
    receive none, and out-of-range ids give zero rows, as the decode path
    does."""
    L = M.make_layer(5, hidden=256, inter=128, experts=24, top_k=3, bits=8, shared=False)
    T = 300
    rng = np.random.default_rng(1)
    idx = np.stack([np.full(T, 3), rng.integers(0, 4, T), rng.integers(10, 12, T)],
                   1).astype(np.int32)
    idx[5, 1] = -1
    idx[17, 2] = 24
    idx[299, 0] = 1 << 20
    x = M.make_x(8, T, 256)
    got = _switch(torch_cuda, L, x, idx)
    bad = (idx < 0) | (idx >= 24)
    assert np.all(got[bad] == 0.0)
    fixed = np.where(bad, 0, idx)
    ref = M.switch_glu(L, x, fixed, mode="prefill")
    ref[bad] = 0.0
    assert _mismatches(got, ref) <= got.size // 500


@pytest.mark.parametrize("bits", [8, 4])
def test_block_sorted_small(torch_cuda, bits):
    import torch
    from runnel_amd import native
    L = M.make_layer(60 + bits, hidden=512, inter=128, experts=32, top_k=4, bits=bits)
    x = M.make_x(9, 48, 512)
    h = layer_to_dev(L)
    out, idx, scores = native.moe_block(h, dev_bf16(x), residual=dev_bf16(x),
                                        return_routing=True)
    torch.cuda.synchronize()
    ref, ref_idx, ref_scores = M.block_forward(L, x, residual_bits=x, mode="prefill")
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.abs(scores.cpu().numpy() - ref_scores).max() <= 2.0 ** -8
    got = M.bf16_to_f32(host_bf16(out))
    r = M.bf16_to_f32(ref)
    assert _mismatches(got, r) <= got.size // 500
    mlx, _, _ = M.block_forward(L, x, residual_bits=x, mode="mlx")
    mx_ = M.bf16_to_f32(mlx)
    assert np.abs(got - mx_).max() <= MAX_ABS
    assert cosine(got.reshape(-1), mx_.reshape(-1)) >= MIN_COS


def test_block_prefill_512_tokens_8bit(torch_cuda):
    """The prefill chunk workload: 512 tokens through one full-size 8-bit
    layer (hidden 2048, 256 experts, top-8 + shared, inter 512)."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lw = synthetic.make_layer(4242, bits=8)
    h = lw.handle()
    x = synthetic.make_x(11, 512, 2048)
    out, idx, scores = native.moe_block(h, x, return_routing=True)
    torch.cuda.synchronize()
    L = layer_from_dev(lw)
    xb = host_bf16(x)
    ref, ref_idx, _ = M.block_forward(L, xb, mode="prefill")
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    got = M.bf16_to_f32(host_bf16(out))
    assert _mismatches(got, M.bf16_to_f32(ref)) <= got.size // 500
    mlx, _, _ = M.block_forward(L, xb, mode="mlx")
    mx_ = M.bf16_to_f32(mlx)
    assert np.abs(got - mx_).max() <= MAX_ABS
    assert cosine(got.reshape(-1), mx_.reshape(-1)) >= MIN_COS


@pytest.mark.parametrize("bits", [8, 4])
def test_prefill_512_tokens_deterministic(torch_cuda, bits):
    """The 512-token chunk through a full-size layer: two calls give the same
    bits (no result depends on which workgroup finishes first), and the
    4-bit layer meets the contract like the 8-bit one above."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lw = synthetic.make_layer(5150 + bits, bits=bits)
    h = lw.handle()
    x = synthetic.make_x(13, 512, 2048)
    out1 = native.moe_block(h, x)
    out2 = native.moe_block(h, x)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    if bits == 4:
        out, idx, _ = native.moe_block(h, x, return_routing=True)
        torch.cuda.synchronize()
        assert torch.equal(out, out1)
        L = layer_from_dev(lw)
        xb = host_bf16(x)
        ref, ref_idx, _ = M.block_forward(L, xb, mode="prefill")
        assert np.array_equal(idx.cpu().numpy(), ref_idx)
        got = M.bf16_to_f32(host_bf16(out))
        assert _mismatches(got, M.bf16_to_f32(ref)) <= got.size // 500
        mlx, _, _ = M.block_forward(L, xb, mode="mlx")
        mx_ = M.bf16_to_f32(mlx)
        assert np.abs(got - mx_).max() <= MAX_ABS
        assert cosine(got.reshape(-1), mx_.reshape(-1)) >= MIN_COS


def test_long_prefill_combine_bit_exact(torch_cuda):
    """2048 tokens through a full-size layer (128-row tiles; the combine
    requests all of a token's rows at once): the output equals, bit for bit,
    the combine restated on the host (fp32 fma over the slots in order, bf16
    rounding, then the residual) from the same routing's per-slot rows (the
    uncombined call); a second call with other inputs on the same workspace
    as well, so no row of an earlier call is read in place of the current
    one."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lw = synthetic.make_layer(5160, bits=8)
    gu = native.qweight_struct(*lw.gate_up, 8)
    dn = native.qweight_struct(*lw.down, 8)
    T, K, H, E = 2048, 8, 2048, 256
    g = torch.Generator(device="cuda")
    g.manual_seed(5161)
    for rep in range(2):
        x = synthetic.make_x(5162 + rep, T, H)
        res = synthetic.make_x(5170 + rep, T, H)
        idx = torch.rand(T, E, generator=g, device="cuda").argsort(dim=1)[:, :K].contiguous()
        w = torch.rand(T, K, generator=g, device="cuda")
        out = native.switch_combine(x, idx, w, gu, dn, residual=res)
        y = native.switch_glu(x, idx, gu, dn)
        torch.cuda.synchronize()
        yf = M.bf16_to_f32(host_bf16(y))
        wf = w.cpu().numpy()
        acc = np.zeros((T, H), np.float32)
        for j in range(K):
            acc = M.fma32(wf[:, j:j + 1], yf[:, j, :], acc)
        ref = M.round_bf16(M.bf16_to_f32(host_bf16(res)) + M.round_bf16(acc))
        got = M.bf16_to_f32(host_bf16(out))
        assert np.array_equal(got, ref), f"call {rep}: {int((got != ref).sum())} values differ"


@pytest.mark.parametrize("shape", [dict(hidden=1024, experts=128, top_k=8),
                                   dict(hidden=512, experts=64, top_k=6),
                                   # the widest eligible rows: two passes of
                                   # four chunks per wave over K, x held in
                                   # eight pieces per lane by the re-check
                                   dict(hidden=4096, experts=64, top_k=4)])
def test_matrix_core_router_selection_is_exact(torch_cuda, shape):
    """Many tokens route through the MFMA logits + exact re-check path:
    indices equal the oracle's bit for bit, scores within a bf16 step."""
    import torch
    from runnel_amd import native
    L = M.make_layer(77, inter=128, bits=8, **shape)
    x = M.make_x(78, 200, shape["hidden"])
    h = layer_to_dev(L)
    out, idx, scores = native.moe_block(h, dev_bf16(x), return_routing=True)
    torch.cuda.synchronize()
    ref_idx, ref_scores, _ = M.route(x, L.router_w, L.top_k)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.abs(scores.cpu().numpy() - ref_scores).max() <= 2.0 ** -8
    ref, _, _ = M.block_forward(L, x, mode="prefill")
    got = M.bf16_to_f32(host_bf16(out))
    assert _mismatches(got, M.bf16_to_f32(ref)) <= got.size // 500


def test_matrix_core_router_ties_break_by_index(torch_cuda):
    """Pairs of identical router rows give exactly tied logits; the lower
    expert index must win each tie, as in the oracle."""
    import torch
    from runnel_amd import native
    L = M.make_layer(79, hidden=512, inter=128, experts=64, top_k=5, bits=8)
    L.router_w[1::2] = L.router_w[0::2]
    x = M.make_x(80, 96, 512)
    h = layer_to_dev(L)
    _, idx, _ = native.moe_block(h, dev_bf16(x), return_routing=True)
    torch.cuda.synchronize()
    ref_idx, _, logits = M.route(x, L.router_w, L.top_k)
    assert M.boundary_ties(logits, L.top_k).any()
    assert np.array_equal(idx.cpu().numpy(), ref_idx)


def test_long_prefill_skewed_routing_4bit(torch_cuda):
    """The long prefill workload: 8192 tokens, full-size 4-bit layer, router
    biased by a Zipf(1.1) ranking (some experts over 1000 rows, many under
    8).  Routing is checked bit-exact on 256 sampled tokens and outputs on 48
    (a token's routing and output depend on that token only)."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lw = synthetic.make_layer(5150, bits=4)
    synthetic.apply_router_bias(lw, synthetic.zipf_bias(5150, 256))
    x = synthetic.make_skewed_x(5151, 8192, 2048)
    h = lw.handle()
    out, idx, _ = native.moe_block(h, x, return_routing=True)
    torch.cuda.synchronize()
    counts = np.bincount(idx.cpu().numpy().reshape(-1), minlength=256)
    assert counts.max() > 1000 and (counts < 8).sum() > 64
    L = layer_from_dev(lw)
    xb = host_bf16(x)
    sample = np.random.default_rng(0).choice(8192, 256, replace=False)
    ref_idx, _, _ = M.route(xb[sample], L.router_w, 8)
    assert np.array_equal(idx.cpu().numpy()[sample], ref_idx)
    few = sample[:48]
    ref, _, _ = M.block_forward(L, xb[few], mode="prefill")
    got = M.bf16_to_f32(host_bf16(out))[few]
    assert _mismatches(got, M.bf16_to_f32(ref)) <= got.size // 500
    mlx, _, _ = M.block_forward(L, xb[few], mode="mlx")
    mx_ = M.bf16_to_f32(mlx)
    assert np.abs(got - mx_).max() <= MAX_ABS
    assert cosine(got.reshape(-1), mx_.reshape(-1)) >= MIN_COS
