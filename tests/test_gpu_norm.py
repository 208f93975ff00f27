"""GPU parity of the decoder layer's post-attention RMSNorm in front of the
block: rmoe_rms_norm bit for bit against the oracle's fixed order; the
block with the norm (single-launch decode, the decode kernels, the
expert-sorted path) routing like the oracle on the normalised input with the
residual taken before the norm; the chained single-launch decode with a norm
per layer, eager and replayed from HIP graphs."""

import numpy as np
import pytest

from helpers import cosine, dev_bf16, host_bf16, layer_from_dev, layer_to_dev
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


def _scaled_x(seed, T, H, scale=4.0):
    rng = np.random.default_rng(seed)
    return M.f32_to_bf16((rng.standard_normal((T, H)) * scale).astype(np.float32))


@pytest.mark.parametrize("T,H,eps", [(7, 2048, 1e-6), (3, 320, 1e-2), (130, 512, 0.0)])
def test_rms_norm_bit_exact(torch_cuda, T, H, eps):
    torch = torch_cuda
    from runnel_amd import native
    x = _scaled_x(T + H, T, H)
    w = M.f32_to_bf16(np.random.default_rng(H).uniform(0.3, 1.7, H).astype(np.float32))
    y = native.rms_norm(dev_bf16(x), dev_bf16(w), eps)
    torch.cuda.synchronize()
    assert np.array_equal(host_bf16(y), M.rms_norm(x, w, eps))


@pytest.mark.parametrize("bits", [8, 4])
def test_block_with_post_norm(torch_cuda, bits):
    """h' = h + MoE(RMSNorm(h)) for 1 token (single launch), 5 tokens and
    40 tokens (expert-sorted): routing equals the oracle's on the normalised
    input; outputs within the contract and the end-to-end tolerance (max-abs 2e-2, cosine 0.9999)."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lw = synthetic.make_layer(6100 + bits, bits=bits, post_norm=True)
    h = lw.handle()
    L = layer_from_dev(lw)
    for T, mode in ((1, "contract"), (5, "contract"), (40, "prefill")):
        xb = _scaled_x(6200 + T, T, 2048)
        x = dev_bf16(xb)
        out, idx, _ = native.moe_block(h, x, residual=x, return_routing=True)
        bare = native.moe_block(h, x)
        torch.cuda.synchronize()
        ref, ref_idx, _ = M.block_forward(L, xb, residual_bits=xb, mode=mode)
        assert np.array_equal(idx.cpu().numpy(), ref_idx), (T, mode)
        got = host_bf16(out)
        assert _mismatches(got, ref) <= max(2, got.size // 200), (T, mode)
        # the tolerance is on the block's own output (the residual stream at
        # |h| ~ 16 has bf16 steps of 0.0625)
        got = host_bf16(bare)
        ref, _, _ = M.block_forward(L, xb, mode=mode)
        assert _mismatches(got, ref) <= max(2, got.size // 200), (T, mode)
        mlx, _, _ = M.block_forward(L, xb, mode="mlx")
        g, m = M.bf16_to_f32(got), M.bf16_to_f32(mlx)
        assert np.abs(g - m).max() <= MAX_ABS
        assert cosine(g, m) >= MIN_COS


def test_post_norm_small_layer_and_module(torch_cuda, tmp_path):
    """A small layer (not the single-launch shape) with its norm, loaded from
    a checkpoint as PostAttentionMoE: the RMSNorm kernel, then the decode
    kernels, the residual taken before the norm; the module and a direct
    rmoe_moe_block call agree exactly."""
    torch = torch_cuda
    import json
    from runnel_amd import checkpoint as C
    from runnel_amd import native
    from test_checkpoint import write_checkpoint
    L = M.make_layer(6300, hidden=512, inter=128, experts=32, top_k=4, bits=8)
    L.post_norm_w = M.f32_to_bf16(np.random.default_rng(1).uniform(0.5, 1.5, 512)
                                  .astype(np.float32))
    L.norm_eps = 1e-5
    write_checkpoint(tmp_path, L, extra={
        "language_model.model.layers.0.post_attention_layernorm.weight": ("BF16", L.post_norm_w)})
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg["text_config"]["rms_norm_eps"] = 1e-5
    step = C.load_decoder_moe(tmp_path, 0, config=cfg)
    xb = _scaled_x(6301, 6, 512)
    out = step(dev_bf16(xb))
    direct = native.moe_block(layer_to_dev(L), dev_bf16(xb), residual=dev_bf16(xb))
    torch.cuda.synchronize()
    assert torch.equal(out, direct)
    ref, _, _ = M.block_forward(L, xb, residual_bits=xb)
    assert _mismatches(host_bf16(out), ref) <= max(2, out.numel() // 200)


def test_chain_with_post_norm_matches_oracle_and_single_calls(torch_cuda):
    """Three layers with a norm each in one launch: equal to per-layer
    single-launch calls bit for bit, and to the sequential oracle within the
    chained tolerance."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lws = [synthetic.make_layer(6400 + l, bits=8, post_norm=True) for l in range(3)]
    hs = [lw.handle() for lw in lws]
    chain = native.Chain(hs)
    xb = _scaled_x(6410, 1, 2048, scale=1.0)
    x = dev_bf16(xb)
    ws = torch.zeros(chain.workspace_bytes(), dtype=torch.uint8, device="cuda")
    y_chain = native.moe_chain(chain, x, workspace=ws)
    y = x
    for hh in hs:
        y = native.moe_block(hh, y, residual=y)
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0
    assert torch.equal(y_chain, y)
    cur = xb
    for lw in lws:
        L = layer_from_dev(lw)
        cur, _, _ = M.block_forward(L, cur, residual_bits=cur)
    g, r = M.bf16_to_f32(host_bf16(y_chain)), M.bf16_to_f32(cur)
    assert np.abs(g - r).max() <= MAX_ABS
    assert cosine(g, r) >= MIN_COS


def test_normed_chain_graph_replays_equal_eager(torch_cuda):
    """The normed chain captured in a HIP graph and replayed with new inputs,
    eager calls on the same workspace in between: every replay equals the
    eager result."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lws = [synthetic.make_layer(6500 + l, bits=4, post_norm=True, gate_bits=8)
           for l in range(2)]
    chain = native.Chain([lw.handle() for lw in lws])
    ws = torch.zeros(chain.workspace_bytes(), dtype=torch.uint8, device="cuda")
    xin = torch.empty((1, 2048), dtype=torch.bfloat16, device="cuda")
    yout = torch.empty_like(xin)
    xin.copy_(dev_bf16(_scaled_x(6510, 1, 2048)))
    native.moe_chain(chain, xin, out=yout, workspace=ws)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        native.moe_chain(chain, xin, out=yout, workspace=ws)
    for k in range(3):
        xin.copy_(dev_bf16(_scaled_x(6520 + k, 1, 2048)))
        eager = native.moe_chain(chain, xin, workspace=ws).clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yout, eager), k
    assert native.workspace_status(ws) == 0
