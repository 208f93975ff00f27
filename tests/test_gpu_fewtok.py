"""GPU parity of the few-token decode kernels (2..8 tokens below the
expert-sorted threshold, hidden 2048, intermediate 512, 8- and 4-bit experts)
against the oracle: the router launch that also runs the shared expert's
gate/up, the gate/up kernel whose units share the rows of a repeated expert,
and the down kernel's bf16-pair dot products.

Bar: expert indices bit-exact; outputs within one bf16 step of the contract
oracle (a few elements may round the other way: accumulation order), and
within the end-to-end tolerance (max-abs 2e-2, cosine 0.9999) of the mlx-lm-style oracle."""

import numpy as np
import pytest

from helpers import cosine, dev_bf16, host_bf16, layer_to_dev
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


def _check(got_bits, ref_bits, mlx_bits):
    g = M.bf16_to_f32(got_bits).astype(np.float64)
    r = M.bf16_to_f32(ref_bits).astype(np.float64)
    tol = np.maximum(np.abs(r), 1e-3) * 2.0 ** -6 + 1e-6
    nbad = int((np.abs(g - r) > tol).sum())
    assert nbad <= max(1, g.size // 500), (nbad, float(np.abs(g - r).max()))
    m = M.bf16_to_f32(mlx_bits)
    assert np.abs(g - m).max() <= MAX_ABS
    assert cosine(g.astype(np.float32), m) >= MIN_COS


@pytest.mark.parametrize("case", [
    # 64 experts: 56 picks of 7 tokens repeat experts (shared rows)
    dict(T=7, experts=64, top_k=8, shared=True, residual=False),
    dict(T=2, experts=256, top_k=8, shared=True, residual=True),
    dict(T=4, experts=256, top_k=8, shared=True, residual=False),
    dict(T=5, experts=32, top_k=8, shared=True, residual=True),
    # no shared expert; 8 tokens of 4 slots
    dict(T=8, experts=32, top_k=4, shared=False, residual=False),
], ids=lambda c: f"T{c['T']}-E{c['experts']}-k{c['top_k']}"
                 f"{'-sh' if c['shared'] else ''}{'-res' if c['residual'] else ''}")
@pytest.mark.parametrize("bits", [8, 4])
def test_few_token_block(torch_cuda, case, bits):
    torch = torch_cuda
    from runnel_amd import native
    print(f"few-token block bits={bits} {case}", flush=True)
    L = M.make_layer(300 + case["T"] + case["experts"] + bits, hidden=2048, inter=512,
                     experts=case["experts"], top_k=case["top_k"], bits=bits,
                     shared=case["shared"])
    x = M.make_x(40 + case["T"], case["T"], 2048)
    res = M.make_x(90 + case["T"], case["T"], 2048) if case["residual"] else None
    h = layer_to_dev(L)
    kw = dict(residual=dev_bf16(res)) if res is not None else {}
    out, idx, _ = native.moe_block(h, dev_bf16(x), return_routing=True, **kw)
    torch.cuda.synchronize()
    ref, ref_idx, _ = M.block_forward(L, x, residual_bits=res)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    mlx, _, _ = M.block_forward(L, x, residual_bits=res, mode="mlx")
    _check(host_bf16(out), ref, mlx)
    if case["experts"] == 64:
        # the case exercises experts chosen by several tokens
        flat = ref_idx.ravel()
        assert len(np.unique(flat)) < flat.size


@pytest.mark.parametrize("bits", [8, 4])
def test_few_token_calls_repeat_bit_exact(torch_cuda, bits):
    """The same call twice gives the same bits (no state carried between
    calls in the workspace), and a 1-token call in between does not disturb
    it."""
    torch = torch_cuda
    from runnel_amd import native
    L = M.make_layer(77 + bits, hidden=2048, inter=512, experts=64, top_k=8, bits=bits)
    h = layer_to_dev(L)
    x4 = dev_bf16(M.make_x(3, 4, 2048))
    x1 = dev_bf16(M.make_x(4, 1, 2048))
    ws = torch.zeros(h.workspace_bytes(4), dtype=torch.uint8, device="cuda")
    a = native.moe_block(h, x4, workspace=ws).clone()
    native.moe_block(h, x1, workspace=ws)
    b = native.moe_block(h, x4, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("bits", [8, 4])
def test_few_token_graph_replays_equal_eager_calls(torch_cuda, bits):
    """Few-token calls captured in a HIP graph: every replay (the router's
    tags come from the workspace's epoch, which each call advances on the
    device) equals the eager calls bit for bit, with eager calls and
    synchronisations between the replays."""
    torch = torch_cuda
    from runnel_amd import native, synthetic
    lw = synthetic.make_layer(7100 + bits, bits=bits)
    h = lw.handle()
    xa = synthetic.make_x(7101, 4, 2048)
    xb = synthetic.make_x(7102, 3, 2048)
    ws = torch.zeros(h.workspace_bytes(4), dtype=torch.uint8, device="cuda")
    ref_a = native.moe_block(h, xa, workspace=ws, check=False).clone()
    ref_b = native.moe_block(h, xb, workspace=ws, check=False).clone()
    oa, ob = torch.empty_like(xa), torch.empty_like(xb)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        native.moe_block(h, xa, out=oa, workspace=ws, check=False)
        native.moe_block(h, xb, out=ob, workspace=ws, check=False)
    for r in range(3):
        oa.zero_()
        ob.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(oa, ref_a), f"replay {r}"
        assert torch.equal(ob, ref_b), f"replay {r}"
        eager = native.moe_block(h, xa, workspace=ws, check=False)
        torch.cuda.synchronize()
        assert torch.equal(eager, ref_a)
    assert native.workspace_status(ws) == 0
