"""The benchmarked decode workload at full depth: the 40-layer 8-bit stack
(hidden 2048, 256 experts, top-8 + shared, inter 512; the same seeds and
first input as bench.py) chained through all 40 layers in one launch, and
every layer checked against the oracle, as the reference checks each of the
40 layers of its real-tensor sweep (bench/run_native_ornith_layers.py:41-111).

The chained kernel's output after l layers comes from a chain of the first
l layers (the same kernel and arithmetic), so each layer's input and output
are known; the oracle copies one layer to the host at a time."""

import numpy as np
import pytest

from helpers import cosine, host_bf16, layer_from_dev
from oracle import moe_ref as M

pytestmark = pytest.mark.gpu

N_LAYERS = 40


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runnel_amd import _lib
    _lib.load()
    return torch


def _contract_mismatches(got_bits, ref_bits):
    g = M.bf16_to_f32(got_bits).astype(np.float64)
    r = M.bf16_to_f32(ref_bits).astype(np.float64)
    tol = np.maximum(np.abs(r), 1e-3) * 2.0 ** -6 + 1e-6
    return int((np.abs(g - r) > tol).sum())


def test_forty_layer_chain_matches_the_oracle_at_every_layer(torch_cuda):
    torch = torch_cuda
    import bench
    from runnel_amd import native, synthetic
    print("building the 40-layer 8-bit stack", flush=True)
    stack = bench.build_stack(N_LAYERS, 8)
    hs = [lw.handle() for lw in stack]
    x = synthetic.make_x(12345, 1, 2048)
    ws = torch.zeros(hs[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")
    ys = [x]
    for n in range(1, N_LAYERS + 1):
        ys.append(native.moe_chain(native.Chain(hs[:n]), x, workspace=ws, check=False))
    full = native.moe_chain(native.Chain(hs), x, workspace=ws, check=False)
    torch.cuda.synchronize()
    assert native.workspace_status(ws) == 0
    assert torch.equal(full, ys[N_LAYERS])
    print("chain done; checking every layer", flush=True)
    # The oracle also runs the chain on its own inputs.  Routing is
    # discontinuous: once rounding differences move a later layer's k-th and
    # (k+1)-th logits past each other the two chains use different experts,
    # so they are compared end to end only up to that layer; every layer is
    # held to the tight bar on the GPU's own input regardless.
    cur_ref = host_bf16(x)
    split_at = None
    for l in range(N_LAYERS):
        L = layer_from_dev(stack[l])
        xin = host_bf16(ys[l])
        ref, ref_idx, _ = M.block_forward(L, xin, residual_bits=xin)
        one, idx, _ = native.moe_block(hs[l], ys[l], residual=ys[l], return_routing=True,
                                       workspace=ws, check=False)
        torch.cuda.synchronize()
        # the single-layer call of the same kernel agrees with the chain
        assert torch.equal(one, ys[l + 1]), f"layer {l}"
        assert np.array_equal(idx.cpu().numpy(), ref_idx), f"layer {l}"
        got = host_bf16(ys[l + 1])
        assert _contract_mismatches(got, ref) <= 4, f"layer {l}"
        if split_at is None:
            nxt, own_idx, _ = M.block_forward(L, cur_ref, residual_bits=cur_ref)
            if not np.array_equal(np.sort(own_idx, -1), np.sort(ref_idx, -1)):
                split_at = l
                lg = M.round_bf16(M.gate_logits(cur_ref, L.router_w))[0]
                srt = np.sort(lg)[::-1]
                print(f"the oracle's own chain routes differently from layer {l} on "
                      f"(its 8th / 9th logits {srt[7]:.5f} / {srt[8]:.5f})", flush=True)
                assert l > 0   # the first layer sees the same input
            else:
                cur_ref = nxt
                # rounding differences compound through the residual stream
                # (which grows to several units, where one bf16 step exceeds
                # 2e-2): the two chains are held to norm-wise bounds
                g = M.bf16_to_f32(got).astype(np.float64)
                r = M.bf16_to_f32(cur_ref).astype(np.float64)
                assert np.linalg.norm(g - r) <= 1e-2 * np.linalg.norm(r), f"layer {l}"
                assert cosine(g, r) >= 0.9999, f"layer {l}"
        del L
        if l % 10 == 9:
            print(f"layers 0..{l} ok", flush=True)
    print(f"end-to-end agreement over {split_at if split_at is not None else N_LAYERS} "
          "layers", flush=True)
