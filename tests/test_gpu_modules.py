"""The reference's Python surfaces on device-resident modules: a two-layer
model of mlx-lm-shaped modules (SparseMoeBlock with a stock SwitchGLU, the
shared MLP and gates), run before and after fuse_routed_gate_up
(src/runnel/mlx.py:84-95, called from src/runnel/cli.py:47-49), and the
packed module's own call (src/runnel/mlx.py:57-82), against the oracle."""

from types import SimpleNamespace

import numpy as np
import pytest

from helpers import bank_to_dev, cosine, dev_bf16, host_bf16
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


def _fill(mod, w, s, b):
    mod.weight.copy_(w)
    mod.scales.copy_(s)
    mod.biases.copy_(b)


def _block_from_oracle(L, bits):
    """An unfused SparseMoeBlock on the GPU holding the oracle layer's
    tensors: the stock SwitchGLU with separate gate / up banks."""
    from runnel_amd import SparseMoeBlock
    H, I, E = L.hidden, L.inter, L.experts
    blk = SparseMoeBlock(H, I, E, L.top_k, shared_expert_intermediate_size=I, bits=bits,
                         device="cuda")
    blk.gate.weight.copy_(dev_bf16(L.router_w))
    w, s, b = bank_to_dev(L.gate_up)
    sm = blk.switch_mlp
    _fill(sm.up_proj, w[:, :I], s[:, :I], b[:, :I])
    _fill(sm.gate_proj, w[:, I:], s[:, I:], b[:, I:])
    _fill(sm.down_proj, *bank_to_dev(L.down))
    w, s, b = bank_to_dev(L.shared_gate_up, squeeze=True)
    se = blk.shared_expert
    _fill(se.up_proj, w[:I], s[:I], b[:I])
    _fill(se.gate_proj, w[I:], s[I:], b[I:])
    _fill(se.down_proj, *bank_to_dev(L.shared_down, squeeze=True))
    blk.shared_expert_gate.weight.copy_(dev_bf16(L.shared_gate_w[None, :]))
    return blk


def _contract_mismatches(got_bits, ref_bits):
    g = M.bf16_to_f32(got_bits).astype(np.float64)
    r = M.bf16_to_f32(ref_bits).astype(np.float64)
    tol = np.maximum(np.abs(r), 1e-3) * 2.0 ** -6 + 1e-6
    return int((np.abs(g - r) > tol).sum())


def _maxabs_cosine(got_bits, ref_bits):
    g, r = M.bf16_to_f32(got_bits), M.bf16_to_f32(ref_bits)
    return float(np.abs(g - r).max()), cosine(g, r)


@pytest.mark.parametrize("bits", [8, 4])
def test_installer_on_a_device_model(torch_cuda, bits):
    """Two layers of device modules: the composed (unfused) block and the
    installed packed block both match the oracle; the installer returns the
    layer count and leaves packed [up; gate] banks."""
    torch = torch_cuda
    from runnel_amd import FusedQuantizedSwitchGLU, fuse_routed_gate_up
    Ls = [M.make_layer(9100 + 10 * bits + i, hidden=512, inter=128, experts=32, top_k=4,
                       bits=bits) for i in range(2)]
    model = SimpleNamespace(language_model=SimpleNamespace(
        layers=[SimpleNamespace(mlp=_block_from_oracle(L, bits)) for L in Ls]))
    xs = {T: M.make_x(9101 + T, T, 512) for T in (3, 40)}
    before = {}
    for i, L in enumerate(Ls):
        for T, x in xs.items():
            # mlx-lm hands the block [B, L, D]
            before[i, T] = host_bf16(model.language_model.layers[i].mlp(
                dev_bf16(x).reshape(1, T, 512)).reshape(T, 512))
    assert fuse_routed_gate_up(model) == 2
    for i, L in enumerate(Ls):
        blk = model.language_model.layers[i].mlp
        sm = blk.switch_mlp
        assert isinstance(sm, FusedQuantizedSwitchGLU) and sm.bits == bits
        assert np.array_equal(sm.weight.cpu().numpy().view(np.uint32), L.gate_up.w)
        assert blk.layer_handle() is not None
        for T, x in xs.items():
            got = host_bf16(blk(dev_bf16(x).reshape(1, T, 512)).reshape(T, 512))
            mode = "prefill" if T * L.top_k >= 64 else "contract"
            ref, _, _ = M.block_forward(L, x, mode=mode)
            assert _contract_mismatches(got, ref) <= got.size // 500, (i, T)
            mlx, _, _ = M.block_forward(L, x, mode="mlx")
            for out in (got, before[i, T]):
                err, cos = _maxabs_cosine(out, mlx)
                assert err <= MAX_ABS and cos >= MIN_COS, (i, T, err, cos)
        blk.check_status()
    torch.cuda.synchronize()


@pytest.mark.parametrize("bits", [8, 4])
def test_packed_module_call_per_slot(torch_cuda, bits):
    """FusedQuantizedSwitchGLU(x, indices) -> [..., k, D], uncombined, for a
    decode-sized and a sorted (>= 64 rows) call, against the oracle's
    per-slot outputs."""
    torch = torch_cuda
    from runnel_amd import fuse_routed_gate_up
    L = M.make_layer(9200 + bits, hidden=512, inter=128, experts=32, top_k=4, bits=bits)
    model = SimpleNamespace(language_model=SimpleNamespace(
        layers=[SimpleNamespace(mlp=_block_from_oracle(L, bits))]))
    assert fuse_routed_gate_up(model) == 1
    sm = model.language_model.layers[0].mlp.switch_mlp
    for T in (2, 48):
        x = M.make_x(9201 + T, T, 512)
        idx, _, _ = M.route(x, L.router_w, L.top_k)
        y = sm(dev_bf16(x).reshape(1, T, 512), torch.from_numpy(idx).cuda().reshape(1, T, 4))
        assert tuple(y.shape) == (1, T, 4, 512)
        got = host_bf16(y.reshape(T * 4, 512))
        mode = "prefill" if T * 4 >= 64 else "contract"
        ref = M.f32_to_bf16(M.switch_glu(L, x, idx, mode).reshape(T * 4, 512))
        assert _contract_mismatches(got, ref) <= got.size // 500, T
