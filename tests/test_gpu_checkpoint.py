"""GPU runs of ingested tensors: the reference's probe datasets read from
their file formats (RNLMOE01 through rmoe_switch_combine, RNLQMV02 through
rmoe_gather_qmm) reproduce the checksums the reference recorded; a layer
loaded from a safetensors checkpoint runs the block to the oracle's
contract; rmoe_switch_combine (caller routing and weights) matches the
oracle on the decode and the expert-sorted paths."""

import json
from pathlib import Path

import numpy as np
import pytest

from helpers import bank_to_dev, cosine, dev_bf16, dev_i32, host_bf16
from oracle import moe_ref as M
from test_checkpoint import write_checkpoint

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
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


@pytest.mark.parametrize("case", [c for c in GOLDEN["fused"] if c["schedule"] == "two-stage"],
                         ids=lambda c: Path(c["source"]).stem)
def test_rnlmoe01_file_reproduces_reference_checksum(torch_cuda, case, tmp_path):
    """The reference fused probe's dataset written as RNLMOE01, read back
    and run: the combined output matches the recorded CPU-oracle checksum
    (kernel rounds x_up, x_gate, act and y to bf16, hence the tolerance)."""
    torch = torch_cuda
    from runnel_amd import checkpoint as C
    bits = case["bits"]
    o = M.fused_dataset(bits, case["total_experts"])
    E = case["total_experts"]
    vpw = 32 // bits
    ds = C.MoeDataset(bits, np.asarray(case["selected"], np.uint32),
                      (o["gate_up"].w.reshape(E, 1024, 2048 // vpw),
                       o["gate_up"].scales.reshape(E, 1024, 32),
                       o["gate_up"].biases.reshape(E, 1024, 32)),
                      (o["down"].w.reshape(E, 2048, 512 // vpw),
                       o["down"].scales.reshape(E, 2048, 8),
                       o["down"].biases.reshape(E, 2048, 8)), o["x"], o["router"])
    p = tmp_path / "layer.bin"
    C.write_rnlmoe01(p, ds)
    out = C.run_rnlmoe01(C.read_rnlmoe01(p))
    torch.cuda.synchronize()
    got = M.bf16_to_f32(host_bf16(out)).astype(np.float64)
    expected, _ = M.fused_reference(bits, o, case["selected"])
    assert np.abs(got - expected).max() <= MAX_ABS
    assert cosine(got, expected) >= 0.999
    assert abs(got.sum() - case["reference_checksum"]) <= 0.05 * max(1.0, abs(case["reference_checksum"]))


@pytest.mark.parametrize("case", [c for c in GOLDEN["qmv"] if c["output_size"] <= 16384],
                         ids=lambda c: Path(c["source"]).stem)
def test_rnlqmv02_file_reproduces_reference_checksum(torch_cuda, case, tmp_path):
    torch = torch_cuda
    from runnel_amd import checkpoint as C
    bits = case["bits"]
    o = M.qmv_dataset(bits, case["output_size"], case["reduction_size"], case["group"],
                      case["bank_rows"], case["rows_per_expert"], case["selected"])
    rpe = case["rows_per_expert"] or case["output_size"]
    ds = C.QmvDataset(bits, case["output_size"], rpe, case["group"], o["w"], o["scales"],
                      o["biases"], o["x"], o["selected"])
    p = tmp_path / "qmv.bin"
    C.write_rnlqmv02(p, ds)
    y = C.run_rnlqmv02(C.read_rnlqmv02(p))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    np.testing.assert_allclose(got, o["expected"], rtol=2e-4, atol=2e-5)
    assert abs(got.astype(np.float64).sum() - case["reference_checksum"]) <= 2e-3
    np.testing.assert_allclose(got[:8], case["first_reference"], atol=1.5e-3)


@pytest.mark.parametrize("router_bits", [None, 8])
@pytest.mark.parametrize("bits", [8, 4])
def test_block_loaded_from_checkpoint(torch_cuda, tmp_path, bits, router_bits):
    """A layer read from a safetensors checkpoint: one token (single-launch
    decode), a few tokens, and a prefill-sized call all route like the
    oracle and land within its contract and the end-to-end tolerance (max-abs 2e-2, cosine 0.9999)."""
    torch = torch_cuda
    from runnel_amd import checkpoint as C
    L = M.make_layer(40 + bits, hidden=512, inter=128, experts=32, top_k=4, bits=bits,
                     router_bits=router_bits)
    write_checkpoint(tmp_path, L, layer=3, bits=bits)
    blk = C.load_moe_block(tmp_path, 3)
    assert blk.layer_handle() is not None
    for T, mode in ((1, "contract"), (5, "contract"), (40, "prefill")):
        x = M.make_x(50 + T, T, 512)
        out = blk(dev_bf16(x))
        torch.cuda.synchronize()
        got = host_bf16(out)
        ref, _, _ = M.block_forward(L, x, mode=mode)
        assert _mismatches(got, ref) <= max(2, got.size // 200), (T, mode)
        mlx, _, _ = M.block_forward(L, x, mode="mlx")
        g, m = M.bf16_to_f32(got), M.bf16_to_f32(mlx)
        assert np.abs(g - m).max() <= MAX_ABS
        assert cosine(g, m) >= MIN_COS


def _combine_ref(L, x, idx, w, residual, mode):
    y = M.switch_glu(L, x, np.where((idx >= 0) & (idx < L.experts), idx, 0), mode)
    y[(idx < 0) | (idx >= L.experts)] = 0.0
    acc = np.zeros((x.shape[0], L.hidden), np.float32)
    for j in range(idx.shape[1]):
        acc = (acc + w[:, j:j + 1] * y[:, j]).astype(np.float32)
    out = M.round_bf16(acc)
    if residual is not None:
        out = M.round_bf16(M.bf16_to_f32(residual) + out)
    return M.f32_to_bf16(out)


@pytest.mark.parametrize("T,mode", [(3, "contract"), (40, "prefill")])
@pytest.mark.parametrize("bits", [8, 4])
def test_switch_combine_matches_oracle(torch_cuda, T, mode, bits):
    """Caller indices (one out of range) and weights, with and without a
    residual: 3 tokens take the decode kernels, 40 tokens x 4 slots the
    expert-sorted GEMMs."""
    torch = torch_cuda
    from runnel_amd import native
    L = M.make_layer(60 + bits, hidden=512, inter=128, experts=24, top_k=4, bits=bits,
                     shared=False)
    rng = np.random.default_rng(T + bits)
    idx = rng.integers(0, 24, size=(T, 4)).astype(np.int32)
    idx[0, 2] = 24
    w = rng.uniform(0.05, 0.6, size=(T, 4)).astype(np.float32)
    x = M.make_x(70 + T, T, 512)
    r = M.make_x(71 + T, T, 512)
    keep = (bank_to_dev(L.gate_up), bank_to_dev(L.down))
    gu = native.qweight_struct(*keep[0], bits)
    dn = native.qweight_struct(*keep[1], bits)
    wt = torch.from_numpy(w).cuda()
    for res in (None, r):
        out = native.switch_combine(dev_bf16(x), dev_i32(idx), wt, gu, dn,
                                    residual=None if res is None else dev_bf16(res))
        torch.cuda.synchronize()
        got = host_bf16(out)
        ref = _combine_ref(L, x, idx, w, res, mode)
        assert _mismatches(got, ref) <= max(2, got.size // 200)
