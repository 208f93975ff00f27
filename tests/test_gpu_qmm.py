"""Dense quantized products at prefill sizes on the matrix cores
(rmoe_gather_qmm without index arrays, 64 rows or more, bf16 out): the
reference's own prefill QMM datasets (native/src/quantized_qmm_probe.mm:
243-307, x bf16 [64, 2048] against an 8- or 4-bit [4096, 2048] weight) and
random shapes, against the oracle.

The matrix-core path rounds every dequantised weight to bf16 (the prefill
contract), so it is held tightly to x . bf16(w)^T, and to the reference's
fp32-weight oracle and its recorded checksum within the error that rounding
the weights and the outputs to bf16 can cause."""

import json
from pathlib import Path

import numpy as np
import pytest

from helpers import dev_bf16, dev_i32, host_bf16
from oracle import moe_ref as M

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
U = 2.0 ** -8  # bf16 unit roundoff


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runnel_amd import _lib
    _lib.load()
    return torch


def _bf16_weight_product(x_bits, w, s, b, bits):
    """float64 x . bf16(fl32(q s + b))^T and the weights' rounding error."""
    w64 = M.dequantize(w, s, b, bits, dtype=np.float64)
    wb = M.round_bf16(w64.astype(np.float32)).astype(np.float64)
    x = M.bf16_to_f32(x_bits).astype(np.float64)
    return x @ wb.T, x, w64, wb


def _check_contract(got_bits, ref64, x, wb):
    """Within one bf16 step of the bf16-weight product plus the fp32
    accumulation's error (order unknown), elementwise."""
    got = M.bf16_to_f32(got_bits).astype(np.float64)
    acc = (np.abs(x) @ np.abs(wb).T) * x.shape[1] * 2.0 ** -24
    tol = U * np.abs(ref64) + acc + 1e-30
    bad = np.abs(got - ref64) > 2 * tol
    return int(bad.sum()), got


@pytest.mark.parametrize("case", GOLDEN["qmm"], ids=lambda c: Path(c["source"]).stem)
def test_reference_qmm_dataset_on_the_matrix_cores(torch_cuda, case):
    torch = torch_cuda
    from runnel_amd import native
    bits = case["bits"]
    ds = M.qmm_dataset(bits, case["tokens"], case["outputs"], case["reduction_size"])
    y = native.gather_qmm(dev_bf16(ds["x"]), dev_i32(ds["w"]), dev_bf16(ds["scales"]),
                          dev_bf16(ds["biases"]), bits)
    torch.cuda.synchronize()
    ref64, x, w64, wb = _bf16_weight_product(ds["x"], ds["w"], ds["scales"], ds["biases"], bits)
    nbad, got = _check_contract(host_bf16(y), ref64, x, wb)
    assert nbad == 0
    # against the reference's fp32-weight oracle (whose checksum the CPU
    # tests pin to the recorded one): weight rounding moves each output by at
    # most sum_k |x| |w - bf16(w)|, the bf16 output by U |y|
    exp = ds["expected"].astype(np.float64)
    dw = np.abs(w64 - wb)
    bound = np.abs(x) @ dw.T + U * np.abs(exp) + (np.abs(x) @ np.abs(wb).T) * 2048 * 2.0 ** -24
    assert (np.abs(got - exp) <= bound * 1.01 + 1e-6).all()
    # the recorded checksum (3 decimals), within the summed bound
    assert abs(got.sum() - case["reference_checksum"]) <= bound.sum() + 5e-4
    # and far inside it in practice: the rounding errors mostly cancel
    print(f"q{bits}: checksum {got.sum():.3f} vs recorded {case['reference_checksum']:.3f} "
          f"(bound {bound.sum():.1f})", flush=True)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("shape", [(64, 256, 128), (130, 768, 384), (300, 512, 2048)])
def test_dense_qmm_random_shapes(torch_cuda, bits, shape):
    """Partial row tiles (130, 300 rows), several column and K tiles."""
    torch = torch_cuda
    from runnel_amd import native
    Mr, N, K = shape
    rng = np.random.default_rng(Mr + N + K + bits)
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    words, s, b = M.quantize(w, bits)
    xb = M.make_x(5 + Mr, Mr, K)
    y = native.gather_qmm(dev_bf16(xb), dev_i32(words), dev_bf16(s), dev_bf16(b), bits)
    torch.cuda.synchronize()
    ref64, x, _, wb = _bf16_weight_product(xb, words, s, b, bits)
    nbad, _ = _check_contract(host_bf16(y), ref64, x, wb)
    assert nbad == 0
