"""rmoe_moe_block_noalloc (the block with the library's static scratch, for
callers that cannot allocate) through the C ABI, against rmoe_moe_block
with a caller workspace: the same kernels, so the outputs, indices and
scores are equal bit for bit.  Two calls in a row on the shared static
scratch, the second with a smaller input, on each path the block takes."""

import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from helpers import dev_bf16, layer_to_dev
from oracle import moe_ref as M

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from runnel_amd import _lib
    _lib.load()
    return torch


def _noalloc(torch, h, x, residual=None):
    from runnel_amd import _lib
    lib = _lib.load()
    T = x.shape[0]
    out = torch.empty_like(x)
    idx = torch.full((T, h.top_k), -1, dtype=torch.int32, device=x.device)
    sc = torch.full((T, h.top_k), -1.0, dtype=torch.float32, device=x.device)
    st = torch.full((1,), 7, dtype=torch.int32, device=x.device)
    rc = lib.rmoe_moe_block_noalloc(ctypes.byref(h.struct), x.data_ptr(), T,
                                    _lib.ptr(residual), out.data_ptr(), idx.data_ptr(),
                                    sc.data_ptr(), st.data_ptr(), _lib.stream_handle(x.device))
    assert rc == _lib.RMOE_OK, lib.rmoe_last_error()
    return out, idx, sc, st


def _with_workspace(torch, h, x, residual=None):
    from runnel_amd import native
    ws = torch.zeros(h.workspace_bytes(x.shape[0]), dtype=torch.uint8, device=x.device)
    out, idx, sc = native.moe_block(h, x, residual=residual, return_routing=True,
                                    workspace=ws, check=False)
    return out, idx, sc, ws


def _same(torch, a, b):
    out, idx, sc, st = a
    out_w, idx_w, sc_w, ws = b
    torch.cuda.synchronize()
    from runnel_amd import native
    assert int(st.item()) == 0
    assert native.workspace_status(ws) == 0
    assert torch.equal(idx, idx_w)
    assert torch.equal(sc, sc_w)
    assert torch.equal(out, out_w)


@pytest.mark.parametrize("bits", [8, 4])
def test_noalloc_full_layer_prefill_then_decode(torch_cuda, bits):
    """A full-size layer: 40 tokens (the expert-sorted matrix-core path),
    then one token (the single-launch decode kernel) with a residual, then
    4 tokens (the few-token kernels, whose router hands its logits over in
    the static scratch)."""
    torch = torch_cuda
    from runnel_amd import synthetic
    print(f"noalloc full layer bits={bits}", flush=True)
    lw = synthetic.make_layer(8800 + bits, bits=bits)
    h = lw.handle()
    x40 = synthetic.make_x(8801, 40, 2048)
    _same(torch, _noalloc(torch, h, x40), _with_workspace(torch, h, x40))
    x1 = synthetic.make_x(8802, 1, 2048)
    r1 = synthetic.make_x(8803, 1, 2048)
    _same(torch, _noalloc(torch, h, x1, r1), _with_workspace(torch, h, x1, r1))
    x4 = synthetic.make_x(8804, 4, 2048)
    for _ in range(2):
        _same(torch, _noalloc(torch, h, x4), _with_workspace(torch, h, x4))


def test_noalloc_small_layer_few_tokens(torch_cuda):
    """A small layer: 5 tokens then 2 (router, gate/up and down kernels),
    and the oracle agrees on the routing."""
    torch = torch_cuda
    print("noalloc small layer", flush=True)
    L = M.make_layer(8810, hidden=512, inter=128, experts=32, top_k=4, bits=8)
    h = layer_to_dev(L)
    for T in (5, 2):
        xn = M.make_x(8811 + T, T, 512)
        x = dev_bf16(xn)
        a = _noalloc(torch, h, x)
        _same(torch, a, _with_workspace(torch, h, x))
        _, ref_idx, _ = M.block_forward(L, xn)
        assert np.array_equal(a[1].cpu().numpy(), ref_idx)


def test_noalloc_first_calls_under_graph_capture(torch_cuda):
    """In a fresh process, the first noalloc calls (1 and 40 tokens) are made
    under graph capture; replays equal the workspace path bit for bit with
    status 0 (tests/noalloc_capture_case.py)."""
    case = Path(__file__).resolve().parent / "noalloc_capture_case.py"
    print("noalloc first calls under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-u", str(case)], capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    assert "noalloc capture ok" in r.stdout
