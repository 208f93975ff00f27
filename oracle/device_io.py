"""Moving oracle (numpy) layers onto the GPU and GPU results back to numpy.

TEST INFRASTRUCTURE ONLY (used by tests/, smoke() and the cpu_baseline leg
of bench.py); the shipped package never imports it.
"""

from __future__ import annotations

import numpy as np


def dev_bf16(a, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).to(
        device).view(torch.bfloat16)


def dev_i32(a, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(device)


def host_bf16(t) -> np.ndarray:
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_u32(t) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy().view(np.uint32)


def bank_to_dev(q, device="cuda", squeeze=False):
    w, s, b = dev_i32(q.w, device), dev_bf16(q.scales, device), dev_bf16(q.biases, device)
    if squeeze:
        w, s, b = w[0], s[0], b[0]
    return (w, s, b)


def gate_to_dev(g, device="cuda"):
    """A bf16 gate (bits) -> bf16 tensor; a quantized one (QWeight [1, rows,
    H]) -> its (weight, scales, biases) device triple without the expert
    axis."""
    from oracle.moe_ref import QWeight
    if isinstance(g, QWeight):
        return bank_to_dev(g, device, squeeze=True)
    return dev_bf16(g, device)


def layer_to_dev(L, device="cuda"):
    """oracle.moe_ref.Layer -> runnel_amd.native.LayerHandle (+ tensors)."""
    from runnel_amd import native
    shared = L.shared_gate_up is not None
    return native.make_layer(
        gate_to_dev(L.router_w, device), bank_to_dev(L.gate_up, device),
        bank_to_dev(L.down, device), L.top_k, L.norm_topk_prob,
        gate_to_dev(L.shared_gate_w, device) if shared and L.shared_gate_w is not None
        else None,
        bank_to_dev(L.shared_gate_up, device, squeeze=True) if shared else None,
        bank_to_dev(L.shared_down, device, squeeze=True) if shared else None,
        bits=L.gate_up.bits,
        post_norm_w=None if L.post_norm_w is None else dev_bf16(L.post_norm_w, device),
        norm_eps=L.norm_eps)


def bank_from_dev(w, s, b, bits):
    from oracle.moe_ref import QWeight
    w, s, b = host_u32(w), host_bf16(s), host_bf16(b)
    if w.ndim == 2:
        w, s, b = w[None], s[None], b[None]
    return QWeight(w, s, b, bits)


def layer_from_dev(lw):
    """runnel_amd.synthetic.LayerWeights -> oracle.moe_ref.Layer (host copy)."""
    from oracle.moe_ref import Layer
    gu = bank_from_dev(*lw.gate_up, lw.bits)
    dn = bank_from_dev(*lw.down, lw.bits)
    E = gu.w.shape[0]

    def gate(g):
        if isinstance(g, tuple):
            return bank_from_dev(*g, 8)
        return host_bf16(g)

    L = Layer(gu.cols, gu.rows // 2, E, lw.top_k, gate(lw.router_w), gu, dn,
              norm_topk_prob=lw.norm_topk_prob)
    if lw.post_norm_w is not None:
        L.post_norm_w = host_bf16(lw.post_norm_w)
        L.norm_eps = lw.norm_eps
    if lw.shared_gate_up is not None:
        L.shared_gate_w = gate(lw.shared_gate_w)
        L.shared_gate_up = bank_from_dev(*lw.shared_gate_up, lw.bits)
        L.shared_down = bank_from_dev(*lw.shared_down, lw.bits)
    return L


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
