"""The packed routed gate/up module and the sparse-MoE block on MI355X.

``fuse_routed_gate_up`` and ``FusedQuantizedSwitchGLU`` keep the call
surface, validation and error messages of src/runnel/mlx.py:8-95;
``SparseMoeBlock`` keeps the surface of the mlx-lm block that calls it
(``layer.mlp(x)``, bench/mlx_component_profile.py:130): router ``gate`` ->
softmax -> top-k -> renormalise -> ``switch_mlp(x, inds)`` -> weighted sum ->
``+ sigmoid(shared_expert_gate(x)) * shared_expert(x)``.

The arithmetic runs in librmoe.so (HIP, gfx950): with the packed module in
place and a SwiGLU activation the whole block is three kernels
(router, gate/up + SwiGLU, down + combine + shared expert).
"""

from __future__ import annotations

import gc

import torch
from torch import nn

from . import native
from .switch_layers import (MLP, Linear, QuantizedLinear, QuantizedSwitchLinear, RMSNorm,
                            SwiGLU, SwitchGLU, swiglu)

BF16 = torch.bfloat16


class FusedQuantizedSwitchGLU(nn.Module):
    """One packed [up; gate] expert bank instead of two
    (src/runnel/mlx.py:23-82)."""

    def __init__(self, old) -> None:
        super().__init__()
        gate = old.gate_proj
        up = old.up_proj
        if not (
            isinstance(gate, type(up))
            and gate.bits == up.bits
            and gate.group_size == up.group_size
            and gate.mode == up.mode
        ):
            raise ValueError("routed gate/up quantization formats differ")
        if ("bias" in gate) or ("bias" in up):
            raise ValueError("module biases are not expected for this checkpoint")

        # Rows [up; gate] along the output axis (src/runnel/mlx.py:38-48).
        self.register_buffer("weight", torch.cat([up["weight"], gate["weight"]], dim=1))
        self.register_buffer("scales", torch.cat([up["scales"], gate["scales"]], dim=1))
        up_biases = up.get("biases")
        gate_biases = gate.get("biases")
        if (up_biases is None) != (gate_biases is None):
            raise ValueError("routed gate/up affine-bias formats differ")
        self.register_buffer(
            "biases", None if up_biases is None else torch.cat([up_biases, gate_biases], dim=1))
        self.group_size = gate.group_size
        self.bits = gate.bits
        self.mode = gate.mode
        self.down_proj = old.down_proj
        self.activation = old.activation
        self._structs = None

    def __contains__(self, name: str) -> bool:
        return self._buffers.get(name) is not None

    def __getitem__(self, name: str):
        return self._buffers[name]

    def get(self, name: str, default=None):
        v = self._buffers.get(name)
        return default if v is None else v

    def _fast_path(self) -> bool:
        dp = self.down_proj
        return (isinstance(self.activation, SwiGLU) and self.mode == "affine"
                and self.get("biases") is not None
                and isinstance(dp, QuantizedSwitchLinear) and dp.mode == "affine"
                and dp.bits == self.bits and dp.group_size == self.group_size
                and "bias" not in dp)

    def qweights(self):
        """(gate_up, down) rmoe_qweight structs (cached)."""
        if self._structs is None:
            gu = native.qweight_struct(self.weight, self.scales, self.biases,
                                       self.bits, self.group_size)
            dp = self.down_proj
            dn = native.qweight_struct(dp.weight, dp.scales, dp.biases, dp.bits,
                                       dp.group_size)
            self._structs = (gu, dn)
        return self._structs

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        D = x.shape[-1]
        k = indices.shape[-1]
        lead = indices.shape[:-1]
        if self._fast_path():
            gu, dn = self.qweights()
            y = native.switch_glu(x.reshape(-1, D), indices.reshape(-1, k), gu, dn)
            return y.reshape(*lead, k, D)
        # Any other activation or down projection: packed gather, split, then
        # the module's own activation and down projection.
        xe = x.unsqueeze(-2).unsqueeze(-3)
        packed = QuantizedSwitchLinear(
            D, self.weight.shape[1], self.weight.shape[0], group_size=self.group_size,
            bits=self.bits, mode=self.mode, weight=self.weight, scales=self.scales,
            biases=self.biases)
        fused = packed(xe, indices)
        x_up, x_gate = torch.chunk(fused, 2, dim=-1)
        out = self.down_proj(self.activation(x_up, x_gate), indices)
        return out.squeeze(-2)


def fuse_routed_gate_up(model) -> int:
    """Replace every layer's routed ``switch_mlp`` by the packed module
    (src/runnel/mlx.py:8-95).  Returns the number of layers changed."""
    count = 0
    for layer in model.language_model.layers:
        old = layer.mlp.switch_mlp
        if not hasattr(old.gate_proj, "bits"):
            raise ValueError("routed gate/up are not quantized as expected")
        fused = FusedQuantizedSwitchGLU(old)
        layer.mlp.switch_mlp = fused
        if isinstance(layer.mlp, SparseMoeBlock):
            layer.mlp._handles = {}
        count += 1
        del old, fused
        gc.collect()
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
    return count


def _gate_linear(hidden_size: int, rows: int, gate_bits: int | None, group_size: int, device):
    if gate_bits is None:
        return Linear(hidden_size, rows, device=device)
    return QuantizedLinear(hidden_size, rows, bits=gate_bits, group_size=group_size,
                           device=device)


def _gate_operand(gate):
    """What the kernels take for a gate module: the bf16 weight, or the
    (weight, scales, biases) triple of an 8-bit group-64 affine gate; None
    for any other format."""
    if isinstance(gate, QuantizedLinear):
        if gate.bits != 8 or gate.group_size != 64 or gate.mode != "affine":
            return None
        return (gate.weight, gate.scales, gate.biases)
    return gate.weight


class SparseMoeBlock(nn.Module):
    """Router + routed experts + sigmoid-gated shared expert.  ``gate_bits``
    quantizes the router ``gate`` and ``shared_expert_gate`` (8 in real
    checkpoints: bench/runnel_bench/checkpoint.py:200-208); None keeps them
    bf16."""

    def __init__(self, hidden_size: int, moe_intermediate_size: int, num_experts: int,
                 num_experts_per_tok: int, shared_expert_intermediate_size: int | None = None,
                 norm_topk_prob: bool = True, bits: int = 8, group_size: int = 64,
                 device=None, gate_bits: int | None = None):
        super().__init__()
        self.num_experts = num_experts
        self.top_k = num_experts_per_tok
        self.norm_topk_prob = norm_topk_prob
        self.gate = _gate_linear(hidden_size, num_experts, gate_bits, group_size, device)
        self.switch_mlp = SwitchGLU(hidden_size, moe_intermediate_size, num_experts,
                                    bits=bits, group_size=group_size, device=device)
        if shared_expert_intermediate_size:
            self.shared_expert = MLP(hidden_size, shared_expert_intermediate_size, bits,
                                     group_size, device=device)
            self.shared_expert_gate = _gate_linear(hidden_size, 1, gate_bits, group_size,
                                                   device)
        else:
            self.shared_expert = None
            self.shared_expert_gate = None
        self._handles = {}

    # ------------------------------------------------------------ fast path
    def layer_handle(self, post_norm: RMSNorm | None = None) -> native.LayerHandle | None:
        """rmoe_layer for the fused path (with `post_norm` in front of the
        block when given), or None when the modules are not in the packed /
        SwiGLU / affine form it needs.  Cached per norm module."""
        key = None if post_norm is None else id(post_norm)
        if key in self._handles:
            return self._handles[key][0]
        sm = self.switch_mlp
        if not isinstance(sm, FusedQuantizedSwitchGLU) or not sm._fast_path():
            return None
        router = _gate_operand(self.gate)
        if router is None:
            return None
        shared = None
        sgate = None
        if self.shared_expert is not None:
            se = self.shared_expert
            if not all(isinstance(p, QuantizedLinear) and p.mode == "affine"
                       and p.bits == sm.bits and p.group_size == sm.group_size
                       for p in (se.gate_proj, se.up_proj, se.down_proj)):
                return None
            # Packed [up; gate] copy of the shared expert (3 MB at 8 bits).
            sgu = (torch.cat([se.up_proj.weight, se.gate_proj.weight], 0).contiguous(),
                   torch.cat([se.up_proj.scales, se.gate_proj.scales], 0).contiguous(),
                   torch.cat([se.up_proj.biases, se.gate_proj.biases], 0).contiguous())
            shared = (sgu, (se.down_proj.weight, se.down_proj.scales, se.down_proj.biases))
            sgate = _gate_operand(self.shared_expert_gate)
            if sgate is None or type(self.shared_expert_gate) is not type(self.gate):
                return None
        dp = sm.down_proj
        h = native.make_layer(
            router, (sm.weight, sm.scales, sm.biases),
            (dp.weight, dp.scales, dp.biases), self.top_k, self.norm_topk_prob,
            shared_gate_w=sgate,
            shared_gate_up=None if shared is None else shared[0],
            shared_down=None if shared is None else shared[1],
            bits=sm.bits, group_size=sm.group_size,
            post_norm_w=None if post_norm is None else post_norm.weight,
            norm_eps=1e-6 if post_norm is None else post_norm.eps)
        self._handles[key] = (h, post_norm)   # the norm module is kept alive with its key
        return h

    def __call__(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        D = x.shape[-1]
        lead = x.shape[:-1]
        h = self.layer_handle()
        if h is not None:
            res = None if residual is None else residual.reshape(-1, D)
            out = native.moe_block(h, x.reshape(-1, D), residual=res)
            return out.reshape(*lead, D)
        return self._composed(x, residual)

    def check_status(self, device="cuda") -> None:
        """Raise RmoeError(RMOE_ETIMEOUT) if a single-launch decode made by
        this block's calls on `device` (current stream) gave up a
        cross-workgroup wait, clearing the sticky word first.  Eager calls
        with plain launches check by themselves; graph users call this after
        a replay (it synchronises)."""
        ws = native.default_workspace(device, "block")
        if ws is not None:
            native.check_status(ws)

    def _composed(self, x, residual):
        """Module-by-module evaluation for unfused or non-SwiGLU layers."""
        D = x.shape[-1]
        lead = x.shape[:-1]
        x2 = x.reshape(-1, D)
        router = _gate_operand(self.gate)
        if router is None:
            raise ValueError("router gate must be bf16 or 8-bit group-64 affine")
        inds, scores = native.router(router, x2, self.top_k, self.norm_topk_prob)
        y = self.switch_mlp(x2, inds)  # [T, k, D]
        out = (y.float() * scores[..., None]).sum(dim=-2)
        if self.shared_expert is not None:
            sh = self.shared_expert(x2).float()
            sg = torch.sigmoid(self.shared_expert_gate(x2).float())
            out = out + sg * sh
        out = out.to(BF16)
        if residual is not None:
            out = (residual.reshape(-1, D).float() + out.float()).to(BF16)
        return out.reshape(*lead, D)


class PostAttentionMoE(nn.Module):
    """The MoE half of a decoder layer: ``h + mlp(post_attention_layernorm(h))``
    (the residual/norm sequence of docs/architecture.md:31-37).  With the
    block's fast path this is one rmoe_moe_block call (RMSNorm, router,
    experts, combine and residual add); `native.Chain` of the same handles
    runs a stack of layers in one launch."""

    def __init__(self, post_attention_layernorm: RMSNorm, mlp: SparseMoeBlock):
        super().__init__()
        self.post_attention_layernorm = post_attention_layernorm
        self.mlp = mlp

    def layer_handle(self) -> native.LayerHandle | None:
        return self.mlp.layer_handle(self.post_attention_layernorm)

    def check_status(self, device="cuda") -> None:
        self.mlp.check_status(device)

    def __call__(self, h: torch.Tensor) -> torch.Tensor:
        D = h.shape[-1]
        lead = h.shape[:-1]
        lh = self.layer_handle()
        h2 = h.reshape(-1, D)
        if lh is not None:
            return native.moe_block(lh, h2, residual=h2).reshape(*lead, D)
        return self.mlp(self.post_attention_layernorm(h2), residual=h2).reshape(*lead, D)
