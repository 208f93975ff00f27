"""torch mirrors of the mlx-lm modules that Runnel's packed module plugs
into: quantized (switch) linears, SwitchGLU, SwiGLU and the shared-expert MLP.

They keep mlx-lm's attribute names (``weight``, ``scales``, ``biases``,
``bits``, ``group_size``, ``mode``, ``gate_proj``, ``up_proj``,
``down_proj``, ``activation``) because ``fuse_routed_gate_up`` reads exactly
those (src/runnel/mlx.py:25-53, :85-90).  The projections run the HIP
gather-QMV through librmoe.so; there is no host fallback.
"""

from __future__ import annotations

import torch
from torch import nn

from . import native

BF16 = torch.bfloat16


class _Params(nn.Module):
    """Buffers addressable like an MLX module: ``"bias" in m``, ``m["weight"]``,
    ``m.get("biases")``."""

    def __contains__(self, name: str) -> bool:
        return self._buffers.get(name) is not None

    def __getitem__(self, name: str):
        return self._buffers[name]

    def get(self, name: str, default=None):
        v = self._buffers.get(name)
        return default if v is None else v


class Linear(_Params):
    """bf16 linear without bias, weight [out, in] (the router ``gate`` and the
    ``shared_expert_gate``)."""

    def __init__(self, input_dims: int, output_dims: int, weight=None, device=None):
        super().__init__()
        if weight is None:
            weight = torch.zeros((output_dims, input_dims), dtype=BF16, device=device)
        self.register_buffer("weight", weight.to(BF16).contiguous())

    def __call__(self, x):  # pragma: no cover - exercised on the GPU
        lead = x.shape[:-1]
        y = native_linear(x.reshape(-1, x.shape[-1]), self.weight)
        return y.reshape(*lead, self.weight.shape[0])


def native_linear(x2d: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """bf16 x @ w.T for the small router-style linears, as bf16.  Routed
    through the block kernels when it is the router itself; for other uses
    this plain matmul is accumulated in fp32 by the library GEMM."""
    return torch.matmul(x2d.to(BF16), w.t().contiguous()).to(BF16)


class RMSNorm(_Params):
    """mlx ``nn.RMSNorm``: ``weight`` bf16 [dims], ``eps``; the decoder's
    ``post_attention_layernorm`` in front of the MoE block."""

    def __init__(self, dims: int, eps: float = 1e-6, weight=None, device=None):
        super().__init__()
        if weight is None:
            weight = torch.ones(dims, dtype=BF16, device=device)
        self.register_buffer("weight", weight.to(BF16).contiguous())
        self.eps = float(eps)

    def __call__(self, x):
        return native.rms_norm(x, self.weight, self.eps)


class QuantizedLinear(_Params):
    """MLX-affine quantized linear: weight int32 [out, in*bits/32], scales /
    biases bf16 [out, in/group]."""

    def __init__(self, input_dims: int, output_dims: int, bits: int = 8,
                 group_size: int = 64, mode: str = "affine", weight=None,
                 scales=None, biases=None, device=None):
        super().__init__()
        self.bits = bits
        self.group_size = group_size
        self.mode = mode
        vpw = native.values_per_word(bits)
        if weight is None:
            weight = torch.zeros((output_dims, input_dims // vpw), dtype=torch.int32, device=device)
            scales = torch.zeros((output_dims, input_dims // group_size), dtype=BF16, device=device)
            biases = torch.zeros_like(scales)
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)

    @property
    def input_dims(self):
        return self.weight.shape[-1] * native.values_per_word(self.bits)

    @property
    def output_dims(self):
        return self.weight.shape[-2]

    @classmethod
    def from_float(cls, w: torch.Tensor, bits: int = 8, group_size: int = 64):
        wq, s, b = native.quantize(w.float(), bits, group_size)
        return cls(w.shape[-1], w.shape[-2], bits, group_size, weight=wq, scales=s, biases=b)

    def __call__(self, x):
        lead = x.shape[:-1]
        y = native.gather_qmm(x.reshape(-1, x.shape[-1]), self.weight, self.scales,
                              self.biases, self.bits, self.group_size)
        return y.reshape(*lead, self.output_dims)


class QuantizedSwitchLinear(_Params):
    """Expert bank [num_experts, out, in] in MLX-affine format with mlx-lm's
    call convention: ``__call__(x, indices, sorted_indices=False)`` where x
    is ``[..., 1 or k, 1, in]`` and indices ``[..., k]``; returns
    ``[..., k, 1, out]`` (gather_qmm with transpose=True)."""

    def __init__(self, input_dims: int, output_dims: int, num_experts: int,
                 bias: bool = False, group_size: int = 64, bits: int = 8,
                 mode: str = "affine", weight=None, scales=None, biases=None,
                 device=None):
        super().__init__()
        self.bits = bits
        self.group_size = group_size
        self.mode = mode
        vpw = native.values_per_word(bits)
        if weight is None:
            weight = torch.zeros((num_experts, output_dims, input_dims // vpw),
                                 dtype=torch.int32, device=device)
            scales = torch.zeros((num_experts, output_dims, input_dims // group_size),
                                 dtype=BF16, device=device)
            biases = torch.zeros_like(scales)
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.register_buffer(
            "bias", torch.zeros((num_experts, output_dims), dtype=BF16, device=weight.device)
            if bias else None)

    @property
    def num_experts(self):
        return self.weight.shape[0]

    @property
    def input_dims(self):
        return self.weight.shape[-1] * native.values_per_word(self.bits)

    @property
    def output_dims(self):
        return self.weight.shape[1]

    @classmethod
    def from_float(cls, w: torch.Tensor, bits: int = 8, group_size: int = 64):
        """w float32 [E, out, in] on the GPU."""
        wq, s, b = native.quantize(w.float(), bits, group_size)
        E, out, inp = w.shape
        return cls(inp, out, E, False, group_size, bits, weight=wq, scales=s, biases=b)

    def __call__(self, x, indices, sorted_indices: bool = False):
        del sorted_indices  # row order does not change any result here
        if self.mode != "affine":
            raise ValueError(f"quantization mode {self.mode!r} is not supported")
        D = x.shape[-1]
        idx_shape = indices.shape
        xb = x.shape[:-2]
        n_x = 1
        for d in xb:
            n_x *= d
        lhs = torch.arange(n_x, device=x.device, dtype=torch.int32).reshape(xb)
        lhs = torch.broadcast_to(lhs, idx_shape).reshape(-1)
        y = native.gather_qmm(x.reshape(n_x, D), self.weight, self.scales, self.biases,
                              self.bits, self.group_size,
                              rhs_indices=indices.reshape(-1), lhs_indices=lhs)
        if "bias" in self:
            y = y + self["bias"][indices.reshape(-1).long()]
        return y.reshape(*idx_shape, 1, self.output_dims)


def swiglu(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.silu(gate) * x


class SwiGLU(nn.Module):
    """mlx-lm ``SwiGLU``: ``activation(x_up, x_gate) = silu(x_gate) * x_up``
    (called as at src/runnel/mlx.py:78)."""

    def __call__(self, x, gate):
        return swiglu(x, gate)


class SwitchGLU(nn.Module):
    """The stock routed MLP (three expert gathers) that
    ``fuse_routed_gate_up`` replaces."""

    def __init__(self, input_dims: int, hidden_dims: int, num_experts: int,
                 activation: nn.Module | None = None, bits: int = 8,
                 group_size: int = 64, device=None):
        super().__init__()
        self.gate_proj = QuantizedSwitchLinear(input_dims, hidden_dims, num_experts,
                                               group_size=group_size, bits=bits, device=device)
        self.up_proj = QuantizedSwitchLinear(input_dims, hidden_dims, num_experts,
                                             group_size=group_size, bits=bits, device=device)
        self.down_proj = QuantizedSwitchLinear(hidden_dims, input_dims, num_experts,
                                               group_size=group_size, bits=bits, device=device)
        self.activation = activation if activation is not None else SwiGLU()

    def __call__(self, x, indices):
        x = x.unsqueeze(-2).unsqueeze(-3)  # expand_dims(x, (-2, -3))
        x_up = self.up_proj(x, indices)
        x_gate = self.gate_proj(x, indices)
        x = self.down_proj(self.activation(x_up, x_gate), indices)
        return x.squeeze(-2)


class MLP(nn.Module):
    """Shared expert: ``down(silu(gate(x)) * up(x))`` with quantized linears."""

    def __init__(self, dim: int, hidden_dim: int, bits: int = 8, group_size: int = 64,
                 device=None):
        super().__init__()
        self.gate_proj = QuantizedLinear(dim, hidden_dim, bits, group_size, device=device)
        self.up_proj = QuantizedLinear(dim, hidden_dim, bits, group_size, device=device)
        self.down_proj = QuantizedLinear(hidden_dim, dim, bits, group_size, device=device)

    def __call__(self, x):
        return self.down_proj(swiglu(self.up_proj(x), self.gate_proj(x)))
