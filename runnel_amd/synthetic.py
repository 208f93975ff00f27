"""Synthetic MoE layers generated on the GPU.

Weights are drawn from N(0, std) with a seeded torch generator on the
device, quantized by the HIP quantizer (rmoe_quantize) in chunks, and kept
resident: a 256-expert 8-bit layer is 0.86 GB, so the 40-layer stack is
34 GB of HBM.  The router and the shared-expert gate are bf16, or 8-bit
group-64 (weight, scales, biases) triples with ``gate_bits=8`` (the format
of real checkpoints).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import native

BF16 = torch.bfloat16


@dataclass
class LayerWeights:
    router_w: "torch.Tensor | tuple"  # bf16 [E, H] or an 8-bit triple [E, ...]
    gate_up: tuple                # (int32 [E, 2I, H/vpw], bf16 [E, 2I, H/64] x2)
    down: tuple                   # (int32 [E, H, I/vpw], ...)
    shared_gate_w: "torch.Tensor | tuple | None"  # bf16 [H] or an 8-bit triple [1, ...]
    shared_gate_up: tuple | None  # [2Is, H/vpw] ...
    shared_down: tuple | None
    bits: int
    top_k: int
    norm_topk_prob: bool = True
    post_norm_w: torch.Tensor | None = None   # bf16 [H]: RMSNorm before the block
    norm_eps: float = 1e-6

    def handle(self) -> native.LayerHandle:
        return native.make_layer(self.router_w, self.gate_up, self.down, self.top_k,
                                 self.norm_topk_prob, self.shared_gate_w,
                                 self.shared_gate_up, self.shared_down, self.bits,
                                 post_norm_w=self.post_norm_w, norm_eps=self.norm_eps)

    def tensors(self):
        def flat(g):
            return list(g) if isinstance(g, tuple) else [g]
        ts = [*flat(self.router_w), *self.gate_up, *self.down]
        if self.shared_gate_up is not None:
            ts += [*flat(self.shared_gate_w), *self.shared_gate_up, *self.shared_down]
        if self.post_norm_w is not None:
            ts.append(self.post_norm_w)
        return ts

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors())


def _quantized_bank(gen, experts, rows, cols, bits, std, device, chunk_rows=1 << 16):
    vpw = native.values_per_word(bits)
    total = experts * rows
    w = torch.empty((total, cols // vpw), dtype=torch.int32, device=device)
    s = torch.empty((total, cols // 64), dtype=BF16, device=device)
    b = torch.empty_like(s)
    for r0 in range(0, total, chunk_rows):
        r1 = min(total, r0 + chunk_rows)
        f = torch.randn((r1 - r0, cols), generator=gen, device=device, dtype=torch.float32)
        f.mul_(std)
        wq, sq, bq = native.quantize(f, bits)
        w[r0:r1].copy_(wq)
        s[r0:r1].copy_(sq)
        b[r0:r1].copy_(bq)
        del f, wq, sq, bq
    shape = (experts, rows) if experts > 1 else (rows,)
    return (w.reshape(*shape, -1), s.reshape(*shape, -1), b.reshape(*shape, -1))


def make_layer(seed: int, hidden=2048, inter=512, experts=256, top_k=8, bits=8,
               shared=True, std=0.02, router_std=0.02, device="cuda",
               shared_inter=None, gate_bits=None, post_norm=False) -> LayerWeights:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shared_inter = inter if shared_inter is None else shared_inter

    def gate(shape):
        w = torch.randn(shape, generator=gen, device=device) * router_std
        if gate_bits is None:
            return w.to(BF16)
        return tuple(t.reshape(-1 if len(shape) > 1 else 1, t.shape[-1])
                     for t in native.quantize(w.reshape(-1, hidden), gate_bits))

    router = gate((experts, hidden))
    gu = _quantized_bank(gen, experts, 2 * inter, hidden, bits, std, device)
    dn = _quantized_bank(gen, experts, hidden, inter, bits, std, device)
    if gu[0].dim() == 2:  # experts == 1 keeps the expert axis for banks
        gu = tuple(t.unsqueeze(0) for t in gu)
        dn = tuple(t.unsqueeze(0) for t in dn)
    sg = sgu = sdn = None
    if shared:
        sg = gate((hidden,))
        sgu = _quantized_bank(gen, 1, 2 * shared_inter, hidden, bits, std, device)
        sdn = _quantized_bank(gen, 1, hidden, shared_inter, bits, std, device)
    lw = LayerWeights(router, gu, dn, sg, sgu, sdn, bits, top_k)
    if post_norm:
        # RMSNorm weights around 1 (uniform in [0.5, 1.5])
        lw.post_norm_w = (torch.rand((hidden,), generator=gen, device=device) + 0.5).to(BF16)
    return lw


def make_x(seed: int, tokens: int, hidden: int, device="cuda") -> torch.Tensor:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return torch.randn((tokens, hidden), generator=gen, device=device).to(BF16)


# Skewed routing for long prefill: a per-expert router logit bias
# -alpha * s * ln(rank) (Zipf exponent s) over a seeded random ranking of the
# experts.  The block has no router bias term, so the bias rides on one input
# feature held constant: x[:, 0] = BIAS_FEATURE for every token and router
# column 0 = bias / BIAS_FEATURE.  With alpha 0.8 and s 1.1, 8192 tokens at
# top-8 of 256 give about 16 experts more than 1000 rows each while about
# half the experts receive fewer than 8.
BIAS_FEATURE = 4.0


def zipf_bias(seed: int, experts: int, s: float = 1.1, alpha: float = 0.8,
              device="cuda") -> torch.Tensor:
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    rank = torch.randperm(experts, generator=gen).to(torch.float64) + 1.0
    return (-alpha * s * torch.log(rank)).to(torch.float32).to(device)


def apply_router_bias(layer: LayerWeights, bias: torch.Tensor) -> None:
    """Route `bias` through input feature 0 (inputs from make_skewed_x).
    A bf16 router only."""
    if isinstance(layer.router_w, tuple):
        raise ValueError("router bias needs a bf16 router")
    layer.router_w[:, 0] = (bias / BIAS_FEATURE).to(BF16)


def make_skewed_x(seed: int, tokens: int, hidden: int, device="cuda") -> torch.Tensor:
    x = make_x(seed, tokens, hidden, device)
    x[:, 0] = BIAS_FEATURE
    return x
