"""runnel_amd: Runnel's quantized sparse-MoE block, MI355X-native.

Drop-in surfaces:
  fuse_routed_gate_up(model) -> int, FusedQuantizedSwitchGLU
      (the reference's src/runnel/mlx.py:8-95)
  SparseMoeBlock   the mlx-lm block that calls the packed module
  native.*         torch-facing wrappers of the C ABI in include/rmoe.h
The compute runs in runnel_amd/librmoe.so (hand-written HIP for gfx950).
"""

from .moe import FusedQuantizedSwitchGLU, PostAttentionMoE, SparseMoeBlock, fuse_routed_gate_up
from .switch_layers import (MLP, Linear, QuantizedLinear, QuantizedSwitchLinear, RMSNorm,
                            SwiGLU, SwitchGLU)

__all__ = [
    "FusedQuantizedSwitchGLU", "PostAttentionMoE", "SparseMoeBlock", "fuse_routed_gate_up",
    "MLP", "Linear", "QuantizedLinear", "QuantizedSwitchLinear", "RMSNorm", "SwiGLU",
    "SwitchGLU",
]
