"""MI355X-native (gfx950) attention-block hot path of the TechJam 2026 Track 3 transformer.

Public API:
  SelfAttention, Int8SelfAttention      drop-in modules for BaselineSelfAttention
  TransformerBlock, Transformer         the benchmark's block and model (every stage on the
                                        kernels, the reference's parameter names)
  build, swap_attention, swap_blocks,
  swap_model,
  make_user_optimized_transformer       the reference's plugin insertion points (swap_blocks: the
                                        attention half of each block fused; swap_model: every
                                        block and the final norm)
  GraphedForward                        whole-forward graph capture / replay (small-shape latency)
  ops                                   torch wrappers of the C-ABI kernels
  workloads                             the measured configurations and seeded inputs
"""
from .attention import Int8SelfAttention, SelfAttention
from .plugin import (build, make_user_optimized_transformer, swap_attention, swap_blocks,
                     swap_model)
from .transformer import Transformer, TransformerBlock
from .graph import GraphedForward
from . import ops, workloads

BaselineSelfAttention = SelfAttention  # the reference's class name

__all__ = [
    "SelfAttention", "Int8SelfAttention", "BaselineSelfAttention", "build", "swap_attention",
    "make_user_optimized_transformer", "swap_blocks", "swap_model", "Transformer",
    "TransformerBlock", "GraphedForward", "ops", "workloads",
]
