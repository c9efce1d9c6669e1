"""The five measured configurations of the attention block and their seeded synthetic inputs.

Shapes, dtypes and initialisations are the configurations the block is measured on. Inputs
follow the reference's generator (`generate_random_case`, torch_transformer_benchmark.py:234-272:
x ~ N(0, 1) * input_scale, all-true mask when padding_ratio = 0) with one difference: values
are drawn in fp32 from a seeded CPU (or device) torch.Generator and then rounded to the
configuration dtype, so a CPU checker and the GPU see bit-identical inputs.
Seed conventions: accuracy trials use seed + trial (:387), timing uses seed + 100000 (:533).
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass
from typing import Dict, Optional

import torch

BASE_SEED = 1234
# Parameters come from their own stream: drawing them with an input seed would make the first
# input rows copies of weight rows (the reference seeds modules from the CPU default generator
# and inputs from a separate device generator, torch_transformer_benchmark.py:683, :241-242).
WEIGHT_SEED = 987654321
FIXED_SEEDS = tuple(BASE_SEED + t for t in range(5))
TIMING_SEED = BASE_SEED + 100000
PROJECTIONS = ("q_proj", "k_proj", "v_proj", "out_proj")


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    seq: int
    d_model: int
    heads: int
    dtype: torch.dtype          # activation dtype at the block boundary
    causal: bool
    int8: bool                  # W8A8 projections (fp16 SDPA)
    weight_init: str            # "normal_inv_d" | "xavier_uniform" | "normal_0.02"
    description: str = ""

    @property
    def head_dim(self) -> int:
        return self.d_model // self.heads

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    def scaled(self, batch: Optional[int] = None, seq: Optional[int] = None) -> "Workload":
        return dataclasses.replace(self, batch=batch or self.batch, seq=seq or self.seq,
                                   name=f"{self.name}[B{batch or self.batch},S{seq or self.seq}]")

    def flops(self) -> Dict[str, float]:
        """Algorithmic operation counts (Project/loop/ceiling.py:93-97 accounting)."""
        T, d = self.tokens, self.d_model
        attn = 4.0 * self.batch * self.heads * self.seq * self.seq * self.head_dim
        if self.causal:
            attn *= 0.5
        return {"qkv": 2.0 * T * d * 3 * d, "out": 2.0 * T * d * d, "attn": attn}

    def bytes(self) -> Dict[str, float]:
        """Algorithmic bytes per stage: every operand read or written once."""
        T, d = self.tokens, self.d_model
        act = 2 if self.dtype in (torch.float16, torch.bfloat16) else 4
        if self.int8:
            return {
                "qkv": T * d * 1 + T * 4 + 3 * d * d * 1 + 3 * d * 4 * 2 + T * 3 * d * 2,
                "attn": T * 3 * d * 2 + T * d * 2,
                "out": T * d * 1 + T * 4 + d * d + d * 4 * 2 + T * d * act,
            }
        return {
            "qkv": (T * d + 3 * d * d + 3 * d + T * 3 * d) * act,
            "attn": (T * 3 * d + T * d) * act,
            "out": (T * d + d * d + d + T * d) * act,
        }


CONFIGS: Dict[str, Workload] = {
    "C1": Workload("C1", 1, 128, 256, 4, torch.float32, False, False, "normal_inv_d",
                   "B1 S128 d256 H4x64 fp32 non-causal"),
    "C2": Workload("C2", 8, 2048, 1024, 16, torch.float16, False, False, "xavier_uniform",
                   "B8 S2048 d1024 H16x64 fp16 non-causal"),
    "C3": Workload("C3", 4, 8192, 2048, 32, torch.bfloat16, True, False, "normal_0.02",
                   "B4 S8192 d2048 H32x64 bf16 causal"),
    "C4": Workload("C4", 16, 4096, 4096, 32, torch.float16, False, True, "normal_0.02",
                   "B16 S4096 d4096 H32x128 int8 W8A8 projections + fp16 SDPA"),
    "C5": Workload("C5", 32, 100000, 512, 8, torch.float16, False, False, "normal_inv_d",
                   "B32 S100000 d512 H8x64 fp16 non-causal (streamed)"),
}


def make_params(w: Workload, seed: int = WEIGHT_SEED) -> Dict[str, torch.Tensor]:
    """fp32 CPU parameters ``{'q_proj.weight': [d, d], 'q_proj.bias': [d], ...}``.

    Weights follow the configuration's init; biases keep nn.Linear's default U(±1/sqrt(d)).
    """
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    d = w.d_model
    out: Dict[str, torch.Tensor] = {}
    for name in PROJECTIONS:
        if w.weight_init == "normal_inv_d":
            wt = torch.randn(d, d, generator=g) / math.sqrt(d)
        elif w.weight_init == "xavier_uniform":
            a = math.sqrt(6.0 / (d + d))
            wt = (torch.rand(d, d, generator=g) * 2.0 - 1.0) * a
        elif w.weight_init == "normal_0.02":
            wt = torch.randn(d, d, generator=g) * 0.02
        else:
            raise ValueError(w.weight_init)
        bound = 1.0 / math.sqrt(d)
        bt = (torch.rand(d, generator=g) * 2.0 - 1.0) * bound
        out[f"{name}.weight"] = wt.contiguous()
        out[f"{name}.bias"] = bt.contiguous()
    return out


def make_input(w: Workload, seed: int, device: str = "cpu", input_scale: float = 1.0) -> torch.Tensor:
    """x ~ N(0, 1) * input_scale of shape [B, S, d], drawn in fp32 then rounded to ``w.dtype``."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    x = torch.randn(w.batch, w.seq, w.d_model, generator=g, device=device, dtype=torch.float32)
    if input_scale != 1.0:
        x = x * input_scale
    return x.to(w.dtype)


def make_core_inputs(w: Workload, seed: int, device: str = "cpu"):
    """The attention core's own inputs, as C5 states them: Q, K, V ~ N(0, 1) / sqrt(head_dim)
    of shape [B, S, H, head_dim], drawn in fp32 (one seeded generator, Q then K then V) and
    rounded to ``w.dtype``."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    shape = (w.batch, w.seq, w.heads, w.head_dim)
    sc = 1.0 / math.sqrt(w.head_dim)
    return tuple((torch.randn(shape, generator=g, device=device, dtype=torch.float32) * sc)
                 .to(w.dtype) for _ in range(3))


def core_flops_bytes(w: Workload):
    """Algorithmic FLOPs and bytes of the attention core alone (Q, K, V read, O written once)."""
    e = 2 if w.dtype in (torch.float16, torch.bfloat16) else 4
    return w.flops()["attn"], 4.0 * w.tokens * w.d_model * e


def round_params(params: Dict[str, torch.Tensor], dtype: torch.dtype) -> Dict[str, torch.Tensor]:
    """Parameters rounded to ``dtype`` (what a ``model.to(dtype)`` holds)."""
    return {k: v.to(dtype) for k, v in params.items()}


# The benchmark's 14 official shapes (Project/shapes.json, "3.7 Appendix Test shapes" of the
# reference README): id -> (batch, d_model, heads, seq_len, layers, ffn_dim); every one causal,
# run by torch_transformer_benchmark.py in float32 unless --dtype says otherwise.
OFFICIAL_SHAPES = {
    1: (64, 128, 4, 128, 4, 128), 2: (1, 128, 4, 128, 4, 128), 3: (4, 128, 4, 128, 4, 128),
    4: (16, 128, 4, 128, 4, 128), 5: (128, 128, 4, 128, 4, 128), 6: (10000, 128, 4, 128, 4, 128),
    7: (64, 32, 4, 128, 4, 32), 8: (64, 1024, 4, 128, 4, 1024), 9: (64, 128, 1, 128, 4, 128),
    10: (64, 128, 2, 128, 4, 128), 11: (64, 128, 16, 128, 4, 128), 12: (64, 128, 4, 32, 4, 128),
    13: (64, 128, 4, 1024, 4, 128), 14: (32, 1024, 16, 100000, 2, 1024),
}


def official_flops(sid: int) -> float:
    """Algorithmic FLOPs of one model forward at an official shape: per layer the four
    projections (8 T d^2), the FFN (4 T d f) and causal attention (2 B S^2 d)."""
    B, d, H, S, L, F = OFFICIAL_SHAPES[sid]
    T = B * S
    return L * (8.0 * T * d * d + 4.0 * T * d * F + 2.0 * B * S * S * d)
