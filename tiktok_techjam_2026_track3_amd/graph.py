"""Whole-forward graph capture of the attention block (the small-shape latency path).

At small shapes (the fp32 configuration: 128 tokens, three kernels of a few microseconds each)
the per-launch host cost of an eager forward is as large as the GPU work. ``GraphedForward``
records one forward of a module -- ``SelfAttention.forward`` or, with ``norm``, the block's
attention half ``forward_residual`` -- into a HIP graph once, on static input buffers, and
replays it per call: one graph launch instead of one launch per kernel plus the Python work
around them. The reference's optimised route does the same with CUDA graphs
(Project/submission/dispatcher_region.py:1220-1363).

The forward is capture-safe by construction: every kernel is launched on torch's current stream,
nothing synchronises the host, and every buffer is allocated through torch's caching allocator
(which keeps graph allocations in the graph's private pool). Each call copies the inputs into
the static buffers, replays, and returns a fresh copy of the output (callers own their output,
as with the eager forward). A captured graph is tied to the shapes, dtype, device, causal flag
and mask presence it was recorded with, and to the module's parameters at capture time (the
graph reads the packed weights -- and, for the attention half, the LayerNorm-folded QKV weights --
the module had then, and keeps them alive): calling it with other inputs, after the parameters
(the module's or the norm's) changed, or after the module rebuilt or dropped its derived weights
(``.to()``, ``load_state_dict``), raises.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn


class GraphedForward:
    """Capture ``module(x, valid_token_mask, causal)`` (or ``module.forward_residual(x, norm,
    valid_token_mask, causal)`` when ``norm`` is given) once and replay it on each call."""

    def __init__(self, module: nn.Module, example_x: torch.Tensor,
                 valid_token_mask: Optional[torch.Tensor] = None, causal: bool = False,
                 norm: Optional[nn.LayerNorm] = None, warmup: int = 2):
        if example_x.device.type != "cuda":
            raise RuntimeError("GraphedForward captures GPU work: example_x must be on the GPU")
        self.module, self.norm, self.causal = module, norm, bool(causal)
        self.static_x = example_x.detach().clone()
        self.static_mask = None if valid_token_mask is None else valid_token_mask.detach().clone()
        with torch.inference_mode():
            # warm-up on a side stream: builds the module's derived caches (packed weights) and
            # lets the allocator settle before capture, as graph capture requires
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(max(1, warmup)):
                    self._run()
            torch.cuda.current_stream().wait_stream(side)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.static_out = self._run()
        self._stamp = self._params_stamp()
        # The graph reads the module's derived weight cache (packed / quantised weights) by
        # address. Holding a reference keeps those tensors alive even if the module drops its
        # cache (_apply, load_state_dict), and __call__ refuses to replay once the module's
        # cache entry is no longer the one captured.
        self._cache = self.module.__dict__.get("_mi355_pack")
        # likewise the LayerNorm-folded QKV weights that forward_residual reads
        self._ln_cache = self.module.__dict__.get("_mi355_lnpack")

    def _cache_current(self) -> bool:
        return (self.module.__dict__.get("_mi355_pack") is self._cache
                and self.module.__dict__.get("_mi355_lnpack") is getattr(self, "_ln_cache", None))

    def _params_stamp(self):
        mods = [self.module] + ([self.norm] if self.norm is not None else [])
        return tuple((p.data_ptr(), p._version) for m in mods for p in m.parameters())

    def _run(self) -> torch.Tensor:
        if self.norm is not None:
            return self.module.forward_residual(self.static_x, self.norm, self.static_mask, self.causal)
        return self.module(self.static_x, self.static_mask, self.causal)

    def __call__(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if x.shape != self.static_x.shape or x.dtype != self.static_x.dtype or x.device != self.static_x.device:
            raise ValueError("input does not match the captured shape / dtype / device")
        if (valid_token_mask is None) != (self.static_mask is None):
            raise ValueError("mask presence differs from the captured forward")
        if self._params_stamp() != self._stamp or not self._cache_current():
            raise RuntimeError("the module's parameters or derived weights changed since capture: "
                               "capture again")
        with torch.inference_mode():
            self.static_x.copy_(x)
            if valid_token_mask is not None:
                if valid_token_mask.shape != self.static_mask.shape:
                    raise ValueError("mask shape differs from the captured forward")
                self.static_mask.copy_(valid_token_mask)
            self.graph.replay()
            return self.static_out.clone()
