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

import gc
import weakref
from collections import OrderedDict
from typing import Optional

import torch
import torch.nn as nn


def version_of(t: torch.Tensor) -> int:
    """The tensor's in-place version counter; -1 for inference tensors, which keep none (their
    in-place updates under torch.inference_mode cannot be seen: caches keyed on them rely on
    load_state_dict / _apply invalidating explicitly)."""
    return -1 if t.is_inference() else t._version


def _record(graph: "torch.cuda.CUDAGraph", fn):
    """``fn()`` recorded into ``graph``; returns its result. No other graph may be destroyed
    while this one records (freeing a graph and its memory pool are calls a capture forbids):
    unreachable objects are collected first, and the garbage collector stays off until the
    capture ends."""
    gc.collect()
    gc_was_on = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph):
            return fn()
    finally:
        if gc_was_on:
            gc.enable()


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
            self.static_out = _record(self.graph, self._run)
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
        return tuple((p.data_ptr(), version_of(p)) for m in mods for p in m.parameters())

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


# Input elements at or below which a module's forward replays a captured graph (AutoGraph): an
# attention block of 128 x 256 (the fp32 configuration) spends ~18 us on the GPU against ~70 us
# of host work per eager forward, and a 4-layer fp16 model of 128 x 128 x 128 (2^21 elements)
# 0.41 ms against 0.50 ms of host work. Larger inputs keep the GPU busier than the host; the
# replay's input copy and output clone grow with the input.
AUTO_GRAPH_MAX_ELEMS = 1 << 22


# Parameter or submodule registrations anywhere in the process (construction, replacement by
# assignment) bump this epoch, so a capture can tell in O(1) that the module it read may have
# other parameter objects now; in-place updates, load_state_dict and _apply are seen through the
# parameters' version counters, data pointers and the derived-weight caches.
_REGISTRATION_EPOCH = [0]


def _bump_epoch(*_args) -> None:
    _REGISTRATION_EPOCH[0] += 1


_REGISTRATION_HOOKS = (
    torch.nn.modules.module.register_module_parameter_registration_hook(_bump_epoch),
    torch.nn.modules.module.register_module_module_registration_hook(_bump_epoch),
)


def _derived_caches(module: nn.Module):
    """(submodule, attribute, object) of every derived-weight cache the forward reads by address
    (module attributes named _mi355_*: packed, LayerNorm-folded and quantised weights)."""
    return [(m, k, v) for m in module.modules() for k, v in m.__dict__.items()
            if k.startswith("_mi355_")]


def _switch_modules(module: nn.Module):
    """The submodules whose plain attributes steer the forward: those listing them in
    ``graph_switches`` (the attention modules' dtype / fold / key-bound switches) and the
    LayerNorms (eps)."""
    return [m for m in module.modules()
            if getattr(type(m), "graph_switches", None) or isinstance(m, nn.LayerNorm)]


def _switch_values(mods) -> tuple:
    """Current values of those attributes (instance or class), in module order (a module that no
    longer exists gives a value no recorded one equals)."""
    return tuple((_GONE,) if m is None else (m.eps,) if isinstance(m, nn.LayerNorm)
                 else tuple(getattr(m, a) for a in type(m).graph_switches) for m in mods)


_GONE = object()


def _alive(refs) -> list:
    """The modules behind weak references (None for a module that no longer exists)."""
    return [r() for r in refs]


def _cache_is(m, k: str, v) -> bool:
    return m is not None and m.__dict__.get(k) is v


class _Capture:
    """One captured forward: static input buffers, the graph, its output, and what it read."""

    def __init__(self, module: nn.Module, fn, x: torch.Tensor, mask: Optional[torch.Tensor]):
        self.static_x = x.detach().clone()
        self.static_mask = None if mask is None else mask.detach().clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                fn(self.static_x, self.static_mask)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        self.static_out = _record(self.graph, lambda: fn(self.static_x, self.static_mask))
        self.epoch = _REGISTRATION_EPOCH[0]
        self.cls = type(module)
        self.params = list(module.parameters())
        self.tracked = [p for p in self.params if not p.is_inference()]
        self.ptrs = [p.data_ptr() for p in self.params]
        self.vers = [p._version for p in self.tracked]
        # the derived weights are held (the graph reads them); the modules only weakly, so a
        # module and its captures form no reference cycle and a dropped module's graphs are
        # freed at once rather than by a later garbage collection
        self.caches = [(weakref.ref(m), k, v) for m, k, v in _derived_caches(module)]
        self.switch_mods = [weakref.ref(m) for m in _switch_modules(module)]
        self.switches = _switch_values(_alive(self.switch_mods))
        self.last = (None, None)                # (weak reference, version) of the inputs copied

    def current(self, module: nn.Module) -> bool:
        """The module still has the parameters, values, derived weights and switches (dtype,
        fold and key-bound attributes of its attention modules, LayerNorm eps) the graph was
        recorded with (the parameter and module lists are walked only when a registration
        happened somewhere: that walk costs ~7 us for an attention block, ~70 us for a 4-layer
        model, per call)."""
        if type(module) is not self.cls:
            return False
        if _REGISTRATION_EPOCH[0] != self.epoch:
            now = list(module.parameters())
            if len(now) != len(self.params) or any(a is not b for a, b in zip(now, self.params)):
                return False
            mods = _switch_modules(module)
            if len(mods) != len(self.switch_mods) or any(a is not b() for a, b in zip(mods, self.switch_mods)):
                return False
            self.epoch = _REGISTRATION_EPOCH[0]
        return ([p._version for p in self.tracked] == self.vers
                and [p.data_ptr() for p in self.params] == self.ptrs
                and all(_cache_is(m(), k, v) for m, k, v in self.caches)
                and _switch_values(_alive(self.switch_mods)) == self.switches)

    def replay(self, x: torch.Tensor, mask: Optional[torch.Tensor]) -> torch.Tensor:
        # The copy is skipped when the caller hands back the same tensor objects with unchanged
        # version counters (the benchmark's timing loop passes one x throughout); any in-place
        # torch update of x or the mask (or of a view of them) bumps the counter. Inference
        # tensors keep no version counter, so they are always copied. Writes that bypass the
        # counter (through x.data, or by a kernel given x's raw pointer) are not seen: callers
        # that update inputs that way set the module's auto_graph to False.
        ref, ver = self.last
        tracked = not x.is_inference() and (mask is None or not mask.is_inference())
        key = (x._version, None if mask is None else mask._version) if tracked else None
        same = (tracked and ref is not None and ref[0]() is x
                and (mask is None) == (ref[1] is None)
                and (mask is None or ref[1]() is mask) and ver == key)
        if not same:
            self.static_x.copy_(x)
            if mask is not None:
                self.static_mask.copy_(mask)
            self.last = ((weakref.ref(x), None if mask is None else weakref.ref(mask)), key)
        self.graph.replay()
        return self.static_out.clone()


class AutoGraph:
    """Graph replay inside a module's forward for launch-bound calls (the reference's route:
    the first forward eager, the second captured, later ones replayed,
    Project/submission/dispatcher_region.py:1220-1363).

    ``__call__(module, fn, x, mask, extra)`` returns ``fn(x, mask)``'s result from a replay, or
    None when the caller should run eagerly: a CPU or large input (more than
    AUTO_GRAPH_MAX_ELEMS elements), autograd enabled, a capture already in progress (the caller's
    own graph then records the eager kernels), the first call of an input signature, or a
    capture that no longer matches the module (its parameters, derived weights or switches --
    the attention modules' ``graph_switches`` attributes, LayerNorm eps -- changed: the graph is
    dropped and the next call captures again). The signature is x's and the mask's
    shape, dtype, device and strides plus ``extra`` (e.g. the causal flag); up to ``max_graphs``
    signatures keep their graphs. Outputs are fresh tensors (a clone of the graph's output)."""

    def __init__(self, max_graphs: int = 4):
        self.max_graphs = max_graphs
        self.entries: "OrderedDict[tuple, dict]" = OrderedDict()

    # copies of a module (deepcopy, pickling) start without captures: a graph belongs to the
    # module and buffers it was recorded with
    def __deepcopy__(self, memo):
        return AutoGraph(self.max_graphs)

    def __getstate__(self):
        return {"max_graphs": self.max_graphs}

    def __setstate__(self, state):
        self.__init__(state["max_graphs"])

    @staticmethod
    def applies(x: torch.Tensor) -> bool:
        return (x.is_cuda and x.numel() <= AUTO_GRAPH_MAX_ELEMS and not torch.is_grad_enabled()
                and not torch.cuda.is_current_stream_capturing())

    def __call__(self, module: nn.Module, fn, x: torch.Tensor, mask: Optional[torch.Tensor],
                 extra=()) -> Optional[torch.Tensor]:
        if not self.applies(x) or (mask is not None and not mask.is_cuda):
            return None
        key = (tuple(x.shape), x.dtype, x.device, tuple(x.stride()),
               None if mask is None else (tuple(mask.shape), mask.dtype, tuple(mask.stride())),
               extra)
        e = self.entries.get(key)
        if e is None:
            e = self.entries[key] = {"calls": 0, "cap": None, "failed": False}
            while len(self.entries) > self.max_graphs:
                self.entries.popitem(last=False)
        else:
            self.entries.move_to_end(key)
        if e["failed"]:
            return None
        cap = e["cap"]
        if cap is not None and not cap.current(module):
            e["cap"], e["calls"], cap = None, 0, None
        if cap is None:
            e["calls"] += 1
            if e["calls"] < 2:
                return None
            try:
                cap = e["cap"] = _Capture(module, fn, x, mask)
            except RuntimeError:
                e["failed"] = True   # not capturable here: this signature stays eager
                return None
        return cap.replay(x, mask)
