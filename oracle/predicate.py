"""Elementwise tolerance predicate — test infrastructure only.

Restates ``compare_outputs`` (torch_transformer_benchmark.py:289-356): an element passes when
both values are finite and ``|opt - ref| <= atol`` OR ``|opt - ref| <= rtol * |ref|`` (the OR
is exact; torch.isclose's ``atol + rtol*|ref|`` is deliberately not used, :312-316).
Defaults are the benchmark's CLI defaults atol=2e-3, rtol=2e-2 (:618-619).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch

ATOL = 2e-3
RTOL = 2e-2


@dataclass
class AccuracyResult:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float

    def summary(self) -> str:
        return (f"{'PASS' if self.passed else 'FAIL'} max_abs={self.max_abs_error:.3g} "
                f"max_rel={self.max_relative_error:.3g} failed={self.failed_elements}/"
                f"{self.total_elements} worst={self.worst_index} "
                f"ref={self.reference_at_worst:.6g} opt={self.optimized_at_worst:.6g}")


def compare_outputs(reference: torch.Tensor, optimized: torch.Tensor, rtol: float = RTOL,
                    atol: float = ATOL) -> AccuracyResult:
    if tuple(reference.shape) != tuple(optimized.shape):
        raise AssertionError(f"shape mismatch: baseline={tuple(reference.shape)}, "
                             f"optimized={tuple(optimized.shape)}")
    ref = reference.detach().float().cpu()
    opt = optimized.detach().float().cpu()
    finite = torch.isfinite(ref) & torch.isfinite(opt)
    abs_err = (opt - ref).abs()
    passed = finite & ((abs_err <= atol) | (abs_err <= rtol * ref.abs()))
    failed = int((~passed).sum().item())
    total = ref.numel()
    if total == 0:
        return AccuracyResult(True, 0, 0, 0.0, 0.0, 0.0, (), 0.0, 0.0)
    # NaN errors (non-finite elements) rank worst
    ranked = torch.where(torch.isnan(abs_err), torch.full_like(abs_err, float("inf")), abs_err)
    flat = int(ranked.reshape(-1).argmax().item())
    idx = []
    rem = flat
    for size in reversed(ref.shape):
        idx.append(rem % size)
        rem //= size
    worst = tuple(reversed(idx))
    rel = abs_err / ref.abs().clamp_min(1e-12)
    return AccuracyResult(
        passed=failed == 0,
        total_elements=total,
        failed_elements=failed,
        max_abs_error=float(abs_err.max().item()),
        max_relative_error=float(rel.max().item()),
        mean_abs_error=float(abs_err.mean().item()),
        worst_index=worst,
        reference_at_worst=float(ref[worst].item()) if worst else float(ref.item()),
        optimized_at_worst=float(opt[worst].item()) if worst else float(opt.item()),
    )
