"""Chunk-wise (streamed) fp32 restatement of the attention core — test infrastructure only.

Restates ``streamed_attention`` (Project/tools/shape14_eval.py:201-236): per (batch, head) and
per query chunk, loop over key chunks (up to the chunk end when causal, :221), compute fp32
scores (:223), apply the causal mask (:224-227), update the running max / sum / accumulator
online (:228-233) and normalise (:234). The S x S table is never formed, so this oracle checks
the long-sequence configurations on sampled query rows.
"""
from __future__ import annotations

from typing import Optional

import torch


def streamed_attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                            causal: bool = False, q_chunk: int = 2048, k_chunk: int = 8192,
                            q_index: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Online-softmax attention on [B, H, S, hd] fp32 CPU tensors.

    ``q_index`` optionally selects the absolute positions of the given query rows (so a sample
    of rows ``q = full_q[:, :, idx]`` is masked causally at its true positions); by default the
    query rows are positions 0..S_q-1. Chunk sizes default to the reference's 2048 / 8192
    (shape14_eval.py:239).
    """
    B, H, S_q, D = q.shape
    S_k = k.shape[2]
    if q_index is None:
        q_index = torch.arange(S_q)
    out = torch.empty((B, H, S_q, v.shape[3]), dtype=torch.float32)
    for b in range(B):
        for h in range(H):
            qb, kb, vb = q[b, h].float(), k[b, h].float(), v[b, h].float()
            for qs in range(0, S_q, q_chunk):
                qe = min(qs + q_chunk, S_q)
                pos = q_index[qs:qe]
                m = torch.full((qe - qs,), float("-inf"))
                l = torch.zeros(qe - qs)
                acc = torch.zeros(qe - qs, v.shape[3])
                k_end = min(int(pos.max()) + 1, S_k) if causal else S_k
                for ks in range(0, k_end, k_chunk):
                    ke = min(ks + k_chunk, k_end)
                    scores = qb[qs:qe] @ kb[ks:ke].T * scale
                    if causal:
                        kidx = torch.arange(ks, ke)[None, :]
                        scores = scores.masked_fill(kidx > pos[:, None], float("-inf"))
                    m_new = torch.maximum(m, scores.amax(dim=1))
                    # rows with no admissible key yet keep m = -inf; guard the 0 * inf case
                    m_safe = torch.where(torch.isinf(m_new), torch.zeros_like(m_new), m_new)
                    alpha = torch.exp(m - m_safe)
                    p = torch.exp(scores - m_safe[:, None])
                    l = l * alpha + p.sum(dim=1)
                    acc = acc * alpha[:, None] + p @ vb[ks:ke]
                    m = m_new
                out[b, h, qs:qe] = acc / l[:, None]
    return out
