"""Sampling restated on the CPU (test infrastructure only).

Reference: tinyvllm/sampling.py:42-43 (greedy argmax) and :75-164
(_sample_batch): s = (logits.float() - rowmax) / T; optional top-k; stable
descending sort; softmax; remove tokens whose preceding cumulative
probability exceeds top_p (the crossing token stays); argmax(p / E).
"""
from __future__ import annotations

import numpy as np
import torch


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """sampling.py:42-43: first index of the row maximum."""
    return logits.float().argmax(dim=-1)


def kept_set(logits_row: torch.Tensor, temperature: float, top_k: int,
             top_p: float) -> np.ndarray:
    """Boolean mask of the tokens that may be sampled, in float64.

    Order is (score descending, index ascending) -- the stable sort of
    sampling.py:123-131; top-k ties are broken the same way."""
    x = logits_row.double().numpy()
    s = (x - x.max()) / temperature
    vocab = s.shape[0]
    order = np.lexsort((np.arange(vocab), -s))  # by -s, then index
    keep = np.zeros(vocab, dtype=bool)
    cand = order
    if 0 < top_k < vocab:
        cand = order[:top_k]
    if top_p < 1.0:
        p = np.exp(s[cand] - s[cand].max())
        p = p / p.sum()
        before = np.concatenate([[0.0], np.cumsum(p)[:-1]])
        cand = cand[before <= top_p]
    keep[cand] = True
    return keep


def sample_with_noise(logits_row: torch.Tensor, temperature: float, top_k: int,
                      top_p: float, noise: np.ndarray) -> int:
    """sampling.py:141-163 given explicit Exp(1) noise: argmax over the kept
    set of p_i / E_i (computed as s_i - log E_i)."""
    keep = kept_set(logits_row, temperature, top_k, top_p)
    x = logits_row.double().numpy()
    s = (x - x.max()) / temperature
    key = np.where(keep, s - np.log(noise), -np.inf)
    return int(np.argmax(key))
