"""Token sampler (reference: tinyvllm/sampling.py:1-192).

Greedy rows use the argmax kernel; temperature / top-k / top-p rows use the
radix-select sampling kernel, all rows of a step in one launch. Each request
owns a sample counter that selects its Philox noise for the next draw, so a
request's stream is reproducible from its seed (the reference keeps a
per-request torch.Generator instead, sampling.py:167-185).
"""
from __future__ import annotations

from collections.abc import Sequence

import torch

from tinyvllm.request import SamplingParams


class Sampler:
    def __init__(self) -> None:
        self._counters: dict[int, tuple[int, int]] = {}  # request -> (seed, draws)

    def counters(self, sampling_params: Sequence[SamplingParams],
                 request_ids: Sequence[int]) -> list[int]:
        """Draw counters for this step; advances each request's stream."""
        out = []
        for params, request_id in zip(sampling_params, request_ids):
            seed, draws = self._counters.get(request_id, (params.seed, 0))
            if seed != params.seed:
                draws = 0
            out.append(draws)
            self._counters[request_id] = (params.seed, draws + 1)
        return out

    @torch.inference_mode()
    def sample(self, logits: torch.Tensor, sampling_params: Sequence[SamplingParams],
               request_ids: Sequence[int]) -> torch.Tensor:
        from tinyvllm.runtime.runner import sample_rows

        rows = logits.shape[0]
        if len(sampling_params) != rows:
            raise ValueError("sampling_params must align with logits rows")
        if len(request_ids) != rows:
            raise ValueError("request_ids must align with logits rows")
        if rows == 0:
            return torch.empty((0,), dtype=torch.long, device=logits.device)
        return sample_rows(logits, sampling_params,
                           self.counters(sampling_params, request_ids))

    def release(self, request_id: int) -> None:
        self._counters.pop(request_id, None)

    def clear(self) -> None:
        self._counters.clear()


# The reference's name for its sampler class.
TorchSampler = Sampler
