"""Sampling kernels: greedy argmax and temperature / top-k / top-p.

Reference: tinyvllm/sampling.py:42-43 (greedy ``logits.argmax(-1)``) and
:75-164 (``TorchSampler._sample_batch``).
"""
from __future__ import annotations

import torch

from tinyvllm.kernels._extension import (
    check, dtype_code, load_kernels, require_gpu, stream_of,
)


def _check_logits(logits: torch.Tensor) -> None:
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise RuntimeError("logits must be [rows, vocab] with unit last stride")
    if logits.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise RuntimeError("logits must be float16, bfloat16 or float32")


def argmax(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """First index of each row's maximum (NaN counts as the maximum)."""
    lib = load_kernels()
    device = require_gpu(logits)
    _check_logits(logits)
    rows, vocab = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.long, device=device)
    if rows:
        check(lib.tvllm_argmax(
            logits.data_ptr(), rows, vocab, logits.stride(0), out.data_ptr(),
            dtype_code(logits.dtype), stream_of(device),
        ))
    return out


def sample(
    logits: torch.Tensor,
    temperature: torch.Tensor,
    top_k: torch.Tensor,
    top_p: torch.Tensor,
    seeds: torch.Tensor,
    counters: torch.Tensor,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-row temperature / top-k / top-p exponential-race sampling.

    All per-row parameters are GPU tensors: ``temperature`` float32 (0 means
    greedy), ``top_k`` int64 (0 means off), ``top_p`` float32 in (0, 1],
    ``seeds`` int64, ``counters`` int64 (the number of tokens the request has
    sampled so far, which selects its noise for this step)."""
    lib = load_kernels()
    device = require_gpu(logits, temperature, top_k, top_p, seeds, counters)
    _check_logits(logits)
    rows, vocab = logits.shape
    for tensor, dtype in ((temperature, torch.float32), (top_k, torch.long),
                          (top_p, torch.float32), (seeds, torch.long),
                          (counters, torch.long)):
        if tensor.dtype != dtype or tensor.shape != (rows,) or not tensor.is_contiguous():
            raise RuntimeError("sampling parameters must be contiguous [rows] tensors")
    if out is None:
        out = torch.empty(rows, dtype=torch.long, device=device)
    if rows:
        # Per-span argmax partials: the row scan is spread over many
        # workgroups (an allocation from torch's pool, graph-capturable).
        size = lib.tvllm_sample_workspace_size(rows, vocab)
        workspace = torch.empty(size, dtype=torch.uint8, device=device) if size else None
        check(lib.tvllm_sample(
            logits.data_ptr(), rows, vocab, logits.stride(0), temperature.data_ptr(),
            top_k.data_ptr(), top_p.data_ptr(), seeds.data_ptr(), counters.data_ptr(),
            out.data_ptr(), None if workspace is None else workspace.data_ptr(), size,
            dtype_code(logits.dtype), stream_of(device),
        ))
    return out


def resolve_tokens(tokens: torch.Tensor, src: torch.Tensor, prev: torch.Tensor) -> torch.Tensor:
    """In place: ``tokens[i] = prev[src[i]]`` wherever ``0 <= src[i] < len(prev)``.

    ``src[i] = -1`` keeps the uploaded token. Lets a step's input ids name the
    previous step's sampled tokens while those are still on the device (the
    reference uploads host token ids only: tinyvllm/runtime/inputs.py:88-111)."""
    lib = load_kernels()
    device = require_gpu(tokens, src, prev)
    for tensor in (tokens, src, prev):
        if tensor.dtype != torch.long or tensor.dim() != 1 or not tensor.is_contiguous():
            raise RuntimeError("resolve_tokens takes contiguous 1-D int64 tensors")
    if src.shape != tokens.shape:
        raise RuntimeError("src must have one entry per token")
    check(lib.tvllm_resolve_tokens(tokens.data_ptr(), src.data_ptr(), prev.data_ptr(),
                                   tokens.numel(), prev.numel(), stream_of(device)))
    return tokens
