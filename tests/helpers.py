"""Tolerance checks and seeded synthetic inputs shared by the tests."""
from __future__ import annotations

import math

import torch

# Tolerances stated by the north star for floating-point outputs in bf16:
# max abs err <= 2e-2 and mean relative error (L1 ratio) <= 1e-3.
MAX_ABS = 2e-2
MEAN_REL = 1e-3


def assert_bf16_close(actual: torch.Tensor, expected: torch.Tensor,
                      max_abs: float = MAX_ABS, mean_rel: float = MEAN_REL) -> None:
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, (a.shape, e.shape)
    assert torch.isfinite(a).all(), "non-finite values in output"
    diff = (a - e).abs()
    worst = diff.max().item() if diff.numel() else 0.0
    rel = (diff.sum() / e.abs().sum().clamp_min(1e-30)).item() if diff.numel() else 0.0
    assert worst <= max_abs, f"max abs err {worst:.3e} > {max_abs}"
    assert rel <= mean_rel, f"mean rel err {rel:.3e} > {mean_rel}"




def paged_decode_case(*, seed: int, batch: int, heads: int, kv_heads: int,
                      head_dim: int = 128, block_size: int = 16,
                      pool_blocks: int = 1024, min_len: int = 64,
                      max_len: int = 1024, lengths: list[int] | None = None,
                      dtype: torch.dtype = torch.bfloat16):
    """The C1 recipe: per-row lengths ~ U[min_len, max_len] from the seed,
    block ids = consecutive slices of randperm(pool_blocks), q/k/v ~ N(0, 1),
    scale 1/sqrt(head_dim). CPU tensors."""
    g = torch.Generator().manual_seed(seed)
    if lengths is None:
        lengths = torch.randint(min_len, max_len + 1, (batch,), generator=g).tolist()
    pages = [math.ceil(length / block_size) for length in lengths]
    assert sum(pages) <= pool_blocks
    perm = torch.randperm(pool_blocks, generator=g)
    blocks, offsets = [], [0]
    for p in pages:
        blocks.extend(perm[offsets[-1]:offsets[-1] + p].tolist())
        offsets.append(offsets[-1] + p)
    slots = pool_blocks * block_size
    k = torch.randn(slots, kv_heads, head_dim, generator=g).to(dtype)
    v = torch.randn(slots, kv_heads, head_dim, generator=g).to(dtype)
    q = torch.randn(batch, heads, head_dim, generator=g).to(dtype)
    return dict(
        q=q, k=k, v=v,
        rows=torch.arange(batch, dtype=torch.long),
        blocks=torch.tensor(blocks, dtype=torch.long),
        offsets=torch.tensor(offsets, dtype=torch.long),
        lengths=torch.tensor(lengths, dtype=torch.long),
        block_size=block_size, scale=head_dim ** -0.5,
    )
