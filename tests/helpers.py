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


class ManualBatches:
    """Hand-rolled PreparedBatch builder for runner tests: each sequence owns
    consecutive slices of a shuffled block pool; prompts are prefilled in
    chunks, then every step decodes one token per sequence."""

    def __init__(self, prompts, *, block_size, num_blocks, seed=0):
        g = torch.Generator().manual_seed(seed)
        perm = torch.randperm(num_blocks, generator=g).tolist()
        self.bs, self.num_blocks = block_size, num_blocks
        per = num_blocks // len(prompts)
        self.tables = [perm[i * per:(i + 1) * per] for i in range(len(prompts))]
        self.tokens = [list(p) for p in prompts]
        self.done = [0] * len(prompts)  # tokens already in the cache
        self.plan = 0

    def _batch(self, items):
        from tinyvllm.batch import PreparedBatch, StepMode
        from tinyvllm.request import SamplingParams

        ids, pos, qoff, before, qlen, after, sidx, srid = [], [], [0], [], [], [], [], []
        tids, toff, slots = [], [0], []
        for seq, n, sample in items:
            start = self.done[seq]
            ids += self.tokens[seq][start:start + n]
            pos += list(range(start, start + n))
            qoff.append(len(ids))
            before.append(start)
            qlen.append(n)
            after.append(start + n)
            table = self.tables[seq][: -(-(start + n) // self.bs)]
            tids += table
            toff.append(len(tids))
            slots += [table[p // self.bs] * self.bs + p % self.bs for p in range(start, start + n)]
            if sample:
                sidx.append(len(ids) - 1)
                srid.append(seq)
        self.plan += 1
        greedy = SamplingParams(max_new_tokens=1 << 20)
        return PreparedBatch(
            plan_id=self.plan, mode=StepMode.MIXED, input_ids=tuple(ids), positions=tuple(pos),
            q_offsets=tuple(qoff), context_lens_before=tuple(before), query_lens=tuple(qlen),
            context_lens_after=tuple(after), sample_token_indices=tuple(sidx),
            sample_request_ids=tuple(srid), sampling_params=(greedy,) * len(sidx),
            kv_block_size=self.bs, kv_num_blocks=self.num_blocks, kv_block_table_ids=tuple(tids),
            kv_block_table_offsets=tuple(toff), kv_slot_mapping=tuple(slots),
            request_ids=tuple(seq for seq, _, _ in items),
        )

    def prefill(self, seq, n, sample):
        batch = self._batch([(seq, n, sample)])
        return batch

    def commit(self, items, tokens):
        """Mark items' tokens as cached and append sampled tokens."""
        it = iter(tokens)
        for seq, n, sample in items:
            self.done[seq] += n
            if sample:
                self.tokens[seq].append(int(next(it)))

    def step(self, items):
        return self._batch(items)
