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


def assert_within_ulp(actual: torch.Tensor, expected: torch.Tensor,
                      scale: torch.Tensor | None = None, ulps: float = 1.0,
                      max_abs: float = MAX_ABS, mean_rel: float = MEAN_REL) -> None:
    """The bf16 bar widened where one bf16 ulp exceeds it: each element within
    max(max_abs, ulps x ulp(max(|expected|, |scale|))) - rounding flips of
    values above 4, where max abs 2e-2 is sub-ulp (``scale``: the operands'
    magnitude, for rounded sums) - and the mean relative (L1) error within
    ``mean_rel``."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, (a.shape, e.shape)
    assert torch.isfinite(a).all(), "non-finite values in output"
    mag = e.abs() if scale is None else torch.maximum(e.abs(), scale.detach().float().abs())
    ulp = torch.exp2(torch.floor(torch.log2(mag.clamp_min(2.0 ** -126))) - 7)
    allowed = torch.clamp(ulps * ulp, min=max_abs)
    excess = ((a - e).abs() / allowed).max().item() if a.numel() else 0.0
    assert excess <= 1.0, f"error {excess:.2f}x max({max_abs}, {ulps} bf16 ulp)"
    rel = ((a - e).abs().sum() / e.abs().sum().clamp_min(1e-30)).item()
    assert rel <= mean_rel, f"mean rel err {rel:.3e} > {mean_rel}"


def bf16_ulp(x: float) -> float:
    """One bf16 unit in the last place at |x| (7 fraction bits)."""
    x = abs(float(x))
    if x == 0.0:
        return 2.0 ** -133
    return 2.0 ** (math.floor(math.log2(x)) - 7)


def build_model(cfg, weights, device):
    """Our Qwen3ForCausalLM for an oracle TinyQwen3 config, loaded with the
    oracle's packed weight dict through the checkpoint weight routes."""
    from tinyvllm.models.qwen3 import Qwen3Config, Qwen3ForCausalLM

    qcfg = Qwen3Config.from_dict(dict(
        model_type="qwen3", vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
        max_position_embeddings=cfg.max_position_embeddings, rope_theta=cfg.rope_theta,
        tie_word_embeddings=cfg.tie_word_embeddings))
    model = Qwen3ForCausalLM(qcfg, device=device, dtype=torch.bfloat16)
    q = cfg.num_attention_heads * cfg.head_dim
    kv = cfg.num_key_value_heads * cfg.head_dim
    for name, tensor in weights.items():
        t = tensor.to(device)
        if name.endswith("qkv_proj.weight"):
            base = name[:-len("qkv_proj.weight")]
            model.load_weight(base + "q_proj.weight", t[:q])
            model.load_weight(base + "k_proj.weight", t[q:q + kv])
            model.load_weight(base + "v_proj.weight", t[q + kv:])
        elif name.endswith("gate_up_proj.weight"):
            base = name[:-len("gate_up_proj.weight")]
            model.load_weight(base + "gate_proj.weight", t[:cfg.intermediate_size])
            model.load_weight(base + "up_proj.weight", t[cfg.intermediate_size:])
        else:
            model.load_weight(name, t)
    return model.eval()
