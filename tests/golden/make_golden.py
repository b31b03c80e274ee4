"""Writes the golden fixtures in this directory from the CPU oracle.

The reference ships no test vectors, so these are this build's own: small,
seeded inputs for every hot-path op and the oracle's outputs on them,
committed so that a change to the oracle (or to a kernel) shows up as a
difference from stored data rather than only from another computation.
tests/test_golden_cpu.py checks the oracle against them and
tests/test_gpu_golden.py the HIP kernels.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
for path in (ROOT, Path(__file__).resolve().parent):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

from golden_io import save  # noqa: E402
from oracle import attention as OA  # noqa: E402
from oracle import paged_kv as OK  # noqa: E402
from oracle import pointwise as OP  # noqa: E402
from oracle import sampling as OS  # noqa: E402

HEADS, KV_HEADS, D, BS = 4, 2, 128, 16


def _tables(g, lengths, pool_pages):
    perm = torch.randperm(pool_pages, generator=g)
    blocks, offsets = [], [0]
    for length in lengths:
        pages = math.ceil(length / BS)
        blocks.extend(perm[offsets[-1]:offsets[-1] + pages].tolist())
        offsets.append(offsets[-1] + pages)
    return torch.tensor(blocks, dtype=torch.long), torch.tensor(offsets, dtype=torch.long)


def decode_case() -> dict:
    """Paged decode: a zero-length row, a one-page row, partial last pages,
    query rows out of order (reference paged_decode.cu:92-466)."""
    g = torch.Generator().manual_seed(1001)
    lengths = [37, 0, 70, 16]
    pool = 10
    blocks, offsets = _tables(g, lengths, pool)
    k = torch.randn(pool * BS, KV_HEADS, D, generator=g).to(torch.bfloat16)
    v = torch.randn(pool * BS, KV_HEADS, D, generator=g).to(torch.bfloat16)
    q = torch.randn(len(lengths), HEADS, D, generator=g).to(torch.bfloat16)
    rows = torch.tensor([2, 0, 3, 1], dtype=torch.long)
    lengths_t = torch.tensor(lengths, dtype=torch.long)
    out = torch.zeros_like(q)
    OA.decode_attention(q, k, v, rows, blocks, offsets, lengths_t, BS, D ** -0.5, out)
    return dict(q=q, k=k, v=v, rows=rows, blocks=blocks, offsets=offsets,
                lengths=lengths_t, block_size=BS, scale=D ** -0.5, out=out)


def prefill_case() -> dict:
    """Chunked prefill: a fresh prompt, a chunk with history, a one-token
    chunk (lower-right causal; reference runtime/attention.py:176-285)."""
    g = torch.Generator().manual_seed(1002)
    items = [(40, 40), (70, 17), (33, 1)]
    pool = 11
    blocks, block_offsets = _tables(g, [c for c, _ in items], pool)
    q_offsets = torch.tensor([0] + list(torch.tensor([ql for _, ql in items]).cumsum(0).tolist()),
                             dtype=torch.long)
    context = torch.tensor([c for c, _ in items], dtype=torch.long)
    k = torch.randn(pool * BS, KV_HEADS, D, generator=g).to(torch.bfloat16)
    v = torch.randn(pool * BS, KV_HEADS, D, generator=g).to(torch.bfloat16)
    q = torch.randn(int(q_offsets[-1]), HEADS, D, generator=g).to(torch.bfloat16)
    out = torch.zeros_like(q)
    OA.prefill_attention(q, k, v, q_offsets, blocks, block_offsets, context, BS, D ** -0.5, out)
    return dict(q=q, k=k, v=v, q_offsets=q_offsets, blocks=blocks,
                block_offsets=block_offsets, context_lens=context, block_size=BS,
                scale=D ** -0.5, out=out)


def pointwise_case() -> dict:
    """The C2 chain at small size: RMSNorm, add+RMSNorm, per-head QK-norm +
    RoPE (theta 1e6), the slot-mapped KV write (one slot -1) and SiLU-mul
    (reference kernels/pointwise.cu, kv_store.cu)."""
    g = torch.Generator().manual_seed(1003)
    tokens, hidden, inter, slots_total = 8, 256, 256, 64
    bf = torch.bfloat16
    x = torch.randn(tokens, hidden, generator=g).to(bf)
    res = torch.randn(tokens, hidden, generator=g).to(bf)
    w = (1 + 0.02 * torch.randn(hidden, generator=g)).to(bf)
    qkv = torch.randn(tokens, (HEADS + 2 * KV_HEADS) * D, generator=g).to(bf)
    qw = (1 + 0.02 * torch.randn(D, generator=g)).to(bf)
    kw = (1 + 0.02 * torch.randn(D, generator=g)).to(bf)
    positions = torch.randint(0, 2048, (tokens,), generator=g)
    gate_up = torch.randn(tokens, 2 * inter, generator=g).to(bf)
    slots = torch.randperm(slots_total, generator=g)[:tokens]
    slots[3] = -1
    rms = OP.rms_norm(x, w)
    normed, residual = OP.add_rms_norm(x, res, w)
    q = qkv[:, :HEADS * D].view(tokens, HEADS, D)
    k = qkv[:, HEADS * D:(HEADS + KV_HEADS) * D].view(tokens, KV_HEADS, D)
    v = qkv[:, (HEADS + KV_HEADS) * D:].view(tokens, KV_HEADS, D).contiguous()
    cos, sin = OP.rope_tables(positions, D, 1e6, bf)
    q_out, k_out = OP.qk_norm_rope(q, k, qw, kw, cos, sin)
    k_cache = torch.full((slots_total, KV_HEADS, D), 1.5).to(bf)
    v_cache = torch.full((slots_total, KV_HEADS, D), -2.5).to(bf)
    OK.kv_write(k_cache, v_cache, slots, k_out.contiguous(), v)
    return dict(x=x, res=res, w=w, rms=rms, normed=normed, residual=residual,
                qkv=qkv, qw=qw, kw=kw, positions=positions, cos=cos, sin=sin,
                q_out=q_out, k_out=k_out, slots=slots, k_cache=k_cache, v_cache=v_cache,
                gate_up=gate_up, silu=OP.silu_and_mul(gate_up))


def sampling_case() -> dict:
    """Greedy indices (a tied maximum resolves to the first index) and the
    kept sets of temperature / top-k / top-p rows (reference sampling.py)."""
    g = torch.Generator().manual_seed(1004)
    rows, vocab = 4, 100
    logits = (2 * torch.randn(rows, vocab, generator=g)).to(torch.bfloat16)
    logits[1, 17] = logits[1, 60] = logits[1].float().max() + 1  # tie
    temperature = torch.tensor([1.0, 0.7, 1.3, 0.5], dtype=torch.float32)
    top_k = torch.tensor([0, 5, 20, 1], dtype=torch.long)
    top_p = torch.tensor([0.9, 1.0, 0.5, 1.0], dtype=torch.float32)
    kept = torch.stack([torch.from_numpy(OS.kept_set(logits[r], float(temperature[r]),
                                                     int(top_k[r]), float(top_p[r])))
                        for r in range(rows)])
    return dict(logits=logits, temperature=temperature, top_k=top_k, top_p=top_p,
                greedy=OS.greedy(logits), kept=kept)


CASES = {"decode": decode_case, "prefill": prefill_case, "pointwise": pointwise_case,
         "sampling": sampling_case}


def main() -> None:
    for name, make in CASES.items():
        path = save(name, make())
        print(f"{path.name}: {path.stat().st_size} bytes")


if __name__ == "__main__":
    main()
