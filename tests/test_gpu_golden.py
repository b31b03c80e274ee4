"""HIP kernels against the committed golden fixtures (tests/golden): the
stored inputs through the C-ABI library, compared with the stored oracle
outputs at the parity bar (bit-exact for the KV write, the slots left alone
and greedy indices; max abs <= 2e-2 and mean relative <= 1e-3 for bf16)."""
import sys
from pathlib import Path

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))

from golden_io import load  # noqa: E402
from helpers import assert_bf16_close  # noqa: E402
from test_gpu_kernels import _Cache  # noqa: E402

pytestmark = pytest.mark.gpu


def test_decode_matches_fixture(device):
    from tinyvllm.kernels.paged_decode import decode_workspace_bytes, paged_decode_attention
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    f = load("decode")
    bs = int(f["block_size"])
    cache = _Cache(f["k"].to(device), f["v"].to(device), bs)
    meta = SingleQueryMetadata(f["rows"].to(device), f["blocks"].to(device),
                               f["offsets"].to(device), f["lengths"].to(device),
                               int(f["lengths"].max()))
    q = f["q"].to(device)
    ws = torch.empty(max(16, decode_workspace_bytes(q.shape[0], q.shape[1], 2, 128,
                                                    int(f["lengths"].max()), bs)),
                     dtype=torch.uint8, device=device)
    out = torch.full_like(q, 7.0)
    paged_decode_attention(q, cache, 0, meta, out, scale=float(f["scale"]), workspace=ws)
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), f["out"])
    assert torch.count_nonzero(out[int(f["rows"][1])]) == 0  # zero-length row


def test_prefill_matches_fixture(device):
    from tinyvllm.kernels.paged_prefill import paged_prefill_attention
    from tinyvllm.runtime.contracts import MultiQueryMetadata

    f = load("prefill")
    cache = _Cache(f["k"].to(device), f["v"].to(device), int(f["block_size"]))
    q_lens = f["q_offsets"][1:] - f["q_offsets"][:-1]
    meta = MultiQueryMetadata(f["q_offsets"].to(device), f["blocks"].to(device),
                              f["block_offsets"].to(device), f["context_lens"].to(device),
                              max_query_len=int(q_lens.max()))
    out = torch.zeros(f["q"].shape, dtype=torch.bfloat16, device=device)
    paged_prefill_attention(f["q"].to(device), cache, 0, meta, out, scale=float(f["scale"]))
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), f["out"])


def test_pointwise_chain_matches_fixture(device):
    from tinyvllm.kernels.kv_store import store_kv
    from tinyvllm.kernels.pointwise import add_rms_norm, qk_norm_rope, rms_norm, silu_and_mul

    f = load("pointwise")
    g = {k: v.to(device) for k, v in f.items()}
    assert_bf16_close(rms_norm(g["x"], g["w"]).cpu(), f["rms"])
    normed, residual = add_rms_norm(g["x"], g["res"], g["w"])
    assert_bf16_close(normed.cpu(), f["normed"])
    assert torch.equal(residual.cpu(), f["residual"])
    heads, kv_heads, d = 4, 2, 128
    qkv = g["qkv"]
    q = qkv[:, :heads * d].view(-1, heads, d)
    k = qkv[:, heads * d:(heads + kv_heads) * d].view(-1, kv_heads, d)
    v = qkv[:, (heads + kv_heads) * d:].view(-1, kv_heads, d)
    q_out, k_out = qk_norm_rope(q, k, g["qw"], g["kw"], g["cos"], g["sin"])
    assert_bf16_close(q_out.cpu(), f["q_out"])
    assert_bf16_close(k_out.cpu(), f["k_out"])
    # The write itself is bit-exact: store the fixture's own rotated K.
    cache = _Cache(torch.full_like(g["k_cache"], 1.5), torch.full_like(g["v_cache"], -2.5), 16)
    store_kv(cache, 0, g["slots"], g["k_out"], v)
    torch.cuda.synchronize()
    assert torch.equal(cache.key[0].cpu(), f["k_cache"])
    assert torch.equal(cache.value[0].cpu(), f["v_cache"])
    assert_bf16_close(silu_and_mul(g["gate_up"]).cpu(), f["silu"])


def test_sampling_matches_fixture(device):
    from tinyvllm.kernels.sampling import argmax, sample

    f = load("sampling")
    logits = f["logits"].to(device)
    assert torch.equal(argmax(logits).cpu(), f["greedy"])
    rows = logits.shape[0]
    temperature, top_k, top_p = (f[n].to(device) for n in ("temperature", "top_k", "top_p"))
    seeds = torch.arange(rows, dtype=torch.long, device=device)
    for step in range(64):  # every draw stays in the oracle's kept set
        counters = torch.full((rows,), step, dtype=torch.long, device=device)
        drawn = sample(logits, temperature, top_k, top_p, seeds, counters).cpu()
        for r in range(rows):
            assert bool(f["kept"][r][drawn[r]]), (step, r, int(drawn[r]))
    greedy = torch.zeros(rows, dtype=torch.float32, device=device)
    drawn = sample(logits, greedy, top_k, top_p, seeds, counters).cpu()
    assert torch.equal(drawn, f["greedy"])  # temperature 0 is greedy
