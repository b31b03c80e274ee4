"""The CPU oracle against the committed golden fixtures (tests/golden).

Integer results (slots written, greedy indices, kept sets) must match bit
for bit; floating-point outputs, recomputed here by the same torch CPU
operations, must match to within one bf16 ulp of their scale (a later
torch may order a reduction differently)."""
import sys
from pathlib import Path

import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))

from golden_io import load  # noqa: E402
from helpers import assert_within_ulp  # noqa: E402
from oracle import attention as OA  # noqa: E402
from oracle import paged_kv as OK  # noqa: E402
from oracle import pointwise as OP  # noqa: E402
from oracle import sampling as OS  # noqa: E402


def _close(actual, expected):
    assert actual.dtype == expected.dtype and actual.shape == expected.shape
    assert_within_ulp(actual, expected, ulps=1.0)


def test_decode_fixture():
    f = load("decode")
    out = torch.zeros_like(f["q"])
    OA.decode_attention(f["q"], f["k"], f["v"], f["rows"], f["blocks"], f["offsets"],
                        f["lengths"], int(f["block_size"]), float(f["scale"]), out)
    _close(out, f["out"])
    assert torch.count_nonzero(out[f["rows"][1]]) == 0  # the zero-length row


def test_prefill_fixture():
    f = load("prefill")
    out = torch.zeros_like(f["q"])
    OA.prefill_attention(f["q"], f["k"], f["v"], f["q_offsets"], f["blocks"],
                         f["block_offsets"], f["context_lens"], int(f["block_size"]),
                         float(f["scale"]), out)
    _close(out, f["out"])


def test_pointwise_fixture():
    f = load("pointwise")
    _close(OP.rms_norm(f["x"], f["w"]), f["rms"])
    normed, residual = OP.add_rms_norm(f["x"], f["res"], f["w"])
    _close(normed, f["normed"])
    assert torch.equal(residual, f["residual"])  # one rounding of x + res
    heads, kv_heads, d = 4, 2, 128
    qkv = f["qkv"]
    q = qkv[:, :heads * d].view(-1, heads, d)
    k = qkv[:, heads * d:(heads + kv_heads) * d].view(-1, kv_heads, d)
    v = qkv[:, (heads + kv_heads) * d:].view(-1, kv_heads, d).contiguous()
    cos, sin = OP.rope_tables(f["positions"], d, 1e6, torch.bfloat16)
    assert torch.equal(cos, f["cos"]) and torch.equal(sin, f["sin"])
    q_out, k_out = OP.qk_norm_rope(q, k, f["qw"], f["kw"], cos, sin)
    _close(q_out, f["q_out"])
    _close(k_out, f["k_out"])
    k_cache = torch.full_like(f["k_cache"], 1.5)
    v_cache = torch.full_like(f["v_cache"], -2.5)
    OK.kv_write(k_cache, v_cache, f["slots"], f["k_out"].contiguous(), v)
    assert torch.equal(k_cache, f["k_cache"]) and torch.equal(v_cache, f["v_cache"])
    _close(OP.silu_and_mul(f["gate_up"]), f["silu"])


def test_sampling_fixture():
    f = load("sampling")
    assert torch.equal(OS.greedy(f["logits"]), f["greedy"])
    assert int(f["greedy"][1]) == 17  # the tied maximum: first index
    for r in range(f["logits"].shape[0]):
        kept = OS.kept_set(f["logits"][r], float(f["temperature"][r]), int(f["top_k"][r]),
                           float(f["top_p"][r]))
        assert torch.equal(torch.from_numpy(kept), f["kept"][r])
    assert int(f["kept"][3].sum()) == 1 and bool(f["kept"][3][f["greedy"][3]])  # top-k 1


@pytest.mark.parametrize("name", ["decode", "prefill", "pointwise", "sampling"])
def test_fixtures_are_plain_arrays(name):
    """Fixtures load without unpickling and hold finite values."""
    for key, value in load(name).items():
        if value.is_floating_point():
            assert torch.isfinite(value.float()).all(), key


def test_attention_fixtures_match_the_float64_textbook():
    """The stored attention outputs against an independent computation: the
    loop-form softmax in float64 over the rows the block tables name."""
    f = load("decode")
    bs = int(f["block_size"])
    for r in range(f["rows"].numel()):
        length = int(f["lengths"][r])
        if length == 0:
            continue
        table = f["blocks"][int(f["offsets"][r]):int(f["offsets"][r + 1])]
        slots = OK.read_slots(table, length, bs)
        row = int(f["rows"][r])
        ref = OA.textbook_attention_f64(f["q"][row:row + 1], f["k"][slots], f["v"][slots],
                                        float(f["scale"]))
        assert_within_ulp(f["out"][row:row + 1], ref.to(torch.bfloat16), ulps=1.0)
    f = load("prefill")
    bs = int(f["block_size"])
    for i in range(f["context_lens"].numel()):
        start, end = int(f["q_offsets"][i]), int(f["q_offsets"][i + 1])
        ctx = int(f["context_lens"][i])
        table = f["blocks"][int(f["block_offsets"][i]):int(f["block_offsets"][i + 1])]
        slots = OK.read_slots(table, ctx, bs)
        ref = OA.textbook_attention_f64(f["q"][start:end], f["k"][slots], f["v"][slots],
                                        float(f["scale"]), causal_offset=ctx - (end - start))
        assert_within_ulp(f["out"][start:end], ref.to(torch.bfloat16), ulps=1.0)
