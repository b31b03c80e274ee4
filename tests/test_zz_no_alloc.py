"""tvllm_paged_decode_noalloc (split-K partials in the library's static
device scratch) against tvllm_paged_decode (caller workspace) through the
C ABI: identical kernels, so the outputs must be bit-identical. Two calls in
a row, the second smaller, so it runs on scratch that still holds the first
call's partials; and a geometry beyond the scratch is rejected."""
import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from helpers import assert_bf16_close, paged_decode_case
from oracle import attention as OA

ROOT = Path(__file__).resolve().parents[1]


def _call(lib, fn, case, dev, out, workspace=None):
    from tinyvllm.kernels._extension import check, stream_of

    q, k, v = case["q_d"], case["k_d"], case["v_d"]
    rows, blocks, offsets, lengths = (case[n + "_d"] for n in
                                      ("rows", "blocks", "offsets", "lengths"))
    hkv, d = k.shape[1], k.shape[2]
    args = [q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
            out.data_ptr(), out.stride(0), out.stride(1), rows.data_ptr(),
            blocks.data_ptr(), offsets.data_ptr(), lengths.data_ptr(), rows.numel(),
            q.shape[1], hkv, d, k.shape[0], k.stride(0), k.stride(1), case["block_size"],
            case["max_len"],
            case["scale"]]
    if workspace is not None:
        args += [workspace.data_ptr() if workspace.numel() else None, workspace.numel()]
    args += [0, 0, 1.0, 1.0, stream_of(dev)]
    check(getattr(lib, fn)(*args))


def _case(seed, batch, heads, kv_heads, lengths, dev):
    c = paged_decode_case(seed=seed, batch=batch, heads=heads, kv_heads=kv_heads,
                          lengths=lengths, pool_blocks=sum(-(-n // 16) for n in lengths) + 8)
    for name in ("q", "k", "v", "rows", "blocks", "offsets", "lengths"):
        c[name + "_d"] = c[name].to(dev)
    c["max_len"] = max(lengths)
    return c


@pytest.mark.gpu
def test_noalloc_decode_matches_workspace_entry_point(device):
    from tinyvllm.kernels._extension import load_kernels

    lib = load_kernels()
    # First call: 2 rows of ~20k tokens (workgroup-level splits, 133 KB of
    # partials); second: 1 row of 5000 tokens (66 KB), on the same scratch.
    for seed, batch, heads, kv_heads, lengths in ((1, 2, 16, 8, [20000, 17001]),
                                                  (2, 1, 32, 8, [5000])):
        print(f"noalloc case seed={seed} rows={batch} heads={heads}/{kv_heads} "
              f"lengths={lengths}", flush=True)
        c = _case(seed, batch, heads, kv_heads, lengths, device)
        if seed == 2:  # a head-major cache: each KV head's slots contiguous
            for name in ("k_d", "v_d"):
                c[name] = c[name].transpose(0, 1).contiguous().transpose(0, 1)
        need = lib.tvllm_paged_decode_workspace_size(
            batch, heads, kv_heads, 128, c["max_len"], 16)
        assert need > 0  # the case exercises the split-K partials
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        expect = torch.empty_like(c["q_d"])
        got = torch.full_like(c["q_d"], float("nan"))
        _call(lib, "tvllm_paged_decode", c, device, expect, workspace=ws)
        _call(lib, "tvllm_paged_decode_noalloc", c, device, got)
        torch.cuda.synchronize()
        assert torch.equal(got, expect)
        ref = torch.empty_like(c["q"])
        OA.decode_attention(c["q"], c["k"], c["v"], c["rows"], c["blocks"], c["offsets"],
                            c["lengths"], 16, c["scale"], ref)
        assert_bf16_close(got.cpu(), ref)


def test_noalloc_rejects_geometry_beyond_scratch():
    """A plan needing more partials than the static scratch holds is refused
    on the host (no GPU touched). The split planner is widened through its
    measurement override in a child process."""
    code = (
        "import sys; sys.path[:0] = [%r, %r]\n"
        "from tinyvllm.kernels._extension import load_kernels\n"
        "lib = load_kernels()\n"
        "need = lib.tvllm_paged_decode_workspace_size(64, 128, 8, 128, 1 << 20, 16)\n"
        "assert need > (8 << 20), need\n"
        "st = lib.tvllm_paged_decode_noalloc(None, 0, 0, None, None, None, 0, 0, None,"
        " None, None, None, 64, 128, 8, 128, 1 << 24, 1024, 128, 16, 1 << 20, 0.1, 0, 0,"
        " 1.0, 1.0, None)\n"
        "assert st == -1, st\n"
        "assert b'static scratch' in lib.tvllm_last_error()\n"
    ) % (str(ROOT / "tiny-vllm_amd"), str(ROOT))
    env = dict(os.environ, TVLLM_DECODE_TUNING="100000,2,4")
    proc = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True,
                          text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr


@pytest.mark.gpu
def test_noalloc_decode_random_sequence(device):
    """Eight seeded geometries in a row on the same static scratch (row
    counts, GQA groups up to 32 - above 16 the general kernel, whose
    split partials use the same scratch - long and short contexts, either cache
    nesting), each bit-identical to the workspace entry point."""
    import random

    from tinyvllm.kernels._extension import load_kernels

    lib = load_kernels()
    r = random.Random(77)
    for step in range(8):
        kv_heads = r.choice([1, 2, 4, 8])
        group = r.choice([1, 2, 4, 8, 16, 32])
        rows = r.randint(1, 6)
        lengths = [r.choice([1, 300, 4000, 12000, 30000]) for _ in range(rows)]
        print(f"noalloc sequence step={step} rows={rows} heads={kv_heads * group}/{kv_heads} "
              f"lengths={lengths}", flush=True)
        c = _case(100 + step, rows, kv_heads * group, kv_heads, lengths, device)
        if r.random() < 0.5:
            for name in ("k_d", "v_d"):
                c[name] = c[name].transpose(0, 1).contiguous().transpose(0, 1)
        need = lib.tvllm_paged_decode_workspace_size(
            rows, kv_heads * group, kv_heads, 128, c["max_len"], 16)
        assert need <= 8 << 20
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device)
        expect = torch.empty_like(c["q_d"])
        got = torch.full_like(c["q_d"], float("nan"))
        _call(lib, "tvllm_paged_decode", c, device, expect, workspace=ws)
        _call(lib, "tvllm_paged_decode_noalloc", c, device, got)
        torch.cuda.synchronize()
        assert torch.equal(got, expect), step
