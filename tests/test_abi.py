"""The C-ABI library loads (no GPU needed) and exports every declared symbol."""
import ctypes
import os
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tinyvllm_hip.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(tvllm_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_bound_entry_points():
    from tinyvllm.kernels._extension import EXPORTED_SYMBOLS

    assert declared_symbols() == set(EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_symbol():
    from tinyvllm.kernels._extension import LIBRARY_PATH, load_kernels

    if not LIBRARY_PATH.exists():
        pytest.fail("libtinyvllm_hip.so is not built (run __graft_entry__.build())")
    lib = load_kernels()
    for name in sorted(declared_symbols()):
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name
    assert lib.tvllm_abi_version() == 5
    assert lib.tvllm_last_error() == b""


def test_argument_errors_surface_without_touching_a_gpu():
    """Contract violations are rejected on the host before any launch."""
    from tinyvllm.kernels._extension import check, load_kernels

    lib = load_kernels()
    status = lib.tvllm_store_kv(None, None, 0, 0, 0, 0, None, None, None,
                                4, 8, 128, 64, 1024, 128, 7, 7, 1.0, 1.0, None)
    assert status == -1
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        check(status)
    status = lib.tvllm_paged_decode(None, 0, 0, None, None, None, 0, 0, None, None,
                                    None, None, 1, 6, 4, 128, 64, 512, 128, 16, 64, 1.0,
                                    None, 0, 0, 0, 1.0, 1.0, None)
    with pytest.raises(RuntimeError, match="GQA"):
        check(status)
    # Zero-sized work is a no-op that never dereferences pointers.
    assert lib.tvllm_store_kv(None, None, 0, 0, 0, 0, None, None, None,
                              0, 8, 128, 64, 1024, 128, 0, 0, 1.0, 1.0, None) == 0
    # KV scales belong to FP8 caches; a 16-bit cache must keep them at 1.
    status = lib.tvllm_store_kv(None, None, 0, 0, 0, 0, None, None, None,
                                0, 8, 128, 64, 1024, 128, 0, 0, 2.0, 1.0, None)
    with pytest.raises(RuntimeError, match="FP8 cache only"):
        check(status)
    status = lib.tvllm_paged_decode(None, 0, 0, None, None, None, 0, 0, None, None,
                                    None, None, 1, 8, 8, 128, 64, 1024, 128, 16, 64, 1.0,
                                    None, 0, 0, 1, 1.0, 1.0, None)
    with pytest.raises(RuntimeError, match="cache dtype"):
        check(status)


def test_qkv_partials_entry_point_contract():
    """The split-K qkv decode entry point refuses rows too narrow for the
    q/k/v heads and strides that are not whole float4 units."""
    from tinyvllm.kernels._extension import check, load_kernels

    lib = load_kernels()
    # parts, slice/row strides, weights, cos, sin, eps x2, slots, caches, out +
    # strides, rows/blocks/offsets/lengths, 0 rows of 32 Q / 8 KV heads, ...
    base = [None, 0, 0, None, None, None, None, 1e-6, 1e-6, None, None, None, None, 0, 0,
            None, None, None, None, 0, 32, 8, 128, 64, 1024, 128, 16, 64, 0.1, None, 0, 0,
            0, 1.0, 1.0, None]
    assert len(base) == 36
    narrow = dict(enumerate(base))
    narrow[2] = 47 * 128  # a row needs (32 + 2 * 8) * 128 columns
    with pytest.raises(RuntimeError, match="q, k and v heads"):
        check(lib.tvllm_paged_decode_qk_norm_rope_partials(*narrow.values()))
    odd = dict(enumerate(base))
    odd[2], odd[1] = 48 * 128, 6
    with pytest.raises(RuntimeError, match="float4"):
        check(lib.tvllm_paged_decode_qk_norm_rope_partials(*odd.values()))
    ok = dict(enumerate(base))
    ok[2], ok[1] = 48 * 128, 48 * 128 * 3
    assert lib.tvllm_paged_decode_qk_norm_rope_partials(*ok.values()) == 0  # no rows


def test_cache_layout_contract():
    """Both cache nestings are accepted (token-major [slots, heads, dim] and
    head-major [heads, slots, dim]); strides whose head rows would overlap
    are refused by every entry point that takes the cache."""
    from tinyvllm.kernels._extension import check, load_kernels

    lib = load_kernels()
    slots, heads, dim = 64, 8, 128
    for ss, hs in ((heads * dim, dim), (dim, slots * dim), (2 * heads * dim, 2 * dim)):
        assert lib.tvllm_store_kv(None, None, 0, 0, 0, 0, None, None, None,
                                  0, heads, dim, slots, ss, hs, 0, 0, 1.0, 1.0, None) == 0
        assert lib.tvllm_paged_decode(None, 0, 0, None, None, None, 0, 0, None, None,
                                      None, None, 0, 16, heads, dim, slots, ss, hs, 16,
                                      64, 1.0, None, 0, 0, 0, 1.0, 1.0, None) == 0
    for ss, hs in ((dim, dim), (heads * dim, dim // 2), (dim, (slots - 1) * dim), (0, 0)):
        status = lib.tvllm_store_kv(None, None, 0, 0, 0, 0, None, None, None,
                                    0, heads, dim, slots, ss, hs, 0, 0, 1.0, 1.0, None)
        with pytest.raises(RuntimeError, match="non-overlapping"):
            check(status)
        status = lib.tvllm_paged_decode(None, 0, 0, None, None, None, 0, 0, None, None,
                                        None, None, 0, 16, heads, dim, slots, ss, hs, 16,
                                        64, 1.0, None, 0, 0, 0, 1.0, 1.0, None)
        with pytest.raises(RuntimeError, match="non-overlapping"):
            check(status)
        status = lib.tvllm_paged_prefill(None, 0, 0, None, None, None, 0, 0, None, None,
                                         None, None, 1, 16, 16, heads, dim, slots, ss, hs, 16,
                                         0.1, None, 0, 0, 0, 1.0, 1.0, None)
        with pytest.raises(RuntimeError, match="non-overlapping"):
            check(status)


def test_resolve_tokens_and_sample_workspace_contracts():
    """Host-side contracts of the pipelined-input and sampling entry points
    (no launch: errors and zero-sized calls only)."""
    from tinyvllm.kernels._extension import check, load_kernels

    lib = load_kernels()
    status = lib.tvllm_resolve_tokens(None, None, None, -1, 0, None)
    with pytest.raises(RuntimeError, match="negative size"):
        check(status)
    assert lib.tvllm_resolve_tokens(None, None, None, 0, 0, None) == 0
    # One 8-byte (value, index) partial per 8192-wide span of each row.
    assert lib.tvllm_sample_workspace_size(64, 151936) == 64 * 19 * 8
    assert lib.tvllm_sample_workspace_size(3, 16384) == 3 * 2 * 8
    assert lib.tvllm_sample_workspace_size(0, 151936) == 0
    status = lib.tvllm_sample(None, 1, 100, 100, None, None, None, None, None, None,
                              None, 64, 0, None)
    with pytest.raises(RuntimeError):
        check(status)


def test_decode_workspace_sizes():
    """Splits inside one workgroup merge in LDS (no workspace); only long
    contexts over few rows also split across workgroups and need HBM
    partials for the merge kernel."""
    from tinyvllm.kernels._extension import load_kernels

    lib = load_kernels()
    # 8B shape at bs64: 512 (row, KV head) units -> 2 splits, one workgroup.
    assert lib.tvllm_paged_decode_workspace_size(64, 32, 8, 128, 4096, 16) == 0
    assert lib.tvllm_paged_decode_workspace_size(64, 16, 8, 128, 1024, 16) == 0
    # One row, 8 KV heads: 16 splits of a 512 context -> 2 workgroups per head.
    assert lib.tvllm_paged_decode_workspace_size(1, 16, 8, 128, 512, 16) == 16 * 2 * 130 * 4
    # 32B shape at bs16, 32k context: 128 units -> 16 splits, long ranges ->
    # 4 waves x 4 workgroups, two KV heads per workgroup.
    assert lib.tvllm_paged_decode_workspace_size(16, 64, 8, 128, 32768, 16) == \
        16 * 64 * 4 * 130 * 4
    # Groups above 16 and other head dims run the general kernel, which
    # splits a context over workgroups (toward 512 of them) only when there
    # are few (row, KV head, 16-head chunk) units: 63 rows x 2 KV heads x 2
    # chunks = 252 units -> 3 splits; 2 units -> 64 splits.
    assert lib.tvllm_paged_decode_workspace_size(63, 64, 2, 128, 16384, 16) == \
        63 * 64 * 3 * 130 * 4
    assert lib.tvllm_paged_decode_workspace_size(1, 17, 1, 128, 32768, 16) == \
        17 * 64 * 130 * 4
    assert lib.tvllm_paged_decode_workspace_size(1, 16, 1, 128, 32768, 16) > 0
    assert lib.tvllm_paged_decode_workspace_size(1, 32, 8, 64, 32768, 16) == 32 * 64 * 66 * 4
    assert lib.tvllm_paged_decode_workspace_size(64, 32, 8, 64, 2048, 16) == 0  # 512 units
    # A split keeps at least two 64-key chunks per wave of its four at head
    # dim 64: a 1000-token context splits twice at most.
    assert lib.tvllm_paged_decode_workspace_size(1, 8, 8, 64, 1000, 16) == 8 * 2 * 66 * 4
    # The largest request of any plan with group <= 16 fits the no-alloc
    # entry point's 8 MiB scratch.
    worst = max(lib.tvllm_paged_decode_workspace_size(rows, kv * g, kv, 128, ctx, 16)
                for kv in (1, 2, 4, 8, 16) for g in (1, 2, 4, 8, 16)
                for rows in (1, 2, 4, 8, 15, 16, 31, 32, 63, 64, 96)
                for ctx in (1024, 8192, 16384, 65536))
    assert 0 < worst <= 8 << 20


def _plan(lib, *args):
    packed = lib.tvllm_paged_decode_split_plan(*args)
    return packed >> 16, (packed >> 8) & 0xFF, packed & 0xFF  # waves, grid, heads


def test_decode_split_plans():
    """Many (row, KV head) units: splits inside one workgroup. Few units with
    long page ranges per split: two KV heads x four ranges per workgroup.
    Few units with short ranges: one head, up to eight ranges."""
    from tinyvllm.kernels._extension import load_kernels

    lib = load_kernels()
    assert _plan(lib, 64, 32, 8, 128, 2048, 16) == (2, 1, 2)      # 8B bs64
    assert _plan(lib, 16, 64, 8, 128, 32768, 16) == (4, 4, 2)     # C5 decode
    assert _plan(lib, 8, 16, 8, 128, 1024, 16) == (8, 4, 1)       # C1
    assert _plan(lib, 16, 32, 8, 128, 8192, 16) == (4, 4, 2)      # 512 tokens per split
    assert _plan(lib, 16, 32, 8, 128, 8191, 16) == (8, 2, 1)
    # One long row: up to 256 page ranges per (row, KV head), so 8 KV heads
    # still put a wave on every SIMD (8 x 32 workgroups of 8 waves).
    assert _plan(lib, 1, 32, 8, 128, 32768, 16) == (8, 32, 1)
    assert _plan(lib, 2, 32, 8, 128, 32768, 16) == (8, 16, 1)
    assert _plan(lib, 1, 64, 8, 128, 131072, 16) == (4, 64, 2)
    # Fewer units: at most 256 workgroups - eight ranges times a power-of-two
    # grid per unit, or one four-wave workgroup per unit past 128 units
    # (heads not paired there).
    assert _plan(lib, 8, 32, 8, 128, 4096, 16) == (8, 4, 1)
    assert _plan(lib, 12, 32, 8, 128, 4096, 16) == (8, 2, 1)
    assert _plan(lib, 20, 32, 8, 128, 4096, 16) == (4, 1, 1)
    assert _plan(lib, 28, 32, 8, 128, 4096, 16) == (4, 1, 1)
    # Groups above 4 (a 16-bit cache's kernel runs 16-token iterations): one
    # eight-range workgroup per unit past 128 units, and a 2048-wave budget
    # from 256 units.
    assert _plan(lib, 24, 64, 8, 128, 4096, 16) == (8, 1, 1)
    assert _plan(lib, 48, 64, 8, 128, 4096, 16) == (4, 1, 1)
    # 256+ (row, KV head) units: the largest power-of-two split count with at
    # most 1024 waves, in four-wave workgroups (one per CU at most).
    assert _plan(lib, 32, 32, 8, 128, 4096, 16) == (4, 1, 1)
    assert _plan(lib, 40, 32, 8, 128, 4096, 16) == (2, 1, 2)
    assert _plan(lib, 56, 32, 8, 128, 4096, 16) == (2, 1, 2)
    assert _plan(lib, 72, 32, 8, 128, 4096, 16) == (1, 1, 4)
    assert _plan(lib, 128, 32, 8, 128, 4096, 16) == (1, 1, 4)
    # Context bounds up to 256: page ranges of at least 64 tokens (four at
    # 256); up to 512: at least 128 (four at 512); past 512, 32-token ranges
    # again.
    assert _plan(lib, 1, 16, 8, 128, 256, 16) == (4, 1, 1)
    assert _plan(lib, 16, 16, 8, 128, 256, 16) == (4, 1, 1)
    assert _plan(lib, 1, 16, 8, 128, 128, 16) == (2, 1, 2)
    assert _plan(lib, 1, 16, 8, 128, 257, 16) == (3, 1, 1)
    assert _plan(lib, 1, 16, 8, 128, 512, 16) == (4, 1, 1)
    assert _plan(lib, 16, 16, 8, 128, 512, 16) == (4, 1, 1)
    assert _plan(lib, 1, 16, 8, 128, 513, 16) == (8, 3, 1)
    # The merge launch holds one workgroup-level split per lane.
    assert max(_plan(lib, rows, 4 * kv, kv, 128, ctx, 16)[1]
               for rows in range(1, 80) for kv in (1, 2, 4, 8)
               for ctx in (16, 512, 4096, 32768, 131072, 1 << 20)) <= 64


@pytest.mark.parametrize("heads,kv_heads,head_dim", [
    (64, 8, 128), (16, 8, 64), (8, 2, 256), (16, 4, 32), (40, 2, 128)])
def test_decode_workspace_at_the_longest_context_covers_shorter_ones(heads, kv_heads,
                                                                     head_dim):
    """The runner sizes the decode workspace once, at max_model_len, for every
    row count; a launch's plan follows its batch's longest context."""
    from tinyvllm.kernels._extension import load_kernels

    lib = load_kernels()
    for max_len in (2048, 8192, 40960):
        for rows in (1, 2, 3, 4, 8, 12, 16, 31, 32, 33, 64):
            cap = lib.tvllm_paged_decode_workspace_size(rows, heads, kv_heads, head_dim,
                                                        max_len, 16)
            for ctx in range(16, max_len + 1, 16 * 37):
                assert lib.tvllm_paged_decode_workspace_size(
                    rows, heads, kv_heads, head_dim, ctx, 16) <= cap


def test_decode_split_plan_under_tuning_override_keeps_the_merge_bound():
    """A TVLLM_DECODE_TUNING override with one page range per workgroup
    would ask for up to 256 workgroup splits; the plan caps them at the
    merge launch's 64, and the workspace size follows the capped plan (the
    override is read once per process, hence the child process)."""
    import subprocess
    import sys

    code = (
        "from tinyvllm.kernels._extension import load_kernels\n"
        "lib = load_kernels()\n"
        "p = lib.tvllm_paged_decode_split_plan(1, 32, 8, 128, 131072, 16)\n"
        "w = lib.tvllm_paged_decode_workspace_size(1, 32, 8, 128, 131072, 16)\n"
        "print(p >> 16, (p >> 8) & 0xFF, p & 0xFF, w)\n")
    env = dict(os.environ, TVLLM_DECODE_TUNING="0,2,4,1")
    root = Path(__file__).resolve().parents[1]
    env["PYTHONPATH"] = os.pathsep.join([str(root / "tiny-vllm_amd"), str(root)])
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True,
                         text=True, timeout=120, check=True).stdout.split()
    waves, grid, heads, workspace = map(int, out)
    assert waves == 1 and grid == 64
    assert workspace == 1 * 32 * 64 * 130 * 4
