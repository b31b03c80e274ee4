"""Decode-loop benchmark: Qwen3-8B bf16, 64 concurrent sequences at 2048-token
context, greedy, on one MI355X.

A step is one decode iteration of the whole batch through the product path:
CPU batch build + validation, one H2D metadata copy, the replayed hipGraph
(36 layers of fused QK-norm/RoPE/KV-write, split-K paged decode attention,
GEMMs, norms, LM head, sampling kernel) and the D2H of the sampled ids.
Weights are random-init N(0, 0.02) (no checkpoints offline); the 2048-token
contexts' KV pages are filled with N(0, 1) values before timing.

Also reported on the same JSON line:
  roofline     -- the dominant kernel (paged decode attention, one layer at
                  the workload's shape) timed with HIP events on the stream
                  it runs on: algorithmic bytes / average launch duration.
  cpu_baseline -- the CPU oracle's decode step, one layer at full batch
                  timed and extrapolated to all layers + LM head.
  engine_ms_per_step -- the same batch driven through Engine.step (scheduler,
                  block manager, batch builder, commit and resolve inside the
                  timing) after prefilling 64 prompts of 2048 ids: the mean
                  decode-only step time, beside the headline's ms_per_step.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "tiny-vllm_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

MODELS = {
    "qwen3-0.6b": dict(vocab_size=151936, hidden_size=1024, intermediate_size=3072,
                       num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8,
                       head_dim=128, tie_word_embeddings=True),
    "qwen3-8b": dict(vocab_size=151936, hidden_size=4096, intermediate_size=12288,
                     num_hidden_layers=36, num_attention_heads=32, num_key_value_heads=8,
                     head_dim=128, tie_word_embeddings=False),
    "qwen3-32b": dict(vocab_size=151936, hidden_size=5120, intermediate_size=25600,
                      num_hidden_layers=64, num_attention_heads=64, num_key_value_heads=8,
                      head_dim=128, tie_word_embeddings=False),
}
HBM_PEAK_GBS = 8000.0


def qwen3_config(name: str, max_position: int):
    from tinyvllm.models.qwen3 import Qwen3Config

    return Qwen3Config.from_dict(dict(model_type="qwen3", rope_theta=1e6, rms_norm_eps=1e-6,
                                      max_position_embeddings=max_position,
                                      **MODELS[name]))


class DecodeWorkload:
    """Synthetic sequences parked at a fixed context, advanced one token per step."""

    def __init__(self, batch: int, context: int, block_size: int, num_blocks: int,
                 vocab: int, seed: int = 0):
        import numpy as np

        rng = np.random.default_rng(seed)
        self.batch, self.bs = batch, block_size
        self.lengths = [context] * batch
        self.max_pages = num_blocks // batch
        perm = rng.permutation(num_blocks)
        self.tables = [perm[i * self.max_pages:(i + 1) * self.max_pages].tolist()
                       for i in range(batch)]
        self.tokens = rng.integers(0, vocab, size=batch).tolist()
        self.np_tables_2d = np.asarray(self.tables, dtype=np.int64)
        self.np_tables = list(self.np_tables_2d)
        self.plan_id = 0
        from tinyvllm.request import SamplingParams

        self.greedy = SamplingParams(max_new_tokens=1 << 20)
        self.full_tables = False  # True: upload every block table each step

    def batch_for_step(self, from_previous: bool = False):
        """The next decode step's PreparedBatch (block tables and slots as
        int64 arrays, like BatchBuilder emits). ``from_previous``: the input
        ids are the previous launched step's sampled rows, taken on the
        device (pipelined steps)."""
        import numpy as np

        from tinyvllm.batch import PreparedBatch, StepMode
        from tinyvllm.request import SamplingParams

        bs = self.bs
        n = self.batch
        pos = np.asarray(self.lengths, dtype=np.int64)  # writes position `length`
        pages = pos // bs + 1
        offsets = np.concatenate(([0], np.cumsum(pages)))
        table_ids = np.concatenate([t[:p] for t, p in zip(self.np_tables, pages)])
        slots = self.np_tables_2d[np.arange(n), pos // bs] * bs + pos % bs
        self.plan_id += 1
        return PreparedBatch(
            plan_id=self.plan_id, mode=StepMode.DECODE_ONLY,
            input_ids=(0,) * n if from_previous else tuple(self.tokens),
            positions=tuple(self.lengths), q_offsets=tuple(range(n + 1)),
            context_lens_before=tuple(self.lengths), query_lens=(1,) * n,
            context_lens_after=tuple(l + 1 for l in self.lengths),
            sample_token_indices=tuple(range(n)), sample_request_ids=tuple(range(n)),
            sampling_params=(self.greedy,) * n, kv_block_size=bs,
            kv_num_blocks=self.max_pages * n, kv_block_table_ids=table_ids,
            kv_block_table_offsets=tuple(offsets.tolist()), kv_slot_mapping=slots,
            request_ids=tuple(range(n)),
            input_token_sources=tuple(range(n)) if from_previous else None,
            # As the engine's builder emits them: one slot per sequence, and a
            # table epoch that never changes (the tables only grow).
            request_slots=None if self.full_tables else tuple(range(n)),
            kv_table_epochs=None if self.full_tables else (1,) * n,
        )

    def advance(self, tokens):
        self.tokens = list(tokens)
        self.lengths = [length + 1 for length in self.lengths]

    def run(self, executor, steps: int, pending=None):
        """``steps`` pipelined decode steps: step i+1 is built and launched
        (its input ids taken from step i's sampled rows on the device)
        before the host waits for step i's tokens. Returns the last step's
        PendingStep; pass it back in to continue the chain."""
        for _ in range(steps):
            launched = executor.launch(self.batch_for_step(from_previous=pending is not None))
            self.lengths = [length + 1 for length in self.lengths]
            if pending is not None:
                self.tokens = list(pending.result().sampled_token_ids)
            pending = launched
        return pending


COUNTERS_FILE = ROOT / "profiles" / "paged_decode_qwen3-8b_bs64_ctx2k_counters.txt"


def measured_traffic() -> int | None:
    """HBM bytes per decode launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (copy-calibrated); None if that summary is absent."""
    import re

    try:
        found = re.search(r"traffic_bytes_per_launch:\s*(\d+)", COUNTERS_FILE.read_text())
    except OSError:
        return None
    return int(found.group(1)) if found else None


def attention_roofline(executor, workload, cfg, iters: int = 30,
                       headline: bool = True) -> dict:
    """Time the decode step's attention kernel - QK-norm + RoPE + KV write +
    split-K paged decode in one launch, as every decode layer runs it - on
    layer 0 of the live cache with the live step metadata (graph-replayed,
    HIP events on the replay stream)."""
    import torch

    from tinyvllm.kernels.paged_decode import paged_decode_qk_norm_rope

    runner = executor.runner
    batch = workload.batch_for_step()
    model_input = runner.decode_inputs.prepare(batch, [0] * batch.num_items)
    runner.decode_inputs.apply_table_updates()
    meta = model_input.kv.decode
    rows, hq, hkv, d = (batch.num_items, cfg.num_attention_heads, cfg.num_key_value_heads,
                        cfg.head_dim)
    qkv = torch.randn(rows, (hq + 2 * hkv) * d, dtype=torch.bfloat16, device=runner.device)
    q = qkv[:, :hq * d].view(rows, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(rows, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(rows, hkv, d)
    layer = runner.model.model.layers[0].self_attn
    cos, sin = runner.model.model.rotary_emb(model_input.positions, torch.bfloat16)
    out = torch.empty_like(q)
    scale = cfg.head_dim ** -0.5
    # Successive calls walk the layers, as a decode step does: every launch
    # reads KV that no recent launch has touched, so the 256 MB memory-side
    # cache holds none of it (repeating one layer would let part of its K
    # rows stay cached between launches).
    nl = runner.kv_cache.num_layers
    calls = [0]

    def call():
        idx = calls[0] % nl
        calls[0] += 1
        paged_decode_qk_norm_rope(
            q, k, v, layer.q_norm.weight, layer.k_norm.weight, cos, sin, layer.q_norm.eps,
            layer.k_norm.eps, runner.kv_cache, idx, meta, model_input.kv.slot_mapping, out,
            scale=scale, workspace=runner.decode_workspace)

    with torch.inference_mode():  # the runner's cache and inputs are inference tensors
        seconds = _event_time(call, iters)
    lengths = batch.context_lens_after
    pages = sum(math.ceil(l / workload.bs) for l in lengths)
    kv = runner.kv_cache.key.element_size()  # 2 (bf16) or 1 (FP8 layout)
    # KV read once per KV head; q/k/v projections read, output and the new
    # K/V rows written; RoPE tables, slots and block tables.
    algorithmic = (sum(lengths) * hkv * d * 2 * kv + rows * (hq + 2 * hkv) * d * 2
                   + rows * hq * d * 2 + rows * 2 * hkv * d * kv + rows * d * 2 * 2
                   + 8 * pages + 8 * (4 * rows + 1))
    achieved = algorithmic / seconds / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            # The committed counter passes cover the headline workload only.
            "traffic": measured_traffic() if headline else None,
            "kernel": "paged_decode_d128",
            "avg_launch_us": round(seconds * 1e6, 2), "bytes_per_launch": algorithmic}


def cpu_baseline(cfg, batch: int, context: int, reps: int = 21) -> dict:
    """The oracle's decode step on the host cores: one decoder layer at full
    batch and context (GEMMs + paged gather + fp32 softmax attention + the
    pointwise chain), timed `reps` times (median; ~14 s of host work at the
    8B shape), extrapolated to all layers plus the LM head (median of 3)."""
    import torch

    from oracle import attention as OA
    from oracle import model as OM
    from oracle import pointwise as OP

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    dt = torch.bfloat16
    h, hq, hkv, d, inter = (cfg.hidden_size, cfg.num_attention_heads,
                            cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size)

    def mat(*shape):
        return (torch.randn(*shape, generator=g) * 0.02).to(dt)

    w_qkv, w_o = mat((hq + 2 * hkv) * d, h), mat(h, hq * d)
    w_gu, w_down = mat(2 * inter, h), mat(h, inter)
    ones_h, ones_d = torch.ones(h, dtype=dt), torch.ones(d, dtype=dt)
    bs = 16
    pages = math.ceil((context + 1) / bs)
    kc = torch.randn(batch * pages * bs, hkv, d, generator=g).to(dt)
    vc = torch.randn(batch * pages * bs, hkv, d, generator=g).to(dt)
    blocks = torch.arange(batch * pages)
    offsets = torch.arange(batch + 1) * pages
    lengths = torch.full((batch,), context + 1)
    x = torch.randn(batch, h, generator=g).to(dt)
    res = torch.randn(batch, h, generator=g).to(dt)
    pos = torch.full((batch,), context)
    cos, sin = OP.rope_tables(pos, d, cfg.rope_theta, dt)
    slots = blocks.view(batch, pages)[:, context // bs] * bs + context % bs

    def layer():
        y, r = OP.add_rms_norm(x, res, ones_h)
        qkv = OM.linear(y, w_qkv)
        q = qkv[:, :hq * d].view(batch, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].view(batch, hkv, d)
        v = qkv[:, (hq + hkv) * d:].view(batch, hkv, d)
        q, k = OP.qk_norm_rope(q, k, ones_d, ones_d, cos, sin)
        kc[slots], vc[slots] = k, v
        out = torch.empty_like(q)
        OA.decode_attention(q, kc, vc, torch.arange(batch), blocks, offsets, lengths, bs,
                            d ** -0.5, out)
        o = OM.linear(out.view(batch, hq * d), w_o)
        y, r = OP.add_rms_norm(o, r, ones_h)
        return OM.linear(OP.silu_and_mul(OM.linear(y, w_gu)), w_down)

    layer()  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        layer()
        times.append(time.perf_counter() - t0)
    per_layer = sorted(times)[len(times) // 2]
    w_head = mat(cfg.vocab_size, h)
    heads = []
    for _ in range(3):
        t0 = time.perf_counter()
        OM.linear(x, w_head).float().argmax(-1)
        heads.append(time.perf_counter() - t0)
    head = sorted(heads)[1]
    step = per_layer * cfg.num_hidden_layers + head
    return {"value": round(batch / step, 3), "unit": "tok/s", "cores": threads,
            "kind": "port",
            "sample": (f"oracle decode step, 1 of {cfg.num_hidden_layers} layers at bs{batch} "
                       f"ctx{context} timed x{reps} (median {per_layer:.2f} s) + LM head "
                       f"({head:.2f} s), extrapolated to the full model")}


def engine_decode_step(model, cfg, batch: int, context: int, steps: int,
                       warmup: int) -> dict:
    """The same decode batch driven through the whole engine: ``batch``
    requests of ``context`` random ids are prefilled (chunks of 512), then
    ``steps`` decode-only ``Engine.step`` calls are timed - scheduler,
    block-manager transaction, BatchBuilder, the launch, commit and the
    resolve of the previous step's tokens all inside the timing, pipelined
    as the engine runs them."""
    import numpy as np
    import torch

    from tinyvllm import SamplingParams
    from tinyvllm.bootstrap import build_engine

    rng = np.random.default_rng(7)
    prompts = [rng.integers(0, cfg.vocab_size, size=context).tolist() for _ in range(batch)]
    # Prefill admits ~4096 tokens a step, so early rows decode meanwhile.
    prefill_steps = -(-batch * context // 4096) + 2
    new = prefill_steps + warmup + steps + 8
    max_model_len = 1 << (context + new + 16 - 1).bit_length()
    engine = build_engine(model, max_model_len=max_model_len, max_num_seqs=batch,
                          max_num_batched_tokens=4096,
                          num_blocks=batch * -(-(context + new) // 16) + 64,
                          prefill_chunk_size=512)
    params = SamplingParams(max_new_tokens=new, ignore_eos=True)
    ids = [engine.submit(p, params) for p in prompts]
    got = {rid: 0 for rid in ids}
    calls = 0
    while min(got.values()) < 2:  # every prompt prefilled, first tokens out
        for ev in engine.step().token_events:
            got[ev.request_id] += 1
        calls += 1
        if calls > 10 * prefill_steps:
            raise RuntimeError("engine benchmark: prefill did not finish")
    for _ in range(warmup):
        engine.step()
    torch.cuda.synchronize()
    tokens = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        tokens += len(engine.step().token_events)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    if tokens != batch * steps:
        raise RuntimeError(f"engine benchmark: {tokens} tokens in {steps} steps of {batch} rows")
    unfinished = engine.has_unfinished()
    engine.close()
    if not unfinished:
        raise RuntimeError("engine benchmark: requests ended inside the timed steps")
    return {"engine_ms_per_step": round(elapsed / steps * 1e3, 3),
            "engine_tok_s": round(tokens / elapsed, 1),
            "engine_steps": steps,
            "engine_sample": f"Engine.step decode-only at bs{batch}, contexts "
                             f"{context}-{context + prefill_steps + warmup + steps}, "
                             f"after {calls} prefill steps"}


def kernel_only(args) -> None:
    """The decode step's attention kernel (QK-norm + RoPE + KV write + split-K
    paged decode) alone at the workload's shape (eight layers of KV visited in
    turn, one step's metadata), plus a 1 GiB device copy for counter calibration. Used for
    rocprofv3 PMC passes, which profile dispatches launched outside graphs."""
    import torch

    from tinyvllm.kernels.paged_decode import decode_workspace_bytes, paged_decode_qk_norm_rope
    from tinyvllm.layers import RotaryEmbedding
    from tinyvllm.paged_kv import PagedKVCache, resolve_layout
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    cfg = qwen3_config(args.model, max_position=40960)
    device = torch.device("cuda", 0)
    bs, rows, ctx = 16, args.batch, args.context + 1
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    pages = math.ceil(ctx / bs)
    layers = 8  # visited in turn: no launch finds its KV in the memory-side cache
    fp8 = args.kv_cache_dtype == "fp8_e4m3"
    cache = PagedKVCache(num_layers=layers, num_blocks=rows * pages, block_size=bs,
                         num_kv_heads=hkv, head_dim=d, device=device,
                         dtype=torch.float8_e4m3fn if fp8 else torch.bfloat16,
                         layout=resolve_layout(args.kv_layout, rows, hkv))
    gen = torch.Generator(device=device).manual_seed(1)
    if fp8:  # N(0, 1) values quantised layer by layer (scales 1)
        for layer in range(layers):
            for t in (cache.key[layer], cache.value[layer]):
                t.copy_(torch.randn(t.shape, generator=gen, device=device))
    else:
        cache.key.normal_(generator=gen)
        cache.value.normal_(generator=gen)
    perm = torch.randperm(rows * pages, device=device, generator=gen)
    max_len = 4096
    meta = SingleQueryMetadata(torch.arange(rows, device=device), perm,
                               torch.arange(rows + 1, device=device) * pages,
                               torch.full((rows,), ctx, device=device), max_len)
    ws_bytes = decode_workspace_bytes(rows, hq, hkv, d, max_len, bs)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=device)
    qkv = torch.randn(rows, (hq + 2 * hkv) * d, dtype=torch.bfloat16, device=device)
    q = qkv[:, :hq * d].view(rows, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(rows, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(rows, hkv, d)
    w = torch.ones(d, dtype=torch.bfloat16, device=device)
    positions = torch.full((rows,), ctx - 1, device=device)
    cos, sin = RotaryEmbedding(d, 40960, base=cfg.rope_theta, device=device)(
        positions, torch.bfloat16)
    slots = perm.view(rows, pages)[:, (ctx - 1) // bs] * bs + (ctx - 1) % bs
    out = torch.empty_like(q)
    for step in range(args.steps):
        paged_decode_qk_norm_rope(q, k, v, w, w, cos, sin, 1e-6, 1e-6, cache, step % layers,
                                  meta, slots, out, scale=d ** -0.5, workspace=ws)
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device=device)  # 1 GiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"kernel_only": True, "rows": rows, "context": ctx,
                      "kv_cache_dtype": "fp8_e4m3" if fp8 else "bf16",
                      "decode_launches": args.steps, "copy_bytes": src.numel() * 2}))


def summarize_profile(directory: str, tail: int = 30) -> None:
    """Print a short text summary of a rocprofv3 --kernel-trace --stats run
    (kernel_stats.csv) and, when present, PMC counter averages per kernel."""
    import csv
    from collections import defaultdict

    root = Path(directory)
    stats = sorted(root.rglob("*kernel_stats.csv"))
    if stats:
        rows = list(csv.DictReader(open(stats[0])))
        rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
        print(f"{'total ms':>9} {'%':>6} {'calls':>6} {'avg us':>9}  kernel")
        for r in rows[:20]:
            print(f"{float(r['TotalDurationNs']) / 1e6:9.2f} {float(r['Percentage']):6.2f} "
                  f"{r['Calls']:>6} {float(r['AverageNs']) / 1e3:9.2f}  {r['Name'][:100]}")
    traces = sorted(root.rglob("*kernel_trace.csv"))
    if traces:
        trace = list(csv.DictReader(open(traces[0])))
        trace.sort(key=lambda r: int(r["Start_Timestamp"]))

        def dur(r):
            return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3

        # bench.py's roofline loop: graph replays of the attention launch
        # alone, i.e. the last run of >= `tail` paged_decode_d128 dispatches
        # with no other kernel between them; its timed part is the last 7
        # replays of `tail` launches each.
        runs, cur = [], []
        for r in trace:
            if "paged_decode_d128" in r["Kernel_Name"]:
                cur.append(dur(r))
            else:
                if len(cur) >= tail:
                    runs.append(cur)
                cur = []
        if len(cur) >= tail:
            runs.append(cur)
        if runs:
            timed = runs[-1][-7 * tail:]
            print(f"-- paged_decode_d128: roofline loop of {len(runs[-1])} back-to-back "
                  f"dispatches; mean of its last {len(timed)} (the timed replays) = "
                  f"{sum(timed) / len(timed):.2f} us, median "
                  f"{sorted(timed)[len(timed) // 2]:.2f} us")
        ends = [i for i, r in enumerate(trace) if "sample_kernel" in r["Kernel_Name"]]
        if len(ends) >= 2:
            step = trace[ends[-2] + 1:ends[-1] + 1]
            wall = (int(trace[ends[-1]]["End_Timestamp"])
                    - int(trace[ends[-2]]["End_Timestamp"])) / 1e3
            busy = sum(dur(r) for r in step)
            groups = defaultdict(lambda: [0.0, 0])
            for r in step:
                name = r["Kernel_Name"]
                key = ("GEMM (hipBLASLt " + name.split("_MT")[1][:10] + ")"
                       if name.startswith("Cijk") else name[:70])
                groups[key][0] += dur(r)
                groups[key][1] += 1
            print(f"-- last decode step (between sampling kernels): wall {wall:.1f} us, "
                  f"kernels busy {busy:.1f} us, {len(step)} dispatches")
            for key, (t, n) in sorted(groups.items(), key=lambda kv: -kv[1][0]):
                print(f"  {t:9.1f} us  x{n:<4d} {key}")
    for counters in sorted(root.rglob("*counter_collection.csv")):
        acc = defaultdict(lambda: defaultdict(list))
        for r in csv.DictReader(open(counters)):
            acc[r["Kernel_Name"][:100]][r["Counter_Name"]].append(float(r["Counter_Value"]))
        print(f"-- counters ({counters.name}): mean per dispatch")
        for name, by_counter in sorted(acc.items()):
            vals = ", ".join(f"{c}={sum(v) / len(v):.1f} (n={len(v)})"
                             for c, v in sorted(by_counter.items()))
            print(f"  {name}: {vals}")


EAGER_OPS = False  # --eager: launch op-benchmark kernels directly (PMC passes)


def _event_time(fn, iters: int, replays: int = 7) -> float:
    """Mean device seconds per call of `fn`: `iters` calls captured in one
    hipGraph (so Python launch overhead is not timed), replayed `replays`
    times back to back, each replay timed with HIP events on the replay
    stream; the median replay is returned. (Single timed replays were
    bimodal on these boxes: a replay that follows host-side idle time runs
    ~4 % slower at the 8B decode shape.) With --eager the calls are launched
    directly (rocprofv3 counter passes see only such dispatches)."""
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    if EAGER_OPS:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            fn()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / 1e3 / iters
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    with torch.cuda.stream(stream):
        events[0].record(stream)
        for i in range(replays):
            graph.replay()
            events[i + 1].record(stream)
    events[-1].synchronize()
    times = sorted(events[i].elapsed_time(events[i + 1]) for i in range(replays))
    return times[len(times) // 2] / 1e3 / iters


def _cpu_time(fn, reps: int = 5) -> float:
    fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def _hbm(bytes_: int, seconds: float) -> dict:
    gbs = bytes_ / seconds / 1e9
    return {"us": round(seconds * 1e6, 2), "bytes": bytes_, "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def op_c1(args) -> dict:
    """C1: the paged-decode op alone at Qwen3-0.6B shapes (8 rows, 16Q/8KV
    heads, D128, L ~ U[64,1024], 16-token pages from a 1024-page pool), plus
    the 8B-shape variant (64 rows, 32Q/8KV, L=2048) and the C5 decode shape
    (16 rows, 64Q/8KV, L ~ U[16k,32k]: workgroup-level split-K + merge)."""
    import torch

    from oracle import attention as OA
    from tinyvllm.kernels.paged_decode import decode_workspace_bytes, paged_decode_attention
    from tinyvllm.paged_kv import PagedKVCache, resolve_layout
    from tinyvllm.runtime.contracts import SingleQueryMetadata

    device = torch.device("cuda", 0)
    result = {}
    for name, rows, hq, lengths_fn, pool in (
            ("c1_qwen3-0.6b_bs8", 8, 16, lambda g: torch.randint(64, 1025, (8,), generator=g), 1024),
            ("qwen3-8b_bs64_ctx2048", 64, 32, lambda g: torch.full((64,), 2048), 64 * 128),
            ("c5_qwen3-32b_bs16_ctx16k-32k", 16, 64,
             lambda g: torch.randint(16384, 32769, (16,), generator=g), 16 * 2048)):
        g = torch.Generator().manual_seed(0)
        lengths = lengths_fn(g)
        pages = [math.ceil(int(l) / 16) for l in lengths]
        perm = torch.randperm(pool, generator=g)
        blocks = perm[:sum(pages)]
        offsets = torch.tensor([0] + list(torch.tensor(pages).cumsum(0).tolist()))
        cache = PagedKVCache(num_layers=1, num_blocks=pool, block_size=16, num_kv_heads=8,
                             head_dim=128, device="cpu", dtype=torch.bfloat16)
        cache.key.normal_(generator=g)
        cache.value.normal_(generator=g)
        q = torch.randn(rows, hq, 128, generator=g).to(torch.bfloat16)
        scale = 128 ** -0.5
        # Copies of the pool, visited in turn (>= 4 GB in all): no launch
        # finds its KV in the memory-side cache, as in a decode step.
        layers = max(1, min(64, math.ceil(4e9 / (2 * cache.key[0].numel() * 2))))
        gcache = PagedKVCache(num_layers=layers, num_blocks=pool, block_size=16,
                              num_kv_heads=8, head_dim=128, device=device,
                              dtype=torch.bfloat16,
                              layout=resolve_layout(args.kv_layout, rows, 8))
        for layer_idx in range(layers):
            gcache.key[layer_idx].copy_(cache.key[0])
            gcache.value[layer_idx].copy_(cache.value[0])
        meta = SingleQueryMetadata(torch.arange(rows, device=device), blocks.to(device),
                                   offsets.to(device), lengths.to(device),
                                   int(lengths.max()))
        ws = torch.empty(max(16, decode_workspace_bytes(rows, hq, 8, 128, int(lengths.max()),
                                                        16)), dtype=torch.uint8, device=device)
        gq, gout = q.to(device), torch.empty(rows, hq, 128, dtype=torch.bfloat16, device=device)
        calls = [0]

        def call():
            paged_decode_attention(gq, gcache, calls[0] % layers, meta, gout, scale=scale,
                                   workspace=ws)
            calls[0] += 1

        seconds = _event_time(call, 200)
        paged_decode_attention(gq, gcache, 0, meta, gout, scale=scale, workspace=ws)
        ref = torch.empty_like(q)
        oracle_call = lambda: OA.decode_attention(  # noqa: E731
            q, cache.key[0], cache.value[0], torch.arange(rows), blocks, offsets, lengths, 16,
            scale, ref)
        cpu = _cpu_time(oracle_call, reps=3)
        err = (gout.cpu().float() - ref.float()).abs()
        algorithmic = (int(lengths.sum()) * 8 * 128 * 4 + 2 * rows * hq * 128 * 2
                       + 8 * sum(pages) + 8 * (3 * rows + 1))
        result[name] = {**_hbm(algorithmic, seconds), "max_abs_err_vs_oracle":
                        round(err.max().item(), 5),
                        "cpu_oracle_us": round(cpu * 1e6, 1), "kv_layout": gcache.layout}
        if rows < 16:
            continue
        # The optional FP8 E4M3 cache layout at the same shape (scales 1).
        del gcache
        k8, v8 = cache.key[0].to(torch.float8_e4m3fn), cache.value[0].to(torch.float8_e4m3fn)
        layers8 = max(1, min(64, math.ceil(4e9 / (2 * k8.numel()))))
        gcache8 = PagedKVCache(num_layers=layers8, num_blocks=pool, block_size=16,
                               num_kv_heads=8, head_dim=128, device=device,
                               dtype=torch.float8_e4m3fn,
                               layout=resolve_layout(args.kv_layout, rows, 8))
        for layer_idx in range(layers8):
            gcache8.key[layer_idx].copy_(k8)
            gcache8.value[layer_idx].copy_(v8)
        calls[0] = 0

        def call8():
            paged_decode_attention(gq, gcache8, calls[0] % layers8, meta, gout, scale=scale,
                                   workspace=ws)
            calls[0] += 1

        seconds8 = _event_time(call8, 200)
        paged_decode_attention(gq, gcache8, 0, meta, gout, scale=scale, workspace=ws)
        OA.decode_attention(q, k8.float(), v8.float(), torch.arange(rows), blocks, offsets,
                            lengths, 16, scale, ref)
        err8 = (gout.cpu().float() - ref.float()).abs()
        algorithmic8 = (int(lengths.sum()) * 8 * 128 * 2 + 2 * rows * hq * 128 * 2
                        + 8 * sum(pages) + 8 * (3 * rows + 1))
        result[name + "_kv_fp8"] = {**_hbm(algorithmic8, seconds8),
                                    "max_abs_err_vs_oracle": round(err8.max().item(), 5),
                                    "kv_layout": gcache8.layout}
        del gcache8
    return result


def op_c2(args) -> dict:
    """C2: the fused pointwise chain at Qwen3-0.6B shapes, 256 tokens: RMSNorm
    (hidden 1024), add+RMSNorm, QK-norm + RoPE + slot-mapped KV write (one
    kernel), SiLU*up (intermediate 3072); per kernel HBM rate."""
    import torch

    from oracle import pointwise as OP
    from tinyvllm.kernels import pointwise as KP

    device = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(0)
    bf = torch.bfloat16
    T, H, hq, hkv, d, inter, pool = 256, 1024, 16, 8, 128, 3072, 16384
    x = torch.randn(T, H, generator=g).to(bf)
    res = torch.randn(T, H, generator=g).to(bf)
    w = (1 + 0.02 * torch.randn(H, generator=g)).to(bf)
    qkv = torch.randn(T, (hq + 2 * hkv) * d, generator=g).to(bf)
    qw = (1 + 0.02 * torch.randn(d, generator=g)).to(bf)
    kw = (1 + 0.02 * torch.randn(d, generator=g)).to(bf)
    pos = torch.randint(0, 2048, (T,), generator=g)
    cos, sin = OP.rope_tables(pos, d, 1e6, bf)
    slots = torch.randperm(pool, generator=g)[:T]
    gu = torch.randn(T, 2 * inter, generator=g).to(bf)
    G = lambda t: t.to(device)  # noqa: E731
    gx, gres, gw, gqkv, gqw, gkw, gcos, gsin, gslots, ggu = map(
        G, (x, res, w, qkv, qw, kw, cos, sin, slots, gu))
    kc = torch.zeros(pool, hkv, d, dtype=bf, device=device)
    vc = torch.zeros_like(kc)
    q_v = gqkv[:, :hq * d].view(T, hq, d)
    k_v = gqkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    v_v = gqkv[:, (hq + hkv) * d:].view(T, hkv, d)
    runs = {
        "rms_norm": (lambda: KP.rms_norm(gx, gw, 1e-6), T * H * 2 * 2 + H * 2),
        "add_rms_norm": (lambda: KP.add_rms_norm(gx, gres, gw, 1e-6), T * H * 2 * 4 + H * 2),
        "qk_norm_rope_kv_write": (
            lambda: KP.qk_norm_rope_store(q_v, k_v, v_v, gqw, gkw, gcos, gsin, 1e-6, 1e-6,
                                          kc, vc, gslots),
            T * (hq + 2 * hkv) * d * 2 + T * hq * d * 2 + T * 2 * hkv * d * 2
            + T * d * 2 + T * 8 + 2 * d * 2),
        "silu_and_mul": (lambda: KP.silu_and_mul(ggu), T * inter * 2 * 3),
    }
    result = {}
    total_s = total_b = 0
    for name, (fn, nbytes) in runs.items():
        s = _event_time(fn, 200)
        result[name] = _hbm(nbytes, s)
        total_s += s
        total_b += nbytes
    result["chain"] = _hbm(total_b, total_s)
    # Parity of the chain on these inputs (bit-exact KV rows, bf16 tolerance).
    q_ref, k_ref = OP.qk_norm_rope(qkv[:, :hq * d].view(T, hq, d),
                                   qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d), qw, kw, cos, sin)
    q_out, k_out = KP.qk_norm_rope_store(q_v, k_v, v_v, gqw, gkw, gcos, gsin, 1e-6, 1e-6,
                                         kc, vc, gslots, key_out=True)
    torch.cuda.synchronize()
    result["parity"] = {
        "rms_norm_max_abs": round((KP.rms_norm(gx, gw, 1e-6).cpu().float()
                                   - OP.rms_norm(x, w).float()).abs().max().item(), 5),
        "q_max_abs": round((q_out.cpu().float() - q_ref.float()).abs().max().item(), 5),
        "k_max_abs": round((k_out.cpu().float() - k_ref.float()).abs().max().item(), 5),
        "kv_write_bitexact": bool(torch.equal(kc.cpu()[slots], k_out.cpu())
                                  and torch.equal(vc.cpu()[slots], v_v.cpu())),
        "silu_max_abs": round((KP.silu_and_mul(ggu).cpu().float()
                               - OP.silu_and_mul(gu).float()).abs().max().item(), 5),
    }
    cpu = _cpu_time(lambda: (OP.rms_norm(x, w), OP.add_rms_norm(x, res, w),
                             OP.qk_norm_rope(qkv[:, :hq * d].view(T, hq, d),
                                             qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d),
                                             qw, kw, cos, sin),
                             OP.silu_and_mul(gu)))
    result["cpu_oracle_chain_us"] = round(cpu * 1e6, 1)
    return result


def op_prefill(args) -> dict:
    """Chunked-prefill paged attention at the C4 chunk shape: 512-query chunks
    of 2048-token prompts (the last chunk sees 2048 keys), Qwen3-8B heads
    (32Q/8KV, D128), 4 items; and a C5 shape: 8 chunks of 512 queries at
    24576 tokens of history with Qwen3-32B heads (64Q/8KV). MFMA roofline
    (flops of the causal region)."""
    import torch

    from oracle import attention as OA
    from tinyvllm.kernels.paged_prefill import paged_prefill_attention
    from tinyvllm.paged_kv import PagedKVCache, resolve_layout
    from tinyvllm.runtime.contracts import MultiQueryMetadata

    device = torch.device("cuda", 0)
    result = {}
    for name, items, qlen, ctx, hq in (("c4_chunk512_ctx2048_x4", 4, 512, 2048, 32),
                                       ("c4_chunk512_ctx512_x4", 4, 512, 512, 32),
                                       ("c5_chunk512_ctx24576_x8_qwen3-32b", 8, 512, 24576, 64)):
        hkv, d, bs = 8, 128, 16
        g = torch.Generator().manual_seed(0)
        pages = ctx // bs
        pool = items * pages
        cache = PagedKVCache(num_layers=1, num_blocks=pool, block_size=bs, num_kv_heads=hkv,
                             head_dim=d, device=device, dtype=torch.bfloat16,
                             layout=resolve_layout(args.kv_layout, items, hkv))
        gen = torch.Generator(device=device).manual_seed(1)
        cache.key.normal_(generator=gen)
        cache.value.normal_(generator=gen)
        blocks = torch.randperm(pool, generator=g)
        meta = MultiQueryMetadata(
            torch.arange(items + 1, device=device) * qlen, blocks.to(device),
            torch.arange(items + 1, device=device) * pages,
            torch.full((items,), ctx, device=device), qlen)
        q = torch.randn(items * qlen, hq, d, dtype=torch.bfloat16, device=device)
        out = torch.empty_like(q)
        scale = d ** -0.5
        seconds = _event_time(lambda: paged_prefill_attention(
            q, cache, 0, meta, out, scale=scale), 50)
        pairs = items * (qlen * (ctx - qlen) + qlen * (qlen + 1) // 2)
        flops = 4 * hq * d * pairs
        tflops = flops / seconds / 1e12
        # Parity on the first item.
        ref = torch.empty(qlen, hq, d, dtype=torch.bfloat16)
        OA.prefill_attention(q[:qlen].cpu(), cache.key[0].cpu(), cache.value[0].cpu(),
                             torch.tensor([0, qlen]), blocks[:pages], torch.tensor([0, pages]),
                             torch.tensor([ctx]), bs, scale, ref)
        err = (out[:qlen].cpu().float() - ref.float()).abs().max().item()
        result[name] = {"us": round(seconds * 1e6, 1), "flops": flops,
                        "TFLOP/s": round(tflops, 1), "frac_bf16_mfma": round(tflops / 2500, 4),
                        "max_abs_err_vs_oracle_item0": round(err, 5), "kv_layout": cache.layout}
    return result


OPS = {"c1": op_c1, "c2": op_c2, "prefill": op_prefill, "published": lambda args: published(args)}


E2E = {
    # name: (model, requests, prompt length(s), new tokens, shared prefix, arrivals)
    "c3": dict(model="qwen3-0.6b", requests=32, prompt=512, new=256),
    "c4": dict(model="qwen3-8b", requests=64, prompt=2048, new=256, poisson_ms=20.0),
    "c5": dict(model="qwen3-32b", requests=16, prompt=(16384, 32768), new=128,
               shared_prefix=4096),
}


def end_to_end(name: str, args) -> None:
    """One of the benchmark end-to-end configurations through the full engine (scheduler,
    chunked prefill, prefix cache, graph-replayed decode): random-init
    weights, random token-id prompts, greedy, output tokens per second."""
    import numpy as np
    import torch

    from tinyvllm import SamplingParams
    from tinyvllm.bootstrap import build_engine
    from tinyvllm.models.qwen3 import Qwen3ForCausalLM
    from tinyvllm.scheduler import ScheduleDecision

    spec = E2E[name]
    rng = np.random.default_rng(0)
    n = spec["requests"]
    if isinstance(spec["prompt"], tuple):
        lengths = rng.integers(spec["prompt"][0], spec["prompt"][1] + 1, size=n).tolist()
    else:
        lengths = [spec["prompt"]] * n
    cfg0 = qwen3_config(spec["model"], max_position=40960)
    shared = rng.integers(0, cfg0.vocab_size, size=spec.get("shared_prefix", 0)).tolist()
    prompts = [shared + rng.integers(0, cfg0.vocab_size, size=L - len(shared)).tolist()
               for L in lengths]
    max_len = max(lengths) + spec["new"] + 16
    max_model_len = 1 << (max_len - 1).bit_length()
    cfg = qwen3_config(spec["model"], max_position=max(max_model_len, 40960))
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    model = Qwen3ForCausalLM.random_init(cfg, device=device, dtype=torch.bfloat16, seed=0)
    # Worst-case KV of every request (no preemption), rounded to blocks.
    blocks = sum(-(-(L + spec["new"]) // 16) for L in lengths) + 64
    init_t0 = time.perf_counter()  # KV allocation and graph capture
    engine = build_engine(model, max_model_len=max_model_len, max_num_seqs=n,
                          max_num_batched_tokens=4096, num_blocks=blocks,
                          prefill_chunk_size=512)
    init_s = time.perf_counter() - init_t0
    params = SamplingParams(max_new_tokens=spec["new"], ignore_eos=True)
    start_ns = time.monotonic_ns()
    offsets = np.zeros(n)
    if spec.get("poisson_ms"):
        offsets = np.cumsum(rng.exponential(spec["poisson_ms"] * 1e6, size=n))
    for p, o in zip(prompts, offsets):
        engine.submit(p, params, arrival_ns=int(start_ns + o))
    torch.cuda.synchronize()
    t0 = last = time.perf_counter()
    generated = 0
    first_token: dict[int, float] = {}
    while engine.has_unfinished():
        events = engine.step()
        now = time.perf_counter()
        generated += len(events.token_events)
        for ev in events.token_events:
            first_token.setdefault(ev.request_id, now - t0)
        if engine.scheduler.last_decision is ScheduleDecision.IDLE:
            arrival = engine.scheduler.next_arrival_ns
            if arrival is not None:
                time.sleep(max(0.0, (arrival - time.monotonic_ns()) / 1e9))
        if now - last > 20:
            print(f"[{name}] {now - t0:.0f}s: {generated} tokens", file=sys.stderr, flush=True)
            last = now
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    hits = engine.scheduler.block_manager.prefix_cache.hit_tokens
    print(json.dumps({
        "metric": f"end-to-end output tok/s ({name})", "value": round(generated / elapsed, 1),
        "unit": "tok/s", "elapsed_s": round(elapsed, 2), "requests": n,
        "prompt_tokens": sum(lengths), "output_tokens": generated,
        "prefix_hit_tokens": hits, "dtype": "bf16", "engine_init_s": round(init_s, 2),
        "mean_ttft_s": round(sum(first_token.values()) / max(1, len(first_token)), 3),
        "data": "synthetic: random-init weights N(0,0.02), random token-id prompts",
        "config": {"workload": name, "model": spec["model"], **{
            k: v for k, v in spec.items() if k != "model"}},
    }), flush=True)
    engine.close()


# The reference's published serving scenarios (README performance.svg /
# arrivals-performance.svg: Qwen3-0.6B bf16, CUDA graphs + prefix caching,
# 896 MiB of KV; RTX 5060 Laptop), with its numbers: (TTFT ms, TPOT ms/tok,
# output tok/s).
PUBLISHED = {
    "1 request, 64->128": (dict(prompts=[64], new=128), (7.12, 4.73, 210.8)),
    "4 requests, 64->128": (dict(prompts=[64] * 4, new=128), (13.31, 4.90, 805.3)),
    "16 requests, 64->128": (dict(prompts=[64] * 16, new=128), (37.18, 5.75, 2668.8)),
    "Long 4 req, 1024->32": (dict(prompts=[1024] * 4, new=32), (82.80, 6.27, 345.9)),
    "Mixed 4 req, 64/512->64": (dict(prompts=[64, 512] * 2, new=64), (39.52, 5.48, 655.9)),
    "Arrivals 16 req, 64/512->64, 20 ms": (dict(prompts=[64, 512] * 8, new=64, gap_ms=20.0),
                                          (22.76, 8.34, 1369.4)),
    "Shared prefix cold, 4x832->64": (dict(prompts=[832] * 4, new=64, shared=768),
                                      (61.75, 5.73, 604.9)),
    "Shared prefix warm, 4x832->64": (dict(prompts=[832] * 4, new=64, shared=768, warm=True),
                                      (19.26, 5.74, 672.2)),
}


def run_requests(engine, prompts, new: int, gap_ns: int):
    """Submit ``prompts`` (arrivals ``gap_ns`` apart), step the engine to
    completion; (mean TTFT ms, mean TPOT ms/token, output tok/s)."""
    import numpy as np
    import torch

    from tinyvllm import SamplingParams
    from tinyvllm.scheduler import ScheduleDecision

    params = SamplingParams(max_new_tokens=new, ignore_eos=True)
    torch.cuda.synchronize()
    start = time.monotonic_ns()
    for i, prompt in enumerate(prompts):
        engine.submit(prompt, params, arrival_ns=start + i * gap_ns)
    done = []
    while engine.has_unfinished():
        events = engine.step()
        done += events.completion_events
        if engine.scheduler.last_decision is ScheduleDecision.IDLE:
            arrival = engine.scheduler.next_arrival_ns
            if arrival is not None:
                time.sleep(max(0.0, (arrival - time.monotonic_ns()) / 1e9))
    end = max(e.finished_ns for e in done)
    ttft = [(e.first_token_ns - e.arrival_ns) / 1e6 for e in done]
    tpot = [(e.finished_ns - e.first_token_ns) / 1e6 / max(1, len(e.output_token_ids) - 1)
            for e in done]
    out = sum(len(e.output_token_ids) for e in done)
    return float(np.mean(ttft)), float(np.mean(tpot)), out / ((end - start) / 1e9)


def published(args) -> dict:
    """The reference's published Qwen3-0.6B serving scenarios through this
    engine (random-init weights, random token ids, greedy, ignore_eos):
    mean TTFT and TPOT over requests and output tok/s over the makespan,
    median of ``replays``; the reference's numbers (other hardware) beside."""
    import numpy as np
    import torch

    from tinyvllm.bootstrap import build_engine
    from tinyvllm.models.qwen3 import Qwen3ForCausalLM
    from tinyvllm.paged_kv import PagedKVCache, resolve_layout

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    cfg = qwen3_config("qwen3-0.6b", max_position=40960)
    model = Qwen3ForCausalLM.random_init(cfg, device=device, dtype=torch.bfloat16, seed=0)
    per_block = PagedKVCache.bytes_per_block(
        num_layers=cfg.num_hidden_layers, block_size=16, num_kv_heads=cfg.num_key_value_heads,
        head_dim=cfg.head_dim, dtype=torch.bfloat16)
    blocks = (896 << 20) // per_block  # the reference's equal KV storage
    init_t0 = time.perf_counter()
    engine = build_engine(model, max_model_len=2048, max_num_seqs=64, num_blocks=blocks,
                          max_num_batched_tokens=4096, prefill_chunk_size=512)
    result = {"engine_init_s": round(time.perf_counter() - init_t0, 2)}
    rng = np.random.default_rng(0)
    replays = 3
    for name, (spec, ref) in PUBLISHED.items():
        runs = []
        for rep in range(replays + 1):  # the first pass warms up (not counted)
            engine.reset_prefix_cache()
            shared = rng.integers(0, cfg.vocab_size, size=spec.get("shared", 0)).tolist()

            def prompts():
                return [shared + rng.integers(0, cfg.vocab_size,
                                              size=n - len(shared)).tolist()
                        for n in spec["prompts"]]

            if spec.get("warm"):  # the shared prefix is computed once, untimed
                run_requests(engine, prompts(), spec["new"], 0)
            runs.append(run_requests(engine, prompts(), spec["new"],
                                     int(spec.get("gap_ms", 0.0) * 1e6)))
        runs = runs[1:]
        med = [float(np.median([r[i] for r in runs])) for i in range(3)]
        result[name] = {"ttft_ms": round(med[0], 2), "tpot_ms": round(med[1], 3),
                        "out_tok_s": round(med[2], 1),
                        "reference_rtx5060_laptop": {"ttft_ms": ref[0], "tpot_ms": ref[1],
                                                     "out_tok_s": ref[2]},
                        "out_tok_s_vs_reference": round(med[2] / ref[2], 2)}
        print(f"[published] {name}: {result[name]}", file=sys.stderr, flush=True)
    engine.close()
    return result


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--model", default="qwen3-8b", choices=sorted(MODELS))
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--context", type=int, default=2048)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-engine-step", action="store_true",
                    help="skip the engine-driven decode step timing beside the headline")
    ap.add_argument("--full-tables", action="store_true",
                    help="upload every block table each step (no device-resident tables)")
    ap.add_argument("--kv-layout", choices=["auto", "head_major", "token_major"],
                    default="auto",
                    help="KV-cache storage order (both keep the [slots, heads, dim] view); "
                         "auto: the engine's choice (op benchmarks: token-major)")
    ap.add_argument("--kv-cache-dtype", choices=["auto", "fp8_e4m3"], default="auto",
                    help="decode workload: KV cache in the model dtype (the metric's "
                         "configuration) or the optional FP8 E4M3 layout")
    ap.add_argument("--workload", choices=["decode", *E2E, *OPS], default="decode",
                    help="decode (the metric), an op benchmark (c1, c2, prefill) or an end-to-end configuration (c3, c4, c5, published)")
    ap.add_argument("--eager", action="store_true",
                    help="op workloads: launch kernels directly instead of graph replay")
    ap.add_argument("--kernel-only", action="store_true",
                    help="run only the decode-attention kernel (for PMC passes)")
    ap.add_argument("--summarize-profile", metavar="DIR",
                    help="print a summary of a rocprofv3 output directory and exit")
    args = ap.parse_args()
    if args.summarize_profile:
        summarize_profile(args.summarize_profile)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode path is single-GPU by design "
              "(multi-GPU sharding is documented, not built); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    if args.kernel_only:
        kernel_only(args)
        return
    if args.workload in OPS:
        import torch

        global EAGER_OPS
        EAGER_OPS = args.eager
        torch.cuda.set_device(0)
        print(json.dumps({"workload": args.workload, "dtype": "bf16",
                          "data": "synthetic, seeded", **OPS[args.workload](args)}), flush=True)
        return
    if args.workload != "decode":
        end_to_end(args.workload, args)
        return

    import torch

    from tinyvllm.executor import Executor
    from tinyvllm.models.qwen3 import Qwen3ForCausalLM

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    bs = 16
    total_steps = args.steps + args.warmup + 2
    max_len = args.context + total_steps + 16
    max_model_len = 1 << max(12, (max_len - 1).bit_length())  # e.g. 4096
    cfg = qwen3_config(args.model, max_position=max(max_model_len, 40960))
    model = Qwen3ForCausalLM.random_init(cfg, device=device, dtype=torch.bfloat16, seed=0)
    pages = math.ceil(max_len / bs)
    num_blocks = args.batch * pages
    # Every step carries exactly `batch` rows: capture that one graph.
    fp8 = args.kv_cache_dtype == "fp8_e4m3"
    executor = Executor(model, block_size=bs, num_blocks=num_blocks,
                        max_model_len=max_model_len, max_num_seqs=args.batch,
                        graph_sizes=(args.batch,),
                        kv_cache_dtype=torch.float8_e4m3fn if fp8 else None,
                        kv_cache_layout=args.kv_layout,
                        prefill_graph_tokens=0)  # every timed step is a decode step
    cache = executor.runner.kv_cache
    gen = torch.Generator(device=device).manual_seed(1)
    if fp8:  # N(0, 1) values quantised layer by layer
        for layer in range(cache.num_layers):
            for t in (cache.key[layer], cache.value[layer]):
                t.copy_(torch.randn(t.shape, generator=gen, device=device))
    else:
        cache.key.normal_(generator=gen)
        cache.value.normal_(generator=gen)
    workload = DecodeWorkload(args.batch, args.context, bs, num_blocks, cfg.vocab_size)
    workload.full_tables = args.full_tables

    # Pipelined like the engine: the host builds and launches step i+1
    # while the GPU runs step i.
    pending = workload.run(executor, args.warmup)
    torch.cuda.synchronize()
    stats = executor.runner.decode_inputs.stats
    before = dict(stats)
    t0 = time.perf_counter()
    pending = workload.run(executor, args.steps, pending)
    workload.tokens = list(pending.result().sampled_token_ids)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tok_s = args.batch * args.steps / elapsed
    steps = max(1, stats["steps"] - before["steps"])
    inputs_cost = {  # per step: host packing of the decode inputs, H2D upload
        "host_prepare_us": round((stats["host_ns"] - before["host_ns"]) / steps / 1e3, 1),
        "h2d_bytes": round((stats["bytes"] - before["bytes"]) / steps),
        "table_entries_uploaded": round((stats["table_entries"] - before["table_entries"])
                                        / steps, 2),
        "device_resident_tables": not args.full_tables,
    }

    roof = attention_roofline(executor, workload, cfg, headline=(
        args.model == "qwen3-8b" and args.batch == 64 and args.context == 2048
        and not fp8))
    engine_line = None
    if not args.no_engine_step:
        # The headline executor's KV stays allocated; the engine adds its own.
        engine_line = engine_decode_step(model, cfg, args.batch, args.context, args.steps,
                                         args.warmup)
        engine_line["engine_vs_ms_per_step"] = round(
            engine_line["engine_ms_per_step"] / (elapsed / args.steps * 1e3), 3)
    cpu = None if args.no_cpu_baseline else cpu_baseline(cfg, args.batch, args.context)
    line = {
        "metric": "decode tok/s Qwen3-8B bs64 ctx2k; paged-attn HBM GB/s and % of peak",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights N(0,0.02), random token ids, "
                "2048-token contexts' KV filled N(0,1)",
        "config": {"workload": f"{args.model} decode bs{args.batch} ctx{args.context}",
                   "model": args.model, "global_batch": args.batch,
                   "seq_len": args.context, "parallelism": "single-gpu",
                   "attention_backend": "hip", "graphs": True,
                   "kv_cache_dtype": "fp8_e4m3" if fp8 else "bf16",
                   "kv_cache_layout": cache.layout},
        "roofline": roof,
        "cpu_baseline": cpu,
        "decode_inputs": inputs_cost,
        "engine_ms_per_step": engine_line and engine_line["engine_ms_per_step"],
        "engine_step": engine_line,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
