"""Model-level parity at the benchmark architectures (configs C3, C4, C5).

* C3: the whole Qwen3-0.6B (28 layers, vocab 151936, tied embeddings) with
  N(0, 0.02) weights, 32 requests of 512 random ids, 256 new tokens each,
  greedy, through the engine (chunked prefill, graph-replayed decode at
  batch 32). 8 rows are checked teacher-forced against the CPU oracle model
  over all their tokens (2048 steps).
* C4: Qwen3-8B (hidden 4096, 32Q/8KV, FFN 12288, vocab 151936, 36 layers,
  untied LM head), 64 requests of 2048 ids, chunked prefill 512, Poisson
  arrivals (mean gap 20 ms on a simulated clock), greedy. The full 36-layer
  model: 2 rows x 64 tokens teacher-forced against the 36-layer oracle, and
  layer 20 of a live batch-64 decode step (attention output, post-attention
  norm, residual and KV write against the oracle layer on the engine's own
  cache). A 2-layer model of the same geometry checks pipelined == serial
  tokens and that all blocks return to the pool.
* C5: the full 64-layer Qwen3-32B (hidden 5120, 64Q/8KV, FFN 25600), 16
  requests of 16k-32k ids sharing a 4096-token prefix through the prefix
  cache, 128 new tokens: the live-layer check at layer 40, the first
  layer's K/V of the shared prefix against the oracle, and shared prefix
  pages.

Greedy agreement (north star: >= 99% of steps) is teacher-forced: a step
agrees when our token is the oracle's argmax for the same context, or when
the oracle scores it within one bf16 ulp of its best logit (a tie at bf16
resolution that another summation order may legitimately break). At the
36-layer depth one ulp is below what bf16 rounding alone does to the
logits: the oracle recomputed with its linear layers summed in four slices
(the same rounding points, another fp32 order) moves them by up to ~10 ulps
and misses its own argmax on a few percent of steps. There a step also
agrees when the deficit is within that step's largest such move, and at
least 90% of steps must still agree within one ulp.
Reference path: models/qwen3.py:458-494 and :703-717, executor.py:126-141.
"""

import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, assert_within_ulp, bf16_ulp
from oracle import attention as OA
from oracle import model as OM
from oracle import pointwise as OP

pytestmark = pytest.mark.gpu

VOCAB = 151936
GEOMETRY = {  # hidden, intermediate, layers, q heads, kv heads, tied embeddings
    "qwen3-0.6b": (1024, 3072, 28, 16, 8, True),
    "qwen3-8b": (4096, 12288, 36, 32, 8, False),
    "qwen3-32b": (5120, 25600, 64, 64, 8, False),
}


def oracle_config(name, layers=None, max_position=4096):
    h, inter, n, hq, hkv, tied = GEOMETRY[name]
    return OM.TinyQwen3(vocab_size=VOCAB, hidden_size=h, intermediate_size=inter,
                        num_hidden_layers=layers or n, num_attention_heads=hq,
                        num_key_value_heads=hkv, head_dim=128, tie_word_embeddings=tied,
                        max_position_embeddings=max_position)


def teacher_forced(cfg, weights, prompt, ours, label="", reorder_band=False):
    """(agreeing steps, worst oracle logit deficit in ulps) of our greedy
    tokens against one oracle forward over prompt + ours. A step agrees when
    the oracle's best logit exceeds its logit of our token (the deficit) by
    at most one bf16 ulp of the best.

    ``reorder_band``: a second oracle forward with every linear layer summed
    in 4 slices (the same roundings, another fp32 summation order) measures
    how far bf16 rounding alone moves this step's logits; a step also agrees
    when the deficit is within that step's largest such move. Returns
    (agree, worst, strict agreements, reordered-oracle misses) then.
    Prints the per-step deficits when ``label`` is given."""
    rows = [len(prompt) - 1 + i for i in range(len(ours))]
    seq = list(prompt) + list(ours)
    logits = OM.forward(cfg, weights, seq, logit_rows=rows)
    band = alt_miss = None
    if reorder_band:
        alt = OM.forward(cfg, weights, seq, logit_rows=rows, k_slices=4)
        band = (logits - alt).abs().amax(-1)
        alt_miss = 0
    agree, strict, worst, deficits = 0, 0, 0.0, []
    for i, token in enumerate(ours):
        row = logits[i]
        best = float(row.max())
        ulp = bf16_ulp(best)
        deficit = (best - float(row[token])) / ulp
        deficits.append(deficit)
        worst = max(worst, deficit)
        strict += int(deficit <= 1.0)
        allowed = 1.0 if band is None else max(1.0, float(band[i]) / ulp)
        agree += int(deficit <= allowed)
        if band is not None:
            alt_miss += int((best - float(row[int(alt[i].argmax())])) / ulp > 1.0)
    if label:
        ties = sum(0.0 < d <= 1.0 for d in deficits)
        extra = "" if band is None else (
            f"; reordered oracle: {alt_miss} misses beyond one ulp, logit moves up to "
            f"{float(band.max()):.3f} (mean of row maxima {float(band.mean()):.3f})")
        print(f"{label}: {agree}/{len(ours)} agree, {strict} within one ulp "
              f"({ties} ties){extra}; per-step deficits (ulp) "
              + " ".join(f"{d:.1f}" for d in deficits), flush=True)
    if band is None:
        return agree, worst
    return agree, worst, strict, alt_miss


def run_engine(engine, prompts, params, arrivals_ns=None, step_ns=2_000_000,
               on_step=None):
    """Step the engine on a simulated clock until every request finishes;
    returns each prompt's output ids (submission order)."""
    from tinyvllm.scheduler import ScheduleDecision

    arrivals_ns = arrivals_ns if arrivals_ns is not None else [0] * len(prompts)
    ids = [engine.submit(p, params, arrival_ns=int(a)) for p, a in zip(prompts, arrivals_ns)]
    out = {rid: [] for rid in ids}
    now = 0
    while engine.has_unfinished():
        events = engine.step(now_ns=now)
        for ev in events.token_events:
            out[ev.request_id].append(ev.token_id)
        if on_step is not None:
            on_step(out)
        now += step_ns
        if engine.scheduler.last_decision is ScheduleDecision.IDLE:
            nxt = engine.scheduler.next_arrival_ns
            if nxt is not None:
                now = max(now, nxt)
    return [out[rid] for rid in ids]


def blocks_for(lengths, new):
    return sum(-(-(n + new) // 16) for n in lengths) + 64


# ------------------------------------------------------- live layer probe --

class LayerProbe:
    """Records one decode-only step's inputs and outputs of decoder layer
    ``idx`` (eager forward hooks; the runner's graphs are bypassed for the
    armed step)."""

    def __init__(self, model, idx, rows):
        self.layer = model.model.layers[idx]
        self.idx, self.rows = idx, rows
        self.armed, self.cap, self.request_ids = False, None, ()
        self._buf = {}
        self.handles = [
            self.layer.register_forward_pre_hook(self._pre, with_kwargs=True),
            self.layer.register_forward_hook(self._post, with_kwargs=True),
            self.layer.self_attn.o_proj.register_forward_pre_hook(self._attn_out),
            self.layer.mlp.register_forward_pre_hook(self._mlp_in),
        ]

    def _pre(self, module, args, kwargs):
        kv = kwargs["attention"].kv
        if not self.armed or kv.prefill is not None or kv.decode is None \
                or kv.decode.query_rows.numel() != self.rows:
            self._buf = {}
            return
        hidden = args[0]
        parts = getattr(hidden, "partials", None)
        d = kv.decode
        self._buf = dict(
            hidden=(parts if parts is not None else hidden).detach().clone(),
            split=parts is not None,
            residual=None if kwargs["residual"] is None else kwargs["residual"].clone(),
            slots=kv.slot_mapping.clone(), blocks=d.block_table_ids.clone(),
            offsets=d.block_table_offsets.clone(), lengths=d.context_lens.clone())

    def _attn_out(self, module, args):
        if self._buf:
            self._buf["attn"] = args[0].detach().clone()

    def _mlp_in(self, module, args):
        if self._buf:
            self._buf["normed"] = args[0].detach().clone()

    def _post(self, module, args, kwargs, output):
        if self._buf and self.cap is None:
            self._buf["residual_out"] = output[1].detach().clone()
            cap = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in self._buf.items()}
            # Decode rows read ceil(length / 16) table entries from offsets[r]
            # (device-resident tables: one pitched row per request slot);
            # restate them as the CSR the oracle takes.
            pages = (cap["lengths"] + 15) // 16
            tables = [cap["blocks"][int(o):int(o) + int(n)]
                      for o, n in zip(cap["offsets"][:-1], pages)]
            cap["blocks"] = torch.cat(tables)
            cap["offsets"] = torch.cat((torch.zeros(1, dtype=torch.long), pages.cumsum(0)))
            self.cap = cap
        self._buf = {}

    def step_eager(self, engine, now_ns):
        """One engine step with this probe armed and decode graphs bypassed."""
        runner = engine.executor.runner
        graphs, runner.decode_graphs = runner.decode_graphs, None
        forward = runner._forward

        def recording(batch, *args, **kwargs):  # batch row -> request id
            if self.cap is None:
                self.request_ids = tuple(batch.request_ids)
            return forward(batch, *args, **kwargs)

        runner._forward = recording
        self.armed = True
        try:
            return engine.step(now_ns=now_ns)
        finally:
            self.armed = False
            runner.decode_graphs = graphs
            del runner._forward

    def close(self):
        for h in self.handles:
            h.remove()


def model_and_weights(cfg, device, seed):
    """Our model with random-init weights N(0, 0.02) (norm weights 1),
    generated on the GPU, and the same weights on the CPU in the oracle's
    naming (packed q|k|v and gate|up, as the model stores them)."""
    from tinyvllm.models.qwen3 import Qwen3ForCausalLM

    model = Qwen3ForCausalLM.random_init(_our_config(cfg), device=device, seed=seed)
    weights = {name: p.detach().cpu() for name, p in model.named_parameters()}
    if cfg.tie_word_embeddings:
        weights.pop("lm_head.weight", None)
    return model, weights


def layer_weights(model, idx):
    """Layer ``idx``'s weights on the CPU, oracle names."""
    layer = model.model.layers[idx]
    return {
        "in": layer.input_layernorm.weight.detach().cpu(),
        "post": layer.post_attention_layernorm.weight.detach().cpu(),
        "qkv": layer.self_attn.qkv_proj.weight.detach().cpu(),
        "o": layer.self_attn.o_proj.weight.detach().cpu(),
        "qn": layer.self_attn.q_norm.weight.detach().cpu(),
        "kn": layer.self_attn.k_norm.weight.detach().cpu(),
    }


def check_kv(our_k, our_v, k, v):
    """K/V rows the engine wrote vs the oracle's projections. The write itself
    is a bit copy (checked bit-exact by the kernel tests); the values come
    from our GEMM, whose summation order may flip one rounding of the
    projection: V within one bf16 ulp, K (then normalised and rotated)
    within two; mean relative error within 1e-3 for both."""
    assert_within_ulp(our_v, v, ulps=1.0)
    assert_within_ulp(our_k, k, ulps=2.0)


def check_layer_against_oracle(cap, w, key_cache, value_cache, cfg, block_size=16):
    """The attention half of one decoder layer restated on the CPU from the
    captured input, over the engine's own KV cache (layer copy, CPU):
    our KV write and attention output must be within the bf16 bar of the
    oracle's, the residual sum within two rounding flips, the post-attention
    norm within the bf16 bar of the oracle norm of our residual."""
    hq, hkv, d, eps = cfg.num_attention_heads, cfg.num_key_value_heads, 128, 1e-6
    hidden = cap["hidden"]
    if cap["split"]:  # split-K partials: summed in order, rounded once
        acc = hidden[0].clone()
        for p in range(1, hidden.shape[0]):
            acc = acc + hidden[p]
        hidden = acc.to(torch.bfloat16)
    if cap["residual"] is None:
        x, res = OP.rms_norm(hidden, w["in"], eps), hidden
    else:
        x, res = OP.add_rms_norm(hidden, cap["residual"], w["in"], eps)
    t = x.shape[0]
    qkv = OM.linear(x, w["qkv"])
    q = qkv[:, :hq * d].view(t, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    positions = cap["lengths"] - 1
    cos, sin = OP.rope_tables(positions, d, cfg.rope_theta, torch.bfloat16)
    q, k = OP.qk_norm_rope(q, k, w["qn"], w["kn"], cos, sin, eps, eps)
    slots = cap["slots"]
    check_kv(key_cache[slots], value_cache[slots], k, v)  # the fused KV write
    attn = torch.empty_like(q)
    OA.decode_attention(q, key_cache, value_cache, torch.arange(t), cap["blocks"],
                        cap["offsets"], cap["lengths"], block_size, d ** -0.5, attn)
    assert_bf16_close(cap["attn"].view(t, hq, d), attn)
    o = OM.linear(attn.view(t, hq * d), w["o"])
    normed, res2 = OP.add_rms_norm(o, res, w["post"], eps)
    # The residual stream grows with depth (|x| ~ 20 at layer 20 of the 8B),
    # where max abs 2e-2 is below one ulp: allow one rounding flip of the
    # projection and one of the sum (2 ulps of the operands' magnitude).
    assert_within_ulp(cap["residual_out"], res2,
                      scale=torch.maximum(o.float().abs(), res.float().abs()), ulps=2.0)
    # The norm given our residual: the strict bar.
    assert_bf16_close(cap["normed"], OP.rms_norm(cap["residual_out"], w["post"], eps))
    # Against the independent oracle chain, element by element: the residual
    # differs by at most 2 ulps of m = max(|o|, |res|) (checked above); where
    # o and the residual cancel that is many ulps of the sum itself, so the
    # bound is carried through the norm: 2 ulp(m) x rstd x |w|, plus the
    # norm's own two roundings (of x * rstd, then of the weight product),
    # with the bar's 2e-2 as the floor; the mean error at the bar.
    rstd = torch.rsqrt(res2.float().pow(2).mean(-1, keepdim=True) + eps)
    ulp_in = _ulp(torch.maximum(o.float().abs(), res.float().abs()))
    e = normed.float()
    allowed = torch.clamp(2 * ulp_in * rstd * w["post"].float().abs() + 2 * _ulp(e.abs()),
                          min=2e-2)
    excess = ((cap["normed"].float() - e).abs() / allowed).max().item()
    assert excess <= 1.0, f"post-attention norm error {excess:.2f}x its element-wise bound"
    assert_bf16_close(cap["normed"], normed, max_abs=float("inf"))


def _ulp(mag):
    """One bf16 ulp at each |value| (7 fraction bits)."""
    return torch.exp2(torch.floor(torch.log2(mag.clamp_min(2.0 ** -126))) - 7)


def probe_run(engine, model, idx, prompts, params, arrivals_ns, step_ns=50_000_000):
    """Run to completion; once every request has two tokens, one decode step
    runs eagerly with the layer probe armed, and the probed layer's cache is
    copied to the CPU right after it. A simulated step of 50 ms lets all
    Poisson arrivals (mean gap 20 ms) land within the prefill phase, so some
    step decodes every request at once."""
    probe = LayerProbe(model, idx, rows=len(prompts))
    state = {"done": False, "cache": None}
    from tinyvllm.scheduler import ScheduleDecision

    ids = [engine.submit(p, params, arrival_ns=int(a)) for p, a in zip(prompts, arrivals_ns)]
    out = {rid: [] for rid in ids}
    now = 0
    try:
        while engine.has_unfinished():
            ready = not state["done"] and all(len(v) >= 2 for v in out.values())
            events = probe.step_eager(engine, now) if ready else engine.step(now_ns=now)
            if ready and probe.cap is not None:
                torch.cuda.synchronize()
                cache = engine.executor.runner.kv_cache
                state["cache"] = (cache.key[idx].cpu(), cache.value[idx].cpu())
                state["done"] = True
            for ev in events.token_events:
                out[ev.request_id].append(ev.token_id)
            now += step_ns
            if engine.scheduler.last_decision is ScheduleDecision.IDLE:
                nxt = engine.scheduler.next_arrival_ns
                if nxt is not None:
                    now = max(now, nxt)
    finally:
        probe.close()
    assert probe.cap is not None, "no decode-only step with every row was probed"
    probe.cap["row_of"] = {ids.index(rid): r for r, rid in enumerate(probe.request_ids)}
    return probe.cap, state["cache"], [out[rid] for rid in ids]


# ---------------------------------------------------------------------- C3 --

def test_c3_qwen3_0_6b_engine_greedy_matches_oracle(device):
    """The whole C3 workload (32 requests x 512 ids, 256 new tokens each,
    greedy); 8 rows spread over the batch are teacher-forced against the
    oracle model over all 256 tokens (2048 steps)."""
    from tinyvllm import SamplingParams
    from tinyvllm.bootstrap import build_engine

    cfg = oracle_config("qwen3-0.6b", max_position=1024)
    model, weights = model_and_weights(cfg, device, seed=3)
    g = torch.Generator().manual_seed(33)
    prompts = [torch.randint(0, VOCAB, (512,), generator=g).tolist() for _ in range(32)]
    new = 256
    engine = build_engine(model, max_model_len=1024, max_num_seqs=32,
                          max_num_batched_tokens=4096, num_blocks=blocks_for([512] * 32, new),
                          prefill_chunk_size=512)
    outs = run_engine(engine, prompts, SamplingParams(max_new_tokens=new, ignore_eos=True))
    assert all(len(o) == new for o in outs)
    manager = engine.scheduler.block_manager
    assert manager.free_block_count == manager.pool.num_blocks
    engine.close()
    agree = total = 0
    worst = 0.0
    for r in (0, 4, 9, 13, 20, 22, 27, 31):
        a, w = teacher_forced(cfg, weights, prompts[r], outs[r], label=f"C3 row {r}")
        agree, total, worst = agree + a, total + new, max(worst, w)
    print(f"C3 teacher-forced agreement {agree}/{total}, worst deficit {worst:.2f} ulp")
    assert total >= 2048
    assert agree / total >= 0.99, (agree, total, worst)


# ---------------------------------------------------------------------- C4 --

def _c4_workload(n=64, prompt=2048, seed=44):
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, VOCAB, size=prompt).tolist() for _ in range(n)]
    arrivals = np.cumsum(rng.exponential(20e6, size=n)).astype(np.int64).tolist()
    return prompts, arrivals


def test_c4_qwen3_8b_geometry_engine_tokens_match_oracle(device):
    """Two layers of the Qwen3-8B geometry through the C4 workload: greedy
    tokens agree with the oracle, pipelined steps give the same tokens as
    serial ones, and every block returns to the pool."""
    from tinyvllm import SamplingParams
    from tinyvllm.bootstrap import build_engine

    cfg = oracle_config("qwen3-8b", layers=2, max_position=4096)
    model, weights = model_and_weights(cfg, device, seed=4)
    prompts, arrivals = _c4_workload()
    new = 6
    params = SamplingParams(max_new_tokens=new, ignore_eos=True)
    runs = []
    for pipelined in (True, False):
        engine = build_engine(model, max_model_len=4096, max_num_seqs=64,
                              max_num_batched_tokens=4096,
                              num_blocks=blocks_for([2048] * 64, new),
                              prefill_chunk_size=512, pipelined=pipelined)
        assert engine._pipelined == pipelined
        runs.append(run_engine(engine, prompts, params, arrivals))
        manager = engine.scheduler.block_manager
        assert manager.free_block_count == manager.pool.num_blocks
        assert not engine.scheduler.has_unresolved_steps
        engine.close()
    assert runs[0] == runs[1]
    agree = total = 0
    worst = 0.0
    for r in (0, 63):
        a, w = teacher_forced(cfg, weights, prompts[r], runs[0][r], label=f"C4 2-layer row {r}")
        agree, total, worst = agree + a, total + new, max(worst, w)
    print(f"C4 teacher-forced agreement {agree}/{total}, worst deficit {worst:.2f} ulp")
    assert agree / total >= 0.99, (agree, total, worst)


@pytest.mark.timeout(900)
def test_c4_qwen3_8b_full_depth_engine_greedy_and_live_layer_match_oracle(device):
    """The full 36-layer Qwen3-8B (random N(0, 0.02), norms 1, untied LM
    head) through the C4 workload (64 x 2048 ids, chunked prefill 512,
    Poisson arrivals, 64 new tokens each, graph-replayed decode at batch 64):

    * greedy tokens: rows 0 and 63 (first and last to arrive) teacher-forced
      against the 36-layer oracle model over all 64 tokens (128 steps; one
      oracle forward of a row is ~29 TFLOP of fp32 CPU work, and a second
      one with the linear layers summed in slices gives each step's rounding
      band);
    * in one decode step at batch 64 (contexts 2050-2100) layer 20 is
      recomputed by the oracle from its captured input over the engine's own
      cache;
    * layer 0's K/V of request 0's whole prompt (written by chunked prefill)
      against the oracle."""
    from tinyvllm import SamplingParams
    from tinyvllm.bootstrap import build_engine

    cfg = oracle_config("qwen3-8b", max_position=4096)
    model, weights = model_and_weights(cfg, device, seed=8)
    assert "lm_head.weight" in weights and len(
        [n for n in weights if n.endswith("down_proj.weight")]) == 36
    prompts, arrivals = _c4_workload(seed=45)
    new = 64
    engine = build_engine(model, max_model_len=4096, max_num_seqs=64,
                          max_num_batched_tokens=4096, num_blocks=blocks_for([2048] * 64, new),
                          prefill_chunk_size=512)
    params = SamplingParams(max_new_tokens=new, ignore_eos=True)
    cap, (kc, vc), outs = probe_run(engine, model, 20, prompts, params, arrivals)
    assert all(len(o) == new for o in outs)
    assert int(cap["lengths"].min()) >= 2049
    check_layer_against_oracle(cap, layer_weights(model, 20), kc, vc, cfg)
    _check_layer0_prompt_kv(engine, model, cfg, prompts[0], cap, row=cap["row_of"][0])
    engine.close()
    del engine, kc, vc
    torch.cuda.empty_cache()
    agree = total = strict = alt_miss = 0
    worst = 0.0
    for r in (0, 63):
        a, w, st, am = teacher_forced(cfg, weights, prompts[r], outs[r],
                                      label=f"C4 36-layer row {r}", reorder_band=True)
        agree, total, worst = agree + a, total + new, max(worst, w)
        strict, alt_miss = strict + st, alt_miss + am
    print(f"C4 36-layer teacher-forced agreement {agree}/{total} within the reorder band, "
          f"{strict}/{total} within one ulp (the reordered oracle itself: {alt_miss} "
          f"misses), worst deficit {worst:.2f} ulp")
    assert total >= 32
    # At 36 layers a reordering of the oracle's own fp32 sums moves the bf16
    # logits by up to ~10 ulps and flips a few percent of near-tied argmaxes
    # by itself; a kernel bug moves them by tens of ulps on most steps.
    assert strict / total >= 0.9, (strict, total, worst)
    assert agree / total >= 0.99, (agree, total, worst)


def _our_config(cfg):
    from tinyvllm.models.qwen3 import Qwen3Config

    return Qwen3Config.from_dict(dict(
        model_type="qwen3", vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
        max_position_embeddings=cfg.max_position_embeddings, rope_theta=cfg.rope_theta,
        tie_word_embeddings=cfg.tie_word_embeddings))


def _check_layer0_prompt_kv(engine, model, cfg, prompt, cap, row, count=None):
    """Layer 0's K/V of ``prompt`` (the first ``count`` tokens) in the
    engine's cache - found through the probed step's block table of ``row``
    - against the oracle's projection of the embeddings."""
    hq, hkv, d, eps = cfg.num_attention_heads, cfg.num_key_value_heads, 128, 1e-6
    n = count or len(prompt)
    ids = torch.tensor(prompt[:n])
    emb = model.model.embed_tokens.weight[ids.to(model.model.embed_tokens.weight.device)].cpu()
    w = layer_weights(model, 0)
    x = OP.rms_norm(emb, w["in"], eps)
    qkv = OM.linear(x, w["qkv"])
    q = qkv[:, :hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(n, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(n, hkv, d)
    cos, sin = OP.rope_tables(torch.arange(n), d, cfg.rope_theta, torch.bfloat16)
    _, k = OP.qk_norm_rope(q, k, w["qn"], w["kn"], cos, sin, eps, eps)
    table = cap["blocks"][int(cap["offsets"][row]):int(cap["offsets"][row + 1])]
    pos = torch.arange(n)
    slots = (table[pos // 16] * 16 + pos % 16).to(model.model.embed_tokens.weight.device)
    cache = engine.executor.runner.kv_cache
    check_kv(cache.key[0].index_select(0, slots).cpu(),
             cache.value[0].index_select(0, slots).cpu(), k, v)


# ---------------------------------------------------------------------- C5 --

@pytest.mark.timeout(600)
def test_c5_qwen3_32b_long_context_shared_prefix(device):
    """The full 64-layer Qwen3-32B (random N(0, 0.02), norms 1), 16 requests
    of U[16k, 32k] random ids sharing a 4096-token prefix, 128 new tokens
    each: prefix pages are shared (not copied) between rows, layer 0's K/V
    of the prefix matches the oracle, and in a live decode step (split-K
    over ~24k-token contexts, 64Q/8KV) layer 40 matches the oracle layer
    over the engine's cache."""
    from tinyvllm import SamplingParams
    from tinyvllm.bootstrap import build_engine
    from tinyvllm.models.qwen3 import Qwen3ForCausalLM

    cfg = oracle_config("qwen3-32b", max_position=40960)
    model = Qwen3ForCausalLM.random_init(_our_config(cfg), device=device, seed=32)
    rng = np.random.default_rng(55)
    lengths = rng.integers(16384, 32768 + 1, size=16).tolist()
    shared = rng.integers(0, VOCAB, size=4096).tolist()
    prompts = [shared + rng.integers(0, VOCAB, size=n - 4096).tolist() for n in lengths]
    engine = build_engine(model, max_model_len=40960, max_num_seqs=16,
                          max_num_batched_tokens=4096, num_blocks=blocks_for(lengths, 128),
                          prefill_chunk_size=512)
    # ~100 chunked-prefill steps: early requests keep decoding until the last
    # prompt is in, so one step decodes all 16 rows.
    params = SamplingParams(max_new_tokens=128, ignore_eos=True)
    cap, (kc, vc), outs = probe_run(engine, model, 40, prompts, params, [0] * 16)
    assert all(len(o) == 128 for o in outs)
    prefix_pages = 4096 // 16
    tables = [cap["blocks"][int(cap["offsets"][r]):int(cap["offsets"][r + 1])]
              for r in range(16)]
    sharing = sum(torch.equal(t[:prefix_pages], tables[0][:prefix_pages]) for t in tables[1:])
    assert sharing >= 8, sharing  # most requests reuse the published prefix pages
    assert engine.scheduler.block_manager.prefix_cache.hit_tokens >= 8 * 4096
    check_layer_against_oracle(cap, layer_weights(model, 40), kc, vc, cfg)
    _check_layer0_prompt_kv(engine, model, cfg, prompts[0], cap, row=cap["row_of"][0],
                            count=4096)
    engine.close()
