"""Scheduler / BlockManager / PrefixCache / Engine on the CPU with a fake
executor that simulates the paged KV cache slot by slot.

Every batch goes through the runner's own CPU validation (slot =
table[p // bs] * bs + p % bs, prefix sharing rules), every write records
(request, position, token) in its slot, and every attended position must
read back exactly the token the request holds there - so slot arithmetic,
chunked prefill and prefix-block sharing are checked bit-exactly, with no
GPU."""
import random

import numpy as np
import pytest

from tinyvllm.batch import StepResult
from tinyvllm.engine import Engine, GenerateRequest
from tinyvllm.executor import ExecutorCapabilities
from tinyvllm.request import RequestStatus, SamplingParams
from tinyvllm.runtime.runner import ModelRunner
from tinyvllm.scheduler import Scheduler

VOCAB = 97
EOS = 5


def next_token(history):
    """Deterministic 'model': depends on the whole context."""
    return (sum((i + 1) * t for i, t in enumerate(history[-8:])) * 31 + len(history)) % VOCAB


class SimExecutor:
    def __init__(self, *, block_size, num_blocks, max_model_len, max_batch):
        self.capabilities = ExecutorCapabilities(vocab_size=VOCAB, max_model_len=max_model_len,
                                                 kv_block_size=block_size, kv_num_blocks=num_blocks,
                                                 max_batch_size=max_batch)
        self.bs = block_size
        self.slots = {}   # slot -> token written there
        self.validator = ModelRunner.__new__(ModelRunner)
        self.validator.vocab_size = VOCAB
        self.validator.max_model_len = max_model_len

        class _Cache:
            pass
        self.cache = _Cache()
        self.cache.block_size, self.cache.num_blocks = block_size, num_blocks
        self.batches = 0
        self.fail_at = None
        self.released = []

    def execute(self, batch):
        self.batches += 1
        if self.fail_at == self.batches:
            raise RuntimeError("injected executor failure")
        self.validator._validate(batch, self.cache)
        out = []
        for i, rid in enumerate(batch.request_ids):
            start, end = batch.q_offsets[i], batch.q_offsets[i + 1]
            before, after = batch.context_lens_before[i], batch.context_lens_after[i]
            # Ground truth: the request's own tokens (prompt + sampled so far).
            hist = self.scheduler.get_request(rid).token_slice(0, after)
            assert list(batch.input_ids[start:end]) == hist[before:after]
            for t, slot in zip(range(start, end), batch.kv_slot_mapping[start:end]):
                self.slots[slot] = batch.input_ids[t]
            # Read back the whole context through the block table.
            toff = batch.kv_block_table_offsets
            table = batch.kv_block_table_ids[toff[i]:toff[i + 1]]
            for p in range(after):
                slot = table[p // self.bs] * self.bs + p % self.bs
                assert self.slots.get(slot) == hist[p], (rid, p)
            if end - 1 in batch.sample_token_indices:
                out.append(next_token(hist[:after]))
        return StepResult(batch.plan_id, batch.sample_request_ids, tuple(out))

    def release(self, request_id):
        self.released.append(request_id)

    def clear(self):
        pass


def expected(prompt, params, max_model_len):
    seq, out = list(prompt), []
    while len(out) < params.max_new_tokens and len(seq) < max_model_len:
        tok = next_token(seq)
        out.append(tok)
        seq.append(tok)
        if tok == EOS and not params.ignore_eos:
            break
    return out


def make_engine(*, bs=4, blocks=96, max_len=96, seqs=4, tokens=24, chunk=10,
                prefix=True, clock=None):
    ex = SimExecutor(block_size=bs, num_blocks=blocks, max_model_len=max_len, max_batch=seqs)
    sched = Scheduler(max_active_requests=seqs, max_step_requests=seqs,
                      max_scheduled_tokens=tokens, prefill_chunk_size=chunk,
                      max_model_len=max_len, prefill_reserve_tokens=4,
                      prefill_reserve_requests=1, kv_block_size=bs, kv_num_blocks=blocks,
                      eos_token_ids=[EOS], enable_prefix_caching=prefix)
    kwargs = {} if clock is None else {"clock": clock, "sleep": lambda s: None}
    ex.scheduler = sched
    return Engine(sched, ex, **kwargs), ex


@pytest.mark.parametrize("prefix", [True, False])
def test_many_requests_chunked_prefill_matches_model(prefix):
    rng = random.Random(0)
    engine, ex = make_engine(prefix=prefix)
    reqs = []
    for _ in range(12):
        prompt = [rng.randrange(6, VOCAB) for _ in range(rng.randrange(1, 40))]
        params = SamplingParams(max_new_tokens=rng.randrange(1, 20), ignore_eos=rng.random() < 0.3)
        reqs.append(GenerateRequest(prompt, params))
    outputs = engine.generate(reqs)
    for req, out in zip(reqs, outputs):
        assert out.status is RequestStatus.FINISHED
        assert list(out.output_token_ids) == expected(req.prompt_token_ids, req.sampling, 96)
    assert engine.scheduler.block_manager.free_block_count == 96  # everything released


def test_shared_prefixes_hit_the_cache_and_stay_exact():
    rng = random.Random(1)
    engine, ex = make_engine(blocks=80, max_len=80, chunk=8, tokens=20)
    shared = [rng.randrange(6, VOCAB) for _ in range(30)]
    reqs = [GenerateRequest(shared + [rng.randrange(6, VOCAB) for _ in range(rng.randrange(1, 6))],
                            SamplingParams(max_new_tokens=6, ignore_eos=True)) for _ in range(6)]
    outs = engine.generate(reqs)
    for req, out in zip(reqs, outs):
        assert list(out.output_token_ids) == expected(req.prompt_token_ids, req.sampling, 80)
    cache = engine.scheduler.block_manager.prefix_cache
    assert cache.hits >= 1 and cache.hit_tokens >= 7 * 4


def test_poisson_arrivals_with_injected_clock():
    now = [0]
    engine, ex = make_engine(clock=lambda: now[0])
    rng = np.random.default_rng(2)
    arrivals = np.cumsum(rng.exponential(5_000_000, size=5)).astype(int)
    for i, at in enumerate(arrivals):
        engine.submit([10 + i] * 7, SamplingParams(max_new_tokens=4, ignore_eos=True),
                      arrival_ns=int(at))
    finished = {}
    t = 0
    while engine.has_unfinished():
        t += 1_000_000
        now[0] = t
        for ev in engine.step(t).completion_events:
            finished[ev.request_id] = ev
            assert ev.admitted_ns >= arrivals[ev.request_id]
    assert len(finished) == 5


def test_cancel_and_eos():
    engine, ex = make_engine()
    a = engine.submit([7] * 12, SamplingParams(max_new_tokens=50, ignore_eos=True))
    b = engine.submit([8] * 5, SamplingParams(max_new_tokens=50))
    engine.step()
    engine.step()
    assert engine.cancel(a)
    events = []
    while engine.has_unfinished():
        events += engine.step().completion_events
    by_id = {e.request_id: e for e in events}
    assert by_id[a].status is RequestStatus.ABORTED
    exp_b = expected([8] * 5, SamplingParams(max_new_tokens=50), 96)
    assert list(by_id[b].output_token_ids) == exp_b
    assert set(ex.released) == {a, b}


def test_executor_failure_is_fail_stop():
    engine, ex = make_engine()
    ex.fail_at = 3
    engine.submit([9] * 30, SamplingParams(max_new_tokens=10))
    with pytest.raises(RuntimeError):
        for _ in range(10):
            engine.step()
    with pytest.raises(RuntimeError, match="failed"):
        engine.step()


def test_requests_that_cannot_fit_are_rejected():
    engine, _ = make_engine(blocks=8, max_len=96)
    with pytest.raises(ValueError, match="KV capacity"):
        engine.submit([6] * 40, SamplingParams(max_new_tokens=10))
    with pytest.raises(ValueError):
        engine.submit([6] * 97, SamplingParams(max_new_tokens=1))
