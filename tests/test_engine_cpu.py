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
from tinyvllm.scheduler import PENDING_TOKEN, Scheduler

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
        self.truth = {}       # request -> every token the simulated model saw or made
        self.last = []        # the previous step's sampled tokens ("on the device")

    def execute(self, batch):
        self.batches += 1
        if self.fail_at == self.batches:
            raise RuntimeError("injected executor failure")
        self.validator._prev_count = len(self.last)
        self.validator._validate(batch, self.cache)
        ids = list(batch.input_ids)
        if batch.input_token_sources is not None:  # resolved "on the device"
            ids = [self.last[s] if s >= 0 else t
                   for t, s in zip(ids, batch.input_token_sources)]
        out = []
        for i, rid in enumerate(batch.request_ids):
            start, end = batch.q_offsets[i], batch.q_offsets[i + 1]
            before, after = batch.context_lens_before[i], batch.context_lens_after[i]
            # Ground truth: the request's own tokens (prompt + sampled so far);
            # the scheduler's copy may still hold placeholders for tokens in flight.
            truth = self.truth.setdefault(
                rid, list(self.scheduler.get_request(rid).prompt_token_ids))
            hist = truth[:after]
            assert ids[start:end] == hist[before:after]
            known = self.scheduler.get_request(rid).token_slice(0, after)
            assert all(k == h for k, h in zip(known, hist) if k >= 0)
            for t, slot in zip(range(start, end), batch.kv_slot_mapping[start:end]):
                self.slots[slot] = ids[t]
            # Read back the whole context through the block table.
            toff = batch.kv_block_table_offsets
            table = batch.kv_block_table_ids[toff[i]:toff[i + 1]]
            for p in range(after):
                slot = table[p // self.bs] * self.bs + p % self.bs
                assert self.slots.get(slot) == hist[p], (rid, p)
            if end - 1 in batch.sample_token_indices:
                token = next_token(hist)
                if len(truth) == after:
                    truth.append(token)
                out.append(token)
        self.last = out
        return StepResult(batch.plan_id, batch.sample_request_ids, tuple(out))

    def release(self, request_id):
        self.released.append(request_id)

    def clear(self):
        pass


class _Launched:
    def __init__(self, result):
        self.sample_request_ids = result.sample_request_ids
        self._result = result

    def result(self):
        return self._result


class PipelinedSimExecutor(SimExecutor):
    """Adds launch(): the engine plans step k+1 before reading step k's
    tokens, whose ids reach the next batch only as input_token_sources."""

    def launch(self, batch):
        if batch.input_token_sources is not None:
            self.pipelined_batches += 1
        return _Launched(self.execute(batch))

    pipelined_batches = 0


def expected(prompt, params, max_model_len):
    seq, out = list(prompt), []
    while len(out) < params.max_new_tokens and len(seq) < max_model_len:
        tok = next_token(seq)
        out.append(tok)
        seq.append(tok)
        if tok == EOS and not params.ignore_eos:
            break
    return out


@pytest.fixture(params=[False, True], ids=["serial", "pipelined"])
def pipelined(request):
    return request.param


def make_engine(*, bs=4, blocks=96, max_len=96, seqs=4, tokens=24, chunk=10,
                prefix=True, clock=None, pipelined=False):
    cls = PipelinedSimExecutor if pipelined else SimExecutor
    ex = cls(block_size=bs, num_blocks=blocks, max_model_len=max_len, max_batch=seqs)
    sched = Scheduler(max_active_requests=seqs, max_step_requests=seqs,
                      max_scheduled_tokens=tokens, prefill_chunk_size=chunk,
                      max_model_len=max_len, prefill_reserve_tokens=4,
                      prefill_reserve_requests=1, kv_block_size=bs, kv_num_blocks=blocks,
                      eos_token_ids=[EOS], enable_prefix_caching=prefix)
    kwargs = {} if clock is None else {"clock": clock, "sleep": lambda s: None}
    ex.scheduler = sched
    return Engine(sched, ex, **kwargs), ex


@pytest.mark.parametrize("prefix", [True, False])
def test_many_requests_chunked_prefill_matches_model(prefix, pipelined):
    rng = random.Random(0)
    engine, ex = make_engine(prefix=prefix, pipelined=pipelined)
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


def test_shared_prefixes_hit_the_cache_and_stay_exact(pipelined):
    rng = random.Random(1)
    engine, ex = make_engine(blocks=80, max_len=80, chunk=8, tokens=20, pipelined=pipelined)
    shared = [rng.randrange(6, VOCAB) for _ in range(30)]
    reqs = [GenerateRequest(shared + [rng.randrange(6, VOCAB) for _ in range(rng.randrange(1, 6))],
                            SamplingParams(max_new_tokens=6, ignore_eos=True)) for _ in range(6)]
    outs = engine.generate(reqs)
    for req, out in zip(reqs, outs):
        assert list(out.output_token_ids) == expected(req.prompt_token_ids, req.sampling, 80)
    cache = engine.scheduler.block_manager.prefix_cache
    assert cache.hits >= 1 and cache.hit_tokens >= 7 * 4


def test_poisson_arrivals_with_injected_clock(pipelined):
    now = [0]
    engine, ex = make_engine(clock=lambda: now[0], pipelined=pipelined)
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


def test_cancel_and_eos(pipelined):
    engine, ex = make_engine(pipelined=pipelined)
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


def test_executor_failure_is_fail_stop(pipelined):
    engine, ex = make_engine(pipelined=pipelined)
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


def _eos_prompts(rng, count, max_new):
    """Prompts whose simulated continuation hits EOS before max_new tokens."""
    found = []
    while len(found) < count:
        prompt = [rng.randrange(6, VOCAB) for _ in range(rng.randrange(1, 30))]
        out = expected(prompt, SamplingParams(max_new_tokens=max_new), 96)
        if out[-1] == EOS and len(out) < max_new:
            found.append(prompt)
    return found


def test_pipelined_eos_drops_rows_launched_past_the_stop():
    """EOS is seen one step late: the request's next row is already launched.
    Its outputs must end at EOS, its extra row be discarded, and every block
    come back to the pool."""
    rng = random.Random(7)
    engine, ex = make_engine(pipelined=True, seqs=4, tokens=24)
    prompts = _eos_prompts(rng, 6, 40)
    reqs = [GenerateRequest(p, SamplingParams(max_new_tokens=40)) for p in prompts]
    reqs += [GenerateRequest([rng.randrange(6, VOCAB) for _ in range(9)],
                             SamplingParams(max_new_tokens=12, ignore_eos=True))
             for _ in range(3)]
    outs = engine.generate(reqs)
    for req, out in zip(reqs, outs):
        assert out.status is RequestStatus.FINISHED
        assert list(out.output_token_ids) == expected(req.prompt_token_ids, req.sampling, 96)
    assert ex.pipelined_batches > 0
    assert engine.scheduler.block_manager.free_block_count == 96
    assert not engine.scheduler.has_unresolved_steps
    # The engine is reusable and still exact afterwards.
    again = engine.generate(reqs[:2])
    assert [list(o.output_token_ids) for o in again] == [list(o.output_token_ids)
                                                          for o in outs[:2]]


def test_pipelined_cancel_drops_the_token_in_flight():
    engine, ex = make_engine(pipelined=True)
    a = engine.submit([7] * 12, SamplingParams(max_new_tokens=50, ignore_eos=True))
    seen = []
    for _ in range(6):
        seen += [e.token_id for e in engine.step().token_events]
    assert engine.cancel(a)
    events = []
    while engine.has_unfinished():
        events += engine.step().completion_events
    (done,) = events
    assert done.status is RequestStatus.ABORTED
    # Only tokens that reached the host count; all of them are the model's.
    assert list(done.output_token_ids) == seen
    assert seen == expected([7] * 12, SamplingParams(max_new_tokens=50, ignore_eos=True),
                            96)[:len(seen)]
    assert PENDING_TOKEN not in done.output_token_ids
    assert engine.scheduler.block_manager.free_block_count == 96


def test_pipelined_token_events_lag_one_step():
    engine, ex = make_engine(pipelined=True)
    engine.submit([9] * 3, SamplingParams(max_new_tokens=3, ignore_eos=True))
    first = engine.step()   # prefill launched, nothing resolved yet
    assert not first.token_events
    second = engine.step()  # decode launched; the prefill's token resolves
    assert len(second.token_events) == 1


def test_pipelined_eos_on_the_last_allowed_token_and_cancel_while_finishing():
    """Length stop known at launch (the request leaves the decode queue) and
    an EOS resolved for that same last token; a request cancelled while its
    last token is still in flight."""
    rng = random.Random(9)
    eos_first = next(p for p in ([rng.randrange(6, VOCAB) for _ in range(rng.randrange(1, 20))]
                                 for _ in range(10000))
                     if next_token(p) == EOS)
    engine, ex = make_engine(pipelined=True)
    a = engine.submit(eos_first, SamplingParams(max_new_tokens=1))  # EOS is also the last
    b = engine.submit([31] * 9, SamplingParams(max_new_tokens=2, ignore_eos=True))
    events = []
    while engine.has_unfinished():
        events += engine.step().completion_events
    by_id = {e.request_id: e for e in events}
    assert list(by_id[a].output_token_ids) == [EOS]
    assert list(by_id[b].output_token_ids) == expected([31] * 9, SamplingParams(
        max_new_tokens=2, ignore_eos=True), 96)
    # Cancel right after the step that launched the last token's row.
    c = engine.submit([32] * 5, SamplingParams(max_new_tokens=1, ignore_eos=True))
    engine.step()  # prefill launched; its (only, last) token is in flight
    assert engine.cancel(c)
    done = []
    while engine.has_unfinished():
        done += engine.step().completion_events
    (ev,) = done
    assert ev.status is RequestStatus.ABORTED and PENDING_TOKEN not in ev.output_token_ids
    assert engine.scheduler.block_manager.free_block_count == 96
    assert not engine.scheduler.has_unresolved_steps
