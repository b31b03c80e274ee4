"""Continuous-batching scheduler (the role of the reference's
tinyvllm/scheduler.py; the policy below is the reference's, so schedules
match, the code is this build's own).

Policy of one step:

* every decoding request contributes one row of one token, oldest first;
* prefill work (admitted prompts still being computed, then newly admitted
  ones, or the other way round on alternate steps when both exist) is cut
  into chunks of at most ``prefill_chunk_size`` tokens;
* the step holds at most ``max_step_requests`` rows and
  ``max_scheduled_tokens`` tokens; when decodes and prefills compete,
  ``prefill_reserve_requests`` rows and ``prefill_reserve_tokens`` tokens
  are held for prefill, spread so each held row gets at least one token;
* a waiting request is admitted when a request slot is free and the pool
  can hold its worst-case KV (prompt + max_new_tokens, less a cached prefix
  it attaches); admitted requests are never preempted. A request whose next
  chunk would compute a prefix block that another request is computing in
  this step waits one step and then attaches that block instead.

A step is a transaction: ``begin_step`` stages its KV (``StepKV``),
``mark_dispatched`` makes admissions and block tables visible right before
execution, ``commit_step`` applies sampled tokens, ``rollback`` undoes a
staged step, and any failure after dispatch is fail-stop (``shutdown``).

Pipelined engines split ``commit_step``: ``commit_launch`` commits the KV
side of a launched step and gives each sampled row a ``PENDING_TOKEN``
output, so the next step can be planned while the GPU runs this one;
``resolve`` fills those outputs in launch order and applies EOS. A request
that hit EOS may already have a row in the next launched step; that row is
discarded when it resolves. A length stop is known at launch: the request
leaves the decode queue at once and finishes when its last token resolves.
"""
from __future__ import annotations

import heapq
from collections import deque
from collections.abc import Iterable
from dataclasses import dataclass, field
from enum import Enum, auto

from tinyvllm._validation import (
    _check_non_negative_int, _check_positive_int, _check_token_id, _normalize_token_ids,
)
from tinyvllm.batch import StepPlan, StepResult, WorkItem
from tinyvllm.cache import BlockAppend, BlockManager, BlockRef, StepKV
from tinyvllm.request import (
    CompletionEvent, RequestState, RequestStatus, SamplingParams, WorkClass,
)


@dataclass(frozen=True, slots=True)
class AddCommand:
    seq: int
    request_id: int
    prompt_token_ids: tuple[int, ...]
    sampling: SamplingParams
    arrival_ns: int

    def __post_init__(self) -> None:
        _check_non_negative_int("seq", self.seq)
        _check_non_negative_int("request_id", self.request_id)
        _check_non_negative_int("arrival_ns", self.arrival_ns)
        if not isinstance(self.sampling, SamplingParams):
            raise TypeError("sampling must be SamplingParams")
        object.__setattr__(self, "prompt_token_ids", tuple(self.prompt_token_ids))


@dataclass(frozen=True, slots=True)
class CancelCommand:
    seq: int
    request_id: int

    def __post_init__(self) -> None:
        _check_non_negative_int("seq", self.seq)
        _check_non_negative_int("request_id", self.request_id)


EngineCommand = AddCommand | CancelCommand

# An output slot whose token id is still on the device (pipelined steps).
PENDING_TOKEN = -1


class ScheduleDecision(Enum):
    PLAN = auto()
    IDLE = auto()


class TxnState(Enum):
    PREPARED = auto()
    DISPATCHED = auto()
    COMMITTED = auto()
    ROLLED_BACK = auto()
    FAILED = auto()


@dataclass(slots=True)
class ScheduleTxn:
    """A planned step: the plan, its KV journal, and whether committing it
    flips which prefill group goes first next time."""

    plan: StepPlan
    kv: StepKV
    alternate: bool = False
    state: TxnState = field(default=TxnState.PREPARED)


@dataclass(slots=True)
class _Candidate:
    """Prefill work one request could do this step."""

    request: RequestState
    slot: int
    start: int                             # first token to compute
    hit: tuple[BlockRef, ...] = ()         # cached prefix it attaches


class Scheduler:
    def __init__(
        self,
        *,
        max_active_requests: int,
        max_step_requests: int,
        max_scheduled_tokens: int,
        prefill_chunk_size: int,
        max_model_len: int,
        prefill_reserve_tokens: int = 128,
        prefill_reserve_requests: int = 1,
        kv_block_size: int = 16,
        kv_num_blocks: int | None = None,
        eos_token_ids: Iterable[int] | None = None,
        enable_prefix_caching: bool = True,
    ) -> None:
        for name, value in (("max_active_requests", max_active_requests),
                            ("max_step_requests", max_step_requests),
                            ("max_scheduled_tokens", max_scheduled_tokens),
                            ("prefill_chunk_size", prefill_chunk_size),
                            ("max_model_len", max_model_len), ("kv_block_size", kv_block_size)):
            _check_positive_int(name, value)
        _check_non_negative_int("prefill_reserve_tokens", prefill_reserve_tokens)
        _check_non_negative_int("prefill_reserve_requests", prefill_reserve_requests)
        if prefill_reserve_tokens < prefill_reserve_requests:
            raise ValueError("each reserved prefill request needs one token")
        if (prefill_reserve_tokens == 0) != (prefill_reserve_requests == 0):
            raise ValueError("prefill reservations must both be zero or positive")
        if max_step_requests > max_active_requests:
            raise ValueError("max_step_requests exceeds active-request capacity")
        if prefill_chunk_size > max_scheduled_tokens:
            raise ValueError("prefill_chunk_size exceeds the step token budget")
        if kv_num_blocks is None:
            kv_num_blocks = max_active_requests * -(-max_model_len // kv_block_size)
        _check_positive_int("kv_num_blocks", kv_num_blocks)
        self.max_active_requests = max_active_requests
        self.max_step_requests = max_step_requests
        self.max_scheduled_tokens = max_scheduled_tokens
        self.prefill_chunk_size = prefill_chunk_size
        self.max_model_len = max_model_len
        self.prefill_reserve_tokens = prefill_reserve_tokens
        self.prefill_reserve_requests = prefill_reserve_requests
        self.kv_block_size = kv_block_size
        self._kv = BlockManager(block_size=kv_block_size, num_blocks=kv_num_blocks,
                                enable_prefix_caching=enable_prefix_caching)
        self._eos = _normalize_token_ids("eos_token_ids", eos_token_ids)
        self._init_state()

    def _init_state(self) -> None:
        self._by_id: dict[int, RequestState] = {}
        self._future: list[tuple[int, int, int]] = []     # (arrival, seq, id) min-heap
        self._dead_future = 0                              # cancelled heap entries
        self._arrived: deque[int] = deque()                # waiting for admission
        self._prefilling: deque[int] = deque()             # admitted, prompt not done
        self._decoding: deque[int] = deque()
        self._slot_owner: list[int | None] = [None] * self.max_active_requests
        self._results: deque[CompletionEvent] = deque()
        self._waiting_first = False
        self._clock: int | None = None
        self._fresh_commands = False
        self._plan_seq = 0
        self._open: ScheduleTxn | None = None
        self._decision = ScheduleDecision.IDLE
        self._seq_seen = getattr(self, "_seq_seen", -1)
        self._dead = getattr(self, "_dead", False)
        # Pipelined steps: launched plans awaiting tokens (plan id, sampled
        # request ids), each request's unfilled outputs (plan id, index), and
        # length-stopped requests waiting for their last token.
        self._in_flight: deque[tuple[int, tuple[int, ...]]] = deque()
        self._unfilled: dict[int, deque[tuple[int, int]]] = {}
        self._last_token_due: set[int] = set()

    # ------------------------------------------------------------- views --

    @property
    def eos_token_ids(self) -> frozenset[int]:
        return self._eos

    @property
    def block_manager(self) -> BlockManager:
        return self._kv

    @property
    def has_open_transaction(self) -> bool:
        return self._open is not None

    @property
    def has_unresolved_steps(self) -> bool:
        """Launched steps whose sampled tokens have not been resolved yet."""
        return bool(self._in_flight)

    @property
    def last_decision(self) -> ScheduleDecision:
        return self._decision

    @property
    def request_ids(self) -> tuple[int, ...]:
        """Includes terminal requests whose results are not consumed yet."""
        return tuple(self._by_id)

    @property
    def waiting_request_ids(self) -> tuple[int, ...]:
        return tuple(self._arrived)

    @property
    def last_command_seq(self) -> int:
        return self._seq_seen

    @property
    def completed_request_ids(self) -> tuple[int, ...]:
        return tuple(e.request_id for e in self._results)

    @property
    def next_arrival_ns(self) -> int | None:
        while self._future and not self._is_current(self._future[0]):
            heapq.heappop(self._future)
            self._dead_future -= 1
        return self._future[0][0] if self._future else None

    def pending_sample_rows(self) -> dict[int, int]:
        """Request -> row of its token among the newest launched step's
        samples, for requests whose latest output is still on the device."""
        if not self._in_flight:
            return {}
        plan_id, rids = self._in_flight[-1]
        rows = {}
        for row, rid in enumerate(rids):
            slots = self._unfilled.get(rid)
            if slots and slots[-1][0] == plan_id:
                rows[rid] = row
        return rows

    def get_request(self, request_id: int) -> RequestState:
        return self._by_id[request_id]

    def worst_case_blocks(self, prompt_len: int, sampling: SamplingParams) -> int:
        """Blocks a request may fill: its prompt plus every output but the
        last (the last sampled token is never written back)."""
        outputs = min(sampling.max_new_tokens, self.max_model_len - prompt_len)
        return 0 if outputs == 0 else self._kv.blocks_for(prompt_len + outputs - 1)

    def validate_request(self, prompt_token_ids, sampling: SamplingParams) -> None:
        """Reject requests that could never finish within the KV pool."""
        if not isinstance(sampling, SamplingParams):
            raise TypeError("sampling must be SamplingParams")
        if not prompt_token_ids:
            raise ValueError("prompt_token_ids must be non-empty")
        for token_id in prompt_token_ids:
            _check_token_id(token_id)
        if len(prompt_token_ids) > self.max_model_len:
            raise ValueError("prompt exceeds max_model_len")
        need = self.worst_case_blocks(len(prompt_token_ids), sampling)
        if need > self._kv.pool.num_blocks:
            raise ValueError(f"request exceeds KV capacity: needs {need} blocks, "
                             f"pool has {self._kv.pool.num_blocks}")

    def consume_finished(self) -> tuple[CompletionEvent, ...]:
        out = tuple(self._results)
        self._results.clear()
        for event in out:
            del self._by_id[event.request_id]
        return out

    # ---------------------------------------------------------- commands --

    def apply_commands(self, commands: tuple[EngineCommand, ...], now_ns: int) -> None:
        """Check a whole command batch, then apply it at once."""
        self._alive()
        if self._open is not None:
            raise RuntimeError("commands cannot be applied while a step is open")
        self._advance(now_ns)
        commands = tuple(commands)
        new: dict[int, RequestState] = {}
        cancels = []
        for offset, command in enumerate(commands):
            if not isinstance(command, (AddCommand, CancelCommand)):
                raise TypeError("commands must be AddCommand or CancelCommand values")
            if command.seq != self._seq_seen + 1 + offset:
                raise ValueError(f"command seq {command.seq} out of order "
                                 f"(expected {self._seq_seen + 1 + offset})")
            rid = command.request_id
            if isinstance(command, AddCommand):
                if rid in self._by_id or rid in new:
                    raise ValueError(f"duplicate request_id: {rid}")
                self.validate_request(command.prompt_token_ids, command.sampling)
                new[rid] = RequestState(
                    request_id=rid, submit_seq=command.seq,
                    prompt_token_ids=list(command.prompt_token_ids),
                    sampling=command.sampling, arrival_ns=command.arrival_ns)
            elif rid not in self._by_id and rid not in new:
                raise KeyError(f"unknown request_id: {rid}")
            else:
                cancels.append(rid)
        for rid, request in new.items():
            self._by_id[rid] = request
            heapq.heappush(self._future, (request.arrival_ns, request.submit_seq, rid))
        for rid in cancels:
            self._cancel(self._by_id[rid], now_ns)
        if commands:
            self._seq_seen = commands[-1].seq
        self._release_arrivals(now_ns)
        self._fresh_commands = True

    # ---------------------------------------------------------- planning --

    def begin_step(self, now_ns: int) -> ScheduleTxn | None:
        self._alive()
        if self._open is not None:
            raise RuntimeError("a step is already open")
        if not self._fresh_commands or now_ns != self._clock:
            raise ValueError("apply_commands must run first with the same now_ns")
        self._decision = ScheduleDecision.IDLE
        decodes = [self._by_id[rid] for rid in self._decoding]
        running = [_Candidate(r, r.active_slot, r.computed_tokens)
                   for r in map(self._by_id.__getitem__, self._prefilling)]
        admitted = self._admit_candidates()
        candidates = admitted + running if self._waiting_first else running + admitted
        n_decode, chunks = self._split_budget(len(decodes), candidates)
        rows = [self._work(r, r.active_slot, WorkClass.DECODE, r.computed_tokens, 1)
                for r in decodes[:n_decode]]
        rows += [self._work(c.request, c.slot, WorkClass.PREFILL, c.start, n)
                 for c, n in chunks]
        if not rows:
            return None
        plan = StepPlan(plan_id=self._plan_seq, items=tuple(rows))
        hits = {c.request.request_id: c.hit for c, _ in chunks if c.hit}
        kv = self._kv.stage(plan.plan_id, [
            BlockAppend(w.request_id, w.token_start, w.query_len, hits.get(w.request_id, ()))
            for w in plan.items])
        if kv is None:
            raise RuntimeError("admitted requests exceeded their KV budget")
        self._open = ScheduleTxn(plan=plan, kv=kv, alternate=bool(running and admitted))
        self._plan_seq += 1
        self._decision = ScheduleDecision.PLAN
        return self._open

    def _split_budget(self, decodes: int, candidates: list[_Candidate]
                      ) -> tuple[int, list[tuple[_Candidate, int]]]:
        """Decode rows taken and prefill chunks (candidate, tokens) of one step."""
        rows, tokens = self.max_step_requests, self.max_scheduled_tokens
        hold_rows = hold_tokens = 0
        if decodes and candidates:  # prefill keeps a share when both compete
            hold_tokens = min(self.prefill_reserve_tokens, tokens - 1)
            hold_rows = min(self.prefill_reserve_requests, rows - 1, len(candidates),
                            hold_tokens)
            hold_tokens = hold_tokens if hold_rows else 0
        taken = min(decodes, rows - hold_rows, tokens - hold_tokens)
        rows, tokens = rows - taken, tokens - taken
        if taken < decodes:
            # Decode-bound: prefill gets the held share only, the rest of the
            # budget goes back to decode rows.
            chunks = self._cut(candidates, hold_rows, hold_tokens, hold_rows)
            used = sum(n for _, n in chunks)
            more = min(decodes - taken, rows - len(chunks), tokens - used)
            return taken + more, chunks
        return taken, self._cut(candidates, rows, tokens, hold_rows)

    def _cut(self, candidates: list[_Candidate], rows: int, tokens: int,
             guaranteed: int) -> list[tuple[_Candidate, int]]:
        """Chunks for candidates in order; each of the first ``guaranteed``
        leaves one token for every guaranteed candidate after it."""
        out: list[tuple[_Candidate, int]] = []
        guaranteed = min(guaranteed, len(candidates), rows, tokens)
        for k, cand in enumerate(candidates[:rows]):
            keep = max(0, guaranteed - k - 1)
            n = min(cand.request.total_tokens - cand.start, self.prefill_chunk_size,
                    tokens - keep)
            if n <= 0:
                break
            out.append((cand, n))
            tokens -= n
        return out

    def _admit_candidates(self) -> list[_Candidate]:
        """Waiting requests, oldest first, that get a free slot and whose
        worst-case KV fits what the admitted requests leave."""
        if not self._arrived:
            return []
        kv, prefix = self._kv, self._kv.prefix_cache
        spare = kv.free_block_count
        computing: set[bytes] = set()   # prefix digests some chunk produces now
        for rid in self._slot_owner:
            if rid is None:
                continue
            req = self._by_id[rid]
            spare -= (self.worst_case_blocks(len(req.prompt_token_ids), req.sampling)
                      - kv.table_length(rid))
            if req.work_class is WorkClass.PREFILL:
                digest = prefix.chunk_digest(rid, req.prompt_token_ids, req.computed_tokens,
                                             self.prefill_chunk_size)
                if digest is not None:
                    computing.add(digest)
        free_slots = [s for s, owner in enumerate(self._slot_owner) if owner is None]
        chosen: list[_Candidate] = []
        repinned: set[BlockRef] = set()
        for rid in self._arrived:
            if len(chosen) == len(free_slots):
                break
            req = self._by_id[rid]
            hit = prefix.lookup(rid, req.prompt_token_ids)
            start = len(hit) * self.kv_block_size
            digest = prefix.chunk_digest(rid, req.prompt_token_ids, start,
                                         self.prefill_chunk_size)
            if digest in computing:
                continue  # reuse that block next step instead of computing it twice
            # Idle cached blocks it attaches leave the free pool.
            revived = {r for r in hit if r not in repinned and kv.pool.is_idle(r)}
            cost = (self.worst_case_blocks(len(req.prompt_token_ids), req.sampling)
                    - len(hit) + len(revived))
            if cost > spare:
                continue
            spare -= cost
            repinned |= revived
            if digest is not None:
                computing.add(digest)
            chosen.append(_Candidate(req, free_slots[len(chosen)], start, hit))
        return chosen

    def _work(self, request: RequestState, slot: int, kind: WorkClass, start: int,
              count: int) -> WorkItem:
        end = start + count
        sample = kind is WorkClass.DECODE or (end == request.total_tokens
                                              and end < self.max_model_len)
        return WorkItem(request_id=request.request_id, request_slot=slot, work_class=kind,
                        token_start=start, query_len=count, context_len_before=start,
                        should_sample=sample)

    # ------------------------------------------------------- transitions --

    def mark_dispatched(self, txn: ScheduleTxn, now_ns: int) -> None:
        """Make the step's admissions and block tables visible (right before
        execution)."""
        self._expect(txn, TxnState.PREPARED)
        self._advance(now_ns)
        txn.kv.go_live()
        txn.state = TxnState.DISPATCHED
        try:
            for item in txn.plan.items:
                req = self._by_id[item.request_id]
                if item.work_class is WorkClass.DECODE:
                    self._decoding.remove(req.request_id)
                elif req.status is RequestStatus.WAITING:
                    self._arrived.remove(req.request_id)
                    req.status = RequestStatus.RUNNING
                    req.active_slot = item.request_slot
                    self._slot_owner[item.request_slot] = req.request_id
                    if req.admitted_ns is None:
                        req.admitted_ns = now_ns
                else:
                    self._prefilling.remove(req.request_id)
            self._fresh_commands = False
        except Exception:
            self.fail_step(txn)
            raise

    def rollback(self, txn: ScheduleTxn) -> None:
        self._expect(txn, TxnState.PREPARED)
        txn.kv.undo()
        txn.state = TxnState.ROLLED_BACK
        self._open = None

    def commit_step(self, txn: ScheduleTxn, result: StepResult,
                    now_ns: int) -> tuple[tuple[int, int], ...]:
        """Apply a step's sampled tokens (serial engines); finish requests on
        EOS or length. Returns the (request id, token id) pairs applied."""
        self._expect(txn, TxnState.DISPATCHED)
        try:
            if result.plan_id != txn.plan.plan_id:
                raise RuntimeError("result plan_id does not match plan")
            sampled = tuple(i.request_id for i in txn.plan.items if i.should_sample)
            self._check_samples(result, sampled)
        except Exception:
            self.fail_step(txn)
            raise
        self.commit_launch(txn, now_ns)
        return self.resolve(result, now_ns)

    def commit_launch(self, txn: ScheduleTxn, now_ns: int) -> None:
        """Commit a launched step's KV writes before its tokens are known;
        each sampled row gets a PENDING_TOKEN output that ``resolve`` fills."""
        self._expect(txn, TxnState.DISPATCHED)
        try:
            self._advance(now_ns)
            txn.kv.writes_done()
            sampled = []
            for item in txn.plan.items:
                req = self._by_id[item.request_id]
                req.computed_tokens = item.token_end
                self._index_known_blocks(req)
                if not item.should_sample:
                    self._prefilling.append(req.request_id)
                    continue
                sampled.append(req.request_id)
                req.output_token_ids.append(PENDING_TOKEN)
                self._unfilled.setdefault(req.request_id, deque()).append(
                    (txn.plan.plan_id, len(req.output_token_ids) - 1))
                req.work_class = WorkClass.DECODE
                if req.remaining_new_tokens == 0 or req.total_tokens >= self.max_model_len:
                    self._last_token_due.add(req.request_id)
                else:
                    self._decoding.append(req.request_id)
            self._in_flight.append((txn.plan.plan_id, tuple(sampled)))
            if txn.alternate and txn.plan.num_prefill_items:
                self._waiting_first = not self._waiting_first
        except Exception:
            self.fail_step(txn)
            raise
        txn.state = TxnState.COMMITTED
        self._open = None

    def resolve(self, result: StepResult, now_ns: int) -> tuple[tuple[int, int], ...]:
        """Fill the oldest launched step's outputs with its sampled tokens and
        apply EOS and length stops. Returns the accepted (request id, token
        id) pairs; rows of requests that ended meanwhile are dropped."""
        self._alive()
        try:
            self._advance(now_ns)
            if not self._in_flight:
                raise RuntimeError("no launched step awaits tokens")
            plan_id, sampled = self._in_flight[0]
            if result.plan_id != plan_id:
                raise RuntimeError(f"tokens of plan {result.plan_id} arrived, "
                                   f"plan {plan_id} was launched first")
            self._check_samples(result, sampled)
            self._in_flight.popleft()
            accepted = []
            for rid, token in zip(sampled, result.sampled_token_ids):
                req = self._by_id.get(rid)
                slots = self._unfilled.get(rid)
                if req is None or req.terminal or not slots or slots[0][0] != plan_id:
                    continue
                _, index = slots.popleft()
                if not slots:
                    del self._unfilled[rid]
                req.output_token_ids[index] = token
                accepted.append((rid, token))
                if req.first_token_ns is None:
                    req.first_token_ns = now_ns
                if token in self._eos and not req.sampling.ignore_eos:
                    self._truncate_after(req, index)
                    self._finish(req, RequestStatus.FINISHED, now_ns)
                elif rid in self._last_token_due and rid not in self._unfilled:
                    self._last_token_due.discard(rid)
                    self._finish(req, RequestStatus.FINISHED, now_ns)
                else:
                    self._index_known_blocks(req)
        except Exception:
            self.shutdown()
            raise
        return tuple(accepted)

    def fail_step(self, txn: ScheduleTxn) -> None:
        self._expect(txn, TxnState.DISPATCHED)
        self.shutdown()

    def shutdown(self) -> None:
        """Stop scheduling for good and drop all KV ownership."""
        txn = self._open
        self._kv.teardown()
        if txn is not None:
            txn.state = TxnState.FAILED
        for req in self._by_id.values():
            req.active_slot = None
        self._dead = True
        self._init_state()

    # ----------------------------------------------------------- helpers --

    def _check_samples(self, result: StepResult, sampled: tuple[int, ...]) -> None:
        if tuple(result.sample_request_ids) != sampled:
            raise RuntimeError("sampled rows do not match the plan's sampling order")
        for token in result.sampled_token_ids:
            _check_token_id(token)

    def _index_known_blocks(self, req: RequestState) -> None:
        """Publish the request's full blocks whose token ids are on the host."""
        unknown = len(self._unfilled.get(req.request_id, ()))
        self._kv.publish_blocks(req.request_id, req.token_slice, req.total_tokens - unknown)

    def _truncate_after(self, req: RequestState, last: int) -> None:
        """Drop outputs past index ``last`` (rows launched after a stop) and
        take the request out of the decode / last-token queues."""
        rid = req.request_id
        del req.output_token_ids[last + 1:]
        self._unfilled.pop(rid, None)
        if rid in self._last_token_due:
            self._last_token_due.discard(rid)
        elif rid in self._decoding:
            self._decoding.remove(rid)

    def _cancel(self, req: RequestState, now_ns: int) -> None:
        if req.terminal:
            return
        rid = req.request_id
        if req.status is RequestStatus.PENDING:
            self._dead_future += 1   # its heap entry is skipped later
        elif req.status is RequestStatus.WAITING:
            self._arrived.remove(rid)
        elif req.work_class is WorkClass.DECODE:
            slots = self._unfilled.get(rid)
            keep = slots[0][1] - 1 if slots else len(req.output_token_ids) - 1
            self._truncate_after(req, keep)  # tokens still on the device never count
        else:
            self._prefilling.remove(rid)
        self._finish(req, RequestStatus.ABORTED, now_ns)

    def _finish(self, req: RequestState, status: RequestStatus, now_ns: int) -> None:
        req.status = status
        req.finished_ns = now_ns
        if req.active_slot is not None:
            self._slot_owner[req.active_slot] = None
            req.active_slot = None
        self._kv.release_request(req.request_id)
        self._results.append(CompletionEvent.from_request(req))

    def _is_current(self, entry: tuple[int, int, int]) -> bool:
        req = self._by_id.get(entry[2])
        return (req is not None and req.status is RequestStatus.PENDING
                and req.submit_seq == entry[1])

    def _release_arrivals(self, now_ns: int) -> None:
        """Requests whose arrival time has come join the waiting queue (or
        finish at once when there is nothing to generate)."""
        while self._future and self._future[0][0] <= now_ns:
            entry = heapq.heappop(self._future)
            if not self._is_current(entry):
                self._dead_future -= 1
                continue
            req = self._by_id[entry[2]]
            if req.sampling.max_new_tokens == 0 or len(req.prompt_token_ids) == self.max_model_len:
                req.admitted_ns = now_ns
                self._finish(req, RequestStatus.FINISHED, now_ns)
            else:
                req.status = RequestStatus.WAITING
                self._arrived.append(req.request_id)
        if self._dead_future > 64 and 2 * self._dead_future > len(self._future):
            self._future = [e for e in self._future if self._is_current(e)]
            heapq.heapify(self._future)
            self._dead_future = 0

    def _alive(self) -> None:
        if self._dead:
            raise RuntimeError("scheduler is failed")

    def _expect(self, txn: ScheduleTxn, state: TxnState) -> None:
        if txn is not self._open:
            raise ValueError("not the scheduler's open step")
        if txn.state is not state:
            raise RuntimeError(f"step is {txn.state.name.lower()}, "
                               f"expected {state.name.lower()}")

    def _advance(self, now_ns: int) -> None:
        _check_non_negative_int("now_ns", now_ns)
        if self._clock is not None and now_ns < self._clock:
            raise ValueError("now_ns cannot move backwards")
        self._clock = now_ns
