"""Continuous-batching scheduler (reference: tinyvllm/scheduler.py:33-1076).

Per step it plans decode rows first (one token each), then prefill chunks
(at most ``prefill_chunk_size`` tokens per request), inside a row budget
(``max_step_requests``) and a token budget (``max_scheduled_tokens``). When
both kinds wait, ``prefill_reserve_requests`` rows and
``prefill_reserve_tokens`` tokens are held back for prefill so a full decode
batch cannot starve admissions. A request is admitted only when a request
slot is free and the pool can hold its whole worst-case KV (prompt +
max_new_tokens), so admitted requests are never preempted. Prompts reuse
cached full blocks through the prefix cache; two requests that would compute
the same prefix block in one step are serialised so the second reuses it.

Every step is a transaction: ``begin_step`` stages blocks, ``mark_dispatched``
publishes ownership right before execution, ``commit_step`` applies the
sampled tokens (EOS / length stop) or ``rollback`` / ``fail_step`` undo it.

Pipelined engines split ``commit_step`` in two (beyond the reference, whose
engine waits for every step's tokens before planning the next):
``commit_launch`` commits the step's KV writes and appends a ``PENDING_TOKEN``
placeholder for each sampled token, so the next step can be planned while the
GPU still runs this one; ``resolve`` later fills the placeholders in launch
order and applies EOS. A request that hit EOS may already sit in the next,
launched step: its extra row is discarded when that step resolves. Length
stops are known at launch; such a request leaves the decode queue at once and
finishes when its last token resolves.
"""
from __future__ import annotations

from collections import deque
from collections.abc import Iterable
from dataclasses import dataclass, field
from enum import Enum, auto
from heapq import heapify, heappop, heappush

from tinyvllm._validation import (
    _check_non_negative_int, _check_positive_int, _check_token_id, _normalize_token_ids,
)
from tinyvllm.batch import StepPlan, StepResult, WorkItem
from tinyvllm.cache import BlockAppend, BlockManager, BlockPlanTxn, BlockRef, BlockState
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


class TxnState(Enum):
    PREPARED = auto()
    DISPATCHED = auto()
    COMMITTED = auto()
    ROLLED_BACK = auto()
    FAILED = auto()


class ScheduleDecision(Enum):
    PLAN = auto()
    IDLE = auto()


@dataclass(frozen=True, slots=True)
class ScheduleTxn:
    plan: StepPlan
    kv: BlockPlanTxn
    rotate_prefill: bool = False
    state: TxnState = field(default=TxnState.PREPARED, init=False)


@dataclass(slots=True)
class _Prefill:
    """A prefill candidate: request, its slot, first token to compute, prefix hit."""

    request: RequestState
    slot: int
    start: int
    prefix: tuple[BlockRef, ...] = ()


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
        self._blocks = BlockManager(block_size=kv_block_size, num_blocks=kv_num_blocks,
                                    enable_prefix_caching=enable_prefix_caching)
        self._eos = _normalize_token_ids("eos_token_ids", eos_token_ids)
        self._requests: dict[int, RequestState] = {}
        self._arrivals: list[tuple[int, int, int]] = []   # (arrival, seq, id) heap
        self._stale_arrivals = 0
        self._waiting: deque[int] = deque()
        self._prefilling: deque[int] = deque()
        self._decoding: deque[int] = deque()
        self._prefer_waiting = False
        self._slots: list[int | None] = [None] * max_active_requests
        self._finished: deque[CompletionEvent] = deque()
        self._last_seq = -1
        self._now: int | None = None
        self._commands_applied = False
        self._next_plan = 0
        self._txn: ScheduleTxn | None = None
        self._decision = ScheduleDecision.IDLE
        self._failed = False
        # Pipelined steps: launched plans awaiting their tokens (plan id,
        # sampled request ids), each request's unresolved output slots
        # (plan id, output index), and length-stopped requests whose last
        # token is unresolved.
        self._launched: deque[tuple[int, tuple[int, ...]]] = deque()
        self._unresolved: dict[int, deque[tuple[int, int]]] = {}
        self._finishing: set[int] = set()

    # ------------------------------------------------------------ queries --

    @property
    def eos_token_ids(self) -> frozenset[int]:
        return self._eos

    @property
    def has_open_transaction(self) -> bool:
        return self._txn is not None

    @property
    def has_unresolved_steps(self) -> bool:
        """Launched steps whose sampled tokens have not been resolved yet."""
        return bool(self._launched)

    def pending_sample_rows(self) -> dict[int, int]:
        """Request -> row of its token among the last launched step's samples,
        for requests whose newest output is still unresolved."""
        if not self._launched:
            return {}
        plan_id, rids = self._launched[-1]
        return {rid: row for row, rid in enumerate(rids)
                if self._unresolved.get(rid) and self._unresolved[rid][-1][0] == plan_id}

    @property
    def last_decision(self) -> ScheduleDecision:
        return self._decision

    @property
    def request_ids(self) -> tuple[int, ...]:
        """Includes terminal requests whose results are not consumed yet."""
        return tuple(self._requests)

    @property
    def waiting_request_ids(self) -> tuple[int, ...]:
        return tuple(self._waiting)

    @property
    def last_command_seq(self) -> int:
        return self._last_seq

    @property
    def block_manager(self) -> BlockManager:
        return self._blocks

    @property
    def completed_request_ids(self) -> tuple[int, ...]:
        return tuple(e.request_id for e in self._finished)

    @property
    def next_arrival_ns(self) -> int | None:
        while self._arrivals:
            if self._live(self._arrivals[0]):
                return self._arrivals[0][0]
            heappop(self._arrivals)
            self._stale_arrivals -= 1
        return None

    def get_request(self, request_id: int) -> RequestState:
        return self._requests[request_id]

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
        demand = self._demand(len(prompt_token_ids), sampling)
        if demand > self._blocks.pool.num_blocks:
            raise ValueError(f"request exceeds KV capacity: needs {demand} blocks, "
                             f"pool has {self._blocks.pool.num_blocks}")

    def consume_finished(self) -> tuple[CompletionEvent, ...]:
        events = tuple(self._finished)
        for event in events:
            del self._requests[event.request_id]
        self._finished.clear()
        return events

    # ----------------------------------------------------------- commands --

    def apply_commands(self, commands: tuple[EngineCommand, ...], now_ns: int) -> None:
        """Validate a whole command batch, then publish it atomically."""
        self._healthy()
        if self._txn is not None:
            raise RuntimeError("cannot apply commands during an open transaction")
        self._check_now(now_ns)
        commands = tuple(commands)
        expected = self._last_seq + 1
        staged: list[RequestState] = []
        staged_ids: set[int] = set()
        cancels: list[CancelCommand] = []
        for command in commands:
            if not isinstance(command, (AddCommand, CancelCommand)):
                raise TypeError("commands must contain AddCommand or CancelCommand")
            if command.seq != expected:
                raise ValueError(f"expected command seq {expected}, got {command.seq}")
            expected += 1
            if isinstance(command, AddCommand):
                if command.request_id in self._requests or command.request_id in staged_ids:
                    raise ValueError(f"duplicate request_id: {command.request_id}")
                self.validate_request(command.prompt_token_ids, command.sampling)
                staged.append(RequestState(
                    request_id=command.request_id, submit_seq=command.seq,
                    prompt_token_ids=list(command.prompt_token_ids),
                    sampling=command.sampling, arrival_ns=command.arrival_ns))
                staged_ids.add(command.request_id)
            else:
                if command.request_id not in self._requests \
                        and command.request_id not in staged_ids:
                    raise KeyError(f"unknown request_id: {command.request_id}")
                cancels.append(command)
        for request in staged:
            self._requests[request.request_id] = request
            heappush(self._arrivals, (request.arrival_ns, request.submit_seq,
                                      request.request_id))
        for command in cancels:
            self._abort(self._requests[command.request_id], now_ns)
        if commands:
            self._last_seq = commands[-1].seq
        self._now = now_ns
        self._promote(now_ns)
        self._compact()
        self._commands_applied = True

    # ------------------------------------------------------------ planning --

    def begin_step(self, now_ns: int) -> ScheduleTxn | None:
        self._healthy()
        if self._txn is not None:
            raise RuntimeError("a scheduling transaction is already open")
        if not self._commands_applied or self._now is None or now_ns != self._now:
            raise ValueError("apply_commands must run first with the same now_ns")
        self._decision = ScheduleDecision.IDLE

        decodes = [self._requests[i] for i in self._decoding]
        active = [_Prefill(r, r.active_slot, r.computed_tokens)
                  for r in (self._requests[i] for i in self._prefilling)]
        waiting = self._admissions()
        prefills = waiting + active if self._prefer_waiting else active + waiting

        reserve_rows = reserve_tokens = 0
        if decodes and prefills:
            reserve_tokens = min(self.prefill_reserve_tokens, self.max_scheduled_tokens - 1)
            reserve_rows = min(self.prefill_reserve_requests, self.max_step_requests - 1,
                               len(prefills), reserve_tokens)
            if reserve_rows == 0:
                reserve_tokens = 0

        rows, tokens = self.max_step_requests, self.max_scheduled_tokens
        n_decode = min(len(decodes), rows - reserve_rows, tokens - reserve_tokens)
        rows -= n_decode
        tokens -= n_decode
        # The reservation goes to prefill; everything if all decodes fit.
        budget = tokens if n_decode == len(decodes) else reserve_tokens
        items, used_candidates, used = self._chunks(prefills, 0, reserve_rows, budget, True)
        rows -= len(items)
        tokens -= used
        extra = min(len(decodes) - n_decode, rows, tokens)
        n_decode += extra
        rows -= extra
        tokens -= extra
        if n_decode == len(decodes):
            more, _, _ = self._chunks(prefills, used_candidates, rows, tokens, False)
            items.extend(more)

        decode_items = [self._item(r, r.active_slot, WorkClass.DECODE, r.computed_tokens, 1)
                        for r in decodes[:n_decode]]
        all_items = decode_items + items
        if not all_items:
            return None
        plan = StepPlan(plan_id=self._next_plan, items=tuple(all_items))
        hits = {p.request.request_id: p.prefix for p in prefills if p.prefix}
        kv = self._blocks.begin_plan(plan_id=plan.plan_id, appends=tuple(
            BlockAppend(i.request_id, i.token_start, i.query_len, hits.get(i.request_id, ()))
            for i in plan.items))
        if kv is None:
            raise RuntimeError("admitted requests exceeded their KV budget")
        self._txn = ScheduleTxn(plan=plan, kv=kv, rotate_prefill=bool(active and waiting))
        self._next_plan += 1
        self._decision = ScheduleDecision.PLAN
        return self._txn

    def mark_dispatched(self, txn: ScheduleTxn, now_ns: int) -> None:
        """Publish block ownership and admissions right before execution."""
        self._require(txn, TxnState.PREPARED)
        self._check_now(now_ns)
        txn.kv.commit_before_dispatch()
        object.__setattr__(txn, "state", TxnState.DISPATCHED)
        try:
            for item in txn.plan.items:
                request = self._requests[item.request_id]
                if item.work_class is WorkClass.DECODE:
                    self._decoding.remove(request.request_id)
                elif request.status is RequestStatus.WAITING:
                    self._waiting.remove(request.request_id)
                    request.status = RequestStatus.RUNNING
                    request.active_slot = item.request_slot
                    self._slots[item.request_slot] = request.request_id
                    if request.admitted_ns is None:
                        request.admitted_ns = now_ns
                else:
                    self._prefilling.remove(request.request_id)
            self._now = now_ns
            self._commands_applied = False
        except Exception:
            self.fail_step(txn)
            raise

    def rollback(self, txn: ScheduleTxn) -> None:
        self._require(txn, TxnState.PREPARED)
        txn.kv.rollback()
        object.__setattr__(txn, "state", TxnState.ROLLED_BACK)
        self._txn = None

    def commit_step(self, txn: ScheduleTxn, result: StepResult,
                    now_ns: int) -> tuple[tuple[int, int], ...]:
        """Apply a step's sampled tokens; finish requests on EOS or length.
        Returns the (request id, token id) pairs applied."""
        self._require(txn, TxnState.DISPATCHED)
        try:
            self._check_result(txn.plan, result)
        except Exception:
            self.fail_step(txn)
            raise
        self.commit_launch(txn, now_ns)
        return self.resolve(result, now_ns)

    def _check_result(self, plan: StepPlan, result: StepResult) -> None:
        if result.plan_id != plan.plan_id:
            raise RuntimeError("result plan_id does not match plan")
        sampled = [i.request_id for i in plan.items if i.should_sample]
        if tuple(sampled) != tuple(result.sample_request_ids):
            raise RuntimeError("result sampling order does not match plan")
        for token_id in result.sampled_token_ids:
            _check_token_id(token_id)

    def commit_launch(self, txn: ScheduleTxn, now_ns: int) -> None:
        """Commit a launched step's KV writes before its tokens are known:
        each sampled row gets a PENDING_TOKEN output that ``resolve`` fills."""
        self._require(txn, TxnState.DISPATCHED)
        try:
            self._check_now(now_ns)
            plan = txn.plan
            txn.kv.complete_writes()
            sampled = []
            for item in plan.items:
                request = self._requests[item.request_id]
                request.computed_tokens = item.token_end
                self._publish_known(request)
                if not item.should_sample:
                    self._prefilling.append(request.request_id)
                    continue
                sampled.append(request.request_id)
                request.output_token_ids.append(PENDING_TOKEN)
                self._unresolved.setdefault(request.request_id, deque()).append(
                    (plan.plan_id, len(request.output_token_ids) - 1))
                request.work_class = WorkClass.DECODE
                if (request.remaining_new_tokens == 0
                        or request.total_tokens >= self.max_model_len):
                    self._finishing.add(request.request_id)
                else:
                    self._decoding.append(request.request_id)
            self._launched.append((plan.plan_id, tuple(sampled)))
            if txn.rotate_prefill and plan.num_prefill_items:
                self._prefer_waiting = not self._prefer_waiting
        except Exception:
            self.fail_step(txn)
            raise
        self._now = now_ns
        object.__setattr__(txn, "state", TxnState.COMMITTED)
        self._txn = None

    def resolve(self, result: StepResult, now_ns: int) -> tuple[tuple[int, int], ...]:
        """Fill the oldest launched step's placeholders with its sampled
        tokens; apply EOS and pending length stops. Returns the accepted
        (request id, token id) pairs - rows of requests that finished or
        were cancelled meanwhile are dropped."""
        self._healthy()
        try:
            self._check_now(now_ns)
            if not self._launched:
                raise RuntimeError("no launched step awaits tokens")
            plan_id, sampled = self._launched[0]
            if result.plan_id != plan_id:
                raise RuntimeError("result plan_id does not match the oldest launched plan")
            if tuple(result.sample_request_ids) != sampled:
                raise RuntimeError("result sampling order does not match plan")
            for token_id in result.sampled_token_ids:
                _check_token_id(token_id)
            self._launched.popleft()
            accepted = []
            for request_id, token_id in zip(sampled, result.sampled_token_ids):
                request = self._requests.get(request_id)
                slots = self._unresolved.get(request_id)
                if request is None or request.terminal or not slots or slots[0][0] != plan_id:
                    continue
                index = slots.popleft()[1]
                if not slots:
                    del self._unresolved[request_id]
                request.output_token_ids[index] = token_id
                accepted.append((request_id, token_id))
                if request.first_token_ns is None:
                    request.first_token_ns = now_ns
                if token_id in self._eos and not request.sampling.ignore_eos:
                    self._stop_speculation(request, index)
                    self._terminate(request, RequestStatus.FINISHED, now_ns)
                elif request_id in self._finishing and request_id not in self._unresolved:
                    self._finishing.discard(request_id)
                    self._terminate(request, RequestStatus.FINISHED, now_ns)
                else:
                    self._publish_known(request)
        except Exception:
            self.shutdown()
            raise
        self._now = now_ns
        return tuple(accepted)

    def _publish_known(self, request: RequestState) -> None:
        """Publish full blocks whose token ids are all on the host."""
        pending = len(self._unresolved.get(request.request_id, ()))
        self._blocks.cache_full_blocks(request.request_id, request.token_slice,
                                       request.total_tokens - pending)

    def _stop_speculation(self, request: RequestState, last: int) -> None:
        """Drop outputs after index ``last`` (rows launched past a stop) and
        take the request out of the decode and finishing queues."""
        request_id = request.request_id
        del request.output_token_ids[last + 1:]
        self._unresolved.pop(request_id, None)
        if request_id in self._finishing:
            self._finishing.discard(request_id)
        elif request_id in self._decoding:
            self._decoding.remove(request_id)

    def fail_step(self, txn: ScheduleTxn) -> None:
        self._require(txn, TxnState.DISPATCHED)
        self.shutdown()

    def shutdown(self) -> None:
        """Permanently stop scheduling and discard all KV ownership."""
        self._failed = True
        txn = self._txn
        self._blocks.teardown(None if txn is None else txn.kv)
        if txn is not None:
            object.__setattr__(txn, "state", TxnState.FAILED)
        for request in self._requests.values():
            request.active_slot = None
        self._requests.clear()
        self._finished.clear()
        self._arrivals.clear()
        self._stale_arrivals = 0
        self._waiting.clear()
        self._prefilling.clear()
        self._decoding.clear()
        self._launched.clear()
        self._unresolved.clear()
        self._finishing.clear()
        self._slots = [None] * self.max_active_requests
        self._txn = None
        self._commands_applied = False

    # ------------------------------------------------------------ helpers --

    def _healthy(self) -> None:
        if self._failed:
            raise RuntimeError("scheduler is failed")

    def _require(self, txn: ScheduleTxn, state: TxnState) -> None:
        if txn is not self._txn:
            raise ValueError("transaction is not the scheduler's open transaction")
        if txn.state is not state:
            raise RuntimeError(f"transaction must be {state.name.lower()}")

    def _check_now(self, now_ns: int) -> None:
        _check_non_negative_int("now_ns", now_ns)
        if self._now is not None and now_ns < self._now:
            raise ValueError("now_ns cannot move backwards")

    def _demand(self, prompt_len: int, sampling: SamplingParams) -> int:
        """Worst-case blocks of a request (its last sampled token is never written)."""
        outputs = min(sampling.max_new_tokens, self.max_model_len - prompt_len)
        if outputs == 0:
            return 0
        return -(-(prompt_len + outputs - 1) // self.kv_block_size)

    def _admissions(self) -> list[_Prefill]:
        """Waiting requests that fit a free slot and the KV budget, in order."""
        if not self._waiting:
            return []
        blocks = self._blocks
        cache = blocks.prefix_cache
        budget = blocks.free_block_count
        pending: set[bytes] = set()
        for request_id in self._slots:
            if request_id is None:
                continue
            request = self._requests[request_id]
            budget -= self._demand(len(request.prompt_token_ids), request.sampling) \
                - len(blocks.block_table(request_id))
            if request.work_class is WorkClass.PREFILL:
                key = cache.next_prefill_key(request_id, request.computed_tokens,
                                             len(request.prompt_token_ids),
                                             self.prefill_chunk_size)
                if key is not None:
                    pending.add(key)
        free_slots = iter([s for s, r in enumerate(self._slots) if r is None])
        slot = next(free_slots, None)
        out: list[_Prefill] = []
        pinned: set[BlockRef] = set()
        for request_id in self._waiting:
            if slot is None:
                break
            request = self._requests[request_id]
            prefix = blocks.match_prefix(request_id, request.prompt_token_ids)
            start = len(prefix) * self.kv_block_size
            key = cache.next_prefill_key(request_id, start, len(request.prompt_token_ids),
                                         self.prefill_chunk_size)
            if key is not None and key in pending:
                continue  # another request is computing this block right now
            repinned = {r for r in prefix
                        if blocks.pool.state(r) is BlockState.CACHED and r not in pinned}
            cost = self._demand(len(request.prompt_token_ids), request.sampling) \
                - len(prefix) + len(repinned)
            if cost > budget:
                continue
            out.append(_Prefill(request, slot, start, prefix))
            budget -= cost
            pinned |= repinned
            if key is not None:
                pending.add(key)
            slot = next(free_slots, None)
        return out

    def _item(self, request: RequestState, slot: int, work: WorkClass, start: int,
              count: int) -> WorkItem:
        end = start + count
        return WorkItem(
            request_id=request.request_id, request_slot=slot, work_class=work,
            token_start=start, query_len=count, context_len_before=start,
            should_sample=(work is WorkClass.DECODE
                           or (end == request.total_tokens and end < self.max_model_len)),
        )

    def _chunks(self, candidates: list[_Prefill], start: int, row_budget: int,
                token_budget: int, spread: bool) -> tuple[list[WorkItem], int, int]:
        """Prefill chunks for candidates[start:]; with ``spread`` every later
        candidate keeps at least one token of the budget."""
        count = min(len(candidates) - start, row_budget, token_budget)
        items: list[WorkItem] = []
        used = 0
        for k in range(count):
            c = candidates[start + k]
            later = count - k - 1 if spread else 0
            n = min(c.request.total_tokens - c.start, self.prefill_chunk_size,
                    token_budget - used - later)
            if n <= 0:
                break
            items.append(self._item(c.request, c.slot, WorkClass.PREFILL, c.start, n))
            used += n
        return items, start + len(items), used

    def _abort(self, request: RequestState, now_ns: int) -> None:
        if request.terminal:
            return
        if request.status is RequestStatus.PENDING:
            self._stale_arrivals += 1
        elif request.status is RequestStatus.WAITING:
            self._waiting.remove(request.request_id)
        elif request.work_class is WorkClass.DECODE:
            slots = self._unresolved.get(request.request_id)
            self._stop_speculation(request, slots[0][1] - 1 if slots
                                   else len(request.output_token_ids) - 1)
        else:
            self._prefilling.remove(request.request_id)
        self._terminate(request, RequestStatus.ABORTED, now_ns)

    def _terminate(self, request: RequestState, status: RequestStatus, now_ns: int) -> None:
        request.status = status
        request.finished_ns = now_ns
        if request.active_slot is not None:
            self._slots[request.active_slot] = None
            request.active_slot = None
        self._blocks.release_request(request.request_id)
        self._finished.append(CompletionEvent.from_request(request))

    def _live(self, entry: tuple[int, int, int]) -> bool:
        request = self._requests.get(entry[2])
        return (request is not None and request.status is RequestStatus.PENDING
                and request.submit_seq == entry[1])

    def _compact(self) -> None:
        if self._stale_arrivals < 64 or self._stale_arrivals * 2 < len(self._arrivals):
            return
        self._arrivals = [e for e in self._arrivals if self._live(e)]
        heapify(self._arrivals)
        self._stale_arrivals = 0

    def _promote(self, now_ns: int) -> None:
        """Move arrived requests to the waiting queue (or finish trivial ones)."""
        while self._arrivals and self._arrivals[0][0] <= now_ns:
            entry = heappop(self._arrivals)
            if not self._live(entry):
                self._stale_arrivals -= 1
                continue
            request = self._requests[entry[2]]
            if (request.sampling.max_new_tokens == 0
                    or len(request.prompt_token_ids) == self.max_model_len):
                request.admitted_ns = now_ns
                self._terminate(request, RequestStatus.FINISHED, now_ns)
            else:
                request.status = RequestStatus.WAITING
                self._waiting.append(request.request_id)
