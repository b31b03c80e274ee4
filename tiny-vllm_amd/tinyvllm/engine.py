"""Serial engine loop (reference: tinyvllm/engine.py:31-564).

``step()`` applies queued commands, asks the scheduler for one plan,
flattens it (BatchBuilder), runs it on the executor and commits the sampled
tokens. With an executor that can ``launch`` (the GPU executor), steps are
pipelined: ``step()`` launches plan k, commits its KV side, then waits for
plan k-1's tokens and resolves them, so the host plans and uploads each step
while the GPU runs the previous one; token and completion events arrive one
step later than the launch that produced them. Any failure after dispatch is fail-stop: the engine releases all
KV ownership and refuses further work. Time is injectable (``clock``,
``sleep``, ``step(now_ns)``) for deterministic arrival schedules.
"""
from __future__ import annotations

import time
from collections.abc import Callable, Sequence
from contextlib import contextmanager
from dataclasses import dataclass, replace
from typing import TYPE_CHECKING, Protocol

from tinyvllm._validation import _check_non_negative_int
from tinyvllm.batch import BatchBuilder, PreparedBatch, StepResult
from tinyvllm.executor import ExecutorCapabilities
from tinyvllm.request import CompletionEvent, RequestStatus, SamplingParams
from tinyvllm.scheduler import (
    AddCommand, CancelCommand, EngineCommand, ScheduleDecision, Scheduler,
)

if TYPE_CHECKING:
    from tinyvllm.config import EngineConfig


class EngineExecutor(Protocol):
    @property
    def capabilities(self) -> ExecutorCapabilities: ...

    def execute(self, batch: PreparedBatch) -> StepResult: ...

    # Optional: ``launch(batch)`` returning an object with ``result() ->
    # StepResult`` enables pipelined steps.

    def release(self, request_id: int) -> None: ...

    def clear(self) -> None: ...


@dataclass(frozen=True, slots=True)
class GenerateRequest:
    prompt_token_ids: tuple[int, ...]
    sampling: SamplingParams
    request_id: int | None = None
    arrival_ns: int | None = None

    def __post_init__(self) -> None:
        object.__setattr__(self, "prompt_token_ids", tuple(self.prompt_token_ids))
        if not isinstance(self.sampling, SamplingParams):
            raise TypeError("sampling must be SamplingParams")


@dataclass(frozen=True, slots=True)
class TokenEvent:
    request_id: int
    token_id: int


@dataclass(frozen=True, slots=True)
class EngineStepEvents:
    token_events: tuple[TokenEvent, ...] = ()
    completion_events: tuple[CompletionEvent, ...] = ()

    def __post_init__(self) -> None:
        object.__setattr__(self, "token_events", tuple(self.token_events))
        object.__setattr__(self, "completion_events", tuple(self.completion_events))


@dataclass(frozen=True, slots=True)
class RequestOutput:
    request_id: int
    status: RequestStatus
    output_token_ids: tuple[int, ...]
    prompt_token_count: int

    @classmethod
    def from_event(cls, event: CompletionEvent) -> "RequestOutput":
        return cls(event.request_id, event.status, event.output_token_ids,
                   event.prompt_token_count)


class Engine:
    """A serial engine; generate() owns its request batch exclusively."""

    def __init__(self, scheduler: Scheduler, executor: EngineExecutor, *,
                 clock: Callable[[], int] = time.monotonic_ns,
                 sleep: Callable[[float], None] = time.sleep,
                 pipelined: bool | None = None) -> None:
        """``pipelined``: None uses pipelined steps when the executor has
        ``launch``; False forces one step at a time."""
        executor.capabilities.validate_configuration(
            max_model_len=scheduler.max_model_len,
            block_size=scheduler.kv_block_size,
            num_blocks=scheduler.block_manager.pool.num_blocks,
            max_batch_size=min(scheduler.max_step_requests, scheduler.max_scheduled_tokens),
        )
        executor.capabilities.validate_token_ids(scheduler.eos_token_ids)
        self.scheduler = scheduler
        self.executor = executor
        self.builder = BatchBuilder(max_model_len=scheduler.max_model_len)
        self._clock = clock
        self._sleep = sleep
        self._commands: list[EngineCommand] = []
        self._next_seq = scheduler.last_command_seq + 1
        self._active: set[int] = set(scheduler.request_ids)
        self._next_id = max(self._active, default=-1) + 1
        self._cancelling: set[int] = set()
        self._closed = False
        self._failed: str | None = None
        self._generating = False
        can_launch = callable(getattr(executor, "launch", None))
        if pipelined and not can_launch:
            raise ValueError("pipelined steps need an executor with launch()")
        self._pipelined = can_launch if pipelined is None else bool(pipelined)
        self._in_flight = None  # the launched step whose tokens are unresolved

    @classmethod
    def from_config(cls, config: "EngineConfig") -> "Engine":
        from tinyvllm.bootstrap import create_engine

        return create_engine(config)

    # ----------------------------------------------------------- requests --

    def submit(self, prompt_token_ids: Sequence[int], sampling: SamplingParams, *,
               arrival_ns: int | None = None, request_id: int | None = None) -> int:
        self._usable()
        if self._generating:
            raise RuntimeError("generate() owns the engine until it returns")
        commands, next_id = self._stage((GenerateRequest(
            tuple(prompt_token_ids), sampling, request_id, arrival_ns),))
        self._publish(commands, next_id)
        return commands[0].request_id

    def _stage(self, specs) -> tuple[tuple[AddCommand, ...], int]:
        """Validate requests and turn them into sequenced AddCommands."""
        commands: list[AddCommand] = []
        staged: set[int] = set()
        next_id = self._next_id
        for spec in specs:
            if not isinstance(spec, GenerateRequest):
                raise TypeError("requests must contain GenerateRequest values")
            self.scheduler.validate_request(spec.prompt_token_ids, spec.sampling)
            self.executor.capabilities.validate_token_ids(spec.prompt_token_ids)
            arrival = self._clock() if spec.arrival_ns is None else spec.arrival_ns
            _check_non_negative_int("arrival_ns", arrival)
            rid = next_id if spec.request_id is None else spec.request_id
            _check_non_negative_int("request_id", rid)
            if rid in self._active or rid in staged:
                raise ValueError(f"duplicate active request_id: {rid}")
            commands.append(AddCommand(seq=self._next_seq + len(commands), request_id=rid,
                                       prompt_token_ids=spec.prompt_token_ids,
                                       sampling=spec.sampling, arrival_ns=arrival))
            staged.add(rid)
            next_id = max(next_id, rid + 1)
        return tuple(commands), next_id

    def _publish(self, commands: tuple[AddCommand, ...], next_id: int) -> None:
        self._commands.extend(commands)
        self._active.update(c.request_id for c in commands)
        self._next_seq += len(commands)
        self._next_id = next_id

    def cancel(self, request_id: int) -> bool:
        self._usable()
        _check_non_negative_int("request_id", request_id)
        if request_id not in self._active or request_id in self._cancelling:
            return False
        self._commands.append(CancelCommand(seq=self._next_seq, request_id=request_id))
        self._next_seq += 1
        self._cancelling.add(request_id)
        return True

    # -------------------------------------------------------------- steps --

    def step(self, now_ns: int | None = None) -> EngineStepEvents:
        """Plan and run one step. Serial: its tokens come back in its events.
        Pipelined: it is launched, and the previous launch's tokens resolve."""
        self._usable()
        fixed = now_ns is not None
        t0 = now_ns if fixed else self._clock()
        _check_non_negative_int("now_ns", t0)
        pending = tuple(self._commands)
        self.scheduler.apply_commands(pending, t0)
        del self._commands[:len(pending)]
        self._cancelling.difference_update(
            c.request_id for c in pending if isinstance(c, CancelCommand))
        launched, accepted = None, None
        txn = self.scheduler.begin_step(t0)
        if txn is not None:
            launched, accepted = self._run(txn, t0, fixed)
        previous, self._in_flight = self._in_flight, launched
        if previous is not None:
            accepted = self._collect(previous, t0 if fixed else None)
        with self._fatal():
            events = self._events(accepted)
        if not self._active and self._in_flight is not None:
            # What is still in flight belongs to finished requests: drain it.
            previous, self._in_flight = self._in_flight, None
            self._collect(previous, t0 if fixed else None)
        return events

    def _later(self, t: int, fixed: bool) -> int:
        return t if fixed else max(t, self._clock())

    def _run(self, txn, t0: int, fixed: bool):
        """Build, dispatch and execute (or launch) a staged step; returns
        (launch handle, None) or (None, accepted tokens)."""
        try:
            requests = tuple(self.scheduler.get_request(i.request_id) for i in txn.plan.items)
            batch = self.builder.prepare(txn.plan, requests, kv=txn.kv,
                                         pending_rows=self.scheduler.pending_sample_rows())
        except BaseException:
            self.scheduler.rollback(txn)  # nothing was dispatched
            raise
        when = self._later(t0, fixed)
        with self._fatal():
            self.scheduler.mark_dispatched(txn, when)
        with self._fatal("executor failed; engine is failed"):
            out = (self.executor.launch(batch) if self._pipelined
                   else self.executor.execute(batch))
        with self._fatal():
            done = self._later(when, fixed)
            if self._pipelined:
                self.scheduler.commit_launch(txn, done)
                return out, None
            return None, self.scheduler.commit_step(txn, out, done)

    def _collect(self, launched, now_ns: int | None) -> tuple[tuple[int, int], ...]:
        """Wait for a launched step's tokens and hand them to the scheduler."""
        with self._fatal("executor failed; engine is failed"):
            result = launched.result()
        with self._fatal():
            return self.scheduler.resolve(result, self._clock() if now_ns is None else now_ns)

    @contextmanager
    def _fatal(self, message: str | None = None):
        """Any failure inside is fail-stop; ``message`` re-raises it wrapped."""
        try:
            yield
        except BaseException as exc:
            self._fail_stop(exc)
            if message is None:
                raise
            raise RuntimeError(message) from exc

    def has_unfinished(self) -> bool:
        return bool(self._active)

    def generate(self, requests: Sequence[GenerateRequest]) -> list[RequestOutput]:
        """Run a batch of requests to completion (arrivals honoured)."""
        self._usable()
        if self._generating or self.has_unfinished():
            raise RuntimeError("generate() requires an idle engine")
        commands, next_id = self._stage(tuple(requests))
        if not commands:
            return []
        ids = tuple(c.request_id for c in commands)
        self._publish(commands, next_id)
        outputs: dict[int, RequestOutput] = {}
        self._generating = True
        try:
            while self.has_unfinished():
                events = self.step()
                for event in events.completion_events:
                    outputs[event.request_id] = RequestOutput.from_event(event)
                if self.scheduler.last_decision is ScheduleDecision.IDLE:
                    arrival = self.scheduler.next_arrival_ns
                    if arrival is not None:
                        delay = (arrival - self._clock()) / 1e9
                        if delay > 0:
                            self._sleep(delay)
        finally:
            self._generating = False
        if len(outputs) != len(ids):
            raise RuntimeError("engine stopped before all requests completed")
        return [outputs[i] for i in ids]

    def _events(self, accepted: tuple[tuple[int, int], ...] | None) -> EngineStepEvents:
        completions = self.scheduler.consume_finished()
        done = {e.request_id for e in completions}
        # A cancel queued during execute may target a request that just
        # finished: drop it before the request id becomes reusable.
        if done & self._cancelling:
            kept = [c for c in self._commands
                    if not (isinstance(c, CancelCommand) and c.request_id in done)]
            first = self.scheduler.last_command_seq + 1
            self._commands = [replace(c, seq=first + k) for k, c in enumerate(kept)]
            self._next_seq = first + len(kept)
        self._active -= done
        self._cancelling -= done
        for event in completions:
            self.executor.release(event.request_id)
        if not accepted:
            return EngineStepEvents(completion_events=completions)
        tokens = tuple(TokenEvent(r, t) for r, t in accepted)
        return EngineStepEvents(token_events=tokens, completion_events=completions)

    def reset_prefix_cache(self) -> None:
        """Drop reusable prefixes between workloads, without reallocating KV."""
        self._usable()
        if self._generating or self.has_unfinished():
            raise RuntimeError("reset_prefix_cache requires an idle engine")
        self.scheduler.block_manager.reset_prefix_cache()

    def close(self) -> None:
        """Release the scheduler's KV and the executor for good; requests
        still pending are dropped. Idempotent."""
        if self._closed:
            return
        if self._generating:
            raise RuntimeError("cannot close while generate() is running")
        self._closed = True
        problems = self._teardown()
        if problems:
            raise RuntimeError("engine cleanup failed: " + "; ".join(problems))

    def _usable(self) -> None:
        if self._closed:
            raise RuntimeError("engine is closed")
        if self._failed is not None:
            raise RuntimeError(f"engine is failed: {self._failed}")

    def _fail_stop(self, cause: BaseException) -> None:
        """After a failure past dispatch no KV state can be trusted: record
        why, drop everything, and refuse further work."""
        if self._failed is None:
            self._failed = f"{type(cause).__name__}: {cause}"
        for problem in self._teardown():
            _note(cause, problem)

    def _teardown(self) -> list[str]:
        """Forget queued work and shut the scheduler and executor down;
        returns what failed to clean up (every part is attempted)."""
        self._in_flight = None
        self._commands.clear()
        self._active.clear()
        self._cancelling.clear()
        problems = []
        for part, shut in (("scheduler", self.scheduler.shutdown),
                           ("executor", self.executor.clear)):
            try:
                shut()
            except BaseException as err:
                problems.append(f"{part} cleanup failed: {err!r}")
        return problems


def _note(exc: BaseException, message: str) -> None:
    """BaseException.add_note, also on Python 3.10."""
    if hasattr(exc, "add_note"):
        exc.add_note(message)
    else:
        exc.__notes__ = [*getattr(exc, "__notes__", []), message]
