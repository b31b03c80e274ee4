"""asyncio bridge to an Engine owned by one worker thread
(reference: tinyvllm/async_engine.py:18-429).

The worker thread is the only thread that touches the Engine and the GPU.
Coroutines submit/cancel through a locked inbox; the worker steps the engine
and hands each request's token and completion events to its stream on the
event loop. Errors: ``RequestRejectedError`` (invalid request),
``OverloadedError`` (too many requests or reserved tokens in flight),
``SlowConsumerError`` (a stream buffered more than ``max_buffered_tokens``
unread tokens; its request is cancelled) and ``WorkerError`` (the engine
failed; every stream ends with it).
"""
from __future__ import annotations

import asyncio
import threading
from collections import deque
from collections.abc import Callable, Sequence

from tinyvllm.engine import Engine, TokenEvent
from tinyvllm.request import CompletionEvent, SamplingParams


class RequestRejectedError(ValueError):
    """The engine refused the request (validation)."""


class OverloadedError(RuntimeError):
    """Too many requests or reserved tokens are in flight."""


class SlowConsumerError(RuntimeError):
    """The stream's consumer fell too far behind; its request was cancelled."""


class WorkerError(RuntimeError):
    """The engine worker failed; the bridge is unusable."""


class RequestStream:
    """Async iterator of TokenEvent values ending with one CompletionEvent."""

    def __init__(self, owner: "AsyncEngine", request_id: int, reserved: int) -> None:
        self._owner = owner
        self._request_id = request_id
        self._reserved = reserved
        self._queue: asyncio.Queue = asyncio.Queue()
        self._done = False
        # Tokens handed over by the worker and not yet taken by the consumer
        # (items still in flight to the event loop count too).
        self._buffered = 0
        self._count_lock = threading.Lock()

    def _add_buffered(self, n: int) -> int:
        with self._count_lock:
            self._buffered += n
            return self._buffered

    @property
    def request_id(self) -> int:
        return self._request_id

    def __aiter__(self) -> "RequestStream":
        return self

    async def __anext__(self) -> TokenEvent | CompletionEvent:
        if self._done:
            raise StopAsyncIteration
        item = await self._queue.get()
        if isinstance(item, TokenEvent):
            self._add_buffered(-1)
        if isinstance(item, BaseException):
            self._done = True
            raise item
        if isinstance(item, CompletionEvent):
            self._done = True
        return item

    async def aclose(self) -> None:
        if not self._done:
            self._done = True
            self._owner._post(("cancel", self._request_id))


class AsyncEngine:
    def __init__(self, engine_factory: Callable[[], Engine] | object, *,
                 max_requests: int = 64, max_reserved_tokens: int = 65536,
                 max_buffered_tokens: int = 128) -> None:
        if not callable(engine_factory):
            config = engine_factory
            engine_factory = lambda: Engine.from_config(config)  # noqa: E731
        self._factory = engine_factory
        self._max_requests = max_requests
        self._max_reserved = max_reserved_tokens
        self._max_buffered = max_buffered_tokens
        self._lock = threading.Condition()
        self._inbox: deque = deque()
        self._streams: dict[int, RequestStream] = {}
        self._reserved = 0
        self._thread: threading.Thread | None = None
        self._loop: asyncio.AbstractEventLoop | None = None
        self._stop = False
        self._error: BaseException | None = None
        self._ready = threading.Event()

    @property
    def is_running(self) -> bool:
        return self._thread is not None and self._thread.is_alive() and self._error is None

    async def __aenter__(self) -> "AsyncEngine":
        self._loop = asyncio.get_running_loop()
        self._thread = threading.Thread(target=self._run, name="tinyvllm-owner", daemon=True)
        self._thread.start()
        await asyncio.to_thread(self._ready.wait)
        if self._error is not None:
            raise WorkerError(str(self._error)) from self._error
        return self

    async def __aexit__(self, exc_type, exc, tb) -> None:
        with self._lock:
            self._stop = True
            self._lock.notify()
        if self._thread is not None:
            await asyncio.to_thread(self._thread.join)

    async def submit(self, prompt_token_ids: Sequence[int],
                     sampling: SamplingParams) -> RequestStream:
        if self._error is not None:
            raise WorkerError(str(self._error))
        reserve = len(prompt_token_ids) + sampling.max_new_tokens
        future = self._loop.create_future()
        with self._lock:
            if len(self._streams) >= self._max_requests \
                    or self._reserved + reserve > self._max_reserved:
                raise OverloadedError("too many requests or reserved tokens in flight")
            self._reserved += reserve
            self._inbox.append(("submit", tuple(prompt_token_ids), sampling, reserve, future))
            self._lock.notify()
        return await future

    def _post(self, message) -> None:
        with self._lock:
            self._inbox.append(message)
            self._lock.notify()

    # ------------------------------------------------------- worker side --

    def _deliver(self, stream: RequestStream, item) -> None:
        self._loop.call_soon_threadsafe(stream._queue.put_nowait, item)

    def _resolve(self, future, value=None, error=None) -> None:
        def apply():
            if future.done():
                return
            if error is not None:
                future.set_exception(error)
            else:
                future.set_result(value)
        self._loop.call_soon_threadsafe(apply)

    def _run(self) -> None:
        try:
            engine = self._factory()
        except BaseException as exc:
            self._error = exc
            self._ready.set()
            return
        self._ready.set()
        try:
            while True:
                with self._lock:
                    while not self._inbox and not self._stop and not engine.has_unfinished():
                        self._lock.wait(timeout=0.05)
                    if self._stop:
                        break
                    messages = list(self._inbox)
                    self._inbox.clear()
                for message in messages:
                    self._handle(engine, message)
                if engine.has_unfinished():
                    self._dispatch(engine, engine.step())
        except BaseException as exc:
            self._error = exc
            failure = WorkerError(f"engine worker failed: {exc}")
            for stream in list(self._streams.values()):
                self._deliver(stream, failure)
            self._streams.clear()
        finally:
            try:
                engine.close()
            except BaseException:
                pass

    def _handle(self, engine: Engine, message) -> None:
        if message[0] == "cancel":
            if message[1] in self._streams:
                engine.cancel(message[1])
            return
        _, tokens, sampling, reserve, future = message
        try:
            request_id = engine.submit(tokens, sampling)
        except (ValueError, TypeError) as exc:
            with self._lock:
                self._reserved -= reserve
            self._resolve(future, error=RequestRejectedError(str(exc)))
            return
        stream = RequestStream(self, request_id, reserve)
        self._streams[request_id] = stream
        self._resolve(future, stream)

    def _dispatch(self, engine: Engine, events) -> None:
        for token in events.token_events:
            stream = self._streams.get(token.request_id)
            if stream is None:
                continue
            if stream._add_buffered(1) > self._max_buffered:
                stream._add_buffered(-1)
                engine.cancel(token.request_id)
                self._deliver(stream, SlowConsumerError("stream consumer is too slow"))
                continue
            self._deliver(stream, token)
        for done in events.completion_events:
            stream = self._streams.pop(done.request_id, None)
            if stream is None:
                continue
            with self._lock:
                self._reserved -= stream._reserved
            self._deliver(stream, done)
