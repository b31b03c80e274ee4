"""tiny-vLLM's decode token loop on MI355X (gfx950): the reference's public
API over hand-written HIP kernels (see include/tinyvllm_hip.h)."""
from tinyvllm.request import (
    CompletionEvent,
    RequestState,
    RequestStatus,
    SamplingParams,
    WorkClass,
)
from tinyvllm.engine import (
    Engine,
    EngineStepEvents,
    GenerateRequest,
    RequestOutput,
    TokenEvent,
)
from tinyvllm.config import EngineConfig
from tinyvllm.serving.llm import LLM, TextOutput
from tinyvllm.serving.async_llm import AsyncLLM, TextDelta
from tinyvllm.async_engine import (
    AsyncEngine,
    OverloadedError,
    RequestRejectedError,
    RequestStream,
    SlowConsumerError,
    WorkerError,
)

__all__ = [
    "AsyncEngine", "OverloadedError", "RequestRejectedError", "RequestStream",
    "SlowConsumerError", "WorkerError", "LLM", "TextOutput", "CompletionEvent",
    "EngineConfig", "RequestState", "RequestStatus", "SamplingParams", "WorkClass",
    "Engine", "EngineStepEvents", "GenerateRequest", "RequestOutput", "TokenEvent",
    "AsyncLLM", "TextDelta",
]
