"""Engine configuration (reference: tinyvllm/config.py:15-91)."""
from __future__ import annotations

import math
from dataclasses import dataclass
from pathlib import Path
from typing import Literal

from tinyvllm._validation import _check_non_negative_int, _check_positive_int

DType = Literal["bfloat16", "float16"]
BACKENDS = ("hip", "reference", "cuda")
KV_CACHE_DTYPES = ("auto", "fp8_e4m3")
KV_CACHE_LAYOUTS = ("auto", "token_major", "head_major")


@dataclass(frozen=True, slots=True)
class EngineConfig:
    """Same fields and defaults as the reference. ``attention_backend`` is
    "hip" (native kernels, default) or "reference" (torch SDPA gather path);
    "cuda", the reference's name for its native backend, maps to "hip".
    Beyond the reference: ``kv_cache_dtype`` "auto" stores K/V in the model
    dtype, "fp8_e4m3" in OCP FP8 E4M3 (one byte per element) with the scales
    ``kv_k_scale``/``kv_v_scale`` (stored = x / scale, saturated to +-448);
    ``kv_cache_layout`` the storage order behind the reference's [slots,
    heads, dim] cache view ("auto": head-major for fewer than 256 (request,
    KV head) pairs, token-major otherwise); ``prefill_graph_tokens`` the
    largest prefill/mixed step replayed from a captured graph (None: sized
    from the model, 0: prefill always eager)."""

    model: Path
    dtype: DType = "bfloat16"
    attention_backend: str = "hip"
    max_model_len: int = 4096
    max_num_seqs: int = 64
    max_num_batched_tokens: int = 4096
    gpu_memory_utilization: float = 0.9
    kv_block_size: int = 16
    kv_cache_memory_bytes: int = 2 * 1024 ** 3
    prefill_chunk_size: int = 512
    prefill_reserve_tokens: int = 128
    prefill_reserve_requests: int = 1
    enforce_eager: bool = False
    enable_prefix_caching: bool = True
    kv_cache_dtype: str = "auto"
    kv_k_scale: float = 1.0
    kv_v_scale: float = 1.0
    kv_cache_layout: str = "auto"
    prefill_graph_tokens: int | None = None

    def __post_init__(self) -> None:
        model = Path(self.model).expanduser().resolve()
        object.__setattr__(self, "model", model)
        if not model.is_dir():
            raise ValueError(f"model directory does not exist: {model}")
        if self.dtype not in ("bfloat16", "float16"):
            raise ValueError(f"unsupported dtype: {self.dtype}")
        if self.attention_backend not in BACKENDS:
            raise ValueError(f"unsupported attention backend: {self.attention_backend}")
        if self.kv_cache_dtype not in KV_CACHE_DTYPES:
            raise ValueError(f"unsupported kv_cache_dtype: {self.kv_cache_dtype}")
        for name in ("kv_k_scale", "kv_v_scale"):
            value = getattr(self, name)
            if type(value) not in (int, float) or not 0.0 < value < math.inf:
                raise ValueError(f"{name} must be a positive finite number")
        if self.kv_cache_dtype == "auto" and (self.kv_k_scale != 1.0
                                              or self.kv_v_scale != 1.0):
            raise ValueError("KV scales apply to kv_cache_dtype fp8_e4m3 only")
        if self.kv_cache_layout not in KV_CACHE_LAYOUTS:
            raise ValueError(f"unsupported kv_cache_layout: {self.kv_cache_layout}")
        graph_tokens = self.prefill_graph_tokens
        if graph_tokens is not None and (type(graph_tokens) is not int or graph_tokens < 0):
            raise ValueError("prefill_graph_tokens must be None or a non-negative int")
        for name in ("enforce_eager", "enable_prefix_caching"):
            if type(getattr(self, name)) is not bool:
                raise TypeError(f"{name} must be bool")
        for name in ("max_model_len", "max_num_seqs", "max_num_batched_tokens",
                     "prefill_chunk_size", "kv_block_size", "kv_cache_memory_bytes"):
            _check_positive_int(name, getattr(self, name))
        for name in ("prefill_reserve_tokens", "prefill_reserve_requests"):
            _check_non_negative_int(name, getattr(self, name))
        utilization = self.gpu_memory_utilization
        if type(utilization) not in (int, float):
            raise TypeError("GPU memory utilization must be a number")
        if not math.isfinite(utilization) or not 0.0 < utilization < 1.0:
            raise ValueError("GPU memory utilization must be between 0 and 1")
        tokens, requests = self.prefill_reserve_tokens, self.prefill_reserve_requests
        if (tokens == 0) != (requests == 0):
            raise ValueError("prefill reservations must both be zero or positive")
        if not tokens < self.max_num_batched_tokens:
            raise ValueError("prefill token reservation leaves no decode capacity")
        if not requests < self.max_num_seqs:
            raise ValueError("prefill request reservation leaves no decode capacity")
        if tokens < requests:
            raise ValueError("each reserved prefill request needs one token")
        if self.prefill_chunk_size > self.max_num_batched_tokens:
            raise ValueError("prefill chunk exceeds the step token budget")
