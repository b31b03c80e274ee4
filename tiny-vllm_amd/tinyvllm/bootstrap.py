"""Engine construction: model, KV-pool sizing, scheduler, executor
(reference: tinyvllm/bootstrap.py:19-208)."""
from __future__ import annotations

import logging
import time
from typing import TYPE_CHECKING

import torch

from tinyvllm.config import EngineConfig
from tinyvllm.paged_kv import PagedKVCache
from tinyvllm.runtime.inputs import DecodeInputs

if TYPE_CHECKING:
    from tinyvllm.engine import Engine

logger = logging.getLogger(__name__)


def plan_kv_blocks(*, total_bytes: int, free_bytes: int, utilization: float,
                   requested_bytes: int, bytes_per_block: int,
                   reserved_bytes: int = 0) -> int:
    """Blocks of an explicit KV budget, checked against the device ceiling
    (total x utilization, counting what is already in use)."""
    if total_bytes <= 0 or not 0 <= free_bytes <= total_bytes:
        raise ValueError("invalid device memory snapshot")
    blocks = requested_bytes // bytes_per_block
    if blocks == 0:
        raise ValueError("KV budget cannot hold one complete block")
    available = min(free_bytes, int(total_bytes * utilization) - (total_bytes - free_bytes))
    available -= reserved_bytes
    if blocks * bytes_per_block > available:
        raise ValueError(
            f"KV allocation needs {blocks * bytes_per_block} bytes, but only "
            f"{max(0, available)} bytes remain below the GPU usage ceiling; lower "
            "kv_cache_memory_bytes or free device memory")
    return blocks


def build_engine(model, *, max_model_len: int, max_num_seqs: int = 64,
                 max_num_batched_tokens: int = 4096, kv_block_size: int = 16,
                 num_blocks: int, prefill_chunk_size: int = 512,
                 prefill_reserve_tokens: int = 128, prefill_reserve_requests: int = 1,
                 attention_backend: str = "hip", enforce_eager: bool = False,
                 enable_prefix_caching: bool = True, eos_token_ids=None,
                 graph_sizes=None, clock=None, kv_cache_dtype: torch.dtype | None = None,
                 kv_scales: tuple[float, float] = (1.0, 1.0),
                 pipelined: bool | None = None, kv_cache_layout: str = "auto",
                 prefill_graph_tokens: int | None = None) -> "Engine":
    """Engine around an already built model (random-init benchmarks, tests).
    ``pipelined=False`` runs one step at a time (the reference's loop)."""
    from tinyvllm.engine import Engine
    from tinyvllm.executor import Executor
    from tinyvllm.scheduler import Scheduler

    executor = Executor(model, block_size=kv_block_size, num_blocks=num_blocks,
                        max_model_len=max_model_len, max_num_seqs=max_num_seqs,
                        attention_backend=attention_backend, enforce_eager=enforce_eager,
                        graph_sizes=graph_sizes, kv_cache_dtype=kv_cache_dtype,
                        kv_scales=kv_scales, kv_cache_layout=kv_cache_layout,
                        prefill_graph_tokens=prefill_graph_tokens)
    scheduler = Scheduler(
        max_active_requests=max_num_seqs, max_step_requests=max_num_seqs,
        max_scheduled_tokens=max_num_batched_tokens, prefill_chunk_size=prefill_chunk_size,
        max_model_len=max_model_len, prefill_reserve_tokens=prefill_reserve_tokens,
        prefill_reserve_requests=prefill_reserve_requests, kv_block_size=kv_block_size,
        kv_num_blocks=num_blocks, eos_token_ids=eos_token_ids,
        enable_prefix_caching=enable_prefix_caching)
    kwargs = {} if clock is None else {"clock": clock}
    return Engine(scheduler, executor, pipelined=pipelined, **kwargs)


def create_engine(config: EngineConfig) -> "Engine":
    """Load Qwen3 from ``config.model`` on the current GPU and size the KV pool."""
    from tinyvllm.models.qwen3 import Qwen3Config, Qwen3ForCausalLM

    started = time.perf_counter()
    if not torch.cuda.is_available():
        raise RuntimeError("create_engine requires a GPU")
    model_config = Qwen3Config.from_model_dir(config.model)
    if config.max_model_len > model_config.max_position_embeddings:
        raise ValueError("max_model_len exceeds model position capacity")
    device = torch.device("cuda", torch.cuda.current_device())
    dtype = getattr(torch, config.dtype)
    kv_dtype = torch.float8_e4m3fn if config.kv_cache_dtype == "fp8_e4m3" else dtype
    logger.info("Loading model=%s device=%s dtype=%s attention_backend=%s",
                config.model, device, config.dtype, config.attention_backend)
    model = Qwen3ForCausalLM.from_pretrained(config.model, device=device, dtype=dtype)
    torch.cuda.synchronize(device)
    torch.cuda.empty_cache()
    free, total = torch.cuda.mem_get_info(device)
    per_block = PagedKVCache.bytes_per_block(
        num_layers=model_config.num_hidden_layers, block_size=config.kv_block_size,
        num_kv_heads=model_config.num_key_value_heads, head_dim=model_config.head_dim,
        dtype=kv_dtype)
    reserved = 0
    if config.attention_backend != "reference":
        reserved = DecodeInputs.device_bytes(max_num_seqs=config.max_num_seqs,
                                             max_model_len=config.max_model_len,
                                             block_size=config.kv_block_size)
    blocks = plan_kv_blocks(total_bytes=total, free_bytes=free,
                            utilization=config.gpu_memory_utilization,
                            requested_bytes=config.kv_cache_memory_bytes,
                            bytes_per_block=per_block, reserved_bytes=reserved)
    engine = build_engine(
        model, max_model_len=config.max_model_len, max_num_seqs=config.max_num_seqs,
        max_num_batched_tokens=config.max_num_batched_tokens,
        kv_block_size=config.kv_block_size, num_blocks=blocks,
        prefill_chunk_size=config.prefill_chunk_size,
        prefill_reserve_tokens=config.prefill_reserve_tokens,
        prefill_reserve_requests=config.prefill_reserve_requests,
        attention_backend=config.attention_backend, enforce_eager=config.enforce_eager,
        enable_prefix_caching=config.enable_prefix_caching,
        eos_token_ids=model_config.eos_token_id, kv_cache_dtype=kv_dtype,
        kv_scales=(config.kv_k_scale, config.kv_v_scale),
        kv_cache_layout=config.kv_cache_layout,
        prefill_graph_tokens=config.prefill_graph_tokens)
    logger.info("engine ready in %.1fs: %d KV blocks of %d tokens",
                time.perf_counter() - started, blocks, config.kv_block_size)
    return engine
