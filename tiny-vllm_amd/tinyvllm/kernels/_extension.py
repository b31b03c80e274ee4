"""Loader for the gfx950 kernel library (``libtinyvllm_hip.so``) over ctypes.

The reference JIT-compiles its CUDA sources and registers them as
``torch.ops.tinyvllm_cuda`` (tinyvllm/kernels/_extension.py:11-42). Here the
kernels are a prebuilt C-ABI shared object (declared in
``include/tinyvllm_hip.h``); this module binds its entry points once and
turns a non-zero status into ``RuntimeError`` carrying the library's message,
the same exception type the reference's ``TORCH_CHECK`` raises.

There is no fallback: if the library is missing or cannot be loaded, every
op raises. Build it with ``python -m tinyvllm.kernels.build``.
"""
from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libtinyvllm_hip.so"
ABI_VERSION = 5

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_INT = ctypes.c_int

_SIGNATURES: dict[str, tuple[type, list[type]]] = {
    "tvllm_last_error": (ctypes.c_char_p, []),
    "tvllm_abi_version": (_INT, []),
    "tvllm_source_hash": (ctypes.c_char_p, []),
    "tvllm_store_kv": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P, _P, _P,
                              _I64, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _F32, _F32,
                              _P]),
    "tvllm_paged_decode_workspace_size": (_I64, [_I64] * 6),
    "tvllm_paged_decode_split_plan": (_I64, [_I64] * 6),
    "tvllm_paged_decode": (_INT, [_P, _I64, _I64, _P, _P, _P, _I64, _I64,
                                  _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                  _I64, _I64, _I64, _I64, _I64, _F32, _P, _I64, _INT, _INT,
                                  _F32, _F32, _P]),
    "tvllm_paged_decode_noalloc": (_INT, [_P, _I64, _I64, _P, _P, _P, _I64, _I64,
                                          _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                          _I64, _I64, _I64, _I64, _I64, _F32, _INT, _INT,
                                          _F32, _F32, _P]),
    "tvllm_paged_decode_qk_norm_rope": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64,
                                               _I64, _P, _P, _P, _P, _F32, _F32, _P, _P,
                                               _P, _P, _I64, _I64, _P, _P, _P, _P, _I64,
                                               _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                               _I64, _F32, _P, _I64, _INT, _INT, _F32, _F32,
                                               _P]),
    "tvllm_paged_decode_qk_norm_rope_partials": (
        _INT, [_P, _I64, _I64, _P, _P, _P, _P, _F32, _F32, _P, _P, _P, _P, _I64, _I64, _P,
               _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _P,
               _I64, _INT, _INT, _F32, _F32, _P]),
    "tvllm_rms_norm": (_INT, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64,
                              _P, _P, _F32, _INT, _P]),
    "tvllm_silu_and_mul": (_INT, [_P, _I64, _I64, _I64, _I64, _I64, _P, _INT, _P]),
    "tvllm_add_rms_norm_partials": (_INT, [_P, _I64, _I64, _I64, _I64, _P, _P, _I64,
                                           _P, _P, _F32, _INT, _P]),
    "tvllm_qk_norm_rope": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P,
                                  _P, _I64, _I64, _I64, _I64, _F32, _F32, _P,
                                  _P, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _I64,
                                  _INT, _INT, _F32, _F32, _P]),
    "tvllm_argmax": (_INT, [_P, _I64, _I64, _I64, _P, _INT, _P]),
    "tvllm_sample_workspace_size": (_I64, [_I64, _I64]),
    "tvllm_sample": (_INT, [_P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P,
                            _I64, _INT, _P]),
    "tvllm_resolve_tokens": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "tvllm_apply_table_updates": (_INT, [_P, _I64, _P, _I64, _P]),
    "tvllm_paged_prefill": (_INT, [_P, _I64, _I64, _P, _P, _P, _I64, _I64, _P,
                                   _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                   _I64, _I64, _I64, _I64, _F32, _P, _I64, _INT, _INT, _F32,
                                   _F32, _P]),
    "tvllm_paged_prefill_workspace_size": (_I64, [_INT, _INT]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2,
               torch.float8_e4m3fn: 3}  # FP8 E4M3: KV-cache storage only


@lru_cache(maxsize=1)
def load_kernels() -> ctypes.CDLL:
    """Load and bind the kernel library once; raises if it is unavailable."""
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"tinyvllm HIP kernels not built: {LIBRARY_PATH} is missing "
            "(run python -m tinyvllm.kernels.build)"
        )
    # torch must own the HIP runtime first so the library binds to the same
    # libamdhip64 instance (one set of streams and graphs per process).
    import torch  # noqa: F401

    lib = ctypes.CDLL(str(LIBRARY_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.tvllm_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(
            f"tinyvllm HIP library ABI {version} does not match {ABI_VERSION}; rebuild it"
        )
    from .build import CSRC_DIR, source_hash

    if CSRC_DIR.is_dir():  # sources travel with the tree; refuse a stale build
        built = lib.tvllm_source_hash().decode()
        expected = source_hash()
        if built != expected:
            raise RuntimeError(
                f"{LIBRARY_PATH.name} was built from other sources (digest {built}, "
                f"sources {expected}); rebuild it (python -m tinyvllm.kernels.build)"
            )
    return lib


def check(status: int) -> None:
    """Raise RuntimeError with the library's message for a failed call."""
    if status != 0:
        message = load_kernels().tvllm_last_error().decode("utf-8", "replace")
        raise RuntimeError(message or f"tinyvllm kernel failed with status {status}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dtype}") from None


def cache_format(cache) -> tuple[int, float, float]:
    """(dtype code, k_scale, v_scale) of a PagedKVCache for the C ABI."""
    return dtype_code(cache.dtype), float(cache.k_scale), float(cache.v_scale)


def stream_of(device: torch.device) -> int:
    """Handle of torch's current stream on ``device`` (captured by graphs)."""
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one GPU; returns that device."""
    device = tensors[0].device
    if device.type != "cuda":
        raise RuntimeError("tinyvllm kernels require GPU tensors")
    for tensor in tensors[1:]:
        if tensor.device != device:
            raise RuntimeError("tensors must share one GPU device")
    return device
