"""Qwen3 building blocks (reference: tinyvllm/layers.py:19-251).

Dense projections stay on PyTorch-ROCm GEMMs (hipBLASLt); normalisation and
activation run on the HIP kernels of ``tinyvllm.kernels.pointwise``.
"""
from __future__ import annotations

import math
from collections.abc import Sequence

import torch
import torch.nn.functional as F
from torch import nn

from tinyvllm._validation import _check_positive_int
from tinyvllm.kernels.pointwise import (
    add_rms_norm, add_rms_norm_partials, rms_norm, silu_and_mul,
)


class PackedLinear(nn.Module):
    """Bias-free linear layer whose output rows pack several named shards
    (q|k|v, gate|up), so one GEMM serves them all (reference layers.py:19-125)."""

    def __init__(
        self,
        input_size: int,
        output_sizes: Sequence[int],
        *,
        shard_names: Sequence[str] | None = None,
        device: torch.device | str | None = None,
        dtype: torch.dtype | None = None,
    ) -> None:
        super().__init__()
        _check_positive_int("input_size", input_size)
        self.input_size = input_size
        self.output_sizes = tuple(output_sizes)
        if not self.output_sizes:
            raise ValueError("output_sizes must be non-empty")
        for size in self.output_sizes:
            _check_positive_int("output_size", size)
        names = (tuple(str(i) for i in range(len(self.output_sizes)))
                 if shard_names is None else tuple(shard_names))
        if len(names) != len(self.output_sizes):
            raise ValueError("shard_names must match output_sizes")
        if len(set(names)) != len(names):
            raise ValueError("shard_names must be unique")
        self.shard_names = names
        self._index = {name: i for i, name in enumerate(names)}
        starts = [0]
        for size in self.output_sizes:
            starts.append(starts[-1] + size)
        self._starts = tuple(starts)
        self.weight = nn.Parameter(
            torch.empty(starts[-1], input_size, device=device, dtype=dtype)
        )
        self.reset_parameters()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(x, self.weight)

    def decode_partials(self, x: torch.Tensor, splits: int = 4) -> torch.Tensor | None:
        """fp32 [splits, rows, out] partial products over ``splits`` slices of
        the reduction axis (one batched torch.bmm), or None where one GEMM
        is faster end to end. For a consumer that sums them itself (the fused
        decode kernel sums the qkv projection's four slices in its prologue,
        which costs it a few more loads per lane). hipBLASLt's single GEMM
        leaves most CUs idle at decode batch sizes; measured on MI355X in
        graph replay (bf16 qkv, us, F.linear -> four slices): 1024 -> 4096
        (0.6B) 64 rows 11.5 -> 7.3, 32 rows 11.1 -> 6.5, 16 rows 7.4 -> 6.7,
        1 row 7.4 -> 5.5; 4096 -> 6144 (8B) 64 rows 17.8 -> 15.6, 16-32 rows
        and 1 row no gain; 5120 -> 10240 (32B) 64 rows 35.6 -> 25.3, 1-32
        rows slower. End to end, gains under ~3 us per layer were taken back
        by the decode kernel's prologue (0.6B at 1 and 16 rows: TPOT 1.40 ->
        1.41 and 1.55 -> 1.60 ms; 8B at 64 rows: no change), so only the
        0.6B width at 32-64 rows (C3: 14.9k -> 15.4k tok/s) and widths of
        5120 and more at 48-64 rows take the split."""
        rows, k = x.shape if x.dim() == 2 else (0, 0)
        if (not x.is_cuda or x.dim() != 2 or not x.is_contiguous() or rows > 64
                or k % (8 * splits)):
            return None
        if not ((k <= 2048 and rows >= 32) or (k >= 5120 and rows >= 48)):
            return None
        xs = x.view(rows, splits, k // splits).transpose(0, 1)
        ws = self.weight.view(self.weight.shape[0], splits, k // splits).permute(1, 2, 0)
        return torch.bmm(xs, ws, out_dtype=torch.float32)

    def reset_parameters(self) -> None:
        if self.weight.device.type == "meta":
            return
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))

    def load_shard(self, shard: str | int, loaded_weight: torch.Tensor) -> None:
        """Copy one logical shard (by name or index) into its packed rows."""
        if isinstance(shard, str):
            if shard not in self._index:
                raise KeyError(f"unknown shard: {shard}")
            index = self._index[shard]
        else:
            index = shard
        if not isinstance(index, int) or not 0 <= index < len(self.output_sizes):
            raise IndexError(f"shard index out of range: {index}")
        start, size = self._starts[index], self.output_sizes[index]
        expected = (size, self.input_size)
        if tuple(loaded_weight.shape) != expected:
            raise ValueError(
                f"expected shard shape {expected}, got {tuple(loaded_weight.shape)}"
            )
        with torch.no_grad():
            self.weight[start:start + size].copy_(loaded_weight)


class SplitKPartials:
    """fp32 partial products [splits, tokens, out_features] of a split-K
    projection; the consumer (RMSNorm.add) sums and rounds them."""

    __slots__ = ("partials", "dtype")

    def __init__(self, partials: torch.Tensor, dtype: torch.dtype) -> None:
        self.partials = partials
        self.dtype = dtype

    @property
    def shape(self) -> torch.Size:
        return self.partials.shape[1:]

    def materialize(self) -> torch.Tensor:
        """The projection's output as F.linear would return it."""
        return self.partials.sum(0).to(self.dtype)


class SplitKLinear(nn.Linear):
    """Bias-free nn.Linear whose output feeds an RMSNorm.add (the attention
    output and MLP down projections). For skinny inputs - the decode batch -
    hipBLASLt's single GEMM leaves most of the GPU idle, so the product runs
    as a batched torch.bmm over ``splits`` slices of the reduction axis with
    fp32 outputs, returned as SplitKPartials for RMSNorm.add to sum inside
    its kernel. Other inputs take F.linear. Measured on MI355X in graph
    replay (bf16, us, F.linear -> split-K):
      4096x12288 (8B down): 64 rows 37 -> 24 (4), 128 rows 67 -> 28 (4);
        1-16 rows 22 -> 22 (4)
      4096x4096 (8B o): 1-16 rows 15.5 -> 9.7 (4), 64 rows 15.0 -> 14.9 (4)
      1024x2048 (0.6B o): 1-16 rows 8.1 -> 4.5-4.8 (8)
      1024x3072 (0.6B down): 1-16 rows 9.4-11.4 -> 4.8-7.0 (8)
      129-512 rows: 8B down 8 slices (256 rows 57 -> 41), 8B o 4 (512 rows
        34 -> 26), 0.6B 2 (512-row down 13.8 -> 10.5)"""

    def __init__(self, in_features: int, out_features: int, *, device=None,
                 dtype=None) -> None:
        super().__init__(in_features, out_features, bias=False, device=device, dtype=dtype)

    def splits_for(self, rows: int) -> int:
        narrow = self.out_features <= 2048
        if rows > 512:
            s = 1
        elif rows > 128:  # prefill chunks and mixed steps
            s = 2 if narrow else 8 if self.in_features >= 8192 else 4
        else:  # narrow outputs need more slices to fill the GPU
            s = 8 if narrow else 4
        return s if self.in_features % (8 * s) == 0 else 1

    def forward(self, x: torch.Tensor) -> torch.Tensor | SplitKPartials:
        # Split-K views the rows in place: only for contiguous 2-D GPU inputs
        # (torch.bmm with an fp32 out_dtype is a GPU-only overload).
        split_ok = x.dim() == 2 and x.is_cuda and x.is_contiguous()
        s = self.splits_for(x.shape[0]) if split_ok else 1
        if s == 1:
            return F.linear(x, self.weight)
        rows, k = x.shape
        xs = x.view(rows, s, k // s).transpose(0, 1)
        ws = self.weight.view(self.out_features, s, k // s).permute(1, 2, 0)
        return SplitKPartials(torch.bmm(xs, ws, out_dtype=torch.float32), x.dtype)


class RMSNorm(nn.Module):
    """Qwen3 RMSNorm, fp32 variance accumulation (reference layers.py:129-164)."""

    def __init__(
        self,
        hidden_size: int,
        *,
        eps: float = 1e-6,
        device: torch.device | str | None = None,
        dtype: torch.dtype | None = None,
    ) -> None:
        super().__init__()
        if hidden_size <= 0:
            raise ValueError("hidden_size must be positive")
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.weight, self.eps)

    def add(
        self, x: torch.Tensor | SplitKPartials, residual: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """(norm(x + residual), x + residual), both rounded to the storage type;
        split-K partials are summed and rounded first, inside the kernel."""
        if isinstance(x, SplitKPartials):
            return add_rms_norm_partials(x.partials, residual, self.weight, self.eps)
        return add_rms_norm(x, residual, self.weight, self.eps)


class RotaryEmbedding(nn.Module):
    """Half-split RoPE tables (reference layers.py:167-245).

    The reference keeps fp32 cos/sin of every position and casts the
    gathered rows to the activation dtype each forward; casting is
    elementwise, so this module stores the tables already cast (per dtype,
    built on first use) and a forward is one gather per table.
    """

    def __init__(
        self,
        head_dim: int,
        max_position: int,
        *,
        base: float = 1_000_000.0,
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        if head_dim <= 0:
            raise ValueError("head_dim must be positive")
        if max_position <= 0:
            raise ValueError("max_position must be positive")
        if base <= 0:
            raise ValueError("base must be positive")
        if head_dim % 2:
            raise ValueError("head_dim must be even")
        exponents = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim
        inv_freq = 1.0 / (base ** exponents)
        positions = torch.arange(max_position, dtype=torch.float32, device=device)
        angles = torch.outer(positions, inv_freq)
        self.register_buffer("cos", angles.cos(), persistent=False)
        self.register_buffer("sin", angles.sin(), persistent=False)
        self._cast: dict[torch.dtype, tuple[torch.Tensor, torch.Tensor]] = {}

    def _apply(self, fn, recurse=True):  # keep cast tables in sync with .to()
        self._cast = {}
        return super()._apply(fn, recurse)

    def forward(
        self, positions: torch.Tensor, dtype: torch.dtype,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """cos, sin of ``positions`` as [tokens, 1, head_dim / 2] in ``dtype``."""
        tables = self._cast.get(dtype)
        if tables is None:
            if self.cos.is_cuda and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("RoPE tables must be cast before graph capture")
            tables = (self.cos.to(dtype), self.sin.to(dtype))
            self._cast[dtype] = tables
        cos = tables[0].index_select(0, positions).unsqueeze(1)
        sin = tables[1].index_select(0, positions).unsqueeze(1)
        return cos, sin


class SiluAndMul(nn.Module):
    """silu(gate) * up of a packed [gate | up] activation (reference layers.py:248-251)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return silu_and_mul(x)
