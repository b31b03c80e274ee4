"""Qwen3 dense decoder (reference: tinyvllm/models/qwen3.py:1-717).

Per layer (reference op order, qwen3.py:263-303 and :386-412):
  add_rms_norm -> qkv GEMM -> QK-norm + RoPE (+ KV write) -> paged attention
  -> o GEMM -> add_rms_norm -> gate_up GEMM -> SiLU*up -> down GEMM.
GEMMs are PyTorch-ROCm ``F.linear``; everything else is a HIP kernel. When the
attention backend offers ``prepare_qkv`` (the native backend does), the
QK-norm/RoPE kernel also writes K/V into the paged cache, so the separate
store_kv launch of the reference disappears.
"""
from __future__ import annotations

import json
from collections.abc import Mapping
from dataclasses import dataclass, field, fields
from pathlib import Path
from typing import Any

import torch
import torch.nn.functional as F
from torch import nn

from tinyvllm._validation import _check_positive_int
from tinyvllm.kernels.pointwise import qk_norm_rope
from tinyvllm.layers import (
    PackedLinear, RMSNorm, RotaryEmbedding, SiluAndMul, SplitKLinear, SplitKPartials,
)
from tinyvllm.runtime.contracts import AttentionBackend

_REQUIRED_FIELDS = frozenset({
    "vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
    "num_attention_heads", "num_key_value_heads", "head_dim",
    "max_position_embeddings",
})


@dataclass(frozen=True, slots=True)
class Qwen3Config:
    """Model geometry (reference qwen3.py:38-217), parsed from a HF-style
    ``config.json`` mapping without needing transformers at run time."""

    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    max_position_embeddings: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    tie_word_embeddings: bool = False
    eos_token_id: tuple[int, ...] = ()
    extra: Mapping[str, Any] = field(default_factory=dict, compare=False)

    def __post_init__(self) -> None:
        for name in ("vocab_size", "hidden_size", "intermediate_size",
                     "num_hidden_layers", "max_position_embeddings",
                     "num_attention_heads", "num_key_value_heads", "head_dim"):
            _check_positive_int(name, getattr(self, name))
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("attention heads must be divisible by key-value heads")
        if self.head_dim % 2:
            raise ValueError("head_dim must be even")

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> "Qwen3Config":
        """Validate and parse a HF ``config.json`` mapping for model_type qwen3."""
        if not isinstance(data, Mapping):
            raise ValueError("Qwen3 config must be a JSON object")
        if data.get("model_type") != "qwen3":
            raise ValueError("only model_type='qwen3' is supported")
        missing = _REQUIRED_FIELDS - data.keys()
        if missing:
            raise ValueError(f"missing Qwen3 config fields: {', '.join(sorted(missing))}")
        rope = data.get("rope_parameters") or data.get("rope_scaling") or {}
        if rope and rope.get("rope_type", rope.get("type", "default")) != "default":
            raise ValueError("rope_scaling is not supported")
        if data.get("hidden_act", "silu") != "silu":
            raise ValueError("only hidden_act='silu' is supported")
        if data.get("attention_bias", False):
            raise ValueError("attention_bias is not supported")
        if data.get("use_sliding_window", False):
            raise ValueError("sliding-window attention is not supported")
        theta = data.get("rope_theta", rope.get("rope_theta", 1_000_000.0))
        eos = data.get("eos_token_id")
        eos_ids = () if eos is None else ((eos,) if isinstance(eos, int) else tuple(eos))
        known = {f.name for f in fields(cls)}
        return cls(
            **{name: data[name] for name in _REQUIRED_FIELDS},
            rms_norm_eps=float(data.get("rms_norm_eps", 1e-6)),
            rope_theta=float(theta),
            tie_word_embeddings=bool(data.get("tie_word_embeddings", False)),
            eos_token_id=eos_ids,
            extra={k: v for k, v in data.items() if k not in known},
        )

    @classmethod
    def from_model_dir(cls, model_dir: str | Path) -> "Qwen3Config":
        root = Path(model_dir).expanduser().resolve()
        if not root.is_dir():
            raise ValueError(f"model directory does not exist: {root}")
        path = root / "config.json"
        try:
            data = json.loads(path.read_text(encoding="utf-8"))
        except (OSError, UnicodeError, json.JSONDecodeError) as exc:
            raise ValueError(f"cannot read Qwen3 config: {path}") from exc
        return cls.from_dict(data)

    @classmethod
    def from_hf(cls, config: Any) -> "Qwen3Config":
        """From a transformers ``Qwen3Config`` object."""
        return cls.from_dict(config.to_dict())

    @property
    def q_proj_size(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def kv_proj_size(self) -> int:
        return self.num_key_value_heads * self.head_dim


class Qwen3Attention(nn.Module):
    def __init__(self, config: Qwen3Config, *, device=None, dtype=None) -> None:
        super().__init__()
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.scale = self.head_dim ** -0.5
        self.qkv_proj = PackedLinear(
            config.hidden_size,
            (config.q_proj_size, config.kv_proj_size, config.kv_proj_size),
            shard_names=("q", "k", "v"), device=device, dtype=dtype,
        )
        # Split-K at decode batch sizes: its partials go to the next
        # RMSNorm.add, like the MLP down projection's.
        self.o_proj = SplitKLinear(config.q_proj_size, config.hidden_size,
                                device=device, dtype=dtype)
        self.q_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps, device=device, dtype=dtype)
        self.k_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps, device=device, dtype=dtype)

    def forward(
        self,
        hidden_states: torch.Tensor,
        position_embeddings: tuple[torch.Tensor, torch.Tensor],
        *,
        layer_idx: int,
        attention: AttentionBackend,
    ) -> torch.Tensor:
        tokens = hidden_states.shape[0]
        q_size = self.num_heads * self.head_dim
        kv_size = self.num_kv_heads * self.head_dim
        cos, sin = position_embeddings
        # Decode-only steps on a backend that takes the qkv projection as
        # split-K partials: the fused decode kernel sums them itself.
        from_partials = getattr(attention, "attend_qkv_partials", None)
        if from_partials is not None and attention.takes_qkv_partials(self.num_heads):
            parts = self.qkv_proj.decode_partials(hidden_states)
            if parts is not None:
                out = from_partials(layer_idx, parts, self.num_heads, self.q_norm.weight,
                                    self.k_norm.weight, cos, sin, self.q_norm.eps,
                                    self.k_norm.eps, scale=self.scale)
                return self.o_proj(out.reshape(tokens, q_size))
        qkv = self.qkv_proj(hidden_states)
        q = qkv[:, :q_size].view(tokens, self.num_heads, self.head_dim)
        k = qkv[:, q_size:q_size + kv_size].view(tokens, self.num_kv_heads, self.head_dim)
        v = qkv[:, q_size + kv_size:].view(tokens, self.num_kv_heads, self.head_dim)
        prepare = getattr(attention, "prepare_qkv", None)
        if prepare is not None:
            q, k, v = prepare(layer_idx, q, k, v, self.q_norm.weight, self.k_norm.weight,
                              cos, sin, self.q_norm.eps, self.k_norm.eps)
        else:
            q, k = qk_norm_rope(q, k, self.q_norm.weight, self.k_norm.weight, cos, sin,
                                self.q_norm.eps, self.k_norm.eps)
        out = attention(layer_idx, q, k, v, scale=self.scale)
        return self.o_proj(out.reshape(tokens, q_size))


class Qwen3MLP(nn.Module):
    def __init__(self, config: Qwen3Config, *, device=None, dtype=None) -> None:
        super().__init__()
        self.gate_up_proj = PackedLinear(
            config.hidden_size, (config.intermediate_size, config.intermediate_size),
            shard_names=("gate", "up"), device=device, dtype=dtype,
        )
        self.down_proj = SplitKLinear(config.intermediate_size, config.hidden_size,
                                      device=device, dtype=dtype)
        self.act_fn = SiluAndMul()

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor | SplitKPartials:
        """Returns SplitKPartials for decode-sized batches (consumed by the
        next RMSNorm.add)."""
        return self.down_proj(self.act_fn(self.gate_up_proj(hidden_states)))


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, config: Qwen3Config, *, device=None, dtype=None) -> None:
        super().__init__()
        eps = config.rms_norm_eps
        self.input_layernorm = RMSNorm(config.hidden_size, eps=eps, device=device, dtype=dtype)
        self.self_attn = Qwen3Attention(config, device=device, dtype=dtype)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=eps,
                                                device=device, dtype=dtype)
        self.mlp = Qwen3MLP(config, device=device, dtype=dtype)

    def forward(self, hidden_states, position_embeddings, *, residual, layer_idx, attention):
        if residual is None:
            residual = hidden_states
            hidden_states = self.input_layernorm(hidden_states)
        else:
            hidden_states, residual = self.input_layernorm.add(hidden_states, residual)
        hidden_states = self.self_attn(hidden_states, position_embeddings,
                                       layer_idx=layer_idx, attention=attention)
        hidden_states, residual = self.post_attention_layernorm.add(hidden_states, residual)
        return self.mlp(hidden_states), residual


class Qwen3Model(nn.Module):
    def __init__(self, config: Qwen3Config, *, device=None, dtype=None) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size,
                                         device=device, dtype=dtype)
        self.rotary_emb = RotaryEmbedding(config.head_dim, config.max_position_embeddings,
                                          base=config.rope_theta, device=device)
        self.layers = nn.ModuleList(
            Qwen3DecoderLayer(config, device=device, dtype=dtype)
            for _ in range(config.num_hidden_layers)
        )
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps,
                            device=device, dtype=dtype)

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, *,
                attention: AttentionBackend) -> torch.Tensor:
        if input_ids.ndim != 1 or input_ids.numel() == 0:
            raise ValueError("input_ids must be a flat 1-D tensor")
        if input_ids.dtype is not torch.long or positions.dtype is not torch.long:
            raise TypeError("input_ids and positions must use torch.long")
        if positions.shape != input_ids.shape or positions.device != input_ids.device:
            raise ValueError("positions must align with input_ids on the same device")
        hidden = self.embed_tokens(input_ids)
        rope = self.rotary_emb(positions, hidden.dtype)
        residual = None
        for index, layer in enumerate(self.layers):
            hidden, residual = layer(hidden, rope, residual=residual, layer_idx=index,
                                     attention=attention)
        hidden, _ = self.norm.add(hidden, residual)
        return hidden


class Qwen3ForCausalLM(nn.Module):
    def __init__(self, config: Qwen3Config, *, device=None, dtype=None) -> None:
        super().__init__()
        self.config = config
        self.model = Qwen3Model(config, device=device, dtype=dtype)
        if config.tie_word_embeddings:
            self.lm_head = None
        else:
            self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False,
                                     device=device, dtype=dtype)
        self._weight_routes = self._make_weight_routes()

    @property
    def lm_head_weight(self) -> torch.Tensor:
        if self.lm_head is None:
            return self.model.embed_tokens.weight
        return self.lm_head.weight

    @classmethod
    def from_pretrained(cls, model_dir: str | Path, *, device=None, dtype=None):
        from tinyvllm.checkpoint import load_weights

        model = cls(Qwen3Config.from_model_dir(model_dir), device=device, dtype=dtype)
        load_weights(model, model_dir)
        return model.eval()

    @classmethod
    def random_init(cls, config: Qwen3Config, *, device, dtype=torch.bfloat16,
                    seed: int = 0, std: float = 0.02) -> "Qwen3ForCausalLM":
        """Random-init weights N(0, std), norm weights 1 (benchmark configs)."""
        with torch.device("meta"):
            model = cls(config, dtype=dtype)
        model = model.to_empty(device=device)
        model.model.rotary_emb = RotaryEmbedding(
            config.head_dim, config.max_position_embeddings, base=config.rope_theta,
            device=device,
        )
        generator = torch.Generator(device=device).manual_seed(seed)
        with torch.no_grad():
            for name, param in model.named_parameters():
                if name.endswith("norm.weight"):
                    param.fill_(1.0)
                else:
                    param.normal_(0.0, std, generator=generator)
        return model.eval()

    @property
    def required_weight_names(self) -> frozenset[str]:
        names = set(self._weight_routes)
        if self.config.tie_word_embeddings:
            names.discard("lm_head.weight")
        return frozenset(names)

    def _make_weight_routes(self) -> dict[str, tuple[str, str | None]]:
        """Checkpoint tensor name -> (parameter / packed module, shard)
        (reference qwen3.py:569-648)."""
        routes: dict[str, tuple[str, str | None]] = {
            "model.embed_tokens.weight": ("model.embed_tokens.weight", None),
            "model.norm.weight": ("model.norm.weight", None),
        }
        for i in range(self.config.num_hidden_layers):
            p = f"model.layers.{i}"
            for name in ("input_layernorm", "post_attention_layernorm"):
                routes[f"{p}.{name}.weight"] = (f"{p}.{name}.weight", None)
            for shard in ("q", "k", "v"):
                routes[f"{p}.self_attn.{shard}_proj.weight"] = (f"{p}.self_attn.qkv_proj", shard)
            for name in ("o_proj", "q_norm", "k_norm"):
                routes[f"{p}.self_attn.{name}.weight"] = (f"{p}.self_attn.{name}.weight", None)
            for shard in ("gate", "up"):
                routes[f"{p}.mlp.{shard}_proj.weight"] = (f"{p}.mlp.gate_up_proj", shard)
            routes[f"{p}.mlp.down_proj.weight"] = (f"{p}.mlp.down_proj.weight", None)
        routes["lm_head.weight"] = (
            "model.embed_tokens.weight" if self.config.tie_word_embeddings
            else "lm_head.weight", None,
        )
        return routes

    def load_weight(self, source_name: str, tensor: torch.Tensor) -> str:
        """Route one checkpoint tensor into its parameter; returns the
        parameter name it filled."""
        try:
            target, shard = self._weight_routes[source_name]
        except KeyError as exc:
            raise KeyError(f"unexpected Qwen3 weight: {source_name}") from exc
        if shard is None:
            param = self.get_parameter(target)
            if tuple(tensor.shape) != tuple(param.shape):
                raise ValueError(f"{source_name}: expected shape {tuple(param.shape)}, "
                                 f"got {tuple(tensor.shape)}")
            with torch.no_grad():
                param.copy_(tensor)
        else:
            self.get_submodule(target).load_shard(shard, tensor)
        if self.config.tie_word_embeddings and source_name == "lm_head.weight":
            return "model.embed_tokens.weight"
        return source_name

    def forward(self, input_ids, positions, *, attention: AttentionBackend):
        return self.model(input_ids, positions, attention=attention)

    def compute_logits(self, hidden_states: torch.Tensor,
                       token_indices: torch.Tensor | None = None) -> torch.Tensor:
        if token_indices is not None:
            hidden_states = hidden_states.index_select(0, token_indices)
        return F.linear(hidden_states, self.lm_head_weight)
