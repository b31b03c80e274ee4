"""Local HF tokenizer wrapper (reference: tinyvllm/serving/tokenizer.py:24-141).
Loads only from the model directory (no network)."""
from __future__ import annotations

from collections.abc import Mapping, Sequence
from pathlib import Path


class Tokenizer:
    def __init__(self, model_dir: str | Path) -> None:
        from transformers import AutoTokenizer

        self._tok = AutoTokenizer.from_pretrained(str(model_dir), local_files_only=True,
                                                  trust_remote_code=False)

    def encode(self, text: str) -> tuple[int, ...]:
        ids = tuple(self._tok.encode(text, add_special_tokens=False))
        if not ids:
            raise ValueError("prompt encodes to no tokens")
        return ids

    def encode_chat(self, messages: Sequence[Mapping[str, str]], *,
                    enable_thinking: bool = False) -> tuple[int, ...]:
        ids = self._tok.apply_chat_template(list(messages), tokenize=True,
                                            add_generation_prompt=True,
                                            enable_thinking=enable_thinking)
        return tuple(ids)

    def decode(self, token_ids: Sequence[int]) -> str:
        return self._tok.decode(list(token_ids), skip_special_tokens=True)
