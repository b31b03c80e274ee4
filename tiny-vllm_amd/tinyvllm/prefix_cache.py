"""Prefix reuse policy over full KV blocks (reference: tinyvllm/prefix_cache.py:14-193).

A full block of a prompt is identified by a chain hash over every token up
to and including that block, so equal keys mean equal prefixes (and equal
K/V contents). The pool maps keys to physical blocks; this class computes
keys, finds the longest cached prefix of a new request and publishes newly
completed blocks. Ownership changes (retain / release) are applied by the
BlockManager.
"""
from __future__ import annotations

import struct
from collections.abc import Callable, Sequence
from hashlib import blake2b
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    from tinyvllm.cache import BlockPool, BlockRef


def chain_key(parent: bytes, tokens: Sequence[int]) -> bytes:
    """Key of a block given its predecessor's key and its token ids."""
    h = blake2b(parent, digest_size=16)
    h.update(struct.pack(f"<{len(tokens)}q", *tokens))
    return h.digest()


class PrefixCache:
    def __init__(self, *, block_size: int, pool: "BlockPool", enabled: bool) -> None:
        self.block_size = block_size
        self.pool = pool
        self.enabled = enabled
        self._keys: dict[int, list[bytes]] = {}       # request -> block keys
        self._published: dict[int, int] = {}          # request -> blocks indexed
        self.hits = 0
        self.hit_tokens = 0

    def _prompt_keys(self, request_id: int, token_ids: Sequence[int]) -> list[bytes]:
        keys = self._keys.get(request_id)
        if keys is None:
            keys, parent = [], b""
            bs = self.block_size
            for start in range(0, len(token_ids) // bs * bs, bs):
                parent = chain_key(parent, token_ids[start:start + bs])
                keys.append(parent)
            self._keys[request_id] = keys
        return keys

    def match(self, request_id: int, token_ids: Sequence[int]) -> tuple["BlockRef", ...]:
        """Longest cached block prefix of a new request. At least one prompt
        token is always left to compute, so the request still produces logits."""
        if not self.enabled:
            return ()
        keys = self._prompt_keys(request_id, token_ids)
        refs = []
        for key in keys[:(len(token_ids) - 1) // self.block_size]:
            ref = self.pool.lookup(key)
            if ref is None:
                break
            refs.append(ref)
        return tuple(refs)

    def next_prefill_key(self, request_id: int, token_start: int, prompt_len: int,
                         chunk_size: int) -> bytes | None:
        """Key of the last reusable block the next prefill chunk would complete;
        two requests with the same key would compute the same block, so the
        scheduler admits only one of them per step."""
        first = token_start // self.block_size
        reusable = (prompt_len - 1) // self.block_size
        if not self.enabled or first >= reusable:
            return None
        span = -(-chunk_size // self.block_size)
        return self._keys[request_id][min(first + span, reusable) - 1]

    def validate_match(self, request_id: int, refs: tuple["BlockRef", ...]) -> None:
        keys = self._keys.get(request_id, ())
        if len(keys) < len(refs):
            raise ValueError("prefix attachment requires a matched new request")
        for key, ref in zip(keys, refs):
            if self.pool.lookup(key) != ref:
                raise ValueError("prefix match is no longer cached")

    def publish(self, request_id: int, table: tuple["BlockRef", ...], valid_tokens: int,
                token_slice: Callable[[int, int], Sequence[int]]
                ) -> tuple[tuple[int, "BlockRef"], ...]:
        """Index the request's newly completed blocks. Returns (index,
        canonical ref) for blocks whose contents were already cached under
        another physical block."""
        if not self.enabled:
            return ()
        full = valid_tokens // self.block_size
        done = self._published.get(request_id, 0)
        if full == done:
            return ()
        keys = self._keys.setdefault(request_id, [])
        bs = self.block_size
        replaced = []
        for index in range(done, full):
            if index == len(keys):
                tokens = token_slice(index * bs, (index + 1) * bs)
                if len(tokens) != bs:
                    raise ValueError("computed prefix must contain a complete block")
                keys.append(chain_key(keys[-1] if keys else b"", tokens))
            canonical = self.pool.publish(keys[index], table[index])
            if canonical != table[index]:
                replaced.append((index, canonical))
        self._published[request_id] = full
        return tuple(replaced)

    def commit_matches(self, prefixes: dict[int, tuple["BlockRef", ...]]) -> None:
        for request_id, refs in prefixes.items():
            self._published[request_id] = len(refs)
        self.hits += len(prefixes)
        self.hit_tokens += sum(len(r) for r in prefixes.values()) * self.block_size

    def forget_request(self, request_id: int) -> None:
        self._keys.pop(request_id, None)
        self._published.pop(request_id, None)

    def clear(self) -> None:
        self.pool.clear_cache()
        self._keys.clear()
        self._published.clear()
        self.hits = 0
        self.hit_tokens = 0
