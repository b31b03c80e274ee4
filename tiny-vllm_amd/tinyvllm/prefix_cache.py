"""Prefix reuse over full KV blocks (the role of the reference's
tinyvllm/prefix_cache.py).

A full block is named by a digest of every token id from position 0 through
its last token: digest_i = SHA-256(digest_{i-1} || ids of block i as int64),
truncated to 16 bytes. Equal digests therefore mean equal prefixes, hence
equal K/V contents, and a new request can attach the longest run of indexed
blocks at the start of its prompt instead of recomputing it. The pool maps
digests to physical blocks; this module computes digests per request (kept
while the request lives), answers lookups and indexes newly written blocks.
"""
from __future__ import annotations

import hashlib
from collections.abc import Callable, Sequence
from typing import TYPE_CHECKING

import numpy as np

if TYPE_CHECKING:
    from tinyvllm.cache import BlockPool, BlockRef


def block_digests(token_ids: Sequence[int], block_size: int, parent: bytes = b"",
                  count: int | None = None) -> list[bytes]:
    """Digests of the first ``count`` full blocks of ``token_ids`` (all full
    blocks by default), chained from ``parent``."""
    ids = np.asarray(token_ids, dtype="<i8")
    full = len(ids) // block_size if count is None else count
    out = []
    for i in range(full):
        h = hashlib.sha256(parent)
        h.update(ids[i * block_size:(i + 1) * block_size].tobytes())
        parent = h.digest()[:16]
        out.append(parent)
    return out


class _Chain:
    """A live request's block digests and how many of its blocks are indexed."""

    __slots__ = ("digests", "indexed")

    def __init__(self, digests: list[bytes]) -> None:
        self.digests = digests
        self.indexed = 0


class PrefixCache:
    def __init__(self, *, block_size: int, pool: "BlockPool", enabled: bool) -> None:
        self.block_size = block_size
        self.pool = pool
        self.enabled = enabled
        self._chains: dict[int, _Chain] = {}
        self.hits = 0         # requests that attached a cached prefix
        self.hit_tokens = 0   # prompt tokens served from the cache

    def _chain(self, request_id: int, prompt: Sequence[int]) -> _Chain:
        chain = self._chains.get(request_id)
        if chain is None:
            chain = _Chain(block_digests(prompt, self.block_size))
            self._chains[request_id] = chain
        return chain

    def lookup(self, request_id: int, prompt: Sequence[int]) -> tuple["BlockRef", ...]:
        """Indexed blocks at the start of a new request's prompt. The last
        prompt token is always recomputed (its logits are needed), so a
        prompt of n tokens can reuse at most (n - 1) // block_size blocks."""
        if not self.enabled:
            return ()
        chain = self._chain(request_id, prompt)
        limit = (len(prompt) - 1) // self.block_size
        found = []
        for digest in chain.digests[:limit]:
            ref = self.pool.find(digest)
            if ref is None:
                break
            found.append(ref)
        return tuple(found)

    def chunk_digest(self, request_id: int, prompt: Sequence[int], token_start: int,
                     chunk_size: int) -> bytes | None:
        """Digest of the last reusable block the request's next prefill chunk
        (from ``token_start``) completes, or None. Two requests whose next
        chunks complete the same digest would compute the same block: the
        scheduler lets one of them run and the other reuse the result."""
        if not self.enabled:
            return None
        reusable = (len(prompt) - 1) // self.block_size
        first_block = token_start // self.block_size
        last_block = min(first_block + -(-chunk_size // self.block_size), reusable)
        if last_block <= first_block:
            return None
        return self._chain(request_id, prompt).digests[last_block - 1]

    def check_hit(self, request_id: int, refs: tuple["BlockRef", ...]) -> None:
        """The prefix a staged step attaches must still be indexed as found."""
        chain = self._chains.get(request_id)
        if chain is None or len(chain.digests) < len(refs):
            raise ValueError(f"request {request_id}: prefix was not looked up")
        for digest, ref in zip(chain.digests, refs):
            if self.pool.find(digest) != ref:
                raise ValueError(f"request {request_id}: cached prefix block {ref} "
                                 "was evicted or replaced")

    def index_blocks(self, request_id: int, table: tuple[np.ndarray, np.ndarray],
                     full_tokens: int, token_slice: Callable[[int, int], Sequence[int]]
                     ) -> list[tuple[int, "BlockRef"]]:
        """Index the request's blocks completed within ``full_tokens``.
        Returns (table index, block) pairs where an identical block was
        already indexed: the caller points its table there."""
        if not self.enabled:
            return []
        chain = self._chains.setdefault(request_id, _Chain([]))
        full = full_tokens // self.block_size
        if full <= chain.indexed:
            return []
        bs = self.block_size
        if len(chain.digests) < full:  # blocks past the prompt (generated ids)
            start = len(chain.digests)
            tokens = token_slice(start * bs, full * bs)
            if len(tokens) != (full - start) * bs:
                raise ValueError(f"request {request_id}: block token ids are incomplete")
            parent = chain.digests[-1] if chain.digests else b""
            chain.digests += block_digests(tokens, bs, parent)
        from tinyvllm.cache import BlockRef

        swaps = []
        ids, gens = table
        for index in range(chain.indexed, full):
            own = BlockRef(int(ids[index]), int(gens[index]))
            kept = self.pool.label(chain.digests[index], own)
            if kept != own:
                swaps.append((index, kept))
        chain.indexed = full
        return swaps

    def note_hits(self, prefixes: dict[int, tuple["BlockRef", ...]]) -> None:
        """Prefixes attached by a completed step: already indexed, and counted."""
        for request_id, refs in prefixes.items():
            chain = self._chains.get(request_id)
            if chain is not None:
                chain.indexed = max(chain.indexed, len(refs))
            self.hits += 1
            self.hit_tokens += len(refs) * self.block_size

    def drop_request(self, request_id: int) -> None:
        self._chains.pop(request_id, None)

    def reset(self) -> None:
        self.pool.forget_digests()
        self._chains.clear()
        self.hits = 0
        self.hit_tokens = 0
