"""Host-side ownership of KV-cache blocks (the role of the reference's
tinyvllm/cache.py; the slot arithmetic of cache.py:696-711 is the shared
contract: logical position p of a request lives at slot
``table[p // block_size] * block_size + p % block_size``).

Design:

* ``BlockPool`` keeps per-block holder counts and generations in numpy
  arrays. Unheld blocks sit in one of two places: a stack of *blank* blocks
  (no reusable contents, handed out first) or an eviction heap of *idle*
  blocks whose contents are still indexed by a prefix digest (handed out
  oldest-released first, losing their digest). Heap entries are stamped, so
  re-holding an idle block needs no removal: the stale entry is skipped.
* ``StepKV`` is one step's journal. Staging applies the step's allocations
  and prefix pins to the pool at once and records them; ``undo`` reverses
  exactly those records. ``go_live`` makes the new tables the requests'
  tables (ownership is visible from the dispatch on), ``writes_done``
  advances each request's valid KV length and counts prefix hits. After
  ``go_live`` the only way back is the fail-stop ``teardown``.
* ``BlockManager`` holds each request's table as an int64 id array plus the
  generations it was taken at; ``BlockRef`` values are built on demand.
"""
from __future__ import annotations

import heapq
from collections.abc import Callable, Sequence
from dataclasses import dataclass

import numpy as np

from tinyvllm._validation import _check_non_negative_int, _check_positive_int
from tinyvllm.prefix_cache import PrefixCache

_NO_IDS = np.zeros(0, dtype=np.int64)


@dataclass(frozen=True, slots=True)
class BlockRef:
    """A physical block at one generation (a reused block gets a new one)."""

    block_id: int
    generation: int

    def __post_init__(self) -> None:
        _check_non_negative_int("block_id", self.block_id)
        _check_non_negative_int("generation", self.generation)


@dataclass(frozen=True, slots=True)
class BlockAppend:
    """One request's KV growth in a step: ``query_len`` tokens written from
    ``token_start``; a new request may first attach cached ``prefix`` blocks."""

    request_id: int
    token_start: int
    query_len: int
    prefix: tuple[BlockRef, ...] = ()

    def __post_init__(self) -> None:
        _check_non_negative_int("request_id", self.request_id)
        _check_non_negative_int("token_start", self.token_start)
        _check_positive_int("query_len", self.query_len)
        object.__setattr__(self, "prefix", tuple(self.prefix))


class BlockPool:
    """Holder counts, generations and reuse order of the physical blocks."""

    def __init__(self, *, num_blocks: int) -> None:
        _check_positive_int("num_blocks", num_blocks)
        self.num_blocks = num_blocks
        self._holders = np.zeros(num_blocks, dtype=np.int32)
        self._gen = np.zeros(num_blocks, dtype=np.int64)
        self._blank: list[int] = list(range(num_blocks - 1, -1, -1))  # pop() -> lowest
        self._idle_stamp = np.zeros(num_blocks, dtype=np.int64)  # 0: not idle
        self._idle_heap: list[tuple[int, int]] = []  # (stamp, block)
        self._idle_count = 0
        self._tick = 0
        self._digest_of: dict[int, bytes] = {}
        self._block_of: dict[bytes, int] = {}
        self.evictions = 0

    # -- views

    @property
    def free_block_count(self) -> int:
        """Blocks an allocation may take now (blank plus idle cached)."""
        return len(self._blank) + self._idle_count

    @property
    def cached_block_count(self) -> int:
        return len(self._block_of)

    def ref(self, block: int) -> BlockRef:
        return BlockRef(int(block), int(self._gen[block]))

    def current(self, ref: BlockRef) -> bool:
        """The ref names its block's present generation."""
        return (isinstance(ref, BlockRef) and ref.block_id < self.num_blocks
                and int(self._gen[ref.block_id]) == ref.generation)

    def held(self, ref: BlockRef) -> int:
        self._expect_current(ref)
        return int(self._holders[ref.block_id])

    def is_idle(self, ref: BlockRef) -> bool:
        """Cached contents with no holder: taking it shrinks the free count."""
        self._expect_current(ref)
        return bool(self._idle_stamp[ref.block_id])

    # -- allocation

    def allocate(self, count: int) -> list[int] | None:
        """``count`` blocks for new contents (blank first, then the oldest idle
        ones, whose digests are dropped), each with one holder; None if the
        pool is short (nothing taken)."""
        _check_positive_int("count", count)
        if count > self.free_block_count:
            return None
        out = []
        while len(out) < count:
            block = self._blank.pop() if self._blank else self._evict_oldest()
            self._gen[block] += 1
            self._holders[block] = 1
            out.append(block)
        return out

    def unallocate(self, blocks: Sequence[int]) -> None:
        """Return blocks taken by ``allocate`` and never used (their
        generation stays advanced, so refs to the old contents stay stale)."""
        for block in reversed(blocks):
            if self._holders[block] != 1:
                raise RuntimeError(f"block {block} is not exclusively allocated")
            self._holders[block] = 0
            self._blank.append(int(block))

    def _evict_oldest(self) -> int:
        while True:
            stamp, block = heapq.heappop(self._idle_heap)
            if self._idle_stamp[block] == stamp:
                break
        self._idle_stamp[block] = 0
        self._idle_count -= 1
        del self._block_of[self._digest_of.pop(block)]
        self.evictions += 1
        return block

    # -- holders

    def hold(self, ref: BlockRef) -> None:
        """One more holder of a block with valid contents."""
        self._expect_current(ref)
        block = ref.block_id
        if self._idle_stamp[block]:
            self._idle_stamp[block] = 0  # its heap entry goes stale
            self._idle_count -= 1
        elif not self._holders[block]:
            raise RuntimeError(f"block {block} has no contents to share")
        self._holders[block] += 1

    def drop(self, ref: BlockRef) -> None:
        """One holder fewer; an unheld block becomes idle (digest kept) or blank."""
        self._expect_current(ref)
        block = ref.block_id
        if self._holders[block] <= 0:
            raise RuntimeError(f"block {block} has no holder to drop")
        self._holders[block] -= 1
        if self._holders[block]:
            return
        if block in self._digest_of:
            self._tick += 1
            self._idle_stamp[block] = self._tick
            heapq.heappush(self._idle_heap, (self._tick, block))
            self._idle_count += 1
        else:
            self._blank.append(block)

    # -- prefix digests

    def find(self, digest: bytes) -> BlockRef | None:
        block = self._block_of.get(digest)
        return None if block is None else self.ref(block)

    def label(self, digest: bytes, ref: BlockRef) -> BlockRef:
        """Index a held block's contents under ``digest``; if another block
        already holds those contents, that block is returned instead."""
        if self.held(ref) == 0:
            raise RuntimeError("only a held, written block can be indexed")
        other = self._block_of.get(digest)
        if other is not None:
            return self.ref(other)
        if ref.block_id in self._digest_of:
            raise RuntimeError(f"block {ref.block_id} is already indexed under another prefix")
        self._block_of[digest] = ref.block_id
        self._digest_of[ref.block_id] = digest
        return ref

    def forget_digests(self) -> None:
        """Drop every digest: idle blocks become blank."""
        for block in self._digest_of:
            if self._idle_stamp[block]:
                self._idle_stamp[block] = 0
                self._blank.append(block)
        self._idle_heap.clear()
        self._idle_count = 0
        self._digest_of.clear()
        self._block_of.clear()
        self.evictions = 0

    def _expect_current(self, ref: BlockRef) -> None:
        if not self.current(ref):
            raise RuntimeError(f"stale or foreign block reference {ref}")


class StepKV:
    """One step's KV journal and the batch builder's view of it (plan id,
    request order, block size, per-request table ids and write slots)."""

    STAGED, LIVE, DONE, UNDONE, FAILED = "staged", "live", "done", "undone", "failed"

    __slots__ = ("plan_id", "request_ids", "phase", "_mgr", "_fresh", "_pins", "_rows",
                 "_epochs")

    def __init__(self, plan_id: int, manager: "BlockManager") -> None:
        self.plan_id = plan_id
        self.phase = StepKV.STAGED
        self._mgr = manager
        self._fresh: list[int] = []                 # allocated by this step
        self._pins: dict[int, tuple[BlockRef, ...]] = {}   # prefix hits held
        # request -> (table ids, table generations, write slots, KV end)
        self._rows: dict[int, tuple[np.ndarray, np.ndarray, np.ndarray, int]] = {}
        self._epochs: dict[int, int] = {}  # table epoch of each request
        self.request_ids: tuple[int, ...] = ()

    @property
    def block_size(self) -> int:
        return self._mgr.block_size

    @property
    def num_blocks(self) -> int:
        return self._mgr.pool.num_blocks

    def append_metadata(self, request_id: int, token_start: int,
                        query_len: int) -> tuple[np.ndarray, np.ndarray]:
        """(table block ids, write slots) of one request as int64 arrays."""
        if self.phase not in (StepKV.STAGED, StepKV.LIVE):
            raise RuntimeError(f"KV step {self.plan_id} is {self.phase}")
        row = self._rows.get(request_id)
        if row is None or row[3] != token_start + query_len or len(row[2]) != query_len:
            raise ValueError(f"request {request_id} has no KV append "
                             f"[{token_start}, {token_start + query_len}) in this step")
        return row[0], row[2]

    def table_epoch(self, request_id: int) -> int:
        """Changes whenever an entry of the request's table other than an
        appended one may differ from an earlier step's (a new table, or a
        prefix-cache swap): a reader holding a copy from the same epoch only
        needs the appended entries."""
        return self._epochs[request_id]

    # -- transitions

    def go_live(self) -> None:
        """The staged tables become the requests' tables (at dispatch)."""
        self._expect(StepKV.STAGED)
        tables = self._mgr._tables
        for rid, (ids, gens, _, _) in self._rows.items():
            tables[rid] = (ids, gens)
        self._mgr._epoch.update(self._epochs)
        self.phase = StepKV.LIVE

    def writes_done(self) -> None:
        """The step's K/V are written: valid lengths advance, hits count."""
        self._expect(StepKV.LIVE)
        valid = self._mgr._valid
        for rid, row in self._rows.items():
            valid[rid] = row[3]
        self._mgr.prefix_cache.note_hits(self._pins)
        self.phase = StepKV.DONE
        self._mgr._open = None

    def undo(self) -> None:
        """Reverse a staged (not dispatched) step."""
        self._expect(StepKV.STAGED)
        self._revert()
        self.phase = StepKV.UNDONE
        self._mgr._open = None

    def _revert(self) -> None:
        pool = self._mgr.pool
        pool.unallocate(self._fresh)
        for refs in self._pins.values():
            for ref in refs:
                pool.drop(ref)
        self._fresh, self._pins = [], {}

    def _expect(self, phase: str) -> None:
        if self._mgr._open is not self or self.phase != phase:
            raise RuntimeError(f"KV step {self.plan_id} is {self.phase}, expected {phase}")


class BlockManager:
    """Request block tables over one BlockPool, grown one StepKV at a time."""

    def __init__(self, *, block_size: int, num_blocks: int,
                 enable_prefix_caching: bool = True) -> None:
        _check_positive_int("block_size", block_size)
        if type(enable_prefix_caching) is not bool:
            raise TypeError("enable_prefix_caching must be bool")
        self.block_size = block_size
        self.pool = BlockPool(num_blocks=num_blocks)
        self.prefix_cache = PrefixCache(block_size=block_size, pool=self.pool,
                                        enabled=enable_prefix_caching)
        self._tables: dict[int, tuple[np.ndarray, np.ndarray]] = {}  # ids, generations
        self._valid: dict[int, int] = {}
        self._epoch: dict[int, int] = {}   # table epochs (see StepKV.table_epoch)
        self._epochs_issued = 0
        self._open: StepKV | None = None

    # -- views

    @property
    def free_block_count(self) -> int:
        return self.pool.free_block_count

    def table_length(self, request_id: int) -> int:
        entry = self._tables.get(request_id)
        return 0 if entry is None else len(entry[0])

    def block_table(self, request_id: int) -> tuple[BlockRef, ...]:
        entry = self._tables.get(request_id)
        if entry is None:
            return ()
        return tuple(BlockRef(int(b), int(g)) for b, g in zip(*entry))

    def valid_token_count(self, request_id: int) -> int:
        return self._valid.get(request_id, 0)

    def blocks_for(self, tokens: int) -> int:
        return -(-tokens // self.block_size)

    # -- one step

    def stage(self, plan_id: int, appends: Sequence[BlockAppend]) -> StepKV | None:
        """Journal a step's appends; None (pool untouched) if blocks run out."""
        _check_non_negative_int("plan_id", plan_id)
        if self._open is not None:
            raise RuntimeError(f"KV step {self._open.plan_id} is still open")
        appends = tuple(appends)
        if not appends:
            raise ValueError("a KV step needs at least one append")
        if len({a.request_id for a in appends}) != len(appends):
            raise ValueError("a request may append only once per step")
        bases = [self._base_of(a) for a in appends]
        wanted = [self.blocks_for(a.token_start + a.query_len) - len(b[0])
                  for a, b in zip(appends, bases)]
        step = StepKV(plan_id, self)
        pool = self.pool
        for append in appends:  # pin hits before allocating, so none is evicted
            if append.prefix:
                for ref in append.prefix:
                    pool.hold(ref)
                step._pins[append.request_id] = append.prefix
        total = sum(wanted)
        fresh = pool.allocate(total) if total else []
        if fresh is None:
            step._revert()
            return None
        step._fresh = fresh
        bs, cursor = self.block_size, 0
        for append, (ids, gens), need in zip(appends, bases, wanted):
            new = np.asarray(fresh[cursor:cursor + need], dtype=np.int64)
            cursor += need
            if need:
                ids = np.concatenate((ids, new))
                gens = np.concatenate((gens, pool._gen[new]))
            end = append.token_start + append.query_len
            pos = np.arange(append.token_start, end, dtype=np.int64)
            step._rows[append.request_id] = (ids, gens, ids[pos // bs] * bs + pos % bs, end)
            epoch = self._epoch.get(append.request_id)
            step._epochs[append.request_id] = self._new_epoch() if epoch is None else epoch
        step.request_ids = tuple(a.request_id for a in appends)
        self._open = step
        return step

    def _new_epoch(self) -> int:
        self._epochs_issued += 1
        return self._epochs_issued

    def _base_of(self, append: BlockAppend) -> tuple[np.ndarray, np.ndarray]:
        """The table an append grows, checked against its start position."""
        if not isinstance(append, BlockAppend):
            raise TypeError("appends must be BlockAppend values")
        rid = append.request_id
        if append.prefix:
            if rid in self._tables:
                raise ValueError(f"request {rid} already owns blocks; prefix not attachable")
            self.prefix_cache.check_hit(rid, append.prefix)
            have = len(append.prefix) * self.block_size
            base = (np.fromiter((r.block_id for r in append.prefix), np.int64),
                    np.fromiter((r.generation for r in append.prefix), np.int64))
        else:
            have = self._valid.get(rid, 0)
            base = self._tables.get(rid, (_NO_IDS, _NO_IDS))
        if append.token_start != have:
            raise ValueError(f"request {rid}: append starts at {append.token_start}, "
                             f"KV holds {have} tokens")
        if self.blocks_for(append.token_start + append.query_len) < len(base[0]):
            raise RuntimeError(f"request {rid}: table longer than its KV")
        return base

    # -- per request

    def publish_blocks(self, request_id: int,
                       token_slice: Callable[[int, int], Sequence[int]],
                       known_tokens: int) -> None:
        """Index the request's newly full blocks whose token ids are known
        (``known_tokens``); a block whose contents another block already
        holds is swapped for that block."""
        if self._open is not None:
            raise RuntimeError("prefix blocks are published between steps")
        entry = self._tables.get(request_id)
        if entry is None:
            return
        full = min(self._valid.get(request_id, 0), known_tokens)
        swaps = self.prefix_cache.index_blocks(request_id, entry, full, token_slice)
        if not swaps:
            return
        ids, gens = entry[0].copy(), entry[1].copy()
        for index, canonical in swaps:
            self.pool.hold(canonical)
            self.pool.drop(BlockRef(int(ids[index]), int(gens[index])))
            ids[index], gens[index] = canonical.block_id, canonical.generation
        self._tables[request_id] = (ids, gens)
        self._epoch[request_id] = self._new_epoch()

    def release_request(self, request_id: int) -> None:
        if self._open is not None:
            raise RuntimeError("requests are released between steps")
        entry = self._tables.pop(request_id, None)
        self._valid.pop(request_id, None)
        self._epoch.pop(request_id, None)
        self.prefix_cache.drop_request(request_id)
        if entry is not None:
            for block, gen in zip(entry[0][::-1], entry[1][::-1]):
                self.pool.drop(BlockRef(int(block), int(gen)))

    def reset_prefix_cache(self) -> None:
        if self._open is not None or self._tables:
            raise RuntimeError("the prefix cache resets only with no request holding KV")
        self.prefix_cache.reset()

    def teardown(self) -> None:
        """Fail-stop: undo or abandon the open step, release every table and
        forget every cached prefix (partly written KV is never reused)."""
        step, self._open = self._open, None
        if step is not None:
            if step.phase == StepKV.STAGED:
                step._revert()
            step.phase = StepKV.FAILED
        for request_id in tuple(self._tables):
            self.release_request(request_id)
        self._valid.clear()
        self.prefix_cache.reset()
