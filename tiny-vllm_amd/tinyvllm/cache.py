"""CPU ownership of KV blocks (reference: tinyvllm/cache.py:15-711).

``BlockPool`` tracks each physical block's state, reference count and
generation; ``BlockManager`` owns per-request block tables and stages one
step's appends as a transaction (``BlockPlanTxn``) whose slot mapping the
runner validates and uploads. The slot of logical position p of a request
is ``table[p // block_size] * block_size + p % block_size`` - the contract
shared with every kernel (``PagedKVCache`` layout).

Free list order: never-cached blocks are handed out first; blocks whose
contents are still indexed by the prefix cache wait at the back, least
recently released first, and are evicted (their key dropped) only when
reused.
"""
from __future__ import annotations

from collections import OrderedDict
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from enum import Enum, auto

import numpy as np

from tinyvllm._validation import _check_non_negative_int, _check_positive_int
from tinyvllm.prefix_cache import PrefixCache


_EMPTY = np.zeros(0, dtype=np.int64)


class BlockState(Enum):
    FREE = auto()
    RESERVED = auto()
    ACTIVE = auto()
    CACHED = auto()   # no owner, contents still indexed by the prefix cache


@dataclass(frozen=True, slots=True)
class BlockRef:
    """Physical block identity; the generation detects reuse."""

    block_id: int
    generation: int

    def __post_init__(self) -> None:
        _check_non_negative_int("block_id", self.block_id)
        _check_non_negative_int("generation", self.generation)


@dataclass(frozen=True, slots=True)
class BlockReservation:
    block_refs: tuple[BlockRef, ...]


@dataclass(frozen=True, slots=True)
class BlockAppend:
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
    """Block states for one serial scheduler (no GPU tensors)."""

    def __init__(self, *, num_blocks: int) -> None:
        _check_positive_int("num_blocks", num_blocks)
        self._state = [BlockState.FREE] * num_blocks
        self._gen = [0] * num_blocks
        self._refs = [0] * num_blocks
        self._idle: OrderedDict[int, None] = OrderedDict.fromkeys(range(num_blocks))
        self._by_key: dict[bytes, BlockRef] = {}
        self._key_of: dict[int, bytes] = {}
        self._reservation: BlockReservation | None = None
        self.evictions = 0

    @property
    def num_blocks(self) -> int:
        return len(self._state)

    @property
    def free_block_count(self) -> int:
        """Blocks a reservation may take (free or idle-cached)."""
        return len(self._idle)

    @property
    def open_reservation_count(self) -> int:
        return int(self._reservation is not None)

    @property
    def cached_block_count(self) -> int:
        return len(self._by_key)

    def snapshot(self):
        """Diagnostic view (allocation order is not a contract)."""
        return tuple(self._idle), tuple(self._gen), tuple(self._state)

    def state(self, ref: BlockRef) -> BlockState:
        if not isinstance(ref, BlockRef):
            raise TypeError("ref must be BlockRef")
        if ref.block_id >= self.num_blocks:
            raise ValueError("block_id is out of range")
        if self._gen[ref.block_id] != ref.generation:
            raise RuntimeError("stale BlockRef generation")
        return self._state[ref.block_id]

    def reserve(self, count: int) -> BlockReservation | None:
        _check_positive_int("count", count)
        if self._reservation is not None:
            raise RuntimeError("a reservation is already open")
        if count > len(self._idle):
            return None
        refs = []
        for _ in range(count):
            block, _ = self._idle.popitem(last=False)
            key = self._key_of.pop(block, None)
            if key is not None:
                del self._by_key[key]
                self.evictions += 1
            self._gen[block] += 1
            self._state[block] = BlockState.RESERVED
            refs.append(BlockRef(block, self._gen[block]))
        self._reservation = BlockReservation(tuple(refs))
        return self._reservation

    def commit(self, reservation: BlockReservation) -> None:
        self._check_reservation(reservation)
        for ref in reservation.block_refs:
            self._state[ref.block_id] = BlockState.ACTIVE
            self._refs[ref.block_id] = 1
        self._reservation = None

    def rollback(self, reservation: BlockReservation) -> None:
        """Return reserved blocks to the front of the free list (generations
        are not rewound, so stale refs stay detectable)."""
        self._check_reservation(reservation)
        for ref in reversed(reservation.block_refs):
            self._state[ref.block_id] = BlockState.FREE
            self._idle[ref.block_id] = None
            self._idle.move_to_end(ref.block_id, last=False)
        self._reservation = None

    def retain(self, ref: BlockRef) -> None:
        state = self.state(ref)
        if state is BlockState.CACHED:
            del self._idle[ref.block_id]
            self._state[ref.block_id] = BlockState.ACTIVE
        elif state is not BlockState.ACTIVE:
            raise RuntimeError("only computed active or cached blocks can be retained")
        self._refs[ref.block_id] += 1

    def release(self, ref: BlockRef) -> None:
        if self.state(ref) is not BlockState.ACTIVE:
            raise RuntimeError("block is not active")
        block = ref.block_id
        self._refs[block] -= 1
        if self._refs[block]:
            return
        self._idle[block] = None
        if block in self._key_of:
            self._state[block] = BlockState.CACHED      # reusable, evict last
        else:
            self._state[block] = BlockState.FREE
            self._idle.move_to_end(block, last=False)   # hand out first

    def lookup(self, key: bytes) -> BlockRef | None:
        return self._by_key.get(key)

    def publish(self, key: bytes, ref: BlockRef) -> BlockRef:
        """Index an active computed block under ``key``; returns the block
        already holding that key, if any."""
        if self.state(ref) is not BlockState.ACTIVE:
            raise RuntimeError("only an active computed block can be cached")
        existing = self._by_key.get(key)
        if existing is not None:
            return existing
        if ref.block_id in self._key_of:
            raise RuntimeError("a cached block cannot change its prefix identity")
        self._by_key[key] = ref
        self._key_of[ref.block_id] = key
        return ref

    def clear_cache(self) -> None:
        if self._reservation is not None:
            raise RuntimeError("cannot clear cache during a reservation")
        for ref in self._by_key.values():
            if self._state[ref.block_id] is BlockState.CACHED:
                self._state[ref.block_id] = BlockState.FREE
        self._by_key.clear()
        self._key_of.clear()
        self.evictions = 0

    def _check_reservation(self, reservation: BlockReservation) -> None:
        if self._reservation is not reservation:
            raise ValueError("reservation is not open in this pool")


class BlockTxnState(Enum):
    PREPARED = auto()
    DISPATCHED = auto()
    COMMITTED = auto()
    ROLLED_BACK = auto()
    FAILED = auto()


class BlockPlanTxn:
    """One step's staged block-table changes and slot mappings."""

    __slots__ = ("_plan_id", "_state", "_manager", "_reservation", "_tables",
                 "_ids", "_slots", "_ends", "_prefixes")

    def __init__(self, *, plan_id, manager, reservation, tables, ids, slots, ends, prefixes):
        self._plan_id = plan_id
        self._state = BlockTxnState.PREPARED
        self._manager = manager
        self._reservation = reservation
        self._tables: dict[int, tuple[BlockRef, ...]] = tables
        self._ids: dict[int, np.ndarray] = ids
        self._slots: dict[int, np.ndarray] = slots
        self._ends: dict[int, int] = ends
        self._prefixes: dict[int, tuple[BlockRef, ...]] = prefixes

    @property
    def state(self) -> BlockTxnState:
        return self._state

    @property
    def plan_id(self) -> int:
        return self._plan_id

    @property
    def request_ids(self) -> tuple[int, ...]:
        self._readable()
        return tuple(self._ends)

    @property
    def block_size(self) -> int:
        return self._manager.block_size

    @property
    def num_blocks(self) -> int:
        return self._manager.pool.num_blocks

    def append_metadata(self, request_id: int, token_start: int,
                        query_len: int) -> tuple[np.ndarray, np.ndarray]:
        """(physical block ids of the request's table, write slots) as int64
        arrays (the reference returns BlockRefs and a slot tuple; ids are
        what every consumer reads, kept as arrays so a step's metadata is
        flattened with memcpys)."""
        self._readable()
        if (request_id not in self._ends
                or self._ends[request_id] != token_start + query_len
                or len(self._slots[request_id]) != query_len):
            raise ValueError("work item does not match its KV append")
        return self._ids[request_id], self._slots[request_id]

    def _readable(self) -> None:
        if self._state not in (BlockTxnState.PREPARED, BlockTxnState.DISPATCHED):
            raise RuntimeError("block transaction metadata is no longer readable")

    def commit_before_dispatch(self) -> None:
        self._manager._commit_before_dispatch(self)

    def complete_writes(self) -> None:
        self._manager._complete_writes(self)

    def rollback(self) -> None:
        self._manager._rollback(self)


class BlockManager:
    """Owns request block tables; stages each step's appends transactionally."""

    def __init__(self, *, block_size: int, num_blocks: int,
                 enable_prefix_caching: bool = True) -> None:
        _check_positive_int("block_size", block_size)
        if type(enable_prefix_caching) is not bool:
            raise TypeError("enable_prefix_caching must be bool")
        self.block_size = block_size
        self.pool = BlockPool(num_blocks=num_blocks)
        self.prefix_cache = PrefixCache(block_size=block_size, pool=self.pool,
                                        enabled=enable_prefix_caching)
        self._tables: dict[int, tuple[BlockRef, ...]] = {}
        self._ids: dict[int, np.ndarray] = {}   # block ids of each table (int64)
        self._valid: dict[int, int] = {}
        self._open: BlockPlanTxn | None = None
        self._last: BlockPlanTxn | None = None

    def block_table(self, request_id: int) -> tuple[BlockRef, ...]:
        return self._tables.get(request_id, ())

    def valid_token_count(self, request_id: int) -> int:
        return self._valid.get(request_id, 0)

    @property
    def free_block_count(self) -> int:
        return self.pool.free_block_count

    def match_prefix(self, request_id: int, token_ids: Sequence[int]) -> tuple[BlockRef, ...]:
        return self.prefix_cache.match(request_id, token_ids)

    def cache_full_blocks(self, request_id: int,
                          token_slice: Callable[[int, int], Sequence[int]],
                          known_tokens: int | None = None) -> None:
        """Publish the request's completed blocks; a block whose contents are
        already cached elsewhere is swapped for the canonical copy.
        ``known_tokens`` caps the publishable prefix (token ids past it are
        still on the device)."""
        if self._open is not None:
            raise RuntimeError("publish prefix blocks only after successful writes")
        table = self._tables[request_id]
        valid = self.valid_token_count(request_id)
        if known_tokens is not None:
            valid = min(valid, known_tokens)
        swaps = self.prefix_cache.publish(request_id, table, valid, token_slice)
        if not swaps:
            return
        updated = list(table)
        ids = self._ids[request_id].copy()
        for index, canonical in swaps:
            self.pool.retain(canonical)
            self.pool.release(table[index])
            updated[index] = canonical
            ids[index] = canonical.block_id
        self._tables[request_id] = tuple(updated)
        self._ids[request_id] = ids

    def reset_prefix_cache(self) -> None:
        if self._open is not None or self._tables:
            raise RuntimeError("reset_prefix_cache requires an idle block manager")
        self.prefix_cache.clear()

    def required_new_blocks(self, append: BlockAppend) -> int:
        """Validate an append; number of blocks it adds to its table."""
        if not isinstance(append, BlockAppend):
            raise TypeError("appends must contain BlockAppend values")
        table = self.block_table(append.request_id)
        if append.prefix:
            if table:
                raise ValueError("prefix attachment requires a matched new request")
            self.prefix_cache.validate_match(append.request_id, append.prefix)
            valid, table = len(append.prefix) * self.block_size, append.prefix
        else:
            valid = self.valid_token_count(append.request_id)
        if append.token_start != valid:
            raise ValueError("token_start does not match valid KV length")
        need = self._blocks_for(append.token_start + append.query_len) - len(table)
        if need < 0:
            raise RuntimeError("block table exceeds valid KV length")
        return need

    def begin_plan(self, *, plan_id: int,
                   appends: tuple[BlockAppend, ...]) -> BlockPlanTxn | None:
        """Stage a step's appends; None (and nothing held) if the pool is short."""
        _check_non_negative_int("plan_id", plan_id)
        if self._open is not None:
            raise RuntimeError("a KV transaction is already open")
        appends = tuple(appends)
        if not appends:
            raise ValueError("KV plan must contain at least one append")
        seen: set[int] = set()
        needs = []
        for append in appends:
            if append.request_id in seen:
                raise ValueError("request appears twice in one KV plan")
            seen.add(append.request_id)
            needs.append(self.required_new_blocks(append))
        prefixes = {a.request_id: a.prefix for a in appends if a.prefix}
        # Pin prefix hits first so the reservation cannot evict them.
        for prefix in prefixes.values():
            for ref in prefix:
                self.pool.retain(ref)
        reservation = None
        total = sum(needs)
        if total:
            reservation = self.pool.reserve(total)
            if reservation is None:
                self._unpin(prefixes)
                return None
        fresh = iter(reservation.block_refs if reservation else ())
        tables, ids, slots, ends = {}, {}, {}, {}
        bs = self.block_size
        for append, need in zip(appends, needs):
            rid = append.request_id
            new = tuple(next(fresh) for _ in range(need))
            if append.prefix:
                base = append.prefix
                base_ids = np.fromiter((r.block_id for r in base), np.int64, len(base))
            else:
                base = self.block_table(rid)
                base_ids = self._ids.get(rid, _EMPTY)
            table = base + new
            table_ids = (np.concatenate((base_ids, np.fromiter(
                (r.block_id for r in new), np.int64, need))) if need else base_ids)
            end = append.token_start + append.query_len
            pos = np.arange(append.token_start, end, dtype=np.int64)
            tables[rid], ids[rid], ends[rid] = table, table_ids, end
            slots[rid] = table_ids[pos // bs] * bs + pos % bs
        self._open = BlockPlanTxn(plan_id=plan_id, manager=self, reservation=reservation,
                                  tables=tables, ids=ids, slots=slots, ends=ends,
                                  prefixes=prefixes)
        self._last = None
        return self._open

    def release_request(self, request_id: int) -> None:
        if self._open is not None:
            raise RuntimeError("cannot release blocks during a KV transaction")
        table = self._tables.pop(request_id, ())
        self._ids.pop(request_id, None)
        self._valid.pop(request_id, None)
        self.prefix_cache.forget_request(request_id)
        for ref in reversed(table):
            self.pool.release(ref)

    def teardown(self, txn: BlockPlanTxn | None = None) -> None:
        """Fail-stop: drop every ownership; partially written KV is never reused."""
        current = self._open or self._last
        if txn is not None and (txn._manager is not self or txn is not current):
            raise ValueError("transaction is not the manager's current step")
        if self._open is not None:
            if self._open.state is BlockTxnState.PREPARED:
                if self._open._reservation is not None:
                    self.pool.rollback(self._open._reservation)
                self._unpin(self._open._prefixes)
            self._open._state = BlockTxnState.FAILED
            self._open = None
        for request_id in tuple(self._tables):
            self.release_request(request_id)
        self.reset_prefix_cache()
        self._last = None
        if txn is not None:
            txn._state = BlockTxnState.FAILED

    # -- transaction transitions

    def _commit_before_dispatch(self, txn: BlockPlanTxn) -> None:
        self._require(txn, BlockTxnState.PREPARED)
        if txn._reservation is not None:
            self.pool.commit(txn._reservation)
        self._tables.update(txn._tables)
        self._ids.update(txn._ids)
        txn._state = BlockTxnState.DISPATCHED

    def _complete_writes(self, txn: BlockPlanTxn) -> None:
        self._require(txn, BlockTxnState.DISPATCHED)
        self._valid.update(txn._ends)
        self.prefix_cache.commit_matches(txn._prefixes)
        txn._state = BlockTxnState.COMMITTED
        self._open = None
        self._last = txn

    def _rollback(self, txn: BlockPlanTxn) -> None:
        self._require(txn, BlockTxnState.PREPARED)
        if txn._reservation is not None:
            self.pool.rollback(txn._reservation)
        self._unpin(txn._prefixes)
        txn._state = BlockTxnState.ROLLED_BACK
        self._open = None

    def _unpin(self, prefixes: dict[int, tuple[BlockRef, ...]]) -> None:
        for prefix in prefixes.values():
            for ref in reversed(prefix):
                self.pool.release(ref)

    def _require(self, txn: BlockPlanTxn, state: BlockTxnState) -> None:
        if self._open is not txn or txn.state is not state:
            raise ValueError("KV transaction is not in the expected state")

    def _blocks_for(self, tokens: int) -> int:
        return -(-tokens // self.block_size)

    def _slot_for_position(self, table: tuple[BlockRef, ...], position: int) -> int:
        """Physical slot of a logical position (reference cache.py:696-711)."""
        block, offset = divmod(position, self.block_size)
        return table[block].block_id * self.block_size + offset
