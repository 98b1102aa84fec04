"""Pure-Python restatement of Paged-Infer's KV memory manager.

TEST INFRASTRUCTURE ONLY: the parity oracle for the product's C++ memory manager. Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it.

Restates, with the same semantics and the same deterministic block ids:
  BlockAllocator   src/memory/allocator.rs:16-109   (FIFO free list, refcounts)
  BlockTable       src/memory/block_table.rs:27-93   (slots, get_physical_location, remap)
  block_hash       src/memory/prefix_cache.rs:28-40  (chained FNV-1a, length folded in)
  PrefixCache      src/memory/prefix_cache.rs:83-175 (LRU tick, evict only refcount-1)
  KvCacheManager   src/memory/kv_cache_manager.rs:38-403
  KvLayout         src/memory/layout.rs:17-96
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from typing import Optional

MASK64 = (1 << 64) - 1
FNV_PRIME = 0x0000_0100_0000_01B3
FNV_OFFSET = 0xCBF2_9CE4_8422_2325
ROOT_HASH = 0


def block_hash(parent: int, tokens) -> int:
    """prefix_cache.rs:28-40: FNV-1a over the parent hash then each token's LE bytes."""
    h = (parent ^ FNV_OFFSET) & MASK64
    for t in tokens:
        t &= 0xFFFFFFFF
        for shift in (0, 8, 16, 24):
            h ^= (t >> shift) & 0xFF
            h = (h * FNV_PRIME) & MASK64
    h ^= len(tokens)
    return (h * FNV_PRIME) & MASK64


class BlockAllocator:
    """allocator.rs:16-109."""

    def __init__(self, total_blocks: int, block_size: int):
        self.block_size = block_size
        self.total = total_blocks
        self.free_list = deque(range(total_blocks))
        self.rc = [0] * total_blocks

    def allocate(self) -> Optional[int]:
        if not self.free_list:
            return None
        b = self.free_list.popleft()
        assert self.rc[b] == 0
        self.rc[b] = 1
        return b

    def _check(self, b: int):
        assert 0 <= b < self.total, f"physical block index {b} out of range (total {self.total})"

    def incref(self, b: int):
        self._check(b)
        assert self.rc[b] > 0, f"incref on a free block (index {b})"
        self.rc[b] += 1

    def free(self, b: int) -> bool:
        self._check(b)
        assert self.rc[b] > 0, f"double free of block {b}"
        self.rc[b] -= 1
        if self.rc[b] == 0:
            self.free_list.append(b)
            return True
        return False

    def ref_count(self, b: int) -> int:
        self._check(b)
        return self.rc[b]

    def is_shared(self, b: int) -> bool:
        return self.ref_count(b) > 1

    def available(self) -> int:
        return len(self.free_list)


@dataclass
class Slot:
    block: int
    hash: Optional[int] = None
    cached: bool = False


@dataclass
class BlockTable:
    """block_table.rs:27-93."""

    slots: list = field(default_factory=list)

    def append_block(self, b: int):
        self.slots.append(Slot(b))

    def get_physical_location(self, t: int, block_size: int):
        lb, off = divmod(t, block_size)
        if lb < len(self.slots):
            return self.slots[lb].block, off
        return None

    def remap(self, lb: int, b: int):
        s = self.slots[lb]
        s.block, s.cached, s.hash = b, False, None

    def blocks(self):
        return [s.block for s in self.slots]

    def copy(self):
        return BlockTable([Slot(s.block, s.hash, s.cached) for s in self.slots])

    def __len__(self):
        return len(self.slots)


class PrefixCache:
    """prefix_cache.rs:83-175."""

    def __init__(self):
        self.entries = {}  # hash -> [block, last_used]
        self.tick = 0
        self.hits = self.misses = self.inserts = self.evictions = self.tokens_saved = 0

    def lookup(self, h: int) -> Optional[int]:
        self.tick += 1
        e = self.entries.get(h)
        if e is None:
            self.misses += 1
            return None
        e[1] = self.tick
        self.hits += 1
        return e[0]

    def insert(self, h: int, b: int, alloc: BlockAllocator):
        if h in self.entries:
            return
        self.tick += 1
        alloc.incref(b)
        self.entries[h] = [b, self.tick]
        self.inserts += 1

    def evict_lru(self, alloc: BlockAllocator) -> bool:
        cands = [(e[1], h) for h, e in self.entries.items() if alloc.ref_count(e[0]) == 1]
        if not cands:
            return False
        _, h = min(cands)
        b, _ = self.entries.pop(h)
        alloc.free(b)
        self.evictions += 1
        return True

    def evict_until_available(self, alloc: BlockAllocator, wanted: int) -> bool:
        while alloc.available() < wanted:
            if not self.evict_lru(alloc):
                return False
        return True

    def clear(self, alloc: BlockAllocator):
        for b, _ in self.entries.values():
            alloc.free(b)
            self.evictions += 1
        self.entries.clear()

    def __len__(self):
        return len(self.entries)


@dataclass
class Admission:
    table: BlockTable
    cached_tokens: int
    reused_blocks: int
    allocated_blocks: int


class KvLayout:
    """layout.rs:17-96: [layer][block][token][kv_head][k|v][head_dim]."""

    def __init__(self, layers, blocks, block_size, kv_heads, head_dim):
        self.layers, self.blocks, self.block_size = layers, blocks, block_size
        self.kv_heads, self.head_dim = kv_heads, head_dim

    def total_floats(self):
        return self.layers * self.blocks * self.block_size * self.kv_heads * 2 * self.head_dim

    def block_stride(self):
        return self.block_size * self.kv_heads * 2 * self.head_dim

    def index(self, layer, pb, off, h, is_value):
        return ((((layer * self.blocks + pb) * self.block_size + off) * self.kv_heads + h) * 2
                + int(is_value)) * self.head_dim

    def write_token(self, cache, layer, table, pos, k, v):
        """The per-entry KV write of run_layers_batch (model.rs:1093-1107): k/v [kv_heads][head_dim]
        stored at pos through the block table (get_physical_location); unmapped -> no write."""
        loc = table.get_physical_location(pos, self.block_size)
        if loc is None:
            return False
        pb, off = loc
        for h in range(self.kv_heads):
            ki = self.index(layer, pb, off, h, False)
            vi = self.index(layer, pb, off, h, True)
            cache[ki:ki + self.head_dim] = k[h]
            cache[vi:vi + self.head_dim] = v[h]
        return True

    def copy_block(self, cache, src: int, dst: int):
        assert src != dst, "copy_block called with src == dst"
        bs = self.block_stride()
        for layer in range(self.layers):
            s = (layer * self.blocks + src) * bs
            d = (layer * self.blocks + dst) * bs
            cache[d:d + bs] = cache[s:s + bs]


class KvCacheManager:
    """kv_cache_manager.rs:38-403. `copy_block(src, dst)` is the caller-supplied data mover
    for copy-on-write (the reference calls KvLayout::copy_block on its host cache)."""

    def __init__(self, total_blocks: int, block_size: int, prefix_cache: bool = True):
        self.alloc = BlockAllocator(total_blocks, block_size)
        self.sequences = {}  # seq_id -> [blocks, last_used_tick]
        self.cache = PrefixCache()
        self.cache_enabled = prefix_cache
        self.cow_copies = 0

    @property
    def block_size(self):
        return self.alloc.block_size

    def available(self):
        return self.alloc.available()

    def admit(self, seq_id: int, tokens, now: int) -> Optional[Admission]:
        bs = self.block_size
        total_blocks = max(1, -(-len(tokens) // bs))
        full = len(tokens) // bs
        hashes, parent = [], ROOT_HASH
        for b in range(full):
            parent = block_hash(parent, tokens[b * bs:(b + 1) * bs])
            hashes.append(parent)
        table, reused = BlockTable(), 0
        if self.cache_enabled:
            for h in hashes:
                blk = self.cache.lookup(h)
                if blk is None:
                    break
                self.alloc.incref(blk)
                table.slots.append(Slot(blk, h, True))
                reused += 1
        to_alloc = total_blocks - reused
        if self.alloc.available() < to_alloc and not self.cache.evict_until_available(self.alloc, to_alloc):
            for s in table.slots:
                self.alloc.free(s.block)
            return None
        for i in range(reused, total_blocks):
            blk = self.alloc.allocate()
            assert blk is not None
            table.slots.append(Slot(blk, hashes[i] if i < len(hashes) else None, False))
        cached_tokens = reused * bs
        self.cache.tokens_saved += cached_tokens
        self.sequences[seq_id] = [table.blocks(), now]
        return Admission(table, cached_tokens, reused, to_alloc)

    def publish_prompt_blocks(self, table: BlockTable) -> int:
        if not self.cache_enabled:
            return 0
        n = 0
        for s in table.slots:
            if s.hash is not None and not s.cached:
                before = len(self.cache)
                self.cache.insert(s.hash, s.block, self.alloc)
                n += len(self.cache) - before
        return n

    def touch(self, seq_id, now):
        if seq_id in self.sequences:
            self.sequences[seq_id][1] = now

    def append_block(self, seq_id, table: BlockTable, now) -> bool:
        self.touch(seq_id, now)
        if self.alloc.available() == 0 and not self.cache.evict_until_available(self.alloc, 1):
            return False
        blk = self.alloc.allocate()
        if blk is None:
            return False
        table.append_block(blk)
        self.sequences.setdefault(seq_id, [[], now])[0].append(blk)
        return True

    def fork(self, parent: BlockTable, child_seq, now) -> BlockTable:
        child = BlockTable()
        for s in parent.slots:
            self.alloc.incref(s.block)
            child.slots.append(Slot(s.block, s.hash, s.cached))
        self.sequences[child_seq] = [child.blocks(), now]
        return child

    def ensure_writable(self, seq_id, table: BlockTable, pos: int, copy_block) -> bool:
        lb = pos // self.block_size
        if lb >= len(table.slots):
            return False
        old = table.slots[lb].block
        if not self.alloc.is_shared(old):
            return False
        if self.alloc.available() == 0 and not self.cache.evict_until_available(self.alloc, 1):
            return False
        fresh = self.alloc.allocate()
        if fresh is None:
            return False
        copy_block(old, fresh)
        table.remap(lb, fresh)
        self.alloc.free(old)
        seq = self.sequences.get(seq_id)
        if seq is not None:
            blocks = seq[0]
            for i, b in enumerate(blocks):
                if b == old:
                    blocks[i] = fresh
                    break
        self.cow_copies += 1
        return True

    def release_sequence(self, seq_id):
        seq = self.sequences.pop(seq_id, None)
        if seq is not None:
            for b in seq[0]:
                self.alloc.free(b)

    def clear(self):
        for sid in list(self.sequences):
            self.release_sequence(sid)
        self.cache.clear(self.alloc)
        self.cache.hits = self.cache.misses = self.cache.inserts = 0
        self.cache.evictions = self.cache.tokens_saved = 0
        self.cow_copies = 0
