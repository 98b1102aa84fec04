"""Memory tier parity: the reference's own unit-test expectations
(src/memory/{allocator,prefix_cache,kv_cache_manager}.rs #[cfg(test)] modules) run against
both the Python restatement (oracle/memory.py) and the product's C++ manager through the C
ABI, plus a seeded differential run of random admit/publish/fork/COW/append/release
sequences in which every block id, refcount and counter must agree exactly. Host-only: the
C++ manager moves no data when no device context is given."""
import numpy as np
import pytest

from oracle import memory as om
import pia


class PyMgr:
    def __init__(self, total, bs, prefix_cache=True):
        self.m = om.KvCacheManager(total, bs, prefix_cache)
        self.kv = None

    def admit(self, seq, tokens, tick):
        a = self.m.admit(seq, list(tokens), tick)
        if a is None:
            return None
        return a.table, (a.cached_tokens, a.reused_blocks, a.allocated_blocks)

    def blocks(self, t):
        return t.blocks()

    def publish(self, t):
        return self.m.publish_prompt_blocks(t)

    def fork(self, t, child, tick):
        return self.m.fork(t, child, tick)

    def ensure_writable(self, seq, t, pos):
        return self.m.ensure_writable(seq, t, pos, lambda s, d: None)

    def append_block(self, seq, t, tick):
        return self.m.append_block(seq, t, tick)

    def release(self, seq):
        self.m.release_sequence(seq)

    def available(self):
        return self.m.available()

    def stats(self):
        c = self.m.cache
        return dict(hits=c.hits, misses=c.misses, inserts=c.inserts, evictions=c.evictions,
                    tokens_saved=c.tokens_saved, cow_copies=self.m.cow_copies, available_blocks=self.m.available(),
                    active_sequences=len(self.m.sequences), cached_entries=len(c))

    def ref_count(self, b):
        return self.m.alloc.ref_count(b)

    def clear_cache(self):
        self.m.cache.clear(self.m.alloc)


class CppMgr:
    def __init__(self, total, bs, prefix_cache=True):
        self.m = pia.KvCacheManager(total, bs, prefix_cache)

    def admit(self, seq, tokens, tick):
        return self.m.admit(seq, tokens, tick)

    def blocks(self, t):
        return t.blocks()

    def publish(self, t):
        return self.m.publish(t)

    def fork(self, t, child, tick):
        return self.m.fork(t, child, tick)

    def ensure_writable(self, seq, t, pos):
        return self.m.ensure_writable(seq, t, pos)

    def append_block(self, seq, t, tick):
        return self.m.append_block(seq, t, tick)

    def release(self, seq):
        self.m.release(seq)

    def available(self):
        return self.m.stats()["available_blocks"]

    def stats(self):
        s = self.m.stats()
        return {k: s[k] for k in ("hits", "misses", "inserts", "evictions", "tokens_saved", "cow_copies",
                                  "available_blocks", "active_sequences", "cached_entries")}

    def ref_count(self, b):
        return self.m.ref_count(b)

    def clear_cache(self):
        # Clearing the cache alone is internal in the reference; release every sequence and
        # clear (KvCacheManager::clear) reaches the same pool state when no sequence is live.
        self.m.clear()


IMPLS = [PyMgr, CppMgr]
BS = 4


def prompt(prefix, suffix):
    return list(prefix) + list(suffix)


@pytest.mark.parametrize("Impl", IMPLS)
def test_block_hash_chain(Impl):
    h = om.block_hash
    toks = [7] * 16
    a = h(h(0, [1, 2, 3]), toks)
    assert a != h(h(0, [1, 2, 4]), toks)
    assert a == h(h(0, [1, 2, 3]), toks)
    assert h(0, [1, 2]) != h(0, [2, 1]) and h(0, [1, 2]) != h(0, [1, 2, 0])
    rng = np.random.default_rng(0)
    for n in [0, 1, 4, 16]:
        t = rng.integers(0, 2 ** 32, n, dtype=np.uint64).tolist()
        p = int(rng.integers(0, 2 ** 63))
        assert pia.block_hash(p, t) == h(p, t)
    # FNV-1a offset basis/prime known answer: empty block from ROOT hashes the basis then
    # folds length 0: (0xcbf29ce484222325 ^ 0) * prime mod 2^64.
    assert h(0, []) == (0xCBF29CE484222325 * 0x100000001B3) % 2 ** 64


@pytest.mark.parametrize("Impl", IMPLS)
def test_second_request_reuses_the_shared_prefix(Impl):
    m = Impl(32, BS)
    shared = list(range(12))
    ta, a = m.admit(1, prompt(shared, [90, 91]), 1)
    assert a[1] == 0 and a[0] == 0
    m.publish(ta)
    tb, b = m.admit(2, prompt(shared, [80, 81]), 2)
    assert b[1] == 3 and b[0] == 12 and b[2] == 1
    assert m.blocks(ta)[:3] == m.blocks(tb)[:3]
    assert m.stats()["tokens_saved"] == 12


@pytest.mark.parametrize("Impl", IMPLS)
def test_reuse_stops_at_the_first_divergent_block(Impl):
    m = Impl(32, BS)
    ta, _ = m.admit(1, list(range(12)), 1)
    m.publish(ta)
    tb, b = m.admit(2, [0, 1, 2, 3, 40, 41, 42, 43, 8, 9, 10, 11], 2)
    assert b[1] == 1
    assert m.blocks(ta)[2] != m.blocks(tb)[2]


@pytest.mark.parametrize("Impl", IMPLS)
def test_disabling_the_cache_removes_all_reuse(Impl):
    m = Impl(32, BS, prefix_cache=False)
    ta, _ = m.admit(1, list(range(12)), 1)
    assert m.publish(ta) == 0
    _, b = m.admit(2, list(range(12)), 2)
    assert b[1] == 0 and b[2] == 3


@pytest.mark.parametrize("Impl", IMPLS)
def test_cached_blocks_survive_their_producer(Impl):
    m = Impl(8, BS)
    ta, _ = m.admit(1, list(range(8)), 1)
    m.publish(ta)
    m.release(1)
    assert m.available() == 6
    _, b = m.admit(2, list(range(8)), 2)
    assert b[1] == 2


@pytest.mark.parametrize("Impl", IMPLS)
def test_admission_under_pressure_evicts_cache_before_failing(Impl):
    m = Impl(4, BS)
    ta, _ = m.admit(1, list(range(8)), 1)
    m.publish(ta)
    m.release(1)
    assert m.available() == 2
    assert m.admit(2, list(range(90, 106)), 2) is not None
    assert m.stats()["evictions"] >= 2


@pytest.mark.parametrize("Impl", IMPLS)
def test_rejected_admission_leaves_no_references_behind(Impl):
    m = Impl(4, BS)
    ta, _ = m.admit(1, list(range(8)), 1)
    m.publish(ta)
    before = m.available()
    assert m.admit(2, list(range(8)) + list(range(200, 240)), 2) is None
    assert m.available() == before
    _, c = m.admit(3, list(range(8)), 3)
    assert c[1] == 2


@pytest.mark.parametrize("Impl", IMPLS)
def test_fork_shares_blocks_and_copies_on_write(Impl):
    m = Impl(8, BS)
    tp, _ = m.admit(1, [1, 2, 3, 4, 5, 6], 1)
    assert len(m.blocks(tp)) == 2
    before = m.available()
    tc = m.fork(tp, 2, 2)
    assert m.available() == before
    assert m.blocks(tc)[1] == m.blocks(tp)[1]
    assert m.ensure_writable(2, tc, 6)
    assert m.blocks(tc)[1] != m.blocks(tp)[1]
    assert m.stats()["cow_copies"] == 1
    assert m.blocks(tc)[0] == m.blocks(tp)[0]
    assert not m.ensure_writable(2, tc, 6)
    assert m.stats()["cow_copies"] == 1


@pytest.mark.parametrize("Impl", IMPLS)
def test_unshared_block_is_never_copied_and_release_after_fork(Impl):
    m = Impl(8, BS)
    t, _ = m.admit(1, [1, 2, 3], 1)
    assert not m.ensure_writable(1, t, 2)
    assert m.stats()["cow_copies"] == 0
    m2 = Impl(8, BS)
    tp, _ = m2.admit(1, [1, 2, 3, 4], 1)
    free_after = m2.available()
    m2.fork(tp, 2, 2)
    m2.release(1)
    assert m2.available() == free_after
    m2.release(2)
    assert m2.available() == 8


@pytest.mark.parametrize("Impl", IMPLS)
def test_churn_returns_every_block(Impl):
    m = Impl(64, BS)
    for r in range(500):
        t, _ = m.admit(r, prompt(range(8), [r * 10 + i for i in range(4)]), r)
        m.publish(t)
        m.release(r)
    assert m.stats()["active_sequences"] == 0
    m.clear_cache()
    assert m.available() == 64


def test_allocator_refcounts_and_asserts():
    a = om.BlockAllocator(4, 16)
    b = a.allocate()
    a.incref(b)
    a.incref(b)
    assert a.ref_count(b) == 3 and a.is_shared(b)
    assert not a.free(b) and not a.free(b) and a.free(b)
    assert a.available() == 4
    with pytest.raises(AssertionError, match="double free"):
        a.free(b)
    with pytest.raises(AssertionError, match="incref on a free block"):
        a.incref(b)
    blocks = [a.allocate() for _ in range(4)]
    assert a.allocate() is None
    a.free(blocks[1])
    assert a.allocate() == blocks[1]


def test_cpp_manager_reports_misuse_as_errors():
    m = pia.KvCacheManager(2, 16)
    assert m.ref_count(0) == 0
    with pytest.raises(pia.PiaError, match="out of range"):
        m.ref_count(5)


def test_differential_random_operations():
    rng = np.random.default_rng(1234)
    for trial in range(20):
        total, bs = int(rng.integers(4, 40)), int(rng.choice([1, 2, 4, 16]))
        cache_on = bool(rng.integers(0, 2))
        py, cc = PyMgr(total, bs, cache_on), CppMgr(total, bs, cache_on)
        tables_py, tables_cc, lens = {}, {}, {}
        next_seq, tick = 0, 0
        vocab = int(rng.integers(2, 6))  # tiny vocab -> many shared prefixes
        for step in range(120):
            tick += 1
            op = rng.integers(0, 6)
            live = sorted(tables_py)
            if op <= 1 or not live:
                n = int(rng.integers(1, 3 * bs + 2))
                toks = rng.integers(0, vocab, n).tolist()
                a, b = py.admit(next_seq, toks, tick), cc.admit(next_seq, toks, tick)
                assert (a is None) == (b is None)
                if a is not None:
                    assert a[1] == b[1] and py.blocks(a[0]) == cc.blocks(b[0])
                    tables_py[next_seq], tables_cc[next_seq], lens[next_seq] = a[0], b[0], n
                    if rng.integers(0, 2):
                        assert py.publish(a[0]) == cc.publish(b[0])
                next_seq += 1
            elif op == 2:
                s = int(rng.choice(live))
                tables_py[next_seq] = py.fork(tables_py[s], next_seq, tick)
                tables_cc[next_seq] = cc.fork(tables_cc[s], next_seq, tick)
                lens[next_seq] = lens[s]
                next_seq += 1
            elif op == 3:
                s = int(rng.choice(live))
                pos = lens[s]
                tp, tc = tables_py[s], tables_cc[s]
                if len(tp) * bs <= pos:
                    assert py.append_block(s, tp, tick) == cc.append_block(s, tc, tick)
                assert py.ensure_writable(s, tp, pos) == cc.ensure_writable(s, tc, pos)
                if len(tp) * bs > pos:
                    lens[s] += 1
            elif op == 4:
                s = int(rng.choice(live))
                py.release(s)
                cc.release(s)
                del tables_py[s], tables_cc[s], lens[s]
            else:
                s = int(rng.choice(live))
                assert py.publish(tables_py[s]) == cc.publish(tables_cc[s])
            assert py.stats() == cc.stats(), (trial, step)
            for s in tables_py:
                assert py.blocks(tables_py[s]) == cc.blocks(tables_cc[s])
            for blk in range(total):
                assert py.ref_count(blk) == cc.ref_count(blk)


def test_kv_layout_write_matches_dimension_order():
    # layout.rs:17-78 fixes [layer][block][token][kv_head][k|v][head_dim]; a 6-D view of the
    # flat cache in that order must see exactly what write_token stored.
    dims = (3, 5, 4, 2, 6)
    L = om.KvLayout(*dims)
    cache = np.zeros(L.total_floats(), np.float32)
    view = cache.reshape(dims[0], dims[1], dims[2], dims[3], 2, dims[4])
    t = om.BlockTable()
    for b in (4, 1):
        t.append_block(b)
    rng = np.random.default_rng(0)
    k, v = rng.normal(size=(2, 6)).astype(np.float32), rng.normal(size=(2, 6)).astype(np.float32)
    assert L.write_token(cache, 2, t, 6, k, v)  # logical block 1 -> block 1, offset 2
    assert np.array_equal(view[2, 1, 2, :, 0], k) and np.array_equal(view[2, 1, 2, :, 1], v)
    assert np.count_nonzero(cache) == k.size + v.size
    assert not L.write_token(cache, 0, t, 8, k, v)  # logical block 2 unmapped: nothing written
    assert np.count_nonzero(cache) == k.size + v.size
