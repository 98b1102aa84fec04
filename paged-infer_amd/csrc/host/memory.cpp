// Refcounted KV block pool, block tables, content-hashed prefix cache and copy-on-write:
// the memory tier of the reference (src/memory/*.rs), with the same policies and the same
// deterministic physical block ids, so block tables built here match the reference's.
// Block data never leaves the device: copy-on-write moves it with a device kernel.
#include <algorithm>
#include <deque>
#include <optional>
#include <unordered_map>
#include <vector>

#include "../common.h"
#include "../kernels.h"
#include "context.h"

namespace pia {

// BlockAllocator (src/memory/allocator.rs:16-109): FIFO free list, per-block refcounts.
class BlockAllocator {
 public:
  BlockAllocator(int64_t total, int64_t block_size) : block_size_(block_size), rc_(total, 0) {
    for (int64_t i = 0; i < total; ++i) free_.push_back(i);
  }
  std::optional<int64_t> allocate() {
    if (free_.empty()) return std::nullopt;
    const int64_t b = free_.front();
    free_.pop_front();
    rc_[b] = 1;
    return b;
  }
  void incref(int64_t b) {
    check(b);
    PIA_REQUIRE(rc_[b] > 0, "incref on a free block (index " + std::to_string(b) + ")");
    ++rc_[b];
  }
  bool free(int64_t b) {
    check(b);
    PIA_REQUIRE(rc_[b] > 0, "double free of block " + std::to_string(b));
    if (--rc_[b] == 0) {
      free_.push_back(b);
      return true;
    }
    return false;
  }
  uint32_t ref_count(int64_t b) const {
    check(b);
    return rc_[b];
  }
  bool is_shared(int64_t b) const { return ref_count(b) > 1; }
  int64_t available() const { return static_cast<int64_t>(free_.size()); }
  int64_t total() const { return static_cast<int64_t>(rc_.size()); }
  int64_t block_size() const { return block_size_; }

 private:
  void check(int64_t b) const {
    PIA_REQUIRE(b >= 0 && b < total(), "physical block index " + std::to_string(b) + " out of range (total " +
                                           std::to_string(total()) + ")");
  }
  int64_t block_size_;
  std::deque<int64_t> free_;
  std::vector<uint32_t> rc_;
};

struct Slot {
  int64_t block;
  std::optional<uint64_t> hash;
  bool cached;
};

// PrefixCache (src/memory/prefix_cache.rs:83-175).
class PrefixCache {
 public:
  std::optional<int64_t> lookup(uint64_t h) {
    ++tick_;
    auto it = map_.find(h);
    if (it == map_.end()) {
      ++misses;
      return std::nullopt;
    }
    it->second.last_used = tick_;
    ++hits;
    return it->second.block;
  }
  void insert(uint64_t h, int64_t b, BlockAllocator& a) {
    if (map_.count(h)) return;
    ++tick_;
    a.incref(b);
    map_[h] = Entry{b, tick_};
    ++inserts;
  }
  // Least recently used entry whose block nobody else maps (refcount 1). Ticks are unique,
  // so the victim does not depend on hash-map iteration order.
  bool evict_lru(BlockAllocator& a) {
    auto victim = map_.end();
    for (auto it = map_.begin(); it != map_.end(); ++it)
      if (a.ref_count(it->second.block) == 1 && (victim == map_.end() || it->second.last_used < victim->second.last_used))
        victim = it;
    if (victim == map_.end()) return false;
    a.free(victim->second.block);
    map_.erase(victim);
    ++evictions;
    return true;
  }
  bool evict_until_available(BlockAllocator& a, int64_t wanted) {
    while (a.available() < wanted)
      if (!evict_lru(a)) return false;
    return true;
  }
  void clear(BlockAllocator& a) {
    for (auto& kv : map_) {
      a.free(kv.second.block);
      ++evictions;
    }
    map_.clear();
  }
  void reset_stats() { hits = misses = inserts = evictions = tokens_saved = 0; }
  int64_t size() const { return static_cast<int64_t>(map_.size()); }

  uint64_t hits = 0, misses = 0, inserts = 0, evictions = 0, tokens_saved = 0;

 private:
  struct Entry {
    int64_t block;
    uint64_t last_used;
  };
  std::unordered_map<uint64_t, Entry> map_;
  uint64_t tick_ = 0;
};

uint64_t block_hash(uint64_t parent, const uint32_t* tokens, int64_t n) {
  constexpr uint64_t kPrime = 0x00000100000001B3ull;
  uint64_t h = parent ^ 0xcbf29ce484222325ull;
  for (int64_t i = 0; i < n; ++i)
    for (int k = 0; k < 4; ++k) {
      h ^= (tokens[i] >> (8 * k)) & 0xffu;
      h *= kPrime;
    }
  h ^= static_cast<uint64_t>(n);
  return h * kPrime;
}

}  // namespace pia

struct pia_table {
  std::vector<pia::Slot> slots;
};

struct pia_kvm {
  struct SeqAlloc {
    std::vector<int64_t> blocks;
    uint64_t last_used;
  };
  pia_kvm(int64_t total, int64_t bs, bool cache_on) : alloc(total, bs), cache_enabled(cache_on) {}
  pia::BlockAllocator alloc;
  pia::PrefixCache cache;
  bool cache_enabled;
  uint64_t cow_copies = 0;
  std::unordered_map<int64_t, SeqAlloc> seqs;

  void touch(int64_t seq, uint64_t tick) {
    auto it = seqs.find(seq);
    if (it != seqs.end()) it->second.last_used = tick;
  }
  void release(int64_t seq) {
    auto it = seqs.find(seq);
    if (it == seqs.end()) return;
    for (int64_t b : it->second.blocks) alloc.free(b);
    seqs.erase(it);
  }
};

using namespace pia;

extern "C" {

uint64_t pia_block_hash(uint64_t parent, const uint32_t* tokens, int64_t n) {
  return pia::block_hash(parent, tokens, n < 0 ? 0 : n);
}

pia_status pia_kvm_create(int64_t total_blocks, int64_t block_size, int32_t enable_prefix_cache, pia_kvm** out) {
  PIA_API_BEGIN
  PIA_REQUIRE(out, "null output");
  PIA_REQUIRE(total_blocks >= 0 && block_size > 0, "bad pool shape");
  *out = new pia_kvm(total_blocks, block_size, enable_prefix_cache != 0);
  PIA_API_END
}

pia_status pia_kvm_destroy(pia_kvm* m) {
  delete m;
  return PIA_OK;
}

// KvCacheManager::admit (src/memory/kv_cache_manager.rs:116-195).
pia_status pia_kvm_admit(pia_kvm* m, int64_t seq_id, const uint32_t* tokens, int64_t n, uint64_t tick,
                         int32_t* admitted, pia_table** out_table, pia_admission* info) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && admitted && out_table, "null argument");
  PIA_REQUIRE(n >= 0 && (n == 0 || tokens), "bad token array");
  *admitted = 0;
  *out_table = nullptr;
  const int64_t bs = m->alloc.block_size();
  const int64_t total_blocks = std::max<int64_t>(1, (n + bs - 1) / bs);
  const int64_t full = n / bs;
  std::vector<uint64_t> hashes;
  uint64_t parent = 0;
  for (int64_t b = 0; b < full; ++b) {
    parent = block_hash(parent, tokens + b * bs, bs);
    hashes.push_back(parent);
  }
  auto* table = new pia_table;
  int64_t reused = 0;
  if (m->cache_enabled) {
    for (uint64_t h : hashes) {
      auto blk = m->cache.lookup(h);
      if (!blk) break;
      m->alloc.incref(*blk);
      table->slots.push_back(Slot{*blk, h, true});
      ++reused;
    }
  }
  const int64_t to_alloc = total_blocks - reused;
  if (m->alloc.available() < to_alloc && !m->cache.evict_until_available(m->alloc, to_alloc)) {
    for (const auto& s : table->slots) m->alloc.free(s.block);
    delete table;
    return PIA_OK;
  }
  for (int64_t i = reused; i < total_blocks; ++i) {
    auto blk = m->alloc.allocate();
    PIA_REQUIRE(blk.has_value(), "allocator ran dry after capacity check");
    std::optional<uint64_t> h;
    if (i < static_cast<int64_t>(hashes.size())) h = hashes[i];
    table->slots.push_back(Slot{*blk, h, false});
  }
  const int64_t cached_tokens = reused * bs;
  m->cache.tokens_saved += static_cast<uint64_t>(cached_tokens);
  pia_kvm::SeqAlloc sa;
  for (const auto& s : table->slots) sa.blocks.push_back(s.block);
  sa.last_used = tick;
  m->seqs[seq_id] = std::move(sa);
  *admitted = 1;
  *out_table = table;
  if (info) *info = pia_admission{cached_tokens, reused, to_alloc};
  PIA_API_END
}

pia_status pia_kvm_publish(pia_kvm* m, const pia_table* t, int64_t* published) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && t, "null argument");
  int64_t n = 0;
  if (m->cache_enabled)
    for (const auto& s : t->slots)
      if (s.hash && !s.cached) {
        const int64_t before = m->cache.size();
        m->cache.insert(*s.hash, s.block, m->alloc);
        n += m->cache.size() - before;
      }
  if (published) *published = n;
  PIA_API_END
}

pia_status pia_kvm_append_block(pia_kvm* m, int64_t seq_id, pia_table* t, uint64_t tick, int32_t* ok) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && t && ok, "null argument");
  *ok = 0;
  m->touch(seq_id, tick);
  if (m->alloc.available() == 0 && !m->cache.evict_until_available(m->alloc, 1)) return PIA_OK;
  auto blk = m->alloc.allocate();
  if (!blk) return PIA_OK;
  t->slots.push_back(Slot{*blk, std::nullopt, false});
  auto it = m->seqs.find(seq_id);
  if (it == m->seqs.end()) it = m->seqs.emplace(seq_id, pia_kvm::SeqAlloc{{}, tick}).first;
  it->second.blocks.push_back(*blk);
  *ok = 1;
  PIA_API_END
}

pia_status pia_kvm_fork(pia_kvm* m, const pia_table* parent, int64_t child_seq, uint64_t tick, pia_table** out) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && parent && out, "null argument");
  auto* child = new pia_table;
  pia_kvm::SeqAlloc sa;
  sa.last_used = tick;
  for (const auto& s : parent->slots) {
    m->alloc.incref(s.block);
    child->slots.push_back(s);
    sa.blocks.push_back(s.block);
  }
  m->seqs[child_seq] = std::move(sa);
  *out = child;
  PIA_API_END
}

pia_status pia_kvm_ensure_writable(pia_kvm* m, int64_t seq_id, pia_table* t, int64_t token_pos, pia_context* ctx,
                                   float* kv, const pia_kv_layout* layout, int32_t* copied) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && t && copied, "null argument");
  PIA_REQUIRE(token_pos >= 0, "negative position");
  *copied = 0;
  const int64_t lb = token_pos / m->alloc.block_size();
  if (lb >= static_cast<int64_t>(t->slots.size())) return PIA_OK;
  const int64_t old = t->slots[lb].block;
  if (!m->alloc.is_shared(old)) return PIA_OK;
  if (m->alloc.available() == 0 && !m->cache.evict_until_available(m->alloc, 1)) return PIA_OK;
  auto fresh = m->alloc.allocate();
  if (!fresh) return PIA_OK;
  if (ctx && kv) {
    check_layout(layout);
    launch_copy_block(kv, *layout, old, *fresh, ctx->stream);
  }
  Slot& s = t->slots[lb];
  s.block = *fresh;
  s.cached = false;
  s.hash.reset();
  m->alloc.free(old);
  auto it = m->seqs.find(seq_id);
  if (it != m->seqs.end()) {
    auto& bl = it->second.blocks;
    auto f = std::find(bl.begin(), bl.end(), old);
    if (f != bl.end()) *f = *fresh;
  }
  ++m->cow_copies;
  *copied = 1;
  PIA_API_END
}

pia_status pia_kvm_touch(pia_kvm* m, int64_t seq_id, uint64_t tick) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null manager");
  m->touch(seq_id, tick);
  PIA_API_END
}

pia_status pia_kvm_release(pia_kvm* m, int64_t seq_id) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null manager");
  m->release(seq_id);
  PIA_API_END
}

pia_status pia_kvm_clear(pia_kvm* m) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null manager");
  std::vector<int64_t> ids;
  for (auto& kv : m->seqs) ids.push_back(kv.first);
  for (int64_t id : ids) m->release(id);
  m->cache.clear(m->alloc);
  m->cache.reset_stats();
  m->cow_copies = 0;
  PIA_API_END
}

pia_status pia_kvm_stats_get(const pia_kvm* m, pia_kvm_stats* out) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && out, "null argument");
  out->hits = m->cache.hits;
  out->misses = m->cache.misses;
  out->inserts = m->cache.inserts;
  out->evictions = m->cache.evictions;
  out->tokens_saved = m->cache.tokens_saved;
  out->cow_copies = m->cow_copies;
  out->available_blocks = m->alloc.available();
  out->total_blocks = m->alloc.total();
  out->active_sequences = static_cast<int64_t>(m->seqs.size());
  out->cached_entries = m->cache.size();
  PIA_API_END
}

pia_status pia_kvm_ref_count(const pia_kvm* m, int64_t block, int64_t* out) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && out, "null argument");
  *out = m->alloc.ref_count(block);
  PIA_API_END
}

pia_status pia_table_create(pia_table** out) {
  PIA_API_BEGIN
  PIA_REQUIRE(out, "null output");
  *out = new pia_table;
  PIA_API_END
}

pia_status pia_table_destroy(pia_table* t) {
  delete t;
  return PIA_OK;
}

int64_t pia_table_len(const pia_table* t) { return t ? static_cast<int64_t>(t->slots.size()) : 0; }

pia_status pia_table_blocks(const pia_table* t, int32_t* out) {
  PIA_API_BEGIN
  PIA_REQUIRE(t && (t->slots.empty() || out), "null argument");
  for (size_t i = 0; i < t->slots.size(); ++i) out[i] = static_cast<int32_t>(t->slots[i].block);
  PIA_API_END
}

pia_status pia_table_append(pia_table* t, int64_t block) {
  PIA_API_BEGIN
  PIA_REQUIRE(t && block >= 0, "bad argument");
  t->slots.push_back(Slot{block, std::nullopt, false});
  PIA_API_END
}

pia_status pia_table_slot(const pia_table* t, int64_t i, uint64_t* hash, int32_t* has_hash, int32_t* cached) {
  PIA_API_BEGIN
  PIA_REQUIRE(t && i >= 0 && i < static_cast<int64_t>(t->slots.size()), "slot index out of range");
  const Slot& s = t->slots[i];
  if (hash) *hash = s.hash.value_or(0);
  if (has_hash) *has_hash = s.hash.has_value() ? 1 : 0;
  if (cached) *cached = s.cached ? 1 : 0;
  PIA_API_END
}

}  // extern "C"
