// Page group over leased Chunks. Allocation, reservation, retire and collect
// rules follow infMain/source/base/shared_kv_arena.cpp:53-229; completion
// fences are C-ABI events recorded on the group's stream.
#include "base/shared_kv_arena.h"

#include "base/page_index.h"

#include <algorithm>
#include <cstring>
#include <deque>
#include <limits>
#include <set>
#include <stdexcept>
#include <unordered_map>
#include <vector>

namespace base {

// ------------------------------------------------------------ LocalChunkOwner

void LocalChunkOwner::register_model(const std::string& model, uint64_t hard_limit) {
  std::lock_guard<std::mutex> lock(mu_);
  allocator_.register_model(model, hard_limit);
}

ChunkLease LocalChunkOwner::acquire(const std::string& model, const std::string& layout,
                                    uint64_t bytes, uint64_t alignment) {
  std::lock_guard<std::mutex> lock(mu_);
  return allocator_.acquire(model, layout, bytes, alignment);
}

void LocalChunkOwner::release(const ChunkLease& lease) {
  std::lock_guard<std::mutex> lock(mu_);
  allocator_.release(lease);
}

std::vector<ChunkLease> LocalChunkOwner::transfer(const std::vector<ChunkLease>& leases,
                                                  const std::string& to_model) {
  std::lock_guard<std::mutex> lock(mu_);
  return allocator_.transfer(leases, to_model);
}

uint64_t LocalChunkOwner::leased_bytes(const std::string& model) const {
  std::lock_guard<std::mutex> lock(mu_);
  return allocator_.leased_bytes(model);
}

uint64_t LocalChunkOwner::free_bytes() const {
  std::lock_guard<std::mutex> lock(mu_);
  return allocator_.free_bytes();
}

size_t LocalChunkOwner::lease_count() const {
  std::lock_guard<std::mutex> lock(mu_);
  return allocator_.lease_count();
}

// ------------------------------------------------------------ SharedKVArenaClient

SharedKVArenaClient::SharedKVArenaClient(std::shared_ptr<ChunkOwner> owner,
                                         const pbe_arena_view& view, std::string model,
                                         uint64_t hard_limit_bytes, int device)
    : owner_(std::move(owner)), view_(view), model_(std::move(model)),
      hard_limit_(hard_limit_bytes), device_(device) {
  if (!owner_ || model_.empty() || !hard_limit_ || view_.nseg == 0 || view_.nseg > PBE_MAX_SEGMENTS)
    throw std::invalid_argument("invalid shared KV arena client");
  if (view_.bytes != owner_->bytes())
    throw std::runtime_error("shared KV mapping and owner arena sizes differ");
}

void* SharedKVArenaClient::data() const { return view_.nseg == 1 ? view_.base[0] : nullptr; }

ChunkLease SharedKVArenaClient::acquire(const std::string& layout, uint64_t bytes,
                                        uint64_t alignment) {
  ChunkLease lease = owner_->acquire(model_, layout, bytes, alignment);
  if (lease.epoch != owner_->epoch() || !lease.id || !lease.generation || lease.model != model_ ||
      lease.layout != layout || lease.bytes != bytes || lease.offset % alignment ||
      lease.offset > view_.bytes || lease.bytes > view_.bytes - lease.offset)
    throw std::runtime_error("invalid owner chunk descriptor");
  return lease;
}

void SharedKVArenaClient::release(const ChunkLease& lease) { owner_->release(lease); }

std::vector<ChunkLease> SharedKVArenaClient::take_over(const std::vector<ChunkLease>& leases) {
  std::vector<ChunkLease> moved = owner_->transfer(leases, model_);
  if (moved.size() != leases.size()) throw std::runtime_error("invalid owner chunk descriptor");
  for (size_t i = 0; i < moved.size(); ++i) {
    const ChunkLease& m = moved[i];
    const ChunkLease& o = leases[i];
    if (m.epoch != owner_->epoch() || m.id != o.id || m.generation == o.generation || m.model != model_ ||
        m.layout != o.layout || m.offset != o.offset || m.bytes != o.bytes || m.offset > view_.bytes ||
        m.bytes > view_.bytes - m.offset)
      throw std::runtime_error("invalid owner chunk descriptor");
  }
  return moved;
}

// ------------------------------------------------------------ SharedKVPageGroup

struct SharedKVPageGroup::Impl {
  struct Chunk;
  // One flag per layer, stored in the page's Chunk (one allocation per Chunk
  // rather than two per page).
  struct LayerFlags {
    char* data = nullptr;
    size_t n = 0;
    char& operator[](size_t i) { return data[i]; }
    char operator[](size_t i) const { return data[i]; }
    char* begin() { return data; }
    char* end() { return data + n; }
    const char* begin() const { return data; }
    const char* end() const { return data + n; }
    void assign(size_t count, char v) {
      if (count != n) throw std::logic_error("page layer flags have a fixed size");
      std::fill(data, data + n, v);
    }
  };
  struct Page {
    uint64_t offset = 0;
    int32_t id = -1;  // offset / half, fixed when the page is laid out
    LayerFlags active;  // per layer
    int active_layers = 0;
    bool retiring = false;
    // Layer 0's reservation of this page is in the reservation log at
    // sequence `seq`; layer l > 0 still holds it reserved (not yet handed
    // out) while seq >= that layer's cursor.
    bool logged = false;
    uint64_t seq = 0;
    pbe_event* fence = nullptr;
    Chunk* chunk = nullptr;
  };
  struct Chunk {
    ChunkLease lease;
    std::vector<Page> pages;  // fixed size: Page* stay valid
    std::vector<char> flags;  // pages x layers (active)
    size_t free_pages = 0;
    // Sizes the pages and points their layer flags into `flags`.
    void lay_out(size_t n_pages, int layers) {
      pages.resize(n_pages);
      flags.assign(n_pages * static_cast<size_t>(layers), 0);
      for (size_t i = 0; i < n_pages; ++i)
        pages[i].active = {flags.data() + i * layers, static_cast<size_t>(layers)};
    }
  };

  std::shared_ptr<SharedKVArenaClient> arena;
  int layers = 0;
  uint64_t half = 0, page = 0, chunk_bytes = 0;
  void* stream = nullptr;
  std::string layout;
  std::unordered_map<uint64_t, std::unique_ptr<Chunk>> chunks;  // by lease id
  std::unordered_map<uint64_t, std::unique_ptr<Chunk>> detached;  // handed to a receiver
  // The arena's pages by page index (page id / (2 * layers)): few enough to
  // index directly, so lookups, inserts and the lowest free id need no tree
  // or hash nodes.
  struct PageTable {
    std::vector<Page*> slots;
    int stride = 1;
    PageIndex index;
    void init(size_t n, int page_stride) {
      slots.assign(n, nullptr);
      stride = page_stride;
      index = PageIndex(page_stride);
    }
    Page* get(int id) const {
      const int32_t i = index.of(id);
      return i >= 0 && static_cast<size_t>(i) < slots.size() ? slots[static_cast<size_t>(i)] : nullptr;
    }
    Page* at(int id) const {
      Page* p = get(id);
      if (!p) throw std::out_of_range("page id not in the group");
      return p;
    }
    size_t count(int id) const { return get(id) ? 1 : 0; }
    void emplace(int id, Page* p) { slots.at(static_cast<size_t>(id / stride)) = p; }
    void erase(int id) {
      if (get(id)) slots[static_cast<size_t>(id / stride)] = nullptr;
    }
  };
  struct FreeIds {  // a bitmap over page indices, lowest id first
    std::vector<uint64_t> bits;
    size_t n = 0;
    int stride = 1;
    mutable size_t first = 0;  // no set bit below word `first`
    void init(size_t pages, int page_stride) {
      bits.assign((pages + 63) / 64, 0);
      stride = page_stride;
    }
    size_t count(int id) const {
      const size_t i = static_cast<size_t>(id / stride);
      return (bits[i / 64] >> (i % 64)) & 1u;
    }
    void insert(int id) {
      const size_t i = static_cast<size_t>(id / stride);
      const uint64_t b = 1ull << (i % 64);
      if (!(bits.at(i / 64) & b)) bits[i / 64] |= b, ++n;
      first = std::min(first, i / 64);
    }
    void erase(int id) {
      const size_t i = static_cast<size_t>(id / stride);
      const uint64_t b = 1ull << (i % 64);
      if (bits.at(i / 64) & b) bits[i / 64] &= ~b, --n;
    }
    bool empty() const { return n == 0; }
    size_t size() const { return n; }
    int lowest() const {
      for (; first < bits.size(); ++first)
        if (bits[first]) return static_cast<int>((first * 64 + __builtin_ctzll(bits[first])) * stride);
      return -1;
    }
  };
  PageTable pages;
  FreeIds free_ids;
  std::deque<Page*> retiring;
  std::vector<pbe_event*> spare_fences;
  // Pages still holding each recorded fence: pages retired together share one.
  std::unordered_map<pbe_event*, size_t> fence_users;
  // Pages reserved by layer 0, in reservation order. Every later layer takes
  // the same pages in the same order (page-major ids), so one log with a
  // read cursor per layer replaces a queue per layer: layer 0 appends once
  // per page, and layer l hands out log[cursor[l]++]. Entry i has sequence
  // log_base + i; a null entry is a reservation rolled back by layer 0's
  // retire before every layer took it. cancelled_ahead[l] counts the null
  // entries at or after cursor[l].
  std::vector<Page*> log;
  // The same entries' page ids (a bulk copy for a layer with no rolled-back
  // entry ahead of its cursor).
  std::vector<int32_t> log_ids;
  uint64_t log_base = 0;
  std::vector<uint64_t> cursor;
  std::vector<uint64_t> cancelled_ahead;
  uint64_t leased = 0;
  bool failed = false;  // an unacknowledged release can never become reusable
  mutable std::mutex mu;

  int id_of(const Page& p) const { return p.id; }

  uint64_t log_end() const { return log_base + log.size(); }
  // Layer `layer` has not yet been handed this page of layer 0's reservation.
  bool reserved(const Page& p, int layer) const {
    return layer > 0 && p.logged && p.seq >= cursor[layer];
  }
  bool any_reserved(const Page& p) const {
    for (int l = 1; l < layers; ++l)
      if (reserved(p, l)) return true;
    return false;
  }
  size_t pending_count(int layer) const {
    return layer > 0 ? static_cast<size_t>(log_end() - cursor[layer] - cancelled_ahead[layer]) : 0;
  }
  // Next page of layer 0's reservations for a later layer, or null.
  Page* take_reserved(int layer) {
    uint64_t& c = cursor[layer];
    const uint64_t end = log_end();
    while (c < end && log[c - log_base] == nullptr) {
      ++c;
      --cancelled_ahead[layer];
    }
    return c < end ? log[c++ - log_base] : nullptr;
  }
  // Drops the log prefix every later layer has read (amortised: only once it
  // is at least half the log).
  void trim_log() {
    uint64_t low = log_end();
    for (int l = 1; l < layers; ++l) low = std::min(low, cursor[l]);
    const uint64_t dead = low - log_base;
    if (dead == log.size()) {
      log.clear();
      log_ids.clear();
    } else if (dead >= 1024 && 2 * dead >= log.size()) {
      log.erase(log.begin(), log.begin() + static_cast<std::ptrdiff_t>(dead));
      log_ids.erase(log_ids.begin(), log_ids.begin() + static_cast<std::ptrdiff_t>(dead));
    } else {
      return;
    }
    log_base = low;
  }

  // True once the fence recorded at the page's last retire has passed.
  bool fence_done(Page& p) {
    if (!p.fence) return true;
    const int rc = pbe_event_query(p.fence);
    if (rc == PBE_NOT_READY) return false;
    if (rc != PBE_OK) {
      failed = true;
      throw std::runtime_error(std::string("shared KV page fence failed: ") + pbe_last_error());
    }
    // The event is recorded again only once every page that shares it has
    // seen it pass.
    auto users = fence_users.find(p.fence);
    if (users != fence_users.end() && --users->second == 0) {
      fence_users.erase(users);
      spare_fences.push_back(p.fence);
    }
    p.fence = nullptr;
    return true;
  }

  void collect_locked() {
    if (failed) throw std::runtime_error("shared KV page group failed; stop GPU domain");
    // Fences are recorded on one stream in retire order: stop at the first
    // that has not passed.
    while (!retiring.empty()) {
      Page* p = retiring.front();
      if (!fence_done(*p)) break;
      retiring.pop_front();
      p->retiring = false;
      free_ids.insert(id_of(*p));
      Chunk* c = p->chunk;
      if (++c->free_pages < c->pages.size()) continue;
      try {
        arena->release(c->lease);
      } catch (...) {
        failed = true;
        throw;
      }
      for (const Page& q : c->pages) {
        free_ids.erase(id_of(q));
        pages.erase(id_of(q));
      }
      leased -= c->lease.bytes;
      chunks.erase(c->lease.id);
    }
  }

  // allocate() with the mutex held; `collect` first returns pages whose fences
  // have passed.
  int allocate_locked(int layer, bool collect = true);

  int reserve(Page& p) {
    const int id = id_of(p);
    std::fill(p.active.begin(), p.active.end(), 1);
    p.active_layers = layers;
    --p.chunk->free_pages;
    free_ids.erase(id);
    if (layers > 1) {
      p.logged = true;
      p.seq = log_end();
      log.push_back(&p);
      log_ids.push_back(id);
    }
    return id;
  }

  // One fence, recorded on the stream now, for pages whose last layer was
  // retired with no stream work in between; then they start retiring.
  void fence_and_retire(const std::vector<Page*>& done) {
    if (done.empty()) return;
    if (arena->device() >= 0) {  // a metadata-only group runs nothing on a GPU
      pbe_event* ev = nullptr;
      if (!spare_fences.empty()) {
        ev = spare_fences.back();
        spare_fences.pop_back();
      } else if (pbe_event_create(arena->device(), 0, &ev) != PBE_OK) {
        throw std::runtime_error(std::string("shared KV fence creation failed: ") + pbe_last_error());
      }
      if (pbe_event_record(ev, stream) != PBE_OK) {
        pbe_event_destroy(ev);
        throw std::runtime_error(std::string("shared KV fence record failed: ") + pbe_last_error());
      }
      fence_users[ev] = done.size();
      for (Page* p : done) p->fence = ev;
    }
    for (Page* p : done) {
      p->retiring = true;
      retiring.push_back(p);
    }
  }

  // One layer of one page let go; a page whose last layer this was joins `done`.
  void retire_locked(int layer, int id, std::vector<Page*>* done) {
    if (failed) throw std::runtime_error("shared KV page group failed; stop GPU domain");
    Page* found = pages.get(id);
    if (!found) throw std::logic_error("page does not belong to current chunk generation");
    Page& p = *found;
    if (layer < 0 || layer >= layers) throw std::out_of_range("invalid layer");
    if (!p.active[layer] || p.retiring || reserved(p, layer)) throw std::logic_error("double/stale page retire");
    if (layer == 0 && p.logged) {
      // Roll back reservations the later layers never consumed.
      bool cancelled = false;
      for (int l = 1; l < layers; ++l) {
        if (!reserved(p, l)) continue;
        p.active[l] = 0;
        --p.active_layers;
        ++cancelled_ahead[l];
        cancelled = true;
      }
      if (cancelled) {
        log[p.seq - log_base] = nullptr;
        log_ids[p.seq - log_base] = -1;
      }
      p.logged = false;
    }
    p.active[layer] = 0;
    // A page is indivisible across layers: one fence after every layer's use.
    if (--p.active_layers == 0) done->push_back(&p);
  }
};

namespace {
uint64_t round_up(uint64_t bytes, uint64_t alignment) {
  if (bytes > std::numeric_limits<uint64_t>::max() - alignment)
    throw std::invalid_argument("KV size overflow");
  return (bytes + alignment - 1) / alignment * alignment;
}
}  // namespace

SharedKVPageGroup::SharedKVPageGroup(std::shared_ptr<SharedKVArenaClient> arena, int layers,
                                     uint64_t half_bytes, uint64_t target, void* stream)
    : impl_(new Impl) {
  if (!arena || layers <= 0 || !half_bytes || half_bytes % 256 || !target ||
      half_bytes > std::numeric_limits<uint64_t>::max() / (2ull * layers))
    throw std::invalid_argument("unsupported shared KV geometry/alignment");
  impl_->arena = std::move(arena);
  impl_->layers = layers;
  impl_->cursor.assign(layers, 0);
  impl_->cancelled_ahead.assign(layers, 0);
  impl_->half = half_bytes;
  impl_->page = half_bytes * 2 * layers;
  impl_->pages.init(impl_->arena->bytes() / impl_->page + 1, 2 * layers);
  impl_->free_ids.init(impl_->arena->bytes() / impl_->page + 1, 2 * layers);
  impl_->chunk_bytes = round_up(std::max(target, impl_->page), impl_->page);
  impl_->stream = stream;
  impl_->layout = "page-major-gqa-v1:" + std::to_string(layers) + ":" + std::to_string(half_bytes);
  if (capacity() <= 0 || impl_->arena->bytes() / half_bytes > static_cast<uint64_t>(INT32_MAX))
    throw std::invalid_argument("shared KV capacity exceeds block ID range or is zero");
  if (impl_->arena->view().nseg > 1 && impl_->arena->view().segment_bytes % impl_->page)
    throw std::invalid_argument("arena segments must hold whole pages");
}

SharedKVPageGroup::~SharedKVPageGroup() {
  // A failed stream sync must quarantine the leases: never return their bytes.
  if (impl_->arena->device() >= 0 &&
      pbe_stream_synchronize(impl_->arena->device(), impl_->stream) != PBE_OK)
    return;
  for (auto& entry : impl_->fence_users) pbe_event_destroy(entry.first);
  for (auto& entry : impl_->chunks) {
    try {
      impl_->arena->release(entry.second->lease);
    } catch (...) {  // domain shutdown
    }
  }
  for (pbe_event* ev : impl_->spare_fences) pbe_event_destroy(ev);
}

void SharedKVPageGroup::collect() {
  std::lock_guard<std::mutex> lock(impl_->mu);
  impl_->collect_locked();
}

int SharedKVPageGroup::allocate(int layer) {
  std::lock_guard<std::mutex> lock(impl_->mu);
  return impl_->allocate_locked(layer);
}

bool SharedKVPageGroup::allocate_many(int layer, int n, std::vector<int32_t>* out) {
  std::lock_guard<std::mutex> lock(impl_->mu);
  Impl& m = *impl_;
  if (m.failed) throw std::runtime_error("shared KV page group failed; stop GPU domain");
  if (layer < 0 || layer >= m.layers) throw std::invalid_argument("invalid layer");
  if (n <= 0) return true;
  if (layer > 0) {
    // Bulk form of the later layers' allocate: the next n pages of layer 0's
    // reservations, in order.
    if (m.pending_count(layer) < static_cast<size_t>(n))
      throw std::logic_error("Allocate shared pages in layer order");
    const size_t at = out->size();
    out->resize(at + static_cast<size_t>(n));
    int32_t* ids = out->data() + at;
    if (m.cancelled_ahead[layer] == 0) {  // no rolled-back entry ahead: one copy
      uint64_t& c = m.cursor[layer];
      std::memcpy(ids, m.log_ids.data() + (c - m.log_base), static_cast<size_t>(n) * sizeof(int32_t));
      c += static_cast<uint64_t>(n);
    } else {
      for (int k = 0; k < n; ++k) ids[k] = m.take_reserved(layer)->id;
    }
    m.trim_log();
    return true;
  }
  // Layer 0 collects (returns pages whose fences have passed) before it
  // leases a Chunk, as allocate() does. Each collect costs a fence query
  // while pages are retiring, so within one batch a collect that found the
  // oldest fence still pending is not repeated: that fence passes in stream
  // order, not within the microseconds a batch takes.
  m.collect_locked();
  bool fence_pending = !m.retiring.empty();
  for (int k = 0; k < n; ++k) {
    int id = m.allocate_locked(0, false);
    if (id < 0 && fence_pending) {  // out of room: one last look before giving up
      id = m.allocate_locked(0, true);
      fence_pending = !m.retiring.empty();
    }
    if (id < 0) return false;
    out->push_back(id);
  }
  return true;
}

int SharedKVPageGroup::Impl::allocate_locked(int layer, bool collect) {
  Impl& m = *this;
  if (m.failed) throw std::runtime_error("shared KV page group failed; stop GPU domain");
  if (layer < 0 || layer >= m.layers) throw std::invalid_argument("invalid layer");
  if (layer > 0) {
    Page* p = m.take_reserved(layer);
    if (!p) throw std::logic_error("Allocate shared pages in layer order");
    if (layer == m.layers - 1) m.trim_log();
    return m.id_of(*p);
  }
  if (collect) m.collect_locked();
  if (!m.free_ids.empty()) return m.reserve(*m.pages.at(m.free_ids.lowest()));
  const uint64_t room = m.arena->hard_limit() - m.leased;
  if (room < m.page) return -1;
  const uint64_t want = room >= m.chunk_bytes ? m.chunk_bytes : m.page;
  ChunkLease lease;
  // Quota / fragmentation may still fit one page; other owner errors propagate.
  try {
    lease = m.arena->acquire(m.layout, want, m.page);
  } catch (const ChunkAllocationError&) {
    if (want == m.page) return -1;
    try {
      lease = m.arena->acquire(m.layout, m.page, m.page);
    } catch (const ChunkAllocationError&) {
      return -1;
    }
  }
  auto chunk = std::make_unique<Impl::Chunk>();
  chunk->lease = lease;
  chunk->lay_out(lease.bytes / m.page, m.layers);
  for (size_t i = 0; i < chunk->pages.size(); ++i) {
    Impl::Page& p = chunk->pages[i];
    p.offset = lease.offset + i * m.page;
    p.id = static_cast<int32_t>(p.offset / m.half);
    p.chunk = chunk.get();
    m.pages.emplace(m.id_of(p), &p);
    m.free_ids.insert(m.id_of(p));
  }
  chunk->free_pages = chunk->pages.size();
  const int id = m.reserve(chunk->pages.front());
  m.leased += lease.bytes;
  m.chunks.emplace(lease.id, std::move(chunk));
  return id;
}

void SharedKVPageGroup::retire(int layer, int id) { retire_many(layer, {id}); }

void SharedKVPageGroup::retire_many(int layer, const std::vector<int32_t>& ids) {
  std::lock_guard<std::mutex> lock(impl_->mu);
  Impl& m = *impl_;
  std::vector<Impl::Page*> done;
  try {
    for (int32_t id : ids) m.retire_locked(layer, id, &done);
  } catch (...) {
    m.fence_and_retire(done);  // what was let go before the bad id retires as usual
    throw;
  }
  if (done.empty()) return;  // no page finished: nothing new to collect
  m.fence_and_retire(done);
  m.collect_locked();
}

void SharedKVPageGroup::detach_for_takeover(const std::vector<int32_t>& ids, PageTakeover* out) {
  if (out == nullptr) throw std::invalid_argument("takeover output is null");
  std::lock_guard<std::mutex> lock(impl_->mu);
  Impl& m = *impl_;
  if (m.failed) throw std::runtime_error("shared KV page group failed; stop GPU domain");
  *out = PageTakeover{};
  std::unordered_map<int, int> listed;
  std::unordered_map<Impl::Chunk*, size_t> touched;
  for (int32_t id : ids) {
    const Impl::Page* found = m.pages.get(id);
    if (!found) throw std::logic_error("takeover page does not belong to this group");
    const Impl::Page& p = *found;
    if (p.active_layers != m.layers || p.retiring || m.any_reserved(p))
      throw std::logic_error("takeover page is not active in every layer");
    if (listed[id]++) throw std::logic_error("takeover page listed twice");
    ++touched[p.chunk];
  }
  // Decide per Chunk before changing anything.
  std::unordered_map<Impl::Chunk*, bool> movable;
  for (const auto& entry : touched) {
    bool whole = true;
    for (const Impl::Page& q : entry.first->pages) {
      const int qid = m.id_of(q);
      if (!listed.count(qid) && !m.free_ids.count(qid)) {
        whole = false;
        break;
      }
    }
    movable[entry.first] = whole;
  }
  out->epoch = m.arena->epoch();
  out->from_model = m.arena->model();
  out->page_ids = ids;
  for (int32_t id : ids) {
    if (movable[m.pages.at(id)->chunk]) out->moved_ids.push_back(id);
    else out->copy_ids.push_back(id);
  }
  for (const auto& entry : movable) {
    if (!entry.second) continue;
    Impl::Chunk* c = entry.first;
    out->chunks.push_back(c->lease);
    for (const Impl::Page& q : c->pages) {
      m.free_ids.erase(m.id_of(q));
      m.pages.erase(m.id_of(q));
    }
    m.leased -= c->lease.bytes;
    auto node = m.chunks.find(c->lease.id);
    m.detached.emplace(c->lease.id, std::move(node->second));
    m.chunks.erase(node);
  }
  std::sort(out->chunks.begin(), out->chunks.end(),
            [](const ChunkLease& a, const ChunkLease& b) { return a.offset < b.offset; });
}

void SharedKVPageGroup::reattach(const PageTakeover& t) {
  std::lock_guard<std::mutex> lock(impl_->mu);
  Impl& m = *impl_;
  for (const ChunkLease& lease : t.chunks)
    if (!m.detached.count(lease.id) || m.detached.at(lease.id)->lease.generation != lease.generation)
      throw std::logic_error("reattach of a Chunk this group did not detach");
  std::set<int> moved(t.moved_ids.begin(), t.moved_ids.end());
  for (const ChunkLease& lease : t.chunks) {
    auto node = m.detached.find(lease.id);
    Impl::Chunk* c = node->second.get();
    for (Impl::Page& q : c->pages) {
      const int qid = m.id_of(q);
      m.pages.emplace(qid, &q);
      if (!moved.count(qid)) m.free_ids.insert(qid);
    }
    m.leased += c->lease.bytes;
    m.chunks.emplace(lease.id, std::move(node->second));
    m.detached.erase(node);
  }
}

void SharedKVPageGroup::finish_takeover(const PageTakeover& t) {
  std::lock_guard<std::mutex> lock(impl_->mu);
  for (const ChunkLease& lease : t.chunks) impl_->detached.erase(lease.id);
}

size_t SharedKVPageGroup::adopt(const PageTakeover& t) {
  std::lock_guard<std::mutex> lock(impl_->mu);
  Impl& m = *impl_;
  if (m.failed) throw std::runtime_error("shared KV page group failed; stop GPU domain");
  if (t.epoch != m.arena->epoch()) throw std::invalid_argument("PD arena epoch mismatch");
  uint64_t bytes = 0;
  std::set<int> in_chunks;
  for (const ChunkLease& lease : t.chunks) {
    if (lease.layout != m.layout || lease.offset % m.page || !lease.bytes || lease.bytes % m.page)
      throw std::invalid_argument("PD shared layout mismatch");
    for (uint64_t off = lease.offset; off < lease.offset + lease.bytes; off += m.page) {
      const int id = static_cast<int>(off / m.half);
      if (m.pages.count(id)) throw std::logic_error("takeover Chunk overlaps this group's pages");
      in_chunks.insert(id);
    }
    bytes += lease.bytes;
  }
  std::set<int> moved;
  for (int32_t id : t.moved_ids)
    if (!in_chunks.count(id) || !moved.insert(id).second)
      throw std::invalid_argument("takeover page outside its Chunks");
  if (bytes > m.arena->hard_limit() - m.leased) throw ChunkAllocationError(ChunkAllocationFailure::kQuota);
  const std::vector<ChunkLease> held = m.arena->take_over(t.chunks);  // all or nothing
  for (const ChunkLease& lease : held) {
    auto chunk = std::make_unique<Impl::Chunk>();
    chunk->lease = lease;
    chunk->lay_out(lease.bytes / m.page, m.layers);
    chunk->free_pages = 0;
    for (size_t i = 0; i < chunk->pages.size(); ++i) {
      Impl::Page& p = chunk->pages[i];
      p.offset = lease.offset + i * m.page;
      p.id = static_cast<int32_t>(p.offset / m.half);
      p.logged = false;
      p.chunk = chunk.get();
      const int id = m.id_of(p);
      if (moved.count(id)) {
        p.active.assign(m.layers, 1);
        p.active_layers = m.layers;
      } else {
        p.active.assign(m.layers, 0);
        m.free_ids.insert(id);
        ++chunk->free_pages;
      }
      m.pages.emplace(id, &p);
    }
    m.leased += lease.bytes;
    m.chunks.emplace(lease.id, std::move(chunk));
  }
  return moved.size();
}

int SharedKVPageGroup::free_blocks(int layer) const {
  std::lock_guard<std::mutex> lock(impl_->mu);
  uint64_t n = (impl_->arena->hard_limit() - impl_->leased) / impl_->page;
  n += impl_->free_ids.size();
  if (layer < 0 || layer >= impl_->layers) throw std::out_of_range("invalid layer");
  n += impl_->pending_count(layer);
  return static_cast<int>(std::min<uint64_t>(INT32_MAX, n));
}

uint64_t SharedKVPageGroup::leased_bytes() const {
  std::lock_guard<std::mutex> lock(impl_->mu);
  return impl_->leased;
}

uint64_t SharedKVPageGroup::arena_bytes() const { return impl_->arena->bytes(); }
uint64_t SharedKVPageGroup::arena_epoch() const { return impl_->arena->epoch(); }
uint64_t SharedKVPageGroup::half_bytes() const { return impl_->half; }
uint64_t SharedKVPageGroup::page_bytes() const { return impl_->page; }
int SharedKVPageGroup::layers() const { return impl_->layers; }
int SharedKVPageGroup::device() const { return impl_->arena->device(); }
void* SharedKVPageGroup::stream() const { return impl_->stream; }
const pbe_arena_view& SharedKVPageGroup::arena_view() const { return impl_->arena->view(); }

int SharedKVPageGroup::capacity() const {
  return static_cast<int>(std::min<uint64_t>(INT32_MAX, impl_->arena->hard_limit() / impl_->page));
}

int SharedKVPageGroup::addressable_blocks() const {
  // Each layer has its own base; the last V plane must stay inside the mapping.
  return static_cast<int>(impl_->arena->bytes() / impl_->half - 2 * impl_->layers + 1);
}

void* SharedKVPageGroup::key_base(int layer) const {
  void* base = impl_->arena->data();
  return base ? static_cast<char*>(base) + 2ull * layer * impl_->half : nullptr;
}

void* SharedKVPageGroup::plane_address(int64_t index) const {
  const pbe_arena_view& v = impl_->arena->view();
  if (index < 0) return nullptr;
  const uint64_t off = static_cast<uint64_t>(index) * impl_->half;
  if (off / impl_->half != static_cast<uint64_t>(index) || off >= v.bytes) return nullptr;
  const uint64_t seg = off / v.segment_bytes;
  return static_cast<char*>(v.base[seg]) + (off - seg * v.segment_bytes);
}

void* SharedKVPageGroup::value_base(int layer) const {
  void* base = impl_->arena->data();
  return base ? static_cast<char*>(base) + (2ull * layer + 1) * impl_->half : nullptr;
}

}  // namespace base
