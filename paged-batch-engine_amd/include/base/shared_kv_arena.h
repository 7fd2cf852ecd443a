// Shared KV arena client and page group: drop-in for the reference's
// base::SharedKVArenaClient / base::SharedKVPageGroup
// (infMain/include/base/shared_kv_arena.h:14-58).
//
// Layout: a page is [layer0 K][layer0 V] ... [layerN K][layerN V], each plane
// `half` bytes; block ids are byte offsets / half, and page ids are multiples
// of 2*layers. The page group leases Chunks from the arena owner, carves them
// into pages, hands the same page id to every layer, and returns a page only
// after a completion fence recorded at its last retire has passed.
//
// The owner is reached through ChunkOwner. The reference talks to an owner
// process over ZMQ (shared_kv_client.cpp); that control plane is not part of
// this build, so LocalChunkOwner serves leases in-process (the owner process
// of a deployment would wrap it behind its RPC).
#ifndef PBE_INCLUDE_BASE_SHARED_KV_ARENA_H_
#define PBE_INCLUDE_BASE_SHARED_KV_ARENA_H_

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "base/global_chunk_allocator.h"
#include "pbe_handoff.h"

namespace base {

class ChunkOwner {
 public:
  virtual ~ChunkOwner() = default;
  // Throws ChunkAllocationError (quota / fragmented / exhausted) or
  // std::runtime_error, like the owner RPC (shared_kv_owner.cpp:71-79).
  virtual ChunkLease acquire(const std::string& model, const std::string& layout, uint64_t bytes,
                             uint64_t alignment) = 0;
  // The caller guarantees every GPU access to the Chunk has completed.
  virtual void release(const ChunkLease& lease) = 0;
  // Re-attributes live Chunks to `to_model`, all or nothing
  // (GlobalChunkAllocator::transfer). The caller presents the identities the
  // current holder sees; they become stale.
  virtual std::vector<ChunkLease> transfer(const std::vector<ChunkLease>& leases,
                                           const std::string& to_model) = 0;
  virtual uint64_t bytes() const = 0;
  virtual uint64_t epoch() const = 0;
};

// In-process owner: a mutex-serialized GlobalChunkAllocator.
class LocalChunkOwner final : public ChunkOwner {
 public:
  LocalChunkOwner(uint64_t bytes, uint64_t epoch) : allocator_(bytes, epoch) {}
  void register_model(const std::string& model, uint64_t hard_limit);
  ChunkLease acquire(const std::string& model, const std::string& layout, uint64_t bytes,
                     uint64_t alignment) override;
  void release(const ChunkLease& lease) override;
  std::vector<ChunkLease> transfer(const std::vector<ChunkLease>& leases,
                                   const std::string& to_model) override;
  uint64_t bytes() const override { return allocator_.bytes(); }
  uint64_t leased_bytes(const std::string& model) const;
  uint64_t epoch() const override { return allocator_.epoch(); }
  uint64_t free_bytes() const;
  size_t lease_count() const;

 private:
  mutable std::mutex mu_;
  GlobalChunkAllocator allocator_;
};

// One process's mapping of the arena plus its model identity and hard limit.
class SharedKVArenaClient {
 public:
  // `view` is this process's mapping (pbe_arena_get_view of a created or
  // imported arena); its size must equal the owner's arena. device < 0 makes
  // a metadata-only client (no completion fences; for planning and tests).
  SharedKVArenaClient(std::shared_ptr<ChunkOwner> owner, const pbe_arena_view& view,
                      std::string model, uint64_t hard_limit_bytes, int device);
  SharedKVArenaClient(const SharedKVArenaClient&) = delete;
  SharedKVArenaClient& operator=(const SharedKVArenaClient&) = delete;
  // Leases a Chunk and checks the owner's answer (shared_kv_client.cpp:102-111).
  ChunkLease acquire(const std::string& layout, uint64_t bytes, uint64_t alignment);
  void release(const ChunkLease& lease);  // caller has completed every GPU access
  // Takes over Chunks another model holds (zero-copy page takeover) and
  // checks the owner's answer like acquire().
  std::vector<ChunkLease> take_over(const std::vector<ChunkLease>& leases);
  // Base of a single-segment arena (nullptr when segmented: use view()).
  void* data() const;
  const pbe_arena_view& view() const { return view_; }
  uint64_t bytes() const { return view_.bytes; }
  uint64_t epoch() const { return owner_->epoch(); }
  uint64_t hard_limit() const { return hard_limit_; }
  int device() const { return device_; }
  const std::string& model() const { return model_; }

 private:
  std::shared_ptr<ChunkOwner> owner_;
  pbe_arena_view view_;
  std::string model_;
  uint64_t hard_limit_;
  int device_;
};

class SharedKVPageGroup {
 public:
  // half_layer_bytes must be a positive multiple of 256; Chunks are
  // max(target, page) rounded up to whole pages (shared_kv_arena.cpp:53-69).
  // `stream` is the stream every user of the pages runs on: retire() records
  // the completion fence there.
  SharedKVPageGroup(std::shared_ptr<SharedKVArenaClient> arena, int layers,
                    uint64_t half_layer_bytes, uint64_t chunk_target_bytes, void* stream);
  ~SharedKVPageGroup();
  SharedKVPageGroup(const SharedKVPageGroup&) = delete;
  SharedKVPageGroup& operator=(const SharedKVPageGroup&) = delete;

  // Layer 0 takes the lowest free page id (leasing a new Chunk if none is
  // free, falling back to a single-page Chunk on quota/fragmentation) and
  // reserves the same id for layers 1..L-1, which must allocate in order.
  // Returns -1 when the model's limit or the arena is exhausted.
  int allocate(int layer);
  // allocate(layer) up to n times under one lock, appending the ids to *out;
  // returns false at the first -1 (ids already appended stay allocated).
  // No counterpart in the reference: a request's pages for one layer in one
  // call, as KVCacheManager::append_slots takes them.
  bool allocate_many(int layer, int n, std::vector<int32_t>* out);
  // Releases one layer of a page. Retiring layer 0 first rolls back the
  // unconsumed layer reservations. When the last layer retires, a fence is
  // recorded on the stream; the page is reused only after it completes.
  void retire(int layer, int block_id);
  // retire(layer, id) for each id in order, under one lock; the pages whose
  // last layer these were share one fence recorded after all of them (the
  // same stream position as one fence each). An invalid id throws as
  // retire() would, after the ids before it have retired. No counterpart in
  // the reference (one event per page).
  void retire_many(int layer, const std::vector<int32_t>& block_ids);
  int free_blocks(int layer) const;
  int capacity() const;
  uint64_t leased_bytes() const;
  uint64_t arena_bytes() const;
  uint64_t arena_epoch() const;
  int addressable_blocks() const;
  // K / V plane bases of a single-segment arena (shared_kv_arena.cpp:224-229).
  void* key_base(int layer) const;
  void* value_base(int layer) const;
  // This process's address of half-plane `index` (byte offset index * half)
  // in any arena, segmented or not; nullptr past the end.
  void* plane_address(int64_t index) const;
  // Returns completed pages, and Chunks whose pages are all free, to the owner.
  void collect();

  // ---- zero-copy page takeover (no counterpart in the reference: its decode
  // side copies every page, docs/single-gpu-2p1d-2026-10-12.md:34) ----
  //
  // Source side. `ids` are pages of one finished request, active in every
  // layer. A Chunk whose every page is either in `ids` or free moves whole:
  // the group stops using it (its pages leave the group; it is neither
  // allocated from nor returned to the owner) and lists its lease in
  // takeover->chunks. Pages of Chunks still shared with live pages stay here
  // and are listed in takeover->copy_ids: the receiver copies those and this
  // group retires them afterwards as usual. The caller orders the receiver's
  // reads after this group's writes (a fence or signal on `stream`).
  struct PageTakeover {
    uint64_t epoch = 0;
    std::string from_model;
    std::vector<ChunkLease> chunks;  // identities as this group held them
    std::vector<int32_t> page_ids;   // the request's pages, in order
    std::vector<int32_t> moved_ids;  // page_ids inside moved Chunks (page order)
    std::vector<int32_t> copy_ids;   // page_ids the receiver must copy
  };
  void detach_for_takeover(const std::vector<int32_t>& ids, PageTakeover* takeover);
  // Receiver side: asks the owner to re-attribute the Chunks to this group's
  // model (all or nothing; ChunkAllocationError kQuota propagates and nothing
  // changes), then holds them: pages in moved_ids become active in every
  // layer, as if allocated, and the Chunks' other pages become free pages of
  // this group. Returns the number of pages taken over.
  size_t adopt(const PageTakeover& takeover);
  // Source side, when the receiver could not adopt: takes the Chunks back
  // exactly as they were detached.
  void reattach(const PageTakeover& takeover);
  // Source side, once the receiver has adopted: forgets the detached Chunks.
  void finish_takeover(const PageTakeover& takeover);
  uint64_t half_bytes() const;
  uint64_t page_bytes() const;
  int layers() const;
  // GPU of the arena mapping (-1 for a metadata-only group) and the stream
  // every user of the pages runs on.
  int device() const;
  void* stream() const;
  // This process's mapping of the whole arena.
  const pbe_arena_view& arena_view() const;

 private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

}  // namespace base

#endif  // PBE_INCLUDE_BASE_SHARED_KV_ARENA_H_
