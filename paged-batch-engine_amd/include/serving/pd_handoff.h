// Prefill->decode handoff descriptors and the connector interface
// (infMain/include/serving/pd_handoff.h:18-93), plus the MI355X shared-arena
// connector: the data path of copy_shared_kv (split_pd_engine.cpp:49-115)
// as one gfx950 run-list kernel per handoff.
#ifndef PBE_INCLUDE_SERVING_PD_HANDOFF_H_
#define PBE_INCLUDE_SERVING_PD_HANDOFF_H_

#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "base/base.h"
#include "base/shared_kv_arena.h"
#include "base/kv_cache_format.h"
#include "cache/transfer_plan.h"
#include "pbe_handoff.h"

namespace serving {

struct GlobalRequestId {
  std::string value;
  bool empty() const { return value.empty(); }
};

struct HandoffId {
  uint64_t value = 0;
  bool valid() const { return value != 0; }
};

struct KVPoolDescriptor {
  int32_t device_id = 0;
  int32_t layer_num = 0;
  int32_t block_size = 0;
  int32_t kv_head_num = 0;
  int32_t head_size = 0;
  base::DataType dtype = base::DataType::kDataTypeUnknown;
  base::BlockStorageMode storage_mode = base::BlockStorageMode::kPlain;

  // K + V payload (+ scales) of one block of one layer; 0 on bad dims.
  int64_t bytes_per_block_per_layer() const;
  bool compatible_with(const KVPoolDescriptor& other) const;
};

struct KVBlockMapping {
  int32_t layer_idx = 0;
  std::vector<int32_t> src_block_ids;
  std::vector<int32_t> dst_block_ids;
};

struct KVBlockManifest {
  GlobalRequestId client_request_id;
  HandoffId handoff_id;
  int32_t prompt_tokens = 0;
  int32_t computed_tokens = 0;
  int32_t first_token = -1;
  KVPoolDescriptor src_pool;
  KVPoolDescriptor dst_pool;
  std::vector<KVBlockMapping> layer_mappings;

  base::Status validate() const;
};

enum class KVTransferState { kPending, kCompleted, kFailed, kCancelled };

struct KVTransferStatus {
  KVTransferState state = KVTransferState::kPending;
  std::string error;

  static KVTransferStatus Pending();
  static KVTransferStatus Completed();
  static KVTransferStatus Failed(std::string message);
  static KVTransferStatus Cancelled(std::string message);
  bool done() const;
  bool ok() const;
};

class KVTransferConnector {
 public:
  virtual ~KVTransferConnector() = default;
  virtual base::Status submit(const KVBlockManifest& manifest, HandoffId* handle) = 0;
  virtual KVTransferStatus poll(HandoffId handle) = 0;
  virtual void cancel(HandoffId handle, const std::string& reason) = 0;
  virtual KVTransferStatus drain(HandoffId handle) { return poll(handle); }
  virtual void release(HandoffId /*handle*/) {}
};

// This process's mapping of the shared KV arena and the owner epoch it
// belongs to (block id = byte offset / half, page-major layout).
struct SharedArenaBinding {
  pbe_arena_view view{};
  uint64_t epoch = 0;
  int device = 0;
};

// The data path of copy_shared_kv: checks the source epoch against the
// binding (split_pd_engine.cpp:54-55), the layer count, that every id is a
// page id inside the arena (:70-77) and that all layers carry identical
// page-major id lists (:78-79, :91-93), then coalesces runs and launches one
// gfx950 copy on `stream` (asynchronous). *copied = bytes copied. Every check
// happens before any device work, so an error leaves the arena untouched.
base::Status CopySharedKV(const SharedArenaBinding& arena, uint64_t source_epoch,
                          const KVBlockManifest& manifest, void* stream, uint64_t* copied);

// Zero-copy handoff, receiver side (no counterpart in the reference, whose
// decode side copies every page: docs/single-gpu-2p1d-2026-10-12.md:34).
// `takeover` comes from the prefill group's detach_for_takeover(). The decode
// group adopts the moved Chunks (their pages are used in place), allocates
// its own pages for takeover.copy_ids and copies those with one kernel on
// `stream` (CopySharedKV). *block_table = the request's page ids in order,
// moved ids unchanged, copied ids replaced by the new ones; *copied = bytes
// copied. On a refused adoption (receiver quota) nothing changes here and the
// prefill side calls reattach(); the caller may then fall back to a full copy.
base::Status TakeOverSharedKV(base::SharedKVPageGroup* decode_group, const SharedArenaBinding& arena,
                              const base::SharedKVPageGroup::PageTakeover& takeover,
                              const KVPoolDescriptor& pool, void* stream,
                              std::vector<int32_t>* block_table, uint64_t* copied);

// A KV pool laid out page-major in an arena mapping (the shared-arena layout):
// the K plane of layer l of block id b is at byte (2l + b)*half, the V plane
// at (2l + 1 + b)*half. FP8 pools add a page-major scale pool of
// 2*layers*block_size*kv_heads fp32 per page ([layer][K|V][token][head]).
struct ArenaKVPool {
  pbe_arena_view view{};
  KVPoolDescriptor pool;
  void* scales = nullptr;  // FP8 only
  uint64_t scale_bytes = 0;
};

// Generic plan form of a handoff (pd_handoff_common.cpp:64-153): builds the
// source and destination page schemas from the pool descriptors, compiles a
// plan (cached by `planner`), packs both layouts and binds one BoundTransfer
// per page over the component addresses of the manifest's block ids. Fails
// before producing anything on incompatible pools, incomplete or duplicate
// layer mappings, or ids outside either arena.
base::Status BindManifestTransfers(const KVBlockManifest& manifest, const ArenaKVPool& source,
                                   const ArenaKVPool& destination, cache::TransferPlanner* planner,
                                   std::vector<cache::BoundTransfer>* transfers);

// The same binding as a flat list of device copy operations (the concatenated
// operations of BindManifestTransfers' transfers, in order), for
// pbe_copy_ops. No counterpart in the reference: every page of a manifest
// shares its schemas, plan and layouts, so the first page is bound in full
// and the others follow its operations at their own component addresses,
// with the same per-page bounds checks and errors.
base::Status BindManifestCopyOps(const KVBlockManifest& manifest, const ArenaKVPool& source,
                                 const ArenaKVPool& destination, cache::TransferPlanner* planner,
                                 std::vector<pbe_copy_op>* ops);

// The binding of a pool pair and its per-page op template (defined with the
// connector).
struct CopyOpTemplate;

// InProcKVBlockCopyConnector (pd_handoff.cpp:80-213) over arena pools: each
// handoff is bound through the TransferPlan and all of its component copies
// (2*layers per page, plus scales for FP8 pools) run as one op-list kernel on
// the connector's stream, followed by a completion event.
class InProcKVBlockCopyConnector final : public KVTransferConnector {
 public:
  InProcKVBlockCopyConnector(ArenaKVPool source, ArenaKVPool destination, int device,
                             void* stream = nullptr);
  ~InProcKVBlockCopyConnector() override;
  InProcKVBlockCopyConnector(const InProcKVBlockCopyConnector&) = delete;
  InProcKVBlockCopyConnector& operator=(const InProcKVBlockCopyConnector&) = delete;

  base::Status submit(const KVBlockManifest& manifest, HandoffId* handle) override;
  KVTransferStatus poll(HandoffId handle) override;
  void cancel(HandoffId handle, const std::string& reason) override;
  KVTransferStatus drain(HandoffId handle) override;
  void release(HandoffId handle) override;
  uint64_t copied_bytes() const { return copied_bytes_; }
  size_t last_op_count() const { return last_ops_; }

 private:
  struct Record {
    HandoffId handle;
    KVTransferStatus status;
    pbe_event* done = nullptr;
    bool cancel_requested = false;
    std::string cancel_reason;
  };
  Record* find(HandoffId handle);
  KVTransferStatus settle(Record& record, bool wait);

  ArenaKVPool source_, destination_;
  int device_;
  void* stream_ = nullptr;
  bool owns_stream_ = false;
  cache::TransferPlanner planner_;
  std::shared_ptr<const CopyOpTemplate> template_;
  uint64_t next_handoff_id_ = 1;
  uint64_t copied_bytes_ = 0;
  size_t last_ops_ = 0;
  std::vector<Record> records_;
};

// KVTransferConnector over CopySharedKV: submit() queues the copy on the
// connector's stream and records a completion event; poll() queries it,
// drain() waits, release() forgets finished handoffs. Handoffs that fail
// validation are recorded as Failed and return the error.
class SharedArenaKVTransferConnector final : public KVTransferConnector {
 public:
  // stream == nullptr: the connector creates (and owns) a non-blocking stream.
  explicit SharedArenaKVTransferConnector(SharedArenaBinding arena, void* stream = nullptr);
  ~SharedArenaKVTransferConnector() override;
  SharedArenaKVTransferConnector(const SharedArenaKVTransferConnector&) = delete;
  SharedArenaKVTransferConnector& operator=(const SharedArenaKVTransferConnector&) = delete;

  // Source epoch = the binding's epoch (both sides map the same arena).
  base::Status submit(const KVBlockManifest& manifest, HandoffId* handle) override;
  // Source epoch as reported by the prefill side.
  base::Status submit_from(uint64_t source_epoch, const KVBlockManifest& manifest,
                           HandoffId* handle);
  KVTransferStatus poll(HandoffId handle) override;
  void cancel(HandoffId handle, const std::string& reason) override;
  KVTransferStatus drain(HandoffId handle) override;
  void release(HandoffId handle) override;

  uint64_t copied_bytes() const { return copied_bytes_; }
  void* stream() const { return stream_; }

 private:
  struct Record {
    HandoffId handle;
    KVTransferStatus status;
    pbe_event* done = nullptr;
    bool cancel_requested = false;
    std::string cancel_reason;
  };
  Record* find(HandoffId handle);
  KVTransferStatus settle(Record& record, bool wait);

  SharedArenaBinding arena_;
  void* stream_ = nullptr;
  bool owns_stream_ = false;
  uint64_t next_handoff_id_ = 1;
  uint64_t copied_bytes_ = 0;
  std::vector<Record> records_;
};

}  // namespace serving

#endif  // PBE_INCLUDE_SERVING_PD_HANDOFF_H_
