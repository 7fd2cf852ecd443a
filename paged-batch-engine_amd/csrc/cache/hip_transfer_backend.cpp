// HIP TransferBackend for the contract of infMain/include/cache/page_migration.h:13-27.
//
// Design: every submission is ONE gfx950 op-list kernel (pbe_copy_ops) on the
// backend's single in-order stream, followed by one completion event. A copy
// kernel already spreads over every CU, so parallel streams would only contend
// for HBM; one stream makes completion monotone, which lets poll() settle
// every earlier launch at once. Launches live in a fixed table of `slots`
// records (the in-flight limit), found by MigrationId through a hash index.
//
// A record moves kQueued -> kDone (event observed) or kQueued -> kBroken (a
// HIP call failed after work may have been queued). Outcomes:
//   kSucceeded   event observed on a healthy record;
//   kFailedSafe  nothing was queued (endpoint check, no free record, the ABI
//                rejected the op list), or a broken record whose stream has
//                since drained, so no write of it can still land;
//   kUnknown     a broken record not yet drained, an unknown id, or a
//                duplicate id: the caller must quarantine.
// release() of a record whose completion is not established terminates the
// process: the copy may still write memory the caller would reuse.
#include <exception>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "cache/page_migration.h"
#include "pbe_handoff.h"

namespace cache {
namespace {

class HipMigrationQueue final : public TransferBackend {
 public:
  HipMigrationQueue(size_t capacity, int device, void* dependency)
      : device_(device < 0 ? 0 : device), dependency_(dependency), launches_(capacity) {
    if (capacity == 0) throw std::invalid_argument("HIP migration needs at least one slot");
    bool ok = pbe_stream_create(device_, &stream_) == PBE_OK;
    for (auto& l : launches_) ok = ok && pbe_event_create(device_, 0, &l.done) == PBE_OK;
    if (!ok) {
      const std::string why = pbe_last_error();
      teardown();
      throw std::runtime_error("HIP migration stream/event allocation failed: " + why);
    }
    by_id_.reserve(capacity);
  }

  ~HipMigrationQueue() override {
    // Queued copies still own their destinations: wait for the stream, and
    // if even that cannot be established the process must not continue.
    if (!by_id_.empty() && pbe_stream_synchronize(device_, stream_) != PBE_OK) std::terminate();
    teardown();
  }

  bool supports(base::DeviceType device) const override { return device == base::DeviceType::kDeviceHIP; }

  BackendResult submit(MigrationId id, TransferDirection direction,
                       const BoundTransfer& transfer) noexcept override {
    if (by_id_.count(id)) return BackendResult::kUnknown;
    std::vector<pbe_copy_op> ops;
    if (!collect_ops(direction, transfer, &ops)) return BackendResult::kFailedSafe;
    Launch* l = idle_launch();
    if (!l) return BackendResult::kFailedSafe;
    if (dependency_ && pbe_stream_wait_raw_event(device_, stream_, dependency_) != PBE_OK)
      return BackendResult::kFailedSafe;  // a failed wait queues nothing
    const int rc = pbe_copy_ops(ops.data(), static_cast<int64_t>(ops.size()), device_, stream_);
    // Rejected on the host (bad op list, or a stream under graph capture):
    // nothing was queued.
    if (rc == PBE_ERR_INVALID || rc == PBE_ERR_UNSUPPORTED) return BackendResult::kFailedSafe;
    try {
      by_id_.emplace(id, static_cast<size_t>(l - launches_.data()));
    } catch (...) {
      // The copy is queued but cannot be tracked: wait for it here.
      return pbe_stream_synchronize(device_, stream_) == PBE_OK && rc == PBE_OK ? BackendResult::kFailedSafe
                                                                                : BackendResult::kUnknown;
    }
    l->id = id;
    l->seq = ++issued_;
    l->state = (rc == PBE_OK && pbe_event_record(l->done, stream_) == PBE_OK) ? State::kQueued : State::kBroken;
    return l->state == State::kQueued ? BackendResult::kPending : BackendResult::kUnknown;
  }

  BackendResult poll(MigrationId id) noexcept override {
    Launch* l = lookup(id);
    if (!l) return BackendResult::kUnknown;
    if (l->state == State::kQueued) observe(l);
    return outcome(*l);
  }

  BackendResult drain(MigrationId id) noexcept override {
    Launch* l = lookup(id);
    if (!l) return BackendResult::kUnknown;
    if (l->state == State::kQueued && pbe_event_synchronize(l->done) == PBE_OK) {
      settle_through(l->seq);
    } else if (l->state != State::kDone && l->state != State::kDrained) {
      // Broken, or its event failed: only an idle stream proves no write of
      // this launch is still in flight.
      if (pbe_stream_synchronize(device_, stream_) != PBE_OK) {
        l->state = State::kBroken;
        return BackendResult::kUnknown;
      }
      settle_through(issued_);
      if (l->state != State::kDone) l->state = State::kDrained;
    }
    return outcome(*l);
  }

  void release(MigrationId id) noexcept override {
    auto it = by_id_.find(id);
    if (it == by_id_.end()) return;  // never queued
    Launch& l = launches_[it->second];
    if (l.state != State::kDone && l.state != State::kDrained) std::terminate();
    l.state = State::kIdle;
    l.id = 0;
    by_id_.erase(it);
  }

 private:
  enum class State { kIdle, kQueued, kDone, kBroken, kDrained };
  struct Launch {
    MigrationId id = 0;
    uint64_t seq = 0;  // submission order on the stream
    State state = State::kIdle;
    pbe_event* done = nullptr;
  };

  static BackendResult outcome(const Launch& l) {
    switch (l.state) {
      case State::kQueued: return BackendResult::kPending;
      case State::kDone: return BackendResult::kSucceeded;
      case State::kDrained: return BackendResult::kFailedSafe;
      default: return BackendResult::kUnknown;
    }
  }

  // Every endpoint checked before anything is queued: the GPU side must be
  // device memory of this backend's GPU, the host side pinned host memory.
  bool collect_ops(TransferDirection direction, const BoundTransfer& transfer,
                   std::vector<pbe_copy_op>* ops) const noexcept {
    const bool src_gpu = direction != TransferDirection::kToGpu;
    const bool dst_gpu = direction != TransferDirection::kToHost;
    try {
      ops->reserve(transfer.operations().size());
      for (const auto& op : transfer.operations()) {
        if (op.bytes == 0 || !op.source || !op.destination) return false;
        if (!endpoint_ok(op.source, op.bytes, src_gpu) || !endpoint_ok(op.destination, op.bytes, dst_gpu))
          return false;
        ops->push_back({reinterpret_cast<uint64_t>(op.source), reinterpret_cast<uint64_t>(op.destination),
                        op.bytes});
      }
    } catch (...) {
      return false;
    }
    return true;
  }

  bool endpoint_ok(const void* p, size_t bytes, bool want_device) const noexcept {
    int kind = PBE_PTR_UNKNOWN, dev = -1;
    if (pbe_pointer_kind(p, bytes, &kind, &dev) != PBE_OK) return false;
    return want_device ? (kind == PBE_PTR_DEVICE && dev == device_) : kind == PBE_PTR_PINNED_HOST;
  }

  Launch* idle_launch() noexcept {
    for (auto& l : launches_)
      if (l.state == State::kIdle) return &l;
    return nullptr;
  }

  Launch* lookup(MigrationId id) noexcept {
    auto it = by_id_.find(id);
    return it == by_id_.end() ? nullptr : &launches_[it->second];
  }

  // Queries one launch's event; on completion everything queued before it on
  // the stream has completed too.
  void observe(Launch* l) noexcept {
    const int rc = pbe_event_query(l->done);
    if (rc == PBE_OK) settle_through(l->seq);
    else if (rc != PBE_NOT_READY) l->state = State::kBroken;
  }

  void settle_through(uint64_t seq) noexcept {
    for (auto& l : launches_)
      if (l.state == State::kQueued && l.seq <= seq) l.state = State::kDone;
  }

  void teardown() noexcept {
    for (auto& l : launches_)
      if (l.done) pbe_event_destroy(l.done), l.done = nullptr;
    if (stream_) pbe_stream_destroy(device_, stream_), stream_ = nullptr;
  }

  int device_;
  void* dependency_;
  void* stream_ = nullptr;
  uint64_t issued_ = 0;
  std::vector<Launch> launches_;
  std::unordered_map<MigrationId, size_t> by_id_;
};

}  // namespace

std::unique_ptr<TransferBackend> MakeHipTransferBackend(size_t slots, int device, void* dependency_event) {
  return std::make_unique<HipMigrationQueue>(slots, device, dependency_event);
}

}  // namespace cache
