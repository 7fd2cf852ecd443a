// HIP TransferBackend: the contract of CudaTransferBackend
// (infMain/source/cache/cuda_transfer_backend.cpp:19-128) with the per-op
// cudaMemcpyAsync loop replaced by one op-list kernel launch per submission.
// All device work goes through the C ABI in pbe_handoff.h.
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

#include "cache/page_migration.h"
#include "pbe_handoff.h"

namespace cache {
namespace {

class HipTransferBackend final : public TransferBackend {
 public:
  HipTransferBackend(size_t slots, int device, void* dependency)
      : device_(device), dependency_(dependency), slots_(slots) {
    if (slots == 0) throw std::invalid_argument("HIP migration needs at least one slot");
    if (device_ < 0) device_ = 0;
    for (auto& slot : slots_) {
      if (pbe_stream_create(device_, &slot.stream) != PBE_OK ||
          pbe_event_create(device_, 0, &slot.fence) != PBE_OK) {
        const std::string why = pbe_last_error();
        destroy();
        throw std::runtime_error("HIP migration stream/event allocation failed: " + why);
      }
    }
  }

  ~HipTransferBackend() override {
    for (auto& slot : slots_)
      if (slot.id && pbe_stream_synchronize(device_, slot.stream) != PBE_OK) std::terminate();
    destroy();
  }

  bool supports(base::DeviceType device) const override {
    return device == base::DeviceType::kDeviceHIP;
  }

  BackendResult submit(MigrationId id, TransferDirection direction,
                       const BoundTransfer& transfer) noexcept override {
    if (find(id)) return BackendResult::kUnknown;
    std::vector<pbe_copy_op> ops;
    try {
      ops.reserve(transfer.operations().size());
    } catch (...) {
      return BackendResult::kFailedSafe;
    }
    // Validate every physical endpoint before queueing anything.
    for (const auto& op : transfer.operations()) {
      if (op.bytes == 0 || !op.source || !op.destination) return BackendResult::kFailedSafe;
      const bool src_gpu = direction != TransferDirection::kToGpu;
      const bool dst_gpu = direction != TransferDirection::kToHost;
      if (!endpoint_ok(op.source, op.bytes, src_gpu) || !endpoint_ok(op.destination, op.bytes, dst_gpu))
        return BackendResult::kFailedSafe;
      ops.push_back({reinterpret_cast<uint64_t>(op.source), reinterpret_cast<uint64_t>(op.destination),
                     op.bytes});
    }
    Slot* slot = nullptr;
    for (auto& candidate : slots_)
      if (!candidate.id) {
        slot = &candidate;
        break;
      }
    if (!slot) return BackendResult::kFailedSafe;
    slot->id = id;
    slot->failed = false;
    slot->safe = false;
    if (dependency_ && pbe_stream_wait_raw_event(device_, slot->stream, dependency_) != PBE_OK) {
      slot->failed = true;
      return BackendResult::kUnknown;
    }
    const int rc = pbe_copy_ops(ops.data(), static_cast<int64_t>(ops.size()), device_, slot->stream);
    if (rc == PBE_ERR_INVALID) {  // rejected on the host: nothing was queued by this call
      slot->id = 0;
      return BackendResult::kFailedSafe;
    }
    if (rc != PBE_OK) {
      slot->failed = true;
      return BackendResult::kUnknown;
    }
    if (pbe_event_record(slot->fence, slot->stream) != PBE_OK) {
      slot->failed = true;
      return BackendResult::kUnknown;
    }
    return BackendResult::kPending;
  }

  BackendResult poll(MigrationId id) noexcept override {
    Slot* slot = find(id);
    if (!slot || slot->failed) return BackendResult::kUnknown;
    const int rc = pbe_event_query(slot->fence);
    if (rc == PBE_NOT_READY) return BackendResult::kPending;
    if (rc != PBE_OK) {
      slot->failed = true;
      return BackendResult::kUnknown;
    }
    slot->safe = true;
    return BackendResult::kSucceeded;
  }

  BackendResult drain(MigrationId id) noexcept override {
    Slot* slot = find(id);
    if (!slot || pbe_stream_synchronize(device_, slot->stream) != PBE_OK) return BackendResult::kUnknown;
    slot->safe = true;
    return slot->failed ? BackendResult::kFailedSafe : BackendResult::kSucceeded;
  }

  void release(MigrationId id) noexcept override {
    Slot* slot = find(id);
    if (!slot) return;  // rejected before any stream submission
    if (!slot->safe) std::terminate();
    slot->id = 0;
  }

 private:
  struct Slot {
    MigrationId id = 0;
    void* stream = nullptr;
    pbe_event* fence = nullptr;
    bool failed = false, safe = false;
  };

  bool endpoint_ok(const void* p, size_t bytes, bool want_device) const noexcept {
    int kind = PBE_PTR_UNKNOWN, dev = -1;
    if (pbe_pointer_kind(p, bytes, &kind, &dev) != PBE_OK) return false;
    return want_device ? (kind == PBE_PTR_DEVICE && dev == device_) : kind == PBE_PTR_PINNED_HOST;
  }

  Slot* find(MigrationId id) noexcept {
    for (auto& slot : slots_)
      if (slot.id == id) return &slot;
    return nullptr;
  }

  void destroy() noexcept {
    for (auto& slot : slots_) {
      if (slot.fence) pbe_event_destroy(slot.fence);
      if (slot.stream) pbe_stream_destroy(device_, slot.stream);
      slot.fence = nullptr;
      slot.stream = nullptr;
    }
  }

  int device_;
  void* dependency_;
  std::vector<Slot> slots_;
};

}  // namespace

std::unique_ptr<TransferBackend> MakeHipTransferBackend(size_t slots, int device,
                                                       void* dependency_event) {
  return std::make_unique<HipTransferBackend>(slots, device, dependency_event);
}

}  // namespace cache
