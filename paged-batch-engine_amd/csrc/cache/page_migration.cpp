// Host-memory TransferBackend (the CPU member of the backend family of
// infMain/include/cache/page_migration.h:13-27). The copy runs inside
// submit(), so a submission is complete, or proven unwritten, before submit
// returns; poll and drain have nothing left to wait for.
#include "cache/page_migration.h"

namespace cache {
namespace {

class HostMemcpyBackend final : public TransferBackend {
 public:
  bool supports(base::DeviceType device) const override { return device == base::DeviceType::kDeviceCPU; }

  // ExecuteCpuTransfer validates every op before its first memcpy, so a
  // rejected transfer has written nothing.
  BackendResult submit(MigrationId, TransferDirection, const BoundTransfer& transfer) noexcept override {
    if (!ExecuteCpuTransfer(transfer)) return BackendResult::kFailedSafe;
    return BackendResult::kSucceeded;
  }
  BackendResult poll(MigrationId) noexcept override { return settled(); }
  BackendResult drain(MigrationId) noexcept override { return settled(); }
  void release(MigrationId) noexcept override {}

 private:
  static BackendResult settled() { return BackendResult::kSucceeded; }
};

}  // namespace

std::unique_ptr<TransferBackend> MakeCpuTransferBackend() { return std::make_unique<HostMemcpyBackend>(); }

}  // namespace cache
