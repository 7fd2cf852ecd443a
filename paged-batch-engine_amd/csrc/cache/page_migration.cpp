// Host memcpy backend: infMain/source/cache/page_migration.cpp:9-18.
#include "cache/page_migration.h"

namespace cache {
namespace {

class CpuTransferBackend final : public TransferBackend {
 public:
  bool supports(base::DeviceType device) const override {
    return device == base::DeviceType::kDeviceCPU;
  }
  BackendResult submit(MigrationId, TransferDirection, const BoundTransfer& transfer) noexcept override {
    return ExecuteCpuTransfer(transfer) ? BackendResult::kSucceeded : BackendResult::kFailedSafe;
  }
  BackendResult poll(MigrationId) noexcept override { return BackendResult::kSucceeded; }
  BackendResult drain(MigrationId) noexcept override { return BackendResult::kSucceeded; }
  void release(MigrationId) noexcept override {}
};

}  // namespace

std::unique_ptr<TransferBackend> MakeCpuTransferBackend() {
  return std::make_unique<CpuTransferBackend>();
}

}  // namespace cache
