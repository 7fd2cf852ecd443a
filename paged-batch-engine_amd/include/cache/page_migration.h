// Transactional page-copy backends. TransferBackend is the plugin boundary of
// the reference's page migration (infMain/include/cache/page_migration.h:8-27):
// submit/poll/drain/release over a BoundTransfer with the same result
// semantics. This build provides a host memcpy backend and a HIP backend that
// executes a whole BoundTransfer as one gfx950 kernel launch.
#ifndef PBE_INCLUDE_CACHE_PAGE_MIGRATION_H_
#define PBE_INCLUDE_CACHE_PAGE_MIGRATION_H_

#include <cstddef>
#include <cstdint>
#include <memory>

#include "base/base.h"
#include "cache/transfer_plan.h"

namespace cache {

using MigrationId = uint64_t;

// kGpuToGpu (device-to-device, e.g. the prefill->decode handoff inside one
// arena) is an addition; kToHost / kToGpu keep the reference's meaning.
enum class TransferDirection { kToHost, kToGpu, kGpuToGpu };

// kFailedSafe proves no remaining writes. kUnknown must retain all resources.
enum class BackendResult { kPending, kSucceeded, kFailedSafe, kUnknown };

class TransferBackend {
 public:
  virtual ~TransferBackend() = default;
  virtual bool supports(base::DeviceType device) const = 0;
  virtual BackendResult submit(MigrationId id, TransferDirection direction,
                               const BoundTransfer& transfer) noexcept = 0;
  virtual BackendResult poll(MigrationId id) noexcept = 0;
  virtual BackendResult drain(MigrationId id) noexcept = 0;
  virtual void release(MigrationId id) noexcept = 0;
};

// Synchronous host memcpy (ExecuteCpuTransfer).
std::unique_ptr<TransferBackend> MakeCpuTransferBackend();

// HIP backend with `slots` concurrent migrations on `device` (-1 = current).
// Each slot owns a non-blocking stream and a completion event. Before the
// first op is queued every endpoint is checked: the GPU side must be device
// memory of `device`, the host side pinned host memory (both device memory
// for kGpuToGpu); a failed check returns kFailedSafe without touching memory.
// All ops of one submission run as a single kernel launch. The optional
// dependency event (a borrowed hipEvent_t that must outlive the backend) is
// waited on by every submission. release() of a migration whose completion
// is not proven terminates the process, as a lost copy cannot be recovered.
std::unique_ptr<TransferBackend> MakeHipTransferBackend(size_t slots, int device,
                                                       void* dependency_event = nullptr);

}  // namespace cache

#endif  // PBE_INCLUDE_CACHE_PAGE_MIGRATION_H_
