// Interface between the C-ABI files: the per-thread error state, the device
// choice and the registry of host tensors with device copies live in
// abi.hip; residency.hip (whole-model upload) uses them through these calls.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <memory>

namespace rsllm_hip::abi {

// A device allocation, freed when the last reference to it goes (hipFree,
// which synchronises the device first, on the device it was made on).
// Registry entries and the calls that use them share ownership, so memory a
// call is reading is never freed under it.
struct DevMem {
    uint8_t *p = nullptr;
    int device = 0;
    DevMem() = default;
    DevMem(const DevMem &) = delete;
    DevMem &operator=(const DevMem &) = delete;
    ~DevMem();
};

// hipMalloc for every device allocation of the library, counted (see
// rsllm_hip_device_allocations).
hipError_t dev_malloc(void **p, size_t bytes);

// Record the calling thread's error (rsllm_hip_last_error) and return status.
int set_error(int status, const char *msg);
// Record success and return RSLLM_HIP_OK.
int ok_status();
// Record a HIP runtime failure at `where` and return RSLLM_HIP_ERR_DEVICE.
int device_error(hipError_t e, const char *where);
// Make the process's device current on this thread (and create the thread's
// stream); returns a status.
int ensure_current_device();
// Host tensor (host, len, dtype, in_dim) -> device copy at dev, owned by the
// uploaded model `owner` (never 0), inside the allocation `keep` holds alive.
// Host-pointer entry points find it.
void registry_add(const uint8_t *host, size_t len, uint32_t dtype, size_t in_dim, uint8_t *dev,
                  uint64_t owner, std::shared_ptr<void> keep);
// Remove every entry of one owner (memory still used by a call in flight is
// freed when that call drops its reference).
void registry_drop_owner(uint64_t owner);

}  // namespace rsllm_hip::abi
