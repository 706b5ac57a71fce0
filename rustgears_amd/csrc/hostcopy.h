// hostcopy.h — host<->device copies of run() inputs and outputs through a
// pinned staging ring.  Nothing here is part of the C ABI.
//
// A run on host buffers moves its whole input to the device and its whole
// output back (InferenceSession::run takes and returns host tensors,
// src/inference/mod.rs:212-221).  hipMemcpyAsync from pageable memory runs
// at roughly half of what the link carries, so large copies are cut into
// slot-sized chunks: host threads copy chunk i into a pinned slot while the
// DMA engine moves chunk i-1, and the slots are recycled once their copy's
// event has completed.  Small copies go straight through hipMemcpyAsync.
#pragma once
#include <hip/hip_runtime_api.h>
#include <stddef.h>

namespace rgnpu {

// Copies of at least this many bytes go through the staging ring, in chunks
// of a quarter of the copy (at least 1 MiB, at most one slot) so that even
// the smallest staged copy overlaps host copying with DMA.
constexpr size_t kStageMinBytes = size_t(1) << 20;

// The pinned ring of one stream (one program handle or worker).  Allocated
// on first use, on the device current at that time; freed with the owner,
// after the owner's stream has drained.
struct Staging {
  static constexpr int kSlots = 4;
  static constexpr size_t kSlotBytes = size_t(8) << 20;
  char* pinned = nullptr;
  hipEvent_t ev[kSlots] = {};
  Staging() = default;
  Staging(const Staging&) = delete;
  Staging& operator=(const Staging&) = delete;
  ~Staging();
  hipError_t ensure();
};

// Both copies return the first HIP error met; the caller then drains s
// before the ring is used again.
// dst_dev <- src_host (n bytes), enqueued on s.  Returns once every byte of
// src_host has been read (the DMA of the last chunk may still be running).
hipError_t copy_to_device(Staging& st, void* dst_dev, const void* src_host, size_t n, hipStream_t s);

// dst_host <- src_dev (n bytes) after the work already enqueued on s.
// Returns once dst_host holds every byte.
hipError_t copy_to_host(Staging& st, void* dst_host, const void* src_dev, size_t n, hipStream_t s);

// memcpy split over the process-wide copy threads (plus the caller).
void parallel_memcpy(void* dst, const void* src, size_t n);

}  // namespace rgnpu
