// The backend object behind the opaque dw_hip_backend handle.
#pragma once

#include "dw_common.h"

#include <atomic>
#include <mutex>

namespace dw {

void set_last_error(const std::string& m);

// Scratch of the no-alloc entry points: one array of this size per device
// (k_noalloc.hip), laid out as the per-channel multipliers and bias' tables
// (kNoAllocMaxChannels entries each) followed by the packed weights.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
constexpr size_t kNoAllocMaxChannels = 4096;
constexpr size_t kNoAllocTableBytes = 2 * kNoAllocMaxChannels * 4;
// Device address of this device's scratch array (looked up on the first
// call per device, which must run with that device current).
void* noalloc_scratch_setup(int device);
// One call's use of its device's scratch, from construction (before the
// first write) to destruction (after the last launch that reads it): holds
// the device's scratch mutex, makes `stream` wait for the previous call's
// work on the scratch, and marks this call's work as the one the next call
// waits for.
struct ScratchUse {
  int device;
  hipStream_t stream;
  std::lock_guard<std::mutex> lock;
  ScratchUse(int device, hipStream_t stream);
  ~ScratchUse();
};

// One device, one in-order stream (default priority).  Op functions that need
// temporary device memory (packed weights, per-channel scales) use grow-only
// workspaces owned by the backend, so repeated calls do not allocate.
//
// Thread safety: every entry point that touches the stream or the
// workspaces holds `mu` for its whole sequence (workspace sizing, parameter
// uploads, launches), so one backend can be shared by several host threads
// (the reference's backends are Send + Sync, backend.rs:42-48).  Work from
// different threads is queued in the order the lock is taken.
struct Backend {
  enum { WS_WPACK = 0, WS_SCALE = 1, WS_BIAS = 2, WS_LUT = 3, WS_POST = 4, kWsSlots = 5 };
  struct Ws {
    void* ptr = nullptr;
    size_t bytes = 0;
  };
  int device = 0;
  int num_cus = 0;
  hipStream_t stream = nullptr;
  Ws ws[kWsSlots];
  std::mutex mu;
  void* scratch = nullptr;  // this device's no-alloc scratch (its device address)

  // Holders: the handle itself, every buffer and every graph runtime made
  // on it (as the reference's Arc<Backend>): destroying the handle while
  // they live only drops its hold, and the last holder frees the device
  // state.
  std::atomic<int> holds{1};

  void* workspace(int slot, size_t bytes);
  void upload_async(void* dst, const void* src, size_t bytes);
  ~Backend();
};

inline void hold(Backend* b) { b->holds.fetch_add(1, std::memory_order_relaxed); }
inline void release(Backend* b) {
  if (b->holds.fetch_sub(1, std::memory_order_acq_rel) == 1) delete b;
}

}  // namespace dw
