// The backend object behind the opaque dw_hip_backend handle.
#pragma once

#include "dw_common.h"

namespace dw {

void set_last_error(const std::string& m);

// One device, one in-order stream (default priority).  Op functions that need
// temporary device memory (packed weights, per-channel scales) use grow-only
// workspaces owned by the backend, so repeated calls do not allocate.
struct Backend {
  enum { WS_WPACK = 0, WS_SCALE = 1, WS_BIAS = 2, WS_LUT = 3, kWsSlots = 4 };
  struct Ws {
    void* ptr = nullptr;
    size_t bytes = 0;
  };
  int device = 0;
  int num_cus = 0;
  hipStream_t stream = nullptr;
  Ws ws[kWsSlots];

  void* workspace(int slot, size_t bytes);
  void upload_async(void* dst, const void* src, size_t bytes);
  ~Backend();
};

}  // namespace dw
