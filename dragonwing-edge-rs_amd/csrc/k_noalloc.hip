// Device scratch for the entry points that allocate nothing
// (dw_hip_qlinearconv_u8s8_noalloc): one file-scope array per device, whose
// device address is looked up once per device when a backend is created on
// it (with that device current) and used from then on.  The array's name is
// only a host-side stand-in for the symbol; host code never passes it to a
// kernel or a copy, only the looked-up address.
#include "backend.h"

#include <mutex>

namespace dw {
namespace {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
// Per device: held from the first write of a call's tables to the launch of
// its last kernel, and the event recorded after that launch, which the next
// call's stream waits on before writing the scratch again.  Together they
// order calls through different backends (streams) on one device.
std::mutex g_use_mu[kMaxDevices];
hipEvent_t g_last_use[kMaxDevices] = {};

}  // namespace

void* noalloc_scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices) fail(-2, "no-alloc scratch: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      fail(-1, std::string("no-alloc scratch: hipGetSymbolAddress failed: ") + hipGetErrorString(e));
    e = hipEventCreateWithFlags(&g_last_use[device], hipEventDisableTiming);
    if (e != hipSuccess) fail(-1, std::string("no-alloc scratch: hipEventCreate failed: ") + hipGetErrorString(e));
    g_scratch_ptr[device] = p;
  }
  return g_scratch_ptr[device];
}

ScratchUse::ScratchUse(int dev, hipStream_t s) : device(dev), stream(s), lock(g_use_mu[dev]) {
  // An event never recorded is complete, so the first call does not wait.
  DW_HIP(hipStreamWaitEvent(stream, g_last_use[device], 0));
}

ScratchUse::~ScratchUse() {
  // After whatever this call enqueued (also when it failed part way).
  (void)hipEventRecord(g_last_use[device], stream);
}

}  // namespace dw
