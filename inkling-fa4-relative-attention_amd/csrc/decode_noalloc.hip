// Allocation-free decode: ifa4_decode_fwd (include/ifa4.h) with the library's
// own workspace, for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
// It has no counterpart in the reference.
//
// The workspace is the file-scope device array `scratch` below, of
// IFA4_DECODE_SCRATCH_BYTES.  Every GPU the library runs on holds its own copy,
// at its own address, until the process ends.  In host code the array's name
// is a host-side stand-in, not a device address: the address is looked up with
// hipGetSymbolAddress once per device, on the entry point's first call there
// (with that device current), kept per device, and passed to the kernels as a
// caller's workspace would be.  The decode kernels write every workspace byte
// they read within the same call, so nothing needs clearing between calls.
// All calls on one GPU share its array: calls that overlap in time on one GPU
// (from other streams or host threads) race.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "ifa4.h"
#include "ifa4_kernels.h"

static __device__ __align__(256) unsigned char scratch[IFA4_DECODE_SCRATCH_BYTES];

namespace {

constexpr size_t kScratchBytes = IFA4_DECODE_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];  // device address of `scratch`, per device
std::mutex g_scratch_mu;

// Device address of the current device's copy of `scratch`; the stream, when
// given, must belong to that device.
int32_t scratch_address(void* stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return IFA4_ELAUNCH;
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess ||
        sdev != dev)
      return IFA4_EINVAL;
  }
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
        return IFA4_ELAUNCH;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return IFA4_OK;
}

}  // namespace

extern "C" int32_t ifa4_decode_fwd_noalloc(const ifa4_args* args, void* stream) {
  // Host checks and the size limit come first: a rejected call touches no device.
  size_t need = 0;
  const int32_t st = ifa4::decode_workspace_need(args, &need);
  if (st != IFA4_OK) return st;
  if (need > kScratchBytes) return IFA4_EWORKSPACE;
  if (args->batch == 0) return IFA4_OK;
  void* ws = nullptr;
  const int32_t sa = scratch_address(stream, &ws);
  if (sa != IFA4_OK) return sa;
  return ifa4::decode_run(args, ws, kScratchBytes, stream);
}
