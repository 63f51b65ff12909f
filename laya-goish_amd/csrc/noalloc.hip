// Device scratch of the allocation-free entry points (lg_decode_noalloc): one file-scope array,
// which every GPU the library runs on holds for the life of the process.  Host code reaches it
// only through the device address hipGetSymbolAddress returns for each device (the array's name
// on the host is a stand-in, not a device address).
#include <hip/hip_runtime.h>

#include <mutex>

#include "common.h"
#include "noalloc.h"

namespace lg {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

std::mutex &noalloc_mutex(int device) {
  static std::mutex mu[kMaxDevices];
  LG_REQUIRE(device >= 0 && device < kMaxDevices, "no-alloc scratch: device %d out of range", device);
  return mu[device];
}

void *noalloc_scratch(int device) {
  static std::mutex mu;
  static void *ptr[kMaxDevices] = {};
  LG_REQUIRE(device >= 0 && device < kMaxDevices, "no-alloc scratch: device %d out of range", device);
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[device]) {  // once per device, with that device current
    int cur = 0;
    HIP_CHECK(hipGetDevice(&cur));
    HIP_CHECK(hipSetDevice(device));
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr)
      fail(LG_ERR_DEVICE, "no-alloc scratch: hipGetSymbolAddress failed on device %d: %s", device, hipGetErrorString(e));
    HIP_CHECK(back);
    ptr[device] = p;
  }
  return ptr[device];
}

}  // namespace lg
