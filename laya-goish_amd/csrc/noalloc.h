// Device scratch of the allocation-free entry points: a fixed-size array per GPU, resolved once per
// device.  Every call on one GPU shares it, so a call holds that GPU's lock (noalloc_mutex) from
// before its first launch until its stream has drained.
#pragma once
#include <cstddef>
#include <mutex>

namespace lg {

constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;  // 16 MiB per GPU

// Device address of this device's scratch array (kNoAllocScratchBytes bytes, 256-byte aligned).
void *noalloc_scratch(int device);

// The lock that serialises the users of one device's scratch (engines on other threads included).
std::mutex &noalloc_mutex(int device);

}  // namespace lg
