// Device scratch of the allocation-free entry points: a fixed-size array per GPU, resolved once per
// device.  Calls that overlap on one GPU share it and race; the engine serialises its own calls.
#pragma once
#include <cstddef>

namespace lg {

constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;  // 16 MiB per GPU

// Device address of this device's scratch array (kNoAllocScratchBytes bytes, 256-byte aligned).
void *noalloc_scratch(int device);

}  // namespace lg
