// Internal declarations shared by device.cpp (memory, copies, views) and bindings.cpp.
#pragma once

#include <c10/core/Allocator.h>

namespace vkt {

// Device memory behind vk tensors: hrt blocks (data_ptr() is the device address).
c10::Allocator* device_allocator();
// Page-locked host memory from the runtime; non_blocking copies between it and dense vk tensors run
// asynchronously.
c10::Allocator* pinned_allocator();

}  // namespace vkt
