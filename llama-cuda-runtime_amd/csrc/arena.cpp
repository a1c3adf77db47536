#include "arena.h"

#include <hip/hip_runtime.h>

namespace lcr {

void DeviceArena::HipFree::operator()(void* p) const { (void)hipFree(p); }

void DeviceArena::reserve(size_t capacity_bytes) {
  block_.reset();
  capacity_ = 0;
  cursor_ = Cursor{};
  if (capacity_bytes == 0) return;
  void* p = nullptr;
  const hipError_t status = hipMalloc(&p, capacity_bytes);
  if (status != hipSuccess) {
    LCR_FAIL("hipMalloc of a " << format_bytes(capacity_bytes)
                               << " device arena failed: " << hipGetErrorString(status));
  }
  block_.reset(static_cast<unsigned char*>(p));
  capacity_ = capacity_bytes;
}

void* DeviceArena::allocate(size_t bytes, size_t alignment) {
  LCR_CHECK(alignment != 0 && (alignment & (alignment - 1)) == 0,
            "arena alignment " << alignment << " is not a power of two");
  const size_t start = align_up(cursor_.used, alignment);
  const size_t room = start <= capacity_ ? capacity_ - start : 0;
  LCR_CHECK(bytes <= room, "device arena is full: " << format_bytes(bytes) << " requested, "
                                                    << format_bytes(room) << " left of "
                                                    << format_bytes(capacity_));
  cursor_.used = start + bytes;
  cursor_.peak = cursor_.used > cursor_.peak ? cursor_.used : cursor_.peak;
  return block_.get() + start;
}

void DeviceArena::release(size_t mark) {
  LCR_CHECK(mark <= cursor_.used,
            "cannot release the arena forward, to " << mark << " from " << cursor_.used);
  cursor_.used = mark;
}

std::string DeviceArena::usage_string() const {
  return format_bytes(cursor_.used) + " in use, " + format_bytes(cursor_.peak) + " peak, " +
         format_bytes(capacity_) + " reserved";
}

}  // namespace lcr
