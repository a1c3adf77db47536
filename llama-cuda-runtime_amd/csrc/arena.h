// Device arena: one hipMalloc reserved when the model loads, carved into
// 256-byte-aligned buffers, so the token loop itself never allocates.
//
// Interface of the reference's DeviceArena (src/arena.h:20-73): allocate /
// alloc<T>, mark / release / reset, used / peak / capacity, usage_string, and
// the ArenaScope guard. The block is owned by a unique_ptr with a hipFree
// deleter; a move hands the block and its counters over and leaves the source
// empty (move-construct, then swap).
#pragma once

#include <cstddef>
#include <memory>
#include <string>
#include <utility>

#include "common.h"

namespace lcr {

class DeviceArena {
 public:
  DeviceArena() = default;
  explicit DeviceArena(size_t capacity_bytes) { reserve(capacity_bytes); }
  DeviceArena(DeviceArena&& other) noexcept { swap(other); }
  DeviceArena& operator=(DeviceArena&& other) noexcept {
    DeviceArena taken(std::move(other));
    swap(taken);
    return *this;
  }
  DeviceArena(const DeviceArena&) = delete;
  DeviceArena& operator=(const DeviceArena&) = delete;

  // Drops the current block (every pointer handed out becomes invalid) and
  // reserves `capacity_bytes` (none when 0).
  void reserve(size_t capacity_bytes);

  // Next `bytes` at an `alignment`-aligned offset (a power of two). Throws
  // lcr::Error ("... arena is full ...") when they do not fit.
  void* allocate(size_t bytes, size_t alignment = 256);

  template <typename T>
  T* alloc(size_t count) {
    return static_cast<T*>(allocate(count * sizeof(T), 256));
  }

  size_t mark() const { return cursor_.used; }
  // Forgets everything allocated after `mark` (a value mark() returned).
  void release(size_t mark);
  void reset() { cursor_.used = 0; }

  size_t used() const { return cursor_.used; }
  size_t peak() const { return cursor_.peak; }
  size_t capacity() const { return capacity_; }
  std::string usage_string() const;

 private:
  struct HipFree {
    void operator()(void* p) const;
  };
  struct Cursor {
    size_t used = 0;
    size_t peak = 0;
  };

  void swap(DeviceArena& other) noexcept {
    block_.swap(other.block_);
    std::swap(capacity_, other.capacity_);
    std::swap(cursor_, other.cursor_);
  }

  std::unique_ptr<unsigned char, HipFree> block_;
  size_t capacity_ = 0;
  Cursor cursor_;
};

// Returns the arena to the mark it saw at construction.
class ArenaScope {
 public:
  explicit ArenaScope(DeviceArena& arena) : arena_(arena), saved_(arena.mark()) {}
  ~ArenaScope() { arena_.release(saved_); }
  ArenaScope(const ArenaScope&) = delete;
  ArenaScope& operator=(const ArenaScope&) = delete;

 private:
  DeviceArena& arena_;
  const size_t saved_;
};

}  // namespace lcr
