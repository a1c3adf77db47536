// Bump allocator for device activations (drop-in for the reference's
// src/arena.h:20-73): one reservation up front, 256-byte aligned carving,
// mark / release scoping and peak tracking, so nothing in the token loop ever
// calls hipMalloc.
#pragma once

#include <cstddef>
#include <string>

#include "common.h"

namespace lcr {

class DeviceArena {
 public:
  DeviceArena() = default;
  explicit DeviceArena(size_t capacity_bytes);
  ~DeviceArena();

  DeviceArena(const DeviceArena&) = delete;
  DeviceArena& operator=(const DeviceArena&) = delete;
  DeviceArena(DeviceArena&& other) noexcept;
  DeviceArena& operator=(DeviceArena&& other) noexcept;

  // Frees any previous block and reserves a new one of this many bytes.
  void reserve(size_t capacity_bytes);

  void* allocate(size_t bytes, size_t alignment = 256);

  template <typename T>
  T* alloc(size_t count) {
    return static_cast<T*>(allocate(count * sizeof(T), 256));
  }

  size_t mark() const { return used_; }
  void release(size_t mark);
  void reset() { release(0); }

  size_t used() const { return used_; }
  size_t peak() const { return peak_; }
  size_t capacity() const { return capacity_; }
  std::string usage_string() const;

 private:
  void free_block();

  char* base_ = nullptr;
  size_t capacity_ = 0;
  size_t used_ = 0;
  size_t peak_ = 0;
};

// Releases to the mark taken at construction.
class ArenaScope {
 public:
  explicit ArenaScope(DeviceArena& arena) : arena_(arena), mark_(arena.mark()) {}
  ~ArenaScope() { arena_.release(mark_); }
  ArenaScope(const ArenaScope&) = delete;
  ArenaScope& operator=(const ArenaScope&) = delete;

 private:
  DeviceArena& arena_;
  size_t mark_;
};

}  // namespace lcr
