// C++ tests of the host classes that need a GPU: the device arena, with the
// checks of the reference's test_arena (tests/test_kernels.cu:510-533) plus
// alignment, scopes that nest, moves, and memory that a kernel-side copy can
// actually use. Built by tests/cpp/Makefile against liblcr_amd.so and run by
// tests/test_gpu_host_classes.py on a GPU.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <exception>
#include <string>
#include <utility>
#include <vector>

#include "arena.h"

namespace {

int g_failures = 0;

void report(bool ok, int line, const char* what) {
  if (ok) return;
  std::fprintf(stderr, "FAIL line %d: %s\n", line, what);
  ++g_failures;
}

#define EXPECT(cond) report((cond), __LINE__, #cond)

template <typename F>
bool throws_with(F&& f, const char* needle) {
  try {
    f();
  } catch (const std::exception& e) {
    return std::string(e.what()).find(needle) != std::string::npos;
  }
  return false;
}

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

void test_reference_cases() {
  lcr::DeviceArena arena(1 << 20);
  EXPECT(arena.used() == 0);
  EXPECT(arena.capacity() == (1u << 20));
  float* first = arena.alloc<float>(100);
  EXPECT(first != nullptr);
  EXPECT(arena.used() == 400);
  const size_t mark = arena.mark();
  float* second = arena.alloc<float>(64);
  EXPECT(second != nullptr && second != first);
  EXPECT(arena.used() > mark);
  const size_t after_second = arena.used();
  {
    lcr::ArenaScope scope(arena);
    arena.alloc<float>(1000);
    EXPECT(arena.used() > after_second);
  }
  EXPECT(arena.used() == after_second);  // the scope gave its allocation back
  EXPECT(arena.peak() >= 400 + 1000 * sizeof(float));
  arena.release(mark);
  EXPECT(arena.used() == mark);
  EXPECT(throws_with([&] { arena.alloc<char>(1 << 21); }, "arena is full"));
  EXPECT(arena.used() == mark);  // a failed allocation takes nothing
}

void test_alignment_and_release_rules() {
  lcr::DeviceArena arena(1 << 16);
  void* a = arena.allocate(3);
  void* b = arena.allocate(5);  // default 256-byte alignment
  EXPECT(aligned(a, 256) && aligned(b, 256));
  EXPECT(static_cast<char*>(b) - static_cast<char*>(a) == 256);
  void* c = arena.allocate(1, 4096);
  EXPECT(aligned(c, 4096));
  EXPECT(throws_with([&] { arena.allocate(8, 3); }, "power of two"));
  EXPECT(throws_with([&] { arena.release(arena.used() + 1); }, "forward"));
  arena.reset();
  EXPECT(arena.used() == 0 && arena.peak() > 0);
  // An allocation that exactly fills the block succeeds; one more byte fails.
  EXPECT(arena.allocate(1 << 16) != nullptr);
  EXPECT(throws_with([&] { arena.allocate(1); }, "arena is full"));
}

void test_move_and_reserve() {
  lcr::DeviceArena a(1 << 12);
  void* p = a.allocate(100);
  lcr::DeviceArena b(std::move(a));
  EXPECT(b.capacity() == (1u << 12) && b.used() == 100);
  EXPECT(a.capacity() == 0 && a.used() == 0);
  EXPECT(throws_with([&] { a.allocate(1); }, "arena is full"));
  lcr::DeviceArena c;
  c = std::move(b);
  EXPECT(c.capacity() == (1u << 12) && c.allocate(8) != p);
  c.reserve(0);
  EXPECT(c.capacity() == 0 && c.used() == 0);
  EXPECT(!c.usage_string().empty());
}

void test_memory_is_usable() {
  lcr::DeviceArena arena(1 << 20);
  std::vector<int32_t> host(4096), back(4096, 0);
  for (int i = 0; i < 4096; ++i) host[i] = i * 7 - 3;
  int32_t* x = arena.alloc<int32_t>(4096);
  int32_t* y = arena.alloc<int32_t>(4096);
  EXPECT(hipMemcpy(x, host.data(), host.size() * 4, hipMemcpyHostToDevice) == hipSuccess);
  EXPECT(hipMemcpy(y, x, host.size() * 4, hipMemcpyDeviceToDevice) == hipSuccess);
  EXPECT(hipMemcpy(back.data(), y, back.size() * 4, hipMemcpyDeviceToHost) == hipSuccess);
  EXPECT(back == host);
}

}  // namespace

int main() {
  int devices = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess || devices < 1) {
    std::fprintf(stderr, "no HIP device\n");
    return 2;
  }
  test_reference_cases();
  test_alignment_and_release_rules();
  test_move_and_reserve();
  test_memory_is_usable();
  if (g_failures != 0) {
    std::fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("all device checks passed\n");
  return 0;
}
