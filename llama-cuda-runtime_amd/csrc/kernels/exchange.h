// Values handed from one block to another inside one grid, with no fence.
//
// A kernel boundary costs about 1.6 us inside a graph on MI355X, and a kernel
// that only waits on memory latency (the decode attention at short contexts:
// 32 blocks reading a few hundred KB) costs that boundary plus its own load
// latency. Running such a consumer as extra blocks of its producer's grid lets
// it issue every load that does not depend on the producer (the cached keys
// and values) while the producer still streams its weights, and then take the
// few values it does depend on from exchange words.
//
// An exchange word is 64 bits: (kExchangeValid | bits of a float). Writer and
// reader use relaxed agent-scope atomics, which reach the memory side past
// the XCD-private L2s, and value and valid bit travel in one store, so a
// reader that sees the bit sees the value: no release fence (an L2 write-back
// on every XCD) is needed. Every word has exactly one reader per launch, which
// clears it after reading, so a word is valid only between its write and its
// read in the same launch; kernel boundaries order a launch's clears before the
// next launch's writes.
//
// Every wait is bounded. A reader that gives up raises the status word (the
// host checks it) and goes on with whatever it holds, so no wave is ever left
// spinning. The consumer blocks have the highest block ids of the grid, so
// they are dispatched after every producer block; the host also checks that
// all blocks of the grid fit on the device at once.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lcr {

constexpr unsigned long long kExchangeValid = 1ull << 32;

__device__ __forceinline__ void exchange_put(unsigned long long* word, float v) {
  __hip_atomic_store(word, kExchangeValid | static_cast<unsigned long long>(__float_as_uint(v)),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long exchange_peek(unsigned long long* word) {
  return __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void exchange_clear(unsigned long long* word) {
  __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool exchange_valid(unsigned long long w) { return (w & kExchangeValid) != 0; }

__device__ __forceinline__ float exchange_value(unsigned long long w) {
  return __uint_as_float(static_cast<uint32_t>(w));
}

__device__ __forceinline__ void exchange_give_up(int* status) {
  __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave reads N words per lane (word lane + 64 k of `words`), waiting until
// all are valid or `spins` polls have failed; then clears them. Returns the
// values in out[k]. Every lane of the wave must call it. Two polls are in
// flight at a time: the next is issued before the current one is checked, so
// a write is seen about half a memory round trip after it lands rather than
// up to a whole one.
template <int N>
__device__ __forceinline__ void exchange_take(unsigned long long* words, float (&out)[N], int spins,
                                              int* status) {
  const int lane = static_cast<int>(threadIdx.x & 63u);
  unsigned long long a[N], b[N];
  auto poll = [&](unsigned long long (&w)[N]) {
#pragma unroll
    for (int k = 0; k < N; ++k) w[k] = exchange_peek(words + lane + 64 * k);
  };
  auto all_valid = [&](const unsigned long long (&w)[N]) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok = ok && exchange_valid(w[k]);
    return __all(ok) != 0;
  };
  poll(a);
  int polls = 0;
  while (true) {
    poll(b);
    if (all_valid(a)) break;
    poll(a);
    if (all_valid(b)) {
#pragma unroll
      for (int k = 0; k < N; ++k) a[k] = b[k];
      break;
    }
    polls += 2;
    if (polls >= spins) {
      if (lane == 0) exchange_give_up(status);
      break;
    }
  }
#pragma unroll
  for (int k = 0; k < N; ++k) {
    out[k] = exchange_value(a[k]);
    exchange_clear(words + lane + 64 * k);
  }
}

// Broadcast words: one writer, any number of readers, never cleared. A word
// is (tag << 32 | 32-bit payload); a reader waits for the tag of the current
// launch, which the writer and every reader derive alike (a step counter that
// only grows, and the launch's place in its graph), so a word left by an
// earlier launch never passes for a current one.
__device__ __forceinline__ void exchange_put_tagged(unsigned long long* word, uint32_t tag, uint32_t payload) {
  __hip_atomic_store(word, (static_cast<unsigned long long>(tag) << 32) | payload, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// One wave waits for N words per lane to carry `tag`, two polls in flight as
// in exchange_take, at most `spins` polls; returns the payloads. Word k of a
// lane is at address(k) (by default word lane + 64 k of `words`).
template <int N, typename Address>
__device__ __forceinline__ void exchange_wait_tagged_at(Address address, uint32_t tag, uint32_t (&out)[N],
                                                        int spins, int* status) {
  const int lane = static_cast<int>(threadIdx.x & 63u);
  unsigned long long a[N], b[N];
  auto poll = [&](unsigned long long (&w)[N]) {
#pragma unroll
    for (int k = 0; k < N; ++k) w[k] = exchange_peek(address(k));
  };
  auto all_current = [&](const unsigned long long (&w)[N]) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok = ok && static_cast<uint32_t>(w[k] >> 32) == tag;
    return __all(ok) != 0;
  };
  poll(a);
  int polls = 0;
  while (true) {
    poll(b);
    if (all_current(a)) break;
    poll(a);
    if (all_current(b)) {
#pragma unroll
      for (int k = 0; k < N; ++k) a[k] = b[k];
      break;
    }
    polls += 2;
    if (polls >= spins) {
      if (lane == 0) exchange_give_up(status);
      break;
    }
  }
#pragma unroll
  for (int k = 0; k < N; ++k) out[k] = static_cast<uint32_t>(a[k]);
}

template <int N>
__device__ __forceinline__ void exchange_wait_tagged(unsigned long long* words, uint32_t tag, uint32_t (&out)[N],
                                                     int spins, int* status) {
  const int lane = static_cast<int>(threadIdx.x & 63u);
  exchange_wait_tagged_at<N>([&](int k) { return words + lane + 64 * k; }, tag, out, spins, status);
}

}  // namespace lcr
