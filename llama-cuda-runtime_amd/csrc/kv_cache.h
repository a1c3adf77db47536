// Key/value cache, contiguous or paged (drop-in for the reference's
// src/kv_cache.cuh:30-118).
//
// Per layer, keys and values are stored head-major, K[kv_head][position][d],
// so one head's history is a straight run of memory. The contiguous layout
// reserves max_seq positions per head; the paged layout hands out pages of
// page_size positions from a pool, in order, as the sequence grows, and keeps a
// per-layer page table on the device. Both are addressed by one formula
// (KvCacheView::offset), with the table lookup compiled away when contiguous.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/lcr_kernels.h"
#include "config.h"
#include "dtype.h"

namespace lcr {

enum class KvLayout { kContiguous, kPaged };

// Non-owning, trivially copyable handle to one layer; same fields and order as
// the C-ABI's lcr_kv_view.
struct KvCacheView {
  elem_t* keys = nullptr;
  elem_t* values = nullptr;
  const int32_t* page_table = nullptr;
  int page_size = 0;
  int page_stride = 0;
  int head_stride = 0;
  int num_kv_heads = 0;
  int head_dim = 0;

  template <bool kPaged>
  __host__ __device__ __forceinline__ size_t offset(int head, int position) const {
    const int page = kPaged ? page_table[position / page_size] : 0;
    const int slot = kPaged ? position % page_size : position;
    return static_cast<size_t>(page) * static_cast<size_t>(page_stride) +
           static_cast<size_t>(head) * static_cast<size_t>(head_stride) +
           static_cast<size_t>(slot) * static_cast<size_t>(head_dim);
  }

  lcr_kv_view to_c() const {
    lcr_kv_view v;
    v.keys = keys;
    v.values = values;
    v.page_table = page_table;
    v.page_size = page_size;
    v.page_stride = page_stride;
    v.head_stride = head_stride;
    v.num_kv_heads = num_kv_heads;
    v.head_dim = head_dim;
    return v;
  }
  static KvCacheView from_c(const lcr_kv_view& c) {
    KvCacheView v;
    v.keys = static_cast<elem_t*>(c.keys);
    v.values = static_cast<elem_t*>(c.values);
    v.page_table = c.page_table;
    v.page_size = c.page_size;
    v.page_stride = c.page_stride;
    v.head_stride = c.head_stride;
    v.num_kv_heads = c.num_kv_heads;
    v.head_dim = c.head_dim;
    return v;
  }
};

class KvCache {
 public:
  KvCache(const ModelConfig& config, int max_seq, KvLayout layout, int page_size = 16);
  ~KvCache();
  KvCache(const KvCache&) = delete;
  KvCache& operator=(const KvCache&) = delete;

  // Makes room for `length` positions: a bound check when contiguous; maps the
  // pages that length needs, in order, when paged. Synchronous (page-table
  // upload), so it is called outside any captured graph.
  void reserve_length(int length);

  KvCacheView view(int layer) const;

  KvLayout layout() const { return layout_; }
  int page_size() const { return page_size_; }
  int max_seq() const { return max_seq_; }
  int length() const { return length_; }
  int max_pages() const { return max_pages_; }
  int pool_pages() const { return pool_pages_; }

  size_t allocated_bytes() const { return allocated_bytes_; }
  size_t live_bytes() const;
  size_t ideal_bytes() const;
  std::string usage_string() const;

  static size_t bytes_for(const ModelConfig& config, int64_t positions);

  // Test and benchmark hook, not in the reference: replaces the page table of
  // every layer with `tables` ([num_layers][max_pages] physical page ids, each
  // a distinct page of the pool) and marks `length` positions as present. Used
  // for the long-context stress case, whose block table is a seeded random
  // permutation of the pool rather than the reference's in-order assignment.
  void set_page_tables(const std::vector<int32_t>& tables, int length);
  // Raw pools, for filling the cache directly in that stress case.
  elem_t* key_pool() const { return key_pool_; }
  elem_t* value_pool() const { return value_pool_; }
  size_t pool_elements() const { return pool_elements_; }

 private:
  size_t layer_elements() const;

  ModelConfig config_;
  KvLayout layout_;
  int max_seq_ = 0;
  int page_size_ = 0;
  int length_ = 0;

  elem_t* key_pool_ = nullptr;
  elem_t* value_pool_ = nullptr;
  size_t pool_elements_ = 0;
  size_t allocated_bytes_ = 0;

  int32_t* page_tables_device_ = nullptr;
  std::vector<int32_t> page_tables_host_;
  int max_pages_ = 0;
  int pool_pages_ = 0;
  int pages_mapped_ = 0;
};

}  // namespace lcr
