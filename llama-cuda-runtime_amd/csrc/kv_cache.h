// Key/value cache of the token loop, contiguous or paged.
//
// Interface of the reference's KvCache and KvCacheView
// (src/kv_cache.cuh:30-118): KvLayout, the view's fields and its offset
// formula (the addressing contract between the KV append and attention),
// reserve_length, view(layer), and the byte accounting.
//
// Design. Both layouts are one geometry (KvGeometry): a page holds
// [kv_head][page_size][head_dim] elements, and the contiguous layout is the
// case of one page of max_seq positions per layer (page_stride 0, no table).
// Keys, values and the page tables live in one device block, allocated once;
// the tables are mirrored on the host, which hands out pages in the
// reference's order (sequentially, layer after layer, as positions are
// reserved: src/kv_cache.cu:84-92) and uploads the changed span of all layers
// in one copy.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "../../include/lcr_kernels.h"
#include "config.h"
#include "dtype.h"

namespace lcr {

enum class KvLayout { kContiguous, kPaged };

// Non-owning, trivially copyable handle to one layer; the fields and order of
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

  // Element offset of (head, position): page * page_stride + head *
  // head_stride + slot * head_dim (src/kv_cache.cuh:49-56).
  template <bool kPaged>
  __host__ __device__ __forceinline__ size_t offset(int head, int position) const {
    const int page = kPaged ? page_table[position / page_size] : 0;
    const int slot = kPaged ? position % page_size : position;
    return static_cast<size_t>(page) * static_cast<size_t>(page_stride) +
           static_cast<size_t>(head) * static_cast<size_t>(head_stride) +
           static_cast<size_t>(slot) * static_cast<size_t>(head_dim);
  }

  lcr_kv_view to_c() const {
    return lcr_kv_view{keys, values, page_table, page_size, page_stride, head_stride, num_kv_heads, head_dim};
  }
  static KvCacheView from_c(const lcr_kv_view& c) {
    return KvCacheView{static_cast<elem_t*>(c.keys), static_cast<elem_t*>(c.values), c.page_table, c.page_size,
                       c.page_stride,  c.head_stride, c.num_kv_heads, c.head_dim};
  }
};

// Sizes of a cache, computed without touching the device.
struct KvGeometry {
  KvLayout layout = KvLayout::kContiguous;
  int num_layers = 0;
  int num_kv_heads = 0;
  int head_dim = 0;
  int max_seq = 0;
  int page_size = 0;        // positions per page (max_seq when contiguous)
  int pages_per_layer = 0;  // table entries per layer (0 when contiguous)
  int pool_pages = 0;       // pages in each of the K and V pools
  size_t page_elements = 0; // num_kv_heads * page_size * head_dim
  size_t pool_elements() const { return static_cast<size_t>(pool_pages) * page_elements; }
  size_t table_entries() const { return static_cast<size_t>(num_layers) * pages_per_layer; }

  static KvGeometry plan(const ModelConfig& config, int max_seq, KvLayout layout, int page_size);
};

class KvCache {
 public:
  KvCache(const ModelConfig& config, int max_seq, KvLayout layout, int page_size = 16);
  ~KvCache();
  KvCache(const KvCache&) = delete;
  KvCache& operator=(const KvCache&) = delete;

  // Makes `length` positions addressable: a bound check when contiguous; in the
  // paged layout, maps the pages that length needs in every layer. Blocking
  // (it uploads table entries), so it runs outside any captured graph.
  void reserve_length(int length);

  KvCacheView view(int layer) const;

  KvLayout layout() const { return geo_.layout; }
  const KvGeometry& geometry() const { return geo_; }
  int page_size() const { return geo_.page_size; }
  int max_seq() const { return geo_.max_seq; }
  int length() const { return length_; }
  int max_pages() const { return geo_.pages_per_layer; }
  int pool_pages() const { return geo_.pool_pages; }

  size_t allocated_bytes() const { return allocated_bytes_; }
  // Bytes of the pages handed out so far (all of both pools when contiguous).
  size_t live_bytes() const;
  // Bytes `length()` positions need with no rounding to pages.
  size_t ideal_bytes() const;
  std::string usage_string() const;

  static size_t bytes_for(const ModelConfig& config, int64_t positions);

  // Test and benchmark hook, not in the reference: installs `tables`
  // ([num_layers][max_pages] physical page ids, distinct, -1 for unmapped) and
  // marks `length` positions present, so a cache can be laid out as a seeded
  // random permutation of the pool instead of in handout order.
  void set_page_tables(const std::vector<int32_t>& tables, int length);
  // Raw pools, for filling a cache directly.
  elem_t* key_pool() const { return keys_; }
  elem_t* value_pool() const { return values_; }
  size_t pool_elements() const { return geo_.pool_elements(); }

 private:
  void upload_tables(size_t first, size_t count);

  struct HipFree {
    void operator()(void* p) const;
  };

  KvGeometry geo_;
  int length_ = 0;
  std::unique_ptr<unsigned char, HipFree> block_;
  elem_t* keys_ = nullptr;
  elem_t* values_ = nullptr;
  int32_t* tables_ = nullptr;        // device, [num_layers][pages_per_layer]
  std::vector<int32_t> host_tables_; // mirror
  int next_page_ = 0;                // next physical page to hand out
  size_t allocated_bytes_ = 0;
};

}  // namespace lcr
