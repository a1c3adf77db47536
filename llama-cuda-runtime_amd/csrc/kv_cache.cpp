#include "kv_cache.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <sstream>

#include "hip_utils.h"

namespace lcr {

void KvCache::HipFree::operator()(void* p) const { (void)hipFree(p); }

KvGeometry KvGeometry::plan(const ModelConfig& config, int max_seq, KvLayout layout, int page_size) {
  LCR_CHECK(max_seq > 0, "KV cache needs a positive maximum sequence length");
  KvGeometry g;
  g.layout = layout;
  g.num_layers = config.num_layers;
  g.num_kv_heads = config.num_kv_heads;
  g.head_dim = config.head_dim;
  g.max_seq = max_seq;
  if (layout == KvLayout::kContiguous) {
    // One page of max_seq positions per layer, addressed without a table.
    g.page_size = max_seq;
    g.pages_per_layer = 0;
    g.pool_pages = g.num_layers;
  } else {
    LCR_CHECK(page_size > 0, "paged KV cache needs a positive page size");
    g.page_size = page_size;
    g.pages_per_layer = (max_seq + page_size - 1) / page_size;
    // Enough pages for every layer to reach max_seq: one sequence can never
    // exhaust the pool.
    g.pool_pages = g.pages_per_layer * g.num_layers;
  }
  g.page_elements = static_cast<size_t>(g.num_kv_heads) * static_cast<size_t>(g.page_size) *
                    static_cast<size_t>(g.head_dim);
  return g;
}

size_t KvCache::bytes_for(const ModelConfig& config, int64_t positions) {
  return static_cast<size_t>(positions) * config.kv_bytes_per_token(sizeof(elem_t));
}

KvCache::KvCache(const ModelConfig& config, int max_seq, KvLayout layout, int page_size)
    : geo_(KvGeometry::plan(config, max_seq, layout, page_size)) {
  const size_t pool_bytes = geo_.pool_elements() * sizeof(elem_t);
  const size_t table_bytes = geo_.table_entries() * sizeof(int32_t);
  // [keys | values | tables], each region starting on a 256-byte boundary.
  const size_t values_at = align_up(pool_bytes, 256);
  const size_t tables_at = values_at + align_up(pool_bytes, 256);
  const size_t total = tables_at + table_bytes;
  void* p = nullptr;
  HIP_CHECK(hipMalloc(&p, total));
  block_.reset(static_cast<unsigned char*>(p));
  keys_ = reinterpret_cast<elem_t*>(block_.get());
  values_ = reinterpret_cast<elem_t*>(block_.get() + values_at);
  tables_ = table_bytes > 0 ? reinterpret_cast<int32_t*>(block_.get() + tables_at) : nullptr;
  // Only written positions are ever read; zeroed pools make a stray read
  // return zeros instead of another allocation's leftovers.
  HIP_CHECK(hipMemset(block_.get(), 0, tables_at));
  host_tables_.assign(geo_.table_entries(), -1);
  if (!host_tables_.empty()) upload_tables(0, host_tables_.size());
  allocated_bytes_ = 2 * pool_bytes + table_bytes;
}

KvCache::~KvCache() = default;

void KvCache::upload_tables(size_t first, size_t count) {
  if (count == 0) return;
  HIP_CHECK(hipMemcpy(tables_ + first, host_tables_.data() + first, count * sizeof(int32_t),
                      hipMemcpyHostToDevice));
}

void KvCache::reserve_length(int length) {
  LCR_CHECK(length <= geo_.max_seq, "sequence reached " << length
                                        << " positions but the KV cache was built for " << geo_.max_seq);
  if (length <= length_) return;
  if (geo_.layout == KvLayout::kPaged) {
    const int from = (length_ + geo_.page_size - 1) / geo_.page_size;
    const int to = (length + geo_.page_size - 1) / geo_.page_size;
    if (to > from) {
      for (int layer = 0; layer < geo_.num_layers; ++layer) {
        int32_t* row = host_tables_.data() + static_cast<size_t>(layer) * geo_.pages_per_layer;
        for (int page = from; page < to; ++page) {
          if (row[page] >= 0) continue;  // already placed by set_page_tables
          LCR_CHECK(next_page_ < geo_.pool_pages,
                    "paged KV cache pool is exhausted after " << next_page_ << " pages");
          row[page] = next_page_++;
        }
      }
      // One copy covers the changed entries of every layer (and the unchanged
      // ones between them, which the mirror holds too).
      const size_t first = static_cast<size_t>(from);
      const size_t last = static_cast<size_t>(geo_.num_layers - 1) * geo_.pages_per_layer + to;
      upload_tables(first, last - first);
    }
  }
  length_ = length;
}

KvCacheView KvCache::view(int layer) const {
  LCR_CHECK(layer >= 0 && layer < geo_.num_layers, "layer " << layer << " is out of range");
  const bool paged = geo_.layout == KvLayout::kPaged;
  // Contiguous: the layer's own page; paged: the whole pool plus its table.
  const size_t base = paged ? 0 : static_cast<size_t>(layer) * geo_.page_elements;
  KvCacheView v;
  v.keys = keys_ + base;
  v.values = values_ + base;
  v.page_table = paged ? tables_ + static_cast<size_t>(layer) * geo_.pages_per_layer : nullptr;
  v.page_size = geo_.page_size;
  v.page_stride = paged ? static_cast<int>(geo_.page_elements) : 0;
  v.head_stride = geo_.page_size * geo_.head_dim;
  v.num_kv_heads = geo_.num_kv_heads;
  v.head_dim = geo_.head_dim;
  return v;
}

void KvCache::set_page_tables(const std::vector<int32_t>& tables, int length) {
  LCR_CHECK(geo_.layout == KvLayout::kPaged, "set_page_tables needs the paged layout");
  LCR_CHECK(tables.size() == host_tables_.size(),
            "page tables hold " << tables.size() << " entries, expected " << host_tables_.size());
  LCR_CHECK(length >= 0 && length <= geo_.max_seq, "length " << length << " out of range");
  const int needed = (length + geo_.page_size - 1) / geo_.page_size;
  std::vector<char> used(static_cast<size_t>(geo_.pool_pages), 0);
  for (size_t i = 0; i < tables.size(); ++i) {
    const int32_t page = tables[i];
    const int index_in_layer = static_cast<int>(i % static_cast<size_t>(geo_.pages_per_layer));
    LCR_CHECK(page >= 0 || index_in_layer >= needed,
              "page " << index_in_layer << " of a layer is unmapped but " << length << " positions are present");
    if (page < 0) continue;
    LCR_CHECK(page < geo_.pool_pages, "page id " << page << " outside the pool");
    LCR_CHECK(!used[static_cast<size_t>(page)], "physical page " << page << " is mapped twice");
    used[static_cast<size_t>(page)] = 1;
  }
  host_tables_ = tables;
  upload_tables(0, host_tables_.size());
  // Pages handed out later come after every id in use.
  const int32_t highest = *std::max_element(host_tables_.begin(), host_tables_.end());
  next_page_ = std::max(next_page_, highest + 1);
  length_ = std::max(length_, length);
}

namespace {
// K and V bytes of one position across every layer.
size_t position_bytes(const KvGeometry& g) {
  return 2 * static_cast<size_t>(g.num_layers) * static_cast<size_t>(g.num_kv_heads) *
         static_cast<size_t>(g.head_dim) * sizeof(elem_t);
}
}  // namespace

size_t KvCache::ideal_bytes() const { return static_cast<size_t>(length_) * position_bytes(geo_); }

size_t KvCache::live_bytes() const {
  if (geo_.layout == KvLayout::kContiguous) return static_cast<size_t>(geo_.max_seq) * position_bytes(geo_);
  // A handed-out page holds page_size positions of one layer, keys and values.
  return static_cast<size_t>(next_page_) * 2 * geo_.page_elements * sizeof(elem_t);
}

std::string KvCache::usage_string() const {
  const size_t live = live_bytes();
  const size_t ideal = ideal_bytes();
  std::ostringstream text;
  if (geo_.layout == KvLayout::kPaged) {
    text << "paged KV, " << geo_.page_size << "-position pages, " << next_page_ << " of " << geo_.pool_pages
         << " pages mapped";
  } else {
    text << "contiguous KV, " << geo_.max_seq << " positions per layer";
  }
  text << "; " << length_ << " positions hold " << format_bytes(ideal) << " in " << format_bytes(live)
       << " committed";
  if (live > ideal) {
    text << " (" << 100.0 * static_cast<double>(live - ideal) / static_cast<double>(live) << "% slack)";
  }
  return text.str();
}

}  // namespace lcr
