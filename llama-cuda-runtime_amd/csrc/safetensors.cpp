#include "safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <set>
#include <sstream>

#include "json.h"

namespace lcr {
namespace {

// Larger headers than this are a corrupt or hostile file, not a checkpoint.
constexpr uint64_t kHeaderLimit = 32ull << 20;

uint64_t load_le64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
  return v;
}

bool is_regular_file(const std::string& path) {
  struct stat st;
  return ::stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

std::string path_join(const std::string& dir, const std::string& name) {
  if (dir.empty()) return name;
  return dir.back() == '/' ? dir + name : dir + "/" + name;
}

std::string shape_text(const std::vector<int64_t>& shape) {
  std::ostringstream oss;
  oss << "[";
  for (size_t i = 0; i < shape.size(); ++i) oss << (i ? ", " : "") << shape[i];
  oss << "]";
  return oss.str();
}

bool int_list(const json::Value& v, std::vector<int64_t>* out) {
  if (!v.is_array()) return false;
  out->clear();
  for (const json::Value& item : v.items()) {
    if (!item.is_integer()) return false;
    out->push_back(item.as_int64());
  }
  return true;
}

}  // namespace

int64_t TensorView::numel() const {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

int64_t TensorView::dim(int index) const {
  LCR_CHECK(index >= 0 && index < rank(), "dim " << index << " out of range for tensor \""
                                                  << name << "\" of rank " << rank());
  return shape[static_cast<size_t>(index)];
}

std::string TensorView::shape_string() const { return shape_text(shape); }

void TensorView::expect_shape(std::initializer_list<int64_t> expected) const {
  expect_shape(std::vector<int64_t>(expected));
}

void TensorView::expect_shape(const std::vector<int64_t>& expected) const {
  LCR_CHECK(expected == shape, "tensor \"" << name << "\" has shape " << shape_string()
                                           << ", expected " << shape_text(expected));
}

MappedFile::MappedFile(const std::string& path) : path_(path) {
  fd_ = ::open(path.c_str(), O_RDONLY);
  LCR_CHECK(fd_ >= 0, "cannot open " << path << ": " << std::strerror(errno));
  struct stat st;
  if (::fstat(fd_, &st) != 0) {
    const int err = errno;
    ::close(fd_);
    fd_ = -1;
    LCR_FAIL("cannot stat " << path << ": " << std::strerror(err));
  }
  size_ = static_cast<size_t>(st.st_size);
  if (size_ <= 8) {
    ::close(fd_);
    fd_ = -1;
    LCR_FAIL(path << " is too small to be a safetensors file (" << size_ << " bytes)");
  }
  void* map = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
  if (map == MAP_FAILED) {
    const int err = errno;
    ::close(fd_);
    fd_ = -1;
    LCR_FAIL("cannot mmap " << path << ": " << std::strerror(err));
  }
  base_ = static_cast<uint8_t*>(map);
}

MappedFile::~MappedFile() {
  if (base_ != nullptr) ::munmap(base_, size_);
  if (fd_ >= 0) ::close(fd_);
}

SafetensorsArchive::SafetensorsArchive(const std::string& model_dir) : dir_(model_dir) {
  const std::string single = path_join(dir_, "model.safetensors");
  const std::string index = path_join(dir_, "model.safetensors.index.json");
  if (is_regular_file(single)) {
    open_file(single);
  } else if (is_regular_file(index)) {
    std::ifstream in(index, std::ios::binary);
    LCR_CHECK(in.good(), "cannot read " << index);
    std::ostringstream buffer;
    buffer << in.rdbuf();
    json::Value doc;
    LCR_CHECK(json::parse(buffer.str(), &doc, nullptr), index << " is not valid JSON");
    const json::Value* map = doc.find("weight_map");
    LCR_CHECK(map != nullptr && map->is_object(), index << " has no weight_map object");
    std::set<std::string> shards;
    for (const auto& member : map->members()) {
      LCR_CHECK(member.second.is_string(),
                "weight_map entry for \"" << member.first << "\" is not a filename");
      shards.insert(member.second.as_string());
    }
    for (const std::string& shard : shards) open_file(path_join(dir_, shard));
  } else {
    LCR_FAIL("no model.safetensors or model.safetensors.index.json in " << dir_);
  }
  LCR_CHECK(!tensors_.empty(), "checkpoint in " << dir_ << " has no tensors");
}

void SafetensorsArchive::open_file(const std::string& path) {
  files_.push_back(std::make_unique<MappedFile>(path));
  const MappedFile& file = *files_.back();
  const uint8_t* base = file.data();
  const size_t size = file.size();

  const uint64_t header_len = load_le64(base);
  LCR_CHECK(header_len > 0 && header_len <= kHeaderLimit,
            path << " declares an implausible header length of " << header_len << " bytes");
  LCR_CHECK(8 + header_len <= size,
            path << " header length " << header_len << " exceeds the file size " << size);

  json::Value header;
  const char* text = reinterpret_cast<const char*>(base + 8);
  LCR_CHECK(json::parse(text, text + header_len, &header, nullptr),
            path << " has a malformed JSON header");
  LCR_CHECK(header.is_object(), path << " header is not a JSON object");

  const uint8_t* payload = base + 8 + header_len;
  const size_t payload_size = size - 8 - header_len;

  for (const auto& member : header.members()) {
    const std::string& name = member.first;
    if (name == "__metadata__") continue;
    const json::Value& spec = member.second;
    LCR_CHECK(spec.is_object(),
              "tensor \"" << name << "\" in " << path << " is not described by an object");
    const json::Value* dtype = spec.find("dtype");
    const json::Value* shape = spec.find("shape");
    const json::Value* offsets = spec.find("data_offsets");
    LCR_CHECK(dtype != nullptr && shape != nullptr && offsets != nullptr,
              "tensor \"" << name << "\" in " << path
                          << " is missing dtype, shape, or data_offsets");
    LCR_CHECK(dtype->is_string(), "tensor \"" << name << "\" has a non-string dtype");

    TensorView view;
    view.name = name;
    view.dtype = dtype_from_string(dtype->as_string());
    LCR_CHECK(int_list(*shape, &view.shape), "tensor \"" << name << "\" has a malformed shape");
    for (int64_t d : view.shape) {
      LCR_CHECK(d >= 0, "tensor \"" << name << "\" has negative extent " << d);
    }
    std::vector<int64_t> range;
    LCR_CHECK(int_list(*offsets, &range) && range.size() == 2,
              "tensor \"" << name << "\" has malformed data_offsets");
    const int64_t begin = range[0];
    const int64_t end = range[1];
    LCR_CHECK(begin >= 0 && end >= begin,
              "tensor \"" << name << "\" has data_offsets [" << begin << ", " << end << "]");
    LCR_CHECK(static_cast<size_t>(end) <= payload_size,
              "tensor \"" << name << "\" ends at " << end << " but the data buffer of "
                          << path << " is only " << payload_size << " bytes");
    view.nbytes = static_cast<size_t>(end - begin);
    const size_t expected = static_cast<size_t>(view.numel()) * dtype_size(view.dtype);
    LCR_CHECK(view.nbytes == expected,
              "tensor \"" << name << "\" spans " << view.nbytes << " bytes but its shape "
                          << view.shape_string() << " of " << dtype_name(view.dtype)
                          << " needs " << expected);
    view.data = payload + begin;
    const bool inserted = tensors_.emplace(name, std::move(view)).second;
    LCR_CHECK(inserted, "tensor \"" << name << "\" appears in more than one shard");
  }
}

const TensorView* SafetensorsArchive::find(const std::string& name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

const TensorView& SafetensorsArchive::get(const std::string& name) const {
  const TensorView* view = find(name);
  LCR_CHECK(view != nullptr, "checkpoint has no tensor named \"" << name << "\"");
  return *view;
}

std::vector<std::string> SafetensorsArchive::names() const {
  std::vector<std::string> out;
  out.reserve(tensors_.size());
  for (const auto& entry : tensors_) out.push_back(entry.first);
  std::sort(out.begin(), out.end());
  return out;
}

size_t SafetensorsArchive::total_bytes() const {
  size_t total = 0;
  for (const auto& entry : tensors_) total += entry.second.nbytes;
  return total;
}

void write_safetensors(
    const std::string& path, const std::vector<TensorSpec>& tensors,
    const std::function<void(size_t index, void* dst, size_t nbytes)>& fill) {
  json::Value header = json::Value::object();
  std::vector<size_t> sizes;
  size_t offset = 0;
  for (const TensorSpec& t : tensors) {
    size_t n = dtype_size(t.dtype);
    json::Value shape = json::Value::array();
    for (int64_t d : t.shape) {
      LCR_CHECK(d >= 0, "tensor \"" << t.name << "\" has negative extent " << d);
      n *= static_cast<size_t>(d);
      shape.push_back(json::Value::integer(d));
    }
    json::Value entry = json::Value::object();
    entry.set("dtype", json::Value::string(dtype_name(t.dtype)));
    entry.set("shape", shape);
    json::Value range = json::Value::array();
    range.push_back(json::Value::integer(static_cast<int64_t>(offset)));
    range.push_back(json::Value::integer(static_cast<int64_t>(offset + n)));
    entry.set("data_offsets", range);
    header.set(t.name, entry);
    sizes.push_back(n);
    offset += n;
  }
  std::string text = header.dump();
  // Pad the header with spaces so the data buffer starts 8-byte aligned, which
  // the format recommends and which keeps every bf16 tensor aligned when mapped.
  while ((8 + text.size()) % 8 != 0) text.push_back(' ');

  const std::string tmp = path + ".tmp";
  FILE* f = std::fopen(tmp.c_str(), "wb");
  LCR_CHECK(f != nullptr, "cannot create " << tmp << ": " << std::strerror(errno));
  uint8_t len[8];
  uint64_t header_len = text.size();
  for (int i = 0; i < 8; ++i) len[i] = static_cast<uint8_t>(header_len >> (8 * i));
  bool ok = std::fwrite(len, 1, 8, f) == 8 &&
            std::fwrite(text.data(), 1, text.size(), f) == text.size();
  std::vector<uint8_t> buffer;
  for (size_t i = 0; ok && i < tensors.size(); ++i) {
    buffer.resize(sizes[i]);
    fill(i, buffer.data(), sizes[i]);
    ok = std::fwrite(buffer.data(), 1, sizes[i], f) == sizes[i];
  }
  ok = (std::fclose(f) == 0) && ok;
  if (!ok) {
    std::remove(tmp.c_str());
    LCR_FAIL("failed writing " << path);
  }
  LCR_CHECK(std::rename(tmp.c_str(), path.c_str()) == 0,
            "cannot rename " << tmp << " to " << path << ": " << std::strerror(errno));
}

}  // namespace lcr
