// safetensors reading and writing.
//
// Reading is two steps. locate_shards() turns a checkpoint directory into the
// list of files to map: model.safetensors alone, or the distinct shard names of
// model.safetensors.index.json's weight_map in first-mention order. Each file
// is then mapped whole and its header is read into TensorViews pointing into
// the mapping; every view is checked against the file (span inside the data
// buffer, span equal to shape x dtype size) before anything can upload it.
// The format rules and the refusal messages follow the reference's loader
// (src/safetensors.cpp:217-322; its tests match the message substrings).
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
#include <iterator>
#include <sstream>
#include <utility>

#include "json.h"

namespace lcr {
namespace {

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__,
              "the header length is read as a native little-endian integer");

// The format's own bound on the header (100 MB); a larger length is a
// corrupt file, not a checkpoint.
constexpr uint64_t kMaxHeaderBytes = 100'000'000;
constexpr size_t kLengthPrefix = 8;

std::string in_dir(const std::string& dir, const std::string& name) {
  if (dir.empty()) return name;
  return dir + (dir.back() == '/' ? "" : "/") + name;
}

bool regular_file(const std::string& path) {
  struct stat st {};
  return ::stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

std::string bracketed(const std::vector<int64_t>& dims) {
  std::string out = "[";
  for (size_t i = 0; i < dims.size(); ++i) {
    if (i > 0) out += ", ";
    out += std::to_string(dims[i]);
  }
  return out + "]";
}

// The files a checkpoint directory's tensors live in.
std::vector<std::string> locate_shards(const std::string& dir) {
  const std::string single = in_dir(dir, "model.safetensors");
  if (regular_file(single)) return {single};
  const std::string index_path = in_dir(dir, "model.safetensors.index.json");
  LCR_CHECK(regular_file(index_path), "no model.safetensors or model.safetensors.index.json in " << dir);

  std::ifstream in(index_path, std::ios::binary);
  const std::string text((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  LCR_CHECK(in.good() || in.eof(), "cannot read " << index_path);
  json::Value index;
  LCR_CHECK(json::parse(text, &index, nullptr), index_path << " is not valid JSON");
  const json::Value* weight_map = index.is_object() ? index.find("weight_map") : nullptr;
  LCR_CHECK(weight_map != nullptr && weight_map->is_object(), index_path << " has no weight_map object");

  std::vector<std::string> shards;
  for (const auto& [tensor, file] : weight_map->members()) {
    LCR_CHECK(file.is_string(), "weight_map entry for \"" << tensor << "\" is not a filename");
    const std::string path = in_dir(dir, file.as_string());
    if (std::find(shards.begin(), shards.end(), path) == shards.end()) shards.push_back(path);
  }
  return shards;
}

// A non-negative integer list (shape or offsets); false if anything else.
bool read_extents(const json::Value* v, std::vector<int64_t>* out) {
  if (v == nullptr || !v->is_array()) return false;
  out->clear();
  for (const json::Value& item : v->items()) {
    if (!item.is_integer() || item.as_int64() < 0) return false;
    out->push_back(item.as_int64());
  }
  return true;
}

// One header entry, checked against the data buffer [payload, payload + size).
TensorView describe(const std::string& file, const std::string& name, const json::Value& entry,
                    const uint8_t* payload, size_t payload_size) {
  LCR_CHECK(entry.is_object(), "tensor \"" << name << "\" in " << file << " is not described by an object");
  const json::Value* dtype = entry.find("dtype");
  const json::Value* shape = entry.find("shape");
  const json::Value* offsets = entry.find("data_offsets");
  LCR_CHECK(dtype != nullptr && shape != nullptr && offsets != nullptr,
            "tensor \"" << name << "\" in " << file << " is missing dtype, shape, or data_offsets");
  LCR_CHECK(dtype->is_string(), "tensor \"" << name << "\" in " << file << " has a non-string dtype");

  TensorView t;
  t.name = name;
  t.dtype = dtype_from_string(dtype->as_string());
  LCR_CHECK(read_extents(shape, &t.shape), "tensor \"" << name << "\" in " << file << " has a malformed shape");
  std::vector<int64_t> span;
  LCR_CHECK(read_extents(offsets, &span) && span.size() == 2 && span[0] <= span[1],
            "tensor \"" << name << "\" in " << file << " has malformed data_offsets");
  const size_t first = static_cast<size_t>(span[0]);
  const size_t last = static_cast<size_t>(span[1]);
  LCR_CHECK(last <= payload_size, "tensor \"" << name << "\" ends at byte " << last << " of the data buffer of "
                                              << file << ", which holds " << payload_size);
  t.nbytes = last - first;
  const size_t wanted = static_cast<size_t>(t.numel()) * dtype_size(t.dtype);
  LCR_CHECK(t.nbytes == wanted, "tensor \"" << name << "\" covers " << t.nbytes << " bytes; "
                                            << dtype_name(t.dtype) << " " << t.shape_string() << " needs "
                                            << wanted);
  t.data = payload + first;
  return t;
}

}  // namespace

int64_t TensorView::numel() const {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

int64_t TensorView::dim(int index) const {
  LCR_CHECK(index >= 0 && index < rank(),
            "tensor \"" << name << "\" has rank " << rank() << ", no dimension " << index);
  return shape[static_cast<size_t>(index)];
}

std::string TensorView::shape_string() const { return bracketed(shape); }

void TensorView::expect_shape(std::initializer_list<int64_t> expected) const {
  expect_shape(std::vector<int64_t>(expected));
}

void TensorView::expect_shape(const std::vector<int64_t>& expected) const {
  LCR_CHECK(shape == expected,
            "tensor \"" << name << "\" is " << shape_string() << ", expected " << bracketed(expected));
}

MappedFile::MappedFile(const std::string& path) : path_(path) {
  // The descriptor is closed on every way out, mapped or not.
  struct Descriptor {
    int fd;
    ~Descriptor() {
      if (fd >= 0) ::close(fd);
    }
  } file{::open(path.c_str(), O_RDONLY | O_CLOEXEC)};
  LCR_CHECK(file.fd >= 0, "cannot open " << path << ": " << std::strerror(errno));
  struct stat st {};
  LCR_CHECK(::fstat(file.fd, &st) == 0, "cannot stat " << path << ": " << std::strerror(errno));
  const size_t bytes = static_cast<size_t>(st.st_size);
  LCR_CHECK(bytes > kLengthPrefix, path << " holds " << bytes << " bytes, too few for a safetensors file");
  void* map = ::mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, file.fd, 0);
  LCR_CHECK(map != MAP_FAILED, "cannot mmap " << path << ": " << std::strerror(errno));
  base_ = static_cast<uint8_t*>(map);
  size_ = bytes;
  // A mapping stays valid after its descriptor is closed.
}

MappedFile::~MappedFile() {
  if (base_ != nullptr) ::munmap(base_, size_);
}

SafetensorsArchive::SafetensorsArchive(const std::string& model_dir) : dir_(model_dir) {
  for (const std::string& path : locate_shards(dir_)) open_file(path);
  LCR_CHECK(!tensors_.empty(), "checkpoint in " << dir_ << " has no tensors");
}

void SafetensorsArchive::open_file(const std::string& path) {
  files_.push_back(std::make_unique<MappedFile>(path));
  const MappedFile& file = *files_.back();

  uint64_t header_bytes = 0;
  std::memcpy(&header_bytes, file.data(), kLengthPrefix);
  LCR_CHECK(header_bytes >= 2 && header_bytes <= kMaxHeaderBytes,
            path << " declares a header of " << header_bytes << " bytes, which no checkpoint has");
  LCR_CHECK(header_bytes <= file.size() - kLengthPrefix,
            path << " header length " << header_bytes << " exceeds the file size " << file.size());

  const char* header_text = reinterpret_cast<const char*>(file.data() + kLengthPrefix);
  json::Value header;
  LCR_CHECK(json::parse(header_text, header_text + header_bytes, &header, nullptr) && header.is_object(),
            path << " has a malformed JSON header");

  const uint8_t* payload = file.data() + kLengthPrefix + header_bytes;
  const size_t payload_size = file.size() - kLengthPrefix - header_bytes;
  for (const auto& [name, entry] : header.members()) {
    if (name == "__metadata__") continue;  // free-form strings, not a tensor
    TensorView t = describe(path, name, entry, payload, payload_size);
    LCR_CHECK(tensors_.emplace(name, std::move(t)).second,
              "tensor \"" << name << "\" is defined twice (again in " << path << ")");
  }
}

const TensorView* SafetensorsArchive::find(const std::string& name) const {
  const auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

const TensorView& SafetensorsArchive::get(const std::string& name) const {
  if (const TensorView* t = find(name)) return *t;
  LCR_FAIL("checkpoint in " << dir_ << " has no tensor named \"" << name << "\"");
}

std::vector<std::string> SafetensorsArchive::names() const {
  std::vector<std::string> out;
  out.reserve(tensors_.size());
  std::transform(tensors_.begin(), tensors_.end(), std::back_inserter(out),
                 [](const auto& entry) { return entry.first; });
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
