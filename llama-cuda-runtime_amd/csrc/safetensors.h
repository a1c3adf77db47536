// safetensors checkpoints: a memory-mapped reader and a streaming writer.
//
// Format: an 8-byte little-endian header length, a JSON header mapping tensor
// names to {dtype, shape, data_offsets}, then the data buffer the offsets are
// relative to. The reader keeps the interface of the reference's
// src/safetensors.h:22-86 (TensorView, MappedFile, SafetensorsArchive with
// get / find / has / names / total_bytes) and its validation rules
// (src/safetensors.cpp:217-322). The writer is this build's addition: it is how
// the seeded random-init checkpoints that the GPU path and the CPU oracle both
// read are produced.
#pragma once

#include <cstdint>
#include <functional>
#include <initializer_list>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace lcr {

struct TensorView {
  std::string name;
  DType dtype = DType::kF32;
  std::vector<int64_t> shape;
  const void* data = nullptr;
  size_t nbytes = 0;

  int64_t numel() const;
  int64_t dim(int index) const;
  int rank() const { return static_cast<int>(shape.size()); }
  std::string shape_string() const;

  void expect_shape(std::initializer_list<int64_t> expected) const;
  void expect_shape(const std::vector<int64_t>& expected) const;
};

class MappedFile {
 public:
  explicit MappedFile(const std::string& path);
  ~MappedFile();
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;

  const uint8_t* data() const { return base_; }
  size_t size() const { return size_; }
  const std::string& path() const { return path_; }

 private:
  std::string path_;
  uint8_t* base_ = nullptr;
  size_t size_ = 0;
};

class SafetensorsArchive {
 public:
  // A directory holding model.safetensors, or model.safetensors.index.json and
  // the shards it names.
  explicit SafetensorsArchive(const std::string& model_dir);

  const TensorView& get(const std::string& name) const;
  const TensorView* find(const std::string& name) const;
  bool has(const std::string& name) const { return find(name) != nullptr; }
  std::vector<std::string> names() const;
  size_t tensor_count() const { return tensors_.size(); }
  size_t total_bytes() const;

 private:
  void open_file(const std::string& path);

  std::string dir_;
  std::vector<std::unique_ptr<MappedFile>> files_;
  std::unordered_map<std::string, TensorView> tensors_;
};

// Writes one safetensors file. Tensors are declared first (name, dtype, shape),
// then their bytes are produced in declaration order by `fill`, which receives
// the tensor index and a destination buffer of exactly nbytes. The file is
// written through a temporary name and renamed into place, so a reader never
// sees a half-written checkpoint.
struct TensorSpec {
  std::string name;
  DType dtype = DType::kBF16;
  std::vector<int64_t> shape;
};

void write_safetensors(
    const std::string& path, const std::vector<TensorSpec>& tensors,
    const std::function<void(size_t index, void* dst, size_t nbytes)>& fill);

}  // namespace lcr
