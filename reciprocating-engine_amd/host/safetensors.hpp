// safetensors.hpp - a read-only, memory-mapped view of a checkpoint's
// safetensors files (model.safetensors, or the shards that
// model.safetensors.index.json lists), the loader the reference's reng-model
// builds on (crates/reng-model/src/lib.rs:1372-1461).
//
// File layout: 8-byte little-endian header length H, H bytes of JSON
// ({"name": {"dtype", "shape", "data_offsets": [begin, end]}, ...,
// "__metadata__": {...}}), then the data; offsets count from the end of the
// header. Every header entry is validated (dtype size x shape == the byte
// range, the range inside the file) before a tensor is handed out.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace reng_model {

// Loader and configuration failures (the reference's Error::Other).
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// A read-only private mapping of a whole file.
class Mapping {
public:
    explicit Mapping(const std::string &path);
    ~Mapping();
    Mapping(const Mapping &) = delete;
    Mapping &operator=(const Mapping &) = delete;
    const uint8_t *data() const { return data_; }
    size_t size() const { return size_; }
    const std::string &path() const { return path_; }

private:
    std::string path_;
    const uint8_t *data_ = nullptr;
    size_t size_ = 0;
};

// The bf16 elements of a weight tensor (the reference's Bf16Slice,
// lib.rs:745-966): a view into a mapped file when the tensor is bf16 at a
// 2-aligned offset (nothing is copied), otherwise an owned buffer (an f32 or
// f16 tensor converted with round-to-nearest-even, or an unaligned bf16 one).
// Copies share the storage.
class Bf16Slice {
public:
    Bf16Slice() = default;
    static Bf16Slice mapped(std::shared_ptr<const Mapping> map, size_t offset, size_t len);
    static Bf16Slice owned(std::vector<uint16_t> v);

    const uint16_t *data() const { return data_; }
    size_t size() const { return len_; }
    bool empty() const { return len_ == 0; }
    uint16_t operator[](size_t i) const { return data_[i]; }
    // Viewed in place in a mapped file.
    bool is_mapped() const { return mapped_; }
    // Bytes held in a buffer of its own (0 for a mapped view).
    size_t owned_bytes() const { return mapped_ ? 0 : len_ * 2; }
    // Elements [start, start + len) as a slice of their own (a sub-view;
    // shares the storage).
    Bf16Slice sub(size_t start, size_t len) const;
    std::vector<uint16_t> to_vector() const { return std::vector<uint16_t>(data_, data_ + len_); }

private:
    std::shared_ptr<const void> owner_;
    const uint16_t *data_ = nullptr;
    size_t len_ = 0;
    bool mapped_ = false;
};

enum class Dtype { BF16, F16, F32, U8, Other };

struct TensorInfo {
    std::string name;
    Dtype dtype = Dtype::Other;
    std::string dtype_name;
    std::vector<size_t> shape;
    size_t begin = 0, end = 0;   // absolute byte offsets in the file
    size_t shard = 0;
};

// One or several mapped safetensors files and their parsed headers.
class Checkpoint {
public:
    // Opens dir/model.safetensors, or the shards dir/model.safetensors.index.json
    // names.
    static Checkpoint open(const std::string &dir);
    // A single file.
    static Checkpoint open_file(const std::string &path);

    bool has(const std::string &name) const { return tensors_.count(name) != 0; }
    const TensorInfo &info(const std::string &name) const;
    std::vector<std::string> names() const;

    // The tensor as bf16 (bf16 in place; f32 / f16 converted).
    Bf16Slice bf16(const std::string &name) const;
    // The tensor as f32 (bf16 / f16 / f32).
    std::vector<float> f32(const std::string &name) const;
    // A [out, in] linear weight, shape-checked (lib.rs:1361-1370).
    Bf16Slice linear(const std::string &name, size_t out_dim, size_t in_dim) const;
    // A U8 tensor's bytes.
    std::vector<uint8_t> u8(const std::string &name) const;
    // The string entries of the files' __metadata__ objects.
    const std::map<std::string, std::string> &metadata() const { return metadata_; }
    // The files the tensors come from, in the order they were opened.
    const std::vector<std::string> &files() const { return paths_; }

private:
    void add_file(const std::string &path, const std::map<std::string, bool> *only);
    std::vector<std::shared_ptr<const Mapping>> files_;
    std::map<std::string, TensorInfo> tensors_;
    std::map<std::string, std::string> metadata_;
    std::vector<std::string> paths_;
};

// One tensor for write_safetensors: dtype "BF16", "F16", "F32" or "U8"; bytes
// must be the shape's element count times the element size.
struct TensorOut {
    std::string name, dtype;
    std::vector<size_t> shape;
    const void *data = nullptr;
    size_t bytes = 0;
};

// Writes a safetensors file (tensors in the given order, no holes, header
// padded to 8 bytes, metadata as the header's __metadata__ strings) to
// path + ".tmp" and renames it over path. Throws Error on an I/O failure.
void write_safetensors(const std::string &path, const std::vector<TensorOut> &tensors,
                       const std::map<std::string, std::string> &metadata);

// bf16 / f16 helpers shared by the loader.
float f16_to_f32(uint16_t h);

}  // namespace reng_model
