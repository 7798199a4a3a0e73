// safetensors.cpp - see safetensors.hpp.
#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <fstream>
#include <set>
#include <sstream>

#include "json.hpp"
#include "reng_fp8.hpp"

namespace reng_model {

namespace {

std::string base_name(const std::string &path) {
    const size_t s = path.find_last_of('/');
    return s == std::string::npos ? path : path.substr(s + 1);
}

std::string read_text(const std::string &path) {
    std::ifstream f(path);
    if (!f) throw Error(base_name(path) + ": " + std::strerror(errno));
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

bool file_exists(const std::string &path) {
    struct stat st;
    return ::stat(path.c_str(), &st) == 0;
}

size_t dtype_size(Dtype d) {
    switch (d) {
        case Dtype::BF16:
        case Dtype::F16: return 2;
        case Dtype::F32: return 4;
        case Dtype::U8: return 1;
        default: return 0;
    }
}

std::string shape_str(const std::vector<size_t> &s) {
    std::string out = "[";
    for (size_t i = 0; i < s.size(); ++i) out += (i ? ", " : "") + std::to_string(s[i]);
    return out + "]";
}

}  // namespace

// ------------------------------------------------------------ Mapping

Mapping::Mapping(const std::string &path) : path_(path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw Error(base_name(path) + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        throw Error(base_name(path) + ": " + std::strerror(e));
    }
    size_ = (size_t)st.st_size;
    if (size_ > 0) {
        void *p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            const int e = errno;
            ::close(fd);
            throw Error(base_name(path) + ": mmap: " + std::strerror(e));
        }
        data_ = static_cast<const uint8_t *>(p);
    }
    ::close(fd);
}

Mapping::~Mapping() {
    if (data_) ::munmap(const_cast<uint8_t *>(data_), size_);
}

// ------------------------------------------------------------ Bf16Slice

Bf16Slice Bf16Slice::mapped(std::shared_ptr<const Mapping> map, size_t offset, size_t len) {
    if (offset > map->size() || len * 2 > map->size() - offset) throw Error("mapped range outside the map");
    Bf16Slice s;
    if (offset % 2 == 0) {
        s.data_ = reinterpret_cast<const uint16_t *>(map->data() + offset);
        s.len_ = len;
        s.mapped_ = true;
        s.owner_ = std::move(map);
        return s;
    }
    // An odd offset cannot be viewed as uint16_t: copy (little-endian bytes).
    std::vector<uint16_t> v(len);
    std::memcpy(v.data(), map->data() + offset, len * 2);
    return owned(std::move(v));
}

Bf16Slice Bf16Slice::owned(std::vector<uint16_t> v) {
    auto p = std::make_shared<std::vector<uint16_t>>(std::move(v));
    Bf16Slice s;
    s.data_ = p->data();
    s.len_ = p->size();
    s.mapped_ = false;
    s.owner_ = std::move(p);
    return s;
}

Bf16Slice Bf16Slice::sub(size_t start, size_t len) const {
    if (start + len > len_) throw Error("sub-slice out of range");
    Bf16Slice s = *this;
    s.data_ = data_ + start;
    s.len_ = len;
    return s;
}

// ------------------------------------------------------------ f16

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            // Subnormal: m * 2^-24, exact in f32.
            float f = std::ldexp((float)m, -24);
            std::memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

// ------------------------------------------------------------ Checkpoint

Checkpoint Checkpoint::open_file(const std::string &path) {
    Checkpoint c;
    c.add_file(path, nullptr);
    return c;
}

Checkpoint Checkpoint::open(const std::string &dir) {
    const std::string single = dir + "/model.safetensors";
    if (file_exists(single)) return open_file(single);
    const std::string idx_path = dir + "/model.safetensors.index.json";
    std::string text;
    try {
        text = read_text(idx_path);
    } catch (const Error &e) {
        throw Error(std::string("neither model.safetensors nor its index: ") + e.what());
    }
    reng_json::Value idx;
    try {
        idx = reng_json::parse(text);
    } catch (const std::exception &e) {
        throw Error(std::string("safetensors index: ") + e.what());
    }
    if (!idx.has("weight_map") || idx["weight_map"].kind != reng_json::Value::Object)
        throw Error("safetensors index has no weight_map");
    // Shard file -> the tensors the index places in it.
    std::map<std::string, std::map<std::string, bool>> by_file;
    for (const auto &kv : idx["weight_map"].obj) {
        if (kv.second.kind != reng_json::Value::String) continue;
        by_file[kv.second.str][kv.first] = true;
    }
    Checkpoint c;
    for (const auto &f : by_file) c.add_file(dir + "/" + f.first, &f.second);
    return c;
}

void Checkpoint::add_file(const std::string &path, const std::map<std::string, bool> *only) {
    auto map = std::make_shared<const Mapping>(path);
    const std::string fname = base_name(path);
    if (map->size() < 8) throw Error("safetensors: " + fname + " is shorter than its header length");
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | map->data()[i];
    if (hlen > map->size() - 8) throw Error("safetensors: " + fname + ": header length past the end of the file");
    const std::string header(reinterpret_cast<const char *>(map->data() + 8), (size_t)hlen);
    reng_json::Value h;
    try {
        h = reng_json::parse(header);
    } catch (const std::exception &e) {
        throw Error("safetensors: " + fname + ": " + e.what());
    }
    if (h.kind != reng_json::Value::Object) throw Error("safetensors: " + fname + ": header is not an object");
    const size_t data0 = 8 + (size_t)hlen, data_len = map->size() - data0;
    const size_t shard = files_.size();
    for (const auto &kv : h.obj) {
        if (kv.first == "__metadata__") {
            if (kv.second.kind == reng_json::Value::Object)
                for (const auto &m : kv.second.obj)
                    if (m.second.kind == reng_json::Value::String) metadata_[m.first] = m.second.str;
            continue;
        }
        if (only && !only->count(kv.first)) continue;
        const reng_json::Value &t = kv.second;
        TensorInfo ti;
        ti.name = kv.first;
        ti.shard = shard;
        try {
            ti.dtype_name = t["dtype"].as_str();
            for (const auto &d : t["shape"].arr) ti.shape.push_back((size_t)d.as_u64());
            const auto &off = t["data_offsets"];
            if (off.size() != 2) throw Error("data_offsets is not a pair");
            ti.begin = (size_t)off[0].as_u64();
            ti.end = (size_t)off[1].as_u64();
        } catch (const std::exception &e) {
            throw Error("safetensors: " + fname + ": tensor " + kv.first + ": " + e.what());
        }
        ti.dtype = ti.dtype_name == "BF16" ? Dtype::BF16
                   : ti.dtype_name == "F16" ? Dtype::F16
                   : ti.dtype_name == "F32" ? Dtype::F32
                   : ti.dtype_name == "U8"  ? Dtype::U8
                                            : Dtype::Other;
        if (ti.begin > ti.end || ti.end > data_len)
            throw Error("safetensors: " + fname + ": tensor " + kv.first + ": data outside the file");
        if (ti.dtype != Dtype::Other) {
            // The element count and its byte size are checked for overflow: a
            // shape whose product wraps could otherwise match the byte range
            // (even 0) while consumers trust the shape.
            size_t n = 1, nbytes = 0;
            for (size_t d : ti.shape)
                if (__builtin_mul_overflow(n, d, &n))
                    throw Error("safetensors: " + fname + ": tensor " + kv.first + ": shape " + shape_str(ti.shape) +
                                " overflows");
            if (__builtin_mul_overflow(n, dtype_size(ti.dtype), &nbytes))
                throw Error("safetensors: " + fname + ": tensor " + kv.first + ": shape " + shape_str(ti.shape) +
                            " overflows");
            if (nbytes != ti.end - ti.begin)
                throw Error("safetensors: " + fname + ": tensor " + kv.first + ": " + std::to_string(ti.end - ti.begin) +
                            " bytes for " + ti.dtype_name + " " + shape_str(ti.shape));
        }
        ti.begin += data0;
        ti.end += data0;
        tensors_[kv.first] = ti;
    }
    files_.push_back(std::move(map));
    paths_.push_back(path);
}

const TensorInfo &Checkpoint::info(const std::string &name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw Error("tensor " + name + ": not in the checkpoint");
    return it->second;
}

std::vector<std::string> Checkpoint::names() const {
    std::vector<std::string> out;
    for (const auto &kv : tensors_) out.push_back(kv.first);
    return out;
}

Bf16Slice Checkpoint::bf16(const std::string &name) const {
    const TensorInfo &t = info(name);
    const auto &map = files_[t.shard];
    const uint8_t *p = map->data() + t.begin;
    switch (t.dtype) {
        case Dtype::BF16: return Bf16Slice::mapped(map, t.begin, (t.end - t.begin) / 2);
        case Dtype::F32: {
            std::vector<uint16_t> v((t.end - t.begin) / 4);
            for (size_t i = 0; i < v.size(); ++i) {
                float f;
                std::memcpy(&f, p + 4 * i, 4);
                v[i] = reng_fp8::f32_to_bf16(f);
            }
            return Bf16Slice::owned(std::move(v));
        }
        case Dtype::F16: {
            std::vector<uint16_t> v((t.end - t.begin) / 2);
            for (size_t i = 0; i < v.size(); ++i) {
                uint16_t hh;
                std::memcpy(&hh, p + 2 * i, 2);
                v[i] = reng_fp8::f32_to_bf16(f16_to_f32(hh));
            }
            return Bf16Slice::owned(std::move(v));
        }
        default: throw Error("tensor " + name + ": unsupported dtype " + t.dtype_name);
    }
}

std::vector<float> Checkpoint::f32(const std::string &name) const {
    const TensorInfo &t = info(name);
    const uint8_t *p = files_[t.shard]->data() + t.begin;
    std::vector<float> out;
    switch (t.dtype) {
        case Dtype::BF16:
            out.resize((t.end - t.begin) / 2);
            for (size_t i = 0; i < out.size(); ++i) {
                uint16_t hh;
                std::memcpy(&hh, p + 2 * i, 2);
                out[i] = reng_fp8::bf16_to_f32(hh);
            }
            break;
        case Dtype::F16:
            out.resize((t.end - t.begin) / 2);
            for (size_t i = 0; i < out.size(); ++i) {
                uint16_t hh;
                std::memcpy(&hh, p + 2 * i, 2);
                out[i] = f16_to_f32(hh);
            }
            break;
        case Dtype::F32:
            out.resize((t.end - t.begin) / 4);
            std::memcpy(out.data(), p, out.size() * 4);
            break;
        default: throw Error("tensor " + name + ": unsupported dtype " + t.dtype_name);
    }
    return out;
}

std::vector<uint8_t> Checkpoint::u8(const std::string &name) const {
    const TensorInfo &t = info(name);
    if (t.dtype != Dtype::U8) throw Error("tensor " + name + ": " + t.dtype_name + ", expected U8");
    const uint8_t *p = files_[t.shard]->data() + t.begin;
    return std::vector<uint8_t>(p, p + (t.end - t.begin));
}

namespace {

std::string json_string(const std::string &v) {
    std::string o = "\"";
    for (unsigned char ch : v) {
        if (ch == '"' || ch == '\\') {
            o += '\\';
            o += (char)ch;
        } else if (ch < 0x20) {
            char b[8];
            std::snprintf(b, sizeof b, "\\u%04x", ch);
            o += b;
        } else {
            o += (char)ch;
        }
    }
    return o + "\"";
}

}  // namespace

void write_safetensors(const std::string &path, const std::vector<TensorOut> &tensors,
                       const std::map<std::string, std::string> &metadata) {
    std::string header = "{";
    if (!metadata.empty()) {
        header += "\"__metadata__\":{";
        bool first = true;
        for (const auto &m : metadata) {
            header += (first ? "" : ",") + json_string(m.first) + ":" + json_string(m.second);
            first = false;
        }
        header += "}";
    }
    size_t off = 0;
    for (size_t i = 0; i < tensors.size(); ++i) {
        const TensorOut &t = tensors[i];
        const Dtype d = t.dtype == "BF16" ? Dtype::BF16 : t.dtype == "F16" ? Dtype::F16
                        : t.dtype == "F32" ? Dtype::F32 : t.dtype == "U8" ? Dtype::U8 : Dtype::Other;
        size_t n = 1;
        for (size_t x : t.shape) n *= x;
        if (d == Dtype::Other || n * dtype_size(d) != t.bytes)
            throw Error("safetensors: tensor " + t.name + ": " + std::to_string(t.bytes) + " bytes for " + t.dtype +
                        " " + shape_str(t.shape));
        header += std::string(header.size() > 1 ? "," : "") + json_string(t.name) + ":{\"dtype\":\"" + t.dtype +
                  "\",\"shape\":" + shape_str(t.shape) + ",\"data_offsets\":[" + std::to_string(off) + "," +
                  std::to_string(off + t.bytes) + "]}";
        off += t.bytes;
    }
    header += "}";
    while (header.size() % 8 != 0) header.push_back(' ');
    const std::string tmp = path + ".tmp";
    FILE *f = std::fopen(tmp.c_str(), "wb");
    if (!f) throw Error("cannot write " + tmp + ": " + std::strerror(errno));
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)((uint64_t)header.size() >> (8 * i));
    bool ok = std::fwrite(len, 1, 8, f) == 8 && std::fwrite(header.data(), 1, header.size(), f) == header.size();
    for (const TensorOut &t : tensors)
        ok = ok && (t.bytes == 0 || std::fwrite(t.data, 1, t.bytes, f) == t.bytes);
    ok = (std::fclose(f) == 0) && ok;
    if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0) {
        std::remove(tmp.c_str());
        throw Error("cannot write " + path + ": " + std::strerror(errno));
    }
}

Bf16Slice Checkpoint::linear(const std::string &name, size_t out_dim, size_t in_dim) const {
    const TensorInfo &t = info(name);
    if (t.shape != std::vector<size_t>{out_dim, in_dim})
        throw Error("tensor " + name + ": shape " + shape_str(t.shape) + ", expected [" + std::to_string(out_dim) +
                    ", " + std::to_string(in_dim) + "]");
    return bf16(name);
}

}  // namespace reng_model
