// bmts.hpp - C++ host mirror of the reference's shard reading
// (cluster/src/bmts.rs: BmtsShard::open, tensor_bytes, read_span,
// write_shard) and Hadamard sign slices (HadRuntime, qwen35.rs:345-356,
// 585-627).  A shard is memory-mapped read-only; tensor bytes are views of
// the mapping, which HipPool::upload_view hands to the device without a host
// copy.  Version-1 shards (JSON tensor table) are read; version 2 (Cap'n
// Proto table) is refused, as the reference's default build refuses it.
// Header-only, POSIX; failures throw ouro::Error(OURO_ERR_INVALID_ARG, ...)
// where the reference bails.
#pragma once

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../ouro_hip.h"

namespace ouro {

#ifndef OURO_ERROR_DEFINED
#define OURO_ERROR_DEFINED
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &what) : std::runtime_error(what), code(c) {}
};
#endif

namespace bmts {

constexpr uint32_t kMagic = 0x4F55524Fu;  // "OURO" little-endian (bmts.rs:21)
constexpr uint16_t kVersion = 1;
constexpr uint16_t kVersionV2 = 2;
constexpr size_t kHeaderLen = 16;

[[noreturn]] inline void bail(const std::string &msg) { throw Error(OURO_ERR_INVALID_ARG, msg); }

struct Tensor {  // bmts.rs:29-37
    std::string name;
    std::vector<uint64_t> shape;  // ggml order: [in_len, out_len] for matrices
    uint32_t dtype = 0;           // ggml type id
    uint64_t offset = 0, length = 0;
};

// A minimal reader for the JSON tensor table: an array of objects whose
// values are strings, numbers or arrays of numbers.
class TableReader {
public:
    explicit TableReader(const std::string &s) : s_(s) {}

    std::vector<Tensor> read() {
        std::vector<Tensor> out;
        ws();
        expect('[');
        ws();
        if (peek() == ']') {
            ++i_;
            return out;
        }
        for (;;) {
            out.push_back(object());
            ws();
            if (peek() == ',') {
                ++i_;
                ws();
                continue;
            }
            expect(']');
            break;
        }
        ws();
        if (i_ != s_.size()) bail("BMTS tensor table: trailing bytes");
        return out;
    }

private:
    char peek() const { return i_ < s_.size() ? s_[i_] : '\0'; }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
    }
    void expect(char c) {
        if (peek() != c) bail(std::string("BMTS tensor table: expected '") + c + "'");
        ++i_;
    }
    std::string str() {
        expect('"');
        std::string out;
        while (i_ < s_.size() && s_[i_] != '"') {
            char c = s_[i_++];
            if (c == '\\') {
                if (i_ >= s_.size()) break;
                const char e = s_[i_++];
                switch (e) {
                case 'n': c = '\n'; break;
                case 't': c = '\t'; break;
                case 'r': c = '\r'; break;
                case 'b': c = '\b'; break;
                case 'f': c = '\f'; break;
                case 'u': {
                    if (i_ + 4 > s_.size()) bail("BMTS tensor table: bad \\u escape");
                    const std::string hex = s_.substr(i_, 4);
                    if (hex.find_first_not_of("0123456789abcdefABCDEF") != std::string::npos)
                        bail("BMTS tensor table: bad \\u escape");
                    const unsigned v = static_cast<unsigned>(std::stoul(hex, nullptr, 16));
                    i_ += 4;
                    if (v > 0x7f) bail("BMTS tensor table: non-ASCII \\u escape");
                    c = static_cast<char>(v);
                    break;
                }
                default: c = e;
                }
            }
            out.push_back(c);
        }
        expect('"');
        return out;
    }
    uint64_t num() {
        const size_t b = i_;
        while (i_ < s_.size() && (std::isdigit(static_cast<unsigned char>(s_[i_])) || s_[i_] == '-' || s_[i_] == '+' ||
                                  s_[i_] == '.' || s_[i_] == 'e' || s_[i_] == 'E'))
            ++i_;
        if (b == i_) bail("BMTS tensor table: expected a number");
        const std::string t = s_.substr(b, i_ - b);
        if (t.find_first_of("-.eE") != std::string::npos) bail("BMTS tensor table: '" + t + "' is not a u64");
        try {
            return std::stoull(t);
        } catch (const std::exception &) {  // out of range, or a lone sign
            bail("BMTS tensor table: '" + t + "' is not a u64");
        }
    }
    Tensor object() {
        Tensor t;
        unsigned seen = 0;
        expect('{');
        ws();
        while (peek() != '}') {
            const std::string key = str();
            ws();
            expect(':');
            ws();
            if (key == "name") {
                t.name = str();
                seen |= 1;
            } else if (key == "shape") {
                expect('[');
                ws();
                while (peek() != ']') {
                    t.shape.push_back(num());
                    ws();
                    if (peek() == ',') {
                        ++i_;
                        ws();
                    }
                }
                ++i_;
                seen |= 2;
            } else if (key == "dtype") {
                t.dtype = static_cast<uint32_t>(num());
                seen |= 4;
            } else if (key == "offset") {
                t.offset = num();
                seen |= 8;
            } else if (key == "length") {
                t.length = num();
                seen |= 16;
            } else {
                bail("BMTS tensor table: unknown field " + key);
            }
            ws();
            if (peek() == ',') {
                ++i_;
                ws();
            }
        }
        ++i_;
        if (seen != 31) bail("BMTS tensor table: a tensor lacks a field");
        return t;
    }

    const std::string &s_;
    size_t i_ = 0;
};

// BmtsShard::open and accessors (bmts.rs:171-308).
class Shard {
public:
    explicit Shard(const std::string &path) : path_(path) {
        const int fd = ::open(path.c_str(), O_RDONLY);
        if (fd < 0) bail("cannot open " + path);
        struct stat st {};
        if (::fstat(fd, &st) != 0) {
            ::close(fd);
            bail("cannot stat " + path);
        }
        size_ = static_cast<size_t>(st.st_size);
        if (size_ < kHeaderLen) {
            ::close(fd);
            bail("BMTS file too short: " + path);
        }
        void *m = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (m == MAP_FAILED) bail("cannot map " + path);
        map_ = static_cast<const uint8_t *>(m);
        try {
            parse();
        } catch (...) {
            ::munmap(const_cast<uint8_t *>(map_), size_);
            throw;
        }
    }
    ~Shard() {
        if (map_) ::munmap(const_cast<uint8_t *>(map_), size_);
    }
    Shard(const Shard &) = delete;
    Shard &operator=(const Shard &) = delete;

    uint16_t node() const { return node_; }
    const std::vector<Tensor> &tensors() const { return tensors_; }
    uint64_t data_start() const { return data_start_; }

    uint64_t data_len() const {  // bmts.rs:273-276
        uint64_t n = 0;
        for (const Tensor &t : tensors_) n += t.length;
        return n;
    }

    const Tensor &tensor(const std::string &name) const {
        for (const Tensor &t : tensors_)
            if (t.name == name) return t;
        bail("tensor " + name + " not in shard");
    }

    // Zero-copy view (pointer into the mapping, length) of a tensor.
    std::pair<const uint8_t *, size_t> tensor_bytes(const std::string &name) const {
        const Tensor &t = tensor(name);
        return range(name, t.offset, t.length);
    }

    std::vector<uint8_t> read_tensor(const std::string &name) const {
        const auto v = tensor_bytes(name);
        return std::vector<uint8_t>(v.first, v.first + v.second);
    }

    // A span of a tensor, refused past the declared length (bmts.rs:286-308).
    std::pair<const uint8_t *, size_t> read_span(const std::string &name, uint64_t offset, uint64_t length) const {
        const Tensor &t = tensor(name);
        if (offset > t.length || length > t.length - offset)
            bail("span exceeds tensor " + name + " of " + std::to_string(t.length) + " bytes");
        if (t.offset > UINT64_MAX - offset)
            bail("tensor " + name + " range exceeds file of " + std::to_string(size_) + " bytes");
        return range(name, t.offset + offset, length);
    }

    // Stage::from_shard's reading of a tensor (mod.rs:114-123): rank 1 = [in],
    // rank 2 = [in, out].
    void weight_shape(const std::string &name, size_t *out_len, size_t *in_len) const {
        const Tensor &t = tensor(name);
        if (t.shape.size() == 1) {
            *in_len = t.shape[0];
            *out_len = 1;
        } else if (t.shape.size() == 2) {
            *in_len = t.shape[0];
            *out_len = t.shape[1];
        } else {
            bail("tensor " + t.name + " has rank " + std::to_string(t.shape.size()));
        }
    }

private:
    template <typename T>
    T le(size_t at) const {
        T v;
        std::memcpy(&v, map_ + at, sizeof(T));
        return v;
    }
    void parse() {
        if (le<uint32_t>(0) != kMagic) {
            char buf[64];
            std::snprintf(buf, sizeof buf, "bad BMTS magic %#010x in ", le<uint32_t>(0));
            bail(buf + path_);
        }
        const uint16_t version = le<uint16_t>(4);
        node_ = le<uint16_t>(6);
        const uint32_t n_tensors = le<uint32_t>(8);
        const uint32_t meta_len = le<uint32_t>(12);
        if (size_ < kHeaderLen + meta_len) bail("BMTS meta truncated: " + path_);
        if (version == kVersionV2) bail("BMTS v2 (Cap'n Proto meta) is not read by this library: " + path_);
        if (version != kVersion) bail("unsupported BMTS version " + std::to_string(version) + " in " + path_);
        const std::string meta(reinterpret_cast<const char *>(map_ + kHeaderLen), meta_len);
        tensors_ = TableReader(meta).read();
        if (tensors_.size() != n_tensors)
            bail("BMTS tensor count mismatch: header " + std::to_string(n_tensors) + " vs meta " +
                 std::to_string(tensors_.size()));
        data_start_ = kHeaderLen + meta_len;
    }
    std::pair<const uint8_t *, size_t> range(const std::string &name, uint64_t offset, uint64_t length) const {
        // offset and length are checked against the data region before any
        // addition, so a table entry near 2^64 cannot wrap into the header
        const uint64_t data_len = size_ - data_start_;
        if (offset > data_len || length > data_len - offset)
            bail("tensor " + name + " range exceeds file of " + std::to_string(size_) + " bytes");
        return {map_ + data_start_ + offset, static_cast<size_t>(length)};
    }

    std::string path_;
    const uint8_t *map_ = nullptr;
    size_t size_ = 0;
    uint16_t node_ = 0;
    uint64_t data_start_ = 0;
    std::vector<Tensor> tensors_;
};

// A version-1 shard (bmts.rs:311-324).
inline void write_shard(const std::string &path, uint16_t node, const std::vector<Tensor> &tensors,
                        const std::vector<uint8_t> &data) {
    std::string meta = "[";
    for (size_t i = 0; i < tensors.size(); ++i) {
        const Tensor &t = tensors[i];
        std::string esc;
        for (char c : t.name) {
            if (c == '"' || c == '\\') esc.push_back('\\');
            esc.push_back(c);
        }
        meta += (i ? "," : "") + std::string("{\"name\":\"") + esc + "\",\"shape\":[";
        for (size_t j = 0; j < t.shape.size(); ++j) meta += (j ? "," : "") + std::to_string(t.shape[j]);
        meta += "],\"dtype\":" + std::to_string(t.dtype) + ",\"offset\":" + std::to_string(t.offset) +
                ",\"length\":" + std::to_string(t.length) + "}";
    }
    meta += "]";
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) bail("cannot write " + path);
    const uint32_t magic = kMagic, n = static_cast<uint32_t>(tensors.size()), ml = static_cast<uint32_t>(meta.size());
    const uint16_t version = kVersion;
    bool ok = std::fwrite(&magic, 4, 1, f) == 1 && std::fwrite(&version, 2, 1, f) == 1 &&
              std::fwrite(&node, 2, 1, f) == 1 && std::fwrite(&n, 4, 1, f) == 1 && std::fwrite(&ml, 4, 1, f) == 1 &&
              std::fwrite(meta.data(), 1, meta.size(), f) == meta.size() &&
              (data.empty() || std::fwrite(data.data(), 1, data.size(), f) == data.size());
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) bail("short write to " + path);
}

}  // namespace bmts

// The Hadamard fold's sign slices (HadRuntime, qwen35.rs:585-627).
class HadRuntime {
public:
    HadRuntime(size_t block, std::vector<size_t> widths, std::vector<float> signs, bool gdn_v_grouped = false)
        : block_(block), widths_(std::move(widths)), signs_(std::move(signs)), v_grouped_(gdn_v_grouped) {
        size_t n = 0;
        for (size_t w : widths_) n += w;
        if (n != signs_.size()) bmts::bail("hadamard signs: count does not match the widths");
    }
    size_t block() const { return block_; }
    bool gdn_v_grouped() const { return v_grouped_; }
    const std::vector<float> &signs() const { return signs_; }

    // Offset of the sign slice whose width is n (qwen35.rs:603-613).
    size_t offset_for(size_t n) const {
        size_t acc = 0;
        for (size_t w : widths_) {
            if (w == n) return acc;
            acc += w;
        }
        bmts::bail("no hadamard sign slice for width " + std::to_string(n));
    }

private:
    size_t block_;
    std::vector<size_t> widths_;
    std::vector<float> signs_;
    bool v_grouped_;
};

}  // namespace ouro
