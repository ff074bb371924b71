// lm_checkpoint.cpp -- SafeTensors checkpoint index and the layer loader (host code).
//
// Reference: SafeTensor::open / find / payload (src/SafeTensor.cpp:30-160),
// WeightStore::open / find / require / read_float32 (src/WeightStore.cpp:52-185)
// and the FFN part of DeepSeekRunner::Impl::resolve_layer
// (src/DeepSeekRunner.cpp:157-225).
//
// A shard is an 8-byte little-endian header length, a JSON object mapping
// tensor names to {dtype, shape, data_offsets}, and the payload; offsets count
// from the end of the header.  Every shard of a directory is mapped read-only
// (sorted by file name; a name present in two shards resolves to the first) and
// indexed once.  Lookups hand out pointers into the mapping, which the layer
// loader passes straight to the upload entry points: the payload is read from
// the page cache exactly once, on its way to HBM.
#include "litemind_moe.h"
#include "lm_error.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <exception>
#include <filesystem>
#include <memory>
#include <new>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace {

constexpr uint64_t kMaxHeaderBytes = 512ull << 20;  // larger: not a SafeTensors shard
constexpr int kMaxDepth = 64;                       // JSON nesting accepted in a header
constexpr int kMaxRank = 8;

// ---- JSON (the subset a SafeTensors header uses, with full string escapes) ----

struct Json {
    enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
    bool integral = false;  // a number written without fraction or exponent, >= 0
    uint64_t integer = 0;   // its value when integral
    std::string text;       // strings
    std::vector<Json> items;                              // arrays
    std::vector<std::pair<std::string, Json>> members;    // objects, in file order

    const Json* find(std::string_view key) const {
        for (const auto& m : members) {
            if (m.first == key) {
                return &m.second;
            }
        }
        return nullptr;
    }
};

class Parser {
public:
    explicit Parser(std::string_view s) : s_(s) {}

    bool parse(Json& out, std::string& error) {
        if (!value(out, 0)) {
            error = error_.empty() ? "malformed JSON" : error_;
            return false;
        }
        skip_space();
        if (pos_ != s_.size()) {
            error = "trailing characters after the JSON header at byte " + std::to_string(pos_);
            return false;
        }
        return true;
    }

private:
    bool fail(const std::string& what) {
        if (error_.empty()) {
            error_ = what + " at byte " + std::to_string(pos_);
        }
        return false;
    }
    void skip_space() {
        while (pos_ < s_.size() && (s_[pos_] == ' ' || s_[pos_] == '\t' || s_[pos_] == '\n' || s_[pos_] == '\r')) {
            ++pos_;
        }
    }
    bool literal(std::string_view word) {
        if (s_.substr(pos_, word.size()) != word) {
            return fail("unexpected token");
        }
        pos_ += word.size();
        return true;
    }
    static void put_utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (pos_ + 4 > s_.size()) {
            return fail("truncated \\u escape");
        }
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = s_[pos_++];
            v <<= 4;
            if (c >= '0' && c <= '9') {
                v |= static_cast<uint32_t>(c - '0');
            } else if (c >= 'a' && c <= 'f') {
                v |= static_cast<uint32_t>(c - 'a' + 10);
            } else if (c >= 'A' && c <= 'F') {
                v |= static_cast<uint32_t>(c - 'A' + 10);
            } else {
                return fail("bad \\u escape");
            }
        }
        return true;
    }
    bool string(std::string& out) {
        ++pos_;  // opening quote
        out.clear();
        while (pos_ < s_.size()) {
            const char c = s_[pos_++];
            if (c == '"') {
                return true;
            }
            if (static_cast<unsigned char>(c) < 0x20) {
                return fail("control character in a string");
            }
            if (c != '\\') {
                out += c;
                continue;
            }
            if (pos_ >= s_.size()) {
                break;
            }
            const char e = s_[pos_++];
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp = 0;
                    if (!hex4(cp)) {
                        return false;
                    }
                    if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
                        uint32_t lo = 0;
                        if (s_.substr(pos_, 2) != "\\u" || (pos_ += 2, !hex4(lo)) || lo < 0xDC00 || lo >= 0xE000) {
                            return fail("unpaired surrogate");
                        }
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("unpaired surrogate");
                    }
                    put_utf8(out, cp);
                    break;
                }
                default:
                    return fail("bad escape");
            }
        }
        return fail("unterminated string");
    }
    bool number(Json& out) {
        const size_t start = pos_;
        if (s_[pos_] == '-') {
            ++pos_;
        }
        const size_t digits = pos_;
        while (pos_ < s_.size() && s_[pos_] >= '0' && s_[pos_] <= '9') {
            ++pos_;
        }
        if (pos_ == digits) {
            return fail("bad number");
        }
        bool fraction = false;
        if (pos_ < s_.size() && s_[pos_] == '.') {
            fraction = true;
            ++pos_;
            const size_t f = pos_;
            while (pos_ < s_.size() && s_[pos_] >= '0' && s_[pos_] <= '9') {
                ++pos_;
            }
            if (pos_ == f) {
                return fail("bad number");
            }
        }
        if (pos_ < s_.size() && (s_[pos_] == 'e' || s_[pos_] == 'E')) {
            fraction = true;
            ++pos_;
            if (pos_ < s_.size() && (s_[pos_] == '+' || s_[pos_] == '-')) {
                ++pos_;
            }
            const size_t x = pos_;
            while (pos_ < s_.size() && s_[pos_] >= '0' && s_[pos_] <= '9') {
                ++pos_;
            }
            if (pos_ == x) {
                return fail("bad number");
            }
        }
        out.kind = Json::kNumber;
        out.integral = !fraction && s_[start] != '-' && pos_ - digits <= 19;
        if (out.integral) {
            uint64_t v = 0;
            for (size_t i = digits; i < pos_; ++i) {
                v = v * 10 + static_cast<uint64_t>(s_[i] - '0');
            }
            out.integer = v;
        }
        return true;
    }
    bool value(Json& out, int depth) {
        if (depth > kMaxDepth) {
            return fail("JSON nested too deeply");
        }
        skip_space();
        if (pos_ >= s_.size()) {
            return fail("unexpected end of the header");
        }
        const char c = s_[pos_];
        if (c == '{') {
            out.kind = Json::kObject;
            ++pos_;
            skip_space();
            if (pos_ < s_.size() && s_[pos_] == '}') {
                ++pos_;
                return true;
            }
            for (;;) {
                skip_space();
                if (pos_ >= s_.size() || s_[pos_] != '"') {
                    return fail("expected a member name");
                }
                std::string key;
                if (!string(key)) {
                    return false;
                }
                skip_space();
                if (pos_ >= s_.size() || s_[pos_] != ':') {
                    return fail("expected ':'");
                }
                ++pos_;
                Json v;
                if (!value(v, depth + 1)) {
                    return false;
                }
                out.members.emplace_back(std::move(key), std::move(v));
                skip_space();
                if (pos_ < s_.size() && s_[pos_] == ',') {
                    ++pos_;
                    continue;
                }
                if (pos_ < s_.size() && s_[pos_] == '}') {
                    ++pos_;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            out.kind = Json::kArray;
            ++pos_;
            skip_space();
            if (pos_ < s_.size() && s_[pos_] == ']') {
                ++pos_;
                return true;
            }
            for (;;) {
                Json v;
                if (!value(v, depth + 1)) {
                    return false;
                }
                out.items.push_back(std::move(v));
                skip_space();
                if (pos_ < s_.size() && s_[pos_] == ',') {
                    ++pos_;
                    continue;
                }
                if (pos_ < s_.size() && s_[pos_] == ']') {
                    ++pos_;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            out.kind = Json::kString;
            return string(out.text);
        }
        if (c == 't') {
            out.kind = Json::kBool;
            return literal("true");
        }
        if (c == 'f') {
            out.kind = Json::kBool;
            return literal("false");
        }
        if (c == 'n') {
            out.kind = Json::kNull;
            return literal("null");
        }
        if (c == '-' || (c >= '0' && c <= '9')) {
            return number(out);
        }
        return fail("unexpected character");
    }

    std::string_view s_;
    size_t pos_ = 0;
    std::string error_;
};

// ---- shards ----

struct DtypeInfo {
    const char* name;
    int32_t code;
    uint32_t size;
};
// The element types SafeTensor accepts (src/SafeTensor.cpp:15-27).
constexpr DtypeInfo kDtypes[] = {
    {"BF16", LM_DT_BF16, 2}, {"F16", LM_DT_F16, 2}, {"F32", LM_DT_F32, 4}, {"F64", LM_DT_F64, 8},
    {"I8", LM_DT_I8, 1},     {"I16", LM_DT_I16, 2}, {"I32", LM_DT_I32, 4}, {"I64", LM_DT_I64, 8},
    {"U8", LM_DT_U8, 1},     {"BOOL", LM_DT_BOOL, 1},
};

const DtypeInfo* dtype_by_name(std::string_view s) {
    for (const auto& d : kDtypes) {
        if (s == d.name) {
            return &d;
        }
    }
    return nullptr;
}

const DtypeInfo* dtype_by_code(int32_t code) {
    for (const auto& d : kDtypes) {
        if (d.code == code) {
            return &d;
        }
    }
    return nullptr;
}

struct Tensor {
    std::string name;
    const DtypeInfo* dtype = nullptr;
    std::vector<int64_t> shape;
    uint64_t offset = 0;  // from the start of the file
    uint64_t bytes = 0;
    int shard = 0;
};

std::string shape_text(const int64_t* shape, size_t rank) {
    std::string s = "[";
    for (size_t i = 0; i < rank; ++i) {
        s += (i == 0 ? "" : ", ") + std::to_string(shape[i]);
    }
    return s + "]";
}

struct Mapping {
    void* base = nullptr;
    uint64_t size = 0;
    ~Mapping() {
        if (base != nullptr) {
            munmap(base, size);
        }
    }
};

// Maps one shard and appends its tensors (SafeTensor::open, src/SafeTensor.cpp:87-152).
bool open_shard(const std::string& path, int shard, std::vector<std::unique_ptr<Mapping>>& maps,
                std::vector<Tensor>& tensors, std::string& error) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        error = "cannot open " + path + ": " + std::strerror(errno);
        return false;
    }
    struct stat st {};
    if (fstat(fd, &st) != 0) {
        error = "cannot stat " + path + ": " + std::strerror(errno);
        ::close(fd);
        return false;
    }
    auto map = std::make_unique<Mapping>();
    map->size = static_cast<uint64_t>(st.st_size);
    if (map->size < 8) {
        ::close(fd);
        error = path + " is too small to be a SafeTensors shard.";
        return false;
    }
    void* base = mmap(nullptr, map->size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (base == MAP_FAILED) {
        error = "cannot map " + path + ": " + std::strerror(errno);
        return false;
    }
    map->base = base;
    const auto* bytes = static_cast<const unsigned char*>(base);
    uint64_t header = 0;
    for (int i = 0; i < 8; ++i) {
        header |= static_cast<uint64_t>(bytes[i]) << (8 * i);
    }
    if (header == 0 || header > kMaxHeaderBytes || header > map->size - 8) {
        error = path + " declares an implausible SafeTensors header length of " + std::to_string(header) + " bytes.";
        return false;
    }
    const uint64_t payload = 8 + header;
    Json doc;
    std::string why;
    if (!Parser(std::string_view(reinterpret_cast<const char*>(bytes + 8), header)).parse(doc, why)) {
        error = path + ": " + why;
        return false;
    }
    if (doc.kind != Json::kObject) {
        error = path + ": the SafeTensors header must be a JSON object.";
        return false;
    }
    const size_t first = tensors.size();
    for (const auto& [name, entry] : doc.members) {
        if (name == "__metadata__") {
            continue;
        }
        auto bad = [&](const std::string& what) {
            error = path + ": tensor '" + name + "' " + what;
            tensors.resize(first);
            return false;
        };
        if (entry.kind != Json::kObject) {
            error = path + ": tensor entry '" + name + "' is not a JSON object.";
            tensors.resize(first);
            return false;
        }
        const Json* dt = entry.find("dtype");
        const DtypeInfo* info = dt != nullptr && dt->kind == Json::kString ? dtype_by_name(dt->text) : nullptr;
        if (info == nullptr) {
            return bad("uses an unsupported dtype '" +
                       (dt != nullptr && dt->kind == Json::kString ? dt->text : std::string("?")) + "'.");
        }
        const Json* sh = entry.find("shape");
        if (sh == nullptr || sh->kind != Json::kArray) {
            return bad("has no shape array.");
        }
        if (sh->items.size() > static_cast<size_t>(kMaxRank)) {
            return bad("has more than " + std::to_string(kMaxRank) + " dimensions.");
        }
        Tensor t;
        t.name = name;
        t.dtype = info;
        t.shard = shard;
        uint64_t count = 1;
        for (const Json& d : sh->items) {
            if (d.kind != Json::kNumber || !d.integral) {
                return bad("has a non-numeric dimension.");
            }
            // element counts beyond the file size are caught below; keep the product finite
            if (d.integer != 0 && count > (UINT64_MAX / 8) / d.integer) {
                return bad("has an element count that overflows.");
            }
            count *= d.integer;
            t.shape.push_back(static_cast<int64_t>(d.integer));
        }
        const Json* off = entry.find("data_offsets");
        if (off == nullptr || off->kind != Json::kArray || off->items.size() != 2 ||
            off->items[0].kind != Json::kNumber || !off->items[0].integral || off->items[1].kind != Json::kNumber ||
            !off->items[1].integral) {
            return bad("has a malformed data_offsets pair.");
        }
        const uint64_t begin = off->items[0].integer, end = off->items[1].integer;
        if (end < begin) {
            return bad("has data_offsets in descending order.");
        }
        t.bytes = count * info->size;
        if (t.bytes != end - begin) {
            return bad("declares " + std::to_string(end - begin) + " payload bytes but its shape and dtype need " +
                       std::to_string(t.bytes) + ".");
        }
        if (begin > map->size - payload || t.bytes > map->size - payload - begin) {
            return bad("extends past the end of the shard.");
        }
        t.offset = payload + begin;
        tensors.push_back(std::move(t));
    }
    if (tensors.size() == first) {
        error = path + " contains no tensors.";
        return false;
    }
    maps.push_back(std::move(map));
    return true;
}

float bf16_to_f32(uint16_t v) {
    const uint32_t u = static_cast<uint32_t>(v) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// IEEE binary16 -> binary32, exact (subnormals normalised, inf and NaN kept).
float f16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t u;
    if (exp == 0x1F) {
        u = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        u = sign | ((exp + 112) << 23) | (man << 13);
    } else if (man == 0) {
        u = sign;
    } else {
        exp = 113;  // 2^-14, before the shifts below
        while ((man & 0x400u) == 0) {
            man <<= 1;
            --exp;
        }
        u = sign | (exp << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

struct lm_checkpoint {
    std::string dir;
    std::vector<std::unique_ptr<Mapping>> maps;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> index;

    const Tensor* find(const std::string& name) const {
        const auto it = index.find(name);
        return it == index.end() ? nullptr : &tensors[it->second];
    }
    const void* payload(const Tensor& t) const {
        return static_cast<const unsigned char*>(maps[static_cast<size_t>(t.shard)]->base) + t.offset;
    }
};

namespace {

// WeightStore::require (src/WeightStore.cpp:119-140).
int require(const lm_checkpoint* ck, const std::string& name, std::vector<int64_t> shape, int32_t dtype,
            const Tensor** out) {
    const Tensor* t = ck->find(name);
    if (t == nullptr) {
        return lm::set_error(LM_EINVAL, "The checkpoint has no tensor named '" + name + "'.");
    }
    if (t->shape != shape) {
        return lm::set_error(LM_EINVAL, "Tensor '" + name + "' has shape " + shape_text(t->shape.data(), t->shape.size()) +
                                            " but the configuration implies " + shape_text(shape.data(), shape.size()) +
                                            ".");
    }
    if (dtype != 0 && t->dtype->code != dtype) {
        return lm::set_error(LM_EINVAL, "Tensor '" + name + "' is stored as " + t->dtype->name +
                                            " but this build reads " + dtype_by_code(dtype)->name + " here.");
    }
    *out = t;
    return LM_OK;
}

// WeightStore::read_float32 (src/WeightStore.cpp:142-185): F32 copied, BF16 and F16 widened.
int read_f32(const lm_checkpoint* ck, const std::string& name, std::vector<int64_t> shape, std::vector<float>& out) {
    const Tensor* t = nullptr;
    const int rc = require(ck, name, std::move(shape), 0, &t);
    if (rc != LM_OK) {
        return rc;
    }
    const uint64_t n = t->bytes / t->dtype->size;
    out.resize(n);
    const void* p = ck->payload(*t);
    switch (t->dtype->code) {
        case LM_DT_F32:
            std::memcpy(out.data(), p, n * 4);
            break;
        case LM_DT_BF16:
        case LM_DT_F16: {
            std::vector<uint16_t> raw(n);
            std::memcpy(raw.data(), p, n * 2);
            for (uint64_t i = 0; i < n; ++i) {
                out[i] = t->dtype->code == LM_DT_BF16 ? bf16_to_f32(raw[i]) : f16_to_f32(raw[i]);
            }
            break;
        }
        default:
            out.clear();
            return lm::set_error(LM_EINVAL, "Tensor '" + name + "' is stored as " + t->dtype->name +
                                                ", which cannot be widened to float32.");
    }
    return LM_OK;
}

// The three projections of one FFN (DeepSeekRunner::Impl::resolve_feed_forward,
// src/DeepSeekRunner.cpp:157-177): gate, up [I, H] and down [H, I], BF16.
int ffn_views(const lm_checkpoint* ck, const std::string& prefix, int64_t inter, int64_t hidden,
              const uint16_t* (&w)[3]) {
    const char* names[3] = {"gate_proj.weight", "up_proj.weight", "down_proj.weight"};
    for (int i = 0; i < 3; ++i) {
        const Tensor* t = nullptr;
        const std::vector<int64_t> shape = i < 2 ? std::vector<int64_t>{inter, hidden} : std::vector<int64_t>{hidden, inter};
        const int rc = require(ck, prefix + names[i], shape, LM_DT_BF16, &t);
        if (rc != LM_OK) {
            return rc;
        }
        w[i] = static_cast<const uint16_t*>(ck->payload(*t));
    }
    return LM_OK;
}

#define LM_CK_GUARD_BEGIN try {
#define LM_CK_GUARD_END                                                                                      \
    }                                                                                                        \
    catch (const std::bad_alloc&) {                                                                          \
        return lm::set_error(LM_ENOMEM, "host allocation failed");                                           \
    }                                                                                                        \
    catch (const std::exception& e) {                                                                        \
        return lm::set_error(LM_EINVAL, e.what());                                                           \
    }

}  // namespace

extern "C" {

int lm_checkpoint_open(const char* model_dir, lm_checkpoint** out) {
    LM_CK_GUARD_BEGIN
    if (model_dir == nullptr || out == nullptr) {
        return lm::set_error(LM_EINVAL, "null argument");
    }
    *out = nullptr;
    namespace fs = std::filesystem;
    std::error_code ec;
    const fs::path dir(model_dir);
    if (!fs::is_directory(dir, ec)) {
        return lm::set_error(LM_EINVAL, "Not a model directory: " + dir.string());
    }
    std::vector<std::string> paths;
    for (const auto& entry : fs::directory_iterator(dir, ec)) {
        if (entry.is_regular_file(ec) && entry.path().extension() == ".safetensors") {
            paths.push_back(entry.path().string());
        }
    }
    std::sort(paths.begin(), paths.end());
    if (paths.empty()) {
        return lm::set_error(LM_EINVAL, "No .safetensors files were found in " + dir.string() + ".");
    }
    auto ck = std::make_unique<lm_checkpoint>();
    ck->dir = dir.string();
    for (const std::string& p : paths) {
        std::string error;
        if (!open_shard(p, static_cast<int>(ck->maps.size()), ck->maps, ck->tensors, error)) {
            return lm::set_error(LM_EINVAL, error);
        }
    }
    for (size_t i = 0; i < ck->tensors.size(); ++i) {
        ck->index.emplace(ck->tensors[i].name, i);  // a name in two shards: the first stays
    }
    *out = ck.release();
    return LM_OK;
    LM_CK_GUARD_END
}

int lm_checkpoint_close(lm_checkpoint* ck) {
    delete ck;
    return LM_OK;
}

int lm_checkpoint_count(const lm_checkpoint* ck, int64_t* tensors, int64_t* shards) {
    if (ck == nullptr) {
        return lm::set_error(LM_EINVAL, "null checkpoint");
    }
    if (tensors != nullptr) {
        *tensors = static_cast<int64_t>(ck->index.size());
    }
    if (shards != nullptr) {
        *shards = static_cast<int64_t>(ck->maps.size());
    }
    return LM_OK;
}

int lm_checkpoint_find(const lm_checkpoint* ck, const char* name, int32_t* dtype, int32_t* rank, int64_t* shape,
                       const void** payload, uint64_t* bytes) {
    LM_CK_GUARD_BEGIN
    if (ck == nullptr || name == nullptr) {
        return lm::set_error(LM_EINVAL, "null argument");
    }
    const Tensor* t = ck->find(name);
    if (t == nullptr) {
        return lm::set_error(LM_EINVAL, std::string("The checkpoint has no tensor named '") + name + "'.");
    }
    if (dtype != nullptr) {
        *dtype = t->dtype->code;
    }
    if (rank != nullptr) {
        *rank = static_cast<int32_t>(t->shape.size());
    }
    if (shape != nullptr) {
        std::copy(t->shape.begin(), t->shape.end(), shape);
    }
    if (payload != nullptr) {
        *payload = ck->payload(*t);
    }
    if (bytes != nullptr) {
        *bytes = t->bytes;
    }
    return LM_OK;
    LM_CK_GUARD_END
}

int lm_checkpoint_require(const lm_checkpoint* ck, const char* name, int32_t rank, const int64_t* shape,
                          int32_t dtype, const void** payload) {
    LM_CK_GUARD_BEGIN
    if (ck == nullptr || name == nullptr || rank < 0 || rank > kMaxRank || (rank > 0 && shape == nullptr) ||
        dtype_by_code(dtype) == nullptr) {
        return lm::set_error(LM_EINVAL, "bad argument");
    }
    const Tensor* t = nullptr;
    const int rc = require(ck, name, std::vector<int64_t>(shape, shape + rank), dtype, &t);
    if (rc == LM_OK && payload != nullptr) {
        *payload = ck->payload(*t);
    }
    return rc;
    LM_CK_GUARD_END
}

int lm_checkpoint_read_f32(const lm_checkpoint* ck, const char* name, int32_t rank, const int64_t* shape, float* out,
                           uint64_t count) {
    LM_CK_GUARD_BEGIN
    if (ck == nullptr || name == nullptr || out == nullptr || rank < 0 || rank > kMaxRank ||
        (rank > 0 && shape == nullptr)) {
        return lm::set_error(LM_EINVAL, "bad argument");
    }
    std::vector<float> values;
    const int rc = read_f32(ck, name, std::vector<int64_t>(shape, shape + rank), values);
    if (rc != LM_OK) {
        return rc;
    }
    if (values.size() != count) {
        return lm::set_error(LM_EINVAL, "output holds " + std::to_string(count) + " floats, tensor '" + name +
                                            "' has " + std::to_string(values.size()));
    }
    std::memcpy(out, values.data(), count * sizeof(float));
    return LM_OK;
    LM_CK_GUARD_END
}

int lm_load_layer(lm_context* ctx, const lm_checkpoint* ck, int32_t layer, int32_t moe) {
    LM_CK_GUARD_BEGIN
    if (ctx == nullptr || ck == nullptr || layer < 0 || moe < -1 || moe > 1) {
        return lm::set_error(LM_EINVAL, "bad argument");
    }
    lm_moe_config cfg{};
    int rc = lm_context_config(ctx, &cfg);
    if (rc != LM_OK) {
        return rc;
    }
    const std::string prefix = "model.layers." + std::to_string(layer) + ".";
    const int64_t H = cfg.hidden_size;
    if (moe < 0) {
        moe = ck->find(prefix + "mlp.gate.weight") != nullptr ? 1 : 0;
    }
    // Every tensor is resolved before anything is uploaded, so a checkpoint
    // that lacks one leaves the context as it was.
    std::vector<float> norm;
    rc = read_f32(ck, prefix + "post_attention_layernorm.weight", {H}, norm);
    if (rc != LM_OK) {
        return rc;
    }
    if (moe == 0) {
        const uint16_t* w[3];
        rc = ffn_views(ck, prefix + "mlp.", cfg.intermediate_size, H, w);
        if (rc == LM_OK) {
            rc = lm_upload_dense(ctx, layer, w[0], w[1], w[2]);
        }
    } else {
        std::vector<float> router;
        rc = read_f32(ck, prefix + "mlp.gate.weight", {cfg.n_routed_experts, H}, router);
        std::vector<std::array<const uint16_t*, 3>> experts(static_cast<size_t>(cfg.n_routed_experts));
        for (int32_t e = 0; rc == LM_OK && e < cfg.n_routed_experts; ++e) {
            const uint16_t* w[3];
            rc = ffn_views(ck, prefix + "mlp.experts." + std::to_string(e) + ".", cfg.moe_intermediate_size, H, w);
            experts[static_cast<size_t>(e)] = {w[0], w[1], w[2]};
        }
        const uint16_t* shared[3] = {nullptr, nullptr, nullptr};
        if (rc == LM_OK && cfg.n_shared_experts > 0) {
            rc = ffn_views(ck, prefix + "mlp.shared_experts.",
                           static_cast<int64_t>(cfg.moe_intermediate_size) * cfg.n_shared_experts, H, shared);
        }
        if (rc == LM_OK) {
            rc = lm_upload_router(ctx, layer, router.data());
        }
        for (int32_t e = 0; rc == LM_OK && e < cfg.n_routed_experts; ++e) {
            const auto& w = experts[static_cast<size_t>(e)];
            rc = lm_upload_expert(ctx, layer, e, w[0], w[1], w[2]);
        }
        if (rc == LM_OK && cfg.n_shared_experts > 0) {
            rc = lm_upload_shared(ctx, layer, shared[0], shared[1], shared[2]);
        }
    }
    if (rc == LM_OK) {
        rc = lm_upload_norm(ctx, layer, norm.data());
    }
    if (rc == LM_OK) {
        rc = lm_finalize_layer(ctx, layer);
    }
    return rc;
    LM_CK_GUARD_END
}

int lm_load_head(lm_context* ctx, const lm_checkpoint* ck, int64_t vocab) {
    LM_CK_GUARD_BEGIN
    if (ctx == nullptr || ck == nullptr || vocab <= 0) {
        return lm::set_error(LM_EINVAL, "bad argument");
    }
    lm_moe_config cfg{};
    int rc = lm_context_config(ctx, &cfg);
    if (rc != LM_OK) {
        return rc;
    }
    const int64_t H = cfg.hidden_size;
    std::vector<float> norm;
    rc = read_f32(ck, "model.norm.weight", {H}, norm);
    if (rc != LM_OK) {
        return rc;
    }
    const std::string name = ck->find("lm_head.weight") != nullptr ? "lm_head.weight" : "model.embed_tokens.weight";
    const Tensor* head = nullptr;
    rc = require(ck, name, {vocab, H}, LM_DT_BF16, &head);
    if (rc != LM_OK) {
        return rc;
    }
    return lm_upload_head(ctx, norm.data(), static_cast<const uint16_t*>(ck->payload(*head)), vocab);
    LM_CK_GUARD_END
}

}  // extern "C"
