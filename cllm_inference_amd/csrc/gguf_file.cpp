// gguf_file.cpp -- GGUF parsing for the weight upload (host code).
//
// Follows GgufLoader::load (src/core/gguf.cpp:122-275): magic, version 2 or 3, tensor and
// key/value counts, the key/value section (only the kinds the reference keeps: u32, i32,
// f32, bool, string and arrays of string / f32 / i32; everything else is skipped), the tensor
// table with dims reversed to rows-first, and the data section at the next multiple of 32
// bytes. The file is mapped read-only once and parsed in place through a bounds-checked
// cursor; a read past the end fails with the message of the reference's read helper.
#include "gguf_file.h"

#include "ggml_blocks.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace cllm_hip {

namespace {

constexpr uint32_t kMaxDims = 4;  // GGML_MAX_DIMS

enum ValueType : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12,
};

// The metadata values the config extraction looks at, by kind (gguf.cpp:53-84).
struct Value {
    enum Kind { None, U32, I32, F32, Bool, Str, ArrStr, ArrF32, ArrI32 } kind = None;
    uint32_t u32 = 0;
    float f32 = 0.0f;
    bool b = false;
    std::string str;
    uint64_t arr_len = 0;
};

struct Cursor {
    const uint8_t* p;
    size_t size, at = 0;
    std::string err;

    bool take(void* dst, size_t n, const char* what) {
        if (!err.empty()) return false;
        if (at > size || size - at < n) {
            err = what;
            return false;
        }
        std::memcpy(dst, p + at, n);
        at += n;
        return true;
    }
    bool skip(uint64_t n) {  // like fseek: moving past the end only fails at the next read
        if (!err.empty()) return false;
        at = n > (uint64_t)(SIZE_MAX - at) ? SIZE_MAX : at + (size_t)n;
        return true;
    }
    bool u8(uint8_t& v) { return take(&v, 1, "read_u8"); }
    bool u32(uint32_t& v) { return take(&v, 4, "read_u32"); }
    bool u64(uint64_t& v) { return take(&v, 8, "read_u64"); }
    bool i32(int32_t& v) { return take(&v, 4, "read_i32"); }
    bool f32(float& v) { return take(&v, 4, "read_f32"); }
    bool str(std::string& s) {
        uint64_t len;
        if (!u64(len)) return false;
        if (at > size || size - at < len) {
            err = "read_string";
            return false;
        }
        s.assign((const char*)p + at, (size_t)len);
        at += (size_t)len;
        return true;
    }
    bool skip_value(uint32_t type, int depth = 0) {
        switch (type) {
            case V_U8: case V_I8: case V_BOOL: return skip(1);
            case V_U16: case V_I16: return skip(2);
            case V_U32: case V_I32: case V_F32: return skip(4);
            case V_U64: case V_I64: case V_F64: return skip(8);
            case V_STR: {
                uint64_t len;
                return u64(len) && skip(len);
            }
            case V_ARR: {
                uint32_t et;
                uint64_t n;
                if (!u32(et) || !u64(n)) return false;
                if (depth > 64) {
                    err = "unknown value type";
                    return false;
                }
                for (uint64_t i = 0; i < n; ++i)
                    if (!skip_value(et, depth + 1)) return false;
                return true;
            }
            default:
                if (err.empty()) err = "unknown value type";
                return false;
        }
    }
    bool value(uint32_t type, Value& v) {
        switch (type) {
            case V_U32: v.kind = Value::U32; return u32(v.u32);
            case V_I32: {
                int32_t t;
                v.kind = Value::I32;
                return i32(t);
            }
            case V_F32: v.kind = Value::F32; return f32(v.f32);
            case V_BOOL: {
                uint8_t t;
                v.kind = Value::Bool;
                if (!u8(t)) return false;
                v.b = t != 0;
                return true;
            }
            case V_STR: v.kind = Value::Str; return str(v.str);
            case V_ARR: {
                uint32_t et;
                uint64_t n;
                if (!u32(et) || !u64(n)) return false;
                if (et == V_STR || et == V_F32 || et == V_I32) {
                    v.kind = et == V_STR ? Value::ArrStr : et == V_F32 ? Value::ArrF32 : Value::ArrI32;
                    v.arr_len = n;
                    std::string s;
                    float f;
                    int32_t i;
                    for (uint64_t k = 0; k < n; ++k) {
                        const bool ok = et == V_STR ? str(s) : et == V_F32 ? f32(f) : i32(i);
                        if (!ok) return false;
                    }
                    return true;
                }
                for (uint64_t k = 0; k < n; ++k)
                    if (!skip_value(et, 1)) return false;
                return true;
            }
            default: return skip_value(type);
        }
    }
};

}  // namespace

GgufFile::~GgufFile() {
    if (map) munmap(map, map_bytes);
}

bool gguf_open(const char* path, GgufFile& out, std::string& err) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        err = std::string("cannot open model file: ") + path;
        return false;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        err = "fstat failed";
        return false;
    }
    const size_t size = (size_t)st.st_size;
    void* base = size ? mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
    close(fd);
    if (size && base == MAP_FAILED) {
        err = "mmap failed";
        return false;
    }
    out.map = base;
    out.map_bytes = size;
    Cursor c{(const uint8_t*)base, size};

    char magic[4];
    if (!c.take(magic, 4, "invalid GGUF magic") || std::memcmp(magic, "GGUF", 4) != 0) {
        err = "invalid GGUF magic";
        return false;
    }
    uint32_t version;
    if (!c.u32(version)) {
        err = c.err;
        return false;
    }
    if (version != 2 && version != 3) {
        err = "unsupported GGUF version: " + std::to_string(version);
        return false;
    }
    out.version = version;
    uint64_t n_tensors, n_kv;
    if (!c.u64(n_tensors) || !c.u64(n_kv)) {
        err = c.err;
        return false;
    }

    std::unordered_map<std::string, Value> kv;
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        uint32_t type;
        Value v;
        if (!c.str(key) || !c.u32(type) || !c.value(type, v)) {
            err = c.err;
            return false;
        }
        kv[key] = std::move(v);
    }

    out.tensors.clear();
    out.index.clear();
    for (uint64_t i = 0; i < n_tensors; ++i) {
        GgufTensor t;
        uint32_t n_dims;
        if (!c.str(t.name) || !c.u32(n_dims)) {
            err = c.err;
            return false;
        }
        // GGML tensors have at most 4 dimensions; a larger count is a malformed file (the
        // reference would allocate whatever the count says)
        if (n_dims > kMaxDims) {
            err = "tensor " + t.name + ": " + std::to_string(n_dims) + " dimensions";
            return false;
        }
        std::vector<uint64_t> dims(n_dims);
        for (uint32_t d = 0; d < n_dims; ++d)
            if (!c.u64(dims[d])) {
                err = c.err;
                return false;
            }
        if (!c.u32(t.type) || !c.u64(t.offset)) {
            err = c.err;
            return false;
        }
        t.shape.assign(dims.rbegin(), dims.rend());
        out.index[t.name] = (int)out.tensors.size();  // a repeated name keeps the last one
        out.tensors.push_back(std::move(t));
    }
    out.data_offset = (c.at + 31) & ~(size_t)31;

    // Every tensor of a known type must lie inside the mapped data section: the device copy
    // is exactly that section, and a pointer past it would send the kernels out of bounds.
    // (The reference does not check; its reads past a truncated file fault on the host.)
    const size_t data_bytes = out.map_bytes > out.data_offset ? out.map_bytes - out.data_offset : 0;
    for (const GgufTensor& t : out.tensors) {
        const int bs = block_elems(t.type);
        const size_t ts = block_bytes(t.type);
        if (bs <= 0 || ts == 0) continue;  // an unknown type: its size cannot be known
        unsigned __int128 elems = 1;
        for (uint64_t d : t.shape) elems *= d;
        const unsigned __int128 bytes = (elems + (unsigned)bs - 1) / (unsigned)bs * ts;
        if ((unsigned __int128)t.offset + bytes > data_bytes) {
            err = "tensor " + t.name + " extends past the end of the file";
            return false;
        }
    }

    // hyper-parameters (gguf.cpp:197-272)
    auto str_of = [&](const std::string& k) -> std::string {
        auto it = kv.find(k);
        return it != kv.end() && it->second.kind == Value::Str ? it->second.str : "";
    };
    auto u32_of = [&](const std::string& k, uint32_t& v) {
        auto it = kv.find(k);
        if (it == kv.end() || it->second.kind != Value::U32) return false;
        v = it->second.u32;
        return true;
    };
    auto f32_of = [&](const std::string& k, float& v) {
        auto it = kv.find(k);
        if (it == kv.end() || it->second.kind != Value::F32) return false;
        v = it->second.f32;
        return true;
    };
    GgufConfig& cfg = out.config;
    cfg.arch = str_of("general.architecture");
    auto field_u32 = [&](const char* suffix) {
        uint32_t v = 0;
        if (u32_of(cfg.arch + "." + suffix, v) || u32_of(std::string("llama.") + suffix, v)) return v;
        return 0u;
    };
    auto field_f32 = [&](const char* suffix) {
        float v = 0.0f;
        if (f32_of(cfg.arch + "." + suffix, v) || f32_of(std::string("llama.") + suffix, v)) return v;
        return 0.0f;
    };
    cfg.n_layers = field_u32("block_count");
    cfg.n_embd = field_u32("embedding_length");
    cfg.n_head = field_u32("attention.head_count");
    cfg.n_head_kv = field_u32("attention.head_count_kv");
    cfg.n_ctx = field_u32("context_length");
    cfg.n_ff = field_u32("feed_forward_length");
    cfg.head_dim_explicit = field_u32("attention.key_length");
    const float rope = field_f32("rope.freq_base");
    if (rope > 0) cfg.rope_theta = rope;
    const float eps = field_f32("attention.layer_norm_rms_epsilon");
    if (eps > 0) cfg.norm_eps = eps;
    cfg.vocab_size = field_u32("vocab_size");
    if (cfg.vocab_size == 0) {
        auto it = kv.find("tokenizer.ggml.tokens");
        if (it != kv.end() && it->second.kind == Value::ArrStr) cfg.vocab_size = (uint32_t)it->second.arr_len;
    }
    if (cfg.n_head_kv == 0) cfg.n_head_kv = cfg.n_head;
    return true;
}

}  // namespace cllm_hip
