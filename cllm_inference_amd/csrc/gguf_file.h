// gguf_file.h -- the GGUF container as the linear path needs it: the tensor table, the
// 32-byte-aligned data section and the model hyper-parameters, read the way the
// reference's GgufLoader::load reads them (src/core/gguf.cpp:122-275). Host code only.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace cllm_hip {

struct GgufTensor {
    std::string name;
    uint32_t type = 0;
    std::vector<uint64_t> shape;  // rows first: the file's dims in reverse (gguf.cpp:163-165)
    uint64_t offset = 0;          // from the start of the data section
};

struct GgufConfig {
    std::string arch;
    uint32_t n_layers = 0, n_embd = 0, n_head = 0, n_head_kv = 0, n_ctx = 0, n_ff = 0;
    uint32_t vocab_size = 0, head_dim_explicit = 0;
    float rope_theta = 10000.0f, norm_eps = 1e-5f;
};

struct GgufFile {
    std::vector<GgufTensor> tensors;          // file order
    std::unordered_map<std::string, int> index;
    GgufConfig config;
    uint32_t version = 0;
    void* map = nullptr;                      // whole file, read-only, MAP_PRIVATE
    size_t map_bytes = 0;
    size_t data_offset = 0;                   // 32-byte aligned start of the data section
    ~GgufFile();
};

// Parses `path` and maps it. On failure returns false with the reference's message in err.
bool gguf_open(const char* path, GgufFile& out, std::string& err);

}  // namespace cllm_hip
