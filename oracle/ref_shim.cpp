// ref_shim.cpp -- extern "C" entry points over the reference's own Quant API, so that
// tests/golden/make_golden.py and bench.py's cpu_baseline leg can drive the reference
// compiled from its unmodified sources (src/core/quant.cpp, src/core/thread_pool.cpp).
//
// TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile into oracle/_ref/, never shipped.
// Interfaces wrapped: include/cllm/core/quant.hpp:90-151, include/cllm/core/thread_pool.hpp:12-24,
// include/cllm/core/gguf.hpp:79-82 (GgufLoader::load, for the GGUF reader's parity),
// include/cllm/core/engine.hpp:24-49 (TransformerEngine, for the device forward's parity).
#include "cllm/core/engine.hpp"
#include "cllm/core/gguf.hpp"
#include "cllm/core/quant.hpp"
#include "cllm/core/thread_pool.hpp"

#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <mutex>

namespace {
thread_local char g_err[256];
std::mutex g_pool_mtx;
std::unique_ptr<cllm::ThreadPool> g_pool;
size_t g_pool_threads = 0;

int set_err(const std::exception& e) {
    std::snprintf(g_err, sizeof g_err, "%s", e.what());
    return 1;
}

// n_threads <= 0: no pool (serial, as the reference's tests call it). Otherwise a pool of
// exactly n_threads workers, kept across calls like the engine keeps its pool.
cllm::ThreadPool* pool_for(int n_threads) {
    if (n_threads <= 0) return nullptr;
    std::lock_guard<std::mutex> lk(g_pool_mtx);
    if (!g_pool || g_pool_threads != (size_t)n_threads) {
        g_pool.reset();
        g_pool = std::make_unique<cllm::ThreadPool>((size_t)n_threads);
        g_pool_threads = (size_t)n_threads;
    }
    return g_pool.get();
}
}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_err; }

int ref_block_size(uint32_t t) { return cllm::block_size((cllm::GgmlType)t); }
size_t ref_type_size(uint32_t t) { return cllm::type_size((cllm::GgmlType)t); }
int ref_has_vec_dot(uint32_t t) { return cllm::has_vec_dot((cllm::GgmlType)t) ? 1 : 0; }

int ref_quantize_row_q8_0(const float* x, int64_t n, int8_t* qs, float* scales, int32_t* bsums) {
    try {
        cllm::QuantizedQ8_0 q;
        cllm::quantize_row_q8_0(x, q, n);
        std::memcpy(qs, q.qs.data(), q.qs.size());
        std::memcpy(scales, q.scales.data(), q.scales.size() * sizeof(float));
        std::memcpy(bsums, q.bsums.data(), q.bsums.size() * sizeof(int32_t));
        return 0;
    } catch (const std::exception& e) {
        return set_err(e);
    }
}

int ref_dequantize(const void* src, float* dst, uint32_t t, int64_t n) {
    try {
        cllm::dequantize_block(src, dst, (cllm::GgmlType)t, n);
        return 0;
    } catch (const std::exception& e) {
        return set_err(e);
    }
}

int ref_dequantize_f16(const void* src, uint16_t* dst, uint32_t t, int64_t n) {
    try {
        cllm::dequantize_block_f16(src, dst, (cllm::GgmlType)t, n);
        return 0;
    } catch (const std::exception& e) {
        return set_err(e);
    }
}

uint16_t ref_float_to_half(float f) { return cllm::float_to_half(f); }

int ref_matmul_quant(const float* x, const void* w, uint32_t t, const float* bias, int in_dim,
                     int out_dim, float* y, int n_threads) {
    try {
        cllm::matmul_quant(x, w, (cllm::GgmlType)t, bias, in_dim, out_dim, y, pool_for(n_threads));
        return 0;
    } catch (const std::exception& e) {
        return set_err(e);
    }
}

int ref_matmul_quant_batch(const float* x, const void* w, uint32_t t, const float* bias,
                           int in_dim, int out_dim, int n_rows, float* y, int n_threads) {
    try {
        cllm::matmul_quant_batch(x, w, (cllm::GgmlType)t, bias, in_dim, out_dim, n_rows, y,
                                 pool_for(n_threads));
        return 0;
    } catch (const std::exception& e) {
        return set_err(e);
    }
}

}  // extern "C"

// GgufLoader::load of path, written as text into buf (cap bytes): one line
//   arch n_layers n_embd n_head n_head_kv n_ctx n_ff vocab_size head_dim rope_theta norm_eps
// (floats as %a), then one line per tensor in file order:
//   name type n_dims dim... offset data_delta
// where data_delta is the tensor's data pointer minus the mapping's base. Returns the length
// written (truncated at cap), or -1 with ref_last_error() set.
extern "C" long ref_gguf_dump(const char* path, char* buf, size_t cap) {
    try {
        cllm::GgufModel m = cllm::GgufLoader::load(path);
        std::string out;
        char line[512];
        const cllm::ModelConfig& c = m.config;
        std::snprintf(line, sizeof line, "%s %u %u %u %u %u %u %u %u %a %a\n",
                      c.arch.empty() ? "-" : c.arch.c_str(), c.n_layers, c.n_embd, c.n_head,
                      c.n_head_kv, c.n_ctx, c.n_ff, c.vocab_size,
                      c.n_head ? c.head_dim() : c.head_dim_explicit, (double)c.rope_theta,
                      (double)c.norm_eps);
        out += line;
        std::vector<std::pair<std::string, const cllm::Tensor*>> named;
        for (const auto& kv : m.tensors) named.emplace_back(kv.first, &kv.second);
        for (const cllm::Tensor& t : m.tensor_list) {
            const std::string* name = nullptr;
            for (const auto& nt : named)
                if (nt.second->data == t.data && nt.second->offset == t.offset) name = &nt.first;
            std::snprintf(line, sizeof line, "%s %u %zu", name ? name->c_str() : "?",
                          (unsigned)t.type, t.shape.size());
            out += line;
            for (uint32_t d : t.shape) {
                std::snprintf(line, sizeof line, " %u", d);
                out += line;
            }
            std::snprintf(line, sizeof line, " %llu %lld\n", (unsigned long long)t.offset,
                          (long long)((const char*)t.data - (const char*)m.mmap_base));
            out += line;
        }
        const size_t n = out.size() < cap ? out.size() : cap;
        std::memcpy(buf, out.data(), n);
        return (long)n;
    } catch (const std::exception& e) {
        set_err(e);
        return -1;
    }
}


// Logits of the reference engine (Quant weight mode, a pool of `threads` workers) on the model
// file path: with use_prefill, prefill(tokens) (the last token's logits, vocab floats);
// otherwise forward(tokens[t]) for each t in turn (n * vocab floats). Returns the number of
// floats written, or -1 with ref_last_error() set.
extern "C" long ref_engine_logits(const char* path, const int* tokens, int n, int use_prefill,
                                  int threads, float* out, size_t cap) {
    try {
        cllm::GgufModel m = cllm::GgufLoader::load(path);
        cllm::ThreadPool pool((size_t)(threads > 0 ? threads : 1));
        cllm::TransformerEngine eng(m, pool);
        size_t at = 0;
        auto put = [&](const std::vector<float>& v) {
            if (at + v.size() > cap) throw std::runtime_error("ref_engine_logits: output too small");
            std::memcpy(out + at, v.data(), v.size() * sizeof(float));
            at += v.size();
        };
        if (use_prefill) {
            put(eng.prefill(std::vector<int>(tokens, tokens + n)));
        } else {
            for (int t = 0; t < n; ++t) put(eng.forward(tokens[t], true));
        }
        return (long)at;
    } catch (const std::exception& e) {
        set_err(e);
        return -1;
    }
}
