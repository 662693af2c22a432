// capi.hip -- the extern "C" boundary of libcllm_hip.so (declared in include/cllm_hip.h).
//
// Host-pointer entry points follow the reference's synchronous contract
// (src/core/quant.cpp:1374-1475): validate in the reference's order with its messages,
// quantize the activation rows once, run every weight row against them, return with y
// written. Device-pointer entry points do the same work stream-ordered.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <barrier>
#include <mutex>
#include <set>
#include <thread>
#include <vector>
#include <string>

#include <fcntl.h>
#include <sys/ioctl.h>
#include <sys/stat.h>
#include <sys/sysmacros.h>
#include <unistd.h>
#include <cerrno>

#include "../../include/cllm_hip.h"
#include "ggml_blocks.h"
#include "gguf_file.h"
#include "launch.h"

using namespace cllm_hip;

namespace {

thread_local char g_err[512] = "";
thread_local int g_device = -1;

// Minimum activation rows for the int8-MFMA path; below it the weight-streaming GEMV wins.
constexpr int kMfmaMinRows = 16;

int set_err(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int set_err(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

#define HIP_TRY(expr)                                                                        \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess)                                                                \
            return set_err(CLLM_HIP_E_RUNTIME, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// Every device (and pinned host) allocation the library makes goes through here, counted, so
// a caller can check that an entry point allocated nothing (cllm_hip_allocation_count).
std::atomic<uint64_t> g_allocations{0};

hipError_t dev_alloc(void** p, size_t bytes) {
    g_allocations.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc(p, bytes);
}

// A device allocation that only grows.
struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    // Grows to at least `bytes`. `stream` is synchronised first so no queued kernel still
    // reads the old allocation.
    hipError_t ensure(size_t bytes, hipStream_t stream) {
        if (bytes <= cap) return hipSuccess;
        size_t want = cap ? cap : (size_t)1 << 20;
        while (want < bytes) want *= 2;
        if (p) {
            hipError_t e = hipStreamSynchronize(stream);
            if (e != hipSuccess) return e;
            e = hipFree(p);
            if (e != hipSuccess) return e;
            p = nullptr;
            cap = 0;
        }
        hipError_t e = dev_alloc(&p, want);
        if (e != hipSuccess) return e;
        cap = want;
        return hipSuccess;
    }
};

// The scratch one matmul call uses, as plain device pointers: the Q8_0 batch qs[m*k] |
// scales[m*k/32] | bsums[m*k/32], the MFMA paths' qh[m*k] (fp16) | px[m*k/32] (dx * bsum) |
// xq[m*k/8] (dx * bsum as bf16 parts), and the weight-row GEMM's split-K region (tile
// counters that must be zero when a launch starts, then the partial sums).
struct WsView {
    int8_t* qs = nullptr;
    float* sc = nullptr;
    int32_t* bs = nullptr;
    _Float16* qh = nullptr;
    float* px = nullptr;
    uint16_t* xq = nullptr;
    float* part = nullptr;
    size_t part_cap = 0;
};

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Bytes of the activation arrays of a k x m batch, and their places from base p.
size_t act_bytes(int k, int m) {
    const size_t n = (size_t)k * (size_t)m;
    return round256(n) + 3 * round256((n / 32) * 4) + round256(2 * n) + round256(n / 4);
}
void carve_act(char* p, int k, int m, WsView& v) {
    const size_t n = (size_t)k * (size_t)m;
    const size_t qs_bytes = round256(n), sc_bytes = round256((n / 32) * 4), qh_bytes = round256(2 * n);
    v.qs = (int8_t*)p;
    v.sc = (float*)(p + qs_bytes);
    v.bs = (int32_t*)(p + qs_bytes + sc_bytes);
    v.px = (float*)(p + qs_bytes + 2 * sc_bytes);
    v.qh = (_Float16*)(p + qs_bytes + 3 * sc_bytes);
    v.xq = (uint16_t*)(p + qs_bytes + 3 * sc_bytes + qh_bytes);
}

// The weight-row kernels' activation format in a caller's buffer (cllm_hip_mfma_act_bytes):
// the Q8_0 scales xs[m * k / 32], the codes as fp16 qh[m * k], and the minimum-term operand
// xq[m * k / 8], each at a multiple of 256 bytes.
size_t mfma_act_bytes(int k, int m) {
    const size_t n = (size_t)k * (size_t)m;
    return round256((n / 32) * 4) + round256(2 * n) + round256(n / 4);
}
void carve_mfma(const void* act, int k, int m, float** xs, _Float16** qh, uint16_t** xq) {
    const size_t n = (size_t)k * (size_t)m;
    char* p = (char*)act;
    *xs = (float*)p;
    *qh = (_Float16*)(p + round256((n / 32) * 4));
    *xq = (uint16_t*)(p + round256((n / 32) * 4) + round256(2 * n));
}

// A growable workspace of the library's own (per device stream, or per device for the host
// entry points).
struct Workspace {
    DevBuf buf;
    DevBuf part;  // split-K partial sums of the weight-row GEMM
    DevBuf att;   // sequence-split partials of the attention kernel
    DevBuf tmp;   // matmul result before a residual add the kernel cannot fuse
    WsView v;
    hipError_t ensure(int k, int m, hipStream_t stream) {
        hipError_t e = buf.ensure(act_bytes(k, m), stream);
        if (e != hipSuccess) return e;
        carve_act((char*)buf.p, k, m, v);
        return hipSuccess;
    }
    // The weight-row GEMM's split-K region; a new allocation is zeroed (its tile counters
    // must start at zero; every launch leaves them zero).
    hipError_t ensure_part(size_t bytes, hipStream_t stream) {
        if (bytes == 0) return hipSuccess;
        const void* before = part.p;
        hipError_t e = part.ensure(bytes, stream);
        if (e != hipSuccess) return e;
        if (part.p != before) e = gemmw_workspace_init(part.p, part.cap, stream);
        v.part = (float*)part.p;
        v.part_cap = part.cap;
        return e;
    }
};

// A host address range whose bytes have a device copy. Automatic regions are read-only file
// mappings found by resolve_weights; they carry the mapping's identity and the mapped file's
// size and times, so a range that was unmapped (and perhaps mapped again with other contents),
// or whose file was rewritten in place, is noticed and dropped.
struct Region {
    size_t bytes;
    void* dev;    // device address of the region's first byte
    void* alloc;  // the allocation to free
    bool automatic = false;
    uint64_t file_off = 0, inode = 0;
    uint32_t dev_major = 0, dev_minor = 0;
    int fd = -1;  // the mapped file, opened at the copy (-1: no longer reachable by its path)
    struct stat at_copy = {};
};

// One mapping (VMA) of this process.
struct Mapping {
    uintptr_t lo = 0, hi = 0;
    bool readable = false, writable = false, shared = false;
    uint64_t off = 0, inode = 0;
    uint32_t dev_major = 0, dev_minor = 0;
    bool file = false;  // backed by a file with a path name
    std::string path;   // filled when asked for
};

// The mapping of this process that holds address p, parsed from /proc/self/maps.
bool parse_mapping(uintptr_t p, Mapping& m, bool want_path) {
    FILE* f = std::fopen("/proc/self/maps", "r");
    if (!f) return false;
    char line[4096];
    bool found = false;
    while (!found && std::fgets(line, sizeof line, f)) {
        unsigned long lo = 0, hi = 0, off = 0, ino = 0;
        unsigned maj = 0, mnr = 0;
        char perms[8] = {};
        int pos = 0;
        if (std::sscanf(line, "%lx-%lx %7s %lx %x:%x %lu %n", &lo, &hi, perms, &off, &maj, &mnr, &ino, &pos) < 7)
            continue;
        if (p < lo || p >= hi) continue;
        m = Mapping{};
        m.lo = lo;
        m.hi = hi;
        m.readable = perms[0] == 'r';
        m.writable = perms[1] == 'w';
        m.shared = perms[3] == 's';
        m.off = off;
        m.inode = ino;
        m.dev_major = maj;
        m.dev_minor = mnr;
        m.file = pos > 0 && line[pos] == '/';
        if (m.file && want_path) {
            m.path.assign(line + pos);
            while (!m.path.empty() && (m.path.back() == '\n' || m.path.back() == '\r')) m.path.pop_back();
        }
        found = true;
    }
    std::fclose(f);
    return found;
}

// The kernel's one-address query of a process's mappings (PROCMAP_QUERY, an ioctl on an open
// /proc/<pid>/maps, Linux 6.11 and later; uapi linux/fs.h). The layout is the kernel's ABI;
// the system headers of this build predate it.
struct ProcmapQuery {
    uint64_t size, query_flags, query_addr;
    uint64_t vma_start, vma_end, vma_flags, vma_page_size, vma_offset, inode;
    uint32_t dev_major, dev_minor, vma_name_size, build_id_size;
    uint64_t vma_name_addr, build_id_addr;
};
static_assert(sizeof(ProcmapQuery) == 104, "struct procmap_query is 104 bytes");
constexpr unsigned long kProcmapQuery = _IOWR('f', 17, ProcmapQuery);
constexpr uint64_t kVmaReadable = 1, kVmaWritable = 2, kVmaShared = 8;

std::mutex g_maps_mtx;
int g_maps_fd = -1;       // /proc/self/maps of process g_maps_pid
pid_t g_maps_pid = -1;
bool g_maps_query = true;  // false once the kernel has refused the query

// The mapping of this process that holds address p: one PROCMAP_QUERY (about 0.3 us) where
// the kernel has it, else a parse of /proc/self/maps (hundreds of us with HIP loaded).
bool find_mapping(uintptr_t p, Mapping& m, bool want_path = false) {
    {
        std::lock_guard<std::mutex> lk(g_maps_mtx);
        if (g_maps_query) {
            const pid_t pid = getpid();  // a forked child must not query its parent's mappings
            if (g_maps_fd >= 0 && g_maps_pid != pid) {
                ::close(g_maps_fd);
                g_maps_fd = -1;
            }
            if (g_maps_fd < 0) {
                g_maps_fd = ::open("/proc/self/maps", O_RDONLY | O_CLOEXEC);
                g_maps_pid = pid;
            }
            char name[4096];
            ProcmapQuery q = {};
            q.size = sizeof q;
            q.query_addr = p;
            if (want_path) {
                q.vma_name_size = sizeof name;
                q.vma_name_addr = (uint64_t)(uintptr_t)name;
            }
            if (g_maps_fd >= 0 && ::ioctl(g_maps_fd, kProcmapQuery, &q) == 0) {
                m = Mapping{};
                m.lo = q.vma_start;
                m.hi = q.vma_end;
                m.readable = q.vma_flags & kVmaReadable;
                m.writable = q.vma_flags & kVmaWritable;
                m.shared = q.vma_flags & kVmaShared;
                m.off = q.vma_offset;
                m.inode = q.inode;
                m.dev_major = q.dev_major;
                m.dev_minor = q.dev_minor;
                m.file = q.inode != 0;
                if (want_path && q.vma_name_size > 0) m.path.assign(name);
                return p >= m.lo && p < m.hi;
            }
            if (errno == ENOENT) return false;  // no mapping holds p
            if (errno == ENOTTY || errno == EINVAL || errno == EOPNOTSUPP) g_maps_query = false;
        }
    }
    return parse_mapping(p, m, want_path);
}

// A private, read-only mapping of a file: what GgufLoader maps (gguf.cpp:178). Its bytes
// cannot change through the mapping, so one device copy serves every later call.
bool immutable_file_mapping(const Mapping& m) {
    return m.file && m.readable && !m.writable && !m.shared && m.inode != 0;
}

// Fixed scratch of cllm_hip_matmul_quant_static_dev, one copy per GPU for the life of the
// process. Host code never uses this name as an address: each device's copy is found with
// hipGetSymbolAddress when its state is built (DeviceState::scratch).
constexpr size_t kStaticScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

struct DeviceState {
    std::mutex mtx;
    hipStream_t stream = nullptr;
    uint8_t* scratch = nullptr;  // this device's copy of the static scratch array
    // the last eager call on the static scratch: its stream and an event after its work
    std::mutex static_mtx;
    hipEvent_t static_done = nullptr;
    hipStream_t static_last = nullptr;
    bool static_pending = false;
    DevBuf x, y, bias, wstage, qin;
    Workspace act;
    std::map<uintptr_t, Region> regions;  // host base -> device copy
    std::set<uintptr_t> no_auto;          // mappings too large to copy to the device
    std::map<hipStream_t, std::unique_ptr<Workspace>> dev_ws;
};

std::mutex g_states_mtx;
std::map<int, std::unique_ptr<DeviceState>> g_states;

int current_device() { return g_device < 0 ? 0 : g_device; }

Tuning g_tuning;

// Makes the calling thread's device current and returns its state (created on first use).
int acquire(DeviceState** out) {
    const int dev = current_device();
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        (void)hipGetLastError();
        return set_err(CLLM_HIP_E_NODEV, "cllm_hip: no HIP device available");
    }
    if (dev >= count) return set_err(CLLM_HIP_E_NODEV, "cllm_hip: device %d not present", dev);
    HIP_TRY(hipSetDevice(dev));
    std::lock_guard<std::mutex> lk(g_states_mtx);
    auto it = g_states.find(dev);
    if (it == g_states.end()) {
        hipDeviceProp_t prop;
        HIP_TRY(hipGetDeviceProperties(&prop, dev));
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            return set_err(CLLM_HIP_E_NODEV,
                           "cllm_hip: device %d is %s; this library is built for gfx950 only", dev,
                           prop.gcnArchName);
        auto st = std::make_unique<DeviceState>();
        HIP_TRY(hipStreamCreateWithFlags(&st->stream, hipStreamNonBlocking));
        // the device is current: its copy of the static scratch array
        HIP_TRY(hipGetSymbolAddress((void**)&st->scratch, HIP_SYMBOL(scratch)));
        if (st->scratch == nullptr || ((uintptr_t)st->scratch & 255u))
            return set_err(CLLM_HIP_E_RUNTIME, "cllm_hip: static scratch of device %d not found", dev);
        HIP_TRY(hipEventCreateWithFlags(&st->static_done, hipEventDisableTiming));
        it = g_states.emplace(dev, std::move(st)).first;
    }
    *out = it->second.get();
    return CLLM_HIP_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

size_t row_bytes(uint32_t type, int in_dim) {
    return (size_t)(in_dim / block_elems(type)) * block_bytes(type);
}

// The reference's checks, in its order (quant.cpp:1376-1380 / 1441-1444). Types without a
// vec_dot kernel take the float-dot kernels (the reference's dequantize fallback,
// 1404-1430), which fail only for an id that is no GGML type (dequantize_block, 387).
int check_matmul(const char* who, uint32_t type, int in_dim, int out_dim) {
    const int bs = block_elems(type);
    if (bs <= 0 || in_dim <= 0 || in_dim % bs != 0)
        return set_err(CLLM_HIP_E_SHAPE, "%s: in_dim not divisible by block size", who);
    if (!has_kernel(type) && !gemv_f_supported(type))
        return set_err(CLLM_HIP_E_TYPE, "unsupported ggml type for dequantize");
    if (out_dim < 0) return set_err(CLLM_HIP_E_ARG, "%s: negative out_dim", who);
    return CLLM_HIP_OK;
}

bool is_device_ptr(const void* p) {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

// Copies [a, a + bytes) of host memory to a new device allocation. The copy keeps the host
// base's offset modulo 256, so host pointers that are 16-byte aligned stay 16-byte aligned on
// the device. On failure nothing is left allocated.
int upload_region(DeviceState* st, uintptr_t a, size_t bytes, Region* out) {
    const size_t lead = a & 255u;
    void* mem = nullptr;
    hipError_t e = dev_alloc(&mem, bytes + lead);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_err(CLLM_HIP_E_RUNTIME, "cllm_hip: cannot allocate %zu bytes for weights: %s",
                       bytes, hipGetErrorString(e));
    }
    e = hipMemcpyAsync((char*)mem + lead, (const void*)a, bytes, hipMemcpyHostToDevice, st->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(st->stream);
    if (e != hipSuccess) {
        (void)hipFree(mem);
        return set_err(CLLM_HIP_E_RUNTIME, "cllm_hip: weight upload failed: %s", hipGetErrorString(e));
    }
    *out = Region{bytes, (char*)mem + lead, mem};
    return CLLM_HIP_OK;
}

// An automatic region is still backed by the read-only file mapping it was copied from, and
// that file still has the size and times it had at the copy. A rewrite in place (same inode)
// changes the times; one of the same size within one timestamp tick of the copy is not seen.
bool same_mapping(uintptr_t base, const Region& r, const Mapping& m) {
    if (!(m.lo == base && m.hi - m.lo == r.bytes && m.inode == r.inode && m.off == r.file_off &&
          m.dev_major == r.dev_major && m.dev_minor == r.dev_minor && immutable_file_mapping(m)))
        return false;
    if (r.fd < 0) return true;
    struct stat now;
    if (::fstat(r.fd, &now) != 0) return false;
    return now.st_ino == r.at_copy.st_ino && now.st_size == r.at_copy.st_size &&
           now.st_mtim.tv_sec == r.at_copy.st_mtim.tv_sec &&
           now.st_mtim.tv_nsec == r.at_copy.st_mtim.tv_nsec &&
           now.st_ctim.tv_sec == r.at_copy.st_ctim.tv_sec &&
           now.st_ctim.tv_nsec == r.at_copy.st_ctim.tv_nsec;
}

// Frees a region's device copy (after the stream's work that may read it) and its file.
int drop_region(DeviceState* st, std::map<uintptr_t, Region>::iterator it) {
    HIP_TRY(hipStreamSynchronize(st->stream));
    HIP_TRY(hipFree(it->second.alloc));
    if (it->second.fd >= 0) ::close(it->second.fd);
    st->regions.erase(it);
    return CLLM_HIP_OK;
}

// An automatic region is live while its mapping and file are unchanged.
bool auto_region_live(uintptr_t base, const Region& r) {
    Mapping m;
    return find_mapping(base, m) && same_mapping(base, r, m);
}

// Frees the automatic regions whose file mappings are gone or changed.
int prune_auto_regions(DeviceState* st) {
    for (auto it = st->regions.begin(); it != st->regions.end();) {
        if (!it->second.automatic || auto_region_live(it->first, it->second)) {
            ++it;
            continue;
        }
        auto dead = it++;
        int rc = drop_region(st, dead);
        if (rc) return rc;
    }
    return CLLM_HIP_OK;
}

// The device copy of [a, a + bytes) if a registered region holds it (null if none). An
// automatic region is checked against the current mapping and file first (one mapping query
// and one fstat), and dropped if either changed since the copy.
int lookup_region(DeviceState* st, uintptr_t a, size_t bytes, const uint8_t** dev) {
    *dev = nullptr;
    auto it = st->regions.upper_bound(a);
    if (it == st->regions.begin()) return CLLM_HIP_OK;
    --it;
    if (a < it->first || a + bytes > it->first + it->second.bytes) return CLLM_HIP_OK;
    if (it->second.automatic && !auto_region_live(it->first, it->second)) return drop_region(st, it);
    *dev = (const uint8_t*)it->second.dev + (a - it->first);
    return CLLM_HIP_OK;
}

// Opens the file behind an automatic region and records its identity and times. The path
// must still name the mapped inode; otherwise (unlinked or replaced) fd stays -1 and the
// region is checked by its mapping alone, since no path reaches the mapped file any more.
void watch_file(const Mapping& m, Region& r) {
    if (m.path.empty() || m.path[0] != '/') return;
    const int fd = ::open(m.path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return;
    struct stat sb;
    if (::fstat(fd, &sb) == 0 && sb.st_ino == m.inode && major(sb.st_dev) == m.dev_major &&
        minor(sb.st_dev) == m.dev_minor) {
        r.fd = fd;
        r.at_copy = sb;
        return;
    }
    ::close(fd);
}

// Device address of `bytes` of weights at host/device pointer w. Registered regions resolve
// by offset; device pointers pass through; a read-only file mapping is copied to the device
// once; anything else is copied into a staging buffer.
int resolve_weights(DeviceState* st, const void* w, size_t bytes, const uint8_t** dev) {
    const uintptr_t a = (uintptr_t)w;
    int rc;
    if ((rc = lookup_region(st, a, bytes, dev))) return rc;
    if (*dev) {
        if (!aligned16(*dev))
            return set_err(CLLM_HIP_E_ARG, "cllm_hip: weight pointer is not 16-byte aligned");
        return CLLM_HIP_OK;
    }
    if (is_device_ptr(w)) {
        if (!aligned16(w))
            return set_err(CLLM_HIP_E_ARG, "cllm_hip: weight pointer is not 16-byte aligned");
        *dev = (const uint8_t*)w;
        return CLLM_HIP_OK;
    }
    // Weights inside a read-only private file mapping (the engine's mmap'd GGUF file): the
    // whole mapping goes to the device once and later calls resolve by offset, as after
    // cllm_hip_register_weights. If the device cannot hold it, the bytes are copied per call.
    Mapping m;
    if (find_mapping(a, m, true) && immutable_file_mapping(m) && a + bytes <= m.hi &&
        st->no_auto.count(m.lo) == 0) {
        if ((rc = prune_auto_regions(st))) return rc;
        Region r;
        if (st->regions.count(m.lo) == 0 && upload_region(st, m.lo, m.hi - m.lo, &r) == CLLM_HIP_OK) {
            r.automatic = true;
            r.file_off = m.off;
            r.inode = m.inode;
            r.dev_major = m.dev_major;
            r.dev_minor = m.dev_minor;
            watch_file(m, r);
            st->regions[m.lo] = r;
            *dev = (const uint8_t*)r.dev + (a - m.lo);
            if (!aligned16(*dev))
                return set_err(CLLM_HIP_E_ARG, "cllm_hip: weight pointer is not 16-byte aligned");
            return CLLM_HIP_OK;
        }
        st->no_auto.insert(m.lo);
    }
    HIP_TRY(st->wstage.ensure(bytes, st->stream));
    HIP_TRY(hipMemcpyAsync(st->wstage.p, w, bytes, hipMemcpyHostToDevice, st->stream));
    *dev = (const uint8_t*)st->wstage.p;
    return CLLM_HIP_OK;
}

// Device address of `bytes` at src for a kernel that needs a 16-byte-aligned start: a
// registered region or a device pointer is used in place when aligned, and anything else
// (host memory, a misaligned device address) is first copied into the staging buffer.
int resolve_span(DeviceState* st, const void* src, size_t bytes, const uint8_t** dev) {
    const uint8_t* d = nullptr;
    int rc;
    if ((rc = lookup_region(st, (uintptr_t)src, bytes, &d))) return rc;
    if (!d && is_device_ptr(src)) d = (const uint8_t*)src;
    if (d && aligned16(d)) {
        *dev = d;
        return CLLM_HIP_OK;
    }
    HIP_TRY(st->wstage.ensure(bytes, st->stream));
    HIP_TRY(hipMemcpyAsync(st->wstage.p, d ? (const void*)d : src, bytes,
                           d ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st->stream));
    *dev = (const uint8_t*)st->wstage.p;
    return CLLM_HIP_OK;
}

// dequantize_block / dequantize_block_f16 into host memory, in passes of at most 2^26
// elements (a multiple of every block size) so the device staging stays bounded.
int dequantize_host(const char* who, const void* src, float* dst32, uint16_t* dst16,
                    uint32_t type, int64_t n) {
    if (!has_kernel(type) && !gemv_f_supported(type))
        return set_err(CLLM_HIP_E_TYPE, "unsupported ggml type for dequantize");
    if (n <= 0) return CLLM_HIP_OK;
    if (!src || (!dst32 && !dst16)) return set_err(CLLM_HIP_E_ARG, "%s: null pointer", who);
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(st->mtx);
    const int64_t bs = block_elems(type);
    const size_t ts = block_bytes(type);
    const size_t esz = dst16 ? sizeof(uint16_t) : sizeof(float);
    constexpr int64_t kPass = (int64_t)1 << 26;
    HIP_TRY(st->y.ensure((size_t)std::min(n, kPass) * esz, st->stream));
    for (int64_t at = 0; at < n; at += kPass) {
        const int64_t len = std::min(kPass, n - at);
        const uint8_t* s = (const uint8_t*)src + (size_t)(at / bs) * ts;
        const uint8_t* d = nullptr;
        if ((rc = resolve_span(st, s, (size_t)((len + bs - 1) / bs) * ts, &d))) return rc;
        void* out = dst16 ? (void*)(dst16 + at) : (void*)(dst32 + at);
        if (dst16 && type == T_F16) {
            // binary16 blocks are copied as they are (quant.cpp:400-403)
            HIP_TRY(hipMemcpyAsync(out, d, (size_t)len * esz, hipMemcpyDeviceToHost, st->stream));
        } else {
            HIP_TRY(launch_dequantize_span(type, d, len, dst16 ? nullptr : (float*)st->y.p,
                                           dst16 ? (uint16_t*)st->y.p : nullptr, st->stream));
            HIP_TRY(hipMemcpyAsync(out, st->y.p, (size_t)len * esz, hipMemcpyDeviceToHost, st->stream));
        }
        // the staging buffers are reused by the next pass
        HIP_TRY(hipStreamSynchronize(st->stream));
    }
    return CLLM_HIP_OK;
}

bool gemm_forced();

// Small batches of the types k_gemm_sm.hip has take it (the weights streamed once for the whole
// batch, int8 MFMA), unless a kernel choice is forced: from 8 rows, up to 32 rows of the
// K-quants and 64 of Q8_0. Measured on MI355X (fused step, cold weights, us): Q5_K 14336x4096
// at 4 / 8 / 16 / 32 / 64 rows 21.3 / 19.5 / 20.7 / 29.0 / 49 against 17.4 (GEMV) / 28.7 /
// 27.7 / 28.9 / 43.5 (MFMA); Q8_0 4096x4096 at 4 / 8 / 16 / 64 rows 13.6 / 13.5 / 12.4 / 20.9
// against 10.2 / 12.8 / 22.0 / 30.6.
// Above 16 rows the K-quants of at least kSmallMaxN output rows take the weight-row MFMA
// kernel instead: Q5_K 14336x4096 at 20 / 24 / 28 / 32 rows 25.9 / 26.5 / 26.5 / 27.0 us
// against 28.2 / 28.6 / 28.8 / 29.6 (Q4_K 4096x4096 and 1024x4096 stay faster here: 15.3
// against 18.9 us at 32 rows).
constexpr int kSmallMinRows = 8;
constexpr int kSmallMaxN = 8192;

bool use_small(uint32_t type, int k, int n, int m) {
    const int knob = tuning().gemm_small.load(std::memory_order_relaxed);
    if (knob == 2 || tuning().gemm_kind.load(std::memory_order_relaxed) != 0 ||
        !gemm_sm_supported(type, k, m))
        return false;
    if (knob == 1) return m >= 3;
    if (type == T_Q6_K) {
        // up to 16 rows (one token tile; two ran 55-57 us on the large shapes against 35-36 on
        // the weight-row kernel), where the GEMV would need two launches or more, or from 4
        // rows on matrices of 32 M weights or more. MI355X, cold weights, us, small-batch
        // kernel against the previous route:
        //   Q6_K 4096x14336, 4 / 8 / 16 rows:  22.1 / 22.3 / 23.2 against 31.5 / 34.9 / 35.7
        //   Q6_K 14336x4096, 4 / 8 / 16 rows:  21.0 / 21.3 / 22.1 against 20.9 / 29.9 / 34.2
        //   Q6_K 1024x4096,  4 / 7 / 8 / 16:   11.3 / 11.4 / 11.5 / 11.4 against 7.4 / 15.6 / 10.3 / 20.4
        // A batch of up to 5 rows the GEMV streams in one launch stays there. MI355X, cold
        // weights, us, streaming GEMV (quantizing in-kernel) against this kernel:
        //   Q6_K 4096x14336, 2 / 3 / 4 rows:   15.6 / 15.3 / 17.3 against 22.1 / 22.1 / 21.7
        //   Q6_K 14336x4096, 5 / 6 rows:       19.2 / 21.8 against 21.4 / 21.3
        if (m <= 5 && gemv_streams_batch(type, k, n, m)) return false;
        const bool large = (int64_t)n * k >= (int64_t(32) << 20);
        return m >= 4 && m <= 16 && (large || gemv_launch_count(type, k, m) >= 2);
    }
    if (type == T_Q4_0 || type == T_Q5_0) {
        // from 8 rows (9 where the GEMV streams the batch in one launch), against the weight-row
        // kernel. MI355X, cold weights, us, this kernel against the previous route:
        //   Q4_0 14336x4096, 9 / 16 / 32 / 64 rows:  17.5 / 17.8 / 26.6 / 42.6 against 23.8 / 24.2 / 25.5 / 44.8
        //   Q5_0 14336x4096, 9 / 16 / 32 / 64 rows:  19.0 / 19.3 / 27.8 / 43.7 against 25.8 / 26.3 / 27.6 / 47.0
        //   Q4_0 4096x4096,  9 / 16 / 32 / 64 rows:  10.4 / 10.6 / 14.2 / 18.6 against 17.5 / 19.8 / 20.5 / 27.5
        //   Q4_0 4096x14336, 8 / 16 / 32 / 64 rows:  17.6 / 17.9 / 28.9 / 56.8 against 30.1 / 30.7 / 31.9 / 43.5
        if (m < (gemv_streams_batch(type, k, n, m) ? 9 : 8)) return false;
        if (k > 4096) return m <= 32;
        return n < kSmallMaxN || m <= 16 || m > 32;
    }
    if (type != T_Q8_0 && m > 16 && n >= kSmallMaxN) return false;
    // Where the GEMV streams the whole batch in one launch it keeps Q8_0 up to 8 rows, Q5_K up
    // to 6 and Q4_K up to 7. MI355X, cold weights, us, streaming GEMV (in-kernel quantization
    // up to 7 rows) against this kernel:
    //   Q8_0 4096x4096,  4 / 6 / 8 rows:  7.7 / 9.1 / 10.6 against 11.1 / 11.2 / 11.4
    //   Q5_K 14336x4096, 5 / 6 / 7 rows:  16.3 / ~16.9 / ~18.3 against 17.6 / 17.6 / 17.6
    //   Q4_K 14336x4096, 7 / 8 rows:      17.2 / 18.6 against 17.8 / 17.6
    int lo = kSmallMinRows;
    if (gemv_streams_batch(type, k, n, m)) lo = type == T_Q8_0 ? 9 : type == T_Q5_K ? 7 : 8;
    return m >= lo && m <= (type == T_Q8_0 ? 64 : 32);
}

// The MFMA kernels walk K in 256-element steps. Crossover from the GEMV (which streams the
// weights once per 8 activation rows) measured on MI355X: 16 rows for the types the
// weight-row kernel has; 64 for the others (and for shapes past the weight-row kernel's 32-bit
// offsets), whose int8 kernel only overtakes the GEMV there
// (Q5_K 14336 x 4096: 155 us at 16 rows against ~50 us on the GEMV). A forced kernel choice
// (the tuning knob gemm_kernel) takes the MFMA route from 16 rows for every type.
bool use_mfma(uint32_t type, int k, int n, int m) {
    if (k % 256 != 0 || !gemm_supported(type) || use_small(type, k, n, m)) return false;
    if (gemm_forced()) return m >= kMfmaMinRows;
    if (!gemmw_supported(type) || !gemmw_fits(type, k, n, m)) return m >= 4 * kMfmaMinRows;
    if (m >= kMfmaMinRows) return true;
    if (type != T_Q6_K && type != T_Q4_0 && type != T_Q5_0) return false;
    // a batch the GEMV streams in one launch stays there (Q5_0 14336x4096 at 6 rows: 19.1 us
    // against 25.7 on the weight-row kernel)
    if (gemv_streams_batch(type, k, n, m)) return false;
    // Q6_K, Q4_0 and Q5_0 have no small-batch kernel. Below 16 rows their GEMV reads the
    // weights once per launch (8, 4 or 2 rows each, as LDS allows), and the weight-row kernel,
    // which pads the batch to one 16-row tile, takes about the time of its 16-row call. On
    // matrices of 32 M weights or more it wins from three GEMV launches or 8 rows (Q6_K: 8 rows
    // in two launches); on smaller ones from four launches. MI355X, cold weights, us, GEMV
    // against weight-row kernel:
    //   Q6_K 4096x14336, 5 / 8 / 15 rows:   41.7 / 58.5 / 107.3 against 34.9 - 35.5
    //   Q6_K 14336x4096, 7 / 8 / 12 rows:   41.2 / 30.2 / 45.9 against 33.8 - 34.4
    //   Q4_0 14336x4096, 7 / 8 / 15 rows:   34.7 / 27.0 / 57.3 against 24.0 - 24.5
    //   Q5_0 4096x4096,  7 / 8 / 15 rows:   20.6 / 12.9 / 30.4 against 19.7 - 19.9
    //   Q6_K 1024x4096,  7 / 8 / 15 rows:   15.5 / 10.5 / 23.2 against 19.9 - 20.4
    const int launches = gemv_launch_count(type, k, m);
    const bool large = (int64_t)n * k >= (int64_t(32) << 20);
    if (launches >= (large ? 3 : 4)) return true;
    if (m < 8 || !large) return false;
    return type != T_Q6_K || launches >= 2;
}

// MFMA kernel choice. Default: the weight-row fp16 kernel (k_gemmw.hip) where it has the
// type, else the int8 kernel (k_gemm.hip). The tuning knob "gemm_kernel" (cllm_hip_tune)
// forces the int8 kernel (1) or the activation-row fp16 kernel (k_gemm16.hip, 2) for every
// type (tests run all three). Shapes past the weight-row kernels' 32-bit offsets (weights of
// 4 GiB and up, such as a Q8_0 262144 x 16384 output head) take the int8 kernel, which
// indexes with 64-bit offsets.
enum class GemmKind { W16, I8, F16 };

bool gemm_forced() { return tuning().gemm_kind.load(std::memory_order_relaxed) != 0; }

GemmKind gemm_kind(uint32_t type, int k, int n, int m) {
    const int knob = tuning().gemm_kind.load(std::memory_order_relaxed);
    if (knob == 2) return GemmKind::F16;
    if (knob == 1) return GemmKind::I8;
    return gemmw_supported(type) && gemmw_fits(type, k, n, m) ? GemmKind::W16 : GemmKind::I8;
}

// Split-K bytes the MFMA route of this shape needs (the weight-row kernel only).
size_t part_bytes_for(uint32_t type, int k, int n, int m) {
    if (use_small(type, k, n, m)) return gemm_sm_partial_bytes(type, k, n, m);
    return gemm_kind(type, k, n, m) == GemmKind::W16 ? gemmw_partial_bytes(type, k, n, m) : 0;
}

// MFMA route on a Q8_0 batch already in device memory; ws supplies the activation formats of
// the fp16 kernels and the split-K region.
hipError_t run_gemm(uint32_t type, const uint8_t* w, int k, int n, int m, const int8_t* qs,
                    const float* sc, const int32_t* bs, const float* bias, float* y,
                    const WsView& ws, hipStream_t stream) {
    if (use_small(type, k, n, m))
        return launch_gemm_sm_q8(type, w, k, n, m, qs, sc, bs, bias, y, ws.part, ws.part_cap, stream);
    const GemmKind kind = gemm_kind(type, k, n, m);
    if (kind == GemmKind::W16) {
        hipError_t e = launch_q8_to_w(qs, sc, bs, (int64_t)m * k / 32, ws.sc, ws.qh,
                                      (type == T_Q4_K || type == T_Q5_K) ? ws.xq : nullptr, stream);
        if (e != hipSuccess) return e;
        return launch_gemmw(type, w, k, n, m, ws.sc, ws.qh, ws.xq, bias, y, ws.part, ws.part_cap,
                            stream);
    }
    if (kind == GemmKind::I8) return launch_gemm(type, w, k, n, m, qs, sc, bs, bias, y, stream);
    hipError_t e = launch_q8_to_mfma(qs, sc, bs, (int64_t)m * k / 32, ws.qh, ws.px, stream);
    if (e != hipSuccess) return e;
    return launch_gemm16(type, w, k, n, m, ws.qh, sc, ws.px, bias, y, stream);
}

// Whether the small-batch route quantizes fp32 activation rows once into the workspace (then
// runs the kernel on that batch) rather than inside every workgroup of the kernel. Once: every
// workgroup of the in-kernel form quantizes all rows of its K range, which bounds that range
// (so longer K needs split-K and its cross-workgroup tail), while a batch quantized once lets
// a workgroup hold K = 4096 for 16 rows. MI355X, cold weights, graph-timed us, quantized once
// against in the kernel (the quantizing launch included):
//   Q5_K 14336x4096, 4 / 8 / 16 rows:  17.8 / 17.9 / 18.6 against 18.8 / 19.4 / 20.4
//   Q8_0 4096x4096, 4 / 8 / 16 / 64:   11.0 / 11.3 / 11.8 / 19.1 against 12.3 / 12.3 / 12.7 / 21.3
// Q6_K, Q4_0 and Q5_0 have only this form; the tuning knob "gemm_small_q8" forces either for
// the others (1 once, 2 in-kernel).
bool small_quantize_once(uint32_t type, int k, int n, int m) {
    (void)k;
    (void)n;
    (void)m;
    if (type == T_Q6_K || type == T_Q4_0 || type == T_Q5_0) return true;
    return tuning().gemm_small_q8.load(std::memory_order_relaxed) != 2;
}

// The small-batch route from fp32 activation rows (small_quantize_once picks the form).
hipError_t run_small_f32(uint32_t type, const uint8_t* w, int k, int n, int m, const float* x,
                         const float* bias, float* y, const WsView& ws, hipStream_t stream) {
    if (small_quantize_once(type, k, n, m)) {
        hipError_t e = launch_quantize_q8_0(x, (int64_t)m * k / 32, ws.qs, ws.sc, ws.bs, stream);
        if (e != hipSuccess) return e;
        return launch_gemm_sm_q8(type, w, k, n, m, ws.qs, ws.sc, ws.bs, bias, y, ws.part,
                                 ws.part_cap, stream);
    }
    return launch_gemm_sm_f32(type, w, k, n, m, x, bias, y, ws.part, ws.part_cap, stream);
}

hipError_t run_gemm_f32(uint32_t type, const uint8_t* w, int k, int n, int m, const float* x,
                        const float* bias, float* y, const WsView& ws, hipStream_t stream) {
    if (use_small(type, k, n, m)) return run_small_f32(type, w, k, n, m, x, bias, y, ws, stream);
    const int64_t nblk = (int64_t)m * k / 32;
    const GemmKind kind = gemm_kind(type, k, n, m);
    if (kind == GemmKind::F16) {
        hipError_t e = launch_quantize_mfma(x, nblk, ws.sc, ws.qh, ws.px, stream);
        if (e != hipSuccess) return e;
        return launch_gemm16(type, w, k, n, m, ws.qh, ws.sc, ws.px, bias, y, stream);
    }
    if (kind == GemmKind::W16) {
        hipError_t e = launch_quantize_w(x, nblk, ws.sc, ws.qh,
                                         (type == T_Q4_K || type == T_Q5_K) ? ws.xq : nullptr, stream);
        if (e != hipSuccess) return e;
        return launch_gemmw(type, w, k, n, m, ws.sc, ws.qh, ws.xq, bias, y, ws.part, ws.part_cap,
                            stream);
    }
    hipError_t e = launch_quantize_q8_0(x, nblk, ws.qs, ws.sc, ws.bs, stream);
    if (e != hipSuccess) return e;
    return run_gemm(type, w, k, n, m, ws.qs, ws.sc, ws.bs, bias, y, ws, stream);
}

// Batches of at most this many rows take the fused GEMV (quantization inside the kernel, one
// launch); larger GEMV batches quantize once into the workspace first, because every fused
// workgroup re-quantizes all of its rows and that redundant work grows with the row count.
constexpr int kFusedMaxRows = 2;

// Whether the GEMV route quantizes inside its kernel: up to kFusedMaxRows rows, and up to 7
// rows of a batch the streaming kernel takes in one launch, where one workgroup per CU
// quantizes the batch (the tuning knob "gemv_fused_rows" sets that bound; 0 = 7). MI355X,
// cold weights, graph-timed us, in-kernel against quantized once first (bit for bit alike):
//   Q5_K 14336x4096, 3 / 4 / 5 rows:      13.2 / 14.3 / 16.3 against 15.0 / 16.3 / 17.6
//   Q8_0 4096x4096, 3 / 4 / 7 / 8 rows:   6.8 / 7.7 / 9.7 / 10.4 against 8.3 / 8.9 / 10.1 / 10.6
//   Q4_0 4096x4096, 4 / 7 / 8 rows:       7.1 / 9.4 / 10.3 against 8.1 / 9.6 / 10.0
bool gemv_fused(uint32_t type, int k, int n, int m) {
    if (m <= kFusedMaxRows) return true;
    const int knob = tuning().gemv_fused_rows.load(std::memory_order_relaxed);
    return m <= (knob > 0 ? knob : 7) && gemv_streams_batch(type, k, n, m);
}

bool needs_workspace(uint32_t type, int k, int n, int m) {
    if (!has_kernel(type)) return false;  // the float-dot kernels read fp32 rows directly
    return use_mfma(type, k, n, m) || use_small(type, k, n, m) || !gemv_fused(type, k, n, m);
}

// GEMV route on fp32 activation rows.
hipError_t run_gemv_f32(uint32_t type, const uint8_t* w, int k, int n, int m, const float* x,
                        const float* bias, float* y, const WsView& ws, hipStream_t stream,
                        bool accumulate = false) {
    if (!accumulate && use_small(type, k, n, m))
        return run_small_f32(type, w, k, n, m, x, bias, y, ws, stream);
    if (gemv_fused(type, k, n, m))
        return launch_gemv_fused(type, w, k, n, m, x, bias, y, stream, accumulate);
    hipError_t e = launch_quantize_q8_0(x, (int64_t)m * k / 32, ws.qs, ws.sc, ws.bs, stream);
    if (e != hipSuccess) return e;
    return launch_gemv(type, w, k, n, m, ws.qs, ws.sc, ws.bs, bias, y, stream, accumulate);
}

// The per-stream workspace of the device entry points, grown to an m x k batch and to the
// split-K region of an n-row MFMA call on it (n = 0: none).
int stream_workspace(DeviceState* st, hipStream_t s, uint32_t type, int k, int n, int m,
                     Workspace** out) {
    std::lock_guard<std::mutex> lk(st->mtx);
    auto& slot = st->dev_ws[s];
    if (!slot) slot = std::make_unique<Workspace>();
    HIP_TRY(slot->ensure(k, m, s));
    if (n > 0 && (use_mfma(type, k, n, m) || use_small(type, k, n, m)))
        HIP_TRY(slot->ensure_part(part_bytes_for(type, k, n, m), s));
    *out = slot.get();
    return CLLM_HIP_OK;
}

// Host-buffer matmul shared by matmul_quant and matmul_quant_batch.
int host_matmul(const char* who, const float* x, const void* w, uint32_t type, const float* bias,
                int in_dim, int out_dim, int n_rows, float* y) {
    int rc = check_matmul(who, type, in_dim, out_dim);
    if (rc) return rc;
    if (!x || !w || !y) return set_err(CLLM_HIP_E_ARG, "%s: null pointer", who);
    if (out_dim == 0) return CLLM_HIP_OK;
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    std::lock_guard<std::mutex> lk(st->mtx);
    const size_t xb = (size_t)n_rows * in_dim * sizeof(float);
    const size_t yb = (size_t)n_rows * out_dim * sizeof(float);
    const uint8_t* wd = nullptr;
    if ((rc = resolve_weights(st, w, row_bytes(type, in_dim) * (size_t)out_dim, &wd))) return rc;
    HIP_TRY(st->x.ensure(xb, st->stream));
    HIP_TRY(st->y.ensure(yb, st->stream));
    if (needs_workspace(type, in_dim, out_dim, n_rows)) {
        HIP_TRY(st->act.ensure(in_dim, n_rows, st->stream));
        if (use_mfma(type, in_dim, out_dim, n_rows) || use_small(type, in_dim, out_dim, n_rows))
            HIP_TRY(st->act.ensure_part(part_bytes_for(type, in_dim, out_dim, n_rows), st->stream));
    }
    HIP_TRY(hipMemcpyAsync(st->x.p, x, xb, hipMemcpyHostToDevice, st->stream));
    const float* bd = nullptr;
    if (bias) {
        HIP_TRY(st->bias.ensure((size_t)out_dim * sizeof(float), st->stream));
        HIP_TRY(hipMemcpyAsync(st->bias.p, bias, (size_t)out_dim * sizeof(float),
                               hipMemcpyHostToDevice, st->stream));
        bd = (const float*)st->bias.p;
    }
    if (!has_kernel(type)) {
        HIP_TRY(launch_gemv_f(type, wd, in_dim, out_dim, n_rows, (const float*)st->x.p, bd,
                              (float*)st->y.p, st->stream));
    } else if (use_mfma(type, in_dim, out_dim, n_rows)) {
        HIP_TRY(run_gemm_f32(type, wd, in_dim, out_dim, n_rows, (const float*)st->x.p, bd,
                             (float*)st->y.p, st->act.v, st->stream));
    } else {
        HIP_TRY(run_gemv_f32(type, wd, in_dim, out_dim, n_rows, (const float*)st->x.p, bd,
                             (float*)st->y.p, st->act.v, st->stream));
    }
    HIP_TRY(hipMemcpyAsync(y, st->y.p, yb, hipMemcpyDeviceToHost, st->stream));
    HIP_TRY(hipStreamSynchronize(st->stream));
    return CLLM_HIP_OK;
}

}  // namespace

namespace cllm_hip {
Tuning& tuning() { return g_tuning; }
}  // namespace cllm_hip

extern "C" {

int cllm_hip_init(int device) {
    if (device < 0) return set_err(CLLM_HIP_E_ARG, "cllm_hip_init: negative device");
    g_device = device;
    DeviceState* st;
    return acquire(&st);
}

const char* cllm_hip_last_error(void) { return g_err; }

int cllm_hip_block_size(uint32_t type) { return block_elems(type); }
size_t cllm_hip_type_size(uint32_t type) { return block_bytes(type); }
int cllm_hip_has_vec_dot(uint32_t type) { return has_kernel(type) ? 1 : 0; }

int cllm_hip_quantize_row_q8_0(const float* x, int64_t n, int n_rows, int8_t* qs, float* scales,
                               int32_t* bsums) {
    if (n < 0 || n % 32 != 0)
        return set_err(CLLM_HIP_E_SHAPE, "quantize_row_q8_0: n not divisible by 32");
    if (n_rows <= 0 || n == 0) return CLLM_HIP_OK;
    if (!x || !qs || !scales || !bsums)
        return set_err(CLLM_HIP_E_ARG, "quantize_row_q8_0: null pointer");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(st->mtx);
    const size_t total = (size_t)n * n_rows;
    if (total / 32 > (size_t)INT32_MAX * 32)
        return set_err(CLLM_HIP_E_ARG, "quantize_row_q8_0: too many elements");
    HIP_TRY(st->x.ensure(total * sizeof(float), st->stream));
    HIP_TRY(st->act.ensure((int)n, n_rows, st->stream));
    HIP_TRY(hipMemcpyAsync(st->x.p, x, total * sizeof(float), hipMemcpyHostToDevice, st->stream));
    HIP_TRY(launch_quantize_q8_0((const float*)st->x.p, (int64_t)(total / 32), st->act.v.qs,
                                 st->act.v.sc, st->act.v.bs, st->stream));
    HIP_TRY(hipMemcpyAsync(qs, st->act.v.qs, total, hipMemcpyDeviceToHost, st->stream));
    HIP_TRY(hipMemcpyAsync(scales, st->act.v.sc, total / 32 * sizeof(float), hipMemcpyDeviceToHost,
                           st->stream));
    HIP_TRY(hipMemcpyAsync(bsums, st->act.v.bs, total / 32 * sizeof(int32_t), hipMemcpyDeviceToHost,
                           st->stream));
    HIP_TRY(hipStreamSynchronize(st->stream));
    return CLLM_HIP_OK;
}

int cllm_hip_vec_dot_rows(const void* w, uint32_t type, int64_t n, int n_w_rows,
                          const int8_t* qs, const float* scales, const int32_t* bsums,
                          float* out) {
    if (!has_kernel(type)) return set_err(CLLM_HIP_E_TYPE, "vec_dot_row: no kernel for this type");
    if (n <= 0 || n % block_elems(type) != 0 || n > INT32_MAX)
        return set_err(CLLM_HIP_E_SHAPE, "vec_dot_row: n not divisible by block size");
    if (n_w_rows <= 0) return CLLM_HIP_OK;
    if (!w || !qs || !scales || !bsums || !out)
        return set_err(CLLM_HIP_E_ARG, "vec_dot_row: null pointer");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(st->mtx);
    const int k = (int)n;
    const uint8_t* wd = nullptr;
    if ((rc = resolve_weights(st, w, row_bytes(type, k) * (size_t)n_w_rows, &wd))) return rc;
    HIP_TRY(st->act.ensure(k, 1, st->stream));
    HIP_TRY(st->y.ensure((size_t)n_w_rows * sizeof(float), st->stream));
    HIP_TRY(hipMemcpyAsync(st->act.v.qs, qs, (size_t)k, hipMemcpyHostToDevice, st->stream));
    HIP_TRY(hipMemcpyAsync(st->act.v.sc, scales, (size_t)k / 32 * sizeof(float),
                           hipMemcpyHostToDevice, st->stream));
    HIP_TRY(hipMemcpyAsync(st->act.v.bs, bsums, (size_t)k / 32 * sizeof(int32_t),
                           hipMemcpyHostToDevice, st->stream));
    HIP_TRY(launch_gemv(type, wd, k, n_w_rows, 1, st->act.v.qs, st->act.v.sc, st->act.v.bs, nullptr,
                        (float*)st->y.p, st->stream));
    HIP_TRY(hipMemcpyAsync(out, st->y.p, (size_t)n_w_rows * sizeof(float), hipMemcpyDeviceToHost,
                           st->stream));
    HIP_TRY(hipStreamSynchronize(st->stream));
    return CLLM_HIP_OK;
}

int cllm_hip_matmul_quant(const float* x, const void* w, uint32_t type, const float* bias,
                          int in_dim, int out_dim, float* y) {
    return host_matmul("matmul_quant", x, w, type, bias, in_dim, out_dim, 1, y);
}

int cllm_hip_matmul_quant_batch(const float* x, const void* w, uint32_t type, const float* bias,
                                int in_dim, int out_dim, int n_rows, float* y) {
    if (n_rows <= 0) return CLLM_HIP_OK;  // quant.cpp:1436
    if (n_rows == 1) return cllm_hip_matmul_quant(x, w, type, bias, in_dim, out_dim, y);
    return host_matmul("matmul_quant_batch", x, w, type, bias, in_dim, out_dim, n_rows, y);
}

int cllm_hip_register_weights(const void* host_base, size_t bytes) {
    if (!host_base || bytes == 0)
        return set_err(CLLM_HIP_E_ARG, "cllm_hip_register_weights: empty region");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(st->mtx);
    const uintptr_t a = (uintptr_t)host_base;
    auto it = st->regions.find(a);
    if (it != st->regions.end() && (rc = drop_region(st, it))) return rc;
    Region r;
    if ((rc = upload_region(st, a, bytes, &r))) return rc;
    st->regions[a] = r;
    return CLLM_HIP_OK;
}

int cllm_hip_file_mapping_identity(const void* p, uint64_t info[9]) {
    if (!info) return set_err(CLLM_HIP_E_ARG, "cllm_hip_file_mapping_identity: null info");
    Mapping m;
    if (!find_mapping((uintptr_t)p, m, true) || !immutable_file_mapping(m))
        return set_err(CLLM_HIP_E_ARG, "cllm_hip_file_mapping_identity: not in a read-only private file mapping");
    Region r;
    watch_file(m, r);
    info[0] = m.lo;
    info[1] = m.hi;
    info[2] = m.off;
    info[3] = m.inode;
    info[4] = ((uint64_t)m.dev_major << 32) | m.dev_minor;
    info[5] = (uint64_t)r.at_copy.st_size;
    info[6] = (uint64_t)r.at_copy.st_mtim.tv_sec * 1000000000ull + (uint64_t)r.at_copy.st_mtim.tv_nsec;
    info[7] = (uint64_t)r.at_copy.st_ctim.tv_sec * 1000000000ull + (uint64_t)r.at_copy.st_ctim.tv_nsec;
    info[8] = r.fd >= 0;
    if (r.fd >= 0) ::close(r.fd);
    return CLLM_HIP_OK;
}

int cllm_hip_unregister_weights(const void* host_base) {
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(st->mtx);
    auto it = st->regions.find((uintptr_t)host_base);
    if (it == st->regions.end())
        return set_err(CLLM_HIP_E_ARG, "cllm_hip_unregister_weights: region not registered");
    return drop_region(st, it);
}

int cllm_hip_dequantize_block(const void* src, float* dst, uint32_t type, int64_t n) {
    return dequantize_host("dequantize_block", src, dst, nullptr, type, n);
}

int cllm_hip_dequantize_block_f16(const void* src, uint16_t* dst, uint32_t type, int64_t n) {
    return dequantize_host("dequantize_block_f16", src, nullptr, dst, type, n);
}

int cllm_hip_quantize_q8_0_dev(const float* x, int64_t n, int n_rows, int8_t* qs, float* scales,
                               int32_t* bsums, void* stream) {
    if (n < 0 || n % 32 != 0)
        return set_err(CLLM_HIP_E_SHAPE, "quantize_row_q8_0: n not divisible by 32");
    if (n_rows <= 0 || n == 0) return CLLM_HIP_OK;
    if (!x || !qs || !scales || !bsums)
        return set_err(CLLM_HIP_E_ARG, "quantize_row_q8_0: null pointer");
    if (!aligned16(x) || ((uintptr_t)qs & 3u) || ((uintptr_t)scales & 3u) || ((uintptr_t)bsums & 3u))
        return set_err(CLLM_HIP_E_ARG, "quantize_row_q8_0: misaligned device pointer");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    HIP_TRY(launch_quantize_q8_0(x, n * n_rows / 32, qs, scales, bsums, (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_read_stream_dev(const void* p, uint64_t bytes, void* stream) {
    if (bytes == 0) return CLLM_HIP_OK;
    if (!p) return set_err(CLLM_HIP_E_ARG, "read_stream: null pointer");
    if (!aligned16(p) || bytes % 16 != 0)
        return set_err(CLLM_HIP_E_ARG, "read_stream: address or size not a multiple of 16 bytes");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    int cus = 0;
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, current_device()));
    HIP_TRY(launch_read_stream(p, (int64_t)bytes, cus, (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_gemv_q8_dev(const void* w, uint32_t type, int in_dim, int out_dim, int n_rows,
                         const int8_t* qs, const float* scales, const int32_t* bsums,
                         const float* bias, float* y, void* stream) {
    int rc = check_matmul("matmul_quant", type, in_dim, out_dim);
    if (rc) return rc;
    if (!has_kernel(type)) return set_err(CLLM_HIP_E_TYPE, "vec_dot_row: no kernel for this type");
    if (n_rows <= 0 || out_dim == 0) return CLLM_HIP_OK;
    if (!w || !qs || !scales || !bsums || !y)
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
    if (!aligned16(w) || !aligned16(qs) || ((uintptr_t)scales & 7u) || ((uintptr_t)bsums & 7u) ||
        ((uintptr_t)y & 3u) || ((uintptr_t)bias & 3u))
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (!use_mfma(type, in_dim, out_dim, n_rows) && !use_small(type, in_dim, out_dim, n_rows)) {
        HIP_TRY(launch_gemv(type, (const uint8_t*)w, in_dim, out_dim, n_rows, qs, scales, bsums,
                            bias, y, s));
        return CLLM_HIP_OK;
    }
    Workspace* ws;
    if ((rc = stream_workspace(st, s, type, in_dim, out_dim, n_rows, &ws))) return rc;
    HIP_TRY(run_gemm(type, (const uint8_t*)w, in_dim, out_dim, n_rows, qs, scales, bsums, bias, y,
                     ws->v, s));
    return CLLM_HIP_OK;
}

int cllm_hip_gemv_q8_multi_dev(uint32_t type, int in_dim, int n_mats, const void* const* w,
                               const int* out_dims, const float* const* bias, float* const* y,
                               int n_rows, const int8_t* qs, const float* scales,
                               const int32_t* bsums, void* stream) {
    if (n_mats < 1 || n_mats > 3 || !w || !out_dims || !y)
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: 1 to 3 matrices expected");
    int rc;
    for (int i = 0; i < n_mats; ++i)
        if ((rc = check_matmul("matmul_quant", type, in_dim, out_dims[i]))) return rc;
    if (!has_kernel(type)) return set_err(CLLM_HIP_E_TYPE, "vec_dot_row: no kernel for this type");
    if (n_rows <= 0) return CLLM_HIP_OK;
    if (!qs || !scales || !bsums) return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
    if (!aligned16(qs) || ((uintptr_t)scales & 7u) || ((uintptr_t)bsums & 7u))
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    for (int i = 0; i < n_mats; ++i) {
        if (!w[i] || !y[i]) return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
        if (!aligned16(w[i]) || ((uintptr_t)y[i] & 3u) || (bias && ((uintptr_t)bias[i] & 3u)))
            return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    }
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    HIP_TRY(launch_gemv_multi(type, in_dim, n_mats, (const uint8_t* const*)w, out_dims, bias, y,
                              n_rows, qs, scales, bsums, (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_gemv_q8_swiglu_dev(uint32_t type, int in_dim, int n_ff, const void* w_gate,
                                const void* w_up, const float* bias_gate, const float* bias_up,
                                int n_rows, const int8_t* qs, const float* scales,
                                const int32_t* bsums, float* h, void* stream) {
    int rc = check_matmul("matmul_quant", type, in_dim, n_ff);
    if (rc) return rc;
    if (!has_kernel(type)) return set_err(CLLM_HIP_E_TYPE, "vec_dot_row: no kernel for this type");
    if (n_rows <= 0 || n_ff == 0) return CLLM_HIP_OK;
    if (!w_gate || !w_up || !h || !qs || !scales || !bsums)
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
    if (!aligned16(w_gate) || !aligned16(w_up) || !aligned16(qs) || ((uintptr_t)scales & 7u) ||
        ((uintptr_t)bsums & 7u) || ((uintptr_t)h & 3u) || ((uintptr_t)bias_gate & 3u) ||
        ((uintptr_t)bias_up & 3u))
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    HIP_TRY(launch_gemv_swiglu(type, in_dim, n_ff, (const uint8_t*)w_gate, (const uint8_t*)w_up,
                               bias_gate, bias_up, h, n_rows, qs, scales, bsums, (hipStream_t)stream));
    return CLLM_HIP_OK;
}

// The one fp32 row a fused RMSNorm staging takes.
static int check_norm_row(int in_dim, const float* x, const float* norm_w) {
    if (in_dim <= 0 || in_dim > 4096 || in_dim % 32 != 0)
        return set_err(CLLM_HIP_E_SHAPE, "rms_norm: a fused row is a multiple of 32 up to 4096");
    if (!x || !norm_w) return set_err(CLLM_HIP_E_ARG, "rms_norm: null pointer");
    if (!aligned16(x) || !aligned16(norm_w))
        return set_err(CLLM_HIP_E_ARG, "rms_norm: misaligned device pointer");
    return CLLM_HIP_OK;
}

int cllm_hip_rmsnorm_gemv_multi_dev(uint32_t type, int in_dim, int n_mats, const void* const* w,
                                    const int* out_dims, const float* const* bias,
                                    float* const* y, const float* x, const float* norm_w,
                                    float eps, void* stream) {
    if (n_mats < 1 || n_mats > 3 || !w || !out_dims || !y)
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: 1 to 3 matrices expected");
    int rc;
    for (int i = 0; i < n_mats; ++i)
        if ((rc = check_matmul("matmul_quant", type, in_dim, out_dims[i]))) return rc;
    if (!has_kernel(type)) return set_err(CLLM_HIP_E_TYPE, "vec_dot_row: no kernel for this type");
    if ((rc = check_norm_row(in_dim, x, norm_w))) return rc;
    for (int i = 0; i < n_mats; ++i) {
        if (!w[i] || !y[i]) return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
        if (!aligned16(w[i]) || ((uintptr_t)y[i] & 3u) || (bias && ((uintptr_t)bias[i] & 3u)))
            return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    }
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    HIP_TRY(launch_rmsnorm_gemv_multi(type, in_dim, n_mats, (const uint8_t* const*)w, out_dims,
                                      bias, y, x, norm_w, eps, (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_rmsnorm_gemv_swiglu_dev(uint32_t type, int in_dim, int n_ff, const void* w_gate,
                                     const void* w_up, const float* bias_gate,
                                     const float* bias_up, const float* x, const float* norm_w,
                                     float eps, float* h, void* stream) {
    int rc = check_matmul("matmul_quant", type, in_dim, n_ff);
    if (rc) return rc;
    if (!has_kernel(type)) return set_err(CLLM_HIP_E_TYPE, "vec_dot_row: no kernel for this type");
    if ((rc = check_norm_row(in_dim, x, norm_w))) return rc;
    if (n_ff == 0) return CLLM_HIP_OK;
    if (!w_gate || !w_up || !h) return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
    if (!aligned16(w_gate) || !aligned16(w_up) || ((uintptr_t)h & 3u) ||
        ((uintptr_t)bias_gate & 3u) || ((uintptr_t)bias_up & 3u))
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    HIP_TRY(launch_rmsnorm_gemv_swiglu(type, in_dim, n_ff, (const uint8_t*)w_gate,
                                       (const uint8_t*)w_up, bias_gate, bias_up, x, norm_w, eps, h,
                                       (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_gemv_q8_residual_dev(const void* w, uint32_t type, int in_dim, int out_dim,
                                  int n_rows, const int8_t* qs, const float* scales,
                                  const int32_t* bsums, const float* bias, float* y,
                                  void* stream) {
    int rc = check_matmul("matmul_quant", type, in_dim, out_dim);
    if (rc) return rc;
    if (!has_kernel(type)) return set_err(CLLM_HIP_E_TYPE, "vec_dot_row: no kernel for this type");
    if (n_rows <= 0 || out_dim == 0) return CLLM_HIP_OK;
    if (!w || !qs || !scales || !bsums || !y)
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
    if (!aligned16(w) || !aligned16(qs) || ((uintptr_t)scales & 7u) || ((uintptr_t)bsums & 7u) ||
        ((uintptr_t)y & 3u) || ((uintptr_t)bias & 3u))
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    HIP_TRY(launch_gemv(type, (const uint8_t*)w, in_dim, out_dim, n_rows, qs, scales, bsums, bias,
                        y, (hipStream_t)stream, true));
    return CLLM_HIP_OK;
}

size_t cllm_hip_mfma_act_bytes(int in_dim, int n_rows) {
    return in_dim > 0 && n_rows > 0 ? mfma_act_bytes(in_dim, n_rows) : 0;
}

namespace {
// The checks shared by the producers of the activation format.
int check_mfma_act(const char* who, int in_dim, int n_rows, const void* act) {
    if (in_dim <= 0 || in_dim % 256 != 0)
        return set_err(CLLM_HIP_E_SHAPE, "%s: in_dim must be a multiple of 256", who);
    if (n_rows < 0) return set_err(CLLM_HIP_E_ARG, "%s: negative n_rows", who);
    if (!act || !aligned16(act)) return set_err(CLLM_HIP_E_ARG, "%s: null or misaligned act", who);
    return CLLM_HIP_OK;
}
}  // namespace

int cllm_hip_quantize_mfma_dev(const float* x, int in_dim, int n_rows, void* act, void* stream) {
    int rc = check_mfma_act("quantize_mfma", in_dim, n_rows, act);
    if (rc) return rc;
    if (n_rows == 0) return CLLM_HIP_OK;
    if (!x || !aligned16(x)) return set_err(CLLM_HIP_E_ARG, "quantize_mfma: null or misaligned x");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    float* xs;
    _Float16* qh;
    uint16_t* xq;
    carve_mfma(act, in_dim, n_rows, &xs, &qh, &xq);
    HIP_TRY(launch_quantize_w(x, (int64_t)n_rows * in_dim / 32, xs, qh, xq, (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_rmsnorm_mfma_dev(const float* x, const float* norm_w, float eps, int in_dim,
                              int n_rows, float* h, void* act, void* stream) {
    int rc = check_mfma_act("rmsnorm_mfma", in_dim, n_rows, act);
    if (rc) return rc;
    if (n_rows == 0) return CLLM_HIP_OK;
    if (!x || !norm_w || !aligned16(x) || !aligned16(norm_w) || !aligned16(h))
        return set_err(CLLM_HIP_E_ARG, "rmsnorm_mfma: null or misaligned pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    float* xs;
    _Float16* qh;
    uint16_t* xq;
    carve_mfma(act, in_dim, n_rows, &xs, &qh, &xq);
    HIP_TRY(launch_rmsnorm_q8_0(x, norm_w, eps, in_dim, n_rows, h, nullptr, xs, nullptr,
                                (hipStream_t)stream, qh, xq));
    return CLLM_HIP_OK;
}

int cllm_hip_swiglu_mfma_dev(const float* gate, const float* up, int n, int n_rows, float* h,
                             void* act, void* stream) {
    int rc = check_mfma_act("swiglu_mfma", n, n_rows, act);
    if (rc) return rc;
    if (n_rows == 0) return CLLM_HIP_OK;
    if (!gate || !up || !aligned16(gate) || !aligned16(up) || !aligned16(h))
        return set_err(CLLM_HIP_E_ARG, "swiglu_mfma: null or misaligned pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    float* xs;
    _Float16* qh;
    uint16_t* xq;
    carve_mfma(act, n, n_rows, &xs, &qh, &xq);
    HIP_TRY(launch_swiglu_q8_0(gate, up, (int64_t)n * n_rows, h, nullptr, xs, nullptr,
                               (hipStream_t)stream, qh, xq));
    return CLLM_HIP_OK;
}

int cllm_hip_matmul_mfma_dev(uint32_t type, int in_dim, int n_mats, const void* const* w,
                             const int* out_dims, const float* const* bias, float* const* y,
                             int n_rows, const void* act, void* stream) {
    if (n_mats < 1 || !w || !out_dims || !y)
        return set_err(CLLM_HIP_E_ARG, "matmul_quant_batch: no matrices");
    int rc;
    for (int i = 0; i < n_mats; ++i)
        if ((rc = check_matmul("matmul_quant_batch", type, in_dim, out_dims[i]))) return rc;
    if ((rc = check_mfma_act("matmul_quant_batch", in_dim, n_rows, act))) return rc;
    if (!gemmw_supported(type))
        return set_err(CLLM_HIP_E_TYPE, "matmul_quant_batch: no weight-row kernel for this type");
    for (int i = 0; i < n_mats; ++i) {
        if (!w[i] || !y[i]) return set_err(CLLM_HIP_E_ARG, "matmul_quant_batch: null pointer");
        if (!aligned16(w[i]) || ((uintptr_t)y[i] & 3u) || (bias && ((uintptr_t)bias[i] & 3u)))
            return set_err(CLLM_HIP_E_ARG, "matmul_quant_batch: misaligned device pointer");
        if (!gemmw_fits(type, in_dim, out_dims[i], n_rows))
            return set_err(CLLM_HIP_E_ARG, "matmul_quant_batch: weights or activations past 4 GiB");
    }
    if (n_rows == 0) return CLLM_HIP_OK;
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    hipStream_t s = (hipStream_t)stream;
    float* xs;
    _Float16* qh;
    uint16_t* xq;
    carve_mfma(act, in_dim, n_rows, &xs, &qh, &xq);
    Workspace* ws;
    {
        std::lock_guard<std::mutex> lk(st->mtx);
        auto& slot = st->dev_ws[s];
        if (!slot) slot = std::make_unique<Workspace>();
        ws = slot.get();
    }
    const uint8_t* const* wb = (const uint8_t* const*)w;
    if (gemmw_multi_supported(type, n_mats)) {
        HIP_TRY(ws->ensure_part(gemmw_multi_partial_bytes(type, in_dim, n_mats, out_dims, n_rows), s));
        HIP_TRY(launch_gemmw_multi(type, in_dim, n_rows, n_mats, wb, out_dims, bias, y, xs, qh, xq,
                                   ws->v.part, ws->v.part_cap, s));
        return CLLM_HIP_OK;
    }
    // one launch per matrix (types without the multi-matrix kernel), all on the one format
    for (int i = 0; i < n_mats; ++i) {
        HIP_TRY(ws->ensure_part(gemmw_partial_bytes(type, in_dim, out_dims[i], n_rows), s));
        HIP_TRY(launch_gemmw(type, wb[i], in_dim, out_dims[i], n_rows, xs, qh, xq,
                             bias ? bias[i] : nullptr, y[i], ws->v.part, ws->v.part_cap, s));
    }
    return CLLM_HIP_OK;
}

const char* cllm_hip_matmul_mfma_plan(uint32_t type, int in_dim, int n_mats, const int* out_dims,
                                      int n_rows) {
    static thread_local char buf[160];
    if (!gemmw_supported(type) || in_dim % 256 != 0 || n_mats < 1 || !out_dims) return "none";
    if (gemmw_multi_supported(type, n_mats)) {
        gemmw_multi_plan_name(type, in_dim, n_mats, out_dims, n_rows, buf, sizeof buf);
        const size_t l = std::strlen(buf);
        snprintf(buf + l, sizeof buf - l, " matrices=%d launches=1", n_mats);
    } else {
        gemmw_plan_name(type, in_dim, out_dims[0], n_rows, buf, sizeof buf);
        const size_t l = std::strlen(buf);
        snprintf(buf + l, sizeof buf - l, " matrices=%d launches=%d", n_mats, n_mats);
    }
    return buf;
}

int cllm_hip_matmul_quant_dev(const float* x, const void* w, uint32_t type, const float* bias,
                              int in_dim, int out_dim, int n_rows, float* y, void* stream) {
    int rc = check_matmul(n_rows > 1 ? "matmul_quant_batch" : "matmul_quant", type, in_dim, out_dim);
    if (rc) return rc;
    if (n_rows <= 0 || out_dim == 0) return CLLM_HIP_OK;
    if (!x || !w || !y) return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
    if (!aligned16(x) || !aligned16(w) || ((uintptr_t)y & 3u) || ((uintptr_t)bias & 3u))
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (!has_kernel(type)) {
        HIP_TRY(launch_gemv_f(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, y, s));
        return CLLM_HIP_OK;
    }
    WsView v;
    if (needs_workspace(type, in_dim, out_dim, n_rows)) {
        Workspace* ws;
        if ((rc = stream_workspace(st, s, type, in_dim, out_dim, n_rows, &ws))) return rc;
        v = ws->v;
    }
    if (!use_mfma(type, in_dim, out_dim, n_rows)) {
        // decode-sized batch: one or two rows in a single launch that quantizes them in LDS
        HIP_TRY(run_gemv_f32(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, y, v, s));
        return CLLM_HIP_OK;
    }
    HIP_TRY(run_gemm_f32(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, y, v, s));
    return CLLM_HIP_OK;
}

namespace {
// The routes of cllm_hip_matmul_quant_dev on scratch v.
int static_routes(uint32_t type, const void* w, int in_dim, int out_dim, int n_rows, const float* x,
                  const float* bias, float* y, const WsView& v, hipStream_t s) {
    if (!use_mfma(type, in_dim, out_dim, n_rows)) {
        HIP_TRY(run_gemv_f32(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, y, v, s));
        return CLLM_HIP_OK;
    }
    HIP_TRY(run_gemm_f32(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, y, v, s));
    return CLLM_HIP_OK;
}
}  // namespace

uint64_t cllm_hip_allocation_count(void) { return g_allocations.load(std::memory_order_relaxed); }

int cllm_hip_matmul_quant_static_dev(const float* x, const void* w, uint32_t type,
                                     const float* bias, int in_dim, int out_dim, int n_rows,
                                     float* y, void* stream) {
    int rc = check_matmul(n_rows > 1 ? "matmul_quant_batch" : "matmul_quant", type, in_dim, out_dim);
    if (rc) return rc;
    if (n_rows <= 0 || out_dim == 0) return CLLM_HIP_OK;
    if (!x || !w || !y) return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
    if (!aligned16(x) || !aligned16(w) || ((uintptr_t)y & 3u) || ((uintptr_t)bias & 3u))
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (!has_kernel(type)) {
        HIP_TRY(launch_gemv_f(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, y, s));
        return CLLM_HIP_OK;
    }
    // The same routes as cllm_hip_matmul_quant_dev, their scratch carved from this device's
    // static array: the activation arrays first, then the split-K region (at a multiple of
    // 256 bytes). Nothing is allocated.
    WsView v;
    size_t act = 0, pb = 0;
    if (needs_workspace(type, in_dim, out_dim, n_rows)) {
        act = act_bytes(in_dim, n_rows);
        if (use_mfma(type, in_dim, out_dim, n_rows) || use_small(type, in_dim, out_dim, n_rows))
            pb = part_bytes_for(type, in_dim, out_dim, n_rows);
    }
    if (act + pb > kStaticScratchBytes)
        return set_err(CLLM_HIP_E_ARG,
                       "matmul_quant: %d rows of %d need %zu bytes of scratch, more than the %zu "
                       "of the fixed buffer; pass fewer rows per call",
                       n_rows, in_dim, act + pb, kStaticScratchBytes);
    if (act + pb == 0) return static_routes(type, w, in_dim, out_dim, n_rows, x, bias, y, v, s);
    // One GPU's array serves every call on it. A call on another stream while an earlier
    // eager call's work may still run would overwrite that call's scratch: it is refused.
    // Calls on one stream are ordered by the stream. Under graph capture nothing runs now, so
    // nothing is checked or recorded (replays of graphs on different streams must be ordered
    // by the caller).
    std::lock_guard<std::mutex> lk(st->static_mtx);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(s, &cap));
    const bool eager = cap == hipStreamCaptureStatusNone;
    if (eager && st->static_pending && st->static_last != s) {
        const hipError_t q = hipEventQuery(st->static_done);
        if (q == hipErrorNotReady) {
            (void)hipGetLastError();
            return set_err(CLLM_HIP_E_BUSY,
                           "matmul_quant: the fixed scratch of device %d is in use by a call on "
                           "another stream; order the calls (same stream, or wait for it)",
                           current_device());
        }
        HIP_TRY(q);
    }
    if (act) carve_act((char*)st->scratch, in_dim, n_rows, v);
    if (pb) {
        v.part = (float*)(st->scratch + act);
        v.part_cap = pb;
        // the tile counters must start at zero; the last call on this GPU may have left
        // activations in these bytes (a fill kernel, so the call can be captured in a graph)
        HIP_TRY(gemmw_workspace_init(v.part, gemmw_counter_bytes(), s));
    }
    if ((rc = static_routes(type, w, in_dim, out_dim, n_rows, x, bias, y, v, s))) return rc;
    if (eager) {
        HIP_TRY(hipEventRecord(st->static_done, s));
        st->static_last = s;
        st->static_pending = true;
    }
    return CLLM_HIP_OK;
}

size_t cllm_hip_static_scratch_bytes(void) { return kStaticScratchBytes; }

int cllm_hip_matmul_quant_residual_dev(const float* x, const void* w, uint32_t type,
                                       const float* bias, int in_dim, int out_dim, int n_rows,
                                       float* y, void* stream) {
    int rc = check_matmul(n_rows > 1 ? "matmul_quant_batch" : "matmul_quant", type, in_dim, out_dim);
    if (rc) return rc;
    if (n_rows <= 0 || out_dim == 0) return CLLM_HIP_OK;
    if (!x || !w || !y) return set_err(CLLM_HIP_E_ARG, "matmul_quant: null pointer");
    if (!aligned16(x) || !aligned16(w) || !aligned16(y) || ((uintptr_t)bias & 3u))
        return set_err(CLLM_HIP_E_ARG, "matmul_quant: misaligned device pointer");
    DeviceState* st;
    if ((rc = acquire(&st))) return rc;
    hipStream_t s = (hipStream_t)stream;
    Workspace* ws = nullptr;
    if ((rc = stream_workspace(st, s, type, in_dim, out_dim, n_rows, &ws))) return rc;
    if (has_kernel(type) && !use_mfma(type, in_dim, out_dim, n_rows) && !use_small(type, in_dim, out_dim, n_rows)) {
        // the GEMV adds into y in its epilogue
        HIP_TRY(run_gemv_f32(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, y, ws->v, s,
                             true));
        return CLLM_HIP_OK;
    }
    const size_t bytes = (size_t)n_rows * out_dim * sizeof(float);
    {
        std::lock_guard<std::mutex> lk(st->mtx);
        HIP_TRY(ws->tmp.ensure(bytes, s));
    }
    float* t = (float*)ws->tmp.p;
    if (!has_kernel(type))
        HIP_TRY(launch_gemv_f(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, t, s));
    else
        HIP_TRY(run_gemm_f32(type, (const uint8_t*)w, in_dim, out_dim, n_rows, x, bias, t, ws->v, s));
    HIP_TRY(launch_add(y, t, (int64_t)n_rows * out_dim, s));
    return CLLM_HIP_OK;
}

int cllm_hip_rmsnorm_q8_0_dev(const float* x, const float* w, float eps, int n, int n_rows,
                              float* h, int8_t* qs, float* scales, int32_t* bsums,
                              void* stream) {
    if (n <= 0 || n_rows < 0) return set_err(CLLM_HIP_E_ARG, "rms_norm: bad shape");
    if (qs && n % 32 != 0)
        return set_err(CLLM_HIP_E_SHAPE, "quantize_row_q8_0: n not divisible by 32");
    if (!x || !w || (!h && !qs) || (qs && (!scales || !bsums)))
        return set_err(CLLM_HIP_E_ARG, "rms_norm: null pointer");
    if (!aligned16(x) || !aligned16(w) || (h && !aligned16(h)) || ((uintptr_t)qs & 3u) ||
        ((uintptr_t)scales & 3u) || ((uintptr_t)bsums & 3u))
        return set_err(CLLM_HIP_E_ARG, "rms_norm: misaligned device pointer");
    if (n_rows == 0) return CLLM_HIP_OK;
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    HIP_TRY(launch_rmsnorm_q8_0(x, w, eps, n, n_rows, h, qs, scales, bsums, (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_swiglu_q8_0_dev(const float* gate, const float* up, int n, int n_rows, float* h,
                             int8_t* qs, float* scales, int32_t* bsums, void* stream) {
    if (n <= 0 || n_rows < 0) return set_err(CLLM_HIP_E_ARG, "swiglu: bad shape");
    if (qs && n % 32 != 0)
        return set_err(CLLM_HIP_E_SHAPE, "quantize_row_q8_0: n not divisible by 32");
    if (!gate || !up || (!h && !qs) || (qs && (!scales || !bsums)))
        return set_err(CLLM_HIP_E_ARG, "swiglu: null pointer");
    if (!aligned16(gate) || !aligned16(up) || (h && !aligned16(h)) || ((uintptr_t)qs & 3u) ||
        ((uintptr_t)scales & 3u) || ((uintptr_t)bsums & 3u))
        return set_err(CLLM_HIP_E_ARG, "swiglu: misaligned device pointer");
    if (n_rows == 0) return CLLM_HIP_OK;
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    HIP_TRY(launch_swiglu_q8_0(gate, up, (int64_t)n * n_rows, h, qs, scales, bsums,
                               (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_add_dev(float* x, const float* d, int64_t n, void* stream) {
    if (n < 0) return set_err(CLLM_HIP_E_ARG, "add: negative length");
    if (n == 0) return CLLM_HIP_OK;
    if (!x || !d) return set_err(CLLM_HIP_E_ARG, "add: null pointer");
    if (!aligned16(x) || !aligned16(d)) return set_err(CLLM_HIP_E_ARG, "add: misaligned device pointer");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    HIP_TRY(launch_add(x, d, n, (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_dequantize_rows_dev(const void* w, uint32_t type, int in_dim, const int32_t* ids,
                                 int n_ids, float* out, void* stream) {
    const int bs = block_elems(type);
    if (!has_kernel(type) && !gemv_f_supported(type))
        return set_err(CLLM_HIP_E_TYPE, "unsupported ggml type for dequantize");
    if (in_dim <= 0 || in_dim % bs != 0)
        return set_err(CLLM_HIP_E_SHAPE, "dequantize: in_dim not divisible by block size");
    if (n_ids < 0) return set_err(CLLM_HIP_E_ARG, "dequantize: negative row count");
    if (n_ids == 0) return CLLM_HIP_OK;
    if (!w || !ids || !out) return set_err(CLLM_HIP_E_ARG, "dequantize: null pointer");
    if (!aligned16(w) || ((uintptr_t)ids & 3u) || ((uintptr_t)out & 15u))
        return set_err(CLLM_HIP_E_ARG, "dequantize: misaligned device pointer");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    HIP_TRY(launch_dequantize_rows(type, (const uint8_t*)w, in_dim, ids, n_ids, out,
                                   (hipStream_t)stream));
    return CLLM_HIP_OK;
}

int cllm_hip_rope_neox_dev(float* x, int n_rows, int n_heads, int head_dim, int pos0,
                           float theta_base, void* stream) {
    return cllm_hip_rope_neox2_dev(x, n_heads, nullptr, 0, n_rows, head_dim, pos0, theta_base,
                                   stream);
}

int cllm_hip_rope_neox2_dev(float* q, int n_head, float* k, int n_head_kv, int n_rows,
                            int head_dim, int pos0, float theta_base, void* stream) {
    if (!k) n_head_kv = 0;
    if (n_rows < 0 || n_head < 0 || n_head_kv < 0 || head_dim <= 0 || head_dim % 2 != 0 ||
        head_dim > 512 || pos0 < 0)
        return set_err(CLLM_HIP_E_ARG, "rope: bad shape");
    if (n_rows == 0 || n_head + n_head_kv == 0) return CLLM_HIP_OK;
    if (!q && n_head > 0) return set_err(CLLM_HIP_E_ARG, "rope: null pointer");
    if (((uintptr_t)q & 3u) || ((uintptr_t)k & 3u))
        return set_err(CLLM_HIP_E_ARG, "rope: misaligned device pointer");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    HIP_TRY(launch_rope_neox(q, n_rows, n_head, k, n_head_kv, head_dim, pos0, theta_base,
                             (hipStream_t)stream));
    return CLLM_HIP_OK;
}

static int attention_impl(const float* q, const float* k_cache, const float* v_cache,
                          int n_rows, int pos0, int n_head, int n_head_kv, int head_dim,
                          float* out, void* stream, float rope_base) {
    if (n_rows < 0 || pos0 < 0) return set_err(CLLM_HIP_E_ARG, "attention: bad shape");
    if (!attention_supported(head_dim, n_head, n_head_kv))
        return set_err(CLLM_HIP_E_ARG,
                       "attention: head_dim must be 64, 128 or 256 and n_head a multiple of "
                       "n_head_kv, at most 8 query heads per KV head");
    if (n_rows == 0) return CLLM_HIP_OK;
    if (!q || !k_cache || !v_cache || !out) return set_err(CLLM_HIP_E_ARG, "attention: null pointer");
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || ((uintptr_t)out & 3u))
        return set_err(CLLM_HIP_E_ARG, "attention: misaligned device pointer");
    DeviceState* st;
    int rc = acquire(&st);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    Workspace* ws;
    if ((rc = stream_workspace(st, s, T_Q8_0, 32, 0, 1, &ws))) return rc;
    const size_t bytes = attention_workspace_bytes(n_rows, n_head, head_dim);
    {
        std::lock_guard<std::mutex> lk(st->mtx);
        const void* before = ws->att.p;
        HIP_TRY(ws->att.ensure(bytes, s));
        // a new allocation starts with zero arrival counters; every launch leaves them zero
        if (ws->att.p != before) HIP_TRY(gemmw_workspace_init(ws->att.p, ws->att.cap, s));
    }
    HIP_TRY(launch_attention(q, k_cache, v_cache, n_rows, pos0, n_head, n_head_kv, head_dim, out,
                             ws->att.p, ws->att.cap, s, rope_base));
    return CLLM_HIP_OK;
}

int cllm_hip_attention_dev(const float* q, const float* k_cache, const float* v_cache,
                           int n_rows, int pos0, int n_head, int n_head_kv, int head_dim,
                           float* out, void* stream) {
    return attention_impl(q, k_cache, v_cache, n_rows, pos0, n_head, n_head_kv, head_dim, out,
                          stream, 0.0f);
}

const char* cllm_hip_attention_plan(int n_rows, int pos0, int n_head, int n_head_kv,
                                    int head_dim) {
    static thread_local char buf[96];
    if (n_rows <= 0 || pos0 < 0 || !attention_supported(head_dim, n_head, n_head_kv)) return "none";
    attention_plan_name(n_rows, pos0, n_head, n_head_kv, head_dim, buf, sizeof buf);
    return buf;
}

int cllm_hip_attention_rope_dev(const float* q, float* k_cache, const float* v_cache, int pos0,
                                int n_head, int n_head_kv, int head_dim, float theta_base,
                                float* out, void* stream) {
    if (!(theta_base > 0.0f)) return set_err(CLLM_HIP_E_ARG, "attention: theta_base must be positive");
    return attention_impl(q, k_cache, v_cache, 1, pos0, n_head, n_head_kv, head_dim, out, stream,
                          theta_base);
}

// ---- GGUF files (gguf.cpp:122-275 of the reference) ---------------------------------------

struct cllm_hip_gguf {
    cllm_hip::GgufFile file;
    int device = -1;        // device holding the upload, -1 if not uploaded
    void* dev = nullptr;    // device copy of the data section
    size_t dev_bytes = 0;
};

int cllm_hip_gguf_open(const char* path, int upload, cllm_hip_gguf** out) {
    if (!path || !out) return set_err(CLLM_HIP_E_ARG, "cllm_hip_gguf_open: null pointer");
    *out = nullptr;
    auto g = std::make_unique<cllm_hip_gguf>();
    std::string err;
    if (!cllm_hip::gguf_open(path, g->file, err)) return set_err(CLLM_HIP_E_ARG, "%s", err.c_str());
    if (upload) {
        DeviceState* st;
        int rc = acquire(&st);
        if (rc) return rc;
        const cllm_hip::GgufFile& f = g->file;
        const size_t bytes = f.map_bytes > f.data_offset ? f.map_bytes - f.data_offset : 0;
        if (bytes > 0) {
            // One pass over the data section through two pinned staging buffers: the host
            // copy into one buffer overlaps the DMA out of the other. The host copy (from the
            // mapped file) is split over a few threads, one slice of each chunk apiece: a
            // single thread copying out of the page cache cannot keep up with the DMA.
            constexpr size_t kChunk = 32u << 20;
            void* stage[2] = {nullptr, nullptr};
            hipEvent_t done[2] = {nullptr, nullptr};
            std::lock_guard<std::mutex> lk(st->mtx);
            hipError_t e = dev_alloc(&g->dev, bytes);
            for (int i = 0; i < 2 && e == hipSuccess; ++i) {
                g_allocations.fetch_add(1, std::memory_order_relaxed);
                e = hipHostMalloc(&stage[i], kChunk, hipHostMallocDefault);
                if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
            }
            const uint8_t* src = (const uint8_t*)f.map + f.data_offset;
            const int n_thr = (int)std::min<unsigned>(8u, std::max(1u, std::thread::hardware_concurrency()));
            struct CopyJob {
                void* dst = nullptr;
                const uint8_t* src = nullptr;
                size_t len = 0;
                bool quit = false;
            } job;
            std::barrier<> sync(n_thr + 1);  // two phases per chunk: job published, job done
            std::vector<std::thread> pool;
            for (int t = 0; t < n_thr; ++t)
                pool.emplace_back([&job, &sync, n_thr, t] {
                    for (;;) {
                        sync.arrive_and_wait();
                        if (job.quit) return;
                        const size_t per = (job.len + n_thr - 1) / n_thr;
                        const size_t a = std::min(job.len, (size_t)t * per), b = std::min(job.len, a + per);
                        if (b > a) std::memcpy((uint8_t*)job.dst + a, job.src + a, b - a);
                        sync.arrive_and_wait();
                    }
                });
            for (size_t off = 0, i = 0; e == hipSuccess && off < bytes; off += kChunk, ++i) {
                const size_t len = std::min(kChunk, bytes - off);
                const int b = (int)(i & 1);
                if (i >= 2) e = hipEventSynchronize(done[b]);
                if (e != hipSuccess) break;
                job.dst = stage[b];
                job.src = src + off;
                job.len = len;
                sync.arrive_and_wait();  // the workers copy the chunk
                sync.arrive_and_wait();
                e = hipMemcpyAsync((char*)g->dev + off, stage[b], len, hipMemcpyHostToDevice,
                                   st->stream);
                if (e == hipSuccess) e = hipEventRecord(done[b], st->stream);
            }
            job.quit = true;
            sync.arrive_and_wait();
            for (auto& th : pool) th.join();
            if (e == hipSuccess) e = hipStreamSynchronize(st->stream);
            for (int i = 0; i < 2; ++i) {
                if (done[i]) (void)hipEventDestroy(done[i]);
                if (stage[i]) (void)hipHostFree(stage[i]);
            }
            if (e != hipSuccess) {
                if (g->dev) (void)hipFree(g->dev);
                return set_err(CLLM_HIP_E_RUNTIME, "cllm_hip_gguf_open: upload failed: %s",
                               hipGetErrorString(e));
            }
            g->dev_bytes = bytes;
            g->device = current_device();
            // host pointers into the data section now resolve to the device copy
            st->regions[(uintptr_t)src] = Region{bytes, g->dev, g->dev};
        }
    }
    *out = g.release();
    return CLLM_HIP_OK;
}

int cllm_hip_gguf_close(cllm_hip_gguf* g) {
    if (!g) return CLLM_HIP_OK;
    std::unique_ptr<cllm_hip_gguf> own(g);
    if (g->dev) {
        const int saved = g_device;
        g_device = g->device;
        DeviceState* st;
        int rc = acquire(&st);
        g_device = saved;
        if (rc) return rc;
        std::lock_guard<std::mutex> lk(st->mtx);
        st->regions.erase((uintptr_t)g->file.map + g->file.data_offset);
        HIP_TRY(hipStreamSynchronize(st->stream));
        HIP_TRY(hipFree(g->dev));
        g->dev = nullptr;
    }
    return CLLM_HIP_OK;
}

int cllm_hip_gguf_tensor_count(const cllm_hip_gguf* g) { return g ? (int)g->file.tensors.size() : 0; }

int cllm_hip_gguf_find(const cllm_hip_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->file.index.find(name);
    return it == g->file.index.end() ? -1 : it->second;
}

int cllm_hip_gguf_tensor(const cllm_hip_gguf* g, int i, const char** name, uint32_t* type,
                         int* n_dims, uint64_t* dims, uint64_t* offset, const void** host,
                         const void** dev) {
    if (!g || i < 0 || i >= (int)g->file.tensors.size())
        return set_err(CLLM_HIP_E_ARG, "cllm_hip_gguf_tensor: no tensor %d", i);
    const cllm_hip::GgufTensor& t = g->file.tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (n_dims) *n_dims = (int)t.shape.size();
    if (dims)
        for (size_t d = 0; d < t.shape.size() && d < 4; ++d) dims[d] = t.shape[d];
    if (offset) *offset = t.offset;
    const size_t at = g->file.data_offset + t.offset;
    if (host) *host = (const uint8_t*)g->file.map + at;
    if (dev) *dev = g->dev ? (const uint8_t*)g->dev + t.offset : nullptr;
    return CLLM_HIP_OK;
}

int cllm_hip_gguf_config(const cllm_hip_gguf* g, cllm_hip_model_config* c) {
    if (!g || !c) return set_err(CLLM_HIP_E_ARG, "cllm_hip_gguf_config: null pointer");
    const cllm_hip::GgufConfig& f = g->file.config;
    std::memset(c, 0, sizeof *c);
    std::snprintf(c->arch, sizeof c->arch, "%s", f.arch.c_str());
    c->n_layers = f.n_layers;
    c->n_embd = f.n_embd;
    c->n_head = f.n_head;
    c->n_head_kv = f.n_head_kv;
    c->n_ctx = f.n_ctx;
    c->n_ff = f.n_ff;
    c->vocab_size = f.vocab_size;
    c->head_dim = f.head_dim_explicit > 0 ? f.head_dim_explicit : (f.n_head ? f.n_embd / f.n_head : 0);
    c->rope_theta = f.rope_theta;
    c->norm_eps = f.norm_eps;
    c->version = g->file.version;
    c->data_offset = g->file.data_offset;
    c->data_bytes = g->file.map_bytes > g->file.data_offset ? g->file.map_bytes - g->file.data_offset : 0;
    return CLLM_HIP_OK;
}

int cllm_hip_tune(const char* knob, const int* values, int n_values) {
    if (!knob || n_values < 0 || (n_values > 0 && !values))
        return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: bad arguments");
    Tuning& t = tuning();
    auto v = [&](int i) { return i < n_values ? values[i] : 0; };
    if (std::strcmp(knob, "gemm_kernel") == 0) {
        if (v(0) < 0 || v(0) > 2) return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: gemm_kernel is 0, 1 or 2");
        t.gemm_kind.store(v(0));
    } else if (std::strcmp(knob, "gemm_tiles") == 0) {
        t.gemm_waves.store(v(0));
        t.gemm_wtiles.store(v(1));
        t.gemm_ttiles.store(v(2));
    } else if (std::strcmp(knob, "gemm_splits") == 0) {
        t.gemm_splits.store(v(0));
    } else if (std::strcmp(knob, "gemv_kernel") == 0) {
        if (v(0) < 0 || v(0) > 3) return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: gemv_kernel is 0 to 3");
        t.gemv_kind.store(v(0));
    } else if (std::strcmp(knob, "gemv_str_grid") == 0) {
        if (v(0) < 0 || v(0) > 65535) return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: gemv_str_grid out of range");
        t.gemv_str_grid.store(v(0));
    } else if (std::strcmp(knob, "gemm_small") == 0) {
        if (v(0) < 0 || v(0) > 2) return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: gemm_small is 0, 1 or 2");
        t.gemm_small.store(v(0));
    } else if (std::strcmp(knob, "gemv_fused_rows") == 0) {
        if (v(0) < 0 || v(0) > 8) return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: gemv_fused_rows is 0 to 8");
        t.gemv_fused_rows.store(v(0));
    } else if (std::strcmp(knob, "gemm_small_q8") == 0) {
        if (v(0) < 0 || v(0) > 2) return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: gemm_small_q8 is 0, 1 or 2");
        t.gemm_small_q8.store(v(0));
    } else if (std::strcmp(knob, "attention_kernel") == 0) {
        if (v(0) < 0 || v(0) > 2) return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: attention_kernel is 0, 1 or 2");
        t.attention_kind.store(v(0));
    } else if (std::strcmp(knob, "gemv_fp_wgs") == 0) {
        if (v(0) < 0 || v(0) > 9) return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: gemv_fp_wgs is 0 to 9");
        t.gemv_fp_wgs.store(v(0));
    } else if (std::strcmp(knob, "gemm_small_plan") == 0) {
        t.gemm_small_splits.store(v(0));
        t.gemm_small_kp.store(v(1));
    } else if (std::strcmp(knob, "gemv_waves") == 0) {
        t.gemv_short_wps.store(v(0));
        t.gemv_deep_wps.store(v(1));
    } else {
        return set_err(CLLM_HIP_E_ARG, "cllm_hip_tune: unknown knob %s", knob);
    }
    return CLLM_HIP_OK;
}

const char* cllm_hip_matmul_plan(uint32_t type, int in_dim, int out_dim, int n_rows) {
    static thread_local char buf[128];
    const char* route = cllm_hip_matmul_route(type, in_dim, out_dim, n_rows);
    if (std::strcmp(route, "gemv") == 0) {
        gemv_plan_name(type, in_dim, out_dim, n_rows, buf, sizeof buf);
    } else if (std::strcmp(route, "small") == 0) {
        gemm_sm_plan_name(type, in_dim, out_dim, n_rows,
                          !small_quantize_once(type, in_dim, out_dim, n_rows), buf, sizeof buf);
    } else if (std::strcmp(route, "mfma") != 0) {
        snprintf(buf, sizeof buf, "%s", route);
    } else {
        const GemmKind kind = gemm_kind(type, in_dim, out_dim, n_rows);
        if (kind == GemmKind::W16)
            gemmw_plan_name(type, in_dim, out_dim, n_rows, buf, sizeof buf);
        else
            snprintf(buf, sizeof buf, "%s", kind == GemmKind::I8 ? "k_gemm_i8" : "k_gemm16");
    }
    return buf;
}

const char* cllm_hip_matmul_route(uint32_t type, int in_dim, int out_dim, int n_rows) {
    if (gemv_f_supported(type)) return "fdot";
    if (!has_kernel(type)) return "none";
    if (use_small(type, in_dim, out_dim, n_rows)) return "small";
    return use_mfma(type, in_dim, out_dim, n_rows) ? "mfma" : "gemv";
}

}  // extern "C"
