// Handle runtime of libfracture_hip.so: the C-ABI mirror of Fracture's `Backend` trait
// (crates/fracture-core/src/backend.rs:8-223) and of the inherent CudaBackend API
// (backends/fracture-cuda/src/lib.rs:76-182, backend.rs:7-710).
//
// One HIP stream per backend, a mutex-guarded id -> device pointer registry, event timers,
// roctx markers. Host-side arguments (positions, token ids, block tables, page pointer
// tables) go through a ring of pinned staging slots copied with hipMemcpyAsync on the
// backend's stream; each slot is reused only after the event recorded behind the kernel that
// read it has completed, so no per-call hipMalloc/hipFree is needed (the reference mallocs
// and frees them synchronously on every call, backend.rs:178-204, 387-410, 643-705).
#include <hip/hip_runtime.h>
#include <dlfcn.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cstdint>
#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "fracture_hip.h"
#include "fhip_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

// Reports a failed HIP call and clears HIP's per-thread last error, so that a recoverable
// failure (an allocation beyond the device, say) is not reported again by the next launch.
int hip_fail(hipError_t e) {
    (void)hipGetLastError();
    return fail(FHIP_ERR_BACKEND, "HIP error (%d): %s", (int)e, hipGetErrorString(e));
}

#define HIP_TRY(call)                                \
    do {                                             \
        hipError_t e_ = (call);                      \
        if (e_ != hipSuccess) return hip_fail(e_);   \
    } while (0)

int launch_result(int e) {
    if (e != hipSuccess) return hip_fail((hipError_t)e);
    return FHIP_OK;
}

size_t dtype_size(int dt) {
    switch (dt) {
        case FHIP_FP16: return 2;
        case FHIP_FP32: return 4;
        case FHIP_BF16: return 2;
        case FHIP_INT8: return 1;
        case FHIP_INT4: return 1;
        default: return 0;
    }
}
const char* dtype_name(int dt) {
    switch (dt) {
        case FHIP_FP16: return "FP16";
        case FHIP_FP32: return "FP32";
        case FHIP_BF16: return "BF16";
        case FHIP_INT8: return "INT8";
        case FHIP_INT4: return "INT4";
        default: return "?";
    }
}

uint64_t numel(const fhip_tensor* t) {
    uint64_t n = 1;
    for (int i = 0; i < t->ndim; ++i) n *= t->shape[i];
    return n;
}
// DeviceTensor::size_bytes (tensor.rs:53-60): INT4 packs two elements per byte.
uint64_t size_bytes(const fhip_tensor* t) {
    const uint64_t n = numel(t);
    return t->dtype == FHIP_INT4 ? (n + 1) / 2 : n * dtype_size(t->dtype);
}
std::string shape_str(const fhip_tensor* t) {
    std::string s = "[";
    for (int i = 0; i < t->ndim; ++i) {
        if (i) s += ", ";
        s += std::to_string(t->shape[i]);
    }
    return s + "]";
}
bool same_shape(const fhip_tensor* a, const fhip_tensor* b) {
    if (a->ndim != b->ndim) return false;
    for (int i = 0; i < a->ndim; ++i)
        if (a->shape[i] != b->shape[i]) return false;
    return true;
}
bool valid_desc(const fhip_tensor* t) {
    return t && t->ndim >= 0 && t->ndim <= FHIP_MAX_DIMS && dtype_size(t->dtype) != 0;
}

// roctx, loaded on first use; markers are no-ops without it.
struct Roctx {
    int (*push)(const char*) = nullptr;
    int (*pop)() = nullptr;
    std::once_flag once;
    void load() {
        std::call_once(once, [this] {
            void* h = dlopen("libroctx64.so", RTLD_LAZY | RTLD_LOCAL);
            if (!h) h = dlopen("/opt/rocm/lib/libroctx64.so", RTLD_LAZY | RTLD_LOCAL);
            if (!h) return;
            push = (int (*)(const char*))dlsym(h, "roctxRangePushA");
            pop = (int (*)())dlsym(h, "roctxRangePop");
        });
    }
} g_roctx;

// Pinned host + device staging slot for small host-side arguments.
struct StageSlot {
    void* host = nullptr;
    void* dev = nullptr;
    size_t cap = 0;
    hipEvent_t ev = nullptr;  // recorded on the group's last slot only
    bool pending = false;
    bool dirty = false;       // handed out since its group's event was last recorded
};

// Device memory for small tensors. Tensors of at most kMaxBytes are carved out of large
// chunks in power-of-two size classes (256 B to 64 KB) and recycled through per-class free
// lists. A chunk that cannot be allocated is retried at half the size down to one tensor, and
// a tensor the arena cannot place gets its own hipMalloc. Freed arena memory stays with the
// backend for reuse until it is destroyed (fhip_available_memory does not count it). A KV cache of one tensor per (block, layer), as the reference's cache managers
// allocate it (quantized_paged_kv_cache.rs:82-133), then lies in a few large mappings instead
// of one small mapping per tensor: on MI355X the TurboQuant decode kernel over such blocks
// measured ~7% faster (the per-tensor mappings cost address-translation misses).
// Callers hold the backend's registry mutex.
struct SmallArena {
    static constexpr int kClasses = 9;
    static constexpr size_t kMinBytes = 256, kMaxBytes = kMinBytes << (kClasses - 1);
    static constexpr size_t kFirstChunk = (size_t)4 << 20, kMaxChunk = (size_t)256 << 20;
    std::vector<void*> chunks;
    std::vector<void*> free_list[kClasses];
    char* cur[kClasses] = {};
    size_t left[kClasses] = {};
    size_t next_chunk[kClasses] = {};
    std::unordered_map<void*, int> owned;  // arena pointer -> size class

    static int size_class(size_t bytes) {
        int c = 0;
        while ((kMinBytes << c) < bytes) ++c;
        return c;
    }
    hipError_t alloc(size_t bytes, void** out) {
        const int c = size_class(bytes ? bytes : 1);
        const size_t sz = kMinBytes << c;
        void* p;
        if (!free_list[c].empty()) {
            p = free_list[c].back();
            free_list[c].pop_back();
        } else {
            if (left[c] < sz) {
                size_t n = next_chunk[c] ? next_chunk[c] : kFirstChunk;
                next_chunk[c] = n < kMaxChunk ? 2 * n : kMaxChunk;
                void* chunk = nullptr;
                hipError_t e = hipMalloc(&chunk, n);
                // a chunk that does not fit: halve it down to one tensor of the class
                while (e != hipSuccess && n > sz) {
                    n = n / 2 > sz ? n / 2 : sz;
                    e = hipMalloc(&chunk, n);
                }
                if (e != hipSuccess) return e;
                (void)hipGetLastError();  // the failed attempts leave no error behind
                next_chunk[c] = n < kMaxChunk ? 2 * n : kMaxChunk;
                chunks.push_back(chunk);
                cur[c] = (char*)chunk;
                left[c] = n;
            }
            p = cur[c];
            cur[c] += sz;
            left[c] -= sz;
        }
        owned[p] = c;
        *out = p;
        return hipSuccess;
    }
    // true if p came from the arena (it is then free for reuse)
    bool release(void* p) {
        auto it = owned.find(p);
        if (it == owned.end()) return false;
        free_list[it->second].push_back(p);
        owned.erase(it);
        return true;
    }
    bool owns(void* p) const { return owned.count(p) != 0; }
    void destroy() {
        for (void* c : chunks) (void)hipFree(c);
        chunks.clear();
        owned.clear();
        for (auto& f : free_list) f.clear();
    }
};

}  // namespace

struct fhip_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string name;
    size_t total_mem = 0;
    std::mutex mu;  // registry, timers
    std::unordered_map<uint64_t, void*> tensors;
    SmallArena arena;  // under mu
    uint64_t next_id = 1;
    std::unordered_map<uint64_t, std::pair<hipEvent_t, hipEvent_t>> timers;
    uint64_t next_timer = 1;
    float* rope_freq = nullptr;
    size_t rope_half = 0;
    // graph capture (fhip_graph_begin / fhip_graph_end): while set, launches on `stream` are
    // recorded into a graph instead of running, and only the ops whose arguments are all
    // device-resident and that never wait on the host are accepted
    std::atomic<bool> capturing{false};
    // A graph keeps the device addresses of the tensors its launches used: the ids resolved
    // while capturing are kept with it, and fhip_free refuses a tensor that a live graph uses
    // (its block could be handed to another tensor, which a replay would then overwrite).
    struct GraphRec {
        hipGraphExec_t exec;
        std::vector<uint64_t> ids;
    };
    std::unordered_map<uint64_t, GraphRec> graphs;  // under mu
    std::unordered_set<uint64_t> capture_ids;       // under mu
    std::unordered_map<uint64_t, int> graph_refs;   // tensor id -> live graphs using it (mu)
    uint64_t next_graph = 1;
    // launch lock: staging ring and workspace are per backend
    std::mutex launch_mu;
    static constexpr int kSlots = 16;
    // slots guarded by one event: reusing a group's first slot waits for the call
    // kSlots - kGroup + 1 calls back, so kSlots - kGroup calls stay queued on the GPU
    static constexpr int kGroup = 8;
    static_assert(kSlots % kGroup == 0 && (kGroup & (kGroup - 1)) == 0, "slot groups");
    StageSlot slots[kSlots];
    // side stream for staging copies that may run ahead of `stream` (default priority)
    hipStream_t copy_stream = nullptr;
    hipEvent_t copy_ev[kSlots] = {};
    int next_slot = 0;
    void* workspace = nullptr;
    size_t ws_cap = 0;
    // registered KV page pools: device-resident arrays of the pool's per-block addresses
    struct PagePool {
        const void** dev = nullptr;          // nlists * pool_len addresses, list-major
        size_t pool_len = 0;
        int nlists = 0;
        std::vector<uint64_t> min_bytes;     // smallest block tensor of each list
        std::vector<int32_t> dtype;          // each list's dtype (-1: mixed)
        std::vector<uint64_t> ids;           // the block tensors
    };
    std::unordered_map<uint64_t, PagePool> pools;  // under mu
    uint64_t next_pool = 1;
    std::unordered_map<uint64_t, int> pooled;      // tensor id -> pools holding it (under mu)
    // TurboQuant plans, keyed on (rotation id, centroids id, bits, levels): what compress and
    // dequantize derive from the per-layer tables the cache manager uploads once
    // (quantized_paged_kv_cache.rs:137-170). A plan is dropped when fhip_free,
    // fhip_copy_to_device or fhip_copy_rows touches either tensor; callers hold plan_mu from
    // the lookup until the launch that uses the plan is enqueued.
    struct PlanEntry {
        uint64_t rot, cent;
        int bits, levels;
        fhip_tq_plan* plan;
    };
    std::mutex plan_mu;
    std::vector<PlanEntry> plans;

    // The plan for these tables (built on first use), or null where the MFMA path does not
    // apply (head_dim other than 128) or the plan cannot be built: callers then launch the
    // unplanned kernels, which compute the same bytes.
    fhip_tq_plan* plan_for(uint64_t rot_id, const void* rot, uint64_t cent_id, const void* cent,
                           int levels, int bits, int head_dim) {
        if (head_dim != 128) return nullptr;
        {
            // no plan from a tensor of a registered pool: the pool's writers (append_kv) do
            // not check for plans
            std::lock_guard<std::mutex> g(mu);
            if (pooled.count(rot_id) || pooled.count(cent_id)) return nullptr;
        }
        for (const PlanEntry& e : plans)
            if (e.rot == rot_id && e.cent == cent_id && e.bits == bits && e.levels == levels)
                return e.plan;
        fhip_tq_plan* p = nullptr;
        if (fhip_tq_plan_create((const float*)rot, (const float*)cent, levels, bits, head_dim,
                                stream, &p) != hipSuccess)
            return nullptr;
        plans.push_back(PlanEntry{rot_id, cent_id, bits, levels, p});
        return p;
    }
    // Called for every tensor an op writes (and for a freed one): a plan built from it is
    // stale and is destroyed. Destroying one waits for its kernels and frees device memory,
    // which a graph capture cannot do, so such a write is refused while capturing.
    int drop_plans(uint64_t id) {
        std::lock_guard<std::mutex> g(plan_mu);
        for (size_t i = 0; i < plans.size();) {
            if (plans[i].rot == id || plans[i].cent == id) {
                if (capturing)
                    return fail(FHIP_ERR_BACKEND, "tensor id %llu holds the tables of a "
                                "TurboQuant plan: it cannot be written during graph capture",
                                (unsigned long long)id);
                fhip_tq_plan_destroy(plans[i].plan);  // waits for kernels still using it
                plans[i] = plans.back();
                plans.pop_back();
            } else {
                ++i;
            }
        }
        return FHIP_OK;
    }

    int get_ptr(uint64_t id, void** out) {
        std::lock_guard<std::mutex> g(mu);
        auto it = tensors.find(id);
        if (it == tensors.end())
            return fail(FHIP_ERR_TENSOR_NOT_FOUND, "tensor id %llu",
                        (unsigned long long)id);
        if (capturing) capture_ids.insert(id);
        *out = it->second;
        return FHIP_OK;
    }

    // The next slot, free (its last reader has completed) and at least `bytes` large.
    // Slots are handed out in ring order and guarded in groups of kGroup: stage_done of a
    // group's last slot records one event after that call's kernels, which follow the
    // kernels of the group's other slots in stream order. An event is a queue packet between
    // two calls' kernels, so one per kGroup calls costs the compute queue less idle time than
    // one per call. A slot handed out again without its group's event recorded since (a call
    // that returned an error before stage_done) waits for both streams instead.
    int next_free_slot(size_t bytes, int* slot_out) {
        const int si = next_slot;
        next_slot = (next_slot + 1) % kSlots;
        StageSlot& s = slots[si];
        StageSlot& last = slots[si | (kGroup - 1)];
        if (last.pending) {
            HIP_TRY(hipEventSynchronize(last.ev));
            last.pending = false;
        }
        if (s.dirty) {
            HIP_TRY(hipStreamSynchronize(stream));
            if (copy_stream) HIP_TRY(hipStreamSynchronize(copy_stream));
            for (StageSlot& o : slots) o.dirty = o.pending = false;
        }
        s.dirty = true;
        if (!s.ev) HIP_TRY(hipEventCreateWithFlags(&s.ev, hipEventDisableTiming));
        if (bytes > s.cap) {
            if (s.host) HIP_TRY(hipHostFree(s.host));
            if (s.dev) HIP_TRY(hipFree(s.dev));
            s.host = s.dev = nullptr;
            s.cap = 0;
            size_t cap = 256;
            while (cap < bytes) cap *= 2;
            HIP_TRY(hipHostMalloc(&s.host, cap, hipHostMallocDefault));
            HIP_TRY(hipMalloc(&s.dev, cap));
            s.cap = cap;
        }
        *slot_out = si;
        return FHIP_OK;
    }
    // Copy `bytes` of host data to a device staging slot; returns the slot index. Callers
    // hold launch_mu and call stage_done(slot) after enqueuing the consumer kernel.
    int stage(const void* src, size_t bytes, void** dev_out, int* slot_out) {
        int si;
        int r = next_free_slot(bytes, &si);
        if (r) return r;
        StageSlot& s = slots[si];
        if (bytes) {
            memcpy(s.host, src, bytes);
            HIP_TRY(hipMemcpyAsync(s.dev, s.host, bytes, hipMemcpyHostToDevice, stream));
        }
        *dev_out = s.dev;
        *slot_out = si;
        return FHIP_OK;
    }
    // A slot of at least `bytes` whose host side the caller fills (host_out), then
    // stage_ahead_copy(slot, bytes) issues its copy on the backend's copy stream, so it
    // proceeds while `stream` still runs earlier calls' kernels (a copy queued on `stream`
    // itself costs the copy plus two hand-offs between the copy engine and the compute queue
    // in the call's own time), and stage_ahead_wait(slot) waits for it on the host before the
    // caller enqueues the kernels that read the slot (host work can run in between): a
    // cross-stream wait on `stream` would be one more packet between two calls' kernels.
    // Callers hold launch_mu and call stage_done(slot) after enqueuing the last kernel that
    // reads the slot.
    int stage_ahead_begin(size_t bytes, void** host_out, void** dev_out, int* slot_out) {
        int si;
        int r = next_free_slot(bytes, &si);
        if (r) return r;
        if (!copy_stream) HIP_TRY(hipStreamCreateWithFlags(&copy_stream, hipStreamNonBlocking));
        if (!copy_ev[si]) HIP_TRY(hipEventCreateWithFlags(&copy_ev[si], hipEventDisableTiming));
        *host_out = slots[si].host;
        *dev_out = slots[si].dev;
        *slot_out = si;
        return FHIP_OK;
    }
    int stage_ahead_copy(int si, size_t bytes) {
        HIP_TRY(hipMemcpyAsync(slots[si].dev, slots[si].host, bytes, hipMemcpyHostToDevice,
                               copy_stream));
        HIP_TRY(hipEventRecord(copy_ev[si], copy_stream));
        return FHIP_OK;
    }
    int stage_ahead_wait(int si) {
        HIP_TRY(hipEventSynchronize(copy_ev[si]));
        return FHIP_OK;
    }
    int stage_done(int si) {
        if ((si & (kGroup - 1)) != kGroup - 1) return FHIP_OK;
        HIP_TRY(hipEventRecord(slots[si].ev, stream));
        slots[si].pending = true;
        for (int i = si - (kGroup - 1); i <= si; ++i) slots[i].dirty = false;
        return FHIP_OK;
    }
    // Backend-owned scratch (softmax partials, attention split partials). Callers hold
    // launch_mu. Every user of the workspace runs on `stream`, so stream order already keeps
    // one call's kernels from overwriting the previous call's partials, and no per-call event
    // is recorded (each one is a queue packet between two calls' kernels); growing the
    // workspace waits for the stream before freeing the old one.
    int get_workspace(size_t bytes, void** out) {
        if (bytes > ws_cap) {
            // a captured graph would keep the old address, and a capturing stream cannot be
            // waited for
            if (capturing)
                return fail(FHIP_ERR_BACKEND, "the workspace must grow to %zu bytes during graph "
                            "capture: run the operation once before capturing it", bytes);
            if (workspace) {
                HIP_TRY(hipStreamSynchronize(stream));
                HIP_TRY(hipFree(workspace));
            }
            workspace = nullptr;
            ws_cap = 0;
            size_t cap = 1 << 20;
            while (cap < bytes) cap *= 2;
            HIP_TRY(hipMalloc(&workspace, cap));
            ws_cap = cap;
        }
        *out = workspace;
        return FHIP_OK;
    }
};

namespace {

#define CHECK_B(b) \
    if (!(b)) return fail(FHIP_ERR_BACKEND, "null backend handle")
#define NO_CAPTURE(b, what)                                                                  \
    if ((b)->capturing)                                                                      \
    return fail(FHIP_ERR_BACKEND, "%s is not allowed during graph capture (it reads host "  \
                "memory, waits on the host or allocates)", what)
#define CHECK_T(t) \
    if (!valid_desc(t)) return fail(FHIP_ERR_INVALID_SHAPE, "invalid tensor descriptor")
#define GET_PTR(b, t, p)                         \
    void* p = nullptr;                           \
    {                                            \
        int r_ = (b)->get_ptr((t)->id, &p);      \
        if (r_ != FHIP_OK) return r_;            \
    }

// An op's output tensor: a TurboQuant plan built from it is dropped (see drop_plans).
#define WRITES(b, t)                              \
    {                                             \
        int w_ = (b)->drop_plans((t)->id);        \
        if (w_ != FHIP_OK) return w_;             \
    }

int set_device(fhip_backend* b) {
    HIP_TRY(hipSetDevice(b->device));
    return FHIP_OK;
}

}  // namespace

extern "C" {

const char* fhip_last_error(void) { return g_last_error.c_str(); }

int fhip_backend_create(int device_id, fhip_backend** out) {
    if (!out) return fail(FHIP_ERR_BACKEND, "null output handle");
    *out = nullptr;
    HIP_TRY(hipSetDevice(device_id));
    hipDeviceProp_t props;
    HIP_TRY(hipGetDeviceProperties(&props, device_id));
    fhip_backend* b = new fhip_backend();
    b->device = device_id;
    hipError_t e = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete b;
        return hip_fail(e);
    }
    b->name = props.name;
    b->total_mem = props.totalGlobalMem;
    *out = b;
    return FHIP_OK;
}

void fhip_backend_destroy(fhip_backend* b) {
    if (!b) return;
    (void)hipSetDevice(b->device);
    if (b->capturing) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(b->stream, &g);
        if (g) (void)hipGraphDestroy(g);
        b->capturing = false;
    }
    (void)hipStreamSynchronize(b->stream);
    for (auto& kv : b->graphs) (void)hipGraphExecDestroy(kv.second.exec);
    for (auto& kv : b->tensors)
        if (!b->arena.owns(kv.second)) (void)hipFree(kv.second);
    b->arena.destroy();
    for (auto& kv : b->timers) {
        (void)hipEventDestroy(kv.second.first);
        (void)hipEventDestroy(kv.second.second);
    }
    if (b->copy_stream) (void)hipStreamSynchronize(b->copy_stream);
    for (auto& s : b->slots) {
        if (s.host) (void)hipHostFree(s.host);
        if (s.dev) (void)hipFree(s.dev);
        if (s.ev) (void)hipEventDestroy(s.ev);
    }
    for (hipEvent_t e : b->copy_ev)
        if (e) (void)hipEventDestroy(e);
    if (b->copy_stream) (void)hipStreamDestroy(b->copy_stream);
    if (b->workspace) (void)hipFree(b->workspace);
    for (auto& e : b->plans) fhip_tq_plan_destroy(e.plan);
    for (auto& kv : b->pools) (void)hipFree((void*)kv.second.dev);
    if (b->rope_freq) (void)hipFree(b->rope_freq);
    (void)hipStreamDestroy(b->stream);
    delete b;
}

int fhip_get_ptr(fhip_backend* b, uint64_t id, void** out) {
    CHECK_B(b);
    if (!out) return fail(FHIP_ERR_BACKEND, "null output pointer");
    return b->get_ptr(id, out);
}

fhip_stream_t fhip_stream(fhip_backend* b) { return b ? (fhip_stream_t)b->stream : nullptr; }

int fhip_precompute_rope_freqs(fhip_backend* b, size_t head_dim, double theta) {
    CHECK_B(b);
    NO_CAPTURE(b, "precompute_rope_freqs");
    if (head_dim < 2 || head_dim % 2 != 0 || head_dim > 4096)
        return fail(FHIP_ERR_INVALID_SHAPE, "rope head_dim must be even and in [2, 4096], got %zu",
                    head_dim);
    set_device(b);
    const size_t half = head_dim / 2;
    std::vector<float> f(half);
    fhip_rope_freqs((int)head_dim, theta, f.data());
    float* dev = nullptr;
    HIP_TRY(hipMalloc(&dev, half * sizeof(float)));
    hipError_t e = hipMemcpy(dev, f.data(), half * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e);
    }
    std::lock_guard<std::mutex> g(b->launch_mu);
    if (b->rope_freq) {
        (void)hipStreamSynchronize(b->stream);
        (void)hipFree(b->rope_freq);
    }
    b->rope_freq = dev;
    b->rope_half = half;
    return FHIP_OK;
}

int fhip_alloc(fhip_backend* b, const uint64_t* shape, int ndim, int dtype, fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "alloc");
    if (!out || ndim < 0 || ndim > FHIP_MAX_DIMS || (ndim > 0 && !shape))
        return fail(FHIP_ERR_INVALID_SHAPE, "invalid shape (ndim %d)", ndim);
    if (dtype_size(dtype) == 0) return fail(FHIP_ERR_UNSUPPORTED_DTYPE, "dtype %d", dtype);
    fhip_tensor t;
    memset(&t, 0, sizeof t);
    t.dtype = dtype;
    t.ndim = ndim;
    unsigned __int128 n = 1;
    for (int i = 0; i < ndim; ++i) {
        t.shape[i] = shape[i];
        n *= shape[i];
    }
    if (n > ((unsigned __int128)1 << 62))
        return fail(FHIP_ERR_BACKEND, "HIP error (%d): %s", (int)hipErrorOutOfMemory,
                    hipGetErrorString(hipErrorOutOfMemory));
    const uint64_t bytes = size_bytes(&t);
    set_device(b);
    void* p = nullptr;
    std::lock_guard<std::mutex> g(b->mu);
    // small tensors (a zero-byte one included, so that its id still resolves) come from the
    // arena
    if (bytes <= SmallArena::kMaxBytes && b->arena.alloc(bytes, &p) == hipSuccess) {
    } else {
        (void)hipGetLastError();
        HIP_TRY(hipMalloc(&p, bytes ? bytes : 1));
    }
    t.id = b->next_id++;
    b->tensors[t.id] = p;
    *out = t;
    return FHIP_OK;
}

int fhip_free(fhip_backend* b, const fhip_tensor* t) {
    CHECK_B(b);
    NO_CAPTURE(b, "free");
    if (!t) return fail(FHIP_ERR_INVALID_SHAPE, "null tensor");
    void* p = nullptr;
    {
        std::lock_guard<std::mutex> g(b->mu);
        auto it = b->tensors.find(t->id);
        if (it == b->tensors.end())
            return fail(FHIP_ERR_TENSOR_NOT_FOUND, "tensor id %llu",
                        (unsigned long long)t->id);
        // a registered page pool keeps the tensor's address in device memory
        if (b->pooled.count(t->id))
            return fail(FHIP_ERR_BACKEND, "tensor id %llu is in a registered page pool",
                        (unsigned long long)t->id);
        if (b->graph_refs.count(t->id))
            return fail(FHIP_ERR_BACKEND, "tensor id %llu is used by a captured graph "
                        "(destroy the graph first)", (unsigned long long)t->id);
        p = it->second;
        b->tensors.erase(it);
    }
    set_device(b);
    (void)b->drop_plans(t->id);  // not capturing (NO_CAPTURE above)
    // Kernels on the backend's stream may still read the buffer.
    HIP_TRY(hipStreamSynchronize(b->stream));
    {
        std::lock_guard<std::mutex> g(b->mu);
        if (b->arena.release(p)) return FHIP_OK;
    }
    HIP_TRY(hipFree(p));
    return FHIP_OK;
}

int fhip_copy_to_device(fhip_backend* b, const fhip_tensor* dst, const void* src, size_t src_len) {
    CHECK_B(b);
    NO_CAPTURE(b, "copy_to_device");
    CHECK_T(dst);
    GET_PTR(b, dst, p);
    const uint64_t size = size_bytes(dst);
    if (src_len < size)
        return fail(FHIP_ERR_INVALID_SHAPE, "source buffer too small: %zu < %llu",
                    src_len, (unsigned long long)size);
    if (size == 0) return FHIP_OK;
    set_device(b);
    WRITES(b, dst);
    HIP_TRY(hipMemcpyAsync(p, src, size, hipMemcpyHostToDevice, b->stream));
    HIP_TRY(hipStreamSynchronize(b->stream));
    return FHIP_OK;
}

int fhip_copy_to_host(fhip_backend* b, const fhip_tensor* src, void* dst, size_t dst_len) {
    CHECK_B(b);
    NO_CAPTURE(b, "copy_to_host");
    CHECK_T(src);
    GET_PTR(b, src, p);
    const uint64_t size = size_bytes(src);
    if (dst_len < size)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "destination buffer too small: %zu < %llu", dst_len,
                    (unsigned long long)size);
    if (size == 0) return FHIP_OK;
    set_device(b);
    HIP_TRY(hipMemcpyAsync(dst, p, size, hipMemcpyDeviceToHost, b->stream));
    HIP_TRY(hipStreamSynchronize(b->stream));
    return FHIP_OK;
}

int fhip_rmsnorm(fhip_backend* b, const fhip_tensor* input, const fhip_tensor* weight, double eps,
                 const fhip_tensor* out) {
    CHECK_B(b);
    CHECK_T(input);
    CHECK_T(weight);
    CHECK_T(out);
    GET_PTR(b, input, pin);
    GET_PTR(b, weight, pw);
    GET_PTR(b, out, pout);
    WRITES(b, out);
    if (input->ndim < 1)
        return fail(FHIP_ERR_INVALID_SHAPE, "rmsnorm input must be 2-D");
    const uint64_t cols = input->shape[input->ndim - 1];
    const uint64_t rows = cols ? numel(input) / cols : 0;
    if (numel(weight) != cols || numel(out) != numel(input) || weight->dtype != input->dtype ||
        out->dtype != input->dtype)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "rmsnorm: input %s %s, weight %s %s, out %s %s",
                    shape_str(input).c_str(), dtype_name(input->dtype), shape_str(weight).c_str(),
                    dtype_name(weight->dtype), shape_str(out).c_str(), dtype_name(out->dtype));
    if (input->dtype != FHIP_FP16 && input->dtype != FHIP_BF16 && input->dtype != FHIP_FP32)
        return fail(FHIP_ERR_UNSUPPORTED_DTYPE, "rmsnorm %s",
                    dtype_name(input->dtype));
    if (rows == 0) return FHIP_OK;
    set_device(b);
    g_roctx.load();
    return launch_result(fhip_launch_rmsnorm_ex(pout, pin, pw, (float)eps, (int)rows, (int)cols,
                                                input->dtype, b->stream));
}

// Backend::matmul (cuda/src/backend.rs:75-128): out = a · bᵀ, a [M, K], b [N, K], out [M, N].
int fhip_matmul(fhip_backend* b, const fhip_tensor* a, const fhip_tensor* bm,
                const fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "matmul");
    CHECK_T(a);
    CHECK_T(bm);
    CHECK_T(out);
    GET_PTR(b, a, pa);
    GET_PTR(b, bm, pb);
    GET_PTR(b, out, pc);
    WRITES(b, out);
    if (a->ndim != 2 || bm->ndim != 2)
        return fail(FHIP_ERR_INVALID_SHAPE, "matmul: A %s and B %s must be 2-D",
                    shape_str(a).c_str(), shape_str(bm).c_str());
    if (a->shape[1] != bm->shape[1])
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "matmul: A inner dim %llu != B inner dim %llu (A is %s, B is %s)",
                    (unsigned long long)a->shape[1], (unsigned long long)bm->shape[1],
                    shape_str(a).c_str(), shape_str(bm).c_str());
    const uint64_t M = a->shape[0], K = a->shape[1], N = bm->shape[0];
    if (a->dtype != FHIP_FP16 || bm->dtype != FHIP_FP16 || out->dtype != FHIP_FP16)
        return fail(FHIP_ERR_UNSUPPORTED_DTYPE, "matmul is fp16 (A %s, B %s, out %s)",
                    dtype_name(a->dtype), dtype_name(bm->dtype), dtype_name(out->dtype));
    if (numel(out) != M * N)
        return fail(FHIP_ERR_INVALID_SHAPE, "matmul: out %s for a [%llu, %llu] result",
                    shape_str(out).c_str(), (unsigned long long)M, (unsigned long long)N);
    if (M > 0x7fffffffu || N > 0x7fffffffu || K > 0x7fffffffu)
        return fail(FHIP_ERR_INVALID_SHAPE, "matmul: dimensions beyond int32");
    if (M == 0 || N == 0) return FHIP_OK;
    set_device(b);
    return launch_result(fhip_launch_matmul(pc, pa, pb, (int)M, (int)N, (int)K, b->stream));
}

int fhip_add_rmsnorm(fhip_backend* b, const fhip_tensor* residual, const fhip_tensor* delta,
                     const fhip_tensor* weight, double eps, const fhip_tensor* normed_out) {
    CHECK_B(b);
    CHECK_T(residual);
    CHECK_T(delta);
    CHECK_T(weight);
    CHECK_T(normed_out);
    GET_PTR(b, residual, ph);
    WRITES(b, residual);
    GET_PTR(b, delta, pd);
    GET_PTR(b, weight, pw);
    GET_PTR(b, normed_out, po);
    WRITES(b, normed_out);
    if (residual->ndim < 1)
        return fail(FHIP_ERR_INVALID_SHAPE, "add_rmsnorm needs 2-D input");
    const uint64_t cols = residual->shape[residual->ndim - 1];
    const uint64_t rows = cols ? numel(residual) / cols : 0;
    if (!same_shape(residual, delta) || numel(normed_out) != numel(residual) ||
        numel(weight) != cols || delta->dtype != residual->dtype ||
        weight->dtype != residual->dtype || normed_out->dtype != residual->dtype)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "add_rmsnorm: residual %s, delta %s, weight %s, out %s",
                    shape_str(residual).c_str(), shape_str(delta).c_str(),
                    shape_str(weight).c_str(), shape_str(normed_out).c_str());
    if (residual->dtype != FHIP_FP16 && residual->dtype != FHIP_BF16 &&
        residual->dtype != FHIP_FP32)
        return fail(FHIP_ERR_UNSUPPORTED_DTYPE, "add_rmsnorm %s",
                    dtype_name(residual->dtype));
    if (rows == 0) return FHIP_OK;
    set_device(b);
    return launch_result(fhip_launch_add_rmsnorm(ph, pd, pw, (float)eps, po, (int)rows, (int)cols,
                                                 residual->dtype, b->stream));
}

}  // extern "C"

namespace {

// fhip_rope / fhip_rope_dev: positions from host memory (staged through the pinned ring) or
// already on the device (dev_pos).
int rope_common(fhip_backend* b, const fhip_tensor* q, const fhip_tensor* k,
                const uint32_t* host_pos, const void* dev_pos, size_t num_positions,
                size_t head_dim) {
    CHECK_T(q);
    CHECK_T(k);
    GET_PTR(b, q, pq);
    WRITES(b, q);
    GET_PTR(b, k, pk);
    WRITES(b, k);
    if (!b->rope_freq)
        return fail(FHIP_ERR_BACKEND,
                    "RoPE frequency table not initialized. Call precompute_rope_freqs() first.");
    if (q->ndim < 2 || k->ndim < 2 || head_dim != 2 * b->rope_half)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "rope: q %s, k %s, head_dim %zu (table for %zu)",
                    shape_str(q).c_str(), shape_str(k).c_str(), head_dim, 2 * b->rope_half);
    const uint64_t qh = q->shape[1], kvh = k->shape[1];
    const uint64_t T = num_positions;
    if (numel(q) < T * qh * head_dim || numel(k) < T * kvh * head_dim || q->dtype != k->dtype)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "rope: %zu positions do not fit q %s / k %s",
                    num_positions, shape_str(q).c_str(), shape_str(k).c_str());
    if (q->dtype != FHIP_FP16 && q->dtype != FHIP_BF16 && q->dtype != FHIP_FP32)
        return fail(FHIP_ERR_UNSUPPORTED_DTYPE, "rope %s", dtype_name(q->dtype));
    if (T == 0) return FHIP_OK;
    if (!host_pos && !dev_pos) return fail(FHIP_ERR_INVALID_SHAPE, "null positions");
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    const void* dpos = dev_pos;
    int slot = -1;
    if (!dpos) {
        void* staged;
        int r = b->stage(host_pos, T * sizeof(uint32_t), &staged, &slot);
        if (r != FHIP_OK) return r;
        dpos = staged;
    }
    int e = fhip_launch_rope_ex(pq, pk, (const uint32_t*)dpos, b->rope_freq, (int)T, (int)qh,
                                (int)kvh, (int)head_dim, q->dtype, b->stream);
    int r = slot >= 0 ? b->stage_done(slot) : FHIP_OK;
    if (e != hipSuccess)
        return fail(FHIP_ERR_BACKEND, "RoPE kernel error: %s", hipGetErrorString((hipError_t)e));
    return r;
}

// fhip_embedding / fhip_embedding_dev: token ids from host memory or already on the device.
int embedding_common(fhip_backend* b, const uint32_t* host_ids, const void* dev_ids,
                     size_t num_tokens, const fhip_tensor* table, const fhip_tensor* out) {
    CHECK_T(table);
    CHECK_T(out);
    GET_PTR(b, table, pt);
    GET_PTR(b, out, po);
    WRITES(b, out);
    if (table->ndim != 2 || (dtype_size(table->dtype) != 2 && dtype_size(table->dtype) != 4))
        return fail(FHIP_ERR_INVALID_SHAPE, "embedding table %s",
                    shape_str(table).c_str());
    const uint64_t vocab = table->shape[0], hidden = table->shape[1];
    if (numel(out) < num_tokens * hidden || out->dtype != table->dtype)
        return fail(FHIP_ERR_INVALID_SHAPE, "embedding out %s for %zu tokens",
                    shape_str(out).c_str(), num_tokens);
    if (num_tokens == 0) return FHIP_OK;
    if (!host_ids && !dev_ids) return fail(FHIP_ERR_INVALID_SHAPE, "null token ids");
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    const void* dids = dev_ids;
    int slot = -1;
    if (!dids) {
        void* staged;
        int r = b->stage(host_ids, num_tokens * sizeof(uint32_t), &staged, &slot);
        if (r != FHIP_OK) return r;
        dids = staged;
    }
    int e = fhip_launch_embedding_ex(po, pt, (const uint32_t*)dids, (int)num_tokens, (int)hidden,
                                     (int)(vocab > 0x7fffffffull ? 0x7fffffff : vocab),
                                     (int)dtype_size(table->dtype), b->stream);
    int r = slot >= 0 ? b->stage_done(slot) : FHIP_OK;
    if (e != hipSuccess)
        return fail(FHIP_ERR_BACKEND, "embedding kernel error: %s", hipGetErrorString((hipError_t)e));
    return r;
}

// A u32 array of n values held by a backend tensor (any dtype: its bytes are read as uint32).
int u32_array(fhip_backend* b, const fhip_tensor* t, size_t n, const char* what, void** out) {
    CHECK_T(t);
    GET_PTR(b, t, p);
    if (size_bytes(t) < n * sizeof(uint32_t))
        return fail(FHIP_ERR_INVALID_SHAPE, "%s: tensor %s holds fewer than %zu uint32 values",
                    what, shape_str(t).c_str(), n);
    *out = p;
    return FHIP_OK;
}

}  // namespace

extern "C" {

int fhip_rope(fhip_backend* b, const fhip_tensor* q, const fhip_tensor* k,
              const uint32_t* positions, size_t num_positions, double theta, size_t head_dim) {
    (void)theta;  // the table from precompute_rope_freqs is used (backend.rs:166)
    CHECK_B(b);
    NO_CAPTURE(b, "rope (host positions; use fhip_rope_dev)");
    if (num_positions && !positions) return fail(FHIP_ERR_INVALID_SHAPE, "null positions");
    return rope_common(b, q, k, positions, nullptr, num_positions, head_dim);
}

int fhip_rope_dev(fhip_backend* b, const fhip_tensor* q, const fhip_tensor* k,
                  const fhip_tensor* positions, size_t num_positions, size_t head_dim) {
    CHECK_B(b);
    if (num_positions == 0) return rope_common(b, q, k, nullptr, nullptr, 0, head_dim);
    void* dp;
    int r = u32_array(b, positions, num_positions, "rope positions", &dp);
    if (r) return r;
    return rope_common(b, q, k, nullptr, dp, num_positions, head_dim);
}

// Backend::attention (backend.rs:54-62) over contiguous K / V caches: not supported, as the
// optional paged methods are on backends without them (backend.rs:74-88); the engine's caches are
// paged.
int fhip_attention(fhip_backend* b, const fhip_tensor* q, const fhip_tensor* k_cache,
                   const fhip_tensor* v_cache, size_t num_kv_heads, size_t start_pos,
                   const fhip_tensor* out) {
    (void)q, (void)k_cache, (void)v_cache, (void)num_kv_heads, (void)start_pos, (void)out;
    CHECK_B(b);
    return fail(FHIP_ERR_BACKEND, "attention (contiguous KV cache) not supported by this backend");
}

int fhip_silu_mul(fhip_backend* b, const fhip_tensor* gate, const fhip_tensor* up,
                  const fhip_tensor* out) {
    CHECK_B(b);
    CHECK_T(gate);
    CHECK_T(up);
    CHECK_T(out);
    if (!same_shape(gate, up))
        return fail(FHIP_ERR_INVALID_SHAPE, "silu_mul: gate shape %s != up shape %s",
                    shape_str(gate).c_str(), shape_str(up).c_str());
    GET_PTR(b, gate, pg);
    GET_PTR(b, up, pu);
    GET_PTR(b, out, po);
    WRITES(b, out);
    if (numel(out) < numel(gate) || up->dtype != gate->dtype || out->dtype != gate->dtype)
        return fail(FHIP_ERR_INVALID_SHAPE, "silu_mul: out %s too small",
                    shape_str(out).c_str());
    set_device(b);
    return launch_result(
        fhip_launch_silu_mul_ex(po, pg, pu, (int64_t)numel(gate), gate->dtype, b->stream));
}

int fhip_add(fhip_backend* b, const fhip_tensor* a, const fhip_tensor* bt, const fhip_tensor* out) {
    CHECK_B(b);
    CHECK_T(a);
    CHECK_T(bt);
    CHECK_T(out);
    if (!same_shape(a, bt))
        return fail(FHIP_ERR_INVALID_SHAPE, "add: a shape %s != b shape %s",
                    shape_str(a).c_str(), shape_str(bt).c_str());
    GET_PTR(b, a, pa);
    GET_PTR(b, bt, pb);
    GET_PTR(b, out, po);
    WRITES(b, out);
    if (numel(out) < numel(a) || bt->dtype != a->dtype || out->dtype != a->dtype)
        return fail(FHIP_ERR_INVALID_SHAPE, "add: out %s too small",
                    shape_str(out).c_str());
    set_device(b);
    return launch_result(fhip_launch_add_ex(po, pa, pb, (int64_t)numel(a), a->dtype, b->stream));
}

int fhip_embedding(fhip_backend* b, const uint32_t* token_ids, size_t num_tokens,
                   const fhip_tensor* table, const fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "embedding (host token ids; use fhip_embedding_dev)");
    if (num_tokens && !token_ids) return fail(FHIP_ERR_INVALID_SHAPE, "null token ids");
    return embedding_common(b, token_ids, nullptr, num_tokens, table, out);
}

int fhip_embedding_dev(fhip_backend* b, const fhip_tensor* token_ids, size_t num_tokens,
                       const fhip_tensor* table, const fhip_tensor* out) {
    CHECK_B(b);
    if (num_tokens == 0) return embedding_common(b, nullptr, nullptr, 0, table, out);
    void* dp;
    int r = u32_array(b, token_ids, num_tokens, "embedding token ids", &dp);
    if (r) return r;
    return embedding_common(b, nullptr, dp, num_tokens, table, out);
}

// Graph capture of the backend's launches (a decode step's elementwise chain, recorded once
// and replayed per step instead of launched kernel by kernel).
int fhip_graph_begin(fhip_backend* b) {
    CHECK_B(b);
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    if (b->capturing) return fail(FHIP_ERR_BACKEND, "graph capture already in progress");
    {
        std::lock_guard<std::mutex> g2(b->mu);
        b->capture_ids.clear();
    }
    HIP_TRY(hipStreamBeginCapture(b->stream, hipStreamCaptureModeThreadLocal));
    b->capturing = true;
    return FHIP_OK;
}

int fhip_graph_end(fhip_backend* b, uint64_t* graph_out) {
    CHECK_B(b);
    if (!graph_out) return fail(FHIP_ERR_BACKEND, "null graph output");
    *graph_out = 0;
    set_device(b);
    hipGraph_t graph = nullptr;
    std::vector<uint64_t> ids;
    {
        std::lock_guard<std::mutex> g(b->launch_mu);
        if (!b->capturing) return fail(FHIP_ERR_BACKEND, "no graph capture in progress");
        b->capturing = false;
        {
            std::lock_guard<std::mutex> g2(b->mu);
            ids.assign(b->capture_ids.begin(), b->capture_ids.end());
            b->capture_ids.clear();
        }
        hipError_t e = hipStreamEndCapture(b->stream, &graph);
        if (e != hipSuccess) {
            if (graph) (void)hipGraphDestroy(graph);
            return hip_fail(e);
        }
    }
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e);
    std::lock_guard<std::mutex> g(b->mu);
    const uint64_t id = b->next_graph++;
    for (uint64_t t : ids) ++b->graph_refs[t];
    b->graphs[id] = fhip_backend::GraphRec{exec, std::move(ids)};
    *graph_out = id;
    return FHIP_OK;
}

int fhip_graph_launch(fhip_backend* b, uint64_t graph) {
    CHECK_B(b);
    NO_CAPTURE(b, "graph_launch");
    hipGraphExec_t exec;
    {
        std::lock_guard<std::mutex> g(b->mu);
        auto it = b->graphs.find(graph);
        if (it == b->graphs.end())
            return fail(FHIP_ERR_BACKEND, "graph %llu not found", (unsigned long long)graph);
        exec = it->second.exec;
    }
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    HIP_TRY(hipGraphLaunch(exec, b->stream));
    return FHIP_OK;
}

int fhip_graph_destroy(fhip_backend* b, uint64_t graph) {
    CHECK_B(b);
    NO_CAPTURE(b, "graph_destroy");
    hipGraphExec_t exec;
    {
        std::lock_guard<std::mutex> g(b->mu);
        auto it = b->graphs.find(graph);
        if (it == b->graphs.end())
            return fail(FHIP_ERR_BACKEND, "graph %llu not found", (unsigned long long)graph);
        exec = it->second.exec;
        for (uint64_t t : it->second.ids)
            if (--b->graph_refs[t] == 0) b->graph_refs.erase(t);
        b->graphs.erase(it);
    }
    set_device(b);
    HIP_TRY(hipStreamSynchronize(b->stream));  // replays queued on the stream finish first
    HIP_TRY(hipGraphExecDestroy(exec));
    return FHIP_OK;
}

int fhip_copy_rows(fhip_backend* b, const fhip_tensor* src, const fhip_tensor* dst,
                   size_t src_offset, size_t dst_offset, size_t count) {
    CHECK_B(b);
    CHECK_T(src);
    CHECK_T(dst);
    if (src->ndim < 1 || dst->ndim < 1)
        return fail(FHIP_ERR_INVALID_SHAPE, "copy_rows needs >= 1-D tensors");
    if (src_offset + count > src->shape[0])
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "copy_rows: src_offset(%zu) + count(%zu) = %zu exceeds src rows(%llu)",
                    src_offset, count, src_offset + count, (unsigned long long)src->shape[0]);
    if (dst_offset + count > dst->shape[0])
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "copy_rows: dst_offset(%zu) + count(%zu) = %zu exceeds dst rows(%llu)",
                    dst_offset, count, dst_offset + count, (unsigned long long)dst->shape[0]);
    bool tail_eq = src->ndim == dst->ndim;
    for (int i = 1; tail_eq && i < src->ndim; ++i) tail_eq = src->shape[i] == dst->shape[i];
    if (!tail_eq)
        return fail(FHIP_ERR_INVALID_SHAPE, "copy_rows: src column shape != dst column shape (%s vs %s)",
                    shape_str(src).c_str(), shape_str(dst).c_str());
    if (src->dtype != dst->dtype)
        return fail(FHIP_ERR_INVALID_SHAPE, "copy_rows: src dtype %s != dst dtype %s",
                    dtype_name(src->dtype), dtype_name(dst->dtype));
    GET_PTR(b, src, ps);
    GET_PTR(b, dst, pdst);
    uint64_t row_elems = 1;
    for (int i = 1; i < src->ndim; ++i) row_elems *= src->shape[i];
    const uint64_t row = row_elems * dtype_size(src->dtype);
    if (count == 0 || row == 0) return FHIP_OK;
    set_device(b);
    WRITES(b, dst);
    HIP_TRY(hipMemcpyAsync((char*)pdst + dst_offset * row, (const char*)ps + src_offset * row,
                           count * row, hipMemcpyDeviceToDevice, b->stream));
    return FHIP_OK;
}

const char* fhip_device_name(fhip_backend* b) { return b ? b->name.c_str() : ""; }
size_t fhip_total_memory(fhip_backend* b) { return b ? b->total_mem : 0; }
size_t fhip_available_memory(fhip_backend* b) {
    if (!b) return 0;
    (void)hipSetDevice(b->device);
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return 0;
    return free_b;
}

int fhip_synchronize(fhip_backend* b) {
    CHECK_B(b);
    NO_CAPTURE(b, "synchronize");
    set_device(b);
    HIP_TRY(hipStreamSynchronize(b->stream));
    return FHIP_OK;
}

int fhip_create_timer(fhip_backend* b, uint64_t* timer_id) {
    CHECK_B(b);
    NO_CAPTURE(b, "create_timer");
    if (!timer_id) return fail(FHIP_ERR_BACKEND, "null timer id");
    set_device(b);
    hipEvent_t s, e;
    HIP_TRY(hipEventCreate(&s));
    hipError_t r = hipEventCreate(&e);
    if (r != hipSuccess) {
        (void)hipEventDestroy(s);
        return hip_fail(r);
    }
    std::lock_guard<std::mutex> g(b->mu);
    *timer_id = b->next_timer++;
    b->timers[*timer_id] = {s, e};
    return FHIP_OK;
}

static int find_timer(fhip_backend* b, uint64_t id, hipEvent_t* s, hipEvent_t* e) {
    std::lock_guard<std::mutex> g(b->mu);
    auto it = b->timers.find(id);
    if (it == b->timers.end()) return fail(FHIP_ERR_BACKEND, "timer %llu not found", (unsigned long long)id);
    *s = it->second.first;
    *e = it->second.second;
    return FHIP_OK;
}

int fhip_start_timer(fhip_backend* b, uint64_t timer_id) {
    CHECK_B(b);
    NO_CAPTURE(b, "start_timer");
    hipEvent_t s, e;
    int r = find_timer(b, timer_id, &s, &e);
    if (r) return r;
    HIP_TRY(hipEventRecord(s, b->stream));
    return FHIP_OK;
}

int fhip_stop_timer(fhip_backend* b, uint64_t timer_id, float* ms_out) {
    CHECK_B(b);
    NO_CAPTURE(b, "stop_timer");
    hipEvent_t s, e;
    int r = find_timer(b, timer_id, &s, &e);
    if (r) return r;
    HIP_TRY(hipEventRecord(e, b->stream));
    HIP_TRY(hipEventSynchronize(e));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, s, e));
    if (ms_out) *ms_out = ms;
    return FHIP_OK;
}

int fhip_destroy_timer(fhip_backend* b, uint64_t timer_id) {
    CHECK_B(b);
    NO_CAPTURE(b, "destroy_timer");
    std::pair<hipEvent_t, hipEvent_t> ev;
    {
        std::lock_guard<std::mutex> g(b->mu);
        auto it = b->timers.find(timer_id);
        if (it == b->timers.end())
            return fail(FHIP_ERR_BACKEND, "timer %llu not found", (unsigned long long)timer_id);
        ev = it->second;
        b->timers.erase(it);
    }
    (void)hipEventDestroy(ev.first);
    (void)hipEventDestroy(ev.second);
    return FHIP_OK;
}

void fhip_marker_push(fhip_backend* b, const char* name) {
    (void)b;
    g_roctx.load();
    if (g_roctx.push && name) g_roctx.push(name);
}

void fhip_marker_pop(fhip_backend* b) {
    (void)b;
    g_roctx.load();
    if (g_roctx.pop) g_roctx.pop();
}

int fhip_turboquant_compress(fhip_backend* b, const fhip_tensor* input, const fhip_tensor* rotation,
                             const fhip_tensor* centroids, uint8_t bits,
                             const fhip_tensor* packed_out, const fhip_tensor* norms_out) {
    CHECK_B(b);
    NO_CAPTURE(b, "turboquant_compress");
    CHECK_T(input);
    CHECK_T(rotation);
    CHECK_T(centroids);
    CHECK_T(packed_out);
    CHECK_T(norms_out);
    GET_PTR(b, input, pin);
    GET_PTR(b, rotation, prot);
    GET_PTR(b, centroids, pc);
    GET_PTR(b, packed_out, pp);
    WRITES(b, packed_out);
    GET_PTR(b, norms_out, pn);
    WRITES(b, norms_out);
    if (input->ndim != 3 || input->dtype != FHIP_FP16)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "turboquant_compress input must be [N, kv_heads, head_dim] FP16, got %s %s",
                    shape_str(input).c_str(), dtype_name(input->dtype));
    const uint64_t N = input->shape[0], H = input->shape[1], hd = input->shape[2];
    const uint64_t L = numel(centroids);
    if (bits < 1 || bits > 8 || L < 1 || L > (1ull << bits) || centroids->dtype != FHIP_FP32)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "turboquant_compress: %llu centroids for %u bits",
                    (unsigned long long)L, (unsigned)bits);
    const uint64_t pd = fhip_tq_packed_dim_per_head(hd, bits);
    if (numel(rotation) != hd * hd || rotation->dtype != FHIP_FP32 ||
        size_bytes(packed_out) < N * H * pd || numel(norms_out) < N * H ||
        norms_out->dtype != FHIP_FP16)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "turboquant_compress: rotation %s, packed %s, norms %s",
                    shape_str(rotation).c_str(), shape_str(packed_out).c_str(),
                    shape_str(norms_out).c_str());
    set_device(b);
    std::lock_guard<std::mutex> g(b->plan_mu);
    if (fhip_tq_plan* plan = b->plan_for(rotation->id, prot, centroids->id, pc, (int)L, bits, (int)hd))
        return launch_result(fhip_launch_tq_compress_planned(plan, pin, pp, pn, (int)N, (int)H,
                                                             b->stream));
    return launch_result(fhip_launch_turboquant_compress(pin, (const float*)prot, (const float*)pc,
                                                         pp, pn, (int)N, (int)H, (int)hd, (int)L,
                                                         bits, (int)pd, b->stream));
}

int fhip_tq_quantize_pack(fhip_backend* b, const fhip_tensor* y, const fhip_tensor* centroids,
                          uint8_t bits, const fhip_tensor* packed_out) {
    CHECK_B(b);
    NO_CAPTURE(b, "tq_quantize_pack");
    CHECK_T(y);
    CHECK_T(centroids);
    CHECK_T(packed_out);
    GET_PTR(b, y, py);
    GET_PTR(b, centroids, pc);
    GET_PTR(b, packed_out, pp);
    WRITES(b, packed_out);
    if (y->ndim < 1 || y->dtype != FHIP_FP32)
        return fail(FHIP_ERR_INVALID_SHAPE, "tq_quantize_pack y %s",
                    shape_str(y).c_str());
    const uint64_t hd = y->shape[y->ndim - 1];
    const uint64_t rows = hd ? numel(y) / hd : 0;
    const uint64_t L = numel(centroids);
    if (bits < 1 || bits > 8 || L < 1 || L > (1ull << bits) || centroids->dtype != FHIP_FP32)
        return fail(FHIP_ERR_INVALID_SHAPE, "%llu centroids for %u bits",
                    (unsigned long long)L, (unsigned)bits);
    const uint64_t pd = fhip_tq_packed_dim_per_head(hd, bits);
    if (size_bytes(packed_out) < rows * pd)
        return fail(FHIP_ERR_INVALID_SHAPE, "packed %s too small",
                    shape_str(packed_out).c_str());
    set_device(b);
    return launch_result(fhip_launch_tq_quantize_pack((const float*)py, (const float*)pc, (int)L,
                                                      bits, pp, (int)rows, (int)hd, (int)pd,
                                                      b->stream));
}

int fhip_tq_dequantize(fhip_backend* b, const fhip_tensor* packed, const fhip_tensor* norms,
                       const fhip_tensor* rotation, const fhip_tensor* centroids, uint8_t bits,
                       const fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "tq_dequantize");
    CHECK_T(packed);
    CHECK_T(norms);
    CHECK_T(rotation);
    CHECK_T(centroids);
    CHECK_T(out);
    GET_PTR(b, packed, pp);
    GET_PTR(b, norms, pn);
    GET_PTR(b, rotation, prot);
    GET_PTR(b, centroids, pc);
    GET_PTR(b, out, po);
    WRITES(b, out);
    if (out->ndim != 3 || out->dtype != FHIP_FP16)
        return fail(FHIP_ERR_INVALID_SHAPE, "dequantize out must be [N, kv_heads, head_dim] FP16");
    const uint64_t N = out->shape[0], H = out->shape[1], hd = out->shape[2];
    const uint64_t L = numel(centroids);
    if (bits < 1 || bits > 8 || L < 1 || L > (1ull << bits) || centroids->dtype != FHIP_FP32)
        return fail(FHIP_ERR_INVALID_SHAPE, "%llu centroids for %u bits",
                    (unsigned long long)L, (unsigned)bits);
    const uint64_t pd = fhip_tq_packed_dim_per_head(hd, bits);
    if (size_bytes(packed) < N * H * pd || numel(norms) < N * H || norms->dtype != FHIP_FP16 ||
        numel(rotation) != hd * hd || rotation->dtype != FHIP_FP32)
        return fail(FHIP_ERR_INVALID_SHAPE, "dequantize packed %s norms %s",
                    shape_str(packed).c_str(), shape_str(norms).c_str());
    set_device(b);
    std::lock_guard<std::mutex> g(b->plan_mu);
    if (fhip_tq_plan* plan = b->plan_for(rotation->id, prot, centroids->id, pc, (int)L, bits, (int)hd))
        return launch_result(fhip_launch_tq_dequant_planned(plan, pp, pn, po, (int)N, (int)H,
                                                            b->stream));
    return launch_result(fhip_launch_tq_dequant(pp, pn, (const float*)prot, (const float*)pc,
                                                (int)L, po, (int)N, (int)H, (int)hd, bits,
                                                (int)pd, b->stream));
}

int fhip_softmax_rows(fhip_backend* b, const fhip_tensor* logits, float temperature,
                      const fhip_tensor* probs) {
    CHECK_B(b);
    NO_CAPTURE(b, "softmax_rows");
    CHECK_T(logits);
    CHECK_T(probs);
    GET_PTR(b, logits, pl);
    GET_PTR(b, probs, pp);
    WRITES(b, probs);
    if (logits->ndim < 1 || logits->dtype != FHIP_FP32 || probs->dtype != FHIP_FP32 ||
        numel(probs) != numel(logits))
        return fail(FHIP_ERR_INVALID_SHAPE, "softmax logits %s probs %s",
                    shape_str(logits).c_str(), shape_str(probs).c_str());
    const uint64_t cols = logits->shape[logits->ndim - 1];
    if (cols == 0) return fail(FHIP_ERR_GENERATION, "empty logits");
    const uint64_t rows = numel(logits) / cols;
    if (rows == 0) return FHIP_OK;
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    void* ws;
    int r = b->get_workspace(fhip_rows_workspace_bytes((int)rows, (int)cols), &ws);
    if (r) return r;
    int e = fhip_launch_softmax_rows((const float*)pl, (float*)pp, (int)rows, (int)cols,
                                     temperature, ws, b->stream);
    if (e != hipSuccess) return hip_fail((hipError_t)e);
    return FHIP_OK;
}

int fhip_argmax_rows(fhip_backend* b, const fhip_tensor* logits, uint32_t* tokens_out,
                     size_t rows_out) {
    CHECK_B(b);
    NO_CAPTURE(b, "argmax_rows");
    CHECK_T(logits);
    GET_PTR(b, logits, pl);
    if (logits->ndim < 1 || logits->dtype != FHIP_FP32)
        return fail(FHIP_ERR_INVALID_SHAPE, "argmax logits %s",
                    shape_str(logits).c_str());
    const uint64_t cols = logits->shape[logits->ndim - 1];
    if (cols == 0) return fail(FHIP_ERR_GENERATION, "empty logits");
    const uint64_t rows = numel(logits) / cols;
    if (rows_out < rows || (rows && !tokens_out))
        return fail(FHIP_ERR_INVALID_SHAPE, "%zu outputs for %llu rows",
                    rows_out, (unsigned long long)rows);
    if (rows == 0) return FHIP_OK;
    set_device(b);
    std::vector<int32_t> idx(rows);
    std::vector<uint32_t> flags(rows);
    {
        std::lock_guard<std::mutex> g(b->launch_mu);
        const size_t part = fhip_rows_workspace_bytes((int)rows, (int)cols);
        const size_t off = (part + 255) & ~(size_t)255;
        void* ws;
        int r = b->get_workspace(off + rows * 8, &ws);
        if (r) return r;
        int32_t* didx = (int32_t*)((char*)ws + off);
        uint32_t* dfl = (uint32_t*)(didx + rows);
        int e = fhip_launch_argmax_rows((const float*)pl, didx, dfl, (int)rows, (int)cols, ws,
                                        b->stream);
        if (e != hipSuccess) return hip_fail((hipError_t)e);
        HIP_TRY(hipMemcpyAsync(idx.data(), didx, rows * 4, hipMemcpyDeviceToHost, b->stream));
        HIP_TRY(hipMemcpyAsync(flags.data(), dfl, rows * 4, hipMemcpyDeviceToHost, b->stream));
        HIP_TRY(hipStreamSynchronize(b->stream));
    }
    // The sampler rejects any NaN first, then any infinity (sampling.rs:51-56).
    for (uint64_t r = 0; r < rows; ++r)
        if (flags[r] & FHIP_ROW_HAS_NAN) return fail(FHIP_ERR_GENERATION, "NaN in logits");
    for (uint64_t r = 0; r < rows; ++r)
        if (flags[r] & FHIP_ROW_HAS_INF) return fail(FHIP_ERR_GENERATION, "Inf in logits");
    for (uint64_t r = 0; r < rows; ++r) tokens_out[r] = (uint32_t)idx[r];
    return FHIP_OK;
}

int fhip_attention_paged_tq(fhip_backend* b, const fhip_tensor* q, const int32_t* block_table,
                            size_t num_blocks, const fhip_tensor* k_packed,
                            const fhip_tensor* k_norms, const fhip_tensor* v_packed,
                            const fhip_tensor* v_norms, size_t pool_len,
                            const fhip_tensor* k_rotation, const fhip_tensor* v_rotation,
                            const fhip_tensor* k_centroids, const fhip_tensor* v_centroids,
                            uint8_t key_bits, uint8_t value_bits, size_t num_kv_heads,
                            size_t kv_len, size_t start_pos, const fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "attention_paged_tq");
    CHECK_T(q);
    CHECK_T(k_rotation);
    CHECK_T(v_rotation);
    CHECK_T(k_centroids);
    CHECK_T(v_centroids);
    CHECK_T(out);
    GET_PTR(b, q, pq);
    GET_PTR(b, out, po);
    WRITES(b, out);
    GET_PTR(b, k_rotation, pkr);
    GET_PTR(b, v_rotation, pvr);
    GET_PTR(b, k_centroids, pkc);
    GET_PTR(b, v_centroids, pvc);
    if (q->ndim != 3 || q->dtype != FHIP_FP16 || out->dtype != FHIP_FP16 ||
        numel(out) != numel(q))
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq q %s out %s",
                    shape_str(q).c_str(), shape_str(out).c_str());
    const uint64_t T = q->shape[0], qh = q->shape[1], hd = q->shape[2];
    if (num_kv_heads == 0 || qh % num_kv_heads != 0 || key_bits < 1 || key_bits > 8 ||
        value_bits < 1 || value_bits > 8 || numel(k_rotation) != hd * hd ||
        numel(v_rotation) != hd * hd || numel(k_centroids) < (1ull << key_bits) ||
        numel(v_centroids) < (1ull << value_bits))
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq arguments");
    const uint64_t needed_blocks = (kv_len + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
    if (num_blocks < needed_blocks)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "block table has %zu blocks for kv_len %zu", num_blocks,
                    kv_len);
    const uint64_t kpd = fhip_tq_packed_dim_per_head(hd, key_bits);
    const uint64_t vpd = fhip_tq_packed_dim_per_head(hd, value_bits);
    // Resolve the per-block tensors the table uses (all pool entries, as the reference does).
    std::vector<const void*> ptrs(4 * pool_len > 0 ? 4 * pool_len : 1, nullptr);
    for (size_t i = 0; i < pool_len; ++i) {
        const fhip_tensor* ts[4] = {&k_packed[i], &k_norms[i], &v_packed[i], &v_norms[i]};
        const uint64_t need[4] = {FHIP_PAGE_TOKENS * num_kv_heads * kpd,
                                  FHIP_PAGE_TOKENS * num_kv_heads * 2,
                                  FHIP_PAGE_TOKENS * num_kv_heads * vpd,
                                  FHIP_PAGE_TOKENS * num_kv_heads * 2};
        for (int k = 0; k < 4; ++k) {
            void* p;
            int r = b->get_ptr(ts[k]->id, &p);
            if (r) return r;
            if (size_bytes(ts[k]) < need[k])
                return fail(FHIP_ERR_INVALID_SHAPE, "page tensor %s too small",
                            shape_str(ts[k]).c_str());
            ptrs[(size_t)k * pool_len + i] = p;
        }
    }
    for (uint64_t i = 0; i < needed_blocks; ++i)
        if (block_table[i] < 0 || (uint64_t)block_table[i] >= pool_len)
            return fail(FHIP_ERR_INVALID_SHAPE, "block id %d outside the pool of %zu",
                        block_table[i], pool_len);
    if (T == 0) return FHIP_OK;
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    void *dbt, *dptr;
    int s1, s2;
    int r = b->stage(block_table, (needed_blocks ? needed_blocks : 1) * sizeof(int32_t), &dbt, &s1);
    if (r) return r;
    r = b->stage(ptrs.data(), ptrs.size() * sizeof(void*), &dptr, &s2);
    if (r) return r;
    const size_t wsb = fhip_attention_tq_workspace_bytes(
        (int)T, (int)qh, (int)hd, needed_blocks ? (int)needed_blocks : 1);
    void* ws;
    r = b->get_workspace(wsb, &ws);
    if (r) return r;
    const void** dp = (const void**)dptr;
    int e = fhip_launch_attention_paged_tq_ws(
        po, pq, (const int*)dbt, dp, dp + pool_len, dp + 2 * pool_len, dp + 3 * pool_len,
        (const float*)pkr, (const float*)pvr, (const float*)pkc, (const float*)pvc, (int)T, (int)qh,
        (int)num_kv_heads, (int)hd, (int)kv_len, (int)start_pos, key_bits, value_bits, (int)kpd,
        (int)vpd, ws, wsb, b->stream);
    b->stage_done(s1);
    b->stage_done(s2);
    if (e != hipSuccess) return hip_fail((hipError_t)e);
    return FHIP_OK;
}

// ---------------------------------------------------------------------------------------
// Registered page pools. The cache managers allocate their block pools once
// (paged_kv_cache.rs, quantized_paged_kv_cache.rs:82-133) and hand every attention call the
// whole pool's tensor lists; the reference copies pool_len pointers to a fresh device
// allocation on every call (cuda/src/backend.rs:295-315, 625-671). A registered pool keeps
// those addresses in device memory, so a call stages only its block table. The pool's
// tensors cannot be freed until the pool is destroyed (fhip_free refuses them).
// ---------------------------------------------------------------------------------------
int fhip_page_pool_create(fhip_backend* b, const fhip_tensor* blocks, size_t nlists,
                          size_t pool_len, uint64_t* pool_out) {
    CHECK_B(b);
    NO_CAPTURE(b, "page_pool_create");
    if (!pool_out || nlists == 0 || nlists > 8 || pool_len == 0 || !blocks)
        return fail(FHIP_ERR_INVALID_SHAPE, "page pool: %zu lists of %zu blocks", nlists,
                    pool_len);
    *pool_out = 0;
    fhip_backend::PagePool pp;
    pp.pool_len = pool_len;
    pp.nlists = (int)nlists;
    pp.min_bytes.assign(nlists, UINT64_MAX);
    pp.dtype.assign(nlists, -2);
    std::vector<const void*> ptrs(nlists * pool_len);
    for (size_t l = 0; l < nlists; ++l)
        for (size_t i = 0; i < pool_len; ++i) {
            const fhip_tensor* t = &blocks[l * pool_len + i];
            void* p;
            int r = b->get_ptr(t->id, &p);
            if (r) return r;
            ptrs[l * pool_len + i] = p;
            pp.ids.push_back(t->id);
            pp.min_bytes[l] = std::min<uint64_t>(pp.min_bytes[l], size_bytes(t));
            pp.dtype[l] = pp.dtype[l] == -2 || pp.dtype[l] == t->dtype ? t->dtype : -1;
        }
    set_device(b);
    void* dev = nullptr;
    HIP_TRY(hipMalloc(&dev, ptrs.size() * sizeof(void*)));
    hipError_t e = hipMemcpy(dev, ptrs.data(), ptrs.size() * sizeof(void*),
                             hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e);
    }
    pp.dev = (const void**)dev;
    const std::vector<uint64_t> ids = pp.ids;
    {
        std::lock_guard<std::mutex> g(b->mu);
        for (uint64_t tid : pp.ids) {
            if (!b->tensors.count(tid)) {  // freed while the pool was being built
                (void)hipFree(dev);
                return fail(FHIP_ERR_TENSOR_NOT_FOUND, "tensor id %llu", (unsigned long long)tid);
            }
        }
        for (uint64_t tid : pp.ids) ++b->pooled[tid];
        const uint64_t id = b->next_pool++;
        b->pools.emplace(id, std::move(pp));
        *pool_out = id;
    }
    // the pool's writers do not look for plans: none may be built from its tensors
    for (uint64_t tid : ids) (void)b->drop_plans(tid);
    return FHIP_OK;
}

int fhip_page_pool_destroy(fhip_backend* b, uint64_t pool) {
    CHECK_B(b);
    NO_CAPTURE(b, "page_pool_destroy");
    const void** dev = nullptr;
    {
        std::lock_guard<std::mutex> g(b->mu);
        auto it = b->pools.find(pool);
        if (it == b->pools.end())
            return fail(FHIP_ERR_TENSOR_NOT_FOUND, "page pool %llu", (unsigned long long)pool);
        dev = it->second.dev;
        for (uint64_t tid : it->second.ids)
            if (--b->pooled[tid] == 0) b->pooled.erase(tid);
        b->pools.erase(it);
    }
    set_device(b);
    // calls already enqueued may still read the addresses
    HIP_TRY(hipStreamSynchronize(b->stream));
    HIP_TRY(hipFree((void*)dev));
    return FHIP_OK;
}

// The pool with `nlists` lists whose list l holds blocks of at least need[l] bytes of dtype
// dt[l] (dt -1: any), or an error.
// What a launch over a pool needs: the device address table and the pool length (copying the
// whole PagePool would copy its id list, nlists * pool_len entries, on every call).
struct PoolView {
    const void** dev = nullptr;
    size_t pool_len = 0;
};

static int find_pool(fhip_backend* b, uint64_t pool, int nlists, const uint64_t* need,
                     const int32_t* dt, PoolView* out) {
    std::lock_guard<std::mutex> g(b->mu);
    auto it = b->pools.find(pool);
    if (it == b->pools.end())
        return fail(FHIP_ERR_TENSOR_NOT_FOUND, "page pool %llu", (unsigned long long)pool);
    const auto& pp = it->second;
    if (pp.nlists != nlists)
        return fail(FHIP_ERR_INVALID_SHAPE, "page pool %llu has %d block lists, need %d",
                    (unsigned long long)pool, pp.nlists, nlists);
    for (int l = 0; l < nlists; ++l) {
        if (pp.min_bytes[l] < need[l])
            return fail(FHIP_ERR_INVALID_SHAPE,
                        "page pool list %d: blocks of %llu bytes, need %llu", l,
                        (unsigned long long)pp.min_bytes[l], (unsigned long long)need[l]);
        if (dt[l] >= 0 && pp.dtype[l] != dt[l])
            return fail(FHIP_ERR_INVALID_SHAPE, "page pool list %d: dtype %s", l,
                        dtype_name(pp.dtype[l] >= 0 ? pp.dtype[l] : -1));
    }
    out->dev = pp.dev;
    out->pool_len = pp.pool_len;
    return FHIP_OK;
}

// Backend::attention_paged over a registered pool of (K blocks, V blocks).
int fhip_attention_paged_pool(fhip_backend* b, const fhip_tensor* q, const int32_t* block_table,
                              size_t num_blocks, uint64_t pool, size_t num_kv_heads,
                              size_t kv_len, size_t start_pos, const fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "attention_paged_pool");
    CHECK_T(q);
    CHECK_T(out);
    GET_PTR(b, q, pq);
    GET_PTR(b, out, po);
    WRITES(b, out);
    if (q->ndim != 3 || q->dtype != FHIP_FP16 || out->dtype != FHIP_FP16 ||
        numel(out) != numel(q))
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged q %s out %s",
                    shape_str(q).c_str(), shape_str(out).c_str());
    const uint64_t T = q->shape[0], qh = q->shape[1], hd = q->shape[2];
    if (num_kv_heads == 0 || qh % num_kv_heads != 0 ||
        hd == 0 || hd > 256)
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged: %zu q heads, %zu kv heads, "
                    "head_dim %zu (1 to 256)", (size_t)qh, num_kv_heads, (size_t)hd);
    if (kv_len > 0x7fffffffu || start_pos > 0x7fffffffu || T > 0x7fffffffu)
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged: sizes beyond int32");
    const uint64_t needed_blocks = (kv_len + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
    if (num_blocks < needed_blocks)
        return fail(FHIP_ERR_INVALID_SHAPE, "block table has %zu blocks for kv_len %zu",
                    num_blocks, kv_len);
    const uint64_t need = FHIP_PAGE_TOKENS * num_kv_heads * hd * 2;
    const uint64_t needs[2] = {need, need};
    const int32_t dts[2] = {FHIP_FP16, FHIP_FP16};
    PoolView pp;
    int r = find_pool(b, pool, 2, needs, dts, &pp);
    if (r) return r;
    for (uint64_t i = 0; i < needed_blocks; ++i)
        if (block_table[i] < 0 || (uint64_t)block_table[i] >= pp.pool_len)
            return fail(FHIP_ERR_INVALID_SHAPE, "block id %d outside the pool of %zu",
                        block_table[i], pp.pool_len);
    if (T == 0) return FHIP_OK;
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    void* dbt;
    int s1;
    r = b->stage(block_table, (needed_blocks ? needed_blocks : 1) * sizeof(int32_t), &dbt, &s1);
    if (r) return r;
    const size_t wsb = fhip_attention_paged_workspace_bytes(
        (int)T, (int)qh, (int)hd, needed_blocks ? (int)needed_blocks : 1);
    void* ws;
    r = b->get_workspace(wsb, &ws);
    if (r) return r;
    int e = fhip_launch_paged_attention_ws(po, pq, (const int*)dbt, pp.dev,
                                           pp.dev + pp.pool_len, (int)T, (int)qh,
                                           (int)num_kv_heads, (int)hd, (int)kv_len,
                                           (int)start_pos, (int)needed_blocks, ws, wsb,
                                           b->stream);
    b->stage_done(s1);
    if (e != hipSuccess) return hip_fail((hipError_t)e);
    return FHIP_OK;
}

// Backend::attention_paged_tq over a registered pool of (K packed, K norms, V packed, V norms).
int fhip_attention_paged_tq_pool(fhip_backend* b, const fhip_tensor* q,
                                 const int32_t* block_table, size_t num_blocks, uint64_t pool,
                                 const fhip_tensor* k_rotation, const fhip_tensor* v_rotation,
                                 const fhip_tensor* k_centroids, const fhip_tensor* v_centroids,
                                 uint8_t key_bits, uint8_t value_bits, size_t num_kv_heads,
                                 size_t kv_len, size_t start_pos, const fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "attention_paged_tq_pool");
    CHECK_T(q);
    CHECK_T(k_rotation);
    CHECK_T(v_rotation);
    CHECK_T(k_centroids);
    CHECK_T(v_centroids);
    CHECK_T(out);
    GET_PTR(b, q, pq);
    GET_PTR(b, out, po);
    WRITES(b, out);
    GET_PTR(b, k_rotation, pkr);
    GET_PTR(b, v_rotation, pvr);
    GET_PTR(b, k_centroids, pkc);
    GET_PTR(b, v_centroids, pvc);
    if (q->ndim != 3 || q->dtype != FHIP_FP16 || out->dtype != FHIP_FP16 ||
        numel(out) != numel(q))
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq q %s out %s",
                    shape_str(q).c_str(), shape_str(out).c_str());
    const uint64_t T = q->shape[0], qh = q->shape[1], hd = q->shape[2];
    if (num_kv_heads == 0 || qh % num_kv_heads != 0 || key_bits < 1 || key_bits > 8 ||
        value_bits < 1 || value_bits > 8 || numel(k_rotation) != hd * hd ||
        numel(v_rotation) != hd * hd || numel(k_centroids) < (1ull << key_bits) ||
        numel(v_centroids) < (1ull << value_bits))
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq arguments");
    if (kv_len > 0x7fffffffu || start_pos > 0x7fffffffu || T > 0x7fffffffu)
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq: sizes beyond int32");
    const uint64_t needed_blocks = (kv_len + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
    if (num_blocks < needed_blocks)
        return fail(FHIP_ERR_INVALID_SHAPE, "block table has %zu blocks for kv_len %zu",
                    num_blocks, kv_len);
    const uint64_t kpd = fhip_tq_packed_dim_per_head(hd, key_bits);
    const uint64_t vpd = fhip_tq_packed_dim_per_head(hd, value_bits);
    const uint64_t needs[4] = {FHIP_PAGE_TOKENS * num_kv_heads * kpd,
                               FHIP_PAGE_TOKENS * num_kv_heads * 2,
                               FHIP_PAGE_TOKENS * num_kv_heads * vpd,
                               FHIP_PAGE_TOKENS * num_kv_heads * 2};
    const int32_t dts[4] = {-1, -1, -1, -1};
    PoolView pp;
    int r = find_pool(b, pool, 4, needs, dts, &pp);
    if (r) return r;
    for (uint64_t i = 0; i < needed_blocks; ++i)
        if (block_table[i] < 0 || (uint64_t)block_table[i] >= pp.pool_len)
            return fail(FHIP_ERR_INVALID_SHAPE, "block id %d outside the pool of %zu",
                        block_table[i], pp.pool_len);
    if (T == 0) return FHIP_OK;
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    void* dbt;
    int s1;
    r = b->stage(block_table, (needed_blocks ? needed_blocks : 1) * sizeof(int32_t), &dbt, &s1);
    if (r) return r;
    const size_t wsb = fhip_attention_tq_workspace_bytes(
        (int)T, (int)qh, (int)hd, needed_blocks ? (int)needed_blocks : 1);
    void* ws;
    r = b->get_workspace(wsb, &ws);
    if (r) return r;
    const void** dp = pp.dev;
    const size_t n = pp.pool_len;
    int e = fhip_launch_attention_paged_tq_ws(
        po, pq, (const int*)dbt, dp, dp + n, dp + 2 * n, dp + 3 * n, (const float*)pkr,
        (const float*)pvr, (const float*)pkc, (const float*)pvc, (int)T, (int)qh,
        (int)num_kv_heads, (int)hd, (int)kv_len, (int)start_pos, key_bits, value_bits, (int)kpd,
        (int)vpd, ws, wsb, b->stream);
    b->stage_done(s1);
    if (e != hipSuccess) return hip_fail((hipError_t)e);
    return FHIP_OK;
}

// QuantizedKvCacheManager::append_kv (quantized_paged_kv_cache.rs:404-500) for one layer over a
// registered TurboQuant pool: compress keys and values and write token t straight into page
// block_table[(start_pos + t) / 16], slot (start_pos + t) % 16 of the pool's per-block
// tensors. The reference compresses into scratch tensors and copies each page's rows with four
// copy_rows calls per page span.
int fhip_tq_append_kv(fhip_backend* b, uint64_t pool, const fhip_tensor* keys,
                      const fhip_tensor* values, const fhip_tensor* k_rotation,
                      const fhip_tensor* v_rotation, const fhip_tensor* k_centroids,
                      const fhip_tensor* v_centroids, uint8_t key_bits, uint8_t value_bits,
                      const int32_t* block_table, size_t num_blocks, size_t start_pos) {
    CHECK_B(b);
    NO_CAPTURE(b, "tq_append_kv");
    CHECK_T(keys);
    CHECK_T(values);
    CHECK_T(k_rotation);
    CHECK_T(v_rotation);
    CHECK_T(k_centroids);
    CHECK_T(v_centroids);
    GET_PTR(b, keys, pk);
    GET_PTR(b, values, pv);
    GET_PTR(b, k_rotation, pkr);
    GET_PTR(b, v_rotation, pvr);
    GET_PTR(b, k_centroids, pkc);
    GET_PTR(b, v_centroids, pvc);
    if (keys->ndim != 3 || keys->dtype != FHIP_FP16 || !same_shape(keys, values) ||
        values->dtype != FHIP_FP16)
        return fail(FHIP_ERR_INVALID_SHAPE,
                    "append_kv keys %s and values %s must be [N, kv_heads, head_dim] FP16",
                    shape_str(keys).c_str(), shape_str(values).c_str());
    const uint64_t N = keys->shape[0], kvh = keys->shape[1], hd = keys->shape[2];
    const uint64_t KL = numel(k_centroids), VL = numel(v_centroids);
    if (key_bits < 1 || key_bits > 8 || value_bits < 1 || value_bits > 8 || KL < 1 ||
        KL > (1ull << key_bits) || VL < 1 || VL > (1ull << value_bits) ||
        k_centroids->dtype != FHIP_FP32 || v_centroids->dtype != FHIP_FP32 ||
        numel(k_rotation) != hd * hd || numel(v_rotation) != hd * hd ||
        k_rotation->dtype != FHIP_FP32 || v_rotation->dtype != FHIP_FP32 || kvh == 0 ||
        hd == 0 || hd > 8192)
        return fail(FHIP_ERR_INVALID_SHAPE, "append_kv: tables for %u/%u bits, head_dim %llu",
                    (unsigned)key_bits, (unsigned)value_bits, (unsigned long long)hd);
    if (N == 0) return FHIP_OK;
    if (start_pos + N > 0x7fffffffu || N * kvh > 0x7fffffffu)
        return fail(FHIP_ERR_INVALID_SHAPE, "append_kv: sizes beyond int32");
    const uint64_t last_block = (start_pos + N - 1) / FHIP_PAGE_TOKENS;
    if (num_blocks <= last_block)
        return fail(FHIP_ERR_INVALID_SHAPE, "block table has %zu blocks for position %llu",
                    num_blocks, (unsigned long long)(start_pos + N - 1));
    const uint64_t kpd = fhip_tq_packed_dim_per_head(hd, key_bits);
    const uint64_t vpd = fhip_tq_packed_dim_per_head(hd, value_bits);
    const uint64_t needs[4] = {FHIP_PAGE_TOKENS * kvh * kpd, FHIP_PAGE_TOKENS * kvh * 2,
                               FHIP_PAGE_TOKENS * kvh * vpd, FHIP_PAGE_TOKENS * kvh * 2};
    const int32_t dts[4] = {-1, FHIP_FP16, -1, FHIP_FP16};
    PoolView pp;
    int r = find_pool(b, pool, 4, needs, dts, &pp);
    if (r) return r;
    for (uint64_t i = start_pos / FHIP_PAGE_TOKENS; i <= last_block; ++i)
        if (block_table[i] < 0 || (uint64_t)block_table[i] >= pp.pool_len)
            return fail(FHIP_ERR_INVALID_SHAPE, "block id %d outside the pool of %zu",
                        block_table[i], pp.pool_len);
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    void* dbt;
    int s1;
    r = b->stage(block_table, (last_block + 1) * sizeof(int32_t), &dbt, &s1);
    if (r) return r;
    void* const* dp = (void* const*)pp.dev;
    const size_t n = pp.pool_len;
    int e;
    {
        std::lock_guard<std::mutex> gp(b->plan_mu);
        struct Side {
            const void* x;
            uint64_t rot_id, cent_id;
            void *rot, *cent;
            int levels, bits, list;
        } sides[2] = {{pk, k_rotation->id, k_centroids->id, pkr, pkc, (int)KL, key_bits, 0},
                      {pv, v_rotation->id, v_centroids->id, pvr, pvc, (int)VL, value_bits, 2}};
        e = hipSuccess;
        fhip_tq_plan* plans[2];
        for (int i = 0; i < 2; ++i)
            plans[i] = b->plan_for(sides[i].rot_id, sides[i].rot, sides[i].cent_id, sides[i].cent,
                                   sides[i].levels, sides[i].bits, (int)hd);
        // both plans: keys and values in one launch
        const bool kv = plans[0] && plans[1];
        if (kv)
            e = (hipError_t)fhip_launch_tq_compress_kv_page_ptrs_planned(
                plans[0], plans[1], pk, pv, dp, dp + n, dp + 2 * n, dp + 3 * n,
                (const int32_t*)dbt, (int)n, (int)start_pos, (int)N, (int)kvh, b->stream);
        for (int i = 0; i < 2 && !kv; ++i) {
            const Side& sd = sides[i];
            if (e != hipSuccess) break;
            fhip_tq_plan* plan = plans[i];
            if (plan)
                e = (hipError_t)fhip_launch_tq_compress_page_ptrs_planned(
                    plan, sd.x, dp + sd.list * n, dp + (sd.list + 1) * n, (const int32_t*)dbt,
                    (int)n, (int)start_pos, (int)N, (int)kvh, b->stream);
            else
                e = (hipError_t)fhip_launch_tq_compress_page_ptrs(
                    sd.x, (const float*)sd.rot, (const float*)sd.cent, sd.levels, sd.bits,
                    dp + sd.list * n, dp + (sd.list + 1) * n, (const int32_t*)dbt, (int)n,
                    (int)start_pos, (int)N, (int)kvh, (int)hd, b->stream);
        }
    }
    b->stage_done(s1);
    if (e != hipSuccess) return hip_fail((hipError_t)e);
    return FHIP_OK;
}

// Decode attention for a batch of sequences over a registered TurboQuant pool in one call:
// sequence i attends seq_lens[i] positions through row i of block_tables [B, max_blocks]. The
// engine dispatches Backend::attention_paged_tq once per sequence instead
// (crates/fracture-engine/src/batched.rs:145-194); the kernels here run the whole batch.
int fhip_attention_paged_tq_batched(fhip_backend* b, const fhip_tensor* q,
                                    const int32_t* block_tables, size_t num_seqs,
                                    size_t max_blocks, const uint32_t* seq_lens, uint64_t pool,
                                    const fhip_tensor* k_rotation, const fhip_tensor* v_rotation,
                                    const fhip_tensor* k_centroids,
                                    const fhip_tensor* v_centroids, uint8_t key_bits,
                                    uint8_t value_bits, size_t num_kv_heads,
                                    const fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "attention_paged_tq_batched");
    CHECK_T(q);
    CHECK_T(k_rotation);
    CHECK_T(v_rotation);
    CHECK_T(k_centroids);
    CHECK_T(v_centroids);
    CHECK_T(out);
    GET_PTR(b, q, pq);
    GET_PTR(b, out, po);
    WRITES(b, out);
    GET_PTR(b, k_rotation, pkr);
    GET_PTR(b, v_rotation, pvr);
    GET_PTR(b, k_centroids, pkc);
    GET_PTR(b, v_centroids, pvc);
    if (q->ndim != 3 || q->dtype != FHIP_FP16 || out->dtype != FHIP_FP16 ||
        numel(out) != numel(q))
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq_batched q %s out %s",
                    shape_str(q).c_str(), shape_str(out).c_str());
    const uint64_t B = q->shape[0], qh = q->shape[1], hd = q->shape[2];
    // the host arrays hold num_seqs rows: never read past them for a q with more rows
    if (num_seqs != B)
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq_batched: %zu sequences in the "
                    "block tables and lengths, %llu queries in q %s", num_seqs,
                    (unsigned long long)B, shape_str(q).c_str());
    if (B > 0 && (block_tables == nullptr || seq_lens == nullptr))
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq_batched: null block tables or "
                    "lengths");
    if (num_kv_heads == 0 || qh % num_kv_heads != 0 || qh / num_kv_heads > 8 || key_bits < 1 ||
        key_bits > 8 || value_bits < 1 || value_bits > 8 || numel(k_rotation) != hd * hd ||
        numel(v_rotation) != hd * hd || numel(k_centroids) < (1ull << key_bits) ||
        numel(v_centroids) < (1ull << value_bits) || hd % 8 != 0 || hd > 256)
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq_batched arguments");
    if (B > 65535 || max_blocks == 0 || max_blocks > 65536)
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged_tq_batched: %llu sequences of up "
                    "to %zu blocks (at most 65535 and 65536)", (unsigned long long)B, max_blocks);
    const uint64_t kpd = fhip_tq_packed_dim_per_head(hd, key_bits);
    const uint64_t vpd = fhip_tq_packed_dim_per_head(hd, value_bits);
    const uint64_t needs[4] = {FHIP_PAGE_TOKENS * num_kv_heads * kpd,
                               FHIP_PAGE_TOKENS * num_kv_heads * 2,
                               FHIP_PAGE_TOKENS * num_kv_heads * vpd,
                               FHIP_PAGE_TOKENS * num_kv_heads * 2};
    const int32_t dts[4] = {-1, -1, -1, -1};
    PoolView pp;
    int r = find_pool(b, pool, 4, needs, dts, &pp);
    if (r) return r;
    // Errors are reported in row order: the first sequence whose length or one of whose block
    // ids is out of range. id_error(n) scans the ids of sequences [0, n) for the first bad one
    // (the error path only: on the way to a launch the ids are checked once staged, below).
    auto id_error = [&](uint64_t n) -> int {
        for (uint64_t i = 0; i < n; ++i) {
            const uint64_t nb = (seq_lens[i] + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
            for (uint64_t j = 0; j < nb; ++j) {
                const int32_t id = block_tables[i * max_blocks + j];
                if (id < 0 || (uint64_t)id >= pp.pool_len)
                    return fail(FHIP_ERR_INVALID_SHAPE, "sequence %llu: block id %d outside the "
                                "pool of %zu", (unsigned long long)i, id, pp.pool_len);
            }
        }
        return FHIP_OK;
    };
    for (uint64_t i = 0; i < B; ++i) {
        if (seq_lens[i] > max_blocks * FHIP_PAGE_TOKENS) {
            r = id_error(i);
            if (r) return r;
            return fail(FHIP_ERR_INVALID_SHAPE, "sequence %llu: %u positions in %zu blocks",
                        (unsigned long long)i, seq_lens[i], max_blocks);
        }
    }
    if (B == 0) return FHIP_OK;
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    // The lengths and the block table travel in one slot, copied on the side stream ahead of
    // the kernels; rows hold their used page ids only (the kernels read no others), at a
    // stride rounded up to 16 bytes.
    const size_t stride = (max_blocks + 3) & ~(size_t)3;
    const size_t lens_bytes = (B * sizeof(int32_t) + 255) & ~(size_t)255;
    const size_t staged = lens_bytes + B * stride * sizeof(int32_t);
    const size_t wsb = fhip_attention_tq_workspace_bytes((int)B, (int)qh, (int)hd, (int)max_blocks);
    void* ws;
    r = b->get_workspace(wsb, &ws);
    if (r) return r;
    void *hslot, *dslot;
    int s1;
    r = b->stage_ahead_begin(staged, &hslot, &dslot, &s1);
    if (r) return r;
    int32_t* hlens = (int32_t*)hslot;
    int32_t* htable = (int32_t*)((char*)hslot + lens_bytes);
    for (uint64_t i = 0; i < B; ++i) {
        hlens[i] = (int32_t)seq_lens[i];
        const uint64_t nb = (seq_lens[i] + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
        memcpy(htable + i * stride, block_tables + i * max_blocks, nb * sizeof(int32_t));
    }
    r = b->stage_ahead_copy(s1, staged);
    if (r) return r;
    // The block ids, checked in the slot while its copy runs: one unsigned compare per id,
    // OR-reduced without branches (the compiler vectorizes it; a loop that leaves at the
    // first bad id does not, and cost ~4x as much at 64 sequences of up to 2048 blocks).
    // Ids are int32, so with a pool of 2^31 blocks or more only the negative ones are out.
    const uint32_t lim = pp.pool_len < 0x80000000ull ? (uint32_t)pp.pool_len : 0x80000000u;
    uint32_t bad = 0;
    for (uint64_t i = 0; i < B; ++i) {
        const uint64_t nb = (seq_lens[i] + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
        const int32_t* row = htable + i * stride;
        uint32_t m = 0;
        for (uint64_t j = 0; j < nb; ++j) m |= (uint32_t)((uint32_t)row[j] >= lim);
        bad |= m;
    }
    r = b->stage_ahead_wait(s1);
    if (r) return r;
    // nothing reads the slot: its next reuse waits for both streams (it stays handed out)
    if (bad) return id_error(B);
    const void** dp = pp.dev;
    const size_t n = pp.pool_len;
    int e = fhip_internal::attention_tq_decode_ptrs_staged(
        po, pq, (const int32_t*)((char*)dslot + lens_bytes), (const int32_t*)dslot, (int)B,
        (int)max_blocks, (int)stride, (int)n, dp, dp + n, dp + 2 * n, dp + 3 * n,
        (const float*)pkr, (const float*)pvr, (const float*)pkc, (const float*)pvc, (int)qh,
        (int)num_kv_heads, (int)hd, key_bits, value_bits, ws, b->stream);
    b->stage_done(s1);
    if (e != hipSuccess) return hip_fail((hipError_t)e);
    return FHIP_OK;
}

// Backend::attention_paged (backend.rs:74-88; cuda/src/backend.rs:255-345): q [T, qh, hd]
// fp16; k_blocks / v_blocks are the pool's per-block tensors, indexed by physical block id
// (batched.rs:92-97). The block table and the pointer arrays go through the pinned staging
// ring instead of per-call device allocations.
int fhip_attention_paged(fhip_backend* b, const fhip_tensor* q, const int32_t* block_table,
                         size_t num_blocks, const fhip_tensor* k_blocks,
                         const fhip_tensor* v_blocks, size_t pool_len, size_t num_kv_heads,
                         size_t kv_len, size_t start_pos, const fhip_tensor* out) {
    CHECK_B(b);
    NO_CAPTURE(b, "attention_paged");
    CHECK_T(q);
    CHECK_T(out);
    GET_PTR(b, q, pq);
    GET_PTR(b, out, po);
    WRITES(b, out);
    if (q->ndim != 3 || q->dtype != FHIP_FP16 || out->dtype != FHIP_FP16 ||
        numel(out) != numel(q))
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged q %s out %s",
                    shape_str(q).c_str(), shape_str(out).c_str());
    const uint64_t T = q->shape[0], qh = q->shape[1], hd = q->shape[2];
    if (num_kv_heads == 0 || qh % num_kv_heads != 0 ||
        hd == 0 || hd > 256)
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged: %zu q heads, %zu kv heads, "
                    "head_dim %zu (1 to 256)", (size_t)qh, num_kv_heads, (size_t)hd);
    if (kv_len > 0x7fffffffu || start_pos > 0x7fffffffu || T > 0x7fffffffu)
        return fail(FHIP_ERR_INVALID_SHAPE, "attention_paged: sizes beyond int32");
    const uint64_t needed_blocks = (kv_len + FHIP_PAGE_TOKENS - 1) / FHIP_PAGE_TOKENS;
    if (num_blocks < needed_blocks)
        return fail(FHIP_ERR_INVALID_SHAPE, "block table has %zu blocks for kv_len %zu",
                    num_blocks, kv_len);
    std::vector<const void*> ptrs(2 * pool_len > 0 ? 2 * pool_len : 1, nullptr);
    const uint64_t need = FHIP_PAGE_TOKENS * num_kv_heads * hd * 2;
    for (size_t i = 0; i < pool_len; ++i) {
        const fhip_tensor* ts[2] = {&k_blocks[i], &v_blocks[i]};
        for (int k = 0; k < 2; ++k) {
            void* p;
            int r = b->get_ptr(ts[k]->id, &p);
            if (r) return r;
            if (ts[k]->dtype != FHIP_FP16 || size_bytes(ts[k]) < need)
                return fail(FHIP_ERR_INVALID_SHAPE, "block tensor %s: need %zu fp16 bytes",
                            shape_str(ts[k]).c_str(), (size_t)need);
            ptrs[(size_t)k * pool_len + i] = p;
        }
    }
    for (uint64_t i = 0; i < needed_blocks; ++i)
        if (block_table[i] < 0 || (uint64_t)block_table[i] >= pool_len)
            return fail(FHIP_ERR_INVALID_SHAPE, "block id %d outside the pool of %zu",
                        block_table[i], pool_len);
    if (T == 0) return FHIP_OK;
    set_device(b);
    std::lock_guard<std::mutex> g(b->launch_mu);
    void *dbt, *dptr;
    int s1, s2;
    int r = b->stage(block_table, (needed_blocks ? needed_blocks : 1) * sizeof(int32_t), &dbt, &s1);
    if (r) return r;
    r = b->stage(ptrs.data(), ptrs.size() * sizeof(void*), &dptr, &s2);
    if (r) return r;
    const size_t wsb = fhip_attention_paged_workspace_bytes(
        (int)T, (int)qh, (int)hd, needed_blocks ? (int)needed_blocks : 1);
    void* ws;
    r = b->get_workspace(wsb, &ws);
    if (r) return r;
    const void** dp = (const void**)dptr;
    int e = fhip_launch_paged_attention_ws(po, pq, (const int*)dbt, dp, dp + pool_len, (int)T,
                                           (int)qh, (int)num_kv_heads, (int)hd, (int)kv_len,
                                           (int)start_pos, (int)needed_blocks, ws, wsb,
                                           b->stream);
    b->stage_done(s1);
    b->stage_done(s2);
    if (e != hipSuccess) return hip_fail((hipError_t)e);
    return FHIP_OK;
}

}  // extern "C"
