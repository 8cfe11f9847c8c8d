// Device layer of libkvpersist.so: memory, copies and the arena staging
// (compaction) kernels that replace the reference's per-row
// cudaMemcpyAsync pairs (reference: src/kv_tile_manager.cu:104-121,
// :153-192). One flush = (optional) KVMap rebuild + ONE gather launch that
// moves every pending K|V row of the step into the arena.
//
// Gather kernel: one workgroup per staged row; the K bytes then the V bytes
// land back to back at arena + dst_row * row_stride (the reference's
// [K half | V half] row format). 16-byte vector moves when source, target and
// sizes are 16-byte aligned, byte moves otherwise. The map scatter rides in
// trailing workgroups of the same launch.
//
// Small flushes (the per-frame case) are run-length encoded: consecutive
// rows with consecutive sources and arena rows form one copy run, consecutive
// map rows with consecutive slots (or all -1) form one map run. When the runs
// fit, they travel as kernel arguments: no host memory is read by the kernel
// and nothing has to be fenced behind it. Larger flushes read their
// descriptors straight from a ring of mapped pinned host memory (no separate
// H2D copy); a ring region is reused only after the event recorded behind
// the launch that read it has completed.
//
// Layer staging (the frame pipeline's whole-layer run) has its own kernel:
// run tables of row copies (the frame pipeline sizes them to ~12 KiB, one
// pass of loads per workgroup) and up to 1024-entry map runs, one workgroup
// per run, read from the same ring; every thread moves 16-byte chunks with
// up to four loads in flight.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "kvp_c_api.h"
#include "kvp_internal.h"
#include "stage_runs.h"

namespace kvp {

namespace {
thread_local std::string g_last_error;
void* g_stream = nullptr;
}  // namespace

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

void* library_stream() { return g_stream; }

namespace {

constexpr int kStageThreads = 256;
constexpr int kMapThreads = 256;

__global__ __launch_bounds__(256) void map_fill_kernel(long* __restrict__ map, long n) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) map[i] = -1L;
}

__device__ __forceinline__ void copy_bytes(unsigned char* __restrict__ dst,
                                           const unsigned char* __restrict__ src,
                                           unsigned bytes) {
    typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
    if ((((uintptr_t)dst | (uintptr_t)src | (uintptr_t)bytes) & 15u) == 0) {
        const unsigned n16 = bytes >> 4;
        const u32x4* s = reinterpret_cast<const u32x4*>(src);
        u32x4* d = reinterpret_cast<u32x4*>(dst);
        for (unsigned i = threadIdx.x; i < n16; i += blockDim.x) d[i] = s[i];
    } else {
        for (unsigned i = threadIdx.x; i < bytes; i += blockDim.x) dst[i] = src[i];
    }
}

// blocks [0, n_copies): one row copy each; blocks after that: map scatter.
__global__ __launch_bounds__(256) void stage_kernel(const KvpRowCopy* __restrict__ copies,
                                                    long n_copies,
                                                    unsigned char* __restrict__ arena,
                                                    long row_stride,
                                                    const long* __restrict__ map_rows,
                                                    const long* __restrict__ map_slots,
                                                    long n_map, long* __restrict__ map) {
    const long b = blockIdx.x;
    if (b < n_copies) {
        const KvpRowCopy c = copies[b];
        unsigned char* dst = arena + c.dst_row * row_stride;
        copy_bytes(dst, static_cast<const unsigned char*>(c.k_src), c.k_bytes);
        copy_bytes(dst + c.k_bytes, static_cast<const unsigned char*>(c.v_src), c.v_bytes);
    } else {
        const long i = (b - n_copies) * blockDim.x + threadIdx.x;
        if (i < n_map) map[map_rows[i]] = map_slots[i];
    }
}

using stage::RunArgs;

__global__ __launch_bounds__(stage::kRunThreads) void stage_runs_kernel(const RunArgs a) {
    stage::stage_runs_block(a, (int)blockIdx.x);
}

// Layer staging: workgroups [0, n_copies) copy one run each, the next
// n_map_runs write one KVMap run each, the ones after that write 256
// group-descriptor entries each. A copy run moves n arena rows of
// 2 * cpr 16-byte chunks; chunk w < cpr of a row comes from its K row, the
// rest from its V row. Each thread keeps four chunks in flight before it
// stores them.
constexpr int kLayerThreads = 256;
constexpr int kLayerBatch = 4;

__global__ __launch_bounds__(kLayerThreads) void layer_stage_kernel(
    const LayerCopyRun* __restrict__ copies, long n_copies,
    const LayerMapRun* __restrict__ map_runs, long n_map_runs,
    const LayerGdWrite* __restrict__ gd_writes, long n_gd, unsigned char* __restrict__ arena,
    const unsigned char* __restrict__ k, const unsigned char* __restrict__ v, unsigned cpr,
    long* __restrict__ map, unsigned* __restrict__ gd) {
    typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
    const long b = blockIdx.x;
    if (b < n_copies) {
        const LayerCopyRun r = copies[b];
        const unsigned per_row = 2u * cpr;
        const unsigned total = (unsigned)r.n * per_row;
        const long rb = 16L * cpr;
        for (unsigned c0 = 0; c0 < total; c0 += kLayerBatch * kLayerThreads) {
            u32x4 val[kLayerBatch];
            unsigned char* dst[kLayerBatch];
#pragma unroll
            for (int u = 0; u < kLayerBatch; ++u) {
                const unsigned c = c0 + u * kLayerThreads + threadIdx.x;
                dst[u] = nullptr;
                if (c < total) {
                    const unsigned row = c / per_row;
                    const unsigned w = c - row * per_row;
                    const long src_row = (long)r.src_row + row;
                    const unsigned char* src = w < cpr ? k + src_row * rb + 16L * w
                                                       : v + src_row * rb + 16L * (w - cpr);
                    val[u] = *reinterpret_cast<const u32x4*>(src);
                    dst[u] = arena + ((long)r.dst_row + row) * 2 * rb + 16L * w;
                }
            }
#pragma unroll
            for (int u = 0; u < kLayerBatch; ++u)
                if (dst[u]) *reinterpret_cast<u32x4*>(dst[u]) = val[u];
        }
    } else if (b < n_copies + n_map_runs) {
        const LayerMapRun m = map_runs[b - n_copies];
        for (int j = (int)threadIdx.x; j < m.n; j += kLayerThreads)
            map[m.index + j] = m.value < 0 ? -1L : (long)m.value + j;
    } else {
        const long i = (b - n_copies - n_map_runs) * kLayerThreads + threadIdx.x;
        if (i < n_gd) {
            const LayerGdWrite w = gd_writes[i];
            typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
            *reinterpret_cast<u32x2*>(gd + 2 * w.index) = u32x2{w.w0, w.w1};
        }
    }
}

__global__ __launch_bounds__(256) void fill_words_kernel(unsigned* __restrict__ dst, long n,
                                                         unsigned value) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
        dst[i] = value;
}

// Descriptor ring in mapped, coherent host memory: the host writes a
// launch's run descriptors at `head`, the staging kernel reads them over
// the bus. A region is written again only after the ring wraps, and the
// wrap first waits for every launch that read the ring (drain). No event is
// recorded per launch: on MI355X an event record between the staging
// kernel and the attention launch after it, with its system-scope fence,
// left the GPU idle for about 5.6 us before the next kernel.
struct Stager {
    unsigned char* host = nullptr;  // mapped pinned memory
    unsigned char* dev = nullptr;   // device view of `host`
    size_t cap = 0;
    size_t head = 0;
    hipStream_t last = nullptr;  // stream of the launches since the last drain
    bool pending = false;        // launches since the last drain may still run

    ~Stager() {
        // the caller's stream may be gone by now: wait for the whole device
        if (pending) (void)hipDeviceSynchronize();
        if (host) (void)hipHostFree(host);
    }
    // Call before a launch on `s` that reads the ring. A launch on another
    // stream than the pending ones first waits for the device: the earlier
    // stream is not used again, as it may have been destroyed.
    bool before_launch(hipStream_t s) {
        if (pending && s != last) {
            if (hipDeviceSynchronize() != hipSuccess) return false;
            pending = false;
        }
        last = s;
        return true;
    }
    void after_launch() { pending = true; }
    // Waits for every launch that read the ring (all on `last`), then
    // restarts at its beginning.
    bool drain() {
        if (pending) {
            if (hipStreamSynchronize(last) != hipSuccess) return false;
            pending = false;
        }
        head = 0;
        return true;
    }
    bool reserve(size_t need) {
        if (need > cap) {
            if (!drain()) return false;
            if (host) (void)hipHostFree(host);
            host = nullptr;
            dev = nullptr;
            cap = 0;
            size_t want = need < ((size_t)4 << 20) ? ((size_t)4 << 20) : need * 2;
            if (hipHostMalloc(reinterpret_cast<void**>(&host), want,
                              hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
                host = nullptr;
                return false;
            }
            if (hipHostGetDevicePointer(reinterpret_cast<void**>(&dev), host, 0) != hipSuccess) {
                (void)hipHostFree(host);
                host = nullptr;
                return false;
            }
            cap = want;
            head = 0;
        }
        if (head + need > cap) {
            if (!drain()) return false;
        }
        return true;
    }
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace
}  // namespace kvp

using kvp::set_error;

extern "C" {

const char* kvp_last_error(void) { return kvp::g_last_error.c_str(); }

void kvp_set_stream(void* stream) { kvp::g_stream = stream; }
void* kvp_get_stream(void) { return kvp::g_stream; }

int kvp_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

void* kvp_dev_alloc(size_t bytes) {
    void* p = nullptr;
    if (bytes == 0) bytes = 1;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        set_error("hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

void kvp_dev_free(void* p) {
    if (p) (void)hipFree(p);
}

int kvp_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                                  static_cast<hipStream_t>(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        set_error("memcpy h2d: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

int kvp_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                                  static_cast<hipStream_t>(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        set_error("memcpy d2h: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

int kvp_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                                  static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        set_error("memcpy d2d: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

int kvp_stream_sync(void* stream) {
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        set_error("stream sync: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

int kvp_device_sync(void) {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        set_error("device sync: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

void* kvp_stager_create(void) { return new (std::nothrow) kvp::Stager(); }

void kvp_stager_destroy(void* s) { delete static_cast<kvp::Stager*>(s); }

int kvp_stage_run(void* stager, void* arena, long row_stride_bytes, const KvpRowCopy* copies,
                  long n_copies, long* map_dev, long map_fill, const long* map_rows,
                  const long* map_slots, long n_map, void* stream) {
    kvp::Stager* st = static_cast<kvp::Stager*>(stager);
    if (!st) {
        set_error("stage: null stager");
        return 1;
    }
    if (n_copies < 0 || n_map < 0 || map_fill < 0) {
        set_error("stage: negative count");
        return 1;
    }
    if (n_copies > 0 && (!arena || row_stride_bytes <= 0 || !copies)) {
        set_error("stage: copies need an arena, a positive row stride and descriptors");
        return 1;
    }
    if ((n_map > 0 || map_fill > 0) && !map_dev) {
        set_error("stage: map entries without a device map");
        return 1;
    }
    if (n_copies == 0 && n_map == 0 && map_fill == 0) return 0;
    hipStream_t hs = static_cast<hipStream_t>(stream);

    if (map_fill == 0) {
        kvp::RunArgs ra;
        if (kvp::stage::encode_runs(ra, static_cast<unsigned char*>(arena), row_stride_bytes, copies,
                             n_copies, map_dev, map_rows, map_slots, n_map)) {
            const long blocks = n_copies + (n_map + kvp::kStageThreads - 1) / kvp::kStageThreads;
            hipLaunchKernelGGL(kvp::stage_runs_kernel, dim3((unsigned)blocks),
                               dim3(kvp::kStageThreads), 0, hs, ra);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) {
                set_error("stage launch: %s", hipGetErrorString(e));
                return 1;
            }
            return 0;
        }
    }

    const size_t copy_bytes = kvp::align256((size_t)n_copies * sizeof(KvpRowCopy));
    const size_t map_bytes = kvp::align256((size_t)n_map * sizeof(long));
    const size_t need = copy_bytes + 2 * map_bytes;
    KvpRowCopy* d_copies = nullptr;
    long* d_rows = nullptr;
    long* d_slots = nullptr;
    if (need > 0) {
        if (!st->before_launch(hs) || !st->reserve(need)) {
            set_error("stage: descriptor ring allocation failed");
            return 1;
        }
        unsigned char* h = st->host + st->head;
        unsigned char* d = st->dev + st->head;
        if (n_copies > 0) memcpy(h, copies, (size_t)n_copies * sizeof(KvpRowCopy));
        if (n_map > 0) {
            memcpy(h + copy_bytes, map_rows, (size_t)n_map * sizeof(long));
            memcpy(h + copy_bytes + map_bytes, map_slots, (size_t)n_map * sizeof(long));
        }
        d_copies = reinterpret_cast<KvpRowCopy*>(d);
        d_rows = reinterpret_cast<long*>(d + copy_bytes);
        d_slots = reinterpret_cast<long*>(d + copy_bytes + map_bytes);
    }
    if (map_fill > 0) {
        long blocks = (map_fill + kvp::kMapThreads - 1) / kvp::kMapThreads;
        if (blocks > 1024) blocks = 1024;
        hipLaunchKernelGGL(kvp::map_fill_kernel, dim3((unsigned)blocks), dim3(kvp::kMapThreads), 0, hs,
                           map_dev, map_fill);
    }
    const long map_blocks = (n_map + kvp::kStageThreads - 1) / kvp::kStageThreads;
    const long blocks = n_copies + map_blocks;
    if (blocks > 0) {
        hipLaunchKernelGGL(kvp::stage_kernel, dim3((unsigned)blocks), dim3(kvp::kStageThreads), 0, hs,
                           d_copies, n_copies, static_cast<unsigned char*>(arena), row_stride_bytes,
                           d_rows, d_slots, n_map, map_dev);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("stage launch: %s", hipGetErrorString(e));
        return 1;
    }
    if (need > 0) {
        st->after_launch();
        st->head += need;
    }
    return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Staging plans: a flush prepared now (host bookkeeping) and launched later.
// ---------------------------------------------------------------------------
namespace kvp {

struct StagePlan {
    bool encoded = false;
    stage::RunArgs ra;
    // kept for the descriptor-ring path when the flush does not encode
    void* stager = nullptr;
    void* arena = nullptr;
    long stride = 0;
    std::vector<KvpRowCopy> copies;
    long* map_dev = nullptr;
    long map_fill = 0;
    std::vector<long> rows, slots;
};

void* stage_plan_create(void* stager, void* arena, long row_stride_bytes, const KvpRowCopy* copies,
                        long n_copies, long* map_dev, long map_fill, const long* map_rows,
                        const long* map_slots, long n_map) {
    StagePlan* p = new (std::nothrow) StagePlan();
    if (!p) {
        set_error("stage plan: out of memory");
        return nullptr;
    }
    if (map_fill == 0 && (n_copies == 0 || arena) &&
        stage::encode_runs(p->ra, static_cast<unsigned char*>(arena), row_stride_bytes, copies, n_copies,
                           map_dev, map_rows, map_slots, n_map)) {
        p->encoded = true;
        return p;
    }
    p->stager = stager;
    p->arena = arena;
    p->stride = row_stride_bytes;
    if (n_copies > 0) p->copies.assign(copies, copies + n_copies);
    p->map_dev = map_dev;
    p->map_fill = map_fill;
    if (n_map > 0) {
        p->rows.assign(map_rows, map_rows + n_map);
        p->slots.assign(map_slots, map_slots + n_map);
    }
    return p;
}

int stage_plan_launch(const void* plan, void* stream) {
    const StagePlan* p = static_cast<const StagePlan*>(plan);
    if (!p) return 0;
    hipStream_t hs = static_cast<hipStream_t>(stream);
    if (p->encoded) {
        const long blocks = stage::run_blocks(p->ra);
        if (blocks == 0) return 0;
        hipLaunchKernelGGL(stage_runs_kernel, dim3((unsigned)blocks), dim3(stage::kRunThreads), 0, hs, p->ra);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            set_error("stage launch: %s", hipGetErrorString(e));
            return 1;
        }
        return 0;
    }
    return kvp_stage_run(p->stager, p->arena, p->stride, p->copies.data(), (long)p->copies.size(),
                         p->map_dev, p->map_fill, p->rows.data(), p->slots.data(), (long)p->rows.size(),
                         stream);
}

void stage_plan_free(void* plan) { delete static_cast<StagePlan*>(plan); }

int fill_words(void* dst, long n, unsigned value, void* stream) {
    if (n <= 0) return 0;
    if (!dst) {
        set_error("fill: null destination");
        return 1;
    }
    const long blocks = std::min<long>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_words_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<unsigned*>(dst), n, value);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("fill launch: %s", hipGetErrorString(e));
        return 1;
    }
    return 0;
}

int layer_stage_launch(void* stager, void* arena, const void* k, const void* v, long row_bytes,
                       const LayerCopyRun* copies, long n_copies, long* map,
                       const LayerMapRun* map_runs, long n_map_runs, unsigned* gd,
                       const LayerGdWrite* gd_writes, long n_gd_writes, void* stream) {
    Stager* st = static_cast<Stager*>(stager);
    if (!st) {
        set_error("layer stage: null stager");
        return 1;
    }
    const long gd_blocks = (n_gd_writes + kLayerThreads - 1) / kLayerThreads;
    if (n_copies < 0 || n_map_runs < 0 || n_gd_writes < 0 ||
        n_copies + n_map_runs + gd_blocks > INT_MAX) {
        set_error("layer stage: bad run counts");
        return 1;
    }
    if (n_copies + n_map_runs + gd_blocks == 0) return 0;
    if (n_copies > 0 && (!arena || !k || !v || row_bytes <= 0 || row_bytes % 16 ||
                         ((uintptr_t)arena | (uintptr_t)k | (uintptr_t)v) % 16)) {
        set_error("layer stage: copies need 16-byte aligned arena, K, V and row size");
        return 1;
    }
    if (n_map_runs > 0 && !map) {
        set_error("layer stage: map runs without a map");
        return 1;
    }
    if (n_gd_writes > 0 && (!gd || (uintptr_t)gd % 8)) {
        set_error("layer stage: descriptor writes need an 8-byte aligned table");
        return 1;
    }
    const size_t copy_bytes = align256((size_t)n_copies * sizeof(LayerCopyRun));
    const size_t map_bytes = align256((size_t)n_map_runs * sizeof(LayerMapRun));
    const size_t need = copy_bytes + map_bytes + align256((size_t)n_gd_writes * sizeof(LayerGdWrite));
    hipStream_t hs = static_cast<hipStream_t>(stream);
    if (!st->before_launch(hs) || !st->reserve(need)) {
        set_error("layer stage: descriptor ring allocation failed");
        return 1;
    }
    unsigned char* h = st->host + st->head;
    unsigned char* d = st->dev + st->head;
    if (n_copies > 0) memcpy(h, copies, (size_t)n_copies * sizeof(LayerCopyRun));
    if (n_map_runs > 0) memcpy(h + copy_bytes, map_runs, (size_t)n_map_runs * sizeof(LayerMapRun));
    if (n_gd_writes > 0)
        memcpy(h + copy_bytes + map_bytes, gd_writes, (size_t)n_gd_writes * sizeof(LayerGdWrite));
    hipLaunchKernelGGL(layer_stage_kernel, dim3((unsigned)(n_copies + n_map_runs + gd_blocks)),
                       dim3(kLayerThreads), 0, hs, reinterpret_cast<const LayerCopyRun*>(d),
                       n_copies, reinterpret_cast<const LayerMapRun*>(d + copy_bytes), n_map_runs,
                       reinterpret_cast<const LayerGdWrite*>(d + copy_bytes + map_bytes),
                       n_gd_writes, static_cast<unsigned char*>(arena),
                       static_cast<const unsigned char*>(k), static_cast<const unsigned char*>(v),
                       (unsigned)(row_bytes / 16), map, gd);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("layer stage launch: %s", hipGetErrorString(e));
        return 1;
    }
    st->after_launch();
    st->head += need;
    return 0;
}

}  // namespace kvp
