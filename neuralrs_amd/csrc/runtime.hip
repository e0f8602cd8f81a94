// Runtime part of the C ABI: device selection, stream, buffers, copies,
// errors and the library's lazily grown scratch. Replaces the reference's
// process-global cudarc backend (src/cuda/backend.rs:10-42) and the
// residency helpers of src/cuda/runtime.rs:39-124.
#include <algorithm>
#include <cstdarg>
#include <cstring>
#include <unordered_map>
#include <vector>

#include "nrs_internal.hpp"

namespace nrs {
namespace {

constexpr int kSlots = 7;

// Scratch of the no-allocation entry points: one per GPU, held until the
// process ends. In host code `scratch` names a host-side stand-in, so it is
// never passed to a kernel or copy; its device address is looked up once per
// device in nrs_init (hipGetSymbolAddress) and handed out by noalloc_scratch().
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];
float* g_scratch_ptr[kMaxDevices] = {};
size_t g_lds_limit[kMaxDevices] = {};

struct State {
    bool init = false;
    int device = 0;
    hipStream_t stream = nullptr;  // null stream unless the caller sets one
    float* ws[kSlots] = {};
    size_t ws_bytes[kSlots] = {};
};

State g;
thread_local char g_err[1024] = "";

// Caching allocator behind nrs_malloc / nrs_free. The reference allocates
// every op's output and gradient with alloc_zeros and frees them on drop
// (src/cuda/runtime.rs:39-51, e.g. src/cuda/graph/matmul.rs:271,410), so a
// drop-in pays one allocation per op; hipMalloc costs tens of microseconds and
// hipFree waits for the device. Blocks are rounded to size classes (512 B
// steps up to 1 MiB, 2 MiB steps above) and a freed block goes to its class's
// free list, to be handed out again by the next nrs_malloc of that class.
// Reuse follows the library stream's order: work enqueued after the reuse
// runs after every launch that read the block before it was freed.
constexpr size_t kSmallLimit = size_t(1) << 20, kSmallStep = 512,
                 kLargeStep = size_t(2) << 20;

struct BlockCache {
    std::unordered_map<void*, size_t> live;               // pointer -> class bytes
    std::unordered_map<size_t, std::vector<void*>> idle;  // class bytes -> free blocks
    size_t live_bytes = 0, idle_bytes = 0;
};
BlockCache cache;

size_t size_class(size_t bytes) {
    if (bytes == 0) bytes = 4;  // a distinct non-null handle for empty tensors
    const size_t step = bytes <= kSmallLimit ? kSmallStep : kLargeStep;
    return (bytes + step - 1) / step * step;
}

// hipFree every idle block (after the stream that freed them has drained).
int release_idle() {
    if (cache.idle_bytes == 0) return NRS_OK;
    NRS_HIP_CHECK(hipStreamSynchronize(g.stream));
    for (auto& kv : cache.idle)
        for (void* p : kv.second) NRS_HIP_CHECK(hipFree(p));
    cache.idle.clear();
    cache.idle_bytes = 0;
    return NRS_OK;
}

// Zero fill in 16-byte units where aligned; a kernel rather than
// hipMemsetAsync so the call stays correct inside a captured HIP graph.
__global__ void fill_zero_kernel(unsigned char* p, size_t bytes) {
    size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t nthreads = (size_t)gridDim.x * blockDim.x;
    size_t head = (16 - ((uintptr_t)p & 15)) & 15;
    if (head > bytes) head = bytes;
    for (size_t i = tid; i < head; i += nthreads) p[i] = 0;
    unsigned char* body = p + head;
    size_t nvec = (bytes - head) / 16;
    uint4* v = reinterpret_cast<uint4*>(body);
    for (size_t i = tid; i < nvec; i += nthreads) v[i] = make_uint4(0, 0, 0, 0);
    size_t tail0 = head + nvec * 16;
    for (size_t i = tail0 + tid; i < bytes; i += nthreads) p[i] = 0;
}

// Device-to-device copy of whole 16-byte units (both ends 16-byte aligned).
__global__ __launch_bounds__(256) void copy16_kernel(uint4* __restrict__ dst,
                                                     const uint4* __restrict__ src, size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
        dst[i] = src[i];
}

}  // namespace

hipStream_t stream() { return g.stream; }

int num_cus() {
    static int cus = 0;
    if (cus == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, g.device) != hipSuccess || v <= 0)
            v = 256;
        cus = v;
    }
    return cus;
}
int device() { return g.device; }
size_t lds_limit() {
    return g.device >= 0 && g.device < kMaxDevices ? g_lds_limit[g.device] : 0;
}
bool initialized() { return g.init; }

float* noalloc_scratch() {
    return g.device >= 0 && g.device < kMaxDevices ? g_scratch_ptr[g.device] : nullptr;
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

float* workspace(size_t bytes, int slot) {
    if (slot < 0 || slot >= kSlots) {
        set_error(NRS_ERR_ARG, "internal: bad scratch slot %d", slot);
        return nullptr;
    }
    if (bytes <= g.ws_bytes[slot]) return g.ws[slot];
    if (g.ws[slot]) {
        // The old buffer may still be read by queued kernels.
        if (hipStreamSynchronize(g.stream) != hipSuccess) return nullptr;
        (void)hipFree(g.ws[slot]);
        g.ws[slot] = nullptr;
        g.ws_bytes[slot] = 0;
    }
    size_t want = bytes + bytes / 4;  // grow with headroom
    want = (want + 255) & ~(size_t)255;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        set_error(NRS_ERR_ALLOC, "scratch allocation of %zu bytes failed: %s", want,
                  hipGetErrorString(e));
        return nullptr;
    }
    g.ws[slot] = static_cast<float*>(p);
    g.ws_bytes[slot] = want;
    return g.ws[slot];
}

int zero_fill(void* ptr, size_t bytes) {
    if (bytes == 0) return NRS_OK;
    size_t units = (bytes + 15) / 16;
    unsigned blocks = (unsigned)std::min<size_t>((units + 255) / 256, 4096);
    if (blocks == 0) blocks = 1;
    fill_zero_kernel<<<blocks, 256, 0, g.stream>>>(static_cast<unsigned char*>(ptr), bytes);
    NRS_LAUNCH_CHECK("memset_zero");
    return NRS_OK;
}

}  // namespace nrs

using nrs::g;

extern "C" {

int nrs_init(int device) {
    int count = 0;
    NRS_HIP_CHECK(hipGetDeviceCount(&count));
    NRS_ARG_CHECK(device >= 0 && device < count, "nrs_init: device %d out of range (count %d)",
                  device, count);
    NRS_ARG_CHECK(device < nrs::kMaxDevices, "nrs_init: device %d beyond the %d supported",
                  device, nrs::kMaxDevices);
    NRS_HIP_CHECK(hipSetDevice(device));
    if (!nrs::g_scratch_ptr[device]) {
        // this device's copy of the no-allocation scratch (a symbol lookup,
        // not an allocation), with the device current
        void* ptr = nullptr;
        NRS_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(nrs::scratch)));
        NRS_ARG_CHECK(ptr != nullptr, "nrs_init: no device address for the scratch array");
        nrs::g_scratch_ptr[device] = static_cast<float*>(ptr);
    }
    if (!nrs::g_lds_limit[device]) {
        int per_block = 0, opt_in = 0;
        NRS_HIP_CHECK(hipDeviceGetAttribute(&per_block, hipDeviceAttributeMaxSharedMemoryPerBlock,
                                            device));
        if (hipDeviceGetAttribute(&opt_in, hipDeviceAttributeSharedMemPerBlockOptin, device) !=
            hipSuccess)
            opt_in = 0;
        nrs::g_lds_limit[device] = (size_t)std::max(std::max(per_block, opt_in), 0);
    }
    g.device = device;
    g.init = true;
    return NRS_OK;
}

int nrs_shutdown(void) {
    if (!g.init) return NRS_OK;
    NRS_HIP_CHECK(hipStreamSynchronize(g.stream));
    if (int rc = nrs::release_idle()) return rc;
    for (int s = 0; s < nrs::kSlots; ++s) {
        if (g.ws[s]) NRS_HIP_CHECK(hipFree(g.ws[s]));
        g.ws[s] = nullptr;
        g.ws_bytes[s] = 0;
    }
    return NRS_OK;
}

int nrs_set_stream(void* stream) {
    // Work queued on the old stream may still read or write library scratch,
    // cached blocks and buffers freed since; work on the new stream is not
    // ordered after it. Drain the old stream before switching.
    if (static_cast<hipStream_t>(stream) != g.stream && g.init)
        NRS_HIP_CHECK(hipStreamSynchronize(g.stream));
    g.stream = static_cast<hipStream_t>(stream);
    return NRS_OK;
}

void* nrs_get_stream(void) { return static_cast<void*>(g.stream); }

const char* nrs_last_error(void) { return nrs::g_err; }

int nrs_malloc(void** ptr, size_t bytes) {
    NRS_REQUIRE_INIT();
    NRS_ARG_CHECK(ptr != nullptr, "nrs_malloc: null out-pointer");
    *ptr = nullptr;
    auto& c = nrs::cache;
    const size_t cls = nrs::size_class(bytes);
    void* p = nullptr;
    auto it = c.idle.find(cls);
    if (it != c.idle.end() && !it->second.empty()) {
        p = it->second.back();
        it->second.pop_back();
        c.idle_bytes -= cls;
    } else {
        hipError_t e = hipMalloc(&p, cls);
        if (e != hipSuccess) {
            // out of memory with blocks idle in the cache: give them back, retry once
            (void)hipGetLastError();
            if (int rc = nrs::release_idle()) return rc;
            e = hipMalloc(&p, cls);
        }
        if (e != hipSuccess)
            return nrs::set_error(NRS_ERR_ALLOC, "nrs_malloc(%zu): %s", bytes,
                                  hipGetErrorString(e));
    }
    c.live.emplace(p, cls);
    c.live_bytes += cls;
    *ptr = p;
    return NRS_OK;
}

int nrs_free(void* ptr) {
    if (!ptr) return NRS_OK;
    auto& c = nrs::cache;
    auto it = c.live.find(ptr);
    NRS_ARG_CHECK(it != c.live.end(),
                  "nrs_free(%p): not a live nrs_malloc buffer (freed twice, or not from "
                  "nrs_malloc)", ptr);
    const size_t cls = it->second;
    c.live.erase(it);
    c.live_bytes -= cls;
    c.idle[cls].push_back(ptr);
    c.idle_bytes += cls;
    return NRS_OK;
}

int nrs_empty_cache(void) { return nrs::release_idle(); }

int nrs_memory_stats(size_t* live_bytes, size_t* cached_bytes) {
    if (live_bytes) *live_bytes = nrs::cache.live_bytes;
    if (cached_bytes) *cached_bytes = nrs::cache.idle_bytes;
    return NRS_OK;
}

int nrs_memcpy_htod(void* dst, const void* src, size_t bytes) {
    NRS_REQUIRE_INIT();
    if (bytes == 0) return NRS_OK;
    NRS_ARG_CHECK(dst && src, "nrs_memcpy_htod: null pointer");
    NRS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g.stream));
    // Pageable source: make the copy complete before the caller may reuse it.
    NRS_HIP_CHECK(hipStreamSynchronize(g.stream));
    return NRS_OK;
}

int nrs_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    NRS_REQUIRE_INIT();
    if (bytes == 0) return NRS_OK;
    NRS_ARG_CHECK(dst && src, "nrs_memcpy_dtoh: null pointer");
    NRS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g.stream));
    NRS_HIP_CHECK(hipStreamSynchronize(g.stream));
    return NRS_OK;
}

int nrs_memcpy_dtod(void* dst, const void* src, size_t bytes) {
    NRS_REQUIRE_INIT();
    if (bytes == 0) return NRS_OK;
    NRS_ARG_CHECK(dst && src, "nrs_memcpy_dtod: null pointer");
    if ((((uintptr_t)dst | (uintptr_t)src | bytes) & 15) == 0) {
        // a copy kernel: a few microseconds sooner than the runtime's blit
        // for the activation-sized copies of reshape and accumulate_into
        const size_t units = bytes / 16;
        const unsigned blocks = (unsigned)std::min<size_t>((units + 255) / 256, 2048);
        nrs::copy16_kernel<<<blocks, 256, 0, g.stream>>>(static_cast<uint4*>(dst),
                                                         static_cast<const uint4*>(src), units);
        NRS_LAUNCH_CHECK("memcpy_dtod");
        return NRS_OK;
    }
    NRS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g.stream));
    return NRS_OK;
}

int nrs_memset_zero(void* ptr, size_t bytes) {
    NRS_REQUIRE_INIT();
    if (bytes == 0) return NRS_OK;
    NRS_ARG_CHECK(ptr != nullptr, "nrs_memset_zero: null pointer");
    return nrs::zero_fill(ptr, bytes);
}

int nrs_sync(void) {
    NRS_REQUIRE_INIT();
    NRS_HIP_CHECK(hipStreamSynchronize(g.stream));
    NRS_HIP_CHECK(hipGetLastError());
    return NRS_OK;
}

}  // extern "C"
