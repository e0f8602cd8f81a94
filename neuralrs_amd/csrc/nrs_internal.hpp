// Internal helpers shared by the HIP translation units of libnrs_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "nrs_hip.h"

namespace nrs {

// Process-global state (one device, one stream), like the reference's
// OnceLock backend (src/cuda/backend.rs:17-28). Not thread-safe, matching the
// reference's single-threaded Rc<RefCell> host model.
hipStream_t stream();
int device();
bool initialized();

// Records a message retrievable with nrs_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);

// Library-owned scratch, grown lazily, one buffer per slot:
//   0 split-K partials, 1 im2col / dcols columns, 2 conv grad in GEMM layout,
//   3 reduction partials, 4 conv weights packed for LDS staging, 5 the conv
//   output or its gradient around a fused pooling (not used by the conv
//   entry points themselves, which the fused ones call), 6 the pooled
//   gradient masked by a ReLU between conv and pooling.
// Returns nullptr (and records an error) when the allocation fails.
float* workspace(size_t bytes, int slot = 0);

// Scratch of the no-allocation entry points: a file-scope device array of
// kNoAllocScratchBytes per GPU, its address looked up by nrs_init. Returns
// nullptr before nrs_init has run on the current device.
constexpr size_t kNoAllocScratchBytes = size_t(14) << 20;
float* noalloc_scratch();

// Zero-fills device memory on the library stream with a kernel.
int zero_fill(void* ptr, size_t bytes);

// Number of compute units of the current device (queried once).
int num_cus();

// LDS bytes one workgroup may allocate dynamically on the current device:
// the larger of its per-block and opt-in maxima, queried by nrs_init
// (160 KiB on gfx950). Kernels whose dynamic LDS would exceed it are not
// launched; their planners report the shape unsupported so that another
// path takes the call. Static LDS needs no such check: the compiler refuses
// a kernel whose static LDS exceeds the target's limit.
size_t lds_limit();

}  // namespace nrs

#define NRS_REQUIRE_INIT()                                                           \
    do {                                                                             \
        if (!nrs::initialized()) {                                                   \
            int _rc = nrs_init(0);                                                   \
            if (_rc != NRS_OK) return _rc;                                           \
        }                                                                            \
    } while (0)

#define NRS_HIP_CHECK(expr)                                                          \
    do {                                                                             \
        hipError_t _e = (expr);                                                      \
        if (_e != hipSuccess)                                                        \
            return nrs::set_error(NRS_ERR_HIP, "%s failed: %s (%s:%d)", #expr,       \
                                  hipGetErrorString(_e), __FILE__, __LINE__);        \
    } while (0)

#define NRS_LAUNCH_CHECK(what)                                                       \
    do {                                                                             \
        hipError_t _e = hipGetLastError();                                           \
        if (_e != hipSuccess)                                                        \
            return nrs::set_error(NRS_ERR_HIP, "%s: launch failed: %s", what,        \
                                  hipGetErrorString(_e));                            \
    } while (0)

#define NRS_ARG_CHECK(cond, ...)                                                     \
    do {                                                                             \
        if (!(cond)) return nrs::set_error(NRS_ERR_ARG, __VA_ARGS__);                \
    } while (0)
