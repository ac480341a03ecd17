// Shared internals of liblcdhip.so (not part of the public C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "lcdhip.h"

namespace lcdhip {

void set_error(const char *format, ...);
hipStream_t resolve_stream(lcdhip_stream stream);
bool initialised();

// Device scratch that lives until shutdown (small flags and counters).
struct Context {
    int device = -1;
    hipStream_t stream = nullptr;
    hipDeviceProp_t props{};
    bool ready = false;
};
Context &context();

// Device memory of the inspector (its temporaries and the arrays of a DAG),
// kept for reuse: hipMalloc and hipFree cost 50 to 150 us a call here, and an
// inspection makes dozens of them.  pool_alloc hands out a block of at least
// `bytes` (an idle one of a fitting size, else a new allocation);
// pool_release takes it back without freeing it -- the caller has made sure
// that no work in flight still uses it.  At most kPoolIdleBytes stay idle,
// what comes back beyond that is freed; lcdhip_shutdown frees every idle
// block.  Blocks belong to the device that was current when they were made.
constexpr size_t kPoolIdleBytes = size_t(1) << 30;
hipError_t pool_alloc(void **out, size_t bytes);
void pool_release(void *pointer);
void pool_trim();
// Give blocks back from a place that cannot know what still uses them (the
// end of an inspector call, the destruction of a DAG): waits for the device
// and keeps them for reuse -- or, while a stream capture begun through
// lcdhip_graph_begin_capture is open (nothing may wait for a capturing
// stream), hands them to hipFree as before the pool existed.
void pool_retire(void *const *pointers, size_t count);

}  // namespace lcdhip

#define LCDHIP_CHECK(call)                                                    \
    do {                                                                      \
        hipError_t lcdhip_status_ = (call);                                   \
        if (lcdhip_status_ != hipSuccess) {                                   \
            lcdhip::set_error("%s failed: %s (%s:%d)", #call,                 \
                              hipGetErrorString(lcdhip_status_), __FILE__,    \
                              __LINE__);                                      \
            return LCDHIP_ERR_HIP;                                            \
        }                                                                     \
    } while (0)

#define LCDHIP_REQUIRE_INIT()                                                 \
    do {                                                                      \
        if (!lcdhip::initialised()) {                                         \
            lcdhip::set_error("lcdhip_init has not been called");             \
            return LCDHIP_ERR_NO_DEVICE;                                      \
        }                                                                     \
    } while (0)
