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
