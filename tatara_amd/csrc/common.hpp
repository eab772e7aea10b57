// Shared helpers for the tatara MI355X (gfx950) training backend.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

namespace tatara {

// Status codes returned by every extern "C" entry point.
enum Status : int32_t {
    kOk = 0,
    kErrHip = -1,        // a HIP runtime call failed (message carries the call and kernel)
    kErrOutOfMemory = -2,
    kErrInvalid = -3,    // argument / shape precondition violated
    kErrState = -4,      // call not valid in the current state
};

// Thread-local last error message ("HIP error {code}: {name}: {msg} [kernel=...]").
void set_error(const std::string& msg);
const char* last_error();

// Converts a HIP error into a status and records the message.
int32_t hip_status(hipError_t e, const char* what);

#define TATARA_HIP(call, what)                                  \
    do {                                                        \
        hipError_t _e = (call);                                 \
        if (_e != hipSuccess) return ::tatara::hip_status(_e, what); \
    } while (0)

// Launch check after a kernel launch: reports a launch error with the kernel name.
#define TATARA_LAUNCHED(name)                                   \
    do {                                                        \
        hipError_t _e = hipGetLastError();                      \
        if (_e != hipSuccess) return ::tatara::hip_status(_e, "launch " name); \
    } while (0)

#define TATARA_REQUIRE(cond, msg)                               \
    do {                                                        \
        if (!(cond)) {                                          \
            ::tatara::set_error(std::string("invalid argument: ") + (msg)); \
            return ::tatara::kErrInvalid;                       \
        }                                                       \
    } while (0)

// Number of XCDs on MI355X.  Workgroups are dispatched to XCDs round-robin by
// workgroup id, so a launch that wants consecutive logical tiles to share one
// XCD's L2 remaps blockIdx with xcd_swizzle().
constexpr uint32_t kNumXcd = 8;

__device__ __forceinline__ uint32_t xcd_swizzle(uint32_t bid, uint32_t nblocks) {
    // Blocks bid = x, x+8, x+16, ... run on XCD x.  Give XCD x the logical
    // range [x*per, (x+1)*per) so that neighbouring logical tiles share an L2.
    const uint32_t per = nblocks / kNumXcd;
    const uint32_t full = per * kNumXcd;
    if (bid >= full) return bid;  // tail that does not divide evenly: identity
    return (bid % kNumXcd) * per + bid / kNumXcd;
}

// A wave-uniform load of data the kernel only reads, through the scalar
// cache (s_load, given a uniform address).  Its wait (lgkmcnt) leaves the
// wave's vector loads in flight, where a vector load of the same address
// would be waited for (vmcnt) behind all of them.
template <typename T>
__device__ __forceinline__ T scalar_load(const T* p) {
    return *(const __attribute__((address_space(4))) T*)p;
}

__device__ __forceinline__ float crelu01(float x) {
    return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x);
}

inline uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

}  // namespace tatara
