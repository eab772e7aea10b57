// C ABI: streams, events, asynchronous copies, pinned host memory and
// code-object modules launched by kernel name.
//
// This is the part of the reference's device runtime that a caller drives
// directly (crates/gpu-runtime/src/native_backend.rs:33-300 and the free
// functions of crates/gpu-runtime/src/lib.rs:186-390): the trainer's own
// streams and events stay inside the library, these are for callers that
// schedule their own uploads or load their own kernels, as the reference's
// upload ring (bins/nnue_train/src/trainer_common.rs:1041-1370) and kernel
// module loader (bins/nnue_train/src/kernel_module.rs:55-70) do.  Streams are
// non-blocking and at the default priority.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/tatara_hip.h"
#include "common.hpp"

struct TataraStream {
    hipStream_t s;
    int device;
};

struct TataraEvent {
    hipEvent_t e;
    int device;
};

struct TataraModule {
    hipModule_t m;
    int device;
    std::mutex mu;
    std::unordered_map<std::string, hipFunction_t> functions;  // name -> function, filled on first launch
};

namespace tatara {
namespace {

inline hipStream_t raw(TataraStream* s) { return s ? s->s : nullptr; }

// A code object as hipcc --genco writes it: an ELF image, or a clang offload
// bundle holding one.  Anything else is refused before the loader sees it.
bool looks_like_code_object(const void* image, uint64_t bytes) {
    static const char kBundle[] = "__CLANG_OFFLOAD_BUNDLE__";
    const unsigned char* p = static_cast<const unsigned char*>(image);
    if (bytes >= 4 && p[0] == 0x7f && p[1] == 'E' && p[2] == 'L' && p[3] == 'F') return true;
    return bytes >= sizeof(kBundle) - 1 && std::memcmp(p, kBundle, sizeof(kBundle) - 1) == 0;
}

}  // namespace
}  // namespace tatara

using namespace tatara;

extern "C" {

int32_t tatara_device_occupancy_attributes(int32_t device, int32_t* cu_count, int32_t* max_threads_per_cu) {
    TATARA_REQUIRE(cu_count && max_threads_per_cu, "null output");
    TATARA_HIP(hipSetDevice(device), "hipSetDevice");
    int cus = 0, threads = 0;
    TATARA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device), "hipDeviceGetAttribute");
    TATARA_HIP(hipDeviceGetAttribute(&threads, hipDeviceAttributeMaxThreadsPerMultiProcessor, device),
               "hipDeviceGetAttribute");
    *cu_count = cus;
    *max_threads_per_cu = threads;
    return kOk;
}

int32_t tatara_device_compute_capability(int32_t device, int32_t* major, int32_t* minor) {
    TATARA_REQUIRE(major && minor, "null output");
    int ma = 0, mi = 0;
    TATARA_HIP(hipDeviceGetAttribute(&ma, hipDeviceAttributeComputeCapabilityMajor, device), "hipDeviceGetAttribute");
    TATARA_HIP(hipDeviceGetAttribute(&mi, hipDeviceAttributeComputeCapabilityMinor, device), "hipDeviceGetAttribute");
    *major = ma;
    *minor = mi;
    return kOk;
}

int32_t tatara_stream_create(int32_t device, TataraStream** out) {
    TATARA_REQUIRE(out, "out is null");
    *out = nullptr;
    TATARA_HIP(hipSetDevice(device), "hipSetDevice");
    hipStream_t s = nullptr;
    TATARA_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    *out = new TataraStream{s, device};
    return kOk;
}

int32_t tatara_stream_destroy(TataraStream* stream) {
    if (!stream) return kOk;
    const hipError_t e = hipStreamDestroy(stream->s);
    delete stream;
    TATARA_HIP(e, "hipStreamDestroy");
    return kOk;
}

int32_t tatara_stream_synchronize(TataraStream* stream) {
    TATARA_HIP(hipStreamSynchronize(raw(stream)), "hipStreamSynchronize");
    return kOk;
}

int32_t tatara_stream_wait_event(TataraStream* stream, TataraEvent* event) {
    TATARA_REQUIRE(event, "event is null");
    TATARA_HIP(hipStreamWaitEvent(raw(stream), event->e, 0), "hipStreamWaitEvent");
    return kOk;
}

int32_t tatara_event_create(int32_t device, uint32_t flags, TataraEvent** out) {
    TATARA_REQUIRE(out, "out is null");
    *out = nullptr;
    TATARA_REQUIRE((flags & ~(uint32_t)(TATARA_EVENT_BLOCKING_SYNC | TATARA_EVENT_DISABLE_TIMING)) == 0,
                   "unknown event flags");
    TATARA_HIP(hipSetDevice(device), "hipSetDevice");
    unsigned hf = hipEventDefault;
    if (flags & TATARA_EVENT_BLOCKING_SYNC) hf |= hipEventBlockingSync;
    if (flags & TATARA_EVENT_DISABLE_TIMING) hf |= hipEventDisableTiming;
    hipEvent_t e = nullptr;
    TATARA_HIP(hipEventCreateWithFlags(&e, hf), "hipEventCreateWithFlags");
    *out = new TataraEvent{e, device};
    return kOk;
}

int32_t tatara_event_destroy(TataraEvent* event) {
    if (!event) return kOk;
    const hipError_t e = hipEventDestroy(event->e);
    delete event;
    TATARA_HIP(e, "hipEventDestroy");
    return kOk;
}

int32_t tatara_event_record(TataraEvent* event, TataraStream* stream) {
    TATARA_REQUIRE(event, "event is null");
    TATARA_REQUIRE(!stream || stream->device == event->device, "event and stream are on different devices");
    TATARA_HIP(hipEventRecord(event->e, raw(stream)), "hipEventRecord");
    return kOk;
}

int32_t tatara_event_synchronize(TataraEvent* event) {
    TATARA_REQUIRE(event, "event is null");
    TATARA_HIP(hipEventSynchronize(event->e), "hipEventSynchronize");
    return kOk;
}

int32_t tatara_event_query(TataraEvent* event, int32_t* done) {
    TATARA_REQUIRE(event && done, "null argument");
    const hipError_t e = hipEventQuery(event->e);
    if (e == hipErrorNotReady) {
        *done = 0;
        return kOk;
    }
    TATARA_HIP(e, "hipEventQuery");
    *done = 1;
    return kOk;
}

int32_t tatara_event_elapsed_ms(TataraEvent* start, TataraEvent* end, float* ms) {
    TATARA_REQUIRE(start && end && ms, "null argument");
    TATARA_HIP(hipEventElapsedTime(ms, start->e, end->e), "hipEventElapsedTime");
    return kOk;
}

int32_t tatara_memset_d8_async(void* dst, uint8_t value, uint64_t bytes, TataraStream* stream) {
    if (bytes == 0) return kOk;
    TATARA_REQUIRE(dst, "dst is null");
    TATARA_HIP(hipMemsetD8Async(reinterpret_cast<hipDeviceptr_t>(dst), value, bytes, raw(stream)),
               "hipMemsetD8Async");
    return kOk;
}

int32_t tatara_memcpy_htod_async(void* dst, const void* src, uint64_t bytes, TataraStream* stream) {
    if (bytes == 0) return kOk;
    TATARA_REQUIRE(dst && src, "null pointer");
    TATARA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, raw(stream)), "hipMemcpyAsync H2D");
    return kOk;
}

int32_t tatara_memcpy_dtoh_async(void* dst, const void* src, uint64_t bytes, TataraStream* stream) {
    if (bytes == 0) return kOk;
    TATARA_REQUIRE(dst && src, "null pointer");
    TATARA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, raw(stream)), "hipMemcpyAsync D2H");
    return kOk;
}

int32_t tatara_host_alloc_pinned(uint64_t bytes, void** out) {
    TATARA_REQUIRE(out, "out is null");
    *out = nullptr;
    TATARA_HIP(hipHostMalloc(out, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc");
    return kOk;
}

int32_t tatara_host_free_pinned(void* ptr) {
    if (ptr) TATARA_HIP(hipHostFree(ptr), "hipHostFree");
    return kOk;
}

int32_t tatara_module_load_image(int32_t device, const void* image, uint64_t bytes, TataraModule** out) {
    TATARA_REQUIRE(out, "out is null");
    *out = nullptr;
    TATARA_REQUIRE(image && bytes > 0, "empty image");
    TATARA_REQUIRE(looks_like_code_object(image, bytes), "image is not a code object (ELF or offload bundle)");
    TATARA_HIP(hipSetDevice(device), "hipSetDevice");
    hipModule_t m = nullptr;
    TATARA_HIP(hipModuleLoadData(&m, image), "hipModuleLoadData");
    TataraModule* mod = new TataraModule;
    mod->m = m;
    mod->device = device;
    *out = mod;
    return kOk;
}

int32_t tatara_module_destroy(TataraModule* module) {
    if (!module) return kOk;
    const hipError_t e = hipModuleUnload(module->m);
    delete module;
    TATARA_HIP(e, "hipModuleUnload");
    return kOk;
}

int32_t tatara_module_launch(TataraModule* module, const char* kernel, TataraStream* stream, const uint32_t grid[3],
                             const uint32_t block[3], uint32_t shared_bytes, void** args) {
    TATARA_REQUIRE(module && kernel && grid && block, "null argument");
    TATARA_REQUIRE(!stream || stream->device == module->device, "module and stream are on different devices");
    TATARA_REQUIRE(grid[0] && grid[1] && grid[2] && block[0] && block[1] && block[2], "zero launch dimension");
    TATARA_REQUIRE((uint64_t)block[0] * block[1] * block[2] <= 1024, "more than 1024 threads per block");
    hipFunction_t f = nullptr;
    {
        std::lock_guard<std::mutex> lock(module->mu);
        auto it = module->functions.find(kernel);
        if (it != module->functions.end()) {
            f = it->second;
        } else {
            const hipError_t e = hipModuleGetFunction(&f, module->m, kernel);
            if (e != hipSuccess) return hip_status(e, (std::string("hipModuleGetFunction ") + kernel).c_str());
            module->functions.emplace(kernel, f);
        }
    }
    TATARA_HIP(hipSetDevice(module->device), "hipSetDevice");
    const hipError_t e = hipModuleLaunchKernel(f, grid[0], grid[1], grid[2], block[0], block[1], block[2], shared_bytes,
                                               raw(stream), args, nullptr);
    if (e != hipSuccess) return hip_status(e, (std::string("hipModuleLaunchKernel ") + kernel).c_str());
    return kOk;
}

}  // extern "C"
