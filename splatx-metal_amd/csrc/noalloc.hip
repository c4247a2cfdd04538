// noalloc.hip — sort_isect on device buffers with no allocation (sxh_sort_isect_noalloc).
//
// For callers that cannot allocate device memory (code under stream capture, tight serving loops):
// the inputs and outputs are the caller's device buffers, and everything else the sort needs — its
// histogram/status/error words and the second ping-pong side of the keys and values — lives in the
// file-scope `scratch` array below, sized for at most kNoAllocMaxKeys keys. Each device the library
// runs on holds its own copy of the array until the process ends. The sort itself is the onesweep
// radix sort of sort_isect (k_sort.hip); it clears the words that must start at zero at the start of
// every call, so the array's left-over contents never matter. Calls that overlap on one device share
// the array and race: the entry point is for one caller at a time per device.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>

#include "sx_host.h"
#include "sx_kernels.h"

namespace {

constexpr int64_t kNoAllocMaxKeys = int64_t{1} << 21;  // 2,097,152 keys
constexpr size_t kSortRegion = size_t{2} << 20;        // the sort's words for kNoAllocMaxKeys keys (1.02 MiB used)
constexpr size_t kKeysRegion = sizeof(uint64_t) * kNoAllocMaxKeys;
constexpr size_t kValsRegion = sizeof(int32_t) * kNoAllocMaxKeys;
constexpr size_t kScratchBytes = kSortRegion + kKeysRegion + kValsRegion;  // 26 MiB

__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};  // the device address of `scratch`, per device

}  // namespace

namespace sxh {

// Resolves the device address of `scratch` on `device`, which must be the current device; once per
// device (the library's init call, sxh_backend_create, runs it).
void noalloc_init(int device) {
    if (device < 0 || device >= kMaxDevices)
        throw std::runtime_error("sort_isect_noalloc: device ordinal " + std::to_string(device) + " out of range");
    if (sxk::sort_scratch_bytes(kNoAllocMaxKeys) > kSortRegion)
        throw std::runtime_error("sort_isect_noalloc: sort scratch region too small");
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[device]) return;
    void* p = nullptr;
    SXH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) throw std::runtime_error("sort_isect_noalloc: hipGetSymbolAddress returned a null address");
    g_ptr[device] = p;
}

}  // namespace sxh

namespace {

void* scratch_of(int device) {
    std::lock_guard<std::mutex> lock(g_mu);
    return (device >= 0 && device < kMaxDevices) ? g_ptr[device] : nullptr;
}

// Device memory of `device` (not host, not another device's): the kernels dereference it.
void need_device(const void* p, int device, const char* name) {
    hipPointerAttribute_t attr{};
    const hipError_t e = hipPointerGetAttributes(&attr, p);
    (void)hipGetLastError();  // an unknown host pointer leaves an error behind; it is reported below
    if (e != hipSuccess || attr.type != hipMemoryTypeDevice || attr.device != device)
        sxh::invalid("sort_isect_noalloc", std::string(name) + " is not device memory of the backend's device");
}

}  // namespace

using namespace sxh;

extern "C" int32_t sxh_sort_isect_noalloc(sxh_backend* b, const uint64_t* keys, const int32_t* values, int64_t n,
                                          uint32_t key_n_bits, uint64_t* keys_sorted, int32_t* values_sorted) {
    return guarded([&] {
        const char* what = "sort_isect_noalloc";
        sxh_sort_inputs in{keys, values, n, key_n_bits};
        validate_sort(in, what);
        if (n > kNoAllocMaxKeys)
            invalid(what, "n = " + std::to_string(n) + " exceeds the scratch capacity of " +
                              std::to_string(kNoAllocMaxKeys) + " keys");
        if (!b) invalid(what, "null backend");
        if (n == 0) return;
        if (!keys_sorted || !values_sorted) invalid(what, "null keys_sorted/values_sorted");
        if (static_cast<const void*>(keys_sorted) == keys || static_cast<const void*>(values_sorted) == values)
            invalid(what, "outputs must not alias the inputs");
        SXH_HIP(hipSetDevice(b->device));
        need_device(keys, b->device, "keys");
        need_device(values, b->device, "values");
        need_device(keys_sorted, b->device, "keys_sorted");
        need_device(values_sorted, b->device, "values_sorted");
        unsigned char* base = static_cast<unsigned char*>(scratch_of(b->device));
        if (!base) throw std::runtime_error("sort_isect_noalloc: scratch not initialised on this device");
        auto* keys_tmp = reinterpret_cast<uint64_t*>(base + kSortRegion);
        auto* vals_tmp = reinterpret_cast<int32_t*>(base + kSortRegion + kKeysRegion);
        hipStream_t s = b->stream;
        sxk::radix_sort_into(keys, values, keys_sorted, values_sorted, keys_tmp, vals_tmp, n, key_n_bits, base, s);
        SXH_HIP(hipGetLastError());
        SXH_HIP(hipMemcpyAsync(b->pinned_word, sxk::sort_error_flag(base), 4, hipMemcpyDeviceToHost, s));
        SXH_HIP(hipStreamSynchronize(s));
        if (*b->pinned_word) throw std::runtime_error("sort_isect_noalloc: radix sort look-back did not complete");
    });
}
