// noalloc.hip — sort_isect on device buffers with no allocation (sxh_sort_isect_noalloc).
//
// For callers that cannot allocate device memory (code under stream capture, tight serving loops):
// the inputs and outputs are the caller's device buffers, and everything else the sort needs — its
// histogram/status/error words and the second ping-pong side of the keys and values — lives in the
// file-scope `scratch` array below, sized for at most kNoAllocMaxKeys keys. Each device the library
// runs on holds its own copy of the array until the process ends. The sort itself is the onesweep
// radix sort of sort_isect (k_sort.hip); it clears the words that must start at zero at the start of
// every call, so the array's left-over contents never matter. Calls on one device share the array, so
// a per-device mutex is held across each call: calls from several host threads are serialised, not
// raced (work the caller queued on other streams that reads the outputs must wait for the return).
#include <hip/hip_runtime.h>

#include <algorithm>
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
std::mutex g_call_mu[kMaxDevices];  // held across a call: one call at a time uses a device's array

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

// Device memory of `device` (not host, not another device's) whose allocation holds `bytes` from p on:
// the kernels read or write all of them.
void need_device(const void* p, size_t bytes, int device, const char* name) {
    hipPointerAttribute_t attr{};
    const hipError_t e = hipPointerGetAttributes(&attr, p);
    (void)hipGetLastError();  // an unknown host pointer leaves an error behind; it is reported below
    if (e != hipSuccess || attr.type != hipMemoryTypeDevice || attr.device != device)
        sxh::invalid("sort_isect_noalloc", std::string(name) + " is not device memory of the backend's device");
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) != hipSuccess || !base) {
        (void)hipGetLastError();
        sxh::invalid("sort_isect_noalloc", std::string(name) + ": the allocation holding it is unknown");
    }
    const size_t off = static_cast<size_t>(static_cast<const char*>(p) - static_cast<const char*>(base));
    if (off > size || size - off < bytes)
        sxh::invalid("sort_isect_noalloc", std::string(name) + " holds fewer than n elements (" +
                                               std::to_string(size - std::min(off, size)) + " bytes from it, " +
                                               std::to_string(bytes) + " needed)");
}

bool overlap(const void* a, size_t na, const void* b, size_t nb) {
    const auto x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + nb && y < x + na;
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
        const size_t nk = sizeof(uint64_t) * static_cast<size_t>(n), nv = sizeof(int32_t) * static_cast<size_t>(n);
        // the outputs are written while the inputs are read: no byte of an output may lie in another buffer
        if (overlap(keys_sorted, nk, keys, nk) || overlap(keys_sorted, nk, values, nv) ||
            overlap(values_sorted, nv, keys, nk) || overlap(values_sorted, nv, values, nv))
            invalid(what, "outputs must not alias the inputs");
        if (overlap(keys_sorted, nk, values_sorted, nv)) invalid(what, "keys_sorted and values_sorted overlap");
        SXH_HIP(hipSetDevice(b->device));
        need_device(keys, nk, b->device, "keys");
        need_device(values, nv, b->device, "values");
        need_device(keys_sorted, nk, b->device, "keys_sorted");
        need_device(values_sorted, nv, b->device, "values_sorted");
        if (b->device < 0 || b->device >= kMaxDevices) invalid(what, "device ordinal out of range");
        std::lock_guard<std::mutex> call_lock(g_call_mu[b->device]);
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
