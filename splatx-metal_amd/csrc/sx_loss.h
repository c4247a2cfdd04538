// sx_loss.h — device code of the training step's host words: system-scope stores into mapped host
// memory, and the step's loss reduced by one wave from the loss kernels' per-block partial sums.
#pragma once

#include <hip/hip_runtime.h>

#include "sx_step.h"

namespace sxk {

// a store into mapped host memory, at system scope (no GPU cache keeps it from the host)
template <class T>
__device__ __forceinline__ void store_host(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Sum of p[0, n) by one 64-lane wave in a fixed order: lane l adds p[l], p[l + 64], ... in ascending order
// (sixteen loads in flight: a single wave's sum is bound by its round trips to memory), then the 64 lane
// sums are added in a fixed butterfly, after which every lane holds the same total (a + b and b + a are
// the same double).
__device__ __forceinline__ double wave_sum_fixed(const double* __restrict__ p, int n) {
    constexpr int kBatch = 16;
    const int lane = threadIdx.x & 63;
    double acc = 0.0;
    int k = lane;
    for (; k + (kBatch - 1) * 64 < n; k += kBatch * 64) {
        double v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; j++) v[j] = p[k + j * 64];
#pragma unroll
        for (int j = 0; j < kBatch; j++) acc += v[j];
    }
    for (; k < n; k += 64) acc += p[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    return acc;
}

// The step's loss by one whole wave: loss = (1-lam) * float(l1_sum / n_px) + lam * (1 - float(ssim_sum /
// M)) (or the L1 alone) into L.out[0]; with L.rb.host set, lane 0 also stores the loss and rb's words into
// mapped host memory, then rb.seq into *rb.seq_host (release order).
__device__ __forceinline__ void loss_final_wave(const StepLoss& L) {
    const double l1s = wave_sum_fixed(L.l1p, L.n_l1);
    const double sss = L.use_ssim ? wave_sum_fixed(L.ssp, L.n_ss) : 0.0;
    if ((threadIdx.x & 63) == 0) {
        const float l1 = static_cast<float>(l1s / L.n_px);
        const float loss =
            L.use_ssim ? (1.0f - L.lam) * l1 + L.lam * (1.0f - static_cast<float>(sss / L.M)) : l1;
        L.out[0] = loss;
        if (L.rb.host) {
            store_host(&L.rb.host[0], __float_as_uint(loss));
            store_host(&L.rb.host[1], *L.rb.sort_err);
            store_host(&L.rb.host[2], *L.rb.max_tile);
            store_host(&L.rb.host[3], L.rb.long_count ? static_cast<uint32_t>(*L.rb.long_count) : 0u);
            __hip_atomic_store(L.rb.seq_host, L.rb.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

}  // namespace sxk
