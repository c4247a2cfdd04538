// sx_philox.h — Philox4x32-10 counter-based generator and the Box-Muller transform, shared by
// the gfx950 kernels and the CPU oracle.
//
// Algorithm: Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As Easy as 1, 2, 3" (SC'11),
// section 3.3 — multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key increments 0x9E3779B9 / 0xBB67AE85,
// ten rounds. Stream mapping of the reference (RngPhilox.h:50-98, CpuKernels.cpp:863-900):
// thread t produces outputs [4t, 4t+4) from counter (t, offset_lo, offset_hi, 0) and key
// (seed_lo, seed_hi); uniform u = (float(x) + 1) * 2^-32 in (0, 1]; normals by Box-Muller
// r = sqrt(-2 ln u1), theta = 2*pi*u2 (float), z0 = r cos theta, z1 = r sin theta.
// Integer and uniform stages are bit-exact everywhere; the transcendentals use sx_fmath.h so the
// normals are bit-identical between host and device as well.
#pragma once

#include <stdint.h>
#include "sx_fmath.h"

namespace sx {

struct Philox4 {
    uint32_t v[4];
};

SX_HD inline Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                   uint32_t k1) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
#endif
    for (int r = 0; r < 10; ++r) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
        const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
        const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
        const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
        const uint32_t n0 = hi1 ^ c1 ^ k0;
        const uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
    }
    Philox4 out;
    out.v[0] = c0;
    out.v[1] = c1;
    out.v[2] = c2;
    out.v[3] = c3;
    return out;
}

SX_HD inline float u32_to_uniform(uint32_t x) {
    return (static_cast<float>(x) + 1.0f) * (1.0f / 4294967296.0f);
}

SX_HD inline void box_muller(uint32_t x0, uint32_t x1, float* z0, float* z1) {
    const float u1 = u32_to_uniform(x0);
    const float u2 = u32_to_uniform(x1);
    const float r = SX_SQRTF(-2.0f * sxm::logf_(u1));
    const float theta = 6.28318530717958647692f * u2;
    float s, c;
    sxm::sincosf_(theta, &s, &c);
    *z0 = r * c;
    *z1 = r * s;
}

// The four normals of Philox block t.
SX_HD inline void philox_normals4(uint32_t t, uint64_t seed, uint64_t offset, float out[4]) {
    const Philox4 r = philox4x32_10(t, static_cast<uint32_t>(offset),
                                    static_cast<uint32_t>(offset >> 32), 0u,
                                    static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32));
    box_muller(r.v[0], r.v[1], &out[0], &out[1]);
    box_muller(r.v[2], r.v[3], &out[2], &out[3]);
}

} // namespace sx
