// sx_common.h — constants and small helpers shared by the gfx950 kernels, the host runtime and
// the CPU oracle. The numeric values are fixed by the reference step
// (Sources/SplatXKernelSrc/KernelConstants.h:17-37, gsplat Common.h) and must stay identical.
#pragma once

#include <stdint.h>
#include "sx_fmath.h"

namespace sx {

// Rasterizer / projection thresholds (KernelConstants.h:17-22)
constexpr float kAlphaThreshold = 1.f / 255.f;
constexpr float kGaussianExtend = 3.33f;
constexpr float kMinCompensation = 0.005f;
constexpr float kMaxAlpha = 0.99f;
constexpr float kTransmittanceThreshold = 1e-4f;
constexpr float kMinOneMinusAlpha = 1e-6f;

// SSIM (KernelConstants.h:25-37): C1=(0.01)^2, C2=(0.03)^2, 11-tap sigma=1.5 window normalized in
// f64 and cast to f32 (the same taps as fixtures/ssim_basic meta.json window_taps_f32).
constexpr float kSsimC1 = 1e-4f;
constexpr float kSsimC2 = 9e-4f;
constexpr int kSsimWin = 11;

// Tile geometry of the rasterizer (KernelConstants.h:72-74).
constexpr int kTile = 16;
constexpr int kTilePixels = kTile * kTile;

// MCMC (strategy/ops.py defaults cited at KernelBackend.h:252-274).
constexpr int kMcmcNMax = 51;

// bits_for_count (CpuKernels.h:69-74): bits needed to index 0..count-1.
SX_HD inline uint32_t bits_for_count(int64_t count) {
    if (count <= 1) return 0u;
    uint32_t bits = 0;
    for (uint64_t v = static_cast<uint64_t>(count) - 1u; v != 0; v >>= 1) bits++;
    return bits;
}

} // namespace sx

// The SSIM window as a macro list so host code and device constant memory share one definition.
#define SX_SSIM_TAPS                                                                           \
    {0.001028380123898387f, 0.0075987582094967365f, 0.036000773310661316f,                    \
     0.10936068743467331f, 0.21300554275512695f, 0.26601171493530273f, 0.21300554275512695f,   \
     0.10936068743467331f, 0.036000773310661316f, 0.0075987582094967365f,                      \
     0.001028380123898387f}
