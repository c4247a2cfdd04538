// hip_kernel_backend.h — splatx::KernelBackend over the splatx-hip C ABI.
//
// This file is the reference-side half of the boundary: it is compiled inside the reference's
// SplatXCore tree (it includes the reference's own "splatx/KernelBackend.h") and linked against
// libsplatx_hip.so. It replaces make_metal_backend (MetalBackend.h:48-57) for callers such as
// TrainC.cpp:552 and the tests' shared backend; Trainer (Trainer.cpp:668) takes the result unchanged.
#pragma once

#include <memory>

#include "splatx/KernelBackend.h"

namespace splatx {

struct HipBackendDesc {
    int device_ordinal = 0;
};

// Creates the HIP backend on one GPU. Failure (no device, library/ABI mismatch) raises
// std::runtime_error, as make_metal_backend does (MetalBackend.h:43-46).
std::unique_ptr<KernelBackend> make_hip_backend(const HipBackendDesc& desc = {});

} // namespace splatx
