// hip_kernel_backend.h — splatx::KernelBackend over the splatx-hip C ABI.
//
// This file is the reference-side half of the boundary: it is compiled inside the reference's
// SplatXCore tree (it includes the reference's own "splatx/KernelBackend.h") and linked against
// libsplatx_hip.so. It replaces make_metal_backend (MetalBackend.h:48-57) for callers such as
// TrainC.cpp:552 and the tests' shared backend; Trainer (Trainer.cpp:668) takes the result unchanged.
#pragma once

#include <cstdint>
#include <memory>
#include <random>
#include <vector>

#include "splatx/KernelBackend.h"

namespace splatx {

struct HipBackendDesc {
    int device_ordinal = 0;
};

// Creates the HIP backend on one GPU. Failure (no device, library/ABI mismatch) raises
// std::runtime_error, as make_metal_backend does (MetalBackend.h:43-46).
std::unique_ptr<KernelBackend> make_hip_backend(const HipBackendDesc& desc = {});

// MCMC refine on the device arena of a resident executor made by make_hip_backend: what
// Trainer::step_resident does on a refine step (Trainer.cpp:957-967: mcmc_refine, then
// mcmc_inject_noise over the new count) without sync_host_for_mutation's download and the next
// step's re-upload (Trainer.cpp:911-914). `rng` is the Trainer's multinomial engine (mcmc_rng_);
// it is advanced by exactly the draws the host path makes. Errors as Trainer::mcmc_refine.
struct HipMcmcRefineInputs {
    int64_t count = 0;                        // cloud_.count
    int64_t cap_max = 0;                      // McmcOptions::cap_max
    float min_opacity = 0.005f;               // McmcOptions::min_opacity
    const std::vector<float>* binoms = nullptr;  // Trainer::binoms_ (make_binoms_lut(51))
    bool inject_noise = false;                // the post-refine noise (Trainer.cpp:966)
    uint64_t noise_seed = 0, noise_offset = 0;
    float noise_scale = 0.f;
};
struct HipMcmcRefineResult {
    int64_t count = 0;  // the new cloud_.count
    std::vector<int64_t> relocated_dead, relocation_src, added_src;  // Trainer::McmcRefineResult
};
HipMcmcRefineResult hip_mcmc_refine(TrainStepExecutor& exec, std::mt19937_64& rng, const HipMcmcRefineInputs& in);

} // namespace splatx

struct sxh_executor;

namespace splatx {

// The C handle of a resident executor made by make_hip_backend, for the device-side data formats
// of include/splatx_hip.h (sxh_exec_export_ply, sxh_exec_save_checkpoint, sxh_exec_load_checkpoint)
// that read or write its arena in place; std::invalid_argument for any other executor.
sxh_executor* hip_executor_handle(TrainStepExecutor& exec);

} // namespace splatx
