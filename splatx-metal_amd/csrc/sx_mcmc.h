// sx_mcmc.h — launchers of the device MCMC refine kernels (k_mcmc.hip), used by refine.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sx_step.h"

namespace sxk {

// error bits the refine kernels OR into a device word
constexpr uint32_t kMcErrWeights = 1u;  // a NaN weight (the multinomial's "weights must be >= 0 and finite")
constexpr uint32_t kMcErrLogit = 2u;    // a new opacity outside (0,1) (logit_f32's domain)
constexpr uint32_t kMcErrScale = 4u;    // a non-positive new scale

// p[0, n) = v (a kernel, so that a captured stream records no memset node)
void fill_u32(uint32_t* p, uint32_t v, int64_t n, hipStream_t s);
// op_act[i] = sigmoid(logits[i]); dead[i] = op_act[i] <= min_opacity (dead may be null)
void mc_activate(const float* logits, int n, float min_opacity, float* op_act, int32_t* dead, uint32_t* err,
                 hipStream_t s);
// stable dead / alive lists from cum = inclusive int64 scan of dead
void mc_compact(const int32_t* dead, const int64_t* cum, int n, int32_t* dead_list, int32_t* alive_list,
                hipStream_t s);
// cdf[i] = the left-to-right f64 running sum of w[gather[i]] (w[i] when gather is null); total = the
// sum (0 when n == 0); scratch: mc_cdf_scratch_bytes(n) bytes, 8-byte aligned
size_t mc_cdf_scratch_bytes(int64_t n);
void mc_cdf(const float* w, const int32_t* gather, int64_t n, double* cdf, double* total, uint32_t* err,
            void* scratch, hipStream_t s);
// state: 312 words + the position word; raw = the next n_out untempered words
void mc_mt_gen(uint64_t* state, int64_t n_out, uint64_t* raw, hipStream_t s);
// multinomial draws over cdf[0, n_w): sampled[j] = gather[idx] (idx when gather is null), counts[src]++
void mc_search(const uint64_t* raw, int64_t n_draw, const double* cdf, int64_t n_w, const double* total,
               const int32_t* gather, int32_t* sampled, uint32_t* counts, hipStream_t s);
// Eq.9 of every draw with ratio = min(counts[src] + 1, n_max); back-converted to logit / log scale
void mc_reloc(const int32_t* sampled, int n_draw, const uint32_t* counts, const float* op_act,
              const float* log_scales, int rows, const float* binoms, int n_max, float min_opacity,
              float* new_logit, float* new_log_scale, uint32_t* err, hipStream_t s);
void mc_apply(const int32_t* sampled, int n_draw, const float* new_logit, const float* new_log_scale, float* logits,
              float* log_scales, int rows, hipStream_t s);
// every parameter column: row dst (dst_list[j], or dst_base + j) <- row src_list[j]
void mc_copy_rows(const Arena& A, const int* dims, const int32_t* dst_list, int dst_base, const int32_t* src_list,
                  int n, hipStream_t s);
// every moment column of rows row_list[j] (or row_base + j) <- 0
void mc_zero_rows(const Arena& A, const int* dims, const int32_t* row_list, int row_base, int n, hipStream_t s);
// tempered words: out[i] = the engine's output for raw[i]
void mc_temper(const uint64_t* raw, int64_t n, uint64_t* out, hipStream_t s);
void mc_noise(const Arena& A, int n, uint64_t seed, uint64_t offset, float noise_scale, hipStream_t s);

}  // namespace sxk
