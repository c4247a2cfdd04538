// sx_io.h — launchers of the format kernels (k_io.hip), used by io.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sx_fmath.h"
#include "sx_step.h"

namespace sxk {

struct Dims6 {
    int d[6];
};

// checkpoint payload encodings
constexpr int kCkptF32 = 0;      // verbatim
constexpr int kCkptF16 = 1;      // IEEE half, RNE, clamped to +-65504
constexpr int kCkptF16Sqrt = 2;  // half of sqrt(x) (exp_avg_sq), squared back on load

// keep[i] = row i passes filter_cloud_for_export; removed[0] += non-finite rows, removed[1] += low-opacity rows
void export_flags(const Arena& A, const Dims6& dims, int count, float min_opacity, int32_t* keep,
                  unsigned long long* removed, hipStream_t s);
// list[cum[i]-1] = i for kept rows (cum = inclusive int64 scan of keep)
void export_list(const int32_t* keep, const int64_t* cum, int count, int32_t* list, hipStream_t s);
// rows list[0 .. n) of one SoA group (R rows per column) -> row-major [n, dim]
void gather_rows(const float* soa, int R, int dim, const int32_t* list, int64_t n, float* out, hipStream_t s);
// sq_err_blocks() f64 partial sums of (clamp(a, 0, 1) - b)^2 over n floats
int sq_err_blocks();
void sq_err(const float* a, const float* b, int64_t n, double* partials, hipStream_t s);
// floats per PLY row with Kw f_rest coefficients per channel
int export_row_floats(int Kw);
// PLY rows [row0, row0 + rows) of the kept list, row-major floats
void export_pack(const Arena& A, int K, int Kw, const int32_t* list, int64_t row0, int64_t rows, float* out,
                 hipStream_t s);
// rows [row0, row0 + rows) of one SoA group (stride R, dim columns) <-> row-major file layout
void ckpt_pack(const float* soa, int R, int dim, int64_t row0, int64_t rows, int mode, void* out, hipStream_t s);
void ckpt_unpack(const void* in, int mode, float* soa, int R, int dim, int64_t row0, int64_t rows, hipStream_t s);
void ckpt_pair_zero(float* m, const float* v, int R, int dim, int n, hipStream_t s);
void zero_tail(float* soa, int R, int dim, int n, hipStream_t s);
// render [n_px, 3] f32 -> RGBA8 words (r | g << 8 | b << 16 | 255 << 24)
void rgba8(const float* rgb, int64_t n_px, uint32_t* out, hipStream_t s);

}  // namespace sxk
