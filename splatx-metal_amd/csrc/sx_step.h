// sx_step.h — launchers of the fused resident-step kernels (k_step.hip).
//
// Device arena layout (MI355X-first): every parameter group and both Adam moments are stored
// coefficient-major (SoA), element j of row i at [j * rows + i], so each per-Gaussian thread's
// reads and writes are fully coalesced 256-byte wave accesses. The host sync format of the
// reference (row-major [rows][dim], KernelBackend.h:348-359) is converted on upload/download.
// Per-Gaussian intermediates are packed in three float4 records:
//   splat[3i+0] = {mean2d.x, mean2d.y, opacity used by isect/raster, depth}
//   splat[3i+1] = {conic a, b, c, compensation}
//   splat[3i+2] = {r, g, b, meta bits: 1 = visible, 2/4/8 = relu mask of r/g/b}
//   grads[3i+0] = {v_mean2d.x, v_mean2d.y, v_opacity, 0}, grads[3i+1] = {v_conic a,b,c, 0},
//   grads[3i+2] = {v_rgb, 0} (raster backward accumulates here atomically)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sxk {

struct Arena {
    float* p[6];
    float* m[6];
    float* v[6];
    int rows;  // arena stride
};

struct StepConst {
    float vm[16];
    float K[9];
    int width, height;
    int count;
    int n_coeffs;  // (sh_degree+1)^2 of the arena
    uint32_t degree;
    float eps2d, near_plane, far_plane, radius_clip;
    int aa;
    int accutile;
    int tile_width, tile_height;
    uint32_t tile_n_bits;
    float lr[6];
    float b1, b2, eps;
    float opacity_reg_w, scale_reg_w;
    int inject_noise;
    uint64_t noise_seed, noise_offset;
    float noise_scale;
};

// vis_part: 4 u32 per block (visible count, tile count, count of Gaussians with tiles, 0); out_vis (5
// u64): {visible count, intersections, Gaussians with tiles, intersections, overflow}, where overflow =
// intersections > isect_cap and then words 2 and 3 read 0 (the counts the rest of the step reads, so
// that it does nothing); block_base: per block, the intersections and the Gaussians with tiles of the
// blocks before it (2 u64)
// host_counts (mapped host memory, may be null) receives words 0 and 1 of out_vis, then `seq` in its
// word 4 (release order: a host that reads seq there reads the counts).
// What a training step's backward starts from, set by its preprocess (null touched: nothing): the
// rows' touched flags cleared, the gather's long-range queue emptied and the backward's stamp advanced
// (never to 0: zeroed entries hold 0).
struct StepClear {
    uint8_t* touched = nullptr;
    uint32_t* stamp = nullptr;
    int32_t* long_count = nullptr;
    int32_t* long_prev = nullptr;  // (when set) receives the previous step's long-range count first
};
// row_int (when set): the arena is in spatial order, row_int[o] the internal row of original row o; the
// tile counts are then also written in original order into tiles_o, and the per-block counts the block
// scan reads are taken again over original rows (for the compaction, which then reads tiles_o).
void step_preprocess(const StepConst& c, const Arena& A, float4* splats, int32_t* radii, int32_t* tiles,
                     uint32_t* vis_part, unsigned long long* out_vis, unsigned long long* block_base,
                     unsigned long long isect_cap, unsigned long long* host_counts, unsigned long long seq,
                     const StepClear& clr, hipStream_t s, const int32_t* row_int = nullptr,
                     int32_t* tiles_o = nullptr);
// number of blocks of step_preprocess
int step_preprocess_blocks(int64_t count);
// The Gaussians with tiles in index order (list[j], j below out_vis[2]) and (cum set) cum[j], the
// inclusive sum of their tile counts: the positions of the index-first emit. row_int (the arena in
// spatial order): the list runs in original order and holds internal rows, and `tiles` must be the tile
// counts in original order (the preprocess's tiles_o).
void step_emit_compact(const StepConst& c, const int32_t* tiles, const unsigned long long* block_base, int32_t* list,
                       int64_t* cum, hipStream_t s, const int32_t* row_int = nullptr);
// depth-first intersections: depth keys of the listed Gaussians (values = index) for a stable 32-bit
// sort of *n_list keys; then, over that order, each Gaussian's tile ids at [cum[j-1], cum[j]) (cum =
// inclusive scan of the tile counts gathered through the order); after a stable sort of the tile ids,
// offsets[t] = lower bound of t. Index-first: order = the list itself, cum from step_emit_compact,
// and the depth order within each tile comes after the tile sort (tile_depth_sort), which reads each
// entry's depth bits from edepth (written by the emit when set). The emit covers positions j below
// *n_pos.
void step_depth_keys(const StepConst& c, const float4* splats, const int32_t* list, const unsigned long long* n_list,
                     uint32_t* keys, int32_t* vals, hipStream_t s);
void step_emit_sorted(const StepConst& c, const float4* splats, const int32_t* radii, const int32_t* order,
                      const int64_t* cum, const unsigned long long* n_pos, uint16_t* keys, int32_t* vals,
                      hipStream_t s, uint32_t* edepth = nullptr);
void step_emit_sorted(const StepConst& c, const float4* splats, const int32_t* radii, const int32_t* order,
                      const int64_t* cum, const unsigned long long* n_pos, uint32_t* keys, int32_t* vals,
                      hipStream_t s, uint32_t* edepth = nullptr);
// Index first in one launch: step_emit_compact (without row_int) and step_emit_sorted over its list
// (order = the list): each workgroup compacts the 256 rows of one preprocess block, writes their list
// entries and offsets (list, cum: for the gather) and emits their tile ids; *n_pos (the count of
// Gaussians with tiles, 0 after an overflow) bounds the positions as in step_emit_sorted.
void step_emit_compact_sorted(const StepConst& c, const float4* splats, const int32_t* radii, const int32_t* tiles,
                              const unsigned long long* block_base, int32_t* list, int64_t* cum,
                              const unsigned long long* n_pos, uint16_t* keys, int32_t* vals, hipStream_t s,
                              uint32_t* edepth);
void step_emit_compact_sorted(const StepConst& c, const float4* splats, const int32_t* radii, const int32_t* tiles,
                              const unsigned long long* block_base, int32_t* list, int64_t* cum,
                              const unsigned long long* n_pos, uint32_t* keys, int32_t* vals, hipStream_t s,
                              uint32_t* edepth);
// n_dev: the key count on the device, read instead of n
void step_tile_offsets(const uint16_t* keys, int64_t n, int n_tiles, int32_t* offsets, hipStream_t s,
                       const int64_t* n_dev = nullptr);
void step_tile_offsets(const uint32_t* keys, int64_t n, int n_tiles, int32_t* offsets, hipStream_t s,
                       const int64_t* n_dev = nullptr);
// The words a step reports to the host, stored straight into mapped host memory (host: 4 u32, the loss
// bits, the sort's error flag, the largest tile's entry count, the gather's long-range count (0 when
// long_count is null)) instead of one copy each, then `seq` into *seq_host (release order: a host that
// reads seq there reads the words). Null host: nothing is stored.
struct StepReadback {
    const uint32_t* sort_err = nullptr;
    const uint32_t* max_tile = nullptr;
    const int32_t* long_count = nullptr;
    uint32_t* host = nullptr;
    unsigned long long* seq_host = nullptr;
    unsigned long long seq = 0;
};
// A training step's loss, reduced by one wave (the gather's first workgroup) from the per-block partial
// sums (fixed order): loss = (1-lam) * float(l1_sum / n_px) + lam * (1 - float(ssim_sum / M)) (or the L1
// alone) into out[0]; with rb.host set, the loss and rb's words also go to the host. Null out: none.
struct StepLoss {
    const double* l1p = nullptr;
    int n_l1 = 0;
    const double* ssp = nullptr;
    int n_ss = 0;
    double n_px = 1.0, M = 1.0;
    float lam = 0.0f;
    int use_ssim = 0;
    float* out = nullptr;
    StepReadback rb{};
};
// The parameter update of a training step with constants c. skip, sort_err (when set): device words;
// either nonzero leaves the arena untouched (the overflow word of out_vis, the tile sort's error word).
void step_postprocess(const StepConst& c, const Arena& A, const float4* splats, const float4* grads,
                      const uint8_t* touched, hipStream_t s, const unsigned long long* skip = nullptr,
                      const uint32_t* sort_err = nullptr, const int32_t* row_orig = nullptr);
// A training step's parameter update (constants cu, its skip and sort error words) and the next step's
// preprocess (constants c, the same rows; then the block scan, as step_preprocess) in one pass over the
// arena: the same results as step_postprocess followed by step_preprocess. touched: the update's
// touched flags, cleared for the new step when clr.touched (which must be the same buffer) is set.
void step_update_preprocess(const StepConst& cu, const StepConst& c, const Arena& A, float4* splats, const float4* grads,
                            uint8_t* touched, const unsigned long long* skip, const uint32_t* sort_err, int32_t* radii,
                            int32_t* tiles, uint32_t* vis_part, unsigned long long* out_vis,
                            unsigned long long* block_base, unsigned long long isect_cap, unsigned long long* host_counts,
                            unsigned long long seq, const StepClear& clr, hipStream_t s,
                            const int32_t* row_orig = nullptr, const int32_t* row_int = nullptr,
                            int32_t* tiles_o = nullptr);
// The arena's spatial order (row_orig[k]: the original row of internal row k; row_int its inverse;
// nothing is reordered past the live rows [0, count)). arena_morton_keys: keys[i] = the 30-bit Morton
// code of row i's mean in the means' bounding box, vals[i] = i (scratch: arena_morton_scratch_floats).
// arena_permute_rows: internal row k of every parameter and moment column takes row src[k] (tmp:
// 45 * count floats at least). perm_maps: the maps of src read as internal row k <- original row src[k].
void arena_morton_keys(const Arena& A, int count, float* scratch, uint32_t* keys, int32_t* vals, hipStream_t s);
size_t arena_morton_scratch_floats(int count);
void arena_permute_rows(const Arena& A, const int dims[6], int count, const int32_t* src, float* tmp, hipStream_t s);
void perm_maps(const int32_t* src, int count, int32_t* row_orig, int32_t* row_int, hipStream_t s);
// L1 gradient without SSIM: v_render = sign(render - gt) / n, per-block f64 sums of |render - gt|.
void step_l1_grad(const float* render, const float* gt, int64_t n, float* v_render, double* partials,
                  int n_blocks, hipStream_t s);
int step_l1_blocks(int64_t n);
// SSIM backward fused with the L1 gradient: v_render = w_l1 * sign(d)/n + G*(...), plus |d| sums.
void step_ssim_bwd_l1(const float* render, const float* gt, const float* cmu, const float* csg,
                      const float* ccr, int H, int W, float G, float w_l1, float g_l1, float* v_render,
                      double* l1_partials, hipStream_t s);
int step_ssim_bwd_blocks(int H, int W);
// *word = value, by a one-thread kernel (a graph-capturable store; no memset node)
void step_set_word(uint32_t* word, uint32_t value, hipStream_t s);
// rb's words to the host without a loss (the loss word is 0): the forward-only step
void step_readback(const StepReadback& rb, hipStream_t s);
void aos_to_soa(const float* aos, float* soa, int rows, int dim, int stride, hipStream_t s);
void soa_to_aos(const float* soa, float* aos, int rows, int dim, int stride, hipStream_t s);

} // namespace sxk
