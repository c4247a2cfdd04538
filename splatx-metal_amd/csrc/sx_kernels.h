// sx_kernels.h — host-side launchers of the gfx950 kernels (one stream argument each).
// Every pointer is a device pointer. Launchers perform no allocation and no synchronization.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sxk {

// ---- elementwise / Adam -------------------------------------------------------------------
void adam(float* param, const float* grad, float* m, float* v, const uint8_t* valid, int64_t n_elems,
          int64_t D, float lr, float b1, float b2, float eps, hipStream_t s);

// ---- projection ---------------------------------------------------------------------------
struct ProjArgs {
    const float* means;
    const float* covars;   // [N,6] or null
    const float* quats;    // [N,4]
    const float* scales;   // [N,3]
    const float* opacities;
    const float* viewmats; // [C,16]
    const float* Ks;       // [C,9]
    int N, C, width, height;
    float eps2d, near_plane, far_plane, radius_clip;
    int calc_comp;
};
void projection_fwd(const ProjArgs& a, int32_t* radii, float* means2d, float* depths, float* conics,
                    float* comps, hipStream_t s);
struct ProjBwdArgs {
    const int32_t* radii;
    const float* conics;
    const float* comps;
    const float* v_means2d;
    const float* v_depths;
    const float* v_conics;
    const float* v_comps;  // or null
    int viewmats_grad;
};
// v_* outputs must be zeroed by the caller (accumulated atomically when C > 1).
void projection_bwd(const ProjArgs& a, const ProjBwdArgs& g, float* v_means, float* v_covars,
                    float* v_quats, float* v_scales, float* v_viewmats, hipStream_t s);

// ---- SH -------------------------------------------------------------------------------------
void sh_fwd(const float* dirs, const float* coeffs, const uint8_t* masks, uint32_t degree, int B, int N,
            int K, int D, float* colors, hipStream_t s);
// v_coeffs / v_dirs zeroed by the caller.
void sh_bwd(const float* dirs, const float* coeffs, const uint8_t* masks, uint32_t degree, int B, int N,
            int K, int D, const float* v_colors, float* v_coeffs, float* v_dirs, hipStream_t s);

// ---- intersection / scan / sort / offsets ---------------------------------------------------
struct IsectArgs {
    const float* means2d;
    const int32_t* radii;
    const float* depths;
    const float* conics;     // null -> AABB
    const float* opacities;  // null -> AABB
    int I, N;
    int tile_size, tile_width, tile_height;
    uint32_t tile_n_bits;
};
void isect_count(const IsectArgs& a, int32_t* tiles_per_gauss, hipStream_t s);
void isect_emit(const IsectArgs& a, const int64_t* cum, uint64_t* keys, int32_t* vals, hipStream_t s);

// inclusive int32 -> int64 scan; scratch needs scan_scratch_bytes(n) bytes. With `gather` the
// scanned sequence is in[gather[0]], in[gather[1]], ...; with n_dev only the first *n_dev (<= n)
// elements are scanned (n sizes the grids)
size_t scan_scratch_bytes(int64_t n);
void scan_i32_i64(const int32_t* in, int64_t* out, int64_t n, void* scratch, hipStream_t s,
                  const int32_t* gather = nullptr, const int64_t* n_dev = nullptr);

// Stable LSD radix sort of (key, i32 value) on bits [0, key_bits), keys u64, u32 or u16. Result
// lands in keys_a/vals_a when the pass count is even, else in keys_b/vals_b; returns 0 or 1
// accordingly. The scratch needs sort_scratch_bytes(n) bytes for n keys. With n_dev the key count is
// read on the device from *n_dev (<= n, which then only sizes the grids; n < 2^30, else -1 is
// returned and nothing is launched): the launches no longer depend on the count. no_wait (u32 keys and
// the position sorts): every pass counts its tiles' digits and scans the counts (reduce-then-scan) at
// any size, so no workgroup waits on another and the sort cannot give up (below 16 tiles of 4096 keys
// the default onesweep passes wait on their predecessors with a bounded spin).
size_t sort_scratch_bytes(int64_t n);
int radix_sort(uint64_t* keys_a, int32_t* vals_a, uint64_t* keys_b, int32_t* vals_b, int64_t n,
               uint32_t key_bits, void* scratch, hipStream_t s, bool clear_err = true,
               const int64_t* n_dev = nullptr);
int radix_sort(uint32_t* keys_a, int32_t* vals_a, uint32_t* keys_b, int32_t* vals_b, int64_t n,
               uint32_t key_bits, void* scratch, hipStream_t s, bool clear_err = true,
               const int64_t* n_dev = nullptr, bool no_wait = false);
int radix_sort(uint16_t* keys_a, int32_t* vals_a, uint16_t* keys_b, int32_t* vals_b, int64_t n,
               uint32_t key_bits, void* scratch, hipStream_t s, bool clear_err = true,
               const int64_t* n_dev = nullptr);
// The same sort with each key's input position as its value (vals_a is not read; the sorted values
// are the positions of the keys in the unsorted array). x_a (optional, then x_b too): a u32 per key
// that moves with it, sorted into x_a or x_b like the keys (x_a is the input and, after an even pass
// count, the output).
int radix_sort_positions(uint16_t* keys_a, int32_t* vals_a, uint16_t* keys_b, int32_t* vals_b, int64_t n,
                         uint32_t key_bits, void* scratch, hipStream_t s, bool clear_err = true,
                         const int64_t* n_dev = nullptr, uint32_t* x_a = nullptr, uint32_t* x_b = nullptr,
                         bool no_wait = false);
int radix_sort_positions(uint32_t* keys_a, int32_t* vals_a, uint32_t* keys_b, int32_t* vals_b, int64_t n,
                         uint32_t key_bits, void* scratch, hipStream_t s, bool clear_err = true,
                         const int64_t* n_dev = nullptr, uint32_t* x_a = nullptr, uint32_t* x_b = nullptr,
                         bool no_wait = false);
// The same sort of n u64 keys from read-only inputs into keys_out/vals_out, with keys_tmp/vals_tmp as
// the second ping-pong side (n > 0, key_bits in 1..64, the onesweep range n < 2^30). No buffer may
// alias another.
void radix_sort_into(const uint64_t* keys, const int32_t* vals, uint64_t* keys_out, int32_t* vals_out,
                     uint64_t* keys_tmp, int32_t* vals_tmp, int64_t n, uint32_t key_bits, void* scratch,
                     hipStream_t s);
// device word in the sort's scratch that a sort sets non-zero when a tile's look-back gave up (a
// broken invariant, never expected). A sort with clear_err zeroes it first; one without adds to
// what the sorts before it left, so several sorts in a row can be checked with one read.
uint32_t* sort_error_flag(void* scratch);
// Equal depths by original row in index-first lists whose Gaussians are numbered in an internal row
// order: the order of equal depths is row_orig[id_of[value]], and an entry's depth is word 3 of its
// Gaussian's splat record, splats[3 id_of[value]].w (the emit's key).
struct TieOrder {
    const int32_t* id_of;
    const int32_t* row_orig;
    const float4* splats;
};
// Index-first intersections: each tile's range [offsets[t], offsets[t+1]) of `vals` (emit positions,
// in Gaussian index order after a stable tile sort) is sorted stably by its entries' depth bits, in
// place: the (depth, index) order within each tile. sdepth[i] is the depth of entry vals[i] (the
// tile sort carried them along, so a tile reads its keys in sequence). The count is *n_dev when set,
// else n_isects; tile_order (optional) is the order the workgroups take the tiles in. Tiles of more
// than 2048 entries pass through scratch_k0 / scratch_k1 / scratch_v (each indexed like vals, at least
// the count long; none of them may overlap sdepth). order_out (optional): the launch also writes the
// rasterisers' tile order (raster_tile_order's, from the same offsets) there and the largest tile's
// count into *max_count, from one extra workgroup; the tiles are then sorted in index order. ties
// (optional): equal depths go by original row instead of index (work only tiles with equal depths do).
void tile_depth_sort(const int32_t* offsets, int n_tiles, int64_t n_isects, const int64_t* n_dev,
                     const int32_t* tile_order, int32_t* vals, const uint32_t* sdepth, uint32_t* scratch_k0,
                     uint32_t* scratch_k1, int32_t* scratch_v, hipStream_t s, int32_t* order_out = nullptr,
                     uint32_t* max_count = nullptr, const TieOrder* ties = nullptr);

// offsets[I*n_tiles] from sorted keys; n_isects > 0.
// key_shift: position of the (image, tile) id in the key (32 for the isect_tiles encoding)
void offset_encode(const uint64_t* keys, int64_t n_isects, int I, int n_tiles, uint32_t tile_n_bits,
                   int32_t* offsets, hipStream_t s, uint32_t key_shift = 32);

// ---- raster ---------------------------------------------------------------------------------
// Packed per-Gaussian record consumed by the rasterizer: 3 x float4
// {x, y, opacity, 0}, {conic a, b, c, 0}, {r, g, b, 0}.
void pack_splats(const float* means2d, const float* conics, const float* colors, const float* opacities,
                 int n, float4* splats, hipStream_t s);
struct RasterArgs {
    const float4* splats;
    const int32_t* offsets;
    const int32_t* flatten_ids;
    const float* backgrounds;  // [I,3] or null
    const uint8_t* masks;      // [I,n_tiles] or null
    int I, width, height, tile_width, tile_height;
    int32_t n_isects;
    // optional (I == 1): workgroup b renders tile tile_order[b] — heaviest tiles first, so the
    // last workgroups to start are the short ones; null = tile b
    const int32_t* tile_order;
    // optional: the intersection count on the device (read instead of n_isects), so that the
    // launches do not depend on it
    const int64_t* n_isects_dev;
    // optional: flatten_ids hold emit positions p and the Gaussian of p is id_of[p] (the resident step)
    const int32_t* id_of;
    // optional (profiling): pair counters the rasterisers add into, kRasterStat* indices; null in
    // production (the counting kernels are separate instantiations)
    unsigned long long* stats;
    // optional: one u16 per intersection, the 4x4 blocks its splat's cutoff set reaches in its tile;
    // the forward stores the mask of every entry it loads, the backward reads it instead of working it
    // out again. Null: both compute it. With block_masks, mask_end (one i32 per tile, required) gets
    // the end of the entries whose masks the forward stored: it stops loading at a batch boundary once
    // every pixel of the tile is done, so it stores masks for [range_start, mask_end). The backward
    // walks from the tile's last contributor down, which lies before mask_end, so it always finds a
    // stored mask; it works out the mask itself for any entry at or past mask_end all the same.
    uint16_t* block_masks;
    int32_t* mask_end;
};
// raster pair counters (RasterArgs::stats): forward wave iterations (x 64 lane pairs), block-list
// entries walked (one splat against a 4x4 block) and pairs composited; backward 4-iteration chunks
// (x 256 lane pairs), block-list entries in them, chunks in which no lane's pair is inside the cutoff,
// lane pairs inside the cutoff and before the pixel's last contributor, pairs that contribute
// (alpha >= 1/255)
enum RasterStat : int {
    kStatFwdIters = 0,
    kStatFwdEntries = 1,
    kStatFwdTaken = 2,
    kStatBwdChunks = 3,
    kStatBwdEntries = 4,
    kStatBwdEmptyChunks = 5,
    kStatBwdInCutoff = 6,
    kStatBwdContrib = 7,
    kRasterStats = 8
};
// tile_order for raster_fwd/raster_bwd: the n_tiles tile ids by descending intersection count
// (counting sort on 256 buckets of the count; order within a bucket unspecified); max_count
// (optional) receives the largest count
void raster_tile_order(const int32_t* offsets, int n_tiles, int64_t n_isects, int32_t* order, hipStream_t s,
                       const int64_t* n_isects_dev = nullptr, uint32_t* max_count = nullptr);
void raster_fwd(const RasterArgs& a, float* render_colors, float* render_alphas, int32_t* last_ids,
                hipStream_t s);
// Gradient outputs zeroed by the caller; packed as 3 x float4 per Gaussian when `packed_grads`
// is set (v_xy.x, v_xy.y, v_op, _ | v_conic a,b,c, _ | v_rgb, _), else SoA pointers are used.
struct RasterBwdGrads {
    float* v_means2d;
    float* v_conics;
    float* v_colors;
    float* v_opacities;
    float* v_means2d_abs;
    float4* packed;  // when set: the resident-step record layout (3 x float4 per Gaussian)
    // when set (with RasterArgs::id_of): no atomics; the sums of each (tile, Gaussian) are stored at the
    // intersection's emit position p (flatten_ids[idx]) as kPartFloats floats (stride kPartStride), with the
    // step's stamp (*stamp) in float kPartFloats, and the Gaussian's `touched` flag is set (cleared by
    // the caller); raster_gather_grads then sums each Gaussian's entries that carry the stamp, in order
    float* part;
    const uint32_t* stamp;
    uint8_t* touched;  // with part: set for every Gaussian that got an entry (cleared by the caller)
};
constexpr int kPartFloats = 9;  // v_xy (2), v_opacity, v_conic (3), v_rgb (3)
constexpr int kPartStride = 12;  // floats per `part` entry: three aligned float4 (the stamp, 2 unused)
// Before each backward in `part` mode: advances the stamp (never 0, the value of zeroed entries), clears
// touched[0, rows) and the gather's queue count
void raster_bwd_begin(uint32_t* stamp, uint8_t* touched, int rows, int32_t* long_count, hipStream_t s);
// For each Gaussian order[j] (j itself when order is null) with touched set: grads[order[j]] (3 x float4 record) = the sum of the `part`
// entries at [cum[j-1], cum[j]) that carry the current stamp (order and cum: the depth order and the
// inclusive scan of its tile counts that placed the emit), in a fixed order per range: the
// deterministic end of raster_bwd's `part` mode. Untouched Gaussians' records are not written. long_list
// holds `count` ints, long_count one (reset by raster_bwd_begin or the step's preprocess; it ends as the
// number of ranges longer than kLongRange). With count_dev the positions are the first *count_dev (<=
// count, which sizes the grid). inline_long: the gather's waves reduce their long ranges themselves
// instead of queueing them for a second launch (same sums; fast while they are few).
// loss (optional): the training step's loss, reduced by the gather's first workgroup (one wave) before
// its own ranges, and the step's host words (see StepLoss)
// positions_per_wave (32 or 64): the positions each one-wave workgroup takes; every lane stages entries,
// the first positions_per_wave lanes own a position each. 32 halves the rounds of the waves whose
// positions hold many entries (Gaussians of one size sit together when the rows are in spatial order);
// the sums are the same either way.
struct StepLoss;
void raster_gather_grads(int count, const int32_t* order, const int64_t* cum, const float* part,
                         const uint32_t* stamp, const uint8_t* touched, float4* grads, int32_t* long_list,
                         int32_t* long_count, hipStream_t s, const int64_t* count_dev = nullptr,
                         bool inline_long = false, const StepLoss* loss = nullptr, int positions_per_wave = 64);
void raster_bwd(const RasterArgs& a, const float* render_alphas, const int32_t* last_ids,
                const float* v_render_colors, const float* v_render_alphas, const RasterBwdGrads& g,
                hipStream_t s);

// ---- SSIM -----------------------------------------------------------------------------------
void ssim_fwd(const float* img1, const float* img2, int I, int H, int W, int C, int need_coeffs,
              float* map, float* cmu, float* csg, float* ccr, double* block_sums, hipStream_t s);
int ssim_fwd_blocks(int I, int H, int W, int C);
void ssim_bwd(const float* img1, const float* img2, const float* cmu, const float* csg, const float* ccr,
              int I, int H, int W, int C, float G, float* v_img1, hipStream_t s);

// ---- RNG / MCMC -----------------------------------------------------------------------------
void rng_philox_u32(uint64_t seed, uint64_t offset, int64_t count, uint32_t* out, hipStream_t s);
void rng_normal_f32(uint64_t seed, uint64_t offset, int64_t count, float* out, hipStream_t s);
void mcmc_relocation(const float* opac, const float* scales, const int32_t* ratios, const float* binoms,
                     int N, int n_max, float min_opacity, float* new_op, float* new_sc, hipStream_t s);
void mcmc_perturb(float* positions, const float* quats, const float* scales_log, const float* logits,
                  const float* noise, int N, float noise_scale, float t, float k, hipStream_t s);

} // namespace sxk
