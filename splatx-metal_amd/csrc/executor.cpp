// executor.cpp — the device-resident train-step executor (TrainStepExecutor, KernelBackend.h:386-392;
// the reference's MetalTrainStepExecutor, MetalBackend.cpp:1628-2460).
//
// One HIP stream. A step is: preprocess (with the previous step's parameter update: bwd chain + Adam +
// noise, fused row by row) -> block scan [sync 1: n_isects, stored into mapped host memory; isect
// buffers grow 1.5x when needed] -> compaction -> emit -> radix sort -> offsets -> raster fwd -> SSIM fwd
// -> SSIM bwd fused with the L1 gradient -> raster bwd -> gather (its first workgroup reduces the loss)
// [sync 2: the loss, stored the same way]. The step's own update waits for the next step's preprocess, or for anything
// else that reads or writes the arena (flush_update). Everything after sync 1 is a captured graph,
// queued before the host waits. Parameters, moments and the GT cache stay
// in HBM; the arena is sized once for arena_rows and never reallocated.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "splatx_hip.h"
#include "sx_host.h"
#include "sx_kernels.h"
#include "sx_step.h"
#include "sx_exec.h"

using namespace sxh;

extern "C" {

int32_t sxh_exec_create(sxh_backend* b, const sxh_exec_desc* desc, sxh_executor** out) {
    return guarded([&] {
        if (!b || !desc || !out) invalid("TrainStepExecutor", "null argument");
        // MetalBackend.cpp:1632-1641
        if (desc->arena_rows < 1) invalid("TrainStepExecutor", "arena_rows must be >= 1");
        if (desc->sh_degree < 0 || desc->sh_degree > 3) invalid("TrainStepExecutor", "sh_degree must be in [0,3]");
        if (!(desc->ssim_weight >= 0.0f && desc->ssim_weight <= 1.0f))
            invalid("TrainStepExecutor", "ssim_weight must be in [0,1]");
        if (desc->isect_mode != SXH_ISECT_ACCUTILE && desc->isect_mode != SXH_ISECT_AABB)
            invalid("TrainStepExecutor", "isect_mode must be ACCUTILE or AABB");
        const int64_t K = static_cast<int64_t>(desc->sh_degree + 1) * (desc->sh_degree + 1);
        if (desc->arena_rows * K * 3 > INT32_MAX) invalid("TrainStepExecutor", "arena_rows*K*3 exceeds int32");
        SXH_HIP(hipSetDevice(b->device));
        auto* e = new sxh_executor();
        try {
            e->b = b;
            e->d = *desc;
            e->n_coeffs = static_cast<int>(K);
            e->dims[5] = static_cast<int>((K - 1) * 3);
            e->rows = static_cast<int>(desc->arena_rows);
            const size_t R = static_cast<size_t>(e->rows);
            for (int g = 0; g < 6; g++) {
                if (e->dims[g] == 0) continue;
                const size_t n = R * e->dims[g];
                e->p[g].alloc(n);
                e->m[g].alloc(n);
                e->v[g].alloc(n);
                SXH_HIP(hipMemsetAsync(e->p[g].p, 0, n * 4, b->stream));
                SXH_HIP(hipMemsetAsync(e->m[g].p, 0, n * 4, b->stream));
                SXH_HIP(hipMemsetAsync(e->v[g].p, 0, n * 4, b->stream));
            }
            e->splats.alloc(R * 3);
            e->grads.alloc(R * 3);
            e->radii.alloc(R * 2);
            e->tiles.alloc(R);
            e->cum.alloc(R);
            e->long_list.alloc(R);
            e->long_count.alloc(2);  // this step's long-range count, the previous step's
            SXH_HIP(hipMemsetAsync(e->long_count.p, 0, 2 * sizeof(int32_t), e->b->stream));
            e->stamp.alloc(1);
            e->max_tile.alloc(1);
            SXH_HIP(hipMemsetAsync(e->stamp.p, 0, sizeof(uint32_t), b->stream));
            e->touched.alloc(R);
            e->scan_scratch.alloc(sxk::scan_scratch_bytes(static_cast<int64_t>(R)));
            e->dkey_a.alloc(R);
            e->dkey_b.alloc(R);
            e->order_a.alloc(R);
            e->order_b.alloc(R);
            e->n_vis.alloc(5);
            e->vis_part.alloc(4 * static_cast<size_t>(sxk::step_preprocess_blocks(desc->arena_rows)));
            e->blk_base.alloc(2 * static_cast<size_t>(sxk::step_preprocess_blocks(desc->arena_rows)));
            e->emit_list.alloc(R);
            e->loss_dev.alloc(1);
            e->staging.alloc(R * 45);
            e->ensure_isect(1 << 16);
            const char* dbg = std::getenv("SXH_DEBUG_FORCE_SORT_ERROR");
            e->debug_sort_error = dbg && dbg[0] == '1';
            for (int k = 0; k < kMaxEvents; k++) SXH_HIP(hipEventCreate(&e->ev[k]));
            SXH_HIP(hipStreamSynchronize(b->stream));
        } catch (...) {
            delete e;
            throw;
        }
        *out = e;
    });
}

void sxh_exec_destroy(sxh_executor* e) {
    if (!e) return;
    (void)hipStreamSynchronize(e->b->stream);
    for (int k = 0; k < kMaxEvents; k++)
        if (e->ev[k]) (void)hipEventDestroy(e->ev[k]);
    for (auto& row : e->graph_b)
        for (hipGraphExec_t x : row)
            if (x) (void)hipGraphExecDestroy(x);
    delete e;
}

static void sync_params(sxh_executor* e, const sxh_param_sync* s, bool up) {
    if (!s) invalid("TrainStepExecutor", "null sync");
    if (s->rows < 0 || s->rows > e->rows) invalid("TrainStepExecutor", "sync rows out of [0, arena_rows]");
    const int rows = static_cast<int>(s->rows);
    sxh_detail::canonicalize(e);  // rows in the caller's order, the pending update applied
    if (rows == 0) return;
    hipStream_t st = e->b->stream;
    for (int g = 0; g < 6; g++) {
        const int dim = e->dims[g];
        if (dim == 0) continue;
        float* host[3] = {s->params[g], s->exp_avg[g], s->exp_avg_sq[g]};
        DevBuf<float>* dev[3] = {&e->p[g], &e->m[g], &e->v[g]};
        for (int k = 0; k < 3; k++) {
            if (!host[k]) invalid("TrainStepExecutor", "null parameter/moment pointer for group " + std::to_string(g));
            const size_t n = static_cast<size_t>(rows) * dim;
            if (up) {
                SXH_HIP(hipMemcpyAsync(e->staging.p, host[k], n * 4, hipMemcpyHostToDevice, st));
                sxk::aos_to_soa(e->staging.p, dev[k]->p, rows, dim, e->rows, st);
            } else {
                sxk::soa_to_aos(dev[k]->p, e->staging.p, rows, dim, e->rows, st);
                SXH_HIP(hipMemcpyAsync(host[k], e->staging.p, n * 4, hipMemcpyDeviceToHost, st));
            }
            SXH_HIP(hipStreamSynchronize(st));  // staging is reused
        }
    }
}

int32_t sxh_exec_upload(sxh_executor* e, const sxh_param_sync* s) {
    return guarded([&] {
        if (!e) invalid("TrainStepExecutor", "null executor");
        SXH_HIP(hipSetDevice(e->b->device));
        sync_params(e, s, true);
    });
}

int32_t sxh_exec_download(sxh_executor* e, const sxh_param_sync* s) {
    return guarded([&] {
        if (!e) invalid("TrainStepExecutor", "null executor");
        SXH_HIP(hipSetDevice(e->b->device));
        sync_params(e, s, false);
    });
}

int32_t sxh_exec_set_gt_cache(sxh_executor* e, const float* images, int32_t n, int32_t width, int32_t height) {
    return guarded([&] {
        if (!e || !images) invalid("TrainStepExecutor", "null argument");
        if (n < 1 || width < 1 || height < 1) invalid("TrainStepExecutor", "bad GT cache shape");
        SXH_HIP(hipSetDevice(e->b->device));
        const size_t per = static_cast<size_t>(width) * height * 3;
        e->gt_cache.alloc(per * n);
        SXH_HIP(hipMemcpyAsync(e->gt_cache.p, images, per * n * 4, hipMemcpyHostToDevice, e->b->stream));
        SXH_HIP(hipStreamSynchronize(e->b->stream));
        e->gt_n = n;
        e->gt_w = width;
        e->gt_h = height;
    });
}

int32_t sxh_exec_set_profiling(sxh_executor* e, int32_t enable) {
    return guarded([&] {
        if (!e) invalid("TrainStepExecutor", "null executor");
        e->prof = enable != 0;
        e->prof_stats = (enable & 2) != 0;
        if (e->prof_stats && !e->rstats.p) e->rstats.alloc(sxk::kRasterStats);
    });
}

int32_t sxh_exec_get_raster_stats(sxh_executor* e, sxh_raster_stats* out) {
    return guarded([&] {
        if (!e || !out) invalid("TrainStepExecutor", "null argument");
        *out = e->rstats_host;
    });
}

int32_t sxh_exec_sync(sxh_executor* e) {
    return guarded([&] {
        if (!e) invalid("TrainStepExecutor", "null executor");
        SXH_HIP(hipSetDevice(e->b->device));
        sxh_detail::flush_update(e);  // the last step's parameter update is part of its work
        SXH_HIP(hipStreamSynchronize(e->b->stream));
    });
}

int32_t sxh_exec_set_graph(sxh_executor* e, int32_t enable) {
    return guarded([&] {
        if (!e) invalid("TrainStepExecutor", "null executor");
        e->use_graph = enable != 0;
    });
}

int32_t sxh_exec_set_isect_order(sxh_executor* e, int32_t mode) {
    return guarded([&] {
        if (!e) invalid("TrainStepExecutor", "null executor");
        if (mode < SXH_ISECT_ORDER_AUTO || mode > SXH_ISECT_ORDER_INDEX_FIRST)
            invalid("TrainStepExecutor", "unknown intersection order");
        e->isect_order = mode;
    });
}

int32_t sxh_exec_set_row_order(sxh_executor* e, int32_t mode) {
    return guarded([&] {
        if (!e) invalid("TrainStepExecutor", "null executor");
        if (mode < SXH_ROW_ORDER_SPATIAL_AUTO || mode > SXH_ROW_ORDER_SPATIAL)
            invalid("TrainStepExecutor", "unknown row order");
        SXH_HIP(hipSetDevice(e->b->device));
        if (mode == SXH_ROW_ORDER_ORIGINAL && e->permuted) sxh_detail::canonicalize(e);
        e->row_order = mode;
    });
}

int32_t sxh_exec_get_timing(sxh_executor* e, sxh_exec_timing* out) {
    return guarded([&] {
        if (!e || !out) invalid("TrainStepExecutor", "null argument");
        *out = e->timing;
    });
}

} // extern "C"

// A sync point of the step: wait until a kernel has stored `seq` into the mapped word (sync 1: the
// block scan, its counts then in place; sync 2: the gather's first workgroup, the loss). The
// stream is polled now and then, so that an error or a stream that finished without the store ends
// the wait instead of spinning forever.
static void wait_count_word(volatile unsigned long long* word, unsigned long long seq, hipStream_t s,
                            const char* what) {
    for (uint32_t spins = 1;; spins++) {
        if (*word == seq) return;
        if ((spins & 1023u) == 0u) {
            const hipError_t q = hipStreamQuery(s);
            if (q == hipSuccess) {
                if (*word == seq) return;
                throw std::runtime_error(std::string(what) + ": the step's read-back word was not written");
            }
            if (q != hipErrorNotReady) SXH_HIP(q);
        }
        __builtin_ia32_pause();
    }
}

void sxh_detail::flush_update(sxh_executor* e) {
    if (!e->update_pending) return;
    e->update_pending = false;
    // gated like the fused launch: the pending step's overflow word (n_vis word 4) and sort error word
    sxk::step_postprocess(e->pending_c, e->arena(), e->splats.p, e->grads.p, e->touched.p, e->b->stream, e->n_vis.p + 4,
                          e->sort_scratch.p ? sxk::sort_error_flag(e->sort_scratch.p) : nullptr,
                          e->permuted ? e->row_orig.p : nullptr);
    SXH_HIP(hipGetLastError());
}

void sxh_detail::canonicalize(sxh_executor* e) {
    flush_update(e);
    e->steps_since_exchange = 0;
    if (!e->permuted) return;
    // original row o takes internal row row_int[o]
    sxk::arena_permute_rows(e->arena(), e->dims, e->perm_count, e->row_int.p, e->staging.p, e->b->stream);
    SXH_HIP(hipGetLastError());
    e->permuted = false;
}

// The live rows [0, count) along a Morton curve over their means (the arena in original order, no
// update pending): keys and a stable sort of them, then every parameter and moment column reordered.
static void spatial_order(sxh_executor* e, int count) {
    hipStream_t s = e->b->stream;
    if (e->row_orig.n < static_cast<size_t>(e->rows)) {
        e->row_orig.alloc(static_cast<size_t>(e->rows));
        e->row_int.alloc(static_cast<size_t>(e->rows));
        e->tiles_o.alloc(static_cast<size_t>(e->rows));
    }
    const size_t sf = sxk::arena_morton_scratch_floats(count);
    if (e->perm_scratch.n < sf) e->perm_scratch.alloc(sf);
    const sxk::Arena A = e->arena();
    sxk::arena_morton_keys(A, count, e->perm_scratch.p, e->dkey_a.p, e->order_a.p, s);
    const int w = sxk::radix_sort(e->dkey_a.p, e->order_a.p, e->dkey_b.p, e->order_b.p, count, 30, e->sort_scratch.p, s,
                                  true, nullptr, true);
    if (w < 0) throw std::runtime_error("TrainStepExecutor: spatial order sort failed");
    const int32_t* src = w ? e->order_b.p : e->order_a.p;
    sxk::arena_permute_rows(A, e->dims, count, src, e->staging.p, s);
    sxk::perm_maps(src, count, e->row_orig.p, e->row_int.p, s);
    SXH_HIP(hipGetLastError());
    e->permuted = true;
    e->perm_count = count;
}

// The step proper. `render_to_dev` (device), when not null, receives a copy of the render.
void sxh_detail::run_step(sxh_executor* e, const sxh_step_inputs* in, sxh_step_outputs* out, float* render_to_dev) {
    const char* what = "TrainStepExecutor::step";
    if (!in || !out) invalid(what, "null inputs/outputs");
    // MetalBackend.cpp:1697-1711
    if (in->count < 1 || in->count > e->rows) invalid(what, "count out of [1, arena_rows]");
    if (in->width < 1 || in->height < 1) invalid(what, "width/height must be positive");
    if (!in->viewmat || !in->K) invalid(what, "null viewmat/K");
    const bool fwd_only = in->forward_only != 0;
    const bool use_gt_cache = in->gt_index >= 0;
    if (!fwd_only && !use_gt_cache && !in->gt_rgb) invalid(what, "null gt_rgb");
    if (use_gt_cache && !fwd_only) {
        if (in->gt_index >= e->gt_n) invalid(what, "gt_index out of range");
        if (in->width != e->gt_w || in->height != e->gt_h) invalid(what, "GT cache image size mismatch");
    }
    const bool use_ssim = e->d.ssim_weight > 0.0f && !fwd_only;
    if (use_ssim && (in->height < 11 || in->width < 11)) invalid(what, "ssim requires H, W >= 11");
    if (in->degrees_to_use > static_cast<uint32_t>(e->d.sh_degree)) invalid(what, "degrees_to_use > sh_degree");

    hipStream_t s = e->b->stream;
    const int W = in->width, H = in->height;
    const int tw = (W + 15) / 16, th = (H + 15) / 16;
    // per-block tile-count sums of the preprocess are 32-bit: 256 Gaussians x at most tw * th tiles
    if (static_cast<int64_t>(tw) * th > (int64_t{1} << 23)) invalid(what, "image too large (over 2^23 tiles)");
    const size_t HW = static_cast<size_t>(W) * H;
    const size_t n_px = HW * 3;
    const size_t map_n = use_ssim ? static_cast<size_t>(H - 10) * (W - 10) * 3 : 0;
    e->ensure_image(W, H, use_ssim);
    e->n_ev = 0;

    sxk::StepConst c{};
    std::memcpy(c.vm, in->viewmat, sizeof(c.vm));
    std::memcpy(c.K, in->K, sizeof(c.K));
    c.width = W;
    c.height = H;
    c.count = static_cast<int>(in->count);
    c.n_coeffs = e->n_coeffs;
    c.degree = in->degrees_to_use;
    c.eps2d = e->d.eps2d;
    c.near_plane = e->d.near_plane;
    c.far_plane = e->d.far_plane;
    c.radius_clip = e->d.radius_clip;
    c.aa = e->d.antialiased ? 1 : 0;
    c.accutile = e->d.isect_mode == SXH_ISECT_ACCUTILE ? 1 : 0;
    c.tile_width = tw;
    c.tile_height = th;
    c.tile_n_bits = sx::bits_for_count(static_cast<int64_t>(tw) * th);
    for (int g = 0; g < 6; g++) c.lr[g] = in->lr[g];
    c.b1 = e->d.b1;
    c.b2 = e->d.b2;
    c.eps = e->d.eps;
    c.opacity_reg_w = in->opacity_reg_w;
    c.scale_reg_w = in->scale_reg_w;
    c.inject_noise = (in->inject_noise && !fwd_only) ? 1 : 0;
    c.noise_seed = in->noise_seed;
    c.noise_offset = in->noise_offset;
    c.noise_scale = in->noise_scale;
    const sxk::Arena A = e->arena();
    // the live rows' order: spatial ones cover this step's rows; a cloud that stayed on the device for a
    // step since it last exchanged rows with the caller goes into spatial order (at most a few ms, once)
    constexpr int kSpatialMinRows = 1 << 16;
    if (e->permuted && e->perm_count != c.count) sxh_detail::canonicalize(e);
    if (!fwd_only && !e->permuted &&
        ((e->row_order == SXH_ROW_ORDER_SPATIAL) ||
         (e->row_order == SXH_ROW_ORDER_SPATIAL_AUTO && c.count >= kSpatialMinRows && e->steps_since_exchange >= 2))) {
        sxh_detail::flush_update(e);
        spatial_order(e, c.count);
    }
    // index-first sorts each tile's list by depth in one workgroup: fast while the tiles stay small
    // (up to 2048 entries in LDS, larger ones through global scratch, correct at any size)
    constexpr int64_t kIndexFirstMaxTile = 4096;
    const bool index_first = e->isect_order == SXH_ISECT_ORDER_INDEX_FIRST ||
                             (e->isect_order == SXH_ISECT_ORDER_AUTO && e->last_max_tile >= 0 &&
                              e->last_max_tile <= kIndexFirstMaxTile);
    // rows in spatial order: depth first compacts the visible rows in original order (its depth sort's
    // ties then go by original row); index first compacts them in internal order, and the per-tile
    // depth sort orders equal depths by original row
    const int32_t* const row_orig = e->permuted ? e->row_orig.p : nullptr;
    const int32_t* const row_int = (e->permuted && !index_first) ? e->row_int.p : nullptr;
    // the last training step's deferred update rides on this step's preprocess when both cover the same
    // rows; a forward-only step (or another row count) applies it first
    if (e->update_pending && (fwd_only || e->pending_c.count != c.count)) sxh_detail::flush_update(e);

    // ---- segment A: preprocess + counts -----------------------------------------------------------
    // `cap`: the intersection capacity segment B may assume; past it, segment B's counts read 0 and the
    // arena update is skipped (n_vis words 3 and 4), so a segment B launched before the count is known
    // leaves everything as it was and the step runs again on grown buffers
    // the step's read-back block: u64 visible, u64 intersections (stored by segment A's block scan), u32
    // loss bits, sort error flag, largest tile, the previous step's long-range count (stored by the
    // gather's first workgroup), u64 segment
    // A's sequence number (word 4, after the counts), u64 the loss's (word 5)
    volatile unsigned long long* const hc = static_cast<volatile unsigned long long*>(e->step_rb.p);
    volatile uint32_t* const hw = reinterpret_cast<volatile uint32_t*>(hc + 2);
    unsigned long long seq = 0;  // the last segment A's sequence number (its count word's tag)
    auto launch_a = [&](unsigned long long cap) {
        seq = ++e->step_seq;
        if (e->prof_stats)
            SXH_HIP(hipMemsetAsync(e->rstats.p, 0, sxk::kRasterStats * sizeof(unsigned long long), s));
        e->mark("start");
        const sxk::StepClear clr =
            fwd_only ? sxk::StepClear{} : sxk::StepClear{e->touched.p, e->stamp.p, e->long_count.p, e->long_count.p + 1};
        if (e->update_pending) {
            // (taken once: an overflowed step that runs segment A again finds the update applied)
            e->update_pending = false;
            sxk::step_update_preprocess(e->pending_c, c, A, e->splats.p, e->grads.p, e->touched.p, e->n_vis.p + 4,
                                        sxk::sort_error_flag(e->sort_scratch.p), e->radii.p, e->tiles.p,
                                        e->vis_part.p, e->n_vis.p, e->blk_base.p, cap,
                                        static_cast<unsigned long long*>(e->step_rb.dev), seq, clr, s, row_orig,
                                        row_int, e->tiles_o.p);
            e->mark("update_preprocess");
        } else {
            sxk::step_preprocess(c, A, e->splats.p, e->radii.p, e->tiles.p, e->vis_part.p, e->n_vis.p, e->blk_base.p,
                                 cap, static_cast<unsigned long long*>(e->step_rb.dev), seq, clr, s, row_int,
                                 e->tiles_o.p);
            e->mark("preprocess");
        }
    };
    const float* gt = nullptr;
    auto upload_gt = [&]() {
        if (fwd_only) return;
        if (use_gt_cache) {
            gt = e->gt_cache.p + static_cast<size_t>(in->gt_index) * n_px;
        } else {
            SXH_HIP(hipMemcpyAsync(e->gt_stage.p, in->gt_rgb, n_px * 4, hipMemcpyHostToDevice, s));
            gt = e->gt_stage.p;
        }
    };
    // the intersection count segment B reads (0 after an overflow; the overflow word, n_vis word 4, gates
    // the step's parameter update)
    const int64_t* n_isects_dev = reinterpret_cast<const int64_t*>(e->n_vis.p) + 3;
    int n_l1 = 0, n_ss = 0;
    int32_t* flat = e->vals_a.p;

    // ---- segment B: everything after the count. With n_dev the launches read the intersection count on
    // the device (grids sized for the capacity), so they can be captured before the count is known.
    auto launch_b = [&](int64_t n_host, const int64_t* n_dev) {
        const int n_tiles = tw * th;
        // the order of the reference's (tile | depth) key sort, two ways. Depth first: the Gaussians
        // sorted by depth, their tile ids emitted in that order, a stable sort on the tile bits. Index
        // first: the tile ids emitted in index order, a stable sort on the tile bits, then each tile's
        // list sorted by depth (order null: position j of the emit is Gaussian j).
        // positions of the emit: the Gaussians with tiles (*n_emit of them), compacted in index order
        const unsigned long long* n_emit = e->n_vis.p + 2;
        const int64_t* n_emit_i = reinterpret_cast<const int64_t*>(n_emit);
        // (index first, the compaction runs inside the emit's launch, below)
        if (!index_first)
            sxk::step_emit_compact(c, row_int ? e->tiles_o.p : e->tiles.p, e->blk_base.p, e->emit_list.p, nullptr, s,
                                   row_int);
        const int32_t* order = e->emit_list.p;
        if (!index_first) {
            sxk::step_depth_keys(c, e->splats.p, e->emit_list.p, n_emit, e->dkey_a.p, e->order_a.p, s);
            // (the step's sorts never wait on another workgroup: they cannot give up halfway through a step)
            const int wd = sxk::radix_sort(e->dkey_a.p, e->order_a.p, e->dkey_b.p, e->order_b.p, c.count, 32,
                                           e->sort_scratch.p, s, true, n_emit_i, true);
            if (wd < 0) throw std::runtime_error(std::string(what) + ": arena too large for a device-count depth sort");
            order = wd ? e->order_b.p : e->order_a.p;
            e->mark("depth_sort");
            sxk::scan_i32_i64(e->tiles.p, e->cum.p, c.count, e->scan_scratch.p, s, order, n_emit_i);
            e->mark("scan");
        }
        // index first: the emit also writes each entry's depth bits, into the upper half of keys_b (u64
        // words; the tile sort's keys and the large tiles' scratch use the lower half of each key buffer);
        // the tile sort carries them with the keys, between there and the upper half of keys_a
        uint32_t* const edepth =
            index_first ? reinterpret_cast<uint32_t*>(e->keys_b.p) + e->isect_cap : nullptr;
        uint32_t* const edepth_b =
            index_first ? reinterpret_cast<uint32_t*>(e->keys_a.p) + e->isect_cap : nullptr;
        int which = 0;
        if (c.tile_n_bits <= 16) {
            uint16_t* ka = reinterpret_cast<uint16_t*>(e->keys_a.p);
            uint16_t* kb = reinterpret_cast<uint16_t*>(e->keys_b.p);
            if (index_first)
                sxk::step_emit_compact_sorted(c, e->splats.p, e->radii.p, e->tiles.p, e->blk_base.p, e->emit_list.p,
                                              e->cum.p, n_emit, ka, e->emit_gid.p, s, edepth);
            else
                sxk::step_emit_sorted(c, e->splats.p, e->radii.p, order, e->cum.p, n_emit, ka, e->emit_gid.p, s,
                                      edepth);
            e->mark("emit");
            which = sxk::radix_sort_positions(ka, e->vals_a.p, kb, e->vals_b.p, n_host, c.tile_n_bits,
                                              e->sort_scratch.p, s, index_first, n_dev, edepth, edepth_b, true);
            e->mark("sort");
            sxk::step_tile_offsets(which ? kb : ka, n_host, n_tiles, e->offsets.p, s, n_dev);
        } else {
            uint32_t* ka = reinterpret_cast<uint32_t*>(e->keys_a.p);
            uint32_t* kb = reinterpret_cast<uint32_t*>(e->keys_b.p);
            if (index_first)
                sxk::step_emit_compact_sorted(c, e->splats.p, e->radii.p, e->tiles.p, e->blk_base.p, e->emit_list.p,
                                              e->cum.p, n_emit, ka, e->emit_gid.p, s, edepth);
            else
                sxk::step_emit_sorted(c, e->splats.p, e->radii.p, order, e->cum.p, n_emit, ka, e->emit_gid.p, s,
                                      edepth);
            e->mark("emit");
            which = sxk::radix_sort_positions(ka, e->vals_a.p, kb, e->vals_b.p, n_host, c.tile_n_bits,
                                              e->sort_scratch.p, s, index_first, n_dev, edepth, edepth_b, true);
            e->mark("sort");
            sxk::step_tile_offsets(which ? kb : ka, n_host, n_tiles, e->offsets.p, s, n_dev);
        }
        if (which < 0) throw std::runtime_error(std::string(what) + ": intersection capacity too large for a device count");
        if (e->debug_sort_error) sxk::step_set_word(sxk::sort_error_flag(e->sort_scratch.p), 1u, s);
        flat = which ? e->vals_b.p : e->vals_a.p;
        e->mark("offsets");
        if (index_first) {
            // the sorted tile keys are spent (the offsets are built): both key buffers and the other
            // value buffer are the scratch of tiles too large for LDS. The rasterisers' tile order comes
            // from one more workgroup of the same launch.
            // (rows in spatial order: the emit ran in that order, and equal depths go by original row)
            const sxk::TieOrder ties{e->emit_gid.p, row_orig, e->splats.p};
            sxk::tile_depth_sort(e->offsets.p, n_tiles, n_host, n_dev, nullptr, flat, which ? edepth_b : edepth,
                                 reinterpret_cast<uint32_t*>(e->keys_a.p), reinterpret_cast<uint32_t*>(e->keys_b.p),
                                 which ? e->vals_a.p : e->vals_b.p, s, e->tile_order.p, e->max_tile.p,
                                 row_orig ? &ties : nullptr);
            e->mark("tile_depth_sort");
        } else {
            sxk::raster_tile_order(e->offsets.p, n_tiles, n_host, e->tile_order.p, s, n_dev, e->max_tile.p);
        }
        sxk::RasterArgs ra{};
        ra.splats = e->splats.p;
        ra.offsets = e->offsets.p;
        ra.flatten_ids = flat;
        ra.I = 1;
        ra.width = W;
        ra.height = H;
        ra.tile_width = tw;
        ra.tile_height = th;
        ra.n_isects = static_cast<int32_t>(n_host);
        ra.n_isects_dev = n_dev;
        ra.id_of = e->emit_gid.p;  // the sorted values are emit positions
        ra.stats = e->prof_stats ? e->rstats.p : nullptr;  // never in a captured graph (profiling launches directly)
        ra.tile_order = e->tile_order.p;
        // the block masks go where the tile ids were: both key buffers are free once the offsets (and,
        // index first, the per-tile depth sort) are done
        ra.block_masks = fwd_only ? nullptr : reinterpret_cast<uint16_t*>(e->keys_a.p);
        ra.mask_end = e->mask_end.p;
        sxk::raster_fwd(ra, e->render.p, e->alpha.p, e->last_ids.p, s);
        e->mark("raster_fwd");
        // the loss words, then the launch's sequence number (word 5 of the block)
        // (the long-range count reported is the previous training step's: this step's gather reports the
        // words while its own ranges are still being counted)
        const sxk::StepReadback rb{sxk::sort_error_flag(e->sort_scratch.p), e->max_tile.p, e->long_count.p + 1,
                                   reinterpret_cast<uint32_t*>(static_cast<unsigned long long*>(e->step_rb.dev) + 2),
                                   static_cast<unsigned long long*>(e->step_rb.dev) + 5, seq};
        if (fwd_only) {
            sxk::step_readback(rb, s);
            return;
        }
        if (use_ssim) {
            n_ss = sxk::ssim_fwd_blocks(1, H, W, 3);
            sxk::ssim_fwd(e->render.p, gt, 1, H, W, 3, 1, nullptr, e->cmu.p, e->csg.p, e->ccr.p, e->ssim_part.p, s);
            e->mark("ssim_fwd");
            const float G = static_cast<float>(-static_cast<double>(e->d.ssim_weight) / static_cast<double>(map_n));
            n_l1 = sxk::step_ssim_bwd_blocks(H, W);
            sxk::step_ssim_bwd_l1(e->render.p, gt, e->cmu.p, e->csg.p, e->ccr.p, H, W, G, 1.0f - e->d.ssim_weight,
                                  1.0f / static_cast<float>(n_px), e->v_render.p, e->l1_part.p, s);
            e->mark("ssim_bwd_l1");
        } else {
            n_l1 = sxk::step_l1_blocks(static_cast<int64_t>(n_px));
            sxk::step_l1_grad(e->render.p, gt, static_cast<int64_t>(n_px), e->v_render.p, e->l1_part.p, n_l1, s);
            e->mark("l1_grad");
        }
        // the backward stores per-(tile, Gaussian) sums; the gather adds them per Gaussian in emit order, so
        // the gradients do not depend on the order in which tiles finish (no float atomics). Its stamp, the
        // touched flags and the long-range queue were set up by the preprocess.
        sxk::RasterBwdGrads gg{nullptr, nullptr,   nullptr,    nullptr,    nullptr,
                               e->grads.p, e->part.p, e->stamp.p, e->touched.p};
        sxk::raster_bwd(ra, e->alpha.p, e->last_ids.p, e->v_render.p, e->v_alpha_zero.p, gg, s);
        e->mark("raster_bwd");
        // the step's loss and host words, reduced by the gather's first workgroup before its own ranges
        sxk::StepLoss loss{};
        loss.l1p = e->l1_part.p;
        loss.n_l1 = n_l1;
        loss.ssp = e->ssim_part.p;
        loss.n_ss = n_ss;
        loss.n_px = static_cast<double>(n_px);
        loss.M = static_cast<double>(map_n);
        loss.lam = e->d.ssim_weight;
        loss.use_ssim = use_ssim ? 1 : 0;
        loss.out = e->loss_dev.p;
        loss.rb = rb;
        // long ranges reduced by the gather's own waves while a recent step had few (no second launch;
        // the count known when this step is queued is the one two steps back), queued for a wave each
        // otherwise (measured: inline 41 -> 35 us at config 3, queued 94 us against 329 inline at
        // config 5); either way the same sums
        constexpr int64_t kInlineLongMax = 1024;
        const bool inline_long = e->last_long >= 0 && e->last_long <= kInlineLongMax;
        // 32 positions per wave where the emit order puts Gaussians of one size together (the rows in
        // spatial order, or the depth order): its waves of large Gaussians take half the staging rounds
        // (config 3 in spatial order 43.6 -> 34.7 us); 64 in the caller's order (33.9 against 39.1 us)
        const int gather_positions = (e->permuted || !index_first) ? 32 : 64;
        sxk::raster_gather_grads(c.count, order, e->cum.p, e->part.p, e->stamp.p, e->touched.p, e->grads.p,
                                 e->long_list.p, e->long_count.p, s, n_emit_i, inline_long, &loss, gather_positions);
        e->mark("gather");
        // (the step's parameter update waits for the next step's preprocess, or a flush)
    };
    // Segment B as a hipGraph (captured while the GPU runs segment A; an executable graph per step kind
    // is updated in place while the step's shape stays the same), unless per-kernel profiling is on or
    // the capacity is past what the device-count sort handles.
    auto graph_ok = [&]() { return e->use_graph && !e->prof && e->isect_cap < (size_t{1} << 30); };
    auto capture_b = [&]() {
        hipGraph_t g = nullptr;
        SXH_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        try {
            launch_b(static_cast<int64_t>(e->isect_cap), n_isects_dev);
        } catch (...) {
            (void)hipStreamEndCapture(s, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        SXH_HIP(hipStreamEndCapture(s, &g));
        hipGraphExec_t& x = e->graph_b[index_first ? 1 : 0][fwd_only ? 1 : 0];
        if (x) {
            hipGraphNode_t err_node = nullptr;
            hipGraphExecUpdateResult res{};
            if (hipGraphExecUpdate(x, g, &err_node, &res) != hipSuccess || res != hipGraphExecUpdateSuccess) {
                (void)hipGetLastError();
                SXH_HIP(hipGraphExecDestroy(x));
                x = nullptr;
            }
        }
        if (!x) {
            const hipError_t err = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            SXH_HIP(err);
        } else {
            SXH_HIP(hipGraphDestroy(g));
        }
    };
    // the render's copies, after segment B
    auto launch_tail = [&]() {
        if (render_to_dev)
            SXH_HIP(hipMemcpyAsync(render_to_dev, e->render.p, n_px * 4, hipMemcpyDeviceToDevice, s));
        if (out->render_colors)
            SXH_HIP(hipMemcpyAsync(out->render_colors, e->render.p, n_px * 4, hipMemcpyDeviceToHost, s));
        SXH_HIP(hipGetLastError());
    };

    // ---- sync 1: n_isects (MetalBackend.cpp:1849-1858) --------------------------------------------
    // With a graph, segment B is queued behind segment A before the host waits for the count (a word
    // the block scan stores into mapped host memory), so the GPU does not idle through the host's
    // wake-up. If the count
    // exceeds the capacity that segment B ran with (nothing done, arena untouched), the step runs again
    // the plain way: sync on the count, grow, capture, launch.
    int64_t n_isects = 0;
    bool done = false;
    e->sync_ms[0] = 0.0;
    if (graph_ok()) {
        const unsigned long long cap = e->isect_cap;
        launch_a(cap);
        upload_gt();
        capture_b();
        SXH_HIP(hipGraphLaunch(e->graph_b[index_first ? 1 : 0][fwd_only ? 1 : 0], s));
        launch_tail();
        const auto t0 = std::chrono::steady_clock::now();
        wait_count_word(hc + 4, seq, s, what);
        e->sync_ms[0] = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        n_isects = static_cast<int64_t>(hc[1]);
        validate_n_isects_readback(n_isects, what);
        done = static_cast<unsigned long long>(n_isects) <= cap;
        if (!done) SXH_HIP(hipStreamSynchronize(s));  // the overflowed pass ends before the buffers move
    } else {
        upload_gt();
    }
    if (!done) {
        launch_a(~0ull);
        const auto t0 = std::chrono::steady_clock::now();
        SXH_HIP(hipStreamSynchronize(s));
        e->sync_ms[0] += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        n_isects = static_cast<int64_t>(hc[1]);
        validate_n_isects_readback(n_isects, what);
        e->mark("sync1");
        e->ensure_isect(static_cast<size_t>(n_isects));
        if (graph_ok()) {
            capture_b();
            SXH_HIP(hipGraphLaunch(e->graph_b[index_first ? 1 : 0][fwd_only ? 1 : 0], s));
        } else {
            launch_b(n_isects, nullptr);
        }
        launch_tail();
    }
    if (!fwd_only) {  // segment B is queued: its update is this step's pending one
        e->update_pending = true;
        e->pending_c = c;
        e->steps_since_exchange++;
    }
    out->n_isects = n_isects;
    out->sort_key_bits = 32 + c.tile_n_bits;
    out->n_visible = static_cast<int64_t>(hc[0]);
    // ---- sync 2: loss (MetalBackend.cpp:2241-2261) ----------------------------------------------------
    // The loss, the sort's error word and the largest tile's count are stored by the gather's first
    // workgroup, with the step's sequence number after them: the host returns once it sees that
    // number, while the gather may still run. The step's parameter update is applied by the next step's preprocess or by a flush before
    // anything else reads or writes the arena (a download, a refine, a checkpoint, a sync). A render
    // read-back or profiling waits for the whole stream.
    const auto t0 = std::chrono::steady_clock::now();
    if (!e->prof && !e->prof_stats && !render_to_dev && !out->render_colors)
        wait_count_word(hc + 5, seq, s, what);
    else
        SXH_HIP(hipStreamSynchronize(s));
    e->sync_ms[1] = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    const uint32_t loss_bits = hw[0], sort_err = hw[1], max_tile = hw[2];
    float loss = 0.0f;
    std::memcpy(&loss, &loss_bits, 4);
    out->loss = fwd_only ? 0.0f : loss;
    e->last_max_tile = n_isects > 0 ? static_cast<int64_t>(max_tile) : 0;
    if (!fwd_only) e->last_long = static_cast<int64_t>(hw[3]);  // the previous training step's count
    if (e->prof_stats) {
        unsigned long long st[sxk::kRasterStats];
        SXH_HIP(hipMemcpy(st, e->rstats.p, sizeof(st), hipMemcpyDeviceToHost));
        e->rstats_host = sxh_raster_stats{st[sxk::kStatFwdIters],       st[sxk::kStatFwdEntries],
                                          st[sxk::kStatFwdTaken],       st[sxk::kStatBwdChunks],
                                          st[sxk::kStatBwdEntries],     st[sxk::kStatBwdEmptyChunks],
                                          st[sxk::kStatBwdInCutoff],    st[sxk::kStatBwdContrib]};
    }
    if (sort_err) throw std::runtime_error(std::string(what) + ": radix sort look-back did not complete");
    if (e->prof) {
        sxh_exec_timing& t = e->timing;
        t.n = 0;
        for (int k = 1; k < e->n_ev && t.n < 30; k++) {
            float ms = 0.f;
            // the interval ending at the sync1 mark is the host wait (reported below); segment B's first
            // interval starts at the sync1 event, which the stream reaches once the host launches again
            if (std::strcmp(e->ev_name[k], "sync1") == 0) continue;
            SXH_HIP(hipEventElapsedTime(&ms, e->ev[k - 1], e->ev[k]));
            t.names[t.n] = e->ev_name[k];
            t.ms[t.n++] = ms;
        }
        t.names[t.n] = "host_sync1_wait";
        t.ms[t.n++] = static_cast<float>(e->sync_ms[0]);
        t.names[t.n] = "host_sync2_wait";
        t.ms[t.n++] = static_cast<float>(e->sync_ms[1]);
    }
}

extern "C" {

int32_t sxh_exec_step(sxh_executor* e, const sxh_step_inputs* in, sxh_step_outputs* out) {
    return guarded([&] {
        if (!e) invalid("TrainStepExecutor::step", "null executor");
        SXH_HIP(hipSetDevice(e->b->device));
        sxh_detail::run_step(e, in, out, nullptr);
    });
}

int32_t sxh_exec_render_to_gt_cache(sxh_executor* e, const sxh_step_inputs* in, int32_t index) {
    return guarded([&] {
        if (!e || !in) invalid("TrainStepExecutor", "null argument");
        if (index < 0 || index >= e->gt_n) invalid("TrainStepExecutor", "GT cache index out of range");
        if (in->width != e->gt_w || in->height != e->gt_h) invalid("TrainStepExecutor", "GT cache image size mismatch");
        SXH_HIP(hipSetDevice(e->b->device));
        sxh_step_inputs f = *in;
        f.forward_only = 1;
        sxh_step_outputs o{};
        const size_t n_px = static_cast<size_t>(in->width) * in->height * 3;
        sxh_detail::run_step(e, &f, &o, e->gt_cache.p + static_cast<size_t>(index) * n_px);
        SXH_HIP(hipStreamSynchronize(e->b->stream));
    });
}

} // extern "C"
