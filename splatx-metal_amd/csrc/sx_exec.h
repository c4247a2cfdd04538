// sx_exec.h — the device-resident executor object (TrainStepExecutor state), shared by the step
// (executor.cpp) and the device MCMC refine (refine.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <cstring>

#include "splatx_hip.h"
#include "sx_host.h"
#include "sx_kernels.h"
#include "sx_step.h"

namespace sxh_detail {

// Pinned host memory, zeroed at allocation: the runtime may hand back a block a destroyed executor
// used, and the step's read-back words are tagged with sequence numbers that every executor starts
// from 1 again, so a stale tag would end a wait before the new step stored its words.
struct PinnedHost {
    void* p = nullptr;
    void* dev = nullptr;  // the device's address of the block (mapped memory)
    explicit PinnedHost(size_t bytes, unsigned flags = hipHostMallocDefault) {
        SXH_HIP(hipHostMalloc(&p, bytes, flags));
        std::memset(p, 0, bytes);
        if (flags & hipHostMallocMapped) SXH_HIP(hipHostGetDevicePointer(&dev, p, 0));
    }
    ~PinnedHost() {
        if (p) (void)hipHostFree(p);
    }
    PinnedHost(const PinnedHost&) = delete;
    PinnedHost& operator=(const PinnedHost&) = delete;
};

constexpr int kMaxEvents = 32;

} // namespace sxh_detail

using sxh_detail::PinnedHost;
using sxh_detail::kMaxEvents;

struct sxh_executor {
    sxh_backend* b = nullptr;
    sxh_exec_desc d{};
    int n_coeffs = 1;
    int dims[6] = {3, 4, 3, 1, 3, 0};
    int rows = 0;
    std::atomic<int> stop_requested{0};  // sxh_exec_request_stop -> the caller loop's next boundary
    sxh::DevBuf<float> p[6], m[6], v[6];
    sxh::DevBuf<float4> splats, grads;
    sxh::DevBuf<int32_t> radii, tiles;
    sxh::DevBuf<int64_t> cum;
    sxh::DevBuf<int32_t> long_list;          // gradient gather: the depth positions of long entry ranges
    sxh::DevBuf<int32_t> long_count;
    sxh::DevBuf<uint8_t> touched;            // rows the raster backward reached this step
    sxh::DevBuf<uint32_t> dkey_a, dkey_b;    // depth sort keys
    sxh::DevBuf<int32_t> order_a, order_b;   // Gaussian indices in depth order
    sxh::DevBuf<uint8_t> scan_scratch;
    sxh::DevBuf<unsigned long long> n_vis;     // visible count, intersections, Gaussians with tiles
    sxh::DevBuf<uint32_t> vis_part;            // preprocess per-block counts
    sxh::DevBuf<unsigned long long> blk_base;  // their prefixes (intersections, Gaussians with tiles)
    sxh::DevBuf<int32_t> emit_list;            // the Gaussians with tiles, in index order
    // intersections (grow 1.5x, reused)
    size_t isect_cap = 0;
    sxh::DevBuf<uint64_t> keys_a, keys_b;
    sxh::DevBuf<int32_t> vals_a, vals_b;   // sorted: emit positions
    sxh::DevBuf<int32_t> emit_gid;         // the Gaussian of each emit position
    sxh::DevBuf<float> part;               // raster backward sums per emit position (kPartStride floats each)
    sxh::DevBuf<uint32_t> stamp;           // the current backward's stamp (one word; entries carry it)
    sxh::DevBuf<uint8_t> sort_scratch;
    // image-sized buffers
    size_t img_px = 0, img_tiles = 0, img_map = 0;
    sxh::DevBuf<int32_t> offsets, last_ids, tile_order, mask_end;
    sxh::DevBuf<float> render, alpha, v_render, v_alpha_zero, gt_stage;
    sxh::DevBuf<float> cmu, csg, ccr;  // SSIM coefficient maps (the map itself is only summed)
    sxh::DevBuf<double> ssim_part, l1_part;
    sxh::DevBuf<float> loss_dev;
    // GT cache
    sxh::DevBuf<float> gt_cache;
    int gt_n = 0, gt_w = 0, gt_h = 0;
    sxh::DevBuf<float> staging;
    PinnedHost host_small{64};
    // the step's counts and read-back words, stored by its kernels (coherent, mapped): u64 visible, u64
    // intersections, then u32 loss bits, sort error flag, largest tile's entry count
    PinnedHost step_rb{64, hipHostMallocMapped | hipHostMallocCoherent};
    // device MCMC refine (allocated on the first refine, arena-sized)
    sxh::DevBuf<float> mc_op_act, mc_new_logit, mc_new_log_scale, mc_binoms;
    sxh::DevBuf<int32_t> mc_dead, mc_alive, mc_sampled;
    sxh::DevBuf<uint32_t> mc_counts, mc_err;
    sxh::DevBuf<double> mc_cdf, mc_total;
    sxh::DevBuf<uint64_t> mc_raw, mc_mt;
    sxh::DevBuf<uint8_t> mc_cdf_scratch;
    // segment B of the step as executable graphs: [index-first][0 training step, 1 forward only]
    hipGraphExec_t graph_b[2][2] = {{nullptr, nullptr}, {nullptr, nullptr}};
    bool use_graph = true;
    // test switch (environment SXH_DEBUG_FORCE_SORT_ERROR=1 at creation): after the tile sort, a kernel
    // sets the sort's error word, as a sort that gave up would; every kernel still runs to its end
    bool debug_sort_error = false;
    int isect_order = SXH_ISECT_ORDER_AUTO;
    // The last training step's parameter update is deferred: the next training step applies it in its
    // preprocess, row by row in the same pass over the arena (step_update_preprocess); anything else that
    // reads or writes the arena applies it first (sxh_detail::flush_update). pending_c: that step's
    // constants.
    bool update_pending = false;
    sxk::StepConst pending_c{};
    // The live rows' order in HBM (sxh_exec_set_row_order, k_perm.hip). With `permuted`, internal row k
    // of the live rows [0, perm_count) holds original row row_orig[k], and row_int is the inverse;
    // steps_since_exchange counts the training steps since the last call that exchanged rows with the
    // caller (which restores the original order: sxh_detail::canonicalize).
    int row_order = SXH_ROW_ORDER_SPATIAL_AUTO;
    bool permuted = false;
    int perm_count = 0;
    int64_t steps_since_exchange = 0;
    sxh::DevBuf<int32_t> row_orig, row_int, tiles_o;  // tiles_o: the tile counts in original order
    sxh::DevBuf<float> perm_scratch;
    int64_t last_max_tile = -1;      // the largest tile's entry count in the previous step (-1: none yet)
    int64_t last_long = -1;          // the previous training step's gather ranges past kLongRange (-1: none yet)
    sxh::DevBuf<uint32_t> max_tile;  // written by the step's tile order
    // profiling: per-kernel events (bit 0), raster pair counts (bit 1)
    bool prof = false;
    bool prof_stats = false;
    sxh::DevBuf<unsigned long long> rstats;
    sxh_raster_stats rstats_host{};
    hipEvent_t ev[kMaxEvents] = {};
    unsigned long long step_seq = 0;  // segment A launches so far (the tag of the step's count word)
    const char* ev_name[kMaxEvents] = {};
    int n_ev = 0;
    sxh_exec_timing timing{};
    double sync_ms[2] = {0, 0};

    sxk::Arena arena() {
        sxk::Arena A{};
        for (int g = 0; g < 6; g++) {
            A.p[g] = p[g].p;
            A.m[g] = m[g].p;
            A.v[g] = v[g].p;
        }
        A.rows = rows;
        return A;
    }

    void mark(const char* name) {
        if (!prof || n_ev >= kMaxEvents) return;
        SXH_HIP(hipEventRecord(ev[n_ev], b->stream));
        ev_name[n_ev++] = name;
    }

    void ensure_isect(size_t n) {
        if (n <= isect_cap) return;
        const size_t cap = std::max<size_t>(n + n / 2, 1 << 16);
        keys_a.alloc(cap);
        keys_b.alloc(cap);
        vals_a.alloc(cap);
        vals_b.alloc(cap);
        emit_gid.alloc(cap);
        part.alloc(cap * sxk::kPartStride);
        // zero stamps: no entry of the new buffer passes for one written this step (stamps are never 0)
        SXH_HIP(hipMemsetAsync(part.p, 0, cap * sxk::kPartStride * sizeof(float), b->stream));
        // shared by the depth sort (rows keys) and the tile sort (intersections)
        sort_scratch.alloc(sxk::sort_scratch_bytes(static_cast<int64_t>(std::max<size_t>(cap, rows))));
        isect_cap = cap;
    }

    void ensure_image(int W, int H, bool use_ssim) {
        const size_t px = static_cast<size_t>(W) * H;
        const size_t tiles_n = static_cast<size_t>((W + 15) / 16) * ((H + 15) / 16);
        const size_t map_n = use_ssim ? static_cast<size_t>(H - 10) * (W - 10) * 3 : 0;
        if (px > img_px) {
            render.alloc(px * 3);
            alpha.alloc(px);
            last_ids.alloc(px);
            v_render.alloc(px * 3);
            v_alpha_zero.alloc(px);
            SXH_HIP(hipMemsetAsync(v_alpha_zero.p, 0, px * sizeof(float), b->stream));
            gt_stage.alloc(px * 3);
            img_px = px;
        }
        // one f64 partial per workgroup of the loss kernels (exact counts of their grids)
        const size_t l1_blocks = std::max<size_t>(sxk::step_ssim_bwd_blocks(H, W),
                                                  sxk::step_l1_blocks(static_cast<int64_t>(px) * 3));
        if (l1_blocks > l1_part.n) l1_part.alloc(l1_blocks);
        if (tiles_n > img_tiles) {
            offsets.alloc(tiles_n);
            tile_order.alloc(tiles_n);
            mask_end.alloc(tiles_n);
            img_tiles = tiles_n;
        }
        if (use_ssim) {
            if (map_n > img_map) {
                cmu.alloc(map_n);
                csg.alloc(map_n);
                ccr.alloc(map_n);
                img_map = map_n;
            }
            const size_t ss_blocks = static_cast<size_t>(sxk::ssim_fwd_blocks(1, H, W, 3));
            if (ss_blocks > ssim_part.n) ssim_part.alloc(ss_blocks);
        }
    }
};

namespace sxh_detail {
// One training (or forward-only) step of the executor; render_to_dev, when not null, receives a
// device copy of the render. Defined in executor.cpp.
void run_step(sxh_executor* e, const sxh_step_inputs* in, sxh_step_outputs* out, float* render_to_dev);
// The deferred parameter update of the last training step, if one is pending, as its own launch on the
// executor's stream (ordered before whatever is queued after it). Defined in executor.cpp.
void flush_update(sxh_executor* e);
// Before a call exchanges rows with the caller: flush_update, then the arena back in the caller's row
// order if it is in spatial order. Defined in executor.cpp.
void canonicalize(sxh_executor* e);
}  // namespace sxh_detail
