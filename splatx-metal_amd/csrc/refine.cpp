// refine.cpp — sxh_exec_mcmc_refine: Trainer::mcmc_refine (Sources/SplatXCore/Trainer.cpp:1273-1280)
// run in place on the executor's arena, plus the noise tail step_resident runs after a refine
// (:960-967). The reference reclaims the whole arena to the host for this
// (sync_host_for_mutation, :911-914) and re-uploads it on the next step; here only the multinomial
// engine state (2.5 KB) and a few counters cross the bus.
//
// Phase order and semantics follow the reference exactly:
//   relocate (:1284-1338)  dead = sigmoid(logit) <= min_opacity; nothing to do without dead or
//                          without alive rows; sources = multinomial(alive, weight = opacity,
//                          n_dead draws); Eq.9 with ratio = min(bincount + 1, n_max); source
//                          opacity / scale <- the new values; dead row <- source row; Adam moments
//                          of the SOURCE rows <- 0 (not the dead rows).
//   add (:1342-1395)       n_add = min(cap_max, ceil(1.05 N)) - N; sources = multinomial(all N,
//                          n_add draws); Eq.9; row N + j <- source row; moments of the NEW rows <- 0
//                          (not the sources); count grows.
// Errors are raised before a phase mutates anything (the reference throws from inside its write
// loop for a non-positive scale; the condition and message are the same).
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "splatx_hip.h"
#include "sx_exec.h"
#include "sx_host.h"
#include "sx_kernels.h"
#include "sx_mcmc.h"

using namespace sxh;

namespace {

constexpr int kMtWords = 312;

void ensure_refine_buffers(sxh_executor* e, int n_max) {
    const size_t R = static_cast<size_t>(e->rows);
    if (e->mc_op_act.n < R) {
        e->mc_op_act.alloc(R);
        e->mc_new_logit.alloc(R);
        e->mc_new_log_scale.alloc(R * 3);
        e->mc_dead.alloc(R);
        e->mc_alive.alloc(R);
        e->mc_sampled.alloc(R);
        e->mc_counts.alloc(R);
        e->mc_cdf.alloc(R);
        e->mc_raw.alloc(R);
        e->mc_cdf_scratch.alloc(sxk::mc_cdf_scratch_bytes(static_cast<int64_t>(R)));
    }
    if (!e->mc_err.p) e->mc_err.alloc(1);
    if (!e->mc_total.p) e->mc_total.alloc(1);
    if (!e->mc_mt.p) e->mc_mt.alloc(kMtWords + 1);
    e->mc_binoms.ensure(static_cast<size_t>(n_max) * n_max);
}

// The refine's host-visible scalars, read back at its sync points.
struct Readback {
    int64_t cum_last;
    double total;
    uint32_t err;
};

struct Ctx {
    sxh_executor* e;
    hipStream_t s;
    Readback* hb;  // pinned
    sxk::Arena A;

    void clear_err() {
        // a one-word fill kernel rather than a memset node: callers may capture the stream
        sxk::fill_u32(e->mc_err.p, 0u, 1, s);
    }
    void read_err_and_total(bool total) {
        SXH_HIP(hipMemcpyAsync(&hb->err, e->mc_err.p, 4, hipMemcpyDeviceToHost, s));
        if (total) SXH_HIP(hipMemcpyAsync(&hb->total, e->mc_total.p, 8, hipMemcpyDeviceToHost, s));
        SXH_HIP(hipStreamSynchronize(s));
    }
};

void put_list(int64_t* dst, const int32_t* dev, int64_t n, hipStream_t s) {
    if (!dst || n <= 0) return;
    std::vector<int32_t> tmp(static_cast<size_t>(n));
    SXH_HIP(hipMemcpyAsync(tmp.data(), dev, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost, s));
    SXH_HIP(hipStreamSynchronize(s));
    for (int64_t i = 0; i < n; i++) dst[i] = tmp[static_cast<size_t>(i)];
}

// multinomial_with_replacement (Trainer.cpp:1199-1218) + run_relocation_for (:1231-1258): draws
// n_draw sources over the n_w weights op_act[gather[i]] (op_act[i] without gather), then computes
// the new logit / log-scale of every draw. Nothing in the arena is written; errors are raised
// after the engine state has been handed back (the reference's engine has advanced as well).
void draw_and_relocate(Ctx& c, const sxh_refine_inputs* in, const int32_t* gather, int64_t n_w, int64_t n_draw,
                       const char* what_scale) {
    sxh_executor* e = c.e;
    hipStream_t s = c.s;
    c.clear_err();
    sxk::mc_cdf(e->mc_op_act.p, gather, n_w, e->mc_cdf.p, e->mc_total.p, e->mc_err.p, e->mc_cdf_scratch.p, s);
    c.read_err_and_total(true);
    if (c.hb->err & sxk::kMcErrWeights) invalid("multinomial", "weights must be >= 0 and finite");
    if (!(c.hb->total > 0.0)) invalid("multinomial", "weight sum must be > 0");
    sxk::mc_mt_gen(e->mc_mt.p, n_draw, e->mc_raw.p, s);
    sxk::fill_u32(e->mc_counts.p, 0u, e->rows, s);
    sxk::mc_search(e->mc_raw.p, n_draw, e->mc_cdf.p, n_w, e->mc_total.p, gather, e->mc_sampled.p, e->mc_counts.p, s);
    sxk::mc_reloc(e->mc_sampled.p, static_cast<int>(n_draw), e->mc_counts.p, e->mc_op_act.p, c.A.p[2], e->rows,
                  e->mc_binoms.p, in->n_max, in->min_opacity, e->mc_new_logit.p, e->mc_new_log_scale.p, e->mc_err.p,
                  s);
    // the engine has advanced whatever happens next: hand its state back now
    SXH_HIP(hipMemcpyAsync(in->rng->x, e->mc_mt.p, kMtWords * 8, hipMemcpyDeviceToHost, s));
    uint64_t p = 0;
    SXH_HIP(hipMemcpyAsync(&p, e->mc_mt.p + kMtWords, 8, hipMemcpyDeviceToHost, s));
    c.read_err_and_total(false);
    in->rng->p = static_cast<uint32_t>(p);
    if (c.hb->err & sxk::kMcErrScale) throw std::logic_error(std::string(what_scale) + ": non-positive new_scale");
    if (c.hb->err & sxk::kMcErrLogit) invalid("logit_f32", "p must be in (0,1)");
}

}  // namespace

extern "C" {

int32_t sxh_mt64_seed(uint64_t seed, sxh_mt64_state* out) {
    return guarded([&] {
        if (!out) invalid("sxh_mt64_seed", "null output");
        // std::mersenne_twister_engine::seed (C++ [rand.eng.mers]): x0 = seed,
        // x_i = f * (x_{i-1} xor (x_{i-1} >> (w-2))) + i with f = 6364136223846793005, w = 64
        out->x[0] = seed;
        for (int i = 1; i < kMtWords; i++)
            out->x[i] = 6364136223846793005ull * (out->x[i - 1] ^ (out->x[i - 1] >> 62)) + static_cast<uint64_t>(i);
        out->p = kMtWords;
    });
}

int32_t sxh_running_sum_f64(sxh_backend* b, const float* w, int64_t n, double* out) {
    return guarded([&] {
        if (!b) invalid("running_sum_f64", "null backend");
        if (n < 0) invalid("running_sum_f64", "negative n");
        if (n == 0) return;
        if (!w || !out) invalid("running_sum_f64", "null w/out");
        SXH_HIP(hipSetDevice(b->device));
        auto dw = upload(w, static_cast<size_t>(n), b->stream);
        DevBuf<double> cdf(static_cast<size_t>(n)), total(1);
        DevBuf<uint32_t> err(1);
        DevBuf<uint8_t> scratch(sxk::mc_cdf_scratch_bytes(n));
        sxk::fill_u32(err.p, 0u, 1, b->stream);
        sxk::mc_cdf(dw.p, nullptr, n, cdf.p, total.p, err.p, scratch.p, b->stream);
        SXH_HIP(hipGetLastError());
        uint32_t herr = 0;
        SXH_HIP(hipMemcpyAsync(&herr, err.p, 4, hipMemcpyDeviceToHost, b->stream));
        download(out, cdf, static_cast<size_t>(n), b->stream);
        SXH_HIP(hipStreamSynchronize(b->stream));
        if (herr & sxk::kMcErrWeights) invalid("running_sum_f64", "weights must be >= 0 and finite");
    });
}

int32_t sxh_mt64_draw(sxh_backend* b, sxh_mt64_state* st, int64_t n, uint64_t* out) {
    return guarded([&] {
        if (!b || !st) invalid("mt64_draw", "null argument");
        if (n < 0) invalid("mt64_draw", "negative n");
        if (st->p > kMtWords) invalid("mt64_draw", "malformed state");
        if (n == 0) return;
        if (!out) invalid("mt64_draw", "null out");
        SXH_HIP(hipSetDevice(b->device));
        DevBuf<uint64_t> state(kMtWords + 1), raw(static_cast<size_t>(n)), tempered(static_cast<size_t>(n));
        uint64_t host_state[kMtWords + 1];
        std::memcpy(host_state, st->x, sizeof(st->x));
        host_state[kMtWords] = st->p;
        SXH_HIP(hipMemcpyAsync(state.p, host_state, sizeof(host_state), hipMemcpyHostToDevice, b->stream));
        sxk::mc_mt_gen(state.p, n, raw.p, b->stream);
        sxk::mc_temper(raw.p, n, tempered.p, b->stream);
        SXH_HIP(hipGetLastError());
        download(out, tempered, static_cast<size_t>(n), b->stream);
        SXH_HIP(hipMemcpyAsync(host_state, state.p, sizeof(host_state), hipMemcpyDeviceToHost, b->stream));
        SXH_HIP(hipStreamSynchronize(b->stream));
        std::memcpy(st->x, host_state, sizeof(st->x));
        st->p = static_cast<uint32_t>(host_state[kMtWords]);
    });
}

int32_t sxh_exec_mcmc_refine(sxh_executor* e, const sxh_refine_inputs* in, sxh_refine_outputs* out) {
    return guarded([&] {
        const char* what = "TrainStepExecutor::mcmc_refine";
        if (!e || !in || !out) invalid(what, "null argument");
        if (in->count < 1 || in->count > e->rows) invalid(what, "count out of [1, arena_rows]");
        if (in->cap_max < in->count || in->cap_max > e->rows) invalid(what, "cap_max out of [count, arena_rows]");
        // Trainer.cpp:682-683
        if (!(in->min_opacity > 0.0f && in->min_opacity < 1.0f)) invalid(what, "min_opacity must be in (0,1)");
        if (in->n_max < 1 || in->n_max > 64) invalid(what, "n_max must be in [1,64]");
        if (!in->binoms) invalid(what, "null binoms");
        if (!in->rng || in->rng->p > kMtWords) invalid(what, "null or malformed rng state");
        if (out->capacity < 0) invalid(what, "negative capacity");
        SXH_HIP(hipSetDevice(e->b->device));
        sxh_detail::canonicalize(e);  // the refine reads the step's updated rows, in the caller's order
        ensure_refine_buffers(e, in->n_max);
        hipStream_t s = e->b->stream;
        Ctx c{e, s, static_cast<Readback*>(e->host_small.p), e->arena()};
        const int N = static_cast<int>(in->count);
        SXH_HIP(hipMemcpyAsync(e->mc_binoms.p, in->binoms, static_cast<size_t>(in->n_max) * in->n_max * 4,
                               hipMemcpyHostToDevice, s));
        SXH_HIP(hipMemcpyAsync(e->mc_mt.p, in->rng->x, kMtWords * 8, hipMemcpyHostToDevice, s));
        const uint64_t p_word = in->rng->p;
        SXH_HIP(hipMemcpyAsync(e->mc_mt.p + kMtWords, &p_word, 8, hipMemcpyHostToDevice, s));
        out->count = in->count;
        out->n_relocated = 0;
        out->n_added = 0;

        // ---- relocate (Trainer.cpp:1284-1338) --------------------------------------------------
        c.clear_err();
        sxk::mc_activate(c.A.p[3], N, in->min_opacity, e->mc_op_act.p, e->tiles.p, e->mc_err.p, s);
        sxk::scan_i32_i64(e->tiles.p, e->cum.p, N, e->scan_scratch.p, s);
        SXH_HIP(hipMemcpyAsync(&c.hb->cum_last, e->cum.p + (N - 1), 8, hipMemcpyDeviceToHost, s));
        c.read_err_and_total(false);
        const int64_t n_dead = c.hb->cum_last, n_alive = N - n_dead;
        const uint32_t nan_seen = c.hb->err & sxk::kMcErrWeights;
        const int64_t n_target = std::min<int64_t>(in->cap_max, (in->count * 21 + 19) / 20);  // :1346-1348
        const int64_t n_add = n_target - in->count;
        if (n_dead > 0 && n_alive > 0) {
            if (nan_seen) invalid("multinomial", "weights must be >= 0 and finite");
            if ((out->relocated_dead || out->relocation_src) && out->capacity < n_dead)
                throw CapacityError(std::string(what) + ": relocation lists need " + std::to_string(n_dead) +
                                    " entries");
        }
        if (n_add > 0 && out->added_src && out->capacity < n_add)
            throw CapacityError(std::string(what) + ": added_src needs " + std::to_string(n_add) + " entries");
        if (n_dead > 0 && n_alive > 0) {
            sxk::mc_compact(e->tiles.p, e->cum.p, N, e->mc_dead.p, e->mc_alive.p, s);
            draw_and_relocate(c, in, e->mc_alive.p, n_alive, n_dead, "Trainer::mcmc_relocate");
            const int nd = static_cast<int>(n_dead);
            sxk::mc_apply(e->mc_sampled.p, nd, e->mc_new_logit.p, e->mc_new_log_scale.p, c.A.p[3], c.A.p[2], e->rows,
                          s);
            sxk::mc_copy_rows(c.A, e->dims, e->mc_dead.p, 0, e->mc_sampled.p, nd, s);
            sxk::mc_zero_rows(c.A, e->dims, e->mc_sampled.p, 0, nd, s);
            put_list(out->relocated_dead, e->mc_dead.p, n_dead, s);
            put_list(out->relocation_src, e->mc_sampled.p, n_dead, s);
            out->n_relocated = n_dead;
        }

        // ---- add (Trainer.cpp:1342-1395) -------------------------------------------------------
        if (n_add > 0) {
            c.clear_err();
            sxk::mc_activate(c.A.p[3], N, in->min_opacity, e->mc_op_act.p, nullptr, e->mc_err.p, s);
            draw_and_relocate(c, in, nullptr, N, n_add, "Trainer::mcmc_add");
            const int na = static_cast<int>(n_add);
            sxk::mc_apply(e->mc_sampled.p, na, e->mc_new_logit.p, e->mc_new_log_scale.p, c.A.p[3], c.A.p[2], e->rows,
                          s);
            sxk::mc_copy_rows(c.A, e->dims, nullptr, N, e->mc_sampled.p, na, s);
            sxk::mc_zero_rows(c.A, e->dims, nullptr, N, na, s);
            put_list(out->added_src, e->mc_sampled.p, n_add, s);
            out->n_added = n_add;
            out->count = in->count + n_add;
        }

        // ---- noise after the refine, over the new count (Trainer.cpp:966, 1400-1418) -------------
        if (in->inject_noise)
            sxk::mc_noise(c.A, static_cast<int>(out->count), in->noise_seed, in->noise_offset, in->noise_scale, s);
        SXH_HIP(hipGetLastError());
        SXH_HIP(hipStreamSynchronize(s));
    });
}

}  // extern "C"
