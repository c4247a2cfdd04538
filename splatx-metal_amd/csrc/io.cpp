// io.cpp — the data formats either side of the step, over the executor's device arena:
//   * INRIA PLY export with its filter (write_inria_ply + filter_cloud_for_export, PlyIO.h:20-51)
//     and the PLY reader (read_inria_ply, PlyIO.h:21);
//   * SXCK checkpoints (Checkpoint.h:11-147: save_checkpoint_file, load_checkpoint_file,
//     load_checkpoint_header, verify_checkpoint_config; the snapshot and restore of
//     Trainer::make_checkpoint / restore_checkpoint, Trainer.cpp:1450-1570);
//   * forward-only render sessions (sx_render_session_*, splatx_train_c.h:604-682).
// The byte layouts (PLY header text and row order, checkpoint field order) are the formats' own;
// the filtering, compaction and packing of rows and tensors happen on the device (k_io.hip), and
// the host only frames and writes the bytes.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "splatx_hip.h"
#include "sx_exec.h"
#include "sx_host.h"
#include "sx_io.h"
#include "sx_kernels.h"

using namespace sxh;

namespace {

constexpr size_t kChunkBytes = size_t{32} << 20;  // pinned host bounce buffer per transfer

struct HostFile {
    std::FILE* f = nullptr;
    HostFile(const std::string& path, const char* mode, const char* what) : f(std::fopen(path.c_str(), mode)) {
        if (!f) throw std::runtime_error(std::string(what) + ": cannot open " + path);
    }
    ~HostFile() {
        if (f) std::fclose(f);
    }
    HostFile(const HostFile&) = delete;
    HostFile& operator=(const HostFile&) = delete;
    void close_checked(const std::string& path, const char* what) {
        const int rc = std::fclose(f);
        f = nullptr;
        if (rc != 0) throw std::runtime_error(std::string(what) + ": close/flush failed for " + path);
    }
};

void put_bytes(std::FILE* f, const void* p, size_t n, const char* what) {
    if (n && std::fwrite(p, 1, n, f) != n) throw std::runtime_error(std::string(what) + ": write failed");
}
void get_bytes(std::FILE* f, void* p, size_t n) {
    if (n && std::fread(p, 1, n, f) != n) throw std::runtime_error("checkpoint: truncated file (short read)");
}
template <class T>
void put_pod(std::FILE* f, T v, const char* what) {
    put_bytes(f, &v, sizeof(T), what);
}
template <class T>
T get_pod(std::FILE* f) {
    T v;
    get_bytes(f, &v, sizeof(T));
    return v;
}

sxk::Dims6 dims_of(const sxh_executor* e) {
    sxk::Dims6 d{};
    for (int g = 0; g < 6; g++) d.d[g] = e->dims[g];
    return d;
}

// The pinned bounce buffer shared by the transfers of one call.
struct Bounce {
    PinnedHost host{kChunkBytes};
    void* p() const { return host.p; }
};

// ---------------------------------------------------------------------------------------------
// SXCK layout constants (Checkpoint.h:11-19)
constexpr char kMagic[4] = {'S', 'X', 'C', 'K'};
constexpr uint32_t kVersion = 1;
constexpr uint32_t kFlagFp16 = 1u;

std::string num(double v) {
    char b[40];
    std::snprintf(b, sizeof(b), "%.9g", v);
    return b;
}

[[noreturn]] void mismatch(const char* field, const std::string& saved, const std::string& current,
                           const char* why = nullptr) {
    std::string m = std::string("checkpoint resume: ") + field + " mismatch (saved " + saved + ", current " + current +
                    ")";
    if (why) m += std::string(" — ") + why;
    throw std::runtime_error(m);
}

// verify_checkpoint_config (Checkpoint.cpp) — same field order and conditions
void verify_config(const sxh_checkpoint_config& s, const sxh_checkpoint_config& c) {
    if (s.sh_degree != c.sh_degree)
        mismatch("sh_degree", std::to_string(s.sh_degree), std::to_string(c.sh_degree),
                 "resume enforces fixed SH degree (design §8.1 — color corruption incident lesson)");
    if (s.mcmc_enabled != c.mcmc_enabled) mismatch("mcmc", s.mcmc_enabled ? "on" : "off", c.mcmc_enabled ? "on" : "off");
    if (s.cap_max != c.cap_max) mismatch("cap_max", std::to_string(s.cap_max), std::to_string(c.cap_max));
    if (s.mcmc_seed != c.mcmc_seed)
        mismatch("mcmc seed", std::to_string(s.mcmc_seed), std::to_string(c.mcmc_seed),
                 "noise(Philox key)/multinomial stream would diverge");
    if (s.factor != c.factor) mismatch("factor", std::to_string(s.factor), std::to_string(c.factor));
    if (s.test_split != c.test_split)
        mismatch("test_split", std::to_string(s.test_split), std::to_string(c.test_split),
                 "train view stream (it % n_train) would diverge and trained views would leak into the test split");
    if (s.total_iters != c.total_iters)
        mismatch("total_iters", std::to_string(s.total_iters), std::to_string(c.total_iters),
                 "ratio schedules (lr decay/SH promotion/refine) are normalized by total_iters — resume iter "
                 "would change meaning");
    if (s.scene_scale != c.scene_scale) mismatch("scene_scale", num(s.scene_scale), num(c.scene_scale));
    if (s.ssim_weight != c.ssim_weight) mismatch("ssim_weight", num(s.ssim_weight), num(c.ssim_weight));
    if (s.antialiased != c.antialiased) mismatch("antialiased", s.antialiased ? "on" : "off", c.antialiased ? "on" : "off");
}

// magic .. alive_count, with the format's checks (Checkpoint.cpp read_header)
sxh_checkpoint_header read_header(std::FILE* f, const std::string& path) {
    char magic[4];
    get_bytes(f, magic, 4);
    if (std::memcmp(magic, kMagic, 4) != 0)
        throw std::runtime_error("checkpoint: bad magic (not a splatx checkpoint): " + path);
    sxh_checkpoint_header h{};
    h.version = get_pod<uint32_t>(f);
    if (h.version != kVersion)
        throw std::runtime_error("checkpoint: unsupported version " + std::to_string(h.version) + " (expected " +
                                 std::to_string(kVersion) + ")");
    const uint32_t flags = get_pod<uint32_t>(f);
    if (flags & ~kFlagFp16) throw std::runtime_error("checkpoint: unknown flags");
    h.fp16 = (flags & kFlagFp16) ? 1 : 0;
    h.config.sh_degree = get_pod<int32_t>(f);
    h.config.factor = get_pod<int32_t>(f);
    h.config.test_split = get_pod<int32_t>(f);
    h.config.total_iters = get_pod<int32_t>(f);
    h.config.mcmc_enabled = get_pod<uint8_t>(f);
    h.config.antialiased = get_pod<uint8_t>(f);
    if (get_pod<uint8_t>(f) != 0)  // the reserved byte: only 0 is a valid file
        throw std::runtime_error("checkpoint: bilateral grid checkpoints are no longer supported (feature removed): " +
                                 path);
    (void)get_pod<uint8_t>(f);  // alignment byte
    h.config.cap_max = get_pod<int64_t>(f);
    h.config.mcmc_seed = get_pod<uint64_t>(f);
    h.config.scene_scale = get_pod<float>(f);
    h.config.ssim_weight = get_pod<float>(f);
    if (h.config.sh_degree < 0 || h.config.sh_degree > 3) throw std::runtime_error("checkpoint: sh_degree out of [0,3]");
    h.iter = get_pod<int32_t>(f);
    if (h.iter < 0) throw std::runtime_error("checkpoint: negative iter");
    h.alive_count = get_pod<int64_t>(f);
    if (h.alive_count < 1 || h.alive_count > (int64_t{1} << 33)) throw std::runtime_error("checkpoint: invalid count");
    return h;
}

int64_t group_dim(int g, int sh_degree) {
    constexpr int64_t fixed[5] = {3, 4, 3, 1, 3};
    return g < 5 ? fixed[g] : (static_cast<int64_t>(sh_degree) + 1) * (sh_degree + 1) * 3 - 3;
}

// device arrays of one group <-> the file, chunked through the pinned bounce buffer
void save_group(sxh_executor* e, Bounce& bb, std::FILE* f, const float* soa, int dim, int64_t n, int mode) {
    if (dim == 0 || n == 0) return;
    const size_t esz = mode == sxk::kCkptF32 ? 4 : 2;
    const int64_t rows_per = std::max<int64_t>(1, static_cast<int64_t>(kChunkBytes / (esz * dim)));
    hipStream_t s = e->b->stream;
    for (int64_t r0 = 0; r0 < n; r0 += rows_per) {
        const int64_t rows = std::min(rows_per, n - r0);
        sxk::ckpt_pack(soa, e->rows, dim, r0, rows, mode, e->staging.p, s);
        SXH_HIP(hipMemcpyAsync(bb.p(), e->staging.p, rows * dim * esz, hipMemcpyDeviceToHost, s));
        SXH_HIP(hipStreamSynchronize(s));
        put_bytes(f, bb.p(), rows * dim * esz, "checkpoint");
    }
}

void load_group(sxh_executor* e, Bounce& bb, std::FILE* f, float* soa, int dim, int64_t n, int mode) {
    if (dim == 0 || n == 0) return;
    const size_t esz = mode == sxk::kCkptF32 ? 4 : 2;
    const int64_t rows_per = std::max<int64_t>(1, static_cast<int64_t>(kChunkBytes / (esz * dim)));
    hipStream_t s = e->b->stream;
    for (int64_t r0 = 0; r0 < n; r0 += rows_per) {
        const int64_t rows = std::min(rows_per, n - r0);
        SXH_HIP(hipStreamSynchronize(s));  // the bounce buffer is free again
        get_bytes(f, bb.p(), rows * dim * esz);
        SXH_HIP(hipMemcpyAsync(e->staging.p, bb.p(), rows * dim * esz, hipMemcpyHostToDevice, s));
        sxk::ckpt_unpack(e->staging.p, mode, soa, e->rows, dim, r0, rows, s);
    }
    SXH_HIP(hipStreamSynchronize(s));
}

void fsync_dir_of(const std::string& path) {  // best effort, as the format's writer does
    std::string dir = ".";
    if (const size_t slash = path.find_last_of('/'); slash != std::string::npos) dir = slash == 0 ? "/" : path.substr(0, slash);
    const int fd = ::open(dir.c_str(), O_RDONLY);
    if (fd >= 0) {
        (void)::fsync(fd);
        (void)::close(fd);
    }
}

// ---------------------------------------------------------------------------------------------
// read_inria_ply (PlyIO.h:21): float properties only, binary little endian, degree from f_rest
struct PlyCloud {
    int64_t count = 0;
    int sh_degree = 0;
    std::vector<float> g[6];  // AoS per group
};

PlyCloud read_ply(const std::string& path, bool want_data) {
    HostFile file(path, "rb", "ply");
    std::FILE* f = file.f;
    std::vector<std::string> props;
    int64_t count = 0;
    bool binary_le = false;
    char line[512];
    for (;;) {
        if (!std::fgets(line, sizeof(line), f)) throw std::runtime_error("ply: bad header");
        std::string s(line);
        while (!s.empty() && (s.back() == '\n' || s.back() == '\r')) s.pop_back();
        if (s == "end_header") break;
        if (s.rfind("format ", 0) == 0) binary_le = s == "format binary_little_endian 1.0";
        else if (s.rfind("element vertex ", 0) == 0) count = std::stoll(s.substr(15));
        else if (s.rfind("property float ", 0) == 0) props.push_back(s.substr(15));
        else if (s.rfind("property ", 0) == 0)
            throw std::runtime_error("ply: only float properties supported (found: " + s + ")");
    }
    if (!binary_le) throw std::runtime_error("ply: only binary_little_endian supported");
    std::map<std::string, size_t> idx;
    for (size_t i = 0; i < props.size(); i++) idx[props[i]] = i;
    int rest = 0;
    while (idx.count("f_rest_" + std::to_string(rest))) rest++;
    if (rest % 3 != 0) throw std::runtime_error("ply: f_rest not divisible by 3");
    const int K = rest / 3;
    int degree = -1;
    for (int d = 0; d <= 4; d++)
        if ((d + 1) * (d + 1) - 1 == K) degree = d;
    if (degree < 0) throw std::runtime_error("ply: unsupported f_rest count " + std::to_string(rest));
    PlyCloud c;
    c.count = count;
    c.sh_degree = degree;
    if (!want_data) return c;
    const auto col = [&](const std::string& n) -> size_t {
        const auto it = idx.find(n);
        if (it == idx.end()) throw std::runtime_error("ply: missing property " + n);
        return it->second;
    };
    // column index of every destination element (group order, AoS within a group)
    std::vector<size_t> src[6];
    for (int k = 0; k < 3; k++) src[0].push_back(col(std::string(1, "xyz"[k])));
    for (int k = 0; k < 4; k++) src[1].push_back(col("rot_" + std::to_string(k)));
    for (int k = 0; k < 3; k++) src[2].push_back(col("scale_" + std::to_string(k)));
    src[3].push_back(col("opacity"));
    for (int k = 0; k < 3; k++) src[4].push_back(col("f_dc_" + std::to_string(k)));
    for (int k = 0; k < K; k++)  // shN [K,3] from the channel-major f_rest
        for (int ch = 0; ch < 3; ch++) src[5].push_back(col("f_rest_" + std::to_string(ch * K + k)));
    for (int g = 0; g < 6; g++) c.g[g].resize(static_cast<size_t>(count) * src[g].size());
    std::vector<float> row(props.size());
    for (int64_t i = 0; i < count; i++) {
        if (std::fread(row.data(), 4, row.size(), f) != row.size()) throw std::runtime_error("ply: truncated body");
        for (int g = 0; g < 6; g++) {
            const size_t dim = src[g].size();
            for (size_t k = 0; k < dim; k++) c.g[g][static_cast<size_t>(i) * dim + k] = row[src[g][k]];
        }
    }
    return c;
}

}  // namespace

struct sxh_render_session {
    sxh_backend* b = nullptr;
    sxh_executor* e = nullptr;
    int64_t count = 0;
    int sh_degree = 0;
    DevBuf<uint32_t> rgba;
};

extern "C" {

int32_t sxh_exec_export_ply(sxh_executor* e, int64_t count, float min_opacity, uint8_t pad_sh_full, const char* path,
                            sxh_export_stats* stats) {
    return guarded([&] {
        const char* what = "export_ply";
        if (!e || !path) invalid(what, "null executor/path");
        if (count < 0 || count > e->rows) invalid(what, "count out of [0, arena_rows]");
        SXH_HIP(hipSetDevice(e->b->device));
        sxh_detail::canonicalize(e);
        hipStream_t s = e->b->stream;
        const int N = static_cast<int>(count);
        const int K = e->n_coeffs - 1;
        const int Kw = (pad_sh_full && K > 0 && K < 15) ? 15 : K;
        DevBuf<unsigned long long> removed(2);
        DevBuf<int32_t> list(std::max<size_t>(1, static_cast<size_t>(N)));
        int64_t kept = 0;
        unsigned long long rm[2] = {0, 0};
        SXH_HIP(hipMemsetAsync(removed.p, 0, 16, s));
        if (N > 0) {
            const sxk::Arena A = e->arena();
            sxk::export_flags(A, dims_of(e), N, min_opacity, e->tiles.p, removed.p, s);
            sxk::scan_i32_i64(e->tiles.p, e->cum.p, N, e->scan_scratch.p, s);
            sxk::export_list(e->tiles.p, e->cum.p, N, list.p, s);
            SXH_HIP(hipMemcpyAsync(&kept, e->cum.p + (N - 1), 8, hipMemcpyDeviceToHost, s));
        }
        SXH_HIP(hipMemcpyAsync(rm, removed.p, 16, hipMemcpyDeviceToHost, s));
        SXH_HIP(hipStreamSynchronize(s));
        // header (PlyIO.cpp:25-34 text)
        std::string h = "ply\nformat binary_little_endian 1.0\n";
        h += "element vertex " + std::to_string(kept) + "\n";
        const auto prop = [&](const std::string& n) { h += "property float " + n + "\n"; };
        for (const char* n : {"x", "y", "z", "nx", "ny", "nz"}) prop(n);
        for (int i = 0; i < 3; i++) prop("f_dc_" + std::to_string(i));
        for (int i = 0; i < 3 * Kw; i++) prop("f_rest_" + std::to_string(i));
        prop("opacity");
        for (int i = 0; i < 3; i++) prop("scale_" + std::to_string(i));
        for (int i = 0; i < 4; i++) prop("rot_" + std::to_string(i));
        h += "end_header\n";
        HostFile file(path, "wb", "ply");
        put_bytes(file.f, h.data(), h.size(), "ply");
        const int row_floats = sxk::export_row_floats(Kw);
        const int64_t rows_per = std::min<int64_t>(static_cast<int64_t>(kChunkBytes / (4 * row_floats)),
                                                   static_cast<int64_t>(e->staging.n / row_floats));
        Bounce bb;
        const sxk::Arena A = e->arena();
        for (int64_t r0 = 0; r0 < kept; r0 += rows_per) {
            const int64_t rows = std::min(rows_per, kept - r0);
            sxk::export_pack(A, K, Kw, list.p, r0, rows, e->staging.p, s);
            SXH_HIP(hipMemcpyAsync(bb.p(), e->staging.p, rows * row_floats * 4, hipMemcpyDeviceToHost, s));
            SXH_HIP(hipStreamSynchronize(s));
            put_bytes(file.f, bb.p(), rows * row_floats * 4, "ply");
        }
        file.close_checked(path, "ply");
        if (stats) {
            stats->input = count;
            stats->removed_nonfinite = static_cast<int64_t>(rm[0]);
            stats->removed_low_opacity = static_cast<int64_t>(rm[1]);
            stats->kept = kept;
        }
    });
}

int32_t sxh_ply_read(const char* path, int64_t* count, int32_t* sh_degree, float* const* params) {
    return guarded([&] {
        if (!path || !count || !sh_degree) invalid("ply_read", "null path/count/sh_degree");
        PlyCloud c = read_ply(path, params != nullptr);
        *count = c.count;
        *sh_degree = c.sh_degree;
        if (!params) return;
        for (int g = 0; g < 6; g++) {
            if (c.g[g].empty()) continue;
            if (!params[g]) invalid("ply_read", "null output array for group " + std::to_string(g));
            std::memcpy(params[g], c.g[g].data(), c.g[g].size() * 4);
        }
    });
}

int32_t sxh_checkpoint_verify_config(const sxh_checkpoint_config* saved, const sxh_checkpoint_config* current) {
    return guarded([&] {
        if (!saved || !current) invalid("verify_checkpoint_config", "null argument");
        verify_config(*saved, *current);
    });
}

int32_t sxh_checkpoint_read_header(const char* path, sxh_checkpoint_header* out) {
    return guarded([&] {
        if (!path || !out) invalid("load_checkpoint_header", "null argument");
        HostFile file(path, "rb", "checkpoint");
        *out = read_header(file.f, path);
    });
}

int32_t sxh_exec_save_checkpoint(sxh_executor* e, const sxh_checkpoint_config* cfg, int32_t iter, int64_t count,
                                 const char* rng_state, uint8_t fp16, const char* path) {
    return guarded([&] {
        const char* what = "save_checkpoint_file";
        if (!e || !cfg || !path) invalid(what, "null argument");
        if (count < 1) invalid(what, "empty cloud");
        if (count > e->rows) invalid(what, "count exceeds arena rows");
        if (cfg->sh_degree != e->d.sh_degree) invalid(what, "cloud/config sh_degree mismatch");
        if (iter < 0) invalid("Trainer::make_checkpoint", "iter must be >= 0");
        SXH_HIP(hipSetDevice(e->b->device));
        sxh_detail::canonicalize(e);
        const std::string rng = rng_state ? rng_state : "";
        const std::string tmp = std::string(path) + ".tmp";
        try {
            HostFile file(tmp, "wb", "checkpoint");
            std::FILE* f = file.f;
            put_bytes(f, kMagic, 4, "checkpoint");
            put_pod<uint32_t>(f, kVersion, "checkpoint");
            put_pod<uint32_t>(f, fp16 ? kFlagFp16 : 0u, "checkpoint");
            put_pod<int32_t>(f, cfg->sh_degree, "checkpoint");
            put_pod<int32_t>(f, cfg->factor, "checkpoint");
            put_pod<int32_t>(f, cfg->test_split, "checkpoint");
            put_pod<int32_t>(f, cfg->total_iters, "checkpoint");
            put_pod<uint8_t>(f, cfg->mcmc_enabled, "checkpoint");
            put_pod<uint8_t>(f, cfg->antialiased, "checkpoint");
            put_pod<uint8_t>(f, 0, "checkpoint");
            put_pod<uint8_t>(f, 0, "checkpoint");
            put_pod<int64_t>(f, cfg->cap_max, "checkpoint");
            put_pod<uint64_t>(f, cfg->mcmc_seed, "checkpoint");
            put_pod<float>(f, cfg->scene_scale, "checkpoint");
            put_pod<float>(f, cfg->ssim_weight, "checkpoint");
            put_pod<int32_t>(f, iter, "checkpoint");
            put_pod<int64_t>(f, count, "checkpoint");
            put_pod<uint64_t>(f, static_cast<uint64_t>(rng.size()), "checkpoint");
            put_bytes(f, rng.data(), rng.size(), "checkpoint");
            Bounce bb;
            const int mode = fp16 ? sxk::kCkptF16 : sxk::kCkptF32;
            for (int g = 0; g < 6; g++) save_group(e, bb, f, e->p[g].p, e->dims[g], count, mode);
            for (int g = 0; g < 6; g++) {
                save_group(e, bb, f, e->m[g].p, e->dims[g], count, mode);
                save_group(e, bb, f, e->v[g].p, e->dims[g], count, fp16 ? sxk::kCkptF16Sqrt : sxk::kCkptF32);
            }
            if (std::fflush(f) != 0) throw std::runtime_error("checkpoint: fflush failed for " + tmp);
            if (::fsync(::fileno(f)) != 0) throw std::runtime_error("checkpoint: fsync failed for " + tmp);
            file.close_checked(tmp, "checkpoint");
        } catch (...) {
            std::remove(tmp.c_str());
            throw;
        }
        if (std::rename(tmp.c_str(), path) != 0) {
            std::remove(tmp.c_str());
            throw std::runtime_error("checkpoint: rename failed: " + tmp + " -> " + path);
        }
        fsync_dir_of(path);
    });
}

int32_t sxh_exec_load_checkpoint(sxh_executor* e, const char* path, const sxh_checkpoint_config* current,
                                 sxh_checkpoint_header* out, char* rng_state, int64_t rng_capacity) {
    return guarded([&] {
        const char* what = "Trainer::restore_checkpoint";
        if (!e || !path) invalid(what, "null executor/path");
        HostFile file(path, "rb", "checkpoint");
        std::FILE* f = file.f;
        const sxh_checkpoint_header h = read_header(f, path);
        const uint64_t rng_len = get_pod<uint64_t>(f);
        if (rng_len > (1u << 20)) throw std::runtime_error("checkpoint: rng state too large");
        std::string rng(static_cast<size_t>(rng_len), '\0');
        get_bytes(f, rng.data(), rng.size());
        // the payload's size is derived from the header: check the file holds exactly that
        const long body_at = std::ftell(f);
        int64_t payload = 0;
        const int64_t esz = h.fp16 ? 2 : 4;
        for (int g = 0; g < 6; g++) payload += 3 * h.alive_count * group_dim(g, h.config.sh_degree) * esz;
        if (std::fseek(f, 0, SEEK_END) != 0) throw std::runtime_error("checkpoint: seek failed");
        const int64_t size = std::ftell(f);
        if (size < body_at + payload) throw std::runtime_error("checkpoint: truncated file (short read)");
        if (size > body_at + payload) throw std::runtime_error("checkpoint: trailing bytes (corrupt or size mismatch)");
        std::fseek(f, body_at, SEEK_SET);
        if (current) verify_config(h.config, *current);
        if (h.config.sh_degree != e->d.sh_degree) invalid(what, "checkpoint sh_degree differs from the arena's");
        if (h.alive_count > e->rows) invalid(what, "checkpoint count exceeds arena rows (cap_max)");
        if (h.config.mcmc_enabled && rng.empty()) invalid(what, "missing mcmc rng state");
        if (rng_state) {
            if (rng_capacity < static_cast<int64_t>(rng.size()) + 1)
                throw CapacityError(std::string(what) + ": rng_state needs " + std::to_string(rng.size() + 1) + " bytes");
            std::memcpy(rng_state, rng.c_str(), rng.size() + 1);
        }
        SXH_HIP(hipSetDevice(e->b->device));
        sxh_detail::canonicalize(e);  // (the loaded rows then replace the updated ones)
        hipStream_t s = e->b->stream;
        const int n = static_cast<int>(h.alive_count);
        const int mode = h.fp16 ? sxk::kCkptF16 : sxk::kCkptF32;
        Bounce bb;
        for (int g = 0; g < 6; g++) load_group(e, bb, f, e->p[g].p, e->dims[g], n, mode);
        for (int g = 0; g < 6; g++) {
            load_group(e, bb, f, e->m[g].p, e->dims[g], n, mode);
            load_group(e, bb, f, e->v[g].p, e->dims[g], n, h.fp16 ? sxk::kCkptF16Sqrt : sxk::kCkptF32);
            if (h.fp16) sxk::ckpt_pair_zero(e->m[g].p, e->v[g].p, e->rows, e->dims[g], n, s);
        }
        for (int g = 0; g < 6; g++) {  // the arena tail is zero (the untouched-tail contract)
            if (e->dims[g] == 0) continue;
            sxk::zero_tail(e->p[g].p, e->rows, e->dims[g], n, s);
            sxk::zero_tail(e->m[g].p, e->rows, e->dims[g], n, s);
            sxk::zero_tail(e->v[g].p, e->rows, e->dims[g], n, s);
        }
        SXH_HIP(hipGetLastError());
        SXH_HIP(hipStreamSynchronize(s));
        if (out) *out = h;
    });
}

int32_t sxh_render_session_open(sxh_backend* b, const sxh_render_session_args* a, sxh_render_session** out) {
    return guarded([&] {
        if (!b || !a || !out) invalid("render_session_open", "null argument");
        if (!a->ply_path) invalid("render_session_open", "ply_path must be given");
        if (a->sh_degree < 0 || a->sh_degree > 3)
            invalid("render_session_open", "sh_degree must be 0..3 (0 = derived from the PLY)");
        PlyCloud c = read_ply(a->ply_path, true);
        if (c.sh_degree > 3) invalid("render_session_open", "PLY sh_degree 4 is beyond the executor's 0..3");
        if (a->sh_degree > 0 && a->sh_degree > c.sh_degree)
            invalid("render_session_open", "sh_degree " + std::to_string(a->sh_degree) + " exceeds PLY sh_degree " +
                                               std::to_string(c.sh_degree) + " (higher-band coefficients absent)");
        if (a->sh_degree > 0 && a->sh_degree < c.sh_degree) {  // keep the lower bands only
            const int Kn = (a->sh_degree + 1) * (a->sh_degree + 1) - 1, Ko = (c.sh_degree + 1) * (c.sh_degree + 1) - 1;
            std::vector<float> shN(static_cast<size_t>(c.count) * Kn * 3);
            for (int64_t i = 0; i < c.count; i++)
                std::memcpy(&shN[static_cast<size_t>(i) * Kn * 3], &c.g[5][static_cast<size_t>(i) * Ko * 3],
                            static_cast<size_t>(Kn) * 3 * 4);
            c.g[5] = std::move(shN);
            c.sh_degree = a->sh_degree;
        }
        if (c.count < 1) invalid("Trainer", "empty cloud");
        sxh_exec_desc d{};
        d.arena_rows = c.count;
        d.sh_degree = c.sh_degree;
        d.eps2d = 0.3f;  // TrainConfig defaults (Trainer.h:219)
        d.near_plane = 0.01f;
        d.far_plane = 1e10f;
        d.radius_clip = 0.0f;
        d.b1 = 0.9f;
        d.b2 = 0.999f;
        d.eps = 1e-15f;
        d.ssim_weight = 0.2f;
        d.antialiased = a->antialiased ? 1 : 0;
        d.isect_mode = SXH_ISECT_ACCUTILE;
        auto* sess = new sxh_render_session();
        try {
            sess->b = b;
            sess->count = c.count;
            sess->sh_degree = c.sh_degree;
            if (sxh_exec_create(b, &d, &sess->e) != SXH_OK) throw std::runtime_error(sxh_last_error());
            sxh_executor* e = sess->e;
            hipStream_t s = b->stream;
            for (int g = 0; g < 6; g++) {  // parameters only; the moments stay zero
                if (e->dims[g] == 0) continue;
                SXH_HIP(hipMemcpyAsync(e->staging.p, c.g[g].data(), c.g[g].size() * 4, hipMemcpyHostToDevice, s));
                sxk::aos_to_soa(e->staging.p, e->p[g].p, static_cast<int>(c.count), e->dims[g], e->rows, s);
                SXH_HIP(hipStreamSynchronize(s));
            }
        } catch (...) {
            if (sess->e) sxh_exec_destroy(sess->e);
            delete sess;
            throw;
        }
        *out = sess;
    });
}

int32_t sxh_render_session_frame(sxh_render_session* sess, const float* viewmat, float fx, float fy, float cx, float cy,
                                 int32_t width, int32_t height, uint8_t* out_rgba) {
    return guarded([&] {
        const char* what = "render_session_frame";
        if (!sess || !viewmat || !out_rgba) invalid(what, "session/viewmat/out_rgba must be given");
        if (width < 1 || height < 1) invalid(what, "width/height must be positive");
        if (!(fx > 0.0f) || !(fy > 0.0f) || !std::isfinite(cx) || !std::isfinite(cy))
            invalid(what, "fx/fy must be positive and cx/cy finite");
        sxh_executor* e = sess->e;
        SXH_HIP(hipSetDevice(e->b->device));
        const float K[9] = {fx, 0.0f, cx, 0.0f, fy, cy, 0.0f, 0.0f, 1.0f};
        sxh_step_inputs in{};
        in.viewmat = viewmat;
        in.K = K;
        in.width = width;
        in.height = height;
        in.gt_rgb = nullptr;
        in.gt_index = -1;
        in.count = sess->count;
        in.degrees_to_use = static_cast<uint32_t>(sess->sh_degree);
        in.forward_only = 1;
        sxh_step_outputs o{};
        sxh_detail::run_step(e, &in, &o, nullptr);
        const size_t n_px = static_cast<size_t>(width) * height;
        sess->rgba.ensure(n_px);
        sxk::rgba8(e->render.p, static_cast<int64_t>(n_px), sess->rgba.p, e->b->stream);
        SXH_HIP(hipGetLastError());
        SXH_HIP(hipMemcpyAsync(out_rgba, sess->rgba.p, n_px * 4, hipMemcpyDeviceToHost, e->b->stream));
        SXH_HIP(hipStreamSynchronize(e->b->stream));
    });
}

void sxh_render_session_close(sxh_render_session* sess) {
    if (!sess) return;
    sxh_exec_destroy(sess->e);
    delete sess;
}

}  // extern "C"
