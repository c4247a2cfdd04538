// k_yardstick.hip — VALU issue-rate yardstick: kernels of one instruction class each, with a known
// number of wave-level instructions, timed with HIP events. It calibrates the cycles-per-instruction
// model that turns the SQ_INSTS_VALU counters of the step's kernels into a VALU issue bound (how
// long the SIMDs need for a kernel's instructions when they issue nothing else). Built into its own
// library (build/libsplatx_yardstick.so), not into the product library: only bench.py's
// --calibrate-valu mode loads it.
#include <hip/hip_runtime.h>

#include <cstdio>

namespace {

constexpr int kAcc = 8;  // independent chains per lane: enough to hide the VALU dependency latency

enum YardOp {
    kFma = 0, kMul, kAddF32, kExp, kRcp, kAndB32, kBfeU32, kAddU32, kMovB32, kMovDpp,
    kFmaLanes32, kFmaLanes16, kFmaExpMix, kYardOps
};

template <int OP>
__global__ void __launch_bounds__(256) k_yard(float* __restrict__ out, int iters, float b, float c) {
    float a[kAcc];
#pragma unroll
    for (int i = 0; i < kAcc; i++) a[i] = static_cast<float>(threadIdx.x) * 0.001f + static_cast<float>(i);
    const int lane = threadIdx.x & 63;
    // a branch around the whole loop: the loop runs with only these lanes in EXEC
    const bool active = OP == kFmaLanes32 ? lane < 32 : OP == kFmaLanes16 ? lane < 16 : true;
    if (active) {
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int i = 0; i < kAcc; i++) {
                if constexpr (OP == kFma || OP == kFmaLanes32 || OP == kFmaLanes16) a[i] = __builtin_fmaf(a[i], b, c);
                else if constexpr (OP == kMul) a[i] = a[i] * b;
                else if constexpr (OP == kAddF32) a[i] = a[i] + b;
                else if constexpr (OP == kExp) a[i] = __builtin_amdgcn_exp2f(a[i]);
                else if constexpr (OP == kRcp) a[i] = __builtin_amdgcn_rcpf(a[i]);
                else if constexpr (OP == kAndB32) a[i] = __int_as_float(__float_as_int(a[i]) & (0x7fffff7f - it));
                else if constexpr (OP == kBfeU32) a[i] = __int_as_float(static_cast<int>(__builtin_amdgcn_ubfe(__float_as_uint(a[i]), 3, 20)));
                else if constexpr (OP == kAddU32) a[i] = __int_as_float(__float_as_int(a[i]) + 3);
                else if constexpr (OP == kMovB32) {
                    float t;
                    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"(a[i]));
                    a[i] = t;
                } else if constexpr (OP == kMovDpp)
                    a[i] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a[i]), 0xB1, 0xF, 0xF, false));
                else if constexpr (OP == kFmaExpMix)
                    a[i] = (i & 1) ? __builtin_amdgcn_exp2f(a[i]) : __builtin_fmaf(a[i], b, c);
            }
        }
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kAcc; i++) s += a[i];
    out[static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x] = s;
}

using YardFn = void (*)(float*, int, float, float);
const YardFn kYard[kYardOps] = {k_yard<0>, k_yard<1>, k_yard<2>, k_yard<3>, k_yard<4>, k_yard<5>, k_yard<6>,
                                k_yard<7>, k_yard<8>, k_yard<9>, k_yard<10>, k_yard<11>, k_yard<12>};
const char* const kYardName[kYardOps] = {"v_fma_f32", "v_mul_f32", "v_add_f32", "v_exp_f32", "v_rcp_f32",
                                         "v_and_b32", "v_bfe_u32", "v_add_u32", "v_mov_b32", "v_mov_b32_dpp",
                                         "v_fma_f32 (32 lanes in EXEC)", "v_fma_f32 (16 lanes in EXEC)",
                                         "v_fma_f32 + v_exp_f32 (alternating)"};

}  // namespace

extern "C" {

// Number of yardstick kernels and the name of kernel `op` (null when out of range).
int sxy_valu_count(void) { return kYardOps; }
const char* sxy_valu_name(int op) { return op >= 0 && op < kYardOps ? kYardName[op] : nullptr; }

// Runs yardstick kernel `op` on device `device` over `blocks` workgroups of 4 waves, `iters` loop trips
// of 8 instructions of the class per wave (the loop adds 3 scalar instructions per trip): one
// untimed launch, then `reps` timed ones; *best_ms receives the fastest. Returns 0, or -1 on a bad
// argument or HIP error (message on stderr).
int sxy_valu(int device, int op, int blocks, int iters, int reps, double* best_ms) {
    if (op < 0 || op >= kYardOps || blocks <= 0 || iters <= 0 || reps <= 0 || !best_ms) return -1;
    float* out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = -1;
    float best = 1e30f;
    auto ok = [](hipError_t e) {
        if (e != hipSuccess) std::fprintf(stderr, "sxy_valu: %s\n", hipGetErrorString(e));
        return e == hipSuccess;
    };
    if (!ok(hipSetDevice(device)) || !ok(hipMalloc(&out, sizeof(float) * 256 * static_cast<size_t>(blocks))))
        return -1;
    if (ok(hipEventCreate(&e0)) && ok(hipEventCreate(&e1))) {
        hipLaunchKernelGGL(kYard[op], dim3(blocks), dim3(256), 0, nullptr, out, iters, 0.999f, 0.001f);
        bool good = ok(hipGetLastError()) && ok(hipDeviceSynchronize());
        for (int r = 0; good && r < reps; r++) {
            good = ok(hipEventRecord(e0, nullptr));
            hipLaunchKernelGGL(kYard[op], dim3(blocks), dim3(256), 0, nullptr, out, iters, 0.999f, 0.001f);
            float ms = 0.f;
            good = good && ok(hipGetLastError()) && ok(hipEventRecord(e1, nullptr)) && ok(hipEventSynchronize(e1)) &&
                   ok(hipEventElapsedTime(&ms, e0, e1));
            if (good && ms < best) best = ms;
        }
        if (good) {
            *best_ms = best;
            rc = 0;
        }
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(out);
    return rc;
}

}  // extern "C"
