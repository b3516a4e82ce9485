// Peak-rate probe of the int8 matrix cores (measurement only; bench.py loads
// libsllm_probe.so, the library never does). Every wave runs chains of
// independent int8 MFMAs on register operands - no memory traffic inside the
// loop - and writes its accumulators once, so the launch time is the matrix
// cores' issue rate:
//   form 0: v_mfma_i32_16x16x32_i8, the instruction the prefill GEMM issues
//           (K = 32 is one Q8_0 block, so each result is one block's exact
//           int32 dot);
//   form 1: v_mfma_i32_16x16x64_i8 (gfx950), the form the published
//           5.0 POPS dense int8 figure is quoted for.
#include <hip/hip_runtime.h>

#include <cstdint>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef long v1l __attribute__((ext_vector_type(1)));

namespace {

constexpr int kChains = 8;  // independent accumulators per wave (cover the MFMA latency)

template <int FORM>
__global__ void __launch_bounds__(256) mfma_loop(v4i *out, int iters, int seed) {
    const int lane = threadIdx.x & 63;
    v4i acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; c++) acc[c] = v4i{0, 0, 0, 0};
    const int s = seed + lane;
    if (FORM == 0) {
        const long a = (long)s * 0x0101010101010101L, b = (long)(s + 3) * 0x0102030405060708L;
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int c = 0; c < kChains; c++) acc[c] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, acc[c], 0, 0, 0);
        }
    } else {
        const v4i a = {s, s + 1, s + 2, s + 3}, b = {s * 3, s * 5, s * 7, s * 9};
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int c = 0; c < kChains; c++) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
        }
    }
    v4i t = acc[0];
#pragma unroll
    for (int c = 1; c < kChains; c++) t += acc[c];
    out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}

}  // namespace

extern "C" {

// Runs `reps` launches of form `form` (0 or 1) over `blocks` workgroups of 4
// waves, `iters` loop trips each, on the current device's null stream, and
// returns the sustained rate in TOPS (2 x M x N x K per MFMA) of the fastest
// launch in *tops. Returns 0 on success, else a hipError_t.
int sllm_probe_mfma_tops(int form, int blocks, int iters, int reps, double *tops) {
    if (!tops || blocks <= 0 || iters <= 0 || reps <= 0 || (form != 0 && form != 1)) return (int)hipErrorInvalidValue;
    v4i *out = nullptr;
    hipError_t e = hipMalloc(&out, (size_t)blocks * 256 * sizeof(v4i));
    if (e != hipSuccess) return (int)e;
    hipEvent_t a, b;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    float best = 0.0f;
    for (int r = 0; r <= reps && e == hipSuccess; r++) {  // launch 0 warms up
        (void)hipEventRecord(a, nullptr);
        if (form == 0) hipLaunchKernelGGL(mfma_loop<0>, dim3(blocks), dim3(256), 0, nullptr, out, iters, r);
        else hipLaunchKernelGGL(mfma_loop<1>, dim3(blocks), dim3(256), 0, nullptr, out, iters, r);
        e = hipGetLastError();
        (void)hipEventRecord(b, nullptr);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        if (e == hipSuccess && r > 0 && (best == 0.0f || ms < best)) best = ms;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipFree(out);
    if (e != hipSuccess) return (int)e;
    const double k = form == 0 ? 32.0 : 64.0;
    const double ops = 2.0 * 16 * 16 * k * (double)kChains * iters * blocks * 4;  // 4 waves per workgroup
    *tops = ops / (best * 1e-3) / 1e12;
    return 0;
}

}  // extern "C"
