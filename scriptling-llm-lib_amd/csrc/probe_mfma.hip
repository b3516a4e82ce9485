// Peak-rate probes (measurement only; bench.py loads libsllm_probe.so, the
// library never does): the int8 matrix cores, and the VALU issue rate of the
// instruction kinds the GEMV kernels use. Every wave of the MFMA probe runs chains of
// independent int8 MFMAs on register operands - no memory traffic inside the
// loop - and writes its accumulators once, so the launch time is the matrix
// cores' issue rate:
//   form 0: v_mfma_i32_16x16x32_i8, the instruction the prefill GEMM issues
//           (K = 32 is one Q8_0 block, so each result is one block's exact
//           int32 dot);
//   form 1: v_mfma_i32_16x16x64_i8 (gfx950), the form the published
//           5.0 POPS dense int8 figure is quoted for;
//   form 2: v_mfma_i32_32x32x32_i8 (gfx950), the instruction the prefill GEMM
//           issues (K = 32 is one Q8_0 block, and the form runs at the full
//           int8 rate).
#include <hip/hip_runtime.h>

#include <cstdint>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

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
    } else if (FORM == 1) {
        const v4i a = {s, s + 1, s + 2, s + 3}, b = {s * 3, s * 5, s * 7, s * 9};
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int c = 0; c < kChains; c++) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
        }
    } else {
        // 32 x 32 results: 4 independent chains of 16 registers each
        const v4i a = {s, s + 1, s + 2, s + 3}, b = {s * 3, s * 5, s * 7, s * 9};
        v16i big[4];
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) big[c][r] = 0;
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int c = 0; c < 4; c++) big[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, big[c], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[c][r] = big[c][r] ^ big[c][r + 4] ^ big[c][r + 8] ^ big[c][r + 12];
    }
    v4i t = acc[0];
#pragma unroll
    for (int c = 1; c < kChains; c++) t += acc[c];
    out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}

// VALU issue rate of one instruction kind: eight independent chains per lane
// (each result feeds the next instruction of its chain only), register
// operands, no memory traffic inside the loop.
#define SLLM_PROBE_CHAINS(ASM)                                          \
    _Pragma("unroll") for (int i = 0; i < 8; i++) asm volatile(ASM : "+v"(r[i]) : "v"(c1), "v"(c2));

template <int OP>
__global__ void __launch_bounds__(256) valu_loop(unsigned *out, int iters, unsigned seed) {
    unsigned r[8];
    const unsigned c1 = seed * 3u + threadIdx.x, c2 = seed ^ 0x0c0c0400u;
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = threadIdx.x * 77u + i;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int u = 0; u < 16; u++) {
            if (OP == 0) { SLLM_PROBE_CHAINS("v_fma_f32 %0, %0, %1, %2") }
            else if (OP == 1) { SLLM_PROBE_CHAINS("v_mul_f32 %0, %0, %1") }
            else if (OP == 2) { SLLM_PROBE_CHAINS("v_add_u32 %0, %0, %1") }
            else if (OP == 3) { SLLM_PROBE_CHAINS("v_lshrrev_b32 %0, %1, %0") }
            else if (OP == 4) { SLLM_PROBE_CHAINS("v_cvt_f32_ubyte1 %0, %0") }
            else if (OP == 5) { SLLM_PROBE_CHAINS("v_cvt_i32_f32 %0, %0") }
            else if (OP == 6) { SLLM_PROBE_CHAINS("v_perm_b32 %0, %0, %1, %2") }
            else if (OP == 7) { SLLM_PROBE_CHAINS("v_dot4_i32_i8 %0, %1, %2, %0") }
            else if (OP == 8) { SLLM_PROBE_CHAINS("v_bfe_u32 %0, %0, %1, %2") }
            else if (OP == 9) { SLLM_PROBE_CHAINS("v_and_or_b32 %0, %0, %1, %2") }
            else { SLLM_PROBE_CHAINS("v_mad_i32_i24 %0, %0, %1, %2") }
        }
    }
    unsigned t = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) t ^= r[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}
#undef SLLM_PROBE_CHAINS

}  // namespace

extern "C" {

// Issue rate of VALU instruction kind `op` (0 v_fma_f32, 1 v_mul_f32,
// 2 v_add_u32, 3 v_lshrrev_b32, 4 v_cvt_f32_ubyte1, 5 v_cvt_i32_f32,
// 6 v_perm_b32, 7 v_dot4_i32_i8, 8 v_bfe_u32, 9 v_and_or_b32,
// 10 v_mad_i32_i24) in T lane-instructions per second, the fastest of `reps`
// launches of `blocks` workgroups of 4 waves. Returns 0 or a hipError_t.
int sllm_probe_valu_rate(int op, int blocks, int iters, int reps, double *rate) {
    if (!rate || blocks <= 0 || iters <= 0 || reps <= 0 || op < 0 || op > 10) return (int)hipErrorInvalidValue;
    unsigned *out = nullptr;
    hipError_t e = hipMalloc(&out, (size_t)blocks * 256 * sizeof(unsigned));
    if (e != hipSuccess) return (int)e;
    hipEvent_t a, b;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    float best = 0.0f;
    for (int r = 0; r <= reps && e == hipSuccess; r++) {  // launch 0 warms up
        (void)hipEventRecord(a, nullptr);
        switch (op) {
        case 0: hipLaunchKernelGGL(valu_loop<0>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 1: hipLaunchKernelGGL(valu_loop<1>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 2: hipLaunchKernelGGL(valu_loop<2>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 3: hipLaunchKernelGGL(valu_loop<3>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 4: hipLaunchKernelGGL(valu_loop<4>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 5: hipLaunchKernelGGL(valu_loop<5>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 6: hipLaunchKernelGGL(valu_loop<6>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 7: hipLaunchKernelGGL(valu_loop<7>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 8: hipLaunchKernelGGL(valu_loop<8>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        case 9: hipLaunchKernelGGL(valu_loop<9>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        default: hipLaunchKernelGGL(valu_loop<10>, dim3(blocks), dim3(256), 0, nullptr, out, iters, (unsigned)r); break;
        }
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
    *rate = (double)blocks * 256 * iters * 16 * 8 / (best * 1e-3) / 1e12;
    return 0;
}

// Runs `reps` launches of form `form` (0, 1 or 2) over `blocks` workgroups of 4
// waves, `iters` loop trips each, on the current device's null stream, and
// returns the sustained rate in TOPS (2 x M x N x K per MFMA) of the fastest
// launch in *tops. Returns 0 on success, else a hipError_t.
int sllm_probe_mfma_tops(int form, int blocks, int iters, int reps, double *tops) {
    if (!tops || blocks <= 0 || iters <= 0 || reps <= 0 || form < 0 || form > 2) return (int)hipErrorInvalidValue;
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
        else if (form == 1) hipLaunchKernelGGL(mfma_loop<1>, dim3(blocks), dim3(256), 0, nullptr, out, iters, r);
        else hipLaunchKernelGGL(mfma_loop<2>, dim3(blocks), dim3(256), 0, nullptr, out, iters, r);
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
    // MACs per wave per loop trip: kChains 16 x 16 x K MFMAs (forms 0, 1) or
    // four 32 x 32 x 32 ones (form 2)
    const double macs = form == 0 ? 16.0 * 16 * 32 * kChains : form == 1 ? 16.0 * 16 * 64 * kChains : 32.0 * 32 * 32 * 4;
    const double ops = 2.0 * macs * iters * blocks * 4;  // 4 waves per workgroup
    *tops = ops / (best * 1e-3) / 1e12;
    return 0;
}

}  // extern "C"
