// Prefill GEMM (xRows >= 64) on the int8 matrix cores.
//
// 1. The activation rows are quantized once into a workspace (xq int8 [M][K],
//    xs fp32 [M][G], Σxq int32 [M][G]) by the same routine as the GEMV prologue.
// 2. Each workgroup computes a 64 (activation rows) x 64 (weight rows) tile of
//    dst. For every 32-element block g, wave w runs v_mfma_i32_16x16x32_i8 on
//    its 16 activation rows against four 16-row slices of the weight tile:
//    K = 32 is exactly one block, so each MFMA returns the exact int32 block
//    dots (the reference's isum / qsum) for a 16 x 16 sub-tile. The epilogue
//    then forms the reference's per-block fp32 term from them, as the GEMV does,
//    and accumulates it.
//
// MFMA operand layout (16x16x32 i8): A[i][k] sits in lane i + 16 (k / 8), byte
// k % 8; B[k][j] in lane j + 16 (k / 8); D[i][j] in lane j + 16 (i / 4),
// element i % 4.
//
// Roofline: the per-block fp32 epilogue (3-6 VALU ops per output per 32 MACs)
// bounds this kernel, not the matrix cores or HBM.
#include <hip/hip_runtime.h>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

namespace sllm {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kBM = 64;  // activation rows per workgroup (4 waves x 16)
constexpr int kBN = 64;  // weight rows per workgroup (4 MFMA column tiles)

// B operand: 8 consecutive elements (chunk c = 0..3 of the block) of weight
// row `row`, block g, as 8 int8 codes (Q4: unsigned nibbles; Q5K1 high: 0/1).
template <int FMT>
__device__ __forceinline__ long b_frag(const Planes &P, size_t idx, int c) {
    if (FMT == SLLM_Q8_0) {
        const int4 *plane = (c < 2) ? P.qs : P.qs2;
        const long *p = (const long *)(plane + idx);
        return p[c & 1];
    }
    // 4-bit formats: byte i = element i (low nibble) | element i+16 (high)
    const long v = ((const long *)(P.qs + idx))[c & 1];
    const long lo = 0x0f0f0f0f0f0f0f0fL;
    return (c < 2) ? (v & lo) : ((v >> 4) & lo);
}

// High-bit operand of Q5K1: elements 8c..8c+7 of the 32-bit mask as 0/1 bytes.
__device__ __forceinline__ long bits_frag(uint32_t hb, int c) {
    const uint32_t t = hb >> (8 * c);
    const uint32_t lo = (uint32_t)spread4(t);
    const uint32_t hi = (uint32_t)spread4(t >> 4);
    return (long)((uint64_t)lo | ((uint64_t)hi << 32));
}

template <int FMT>
__global__ void __launch_bounds__(256) gemm_kernel(Planes P, const int8_t *__restrict__ xq,
                                                   const float *__restrict__ xs, const int *__restrict__ sx,
                                                   float *__restrict__ dst, int M, int N, int G, int mtiles,
                                                   int ntiles) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int K = G * 32;
    // XCD-aware tile order: workgroups are dealt round-robin to the 8 XCDs;
    // tile t = (id / 8) + (id % 8) * per_xcd keeps the M-tiles of one weight
    // tile on one XCD, so its weight rows come from HBM once into that L2.
    const int total = mtiles * ntiles;
    const int per_xcd = (total + 7) / 8;
    const int id = blockIdx.x;
    const int t = (id % 8) * per_xcd + id / 8;
    if (t >= total) return;
    const int mt = t % mtiles, nt = t / mtiles;
    const int r16 = lane & 15, c4 = lane >> 4;
    const int m_a = min(mt * kBM + wave * 16 + r16, M - 1);  // A-operand row (clamped; discarded if >= M)
    const int m_o = mt * kBM + wave * 16 + 4 * c4;           // first of this lane's 4 output rows
    size_t nidx[4];
#pragma unroll
    for (int j = 0; j < 4; j++) nidx[j] = (size_t)min(nt * kBN + 16 * j + r16, N - 1) * G;

    float acc[4][4], acc2[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[j][r] = acc2[j][r] = 0.0f;

    const int8_t *arow = xq + (size_t)m_a * K + c4 * 8;
    for (int g = 0; g < G; g++) {
        const long a = *(const long *)(arow + (size_t)g * 32);
        float xsr[4], fsx[4];
        int sxr[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = min(m_o + r, M - 1);
            xsr[r] = xs[(size_t)m * G + g];
            sxr[r] = sx[(size_t)m * G + g];
            fsx[r] = (float)sxr[r];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const size_t idx = nidx[j] + g;
            const v4i z = {0, 0, 0, 0};
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b_frag<FMT>(P, idx, c4), z, 0, 0, 0);
            if (FMT == SLLM_Q8_0) {
                const float ws = f16_lut(P.d[idx]);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float cmb = ws * xsr[r];
                    const float term = cmb * (float)d[r];
                    acc[j][r] = acc[j][r] + term;
                }
            } else if (FMT == SLLM_Q4_0) {
                const float ws = f16_exact(P.d[idx]);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float cmb = ws * xsr[r];
                    const float term = cmb * (float)(d[r] - 8 * sxr[r]);
                    acc[j][r] = acc[j][r] + term;
                }
            } else {
                const float wd = f16_exact(P.d[idx]), wm = f16_exact(P.m[idx]);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float t1 = (float)d[r] * wd;
                    const float t2 = fsx[r] * wm;
                    float tt = t1 + t2;
                    tt = tt * xsr[r];
                    acc[j][r] = acc[j][r] + tt;
                }
                if (FMT == SLLM_Q5K1) {
                    const v4i h = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bits_frag(P.qh[idx], c4), z, 0, 0, 0);
                    const float wdh = f16_exact(P.dh[idx]);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float h1 = (float)h[r] * wdh;
                        const float h2 = fsx[r] * 0.0f;
                        float hh = h1 + h2;
                        hh = hh * xsr[r];
                        acc2[j][r] = acc2[j][r] + hh;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = nt * kBN + 16 * j + r16;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = m_o + r;
            if (m < M && n < N) dst[(size_t)m * N + n] = (FMT == SLLM_Q5K1) ? acc[j][r] + acc2[j][r] : acc[j][r];
        }
    }
}

}  // namespace

size_t gemm_workspace_bytes(int fmt, int N, int G, int M) {
    (void)fmt;
    (void)N;
    const size_t q = ((size_t)M * G * 32 + 255) & ~(size_t)255;
    const size_t s = ((size_t)M * G * 4 + 255) & ~(size_t)255;
    return q + 2 * s;
}

sllm_status launch_gemm(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M, void *ws,
                        size_t ws_bytes, hipStream_t s) {
    if (ws_bytes < gemm_workspace_bytes(fmt, N, G, M)) return set_error(SLLM_ERR_ARG, "gemm: workspace too small");
    int8_t *xq = (int8_t *)ws;
    const size_t q = ((size_t)M * G * 32 + 255) & ~(size_t)255;
    const size_t sb = ((size_t)M * G * 4 + 255) & ~(size_t)255;
    float *xsp = (float *)((char *)ws + q);
    int *sxp = (int *)((char *)ws + q + sb);
    sllm_status st = launch_quantize_act(x, M, G, xq, xsp, sxp, s);
    if (st != SLLM_OK) return st;
    const int mtiles = (M + kBM - 1) / kBM, ntiles = (N + kBN - 1) / kBN;
    const int total = mtiles * ntiles;
    const int grid = ((total + 7) / 8) * 8;
    switch (fmt) {
    case SLLM_Q8_0: hipLaunchKernelGGL(gemm_kernel<SLLM_Q8_0>, dim3(grid), dim3(256), 0, s, P, xq, xsp, sxp, dst, M, N, G, mtiles, ntiles); break;
    case SLLM_Q4_0: hipLaunchKernelGGL(gemm_kernel<SLLM_Q4_0>, dim3(grid), dim3(256), 0, s, P, xq, xsp, sxp, dst, M, N, G, mtiles, ntiles); break;
    case SLLM_Q4_1: hipLaunchKernelGGL(gemm_kernel<SLLM_Q4_1>, dim3(grid), dim3(256), 0, s, P, xq, xsp, sxp, dst, M, N, G, mtiles, ntiles); break;
    case SLLM_Q5K1: hipLaunchKernelGGL(gemm_kernel<SLLM_Q5K1>, dim3(grid), dim3(256), 0, s, P, xq, xsp, sxp, dst, M, N, G, mtiles, ntiles); break;
    default: return set_error(SLLM_ERR_QTYPE, "gemm: format has no int8 MFMA path");
    }
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

}  // namespace sllm
