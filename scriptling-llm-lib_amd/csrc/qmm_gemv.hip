// Decode GEMV (xRows < 64) for every weight format.
//
// One launch computes dst[m][n] = Σ_g term(m, n, g) for up to MT activation rows:
//   prologue  every workgroup quantizes the activation rows into LDS with the
//             bit-exact Q8_0 quantizer (or, for Q5_0, stages the fp32 rows);
//   main      rows are taken in batches of R = waves / S rows per workgroup; the
//             S waves of a row each own a contiguous slice of its blocks, and
//             lane l of a wave owns blocks slice_start + l + 64 i. A lane loads
//             its blocks' planes with 16-byte loads (consecutive lanes read
//             consecutive 16 B), forms the reference's per-block term exactly,
//             and accumulates; the wave then reduces across lanes and the S
//             slice partials are added in slice order (fixed order, so results
//             are bit-reproducible run to run).
// The per-block term equals the reference's bit for bit; only the order in
// which the terms of a row are added differs from the reference's sequential
// loop (reassociation).
#include <hip/hip_runtime.h>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

namespace sllm {

namespace {

constexpr int kMaxWaves = 16;

// LDS image of the prologue for MT activation rows of G blocks.
struct ActView {
    int4 *xl;    // [MT][G] elements 0..15 of each block (int8)
    int4 *xh;    // [MT][G] elements 16..31
    float *xs;   // [MT][G] activation scale
    int *sx;     // [MT][G] Σxq
    float *xf;   // Q5_0: [MT][G][kXfStride] fp32 activations
    float *red;  // [kMaxWaves][2*MT] slice partials
};

__host__ __device__ inline size_t act_lds_bytes(int fmt, int MT, int G) {
    size_t red = (size_t)kMaxWaves * 2 * MT * sizeof(float);
    if (fmt == SLLM_Q5_0) return (size_t)MT * G * kXfStride * sizeof(float) + red;
    return (size_t)MT * G * (2 * sizeof(int4) + sizeof(float) + sizeof(int)) + red;
}

__device__ inline ActView carve_act(unsigned char *lds, int fmt, int MT, int G) {
    ActView v{};
    if (fmt == SLLM_Q5_0) {
        v.xf = (float *)lds;
        v.red = v.xf + (size_t)MT * G * kXfStride;
    } else {
        v.xl = (int4 *)lds;
        v.xh = v.xl + (size_t)MT * G;
        v.xs = (float *)(v.xh + (size_t)MT * G);
        v.sx = (int *)(v.xs + (size_t)MT * G);
        v.red = (float *)(v.sx + (size_t)MT * G);
    }
    return v;
}

// Prologue: quantize (or stage) M activation rows of K = 32 G fp32 into LDS.
template <int FMT>
__device__ inline void stage_activations(const float *__restrict__ x, int M, int G, const ActView &A) {
    const int T = blockDim.x;
    const int total = M * G * 8;  // 8 lanes per block, 4 elements each
    for (int i = threadIdx.x; i < total; i += T) {
        const int blk = i >> 3, sub = i & 7;
        const float4 v = *(const float4 *)(x + (size_t)blk * 32 + sub * 4);
        if (FMT == SLLM_Q5_0) {
            *(float4 *)(A.xf + (size_t)blk * kXfStride + sub * 4) = v;
        } else {
            float s;
            int sm;
            uint32_t packed = quantize_quarter(v, &s, &sm);
            int *dstw = (int *)((sub < 4) ? (A.xl + blk) : (A.xh + blk));
            dstw[sub & 3] = (int)packed;
            if (sub == 0) {
                A.xs[blk] = s;
                A.sx[blk] = sm;
            }
        }
    }
}

// Per-lane register image of one weight block.
struct BlockRegs {
    int4 q, q2;
    uint16_t d, m, dh;
    uint32_t qh;
};

template <int FMT>
__device__ __forceinline__ void load_block(const Planes &P, size_t idx, BlockRegs &b) {
    b.q = P.qs[idx];
    b.d = P.d[idx];
    if (FMT == SLLM_Q8_0) b.q2 = P.qs2[idx];
    if (FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) b.m = P.m[idx];
    if (FMT == SLLM_Q5K1) b.dh = P.dh[idx];
    if (FMT == SLLM_Q5_0 || FMT == SLLM_Q5K1) b.qh = P.qh[idx];
}

// Adds block g's term for activation row m to acc (acc2: the Q5K1 high half).
template <int FMT>
__device__ __forceinline__ void block_term(const BlockRegs &b, const ActView &A, int G, int m, int g,
                                           float &acc, float &acc2) {
    const size_t a = (size_t)m * G + g;
    if (FMT == SLLM_Q5_0) {
        const float4 *xb = (const float4 *)(A.xf + a * kXfStride);
        float sum = q5_block_sum(b.q, b.qh, xb);
        float s = f16_lut(b.d);
        float grp = s * sum;  // float32_ops.go:366 `s * sum`
        acc = acc + grp;
        return;
    }
    const int4 xl = A.xl[a], xh = A.xh[a];
    const float xs = A.xs[a];
    if (FMT == SLLM_Q8_0) {
        // q8q8.go:187-195 + vnni_amd64.s:70-73: cmb = ws*xs, term = float(isum)*cmb
        int isum = q8_isum(b.q, b.q2, xl, xh);
        float ws = f16_lut(b.d);
        float cmb = ws * xs;
        float term = cmb * (float)isum;
        acc = acc + term;
    } else if (FMT == SLLM_Q4_0) {
        // q4q8.go:37-43: ws*xs*float(Σ(nib-8)·xq); Σ(nib-8)xq = Σnib·xq - 8Σxq exactly
        int isum = nib_isum(b.q, xl, xh) - 8 * A.sx[a];
        float ws = f16_exact(b.d);
        float cmb = ws * xs;
        float term = cmb * (float)isum;
        acc = acc + term;
    } else {
        // q41q8_row_amd64.s:65-71: ((float(qsum)*d) + (float(Σxq)*m)) * xs
        const float fsx = (float)A.sx[a];
        int qsum = nib_isum(b.q, xl, xh);
        float t1 = (float)qsum * f16_exact(b.d);
        float t2 = fsx * f16_exact(b.m);
        float t = t1 + t2;
        t = t * xs;
        acc = acc + t;
        if (FMT == SLLM_Q5K1) {
            // high Q4_1 block of convertQ5KToTwoQ41: scale dh, min +0, 0/1 nibbles
            int hsum = bits_isum(b.qh, xl, xh);
            float h1 = (float)hsum * f16_exact(b.dh);
            float h2 = fsx * 0.0f;
            float h = h1 + h2;
            h = h * xs;
            acc2 = acc2 + h;
        }
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <int FMT, int NB, int MT>
__global__ void __launch_bounds__(1024) gemv_kernel(Planes P, const float *__restrict__ x,
                                                    float *__restrict__ dst, int N, int G, int M, int S,
                                                    int nbatch) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const ActView A = carve_act(lds, FMT, MT, G);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int W = blockDim.x >> 6;
    const int R = W / S;
    const int row_in_batch = wave / S;
    const int slice = wave - row_in_batch * S;
    const int gps = (G + S - 1) / S;
    const int g0 = slice * gps;
    const int g1 = min(G, g0 + gps);

    stage_activations<FMT>(x, M, G, A);
    __syncthreads();

    for (int bt = blockIdx.x; bt < nbatch; bt += gridDim.x) {
        const int n = bt * R + row_in_batch;
        float acc[MT], acc2[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) acc[m] = acc2[m] = 0.0f;
        if (n < N) {
            BlockRegs regs[NB];
            const size_t rowbase = (size_t)n * G;
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const int g = g0 + lane + 64 * i;
                if (g < g1) load_block<FMT>(P, rowbase + g, regs[i]);
            }
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const int g = g0 + lane + 64 * i;
                if (g < g1) {
#pragma unroll
                    for (int m = 0; m < MT; m++)
                        if (m < M) block_term<FMT>(regs[i], A, G, m, g, acc[m], acc2[m]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
            acc[m] = wave_sum(acc[m]);
            if (FMT == SLLM_Q5K1) acc2[m] = wave_sum(acc2[m]);
        }
        if (S == 1) {
            if (lane == 0 && n < N) {
#pragma unroll
                for (int m = 0; m < MT; m++)
                    if (m < M) dst[(size_t)m * N + n] = (FMT == SLLM_Q5K1) ? acc[m] + acc2[m] : acc[m];
            }
        } else {
            if (lane == 0) {
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    A.red[wave * 2 * MT + m] = acc[m];
                    A.red[wave * 2 * MT + MT + m] = acc2[m];
                }
            }
            __syncthreads();
            if (slice == 0 && lane == 0 && n < N) {
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    if (m >= M) continue;
                    float lo = A.red[wave * 2 * MT + m], hi = A.red[wave * 2 * MT + MT + m];
                    for (int s = 1; s < S; s++) {
                        lo = lo + A.red[(wave + s) * 2 * MT + m];
                        hi = hi + A.red[(wave + s) * 2 * MT + MT + m];
                    }
                    dst[(size_t)m * N + n] = (FMT == SLLM_Q5K1) ? lo + hi : lo;
                }
            }
            __syncthreads();
        }
    }
}

template <int FMT, int NB, int MT>
sllm_status launch_t(const Planes &P, const float *x, float *dst, int N, int G, int M, int S, int W,
                     int grid, int nbatch, size_t lds, hipStream_t s) {
    hipLaunchKernelGGL((gemv_kernel<FMT, NB, MT>), dim3(grid), dim3(W * 64), lds, s, P, x, dst, N, G, M, S,
                       nbatch);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

template <int FMT, int MT>
sllm_status launch_nb(int NB, const Planes &P, const float *x, float *dst, int N, int G, int M, int S, int W,
                      int grid, int nbatch, size_t lds, hipStream_t s) {
    switch (NB) {
    case 1: return launch_t<FMT, 1, MT>(P, x, dst, N, G, M, S, W, grid, nbatch, lds, s);
    case 2: return launch_t<FMT, 2, MT>(P, x, dst, N, G, M, S, W, grid, nbatch, lds, s);
    case 3: return launch_t<FMT, 3, MT>(P, x, dst, N, G, M, S, W, grid, nbatch, lds, s);
    case 4: return launch_t<FMT, 4, MT>(P, x, dst, N, G, M, S, W, grid, nbatch, lds, s);
    }
    return set_error(SLLM_ERR_SHAPE, "gemv: unsupported blocks-per-lane");
}

template <int FMT>
sllm_status launch_mt(int MT, int NB, const Planes &P, const float *x, float *dst, int N, int G, int M, int S,
                      int W, int grid, int nbatch, size_t lds, hipStream_t s) {
    switch (MT) {
    case 1: return launch_nb<FMT, 1>(NB, P, x, dst, N, G, M, S, W, grid, nbatch, lds, s);
    case 2: return launch_nb<FMT, 2>(NB, P, x, dst, N, G, M, S, W, grid, nbatch, lds, s);
    case 4: return launch_nb<FMT, 4>(NB, P, x, dst, N, G, M, S, W, grid, nbatch, lds, s);
    }
    return set_error(SLLM_ERR_SHAPE, "gemv: unsupported row tile");
}

constexpr size_t kMaxLds = 64 * 1024;

}  // namespace

// Launch shape: W waves per workgroup; S waves per weight row (K split), so a
// workgroup covers R = W/S rows per batch; NB blocks per lane (<= 4).
sllm_status launch_gemv(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M,
                        hipStream_t s) {
    if (N <= 0 || G <= 0 || M <= 0) return set_error(SLLM_ERR_ARG, "gemv: empty shape");
    const Tuning &T = tuning();
    const int W = T.gemv_waves;
    // K split: enough row batches to fill the device, but never below 64 blocks
    // per wave, and at most 4 blocks per lane.
    int S = 1;
    const int s_cap = G >= 64 ? (G / 64 < W ? G / 64 : W) : 1;
    while (S * 2 <= s_cap && ((int64_t)N * S + W - 1) / W < T.gemv_min_batches) S *= 2;
    while ((G + 64 * S - 1) / (64 * S) > 4 && S * 2 <= W) S *= 2;
    const int NB = (G + 64 * S - 1) / (64 * S);
    if (NB > 4) return set_error(SLLM_ERR_SHAPE, "gemv: cols too large for the decode kernel");
    const int R = W / S;
    const int nbatch = (N + R - 1) / R;
    const int grid = nbatch < T.gemv_grid_cap ? nbatch : T.gemv_grid_cap;
    // Activation rows per launch, limited by LDS.
    int done = 0;
    while (done < M) {
        int left = M - done;
        int MT = left >= 4 ? 4 : (left >= 2 ? 2 : 1);
        while (MT > 1 && act_lds_bytes(fmt, MT, G) > kMaxLds) MT >>= 1;
        if (act_lds_bytes(fmt, MT, G) > kMaxLds)
            return set_error(SLLM_ERR_SHAPE, "gemv: activation row does not fit in LDS");
        const int mrows = left < MT ? left : MT;
        const size_t lds = act_lds_bytes(fmt, MT, G);
        const float *xp = x + (size_t)done * G * 32;
        float *dp = dst + (size_t)done * N;
        sllm_status st;
        switch (fmt) {
        case SLLM_Q8_0: st = launch_mt<SLLM_Q8_0>(MT, NB, P, xp, dp, N, G, mrows, S, W, grid, nbatch, lds, s); break;
        case SLLM_Q4_0: st = launch_mt<SLLM_Q4_0>(MT, NB, P, xp, dp, N, G, mrows, S, W, grid, nbatch, lds, s); break;
        case SLLM_Q4_1: st = launch_mt<SLLM_Q4_1>(MT, NB, P, xp, dp, N, G, mrows, S, W, grid, nbatch, lds, s); break;
        case SLLM_Q5_0: st = launch_mt<SLLM_Q5_0>(MT, NB, P, xp, dp, N, G, mrows, S, W, grid, nbatch, lds, s); break;
        case SLLM_Q5K1: st = launch_mt<SLLM_Q5K1>(MT, NB, P, xp, dp, N, G, mrows, S, W, grid, nbatch, lds, s); break;
        default: return set_error(SLLM_ERR_QTYPE, "gemv: unknown format");
        }
        if (st != SLLM_OK) return st;
        done += mrows;
    }
    return SLLM_OK;
}

// ------------------------------------------------------ verification ----

namespace {

__global__ void quantize_act_kernel(const float *__restrict__ x, int nblocks, int8_t *__restrict__ xq,
                                    float *__restrict__ xs, int32_t *__restrict__ sx) {
    // Same device routine as the GEMV/GEMM prologue; 8 lanes per block.
    const int total = nblocks * 8;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int blk = i >> 3, sub = i & 7;
        const float4 v = *(const float4 *)(x + (size_t)blk * 32 + sub * 4);
        float s;
        int sm;
        uint32_t packed = quantize_quarter(v, &s, &sm);
        *(uint32_t *)(xq + (size_t)blk * 32 + sub * 4) = packed;
        if (sub == 0) {
            xs[blk] = s;
            if (sx) sx[blk] = sm;
        }
    }
}

template <int FMT>
__global__ void block_dots_kernel(Planes P, const float *__restrict__ x, int N, int G, int M,
                                  int32_t *__restrict__ out) {
    // One thread per (m, n, g); activations quantized on the fly by the 8-lane
    // routine (each thread of an 8-group handles one quarter of block g).
    const int64_t total = (int64_t)M * N * G;
    for (int64_t t = (int64_t)blockIdx.x * (blockDim.x / 8) + (threadIdx.x >> 3); t < total;
         t += (int64_t)gridDim.x * (blockDim.x / 8)) {
        const int sub = threadIdx.x & 7;
        const int g = (int)(t % G);
        const int n = (int)((t / G) % N);
        const int m = (int)(t / ((int64_t)G * N));
        const float *xb = x + ((size_t)m * G + g) * 32;
        const float4 v = *(const float4 *)(xb + sub * 4);
        float s;
        int sm;
        uint32_t packed = quantize_quarter(v, &s, &sm);
        // gather the 8 packed quarters of the block into every lane
        int w[8];
#pragma unroll
        for (int k = 0; k < 8; k++) w[k] = __shfl((int)packed, (threadIdx.x & ~7) + k);
        if (sub != 0) continue;
        const int4 xl = make_int4(w[0], w[1], w[2], w[3]);
        const int4 xh = make_int4(w[4], w[5], w[6], w[7]);
        const size_t idx = (size_t)n * G + g;
        if (FMT == SLLM_Q8_0) {
            out[t] = q8_isum(P.qs[idx], P.qs2[idx], xl, xh);
        } else if (FMT == SLLM_Q4_0) {
            out[t] = nib_isum(P.qs[idx], xl, xh) - 8 * sm;
        } else if (FMT == SLLM_Q4_1) {
            out[t] = nib_isum(P.qs[idx], xl, xh);
        } else if (FMT == SLLM_Q5K1) {
            out[2 * t] = nib_isum(P.qs[idx], xl, xh);
            out[2 * t + 1] = bits_isum(P.qh[idx], xl, xh);
        } else {
            float4 xv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) xv[k] = ((const float4 *)xb)[k];
            float sum = q5_block_sum(P.qs[idx], P.qh[idx], xv);
            out[t] = __builtin_bit_cast(int32_t, sum);
        }
    }
}

__global__ void argmax_kernel(const float *__restrict__ v, int n, int *__restrict__ out) {
    // float32_ops.go:812-822: bv starts at v[0] and v[i] replaces it only if
    // v[i] > bv. So the result is 0 when v[0] is NaN, and otherwise the first
    // index of the largest non-NaN value. Single workgroup: each thread scans a
    // contiguous chunk in index order, then chunks merge in index order.
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    const int T = blockDim.x;
    const int chunk = (n + T - 1) / T;
    const int lo = threadIdx.x * chunk;
    const int hi = min(n, lo + chunk);
    float best = 0.0f;
    int besti = -1;
    for (int i = lo; i < hi; i++) {
        const float f = v[i];
        if (f != f) continue;
        if (besti < 0 || f > best) {
            best = f;
            besti = i;
        }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = besti;
    __syncthreads();
    if (threadIdx.x == 0) {
        // merge chunks in index order with the same rule as the serial loop
        float b = 0.0f;
        int idx = -1;
        for (int t = 0; t < T; t++) {
            if (bi[t] < 0) continue;
            if (idx < 0 || bv[t] > b) {
                b = bv[t];
                idx = bi[t];
            }
        }
        const float v0 = v[0];
        *out = (idx < 0 || v0 != v0) ? 0 : idx;
    }
}

}  // namespace

sllm_status launch_quantize_act(const float *x, int rows, int G, int8_t *xq, float *xs, int32_t *sx,
                                hipStream_t s) {
    const int nblocks = rows * G;
    int grid = (nblocks * 8 + 255) / 256;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(quantize_act_kernel, dim3(grid), dim3(256), 0, s, x, nblocks, xq, xs, sx);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

sllm_status launch_block_dots(int fmt, const Planes &P, const float *x, int N, int G, int M, int32_t *out,
                              hipStream_t s) {
    int64_t total = (int64_t)M * N * G;
    int64_t grid64 = (total + 31) / 32;
    int grid = grid64 > 8192 ? 8192 : (int)grid64;
    switch (fmt) {
    case SLLM_Q8_0: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q8_0>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q4_0: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q4_0>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q4_1: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q4_1>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q5_0: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q5_0>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q5K1: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q5K1>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    default: return set_error(SLLM_ERR_QTYPE, "block_dots: unknown format");
    }
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

sllm_status launch_argmax(const float *v, int n, int *out_dev, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, v, n, out_dev);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

}  // namespace sllm
