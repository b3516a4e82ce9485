// Decode GEMV (xRows < 64) planner: launch shapes for one or several weights
// sharing their activation rows, and the verification kernels. The kernel
// templates are in qmm_gemv_kernel.hpp; each weight format's launch chain is
// instantiated in its own translation unit (qmm_gemv_<fmt>.hip).
#include <hip/hip_runtime.h>

#include "qmm_gemv_kernel.hpp"

namespace sllm {

namespace gemv {
extern template sllm_status launch_mt<SLLM_Q8_0, false>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q8_0, true>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q4_0, false>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q4_0, true>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q4_1, false>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q4_1, true>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q5_0, false>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q5_0, true>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q5K1, false>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q5K1, true>(int, int, int, const SegTable &, const float *, int, int, int,
                                                          int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q4K_STREAM, false>(int, int, int, const SegTable &, const float *, int, int,
                                                                int, int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q4K_STREAM, true>(int, int, int, const SegTable &, const float *, int, int,
                                                               int, int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q6K_STREAM, false>(int, int, int, const SegTable &, const float *, int, int,
                                                                int, int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q6K_STREAM, true>(int, int, int, const SegTable &, const float *, int, int,
                                                               int, int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q2K, false>(int, int, int, const SegTable &, const float *, int, int, int,
                                                         int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q2K, true>(int, int, int, const SegTable &, const float *, int, int, int,
                                                        int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q3K, false>(int, int, int, const SegTable &, const float *, int, int, int,
                                                         int, int, int, size_t, hipStream_t);
extern template sllm_status launch_mt<SLLM_Q3K, true>(int, int, int, const SegTable &, const float *, int, int, int,
                                                        int, int, int, size_t, hipStream_t);
}  // namespace gemv

using namespace gemv;

namespace {

constexpr size_t kMaxLds = 64 * 1024;

int device_cus() {
    static thread_local int dev = -1, cus = 0;
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess) return 256;
    if (d != dev) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || v <= 0) v = 256;
        dev = d;
        cus = v;
    }
    return cus;
}

}  // namespace

namespace {

// pair: P[0] / P[1] are the gate / up weights of one FFN (N[0] == N[1]) and
// dst[0..2] receive SwiGLU(gate, up), gate (may be null), up (may be null).
sllm_status plan_and_launch(int fmt, const Planes *P, float *const *dst, const int *N, int nseg, bool pair,
                            const float *x, int G, int M, hipStream_t s, const float *norm_w, float eps,
                            unsigned long long *amax_key = nullptr, unsigned int *amax_cnt = nullptr,
                            int *amax_out = nullptr, bool accum = false) {
    if (nseg < 1 || nseg > kMaxSegs) return set_error(SLLM_ERR_ARG, "gemv: 1 to 4 weights per launch");
    if (G <= 0 || M <= 0) return set_error(SLLM_ERR_ARG, "gemv: empty shape");
    if (pair && (nseg != 2 || N[0] != N[1])) return set_error(SLLM_ERR_ARG, "gemv: gate / up shapes differ");
    int64_t Ntot = 0;
    for (int i = 0; i < (pair ? 1 : nseg); i++) {
        if (N[i] <= 0) return set_error(SLLM_ERR_ARG, "gemv: empty shape");
        Ntot += N[i];
    }
    const int nrow_segs = pair ? 1 : nseg;  // segments of row waves
    const Tuning &T = tuning();
    const int64_t wgs = (int64_t)device_cus() * T.gemv_wg_per_cu;
    // Rows per wave: the fewest that fit every segment's rows into
    // gemv_waves waves per workgroup slot. Each segment gets just enough waves
    // for that many rows each; the waves per workgroup are then the fewest
    // (>= 4, for the prologue) that spread them over every workgroup slot.
    const int64_t slots = wgs * T.gemv_waves;
    int RPW = (int)((Ntot + slots - 1) / slots);
    auto count_waves = [&](int rpw) {
        int64_t w = 0;
        for (int i = 0; i < nrow_segs; i++) w += ((int64_t)N[i] + rpw - 1) / rpw;
        return w;
    };
    while (count_waves(RPW) > slots) RPW++;
    // Paired gate / up: half of a workgroup's waves stream gate rows, the other
    // half the same rows of up, RPW consecutive rows per wave, so both weights
    // stream as one unpaired launch over the 2N rows would; the workgroup's
    // gate and up waves then meet in LDS.
    if (pair) {
        RPW = (int)((2 * (int64_t)N[0] + slots - 1) / slots);
        while (2 * (((int64_t)N[0] + RPW - 1) / RPW) > slots) RPW++;
    }
    if (RPW > 64) return set_error(SLLM_ERR_SHAPE, "gemv: more than 64 rows per wave (rows too many)");
    const int64_t waves = pair ? 2 * (((int64_t)N[0] + RPW - 1) / RPW) : count_waves(RPW);
    // Blocks per lane per unit (NB) and K-chunks per row (KCH). Rows of up to
    // gemv_max_nb x 64 blocks are one chunk; longer rows are split into chunks
    // of the largest lane-group count that divides them (no partial chunks).
    // While a wave would stream fewer than 4 units, its rows are split further,
    // so that it overlaps its loads with its compute instead of issuing
    // everything at once and doing all its compute after the last byte lands.
    const int lg = (G + 63) / 64;
    // Q5_0 reads 32 fp32 activations per block from LDS: more than two blocks
    // per lane per unit only adds registers (measured: 3 % slower at NB 7)
    // Q6_K streamed: one block per lane per unit - its requantization holds
    // about 40 registers per block, and with several blocks of one unit
    // interleaved the GEMV spills (the ring's depth D still covers the latency)
    int nb_cap = fmt == SLLM_Q5_0 && T.gemv_max_nb > 2 ? 2 : T.gemv_max_nb;
    if (fmt == SLLM_Q6K_STREAM) nb_cap = 1;
    int NB = lg;
    if (lg > nb_cap) {
        NB = nb_cap;
        while (NB > 1 && lg % NB) NB--;
        if (NB * 2 < nb_cap) NB = nb_cap;  // no good divisor: accept one partial chunk
    }
    while (NB > 1 && RPW * ((lg + NB - 1) / NB) < 4) {
        int nb = NB - 1;
        while (nb > 1 && lg % nb) nb--;
        NB = nb;
    }
    const int KCH = (G + 64 * NB - 1) / (64 * NB);
    int W = (int)((waves + wgs - 1) / wgs);
    W = W < 4 ? 4 : (W > T.gemv_waves ? T.gemv_waves : W);
    if (pair) W = (W + 1) & ~1;  // as many gate waves as up waves (gemv_waves is even)
    const int grid = pair ? (int)(((int64_t)N[0] + (int64_t)(W / 2) * RPW - 1) / ((int64_t)(W / 2) * RPW))
                          : (int)((waves + W - 1) / W);
    if (amax_key && (M != 1 || nseg != 1 || pair)) return set_error(SLLM_ERR_ARG, "gemv: argmax needs one row");
    if (norm_w && M != 1) return set_error(SLLM_ERR_ARG, "gemv: the fused RMSNorm takes one activation row");
    SegTable S{};
    S.n = nrow_segs;
    S.amax_key = amax_key;
    S.amax_cnt = amax_cnt;
    S.amax_out = amax_out;
    S.accum = accum ? 1 : 0;
    S.norm_w = norm_w;
    S.norm_eps = eps;
    S.wave0[0] = 0;
    for (int i = 0; i < nseg; i++) {
        S.P[i] = P[i];
        S.N[i] = N[i];
    }
    for (int i = 0; i < nrow_segs; i++) S.wave0[i + 1] = S.wave0[i] + (N[i] + RPW - 1) / RPW;
    S.wave0[nrow_segs] = grid * W;  // the last segment also takes the spare waves
    const int U = RPW * KCH;
    int done = 0;
    while (done < M) {
        const int left = M - done;
        int MT = left >= 4 ? 4 : (left >= 2 ? 2 : 1);
        while (MT > 1 && act_lds_bytes(fmt, MT, G) > kMaxLds) MT >>= 1;
        if (act_lds_bytes(fmt, MT, G) > kMaxLds)
            return set_error(SLLM_ERR_SHAPE, "gemv: activation row does not fit in LDS");
        // ring depth: units in flight per wave, bounded by registers (NB*D*MT
        // <= 8 blocks per lane), by the wave's unit count (D <= U), and by the bytes in
        // flight over the whole device (enough to cover HBM latency; more only
        // piles compute into the tail)
        const int64_t unit_bytes = (int64_t)64 * NB * plane_block_bytes(fmt);
        const int64_t inflight = (int64_t)T.gemv_inflight_kb * 1024;
        int D = 1;
        while (D * 2 * NB * MT <= 8 && D * 2 <= U && waves * unit_bytes * D * 2 <= inflight) D *= 2;
        // the RMSNorm prologue is longer than the plain one: a launch whose
        // waves stream many units keeps two in flight, so that more weight
        // bytes arrive while the row statistics are formed. Measured (rotating
        // copies, two boxes): RMSNorm + head + argmax (Q8_0 128256x4096, 32
        // rows per wave) 85.4-86.4 µs against 86.3-87.2 with one unit; the
        // plain head is faster with one (84.0 against 86.9), and RMSNorm +
        // gate/up + SwiGLU slower with four (16.0 against 15.1 with two)
        if (norm_w && D == 1 && U >= 16 && 2 * NB * MT <= 8) D = 2;
        const int mrows = left < MT ? left : MT;
        const size_t lds = act_lds_bytes(fmt, MT, G);
        const float *xp = x + (size_t)done * G * 32;
        const int ndst = pair ? 3 : nseg;
        for (int i = 0; i < ndst; i++) {
            const int rows_i = pair ? N[0] : N[i];  // output i: M x rows_i, rows contiguous per activation row
            S.dst[i] = dst[i] ? dst[i] + (size_t)done * rows_i : nullptr;
        }
        sllm_status st;
#define SLLM_GEMV_FMT(F)                                                                                  \
    (pair ? launch_mt<F, true>(MT, NB, D, S, xp, G, mrows, KCH, RPW, W, grid, lds, s)                 \
          : launch_mt<F, false>(MT, NB, D, S, xp, G, mrows, KCH, RPW, W, grid, lds, s))
        switch (fmt) {
        case SLLM_Q8_0: st = SLLM_GEMV_FMT(SLLM_Q8_0); break;
        case SLLM_Q4_0: st = SLLM_GEMV_FMT(SLLM_Q4_0); break;
        case SLLM_Q4_1: st = SLLM_GEMV_FMT(SLLM_Q4_1); break;
        case SLLM_Q5_0: st = SLLM_GEMV_FMT(SLLM_Q5_0); break;
        case SLLM_Q5K1: st = SLLM_GEMV_FMT(SLLM_Q5K1); break;
        case SLLM_Q4K_STREAM: st = SLLM_GEMV_FMT(SLLM_Q4K_STREAM); break;
        case SLLM_Q6K_STREAM: st = SLLM_GEMV_FMT(SLLM_Q6K_STREAM); break;
        case SLLM_Q2K: st = SLLM_GEMV_FMT(SLLM_Q2K); break;
        case SLLM_Q3K: st = SLLM_GEMV_FMT(SLLM_Q3K); break;
        default: return set_error(SLLM_ERR_QTYPE, "gemv: unknown format");
        }
#undef SLLM_GEMV_FMT
        if (st != SLLM_OK) return st;
        done += mrows;
    }
    return SLLM_OK;
}

}  // namespace

sllm_status launch_gemv_multi(int fmt, const Planes *P, float *const *dst, const int *N, int nseg,
                              const float *x, int G, int M, hipStream_t s, const float *norm_w, float eps) {
    return plan_and_launch(fmt, P, dst, N, nseg, false, x, G, M, s, norm_w, eps);
}

sllm_status launch_gemv_swiglu(int fmt, const Planes &Pg, const Planes &Pu, const float *x, float *h,
                               float *gate, float *up, int N, int G, int M, hipStream_t s, const float *norm_w,
                               float eps) {
    const Planes P[2] = {Pg, Pu};
    float *const dst[3] = {h, gate, up};
    const int Ns[2] = {N, N};
    return plan_and_launch(fmt, P, dst, Ns, 2, true, x, G, M, s, norm_w, eps);
}

sllm_status launch_gemv(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M,
                        hipStream_t s) {
    return launch_gemv_multi(fmt, &P, &dst, &N, 1, x, G, M, s);
}

sllm_status launch_gemv_add(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M,
                            hipStream_t s) {
    return plan_and_launch(fmt, &P, &dst, &N, 1, false, x, G, M, s, nullptr, 0.0f, nullptr, nullptr, nullptr,
                           true);
}

sllm_status launch_gemv_argmax(int fmt, const Planes &P, const float *x, float *logits, int N, int G,
                               unsigned long long *key, unsigned int *cnt, int *out, hipStream_t s,
                               const float *norm_w, float eps) {
    return plan_and_launch(fmt, &P, &logits, &N, 1, false, x, G, 1, s, norm_w, eps, key, cnt, out);
}

namespace {
// One workgroup of 256 threads per row: the same statistics as the GEMV
// prologue (rms_inv), then normed = (x * inv) * w.
__global__ void __launch_bounds__(256) rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ nw,
                                                      float eps, int K, float *__restrict__ out) {
    __shared__ float red[4];
    const size_t off = (size_t)blockIdx.x * K;
    const float inv = rms_inv<16>(x + off, K, eps, red);
    for (int i = threadIdx.x; i < K; i += 256) out[off + i] = (x[off + i] * inv) * nw[i];
}
}  // namespace

sllm_status launch_rmsnorm(const float *x, const float *norm_w, float eps, int rows, int K, float *out,
                           hipStream_t s) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, norm_w, eps, K, out);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

// ------------------------------------------------------ verification ----

namespace {

__global__ void quantize_act_kernel(const float *__restrict__ x, int nblocks, int8_t *__restrict__ xq,
                                    float *__restrict__ xs, int32_t *__restrict__ sx) {
    // The GEMV prologue routine with 8 lanes per 32-element block (one float4 each).
    const int total = nblocks * 8;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int blk = i >> 3, sub = i & 7;
        const float4 v[1] = {*((const float4 *)(x + (size_t)blk * 32) + sub)};
        int w[1];
        float s;
        int sm;
        quantize_part<8>(v, w, s, sm);
        ((int *)(xq + (size_t)blk * 32))[sub] = w[0];
        if (sub == 0) {
            xs[blk] = s;
            if (sx) sx[blk] = sm;
        }
    }
}

template <int FMT>
__global__ void block_dots_kernel(Planes P, const float *__restrict__ x, int N, int G, int M,
                                  int32_t *__restrict__ out) {
    // One thread per (m, n, g); the activation block is quantized with the
    // prologue routine, the block dot with the GEMV's block routine.
    const int64_t total = (int64_t)M * N * G;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int g = (int)(t % G);
        const int n = (int)((t / G) % N);
        const int m = (int)(t / ((int64_t)G * N));
        const float4 *xb = (const float4 *)(x + ((size_t)m * G + g) * 32);
        float4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = xb[k];
        const size_t idx = (size_t)n * G + g;
        if (FMT == SLLM_Q5_0) {
            const float sum = q5_block_sum(P.qs[idx], P.qh[idx], v);
            out[t] = __builtin_bit_cast(int32_t, sum);
            continue;
        }
        if (kq_native(FMT)) {
            // the GEMV's own block term (elements in order) from a zero start
            BlockRegs b;
            load_block<FMT>(P, (uint32_t)idx, b);
            ActRegs xa;
#pragma unroll
            for (int k = 0; k < 8; k++) xa.xf[k] = v[k];
            float sum = 0.0f, unused = 0.0f;
            block_term<FMT>(b, xa, sum, unused);
            out[t] = __builtin_bit_cast(int32_t, sum);
            continue;
        }
        int w[8];
        float s;
        int sm;
        quantize_part<1>(v, w, s, sm);
        const int4 xl = make_int4(w[0], w[1], w[2], w[3]), xh = make_int4(w[4], w[5], w[6], w[7]);
        if (FMT == SLLM_Q8_0) {
            out[t] = q8_isum(P.qs[idx], P.qs2[idx], xl, xh);
        } else if (FMT == SLLM_Q4_0) {
            out[t] = nib_isum(P.qs[idx], xl, xh) - 8 * sm;
        } else if (FMT == SLLM_Q4_1) {
            out[t] = nib_isum(P.qs[idx], xl, xh);
        } else {
            out[2 * t] = nib_isum(P.qs[idx], xl, xh);
            out[2 * t + 1] = bits_isum(P.qh[idx], xl, xh);
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
    int64_t grid64 = (total + 255) / 256;
    int grid = grid64 > 8192 ? 8192 : (int)grid64;
    switch (fmt) {
    case SLLM_Q8_0: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q8_0>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q4_0: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q4_0>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q4_1: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q4_1>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q5_0: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q5_0>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q5K1: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q5K1>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q2K: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q2K>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
    case SLLM_Q3K: hipLaunchKernelGGL(block_dots_kernel<SLLM_Q3K>, dim3(grid), dim3(256), 0, s, P, x, N, G, M, out); break;
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

namespace {
__global__ void swiglu_kernel(const float *__restrict__ gate, const float *__restrict__ up, float *__restrict__ h,
                              size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        h[i] = swiglu(gate[i], up[i]);
}
__global__ void add_kernel(float *__restrict__ dst, const float *__restrict__ src, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = dst[i] + src[i];
}
}  // namespace

sllm_status launch_swiglu(const float *gate, const float *up, float *h, size_t n, hipStream_t s) {
    if (n == 0) return SLLM_OK;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, gate, up,
                       h, n);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

sllm_status launch_add(float *dst, const float *src, size_t n, hipStream_t s) {
    if (n == 0) return SLLM_OK;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, dst, src, n);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

}  // namespace sllm
