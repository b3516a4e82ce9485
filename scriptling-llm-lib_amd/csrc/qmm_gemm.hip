// Prefill GEMM (xRows >= 64): int8 matrix cores for Q8_0 / Q4_0 / Q4_1 / Q5K1,
// and a VALU GEMM for Q5_0 (fp32 activations; see gemm_q5_kernel below).
//
// 1. The activation rows are quantized once into a workspace (xq int8 [M][K],
//    xs fp32 [M][G], Σxq int32 [M][G]) by the GEMV prologue's routine.
// 2. A workgroup of 2 x WN waves computes a 64 x BN tile of dst (64
//    activation rows x BN = 32 WN weight rows), each wave a 32 x 32 sub-tile.
//    K is staged KB blocks at a time through LDS, double-buffered: the global
//    loads of stage s+1 are in flight while stage s is computed. Per 32-element
//    block each wave runs v_mfma_i32_16x16x32_i8 on its four 16 x 16 pieces:
//    K = 32 is exactly one block, so every MFMA returns exact int32 block dots
//    (the reference's isum / qsum). The epilogue forms the reference's
//    per-block fp32 term from them, exactly as the GEMV does, and accumulates.
// 3. When there are too few tiles to fill the device, K is split over S
//    workgroups; each writes its partial tile and a second kernel adds the S
//    partials in split order (fixed order: results are reproducible).
//
// MFMA operand layout (16x16x32 i8): A[i][k] in lane i + 16 (k / 8), byte
// k % 8; B[k][j] in lane j + 16 (k / 8); D[i][j] in lane j + 16 (i / 4),
// element i % 4.
//
// Roofline: the per-block fp32 epilogue (4-6 VALU ops per output per 32 MACs)
// bounds this kernel, not the matrix cores (which it keeps about 10 % busy) or,
// from M ~ 64 up, HBM.
#include <hip/hip_runtime.h>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

namespace sllm {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kBM = 64;   // activation rows per workgroup
constexpr int kKB = 4;    // blocks (x 32 elements) per K stage
constexpr int kARow = kKB * 32 + 8;  // LDS bytes per activation row (padded: conflict-free b64 reads)

// Bytes of weight codes per block in HBM, per format; in LDS every format
// holds 32 one-byte codes per block (Q4 nibbles are expanded when a stage is
// stored, once per workgroup instead of once per wave that reads them).
template <int FMT>
constexpr int wcode_bytes() {
    return FMT == SLLM_Q8_0 ? 32 : 16;
}
template <int FMT>
constexpr int brow_bytes() {
    return kKB * 32 + 8;  // padded
}

template <int FMT, int BN>
struct alignas(16) Stage {
    // LDS image of one K stage
    int8_t a[kBM * kARow];                       // activation codes
    int8_t b[BN * brow_bytes<FMT>()];            // weight codes
    float xs[kKB][kBM];                          // activation scales
    int sx[kKB][kBM];                            // Σxq (Q4_1 / Q5K1: float(Σxq), exact, as bits)
    // weight scales and mins, decoded to fp32 once per workgroup (Q8_0: the
    // reference's f16 table, the others exact)
    float d[kKB][BN];
    float m[(FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) ? kKB : 1][BN];
    float dh[FMT == SLLM_Q5K1 ? kKB : 1][BN];
    uint32_t hb[FMT == SLLM_Q5K1 ? kKB : 1][BN];
};

// Global -> register staging of one K stage (issued before the compute of the
// previous stage, stored to LDS after it). T threads.
template <int FMT, int BN, int T>
struct Fetch {
    static constexpr int A_N = kBM * kKB * 32 / 16;              // int4 of activation codes
    static constexpr int B_N = BN * kKB * wcode_bytes<FMT>() / 16; // int4 of weight codes
    static constexpr int S_N = kKB * kBM;                         // activation scalars
    static constexpr int W_N = kKB * BN;                          // weight scalars
    static constexpr int A_PER = (A_N + T - 1) / T, B_PER = (B_N + T - 1) / T;
    static constexpr int S_PER = (S_N + T - 1) / T, W_PER = (W_N + T - 1) / T;
    int4 a[A_PER];
    int4 b[B_PER];
    float xs[S_PER];
    int sx[S_PER];
    uint16_t d[W_PER], m[W_PER], dh[W_PER];
    uint32_t hb[W_PER];
};

template <int FMT, int BN, int T>
__device__ __forceinline__ void fetch_stage(Fetch<FMT, BN, T> &f, const Planes &P, const int8_t *__restrict__ xq,
                                            const float *__restrict__ xs, const int *__restrict__ sx, int m0,
                                            int n0, int M, int N, int G, int g0) {
    using F = Fetch<FMT, BN, T>;
    const int tid = threadIdx.x;
    const int K = G * 32;
    constexpr int A_ROW_INT4 = kKB * 2;
#pragma unroll
    for (int i = 0; i < F::A_PER; i++) {
        const int e = tid + T * i;
        if (F::A_N % T == 0 || e < F::A_N) {
            const int r = e / A_ROW_INT4, c = e % A_ROW_INT4;
            const int m = min(m0 + r, M - 1);
            f.a[i] = *(const int4 *)(xq + (size_t)m * K + (size_t)g0 * 32 + c * 16);
        }
    }
    constexpr int WB = wcode_bytes<FMT>() / 16;  // int4 per block (2 for Q8_0: qs, qs2)
#pragma unroll
    for (int i = 0; i < F::B_PER; i++) {
        const int e = tid + T * i;
        if (F::B_N % T == 0 || e < F::B_N) {
            const int r = e / (kKB * WB), rem = e % (kKB * WB);
            const int blk = rem / WB, half = rem % WB;
            const int n = min(n0 + r, N - 1);
            const size_t idx = (size_t)n * G + g0 + blk;
            f.b[i] = (FMT == SLLM_Q8_0 && half) ? P.qs2[idx] : P.qs[idx];
        }
    }
#pragma unroll
    for (int i = 0; i < F::S_PER; i++) {
        const int e = tid + T * i;
        if (F::S_N % T == 0 || e < F::S_N) {
            const int blk = e / kBM, r = e % kBM;
            const int m = min(m0 + r, M - 1);
            f.xs[i] = xs[(size_t)m * G + g0 + blk];
            f.sx[i] = sx[(size_t)m * G + g0 + blk];
        }
    }
#pragma unroll
    for (int i = 0; i < F::W_PER; i++) {
        const int e = tid + T * i;
        if (F::W_N % T == 0 || e < F::W_N) {
            const int blk = e / BN, c = e % BN;
            const int n = min(n0 + c, N - 1);
            const size_t idx = (size_t)n * G + g0 + blk;
            f.d[i] = P.d[idx];
            if (FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) f.m[i] = P.m[idx];
            if (FMT == SLLM_Q5K1) {
                f.dh[i] = P.dh[idx];
                f.hb[i] = P.qh[idx];
            }
        }
    }
}

template <int FMT, int BN, int T>
__device__ __forceinline__ void store_stage(const Fetch<FMT, BN, T> &f, Stage<FMT, BN> &S) {
    using F = Fetch<FMT, BN, T>;
    const int tid = threadIdx.x;
    constexpr int A_ROW_INT4 = kKB * 2;
#pragma unroll
    for (int i = 0; i < F::A_PER; i++) {
        const int e = tid + T * i;
        if (F::A_N % T == 0 || e < F::A_N) {
            const int r = e / A_ROW_INT4, c = e % A_ROW_INT4;
            int2 *p = (int2 *)(S.a + r * kARow + c * 16);  // padded rows: 8-byte aligned
            p[0] = make_int2(f.a[i].x, f.a[i].y);
            p[1] = make_int2(f.a[i].z, f.a[i].w);
        }
    }
    constexpr int WB = wcode_bytes<FMT>() / 16;
#pragma unroll
    for (int i = 0; i < F::B_PER; i++) {
        const int e = tid + T * i;
        if (F::B_N % T == 0 || e < F::B_N) {
            const int r = e / (kKB * WB), rem = e % (kKB * WB);
            const int blk = rem / WB, half = rem % WB;
            int2 *p = (int2 *)(S.b + r * brow_bytes<FMT>() + blk * 32 + half * 16);
            if (FMT == SLLM_Q8_0) {
                p[0] = make_int2(f.b[i].x, f.b[i].y);
                p[1] = make_int2(f.b[i].z, f.b[i].w);
            } else {
                // byte j holds element j (low nibble) and j + 16 (high nibble)
                const int lo = 0x0f0f0f0f;
                p[0] = make_int2(f.b[i].x & lo, f.b[i].y & lo);
                p[1] = make_int2(f.b[i].z & lo, f.b[i].w & lo);
                p[2] = make_int2((f.b[i].x >> 4) & lo, (f.b[i].y >> 4) & lo);
                p[3] = make_int2((f.b[i].z >> 4) & lo, (f.b[i].w >> 4) & lo);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < F::S_PER; i++) {
        const int e = tid + T * i;
        if (F::S_N % T == 0 || e < F::S_N) {
            const int blk = e / kBM, r = e % kBM;
            S.xs[blk][r] = f.xs[i];
            // the float form is converted once here instead of per output
            S.sx[blk][r] = (FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) ? __float_as_int((float)f.sx[i]) : f.sx[i];
        }
    }
#pragma unroll
    for (int i = 0; i < F::W_PER; i++) {
        const int e = tid + T * i;
        if (F::W_N % T == 0 || e < F::W_N) {
            const int blk = e / BN, c = e % BN;
            S.d[blk][c] = (FMT == SLLM_Q8_0) ? f16_lut(f.d[i]) : f16_exact(f.d[i]);
            if (FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1)
                S.m[(FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) ? blk : 0][c] = f16_exact(f.m[i]);
            if (FMT == SLLM_Q5K1) {
                S.dh[FMT == SLLM_Q5K1 ? blk : 0][c] = f16_exact(f.dh[i]);
                S.hb[FMT == SLLM_Q5K1 ? blk : 0][c] = f.hb[i];
            }
        }
    }
}

// B operand from LDS: 8 codes (chunk c of the block) of weight row `row`.
template <int FMT, int BN>
__device__ __forceinline__ long b_frag(const Stage<FMT, BN> &S, int row, int blk, int c) {
    return *(const long *)(S.b + row * brow_bytes<FMT>() + blk * 32 + c * 8);
}

// Q5K1 high operand: elements 8c..8c+7 of the mask as 0/1 bytes.
__device__ __forceinline__ long bits_frag(uint32_t hb, int c) {
    const uint32_t t = hb >> (8 * c);
    return (long)((uint64_t)(uint32_t)spread4(t) | ((uint64_t)(uint32_t)spread4(t >> 4) << 32));
}

// Workgroup = 2 x WN waves; tile 64 x BN (BN = 32 WN); K stages [st0, st1).
template <int FMT, int WN>
__global__ void __launch_bounds__(128 * WN) gemm_kernel(Planes P, const int8_t *__restrict__ xq,
                                                        const float *__restrict__ xs, const int *__restrict__ sx,
                                                        float *__restrict__ out, int M, int N, int G, int mtiles,
                                                        int ntiles, int splits, int sps) {
    constexpr int BN = 32 * WN, T = 128 * WN;
    constexpr bool DUAL = FMT == SLLM_Q5K1;
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
    Stage<FMT, BN> *stages = (Stage<FMT, BN> *)lds_raw;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    // XCD-aware order: workgroup id -> XCD (id % 8); consecutive linear indices
    // (the M-tiles of one weight tile and split) stay on one XCD, so that
    // weight tile comes from HBM once into that XCD's L2.
    const int total = mtiles * ntiles * splits;
    const int per_xcd = (total + 7) / 8;
    const int lin = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (lin >= total) return;
    const int mt = lin % mtiles;
    const int rest = lin / mtiles;
    const int sp = rest % splits, nt = rest / splits;
    const int m0 = mt * kBM, n0 = nt * BN;
    const int r16 = lane & 15, c4 = lane >> 4;
    const int nst = G / kKB;
    const int st0 = sp * sps, st1 = min(nst, st0 + sps);

    float acc[2][2][4], acc2[DUAL ? 2 : 1][DUAL ? 2 : 1][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[i][j][r] = 0.0f;
                acc2[DUAL ? i : 0][DUAL ? j : 0][r] = 0.0f;
            }

    Fetch<FMT, BN, T> f;
    if (st0 < st1) {
        fetch_stage<FMT, BN, T>(f, P, xq, xs, sx, m0, n0, M, N, G, st0 * kKB);
        store_stage<FMT, BN, T>(f, stages[0]);
    }
    __syncthreads();

    for (int s = st0; s < st1; s++) {
        if (s + 1 < st1) fetch_stage<FMT, BN, T>(f, P, xq, xs, sx, m0, n0, M, N, G, (s + 1) * kKB);
        const Stage<FMT, BN> &S = stages[(s - st0) & 1];
#pragma unroll 1
        for (int blk = 0; blk < kKB; blk++) {
            long a[2];
            float4 xsr[2];
            int4 sxr[2];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int row = wm * 32 + 16 * i;
                a[i] = *(const long *)(S.a + (row + r16) * kARow + blk * 32 + c4 * 8);
                xsr[i] = *(const float4 *)&S.xs[blk][row + 4 * c4];
                sxr[i] = *(const int4 *)&S.sx[blk][row + 4 * c4];
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int col = wn * 32 + 16 * j + r16;
                const long b = b_frag<FMT, BN>(S, col, blk, c4);
                const float wd = S.d[blk][col];
                float wmn = 0.0f, wdh = 0.0f;
                long bh = 0;
                if (FMT == SLLM_Q4_1 || DUAL) wmn = S.m[(FMT == SLLM_Q4_1 || DUAL) ? blk : 0][col];
                if (DUAL) {
                    wdh = S.dh[DUAL ? blk : 0][col];
                    bh = bits_frag(S.hb[DUAL ? blk : 0][col], c4);
                }
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const v4i z = {0, 0, 0, 0};
                    const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], b, z, 0, 0, 0);
                    const float xv[4] = {xsr[i].x, xsr[i].y, xsr[i].z, xsr[i].w};
                    const int sv[4] = {sxr[i].x, sxr[i].y, sxr[i].z, sxr[i].w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        if (FMT == SLLM_Q8_0) {
                            // q8q8.go:193-195 + vnni_amd64.s:70-73
                            const float cmb = wd * xv[r];
                            const float term = cmb * (float)d[r];
                            acc[i][j][r] = acc[i][j][r] + term;
                        } else if (FMT == SLLM_Q4_0) {
                            // q4q8.go:37-43
                            const float cmb = wd * xv[r];
                            const float term = cmb * (float)(d[r] - 8 * sv[r]);
                            acc[i][j][r] = acc[i][j][r] + term;
                        } else {
                            // q41q8_row_amd64.s:65-71
                            const float t1 = (float)d[r] * wd;
                            const float t2 = __int_as_float(sv[r]) * wmn;
                            float tt = t1 + t2;
                            tt = tt * xv[r];
                            acc[i][j][r] = acc[i][j][r] + tt;
                        }
                    }
                    if (DUAL) {
                        const v4i h = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], bh, z, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            // The reference's high pass adds float(Σxq) * (+0), a
                            // signed zero (Σxq is finite): h1 + ±0 is h1 unless h1
                            // is itself a zero, and a zero term leaves acc2 (which
                            // starts at +0, so is never -0) unchanged whatever its
                            // sign. Omitting that add gives the same acc2 bits.
                            const float h1 = (float)h[r] * wdh;
                            const float hh = h1 * xv[r];
                            acc2[DUAL ? i : 0][DUAL ? j : 0][r] = acc2[DUAL ? i : 0][DUAL ? j : 0][r] + hh;
                        }
                    }
                }
            }
        }
        if (s + 1 < st1) store_stage<FMT, BN, T>(f, stages[(s + 1 - st0) & 1]);
        __syncthreads();
    }

    float *o = out + (size_t)sp * M * N;  // splits > 1: partial tile of split sp
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn * 32 + 16 * j + r16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 32 + 16 * i + 4 * c4 + r;
                if (m < M && n < N) {
                    float v = acc[i][j][r];
                    if (DUAL) v = v + acc2[DUAL ? i : 0][DUAL ? j : 0][r];
                    o[(size_t)m * N + n] = v;
                }
            }
        }
    }
}

// ------------------------------------------------------------- Q5_0 ----
//
// Q5_0 keeps fp32 activations (no int8 operand, float32_ops.go:427-436), so
// its prefill GEMM runs on the VALU. Each output's per-block sum is formed in
// the reference's operation order (q5DotGroupXF32, float32_ops.go:335-367):
// for j = 0..15, p0 = v0*x[j], p1 = v1*x[j+16], sum = sum + (p0 + p1), with
// v = float(q5) - 16; then term = d * sum, accumulated block by block. That
// is two fp32 VALU ops per weight and activation, so the VALU bounds it.
// A workgroup of 256 threads owns a 64 x 64 tile of dst; thread (tm, tn)
// owns activation rows tm + 16 r and weight rows tn + 16 c (r, c < 4). Per
// block the x tile and the decoded weight tile (fp32) are staged in LDS,
// double-buffered: the next block's global loads are in flight during the
// current block's arithmetic.
constexpr int kQ5Tile = 64;
constexpr int kQ5Stride = 36;  // floats per LDS row: 16-byte aligned, rows spread over the banks

struct alignas(16) Q5Stage {
    float x[kQ5Tile * kQ5Stride];
    float v[kQ5Tile * kQ5Stride];
    float d[kQ5Tile];
};

// This thread's share of one block's global operands: two float4 of x (rows
// t/8 and t/8 + 32) and four nibble bytes + high bits + scale of weight row t/4.
typedef float v4f __attribute__((ext_vector_type(4)));

struct Q5Fetch {
    v4f x0, x1;
    uint32_t qs, qh;
    uint16_t d;
};

__device__ __forceinline__ void q5_fetch(const Planes &P, const float *__restrict__ x, int M, int N, int G, int m0,
                                         int n0, int g, Q5Fetch &f) {
    const int t = threadIdx.x;
    // rows past M / N load the last row again; their outputs are not stored
    const int r = t >> 3, c = t & 7;
    const int ma = min(m0 + r, M - 1), mb = min(m0 + r + 32, M - 1);
    f.x0 = *((const v4f *)(x + ((size_t)ma * G + g) * 32) + c);
    f.x1 = *((const v4f *)(x + ((size_t)mb * G + g) * 32) + c);
    const int n = min(n0 + (t >> 2), N - 1);
    const size_t idx = (size_t)n * G + g;
    f.qs = ((const uint32_t *)(P.qs + idx))[t & 3];
    f.qh = P.qh[idx];
    f.d = P.d[idx];
}

__device__ __forceinline__ void q5_store(Q5Stage &S, const Q5Fetch &f) {
    const int t = threadIdx.x;
    const int r = t >> 3, c = t & 7;
    *(v4f *)(S.x + r * kQ5Stride + 4 * c) = f.x0;
    *(v4f *)(S.x + (r + 32) * kQ5Stride + 4 * c) = f.x1;
    // weight row t/4, elements 4 part .. 4 part + 3 (low nibbles) and 16 + those
    // (high nibbles); bit e of qh is bit 4 of element e (gguf.go:472-490)
    const int row = t >> 2, part = t & 3;
    float lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = 4 * part + i;
        const uint32_t b = (f.qs >> (8 * i)) & 0xffu;
        const int q0 = (int)((b & 0x0fu) | (((f.qh >> e) & 1u) << 4));
        const int q1 = (int)((b >> 4) | (((f.qh >> (e + 16)) & 1u) << 4));
        lo[i] = (float)q0 - 16.0f;
        hi[i] = (float)q1 - 16.0f;
    }
    *(v4f *)(S.v + row * kQ5Stride + 4 * part) = v4f{lo[0], lo[1], lo[2], lo[3]};
    *(v4f *)(S.v + row * kQ5Stride + 16 + 4 * part) = v4f{hi[0], hi[1], hi[2], hi[3]};
    if (part == 0) S.d[row] = f16_lut(f.d);
}

__device__ __forceinline__ float comp(const v4f &v, int k) { return v[k]; }

// Tile (mt, nt) of split sp; blocks [sp * bps, min(G, (sp + 1) * bps)).
__global__ void __launch_bounds__(256, 4) gemm_q5_kernel(Planes P, const float *__restrict__ x,
                                                      float *__restrict__ out, int M, int N, int G, int mtiles,
                                                      int ntiles, int splits, int bps) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
    Q5Stage *st = (Q5Stage *)lds_raw;
    // XCD-aware order, as in gemm_kernel: the M-tiles of one weight tile and
    // split run on one XCD, so the weight tile is read from HBM once into its L2
    const int total = mtiles * ntiles * splits;
    const int per_xcd = (total + 7) / 8;
    const int lin = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (lin >= total) return;
    const int mt = lin % mtiles;
    const int rest = lin / mtiles;
    const int sp = rest % splits, nt = rest / splits;
    const int m0 = mt * kQ5Tile, n0 = nt * kQ5Tile;
    const int g0 = sp * bps, g1 = min(G, g0 + bps);
    const int tn = threadIdx.x & 15, tm = threadIdx.x >> 4;

    float acc[4][4], sum[4][4];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[r][c] = 0.0f;

    Q5Fetch f;
    if (g0 < g1) {
        q5_fetch(P, x, M, N, G, m0, n0, g0, f);
        q5_store(st[0], f);
    }
    __syncthreads();
    for (int g = g0; g < g1; g++) {
        const int cur = (g - g0) & 1;
        if (g + 1 < g1) q5_fetch(P, x, M, N, G, m0, n0, g + 1, f);
        const Q5Stage &S = st[cur];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int c = 0; c < 4; c++) sum[r][c] = 0.0f;
#pragma unroll 1
        for (int j0 = 0; j0 < 16; j0 += 4) {
            // elements j0..j0+3 and 16+j0..: each output's sum still adds its
            // pairs in increasing j (the order across outputs is free)
            v4f xa[4], xb[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                xa[r] = *(const v4f *)(S.x + (tm + 16 * r) * kQ5Stride + j0);
                xb[r] = *(const v4f *)(S.x + (tm + 16 * r) * kQ5Stride + 16 + j0);
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const v4f va = *(const v4f *)(S.v + (tn + 16 * c) * kQ5Stride + j0);
                const v4f vb = *(const v4f *)(S.v + (tn + 16 * c) * kQ5Stride + 16 + j0);
#pragma unroll
                for (int k = 0; k < 4; k++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float p0 = comp(va, k) * comp(xa[r], k);
                        const float p1 = comp(vb, k) * comp(xb[r], k);
                        const float pair = p0 + p1;
                        sum[r][c] = sum[r][c] + pair;
                    }
            }
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float dd = S.d[tn + 16 * c];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float grp = dd * sum[r][c];
                acc[r][c] = acc[r][c] + grp;
            }
        }
        if (g + 1 < g1) q5_store(st[cur ^ 1], f);
        __syncthreads();
    }

    float *o = out + (size_t)sp * M * N;  // splits > 1: partial tile of split sp
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = m0 + tm + 16 * r;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int n = n0 + tn + 16 * c;
            if (m < M && n < N) o[(size_t)m * N + n] = acc[r][c];
        }
    }
}

// dst = part[0] + part[1] + ... + part[S-1], in split order.
__global__ void reduce_splits_kernel(const float *__restrict__ part, float *__restrict__ dst, size_t n, int S) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v = part[i];
        for (int s = 1; s < S; s++) v = v + part[(size_t)s * n + i];
        dst[i] = v;
    }
}

struct GemmPlan {
    int wn, splits, sps, mtiles, ntiles;
};

GemmPlan plan_gemm_q5(int M, int N, int G) {
    const int cus = 256;
    GemmPlan p{};
    p.wn = 0;
    p.mtiles = (M + kQ5Tile - 1) / kQ5Tile;
    p.ntiles = (N + kQ5Tile - 1) / kQ5Tile;
    int S = 1;
    while ((int64_t)p.mtiles * p.ntiles * S < 2 * cus && G / (S * 2) >= 4) S *= 2;
    p.splits = S;
    p.sps = (G + S - 1) / S;  // blocks per split
    return p;
}

GemmPlan plan_gemm(int fmt, int M, int N, int G) {
    if (fmt == SLLM_Q5_0) return plan_gemm_q5(M, N, G);
    const int cus = 256;
    GemmPlan p{};
    p.mtiles = (M + kBM - 1) / kBM;
    auto tiles = [&](int wn) { return (int64_t)p.mtiles * ((N + 32 * wn - 1) / (32 * wn)); };
    // 8-wave workgroups (64 x 128 tiles) from 64 such tiles, else 4-wave ones;
    // then K splits double until there are 1.5 workgroups per CU, each split
    // keeping >= 4 stages. Measured at M = 64 / 128 (µs): Q4_1 14336x4096
    // 44-46 -> 39-40 / 70-74 -> 62 against 4-wave tiles with 2 workgroups per
    // CU; Q8_0 4096x14336 at M = 64 keeps 4-wave tiles (35-38; 8-wave ones
    // 40); 2-wave workgroups were slower everywhere (Q8_0 at M = 64: 50)
    p.wn = tiles(4) >= 64 ? 4 : 2;
    if (tuning().gemm_wn) p.wn = tuning().gemm_wn;
    p.ntiles = (N + 32 * p.wn - 1) / (32 * p.wn);
    const int nst = G / kKB;
    int S = 1;
    while ((int64_t)p.mtiles * p.ntiles * S * 2 < 3 * cus && nst / (S * 2) >= 4) S *= 2;
    if (tuning().gemm_splits) S = tuning().gemm_splits < nst ? tuning().gemm_splits : nst;
    p.splits = S;
    p.sps = (nst + S - 1) / S;
    return p;
}

template <int FMT, int WN>
sllm_status launch_wn(const Planes &P, const int8_t *xq, const float *xsp, const int *sxp, float *out, int M,
                      int N, int G, const GemmPlan &p, hipStream_t s) {
    const int total = p.mtiles * p.ntiles * p.splits;
    const int grid = ((total + 7) / 8) * 8;
    const size_t lds = 2 * sizeof(Stage<FMT, 32 * WN>);
    hipLaunchKernelGGL((gemm_kernel<FMT, WN>), dim3(grid), dim3(128 * WN), lds, s, P, xq, xsp, sxp, out, M, N, G,
                       p.mtiles, p.ntiles, p.splits, p.sps);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

template <int FMT>
sllm_status launch_fmt(const Planes &P, const int8_t *xq, const float *xsp, const int *sxp, float *out, int M,
                       int N, int G, const GemmPlan &p, hipStream_t s) {
    switch (p.wn) {
    case 4: return launch_wn<FMT, 4>(P, xq, xsp, sxp, out, M, N, G, p, s);
    case 2: return launch_wn<FMT, 2>(P, xq, xsp, sxp, out, M, N, G, p, s);
    default: return launch_wn<FMT, 1>(P, xq, xsp, sxp, out, M, N, G, p, s);
    }
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

bool gemm_supported(int fmt, int G) {
    if (kq_native(fmt)) return false;  // the GEMV takes every row count
    return fmt == SLLM_Q5_0 ? G >= 1 : G % kKB == 0;
}

size_t gemm_workspace_bytes(int fmt, int N, int G, int M) {
    const GemmPlan p = plan_gemm(fmt, M, N, G);
    const size_t parts = p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
    if (fmt == SLLM_Q5_0) return align256(parts);
    return align256((size_t)M * G * 32) + 2 * align256((size_t)M * G * 4) + align256(parts);
}

sllm_status launch_gemm(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M, void *ws,
                        size_t ws_bytes, hipStream_t s) {
    if (ws_bytes < gemm_workspace_bytes(fmt, N, G, M)) return set_error(SLLM_ERR_ARG, "gemm: workspace too small");
    if (!gemm_supported(fmt, G)) return set_error(SLLM_ERR_SHAPE, "gemm: format or cols not supported");
    const GemmPlan p = plan_gemm(fmt, M, N, G);
    sllm_status st = SLLM_OK;
    float *part;
    if (fmt == SLLM_Q5_0) {
        part = (float *)ws;
        const int total = p.mtiles * p.ntiles * p.splits;
        hipLaunchKernelGGL(gemm_q5_kernel, dim3(((total + 7) / 8) * 8), dim3(256), 2 * sizeof(Q5Stage), s, P, x,
                           p.splits > 1 ? part : dst, M, N, G, p.mtiles, p.ntiles, p.splits, p.sps);
        SLLM_HIP(hipGetLastError());
    } else {
        int8_t *xq = (int8_t *)ws;
        const size_t q = align256((size_t)M * G * 32), sb = align256((size_t)M * G * 4);
        float *xsp = (float *)((char *)ws + q);
        int *sxp = (int *)((char *)ws + q + sb);
        part = (float *)((char *)ws + q + 2 * sb);
        st = launch_quantize_act(x, M, G, xq, xsp, sxp, s);
        if (st != SLLM_OK) return st;
        float *out = p.splits > 1 ? part : dst;
        switch (fmt) {
        case SLLM_Q8_0: st = launch_fmt<SLLM_Q8_0>(P, xq, xsp, sxp, out, M, N, G, p, s); break;
        case SLLM_Q4_0: st = launch_fmt<SLLM_Q4_0>(P, xq, xsp, sxp, out, M, N, G, p, s); break;
        case SLLM_Q4_1: st = launch_fmt<SLLM_Q4_1>(P, xq, xsp, sxp, out, M, N, G, p, s); break;
        case SLLM_Q5K1: st = launch_fmt<SLLM_Q5K1>(P, xq, xsp, sxp, out, M, N, G, p, s); break;
        default: return set_error(SLLM_ERR_QTYPE, "gemm: format has no int8 MFMA path");
        }
    }
    if (st != SLLM_OK || p.splits == 1) return st;
    const size_t n = (size_t)M * N;
    int grid = (int)((n + 255) / 256);
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(reduce_splits_kernel, dim3(grid), dim3(256), 0, s, part, dst, n, p.splits);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

}  // namespace sllm
