// Prefill GEMM (xRows >= 64): int8 matrix cores for Q8_0 / Q4_0 / Q4_1 / Q5K1,
// and a VALU GEMM for Q5_0 (fp32 activations; see gemm_q5_kernel below).
//
// 1. The activation rows are quantized once into a workspace (xq int8 [M][K],
//    xs fp32 [M][G], Σxq int32 [M][G]) by the GEMV prologue's routine.
// 2. A workgroup of WM x WN x WK waves computes a (32 WM) x (64 WN) tile of
//    dst; each wave a 32 x 64 sub-tile (two 32 x 32 MFMA tiles) over every
//    WK-th block of each K stage, the WK partial tiles added at the end in a
//    fixed tree order. K is staged KB blocks at a time through LDS,
//    double-buffered: the global loads of stage s+1 are in flight while stage
//    s is computed.
// 3. Per 32-element block a wave issues v_mfma_i32_32x32x32_i8 per 32 x 32
//    tile: K = 32 is exactly one block, so every result is one block's exact
//    int32 dot (the reference's isum / qsum). Its C operand is the int32 bit
//    pattern of 1.5 * 2^23 (Q4_0: minus 8 Σxq, q4q8.go:66-77), so each result
//    is the bit pattern of the float 1.5 * 2^23 + dot (exact: |dot| < 2^22):
//    the epilogue needs no int-to-float conversion.
// 4. The epilogue scales each block dot by its weight and activation scales
//    with fused multiply-adds, in the arrangement of the reference's arm64
//    kernels (q4q8_row_arm64.s, q41q8_row_arm64.s:59-63: per-lane FMLA
//    accumulators added at the end):
//      t   = fma(F, d, -1.5 * 2^23 * d)   = round(dot * d)  (exact addend)
//      Q4_1 / Q5K1: t = fma(float(Σxq), m, t)              (min term)
//      Q5K1: t = t + round(dot_high * d_high)               (high block)
//      acc = fma(t, xs, acc)
//    Each per-block term is rounded at most twice fewer times than in the
//    reference's x86 order (cmb = d * xs, term = cmb * float(dot), acc += term),
//    so every output differs from the reference's sequential sum by a few
//    ulp of sum |term| at most; the tests hold it to 1e-5 * sum |term|.
//    A K stage whose weight scales are not finite, or whose activation scales
//    reach 2^90 (where d * xs could overflow while dot * d does not), is
//    computed in the reference's exact operation order instead: the choice is
//    one per workgroup and stage (any thread that stores such a scale tags the
//    stage in LDS), and it keeps the reference's Inf / NaN results.
// 5. When there are too few tiles to fill the device, K is also split over S
//    workgroups; each writes its partial tile and a second kernel adds the S
//    partials in split order (fixed order: results are reproducible).
//
// MFMA operand layout (32x32x32 i8): A row i in lanes i and i + 32, 16 bytes
// each; B column j in lanes j and j + 32; D[i][j] in lane j + 32 h, element
// 4 q + r for i = 8 q + 4 h + r. A block's 32 codes are stored in LDS in the
// order (0..7, 16..23, 8..15, 24..31), so lane half h reads its 16 bytes with
// one ds_read_b128 and both operands pair the same elements.
#include <hip/hip_runtime.h>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

namespace sllm {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kMagicBits = 0x4B400000;  // 1.5 * 2^23
constexpr float kMagic = 12582912.0f;
constexpr float kHugeXs = 0x1p90f;      // activation scales from here on take the exact path

__host__ __device__ constexpr int row_bytes(int KB) { return KB * 32 + 16; }  // padded: conflict-free b128 reads

template <int FMT, int KB, int BM, int BN>
struct alignas(16) Stage {
    static constexpr bool HAS_MIN = FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1;
    static constexpr bool DUAL = FMT == SLLM_Q5K1;
    int8_t a[BM * row_bytes(KB)];                          // activation codes
    int8_t b[BN * row_bytes(KB)];  // weight codes (Q4_0: nib - 8, Q4_1 / Q5K1: nib, one per byte)
    int8_t bh[(DUAL ? BN : 1) * row_bytes(KB)];            // Q5K1 high bits as 0 / 1 bytes
    float xs[KB][BM];                                      // activation scales
    int aux[(FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) ? KB : 1][BM];  // float(Σxq) bits (exact, |Σxq| < 2^24)
    float d[KB][BN];                                       // weight scales (Q8_0: the reference's f16 table)
    float m[HAS_MIN ? KB : 1][BN];                         // mins
    float dh[DUAL ? KB : 1][BN];                           // Q5K1 high-block scales
    int tag;  // the K stage index whose data needs the exact epilogue (any thread that sees it writes it)
};

// Global -> register staging of one K stage, T threads; unit e of each kind is
// (row e / KB, block e % KB).
template <int FMT, int KB, int BM, int BN, int T>
struct Fetch {
    static constexpr int A_N = BM * KB, B_N = BN * KB;
    static constexpr int A_PER = (A_N + T - 1) / T, B_PER = (B_N + T - 1) / T;
    static constexpr bool Q8 = FMT == SLLM_Q8_0;
    int4 a[A_PER][2];
    int4 b[B_PER][Q8 ? 2 : 1];
    float xs[A_PER];
    int sx[A_PER];
    uint16_t d[B_PER], m[B_PER], dh[B_PER];
    uint32_t hb[B_PER];
};

template <int FMT, int KB, int BM, int BN, int T>
__device__ __forceinline__ void fetch_stage(Fetch<FMT, KB, BM, BN, T> &f, const Planes &P,
                                            const int8_t *__restrict__ xq, const float *__restrict__ xs,
                                            const int *__restrict__ sx, int m0, int n0, int M, int N, int G,
                                            int g0) {
    using F = Fetch<FMT, KB, BM, BN, T>;
    const int tid = threadIdx.x;
    const size_t K = (size_t)G * 32;
#pragma unroll
    for (int i = 0; i < F::A_PER; i++) {
        const int e = tid + T * i;
        if (F::A_N % T == 0 || e < F::A_N) {
            const int m = min(m0 + e / KB, M - 1);  // rows past M reload the last row; never stored
            const int4 *p = (const int4 *)(xq + (size_t)m * K + (size_t)(g0 + e % KB) * 32);
            f.a[i][0] = p[0];
            f.a[i][1] = p[1];
            const size_t si = (size_t)m * G + g0 + e % KB;
            f.xs[i] = xs[si];
            f.sx[i] = sx[si];
        }
    }
#pragma unroll
    for (int i = 0; i < F::B_PER; i++) {
        const int e = tid + T * i;
        if (F::B_N % T == 0 || e < F::B_N) {
            const int n = min(n0 + e / KB, N - 1);
            const size_t idx = (size_t)n * G + g0 + e % KB;
            f.b[i][0] = P.qs[idx];
            if (F::Q8) f.b[i][F::Q8 ? 1 : 0] = P.qs2[idx];
            f.d[i] = P.d[idx];
            if (FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) f.m[i] = P.m[idx];
            if (FMT == SLLM_Q5K1) {
                f.dh[i] = P.dh[idx];
                f.hb[i] = P.qh[idx];
            }
        }
    }
}

__device__ __forceinline__ bool f16_nonfinite(uint16_t h) { return (h & 0x7c00u) == 0x7c00u; }

// 8 bits -> 8 bytes of 0 / 1 (bit i -> byte i).
__device__ __forceinline__ int2 spread8(uint32_t b) {
    return make_int2(spread4(b & 0xfu), spread4((b >> 4) & 0xfu));
}

// Stores the fetched stage `stage` into LDS in the MFMA's element order; a
// thread that sees a scale needing the exact epilogue writes `stage` to S.tag.
template <int FMT, int KB, int BM, int BN, int T>
__device__ __forceinline__ void store_stage(const Fetch<FMT, KB, BM, BN, T> &f, Stage<FMT, KB, BM, BN> &S,
                                            int stage) {
    using F = Fetch<FMT, KB, BM, BN, T>;
    constexpr int RB = row_bytes(KB);
    const int tid = threadIdx.x;
    bool slow = false;
#pragma unroll
    for (int i = 0; i < F::A_PER; i++) {
        const int e = tid + T * i;
        if (F::A_N % T == 0 || e < F::A_N) {
            const int r = e / KB, blk = e % KB;
            // elements 0..15 = (x, y | z, w), 16..31 = (x, y | z, w) of the second int4
            const int4 lo = f.a[i][0], hi = f.a[i][1];
            int4 *p = (int4 *)(S.a + r * RB + blk * 32);
            p[0] = make_int4(lo.x, lo.y, hi.x, hi.y);
            p[1] = make_int4(lo.z, lo.w, hi.z, hi.w);
            S.xs[blk][r] = f.xs[i];
            if (FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) S.aux[blk][r] = __float_as_int((float)f.sx[i]);
            slow |= !(f.xs[i] < kHugeXs);
        }
    }
#pragma unroll
    for (int i = 0; i < F::B_PER; i++) {
        const int e = tid + T * i;
        if (F::B_N % T == 0 || e < F::B_N) {
            const int r = e / KB, blk = e % KB;
            int4 *p = (int4 *)(S.b + r * RB + blk * 32);
            if (F::Q8) {
                const int4 lo = f.b[i][0], hi = f.b[i][F::Q8 ? 1 : 0];
                p[0] = make_int4(lo.x, lo.y, hi.x, hi.y);
                p[1] = make_int4(lo.z, lo.w, hi.z, hi.w);
            } else {
                // byte j holds element j (low nibble) and element j + 16 (high nibble)
                const int4 v = f.b[i][0];
                int c[8] = {v.x & 0x0f0f0f0f, v.y & 0x0f0f0f0f, (v.x >> 4) & 0x0f0f0f0f, (v.y >> 4) & 0x0f0f0f0f,
                            v.z & 0x0f0f0f0f, v.w & 0x0f0f0f0f, (v.z >> 4) & 0x0f0f0f0f, (v.w >> 4) & 0x0f0f0f0f};
                if (FMT == SLLM_Q4_0) {
                    // the signed code nib - 8 per byte (q4q8.go:37-43): 0x80 + nib - 8 never
                    // borrows across bytes, and ^ 0x80 gives (nib - 8) mod 256
#pragma unroll
                    for (int k = 0; k < 8; k++) c[k] = ((c[k] | (int)0x80808080) - 0x08080808) ^ (int)0x80808080;
                }
                p[0] = make_int4(c[0], c[1], c[2], c[3]);
                p[1] = make_int4(c[4], c[5], c[6], c[7]);
            }
            S.d[blk][r] = (FMT == SLLM_Q8_0) ? f16_lut(f.d[i]) : f16_exact(f.d[i]);
            slow |= f16_nonfinite(f.d[i]);
            if (FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) {
                S.m[(FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) ? blk : 0][r] = f16_exact(f.m[i]);
                slow |= f16_nonfinite(f.m[i]);
            }
            if (FMT == SLLM_Q5K1) {
                S.dh[FMT == SLLM_Q5K1 ? blk : 0][r] = f16_exact(f.dh[i]);
                slow |= f16_nonfinite(f.dh[i]);
                const uint32_t hb = f.hb[i];  // bit e = high bit of element e
                int4 *q = (int4 *)(S.bh + r * RB + blk * 32);
                const int2 c0 = spread8(hb & 0xffu), c1 = spread8((hb >> 8) & 0xffu);
                const int2 c2 = spread8((hb >> 16) & 0xffu), c3 = spread8(hb >> 24);
                q[0] = make_int4(c0.x, c0.y, c2.x, c2.y);
                q[1] = make_int4(c1.x, c1.y, c3.x, c3.y);
            }
        }
    }
    if (slow) S.tag = stage;
}

// The LDS operands of one 32-element block for one wave's 32 x (32 CF) tile:
// the MFMA operands and the scales the epilogue applies.
template <int FMT, int CF>
struct Ops {
    static constexpr bool DUAL = FMT == SLLM_Q5K1;
    static constexpr bool HAS_MIN = FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1;
    v4i a;
    v4i b[CF], bh[DUAL ? CF : 1];
    float xv[16];                   // activation scales of the lane's 16 rows
    int av[HAS_MIN ? 16 : 1];       // float(Σxq) of those rows
    float wd[CF], wm[HAS_MIN ? CF : 1], wdh[DUAL ? CF : 1];
};

template <int FMT, int KB, int BM, int BN, int CF>
__device__ __forceinline__ void load_ops(Ops<FMT, CF> &o, const Stage<FMT, KB, BM, BN> &S, int blk, int wm, int wn,
                                         int lane) {
    constexpr int RB = row_bytes(KB);
    using O = Ops<FMT, CF>;
    const int r32 = lane & 31, h = lane >> 5;
    o.a = *(const v4i *)(S.a + (wm * 32 + r32) * RB + blk * 32 + 16 * h);
#pragma unroll
    for (int j = 0; j < CF; j++) {
        const int col = wn * 32 * CF + 32 * j + r32;
        o.b[j] = *(const v4i *)(S.b + col * RB + blk * 32 + 16 * h);
        if (O::DUAL) o.bh[O::DUAL ? j : 0] = *(const v4i *)(S.bh + col * RB + blk * 32 + 16 * h);
        o.wd[j] = S.d[blk][col];
        if (O::HAS_MIN) o.wm[O::HAS_MIN ? j : 0] = S.m[O::HAS_MIN ? blk : 0][col];
        if (O::DUAL) o.wdh[O::DUAL ? j : 0] = S.dh[O::DUAL ? blk : 0][col];
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 t = *(const float4 *)&S.xs[blk][wm * 32 + 8 * q + 4 * h];
        o.xv[4 * q] = t.x; o.xv[4 * q + 1] = t.y; o.xv[4 * q + 2] = t.z; o.xv[4 * q + 3] = t.w;
        if (O::HAS_MIN) {
            const int4 u = *(const int4 *)&S.aux[O::HAS_MIN ? blk : 0][wm * 32 + 8 * q + 4 * h];
            o.av[O::HAS_MIN ? 4 * q : 0] = u.x;
            o.av[O::HAS_MIN ? 4 * q + 1 : 0] = u.y;
            o.av[O::HAS_MIN ? 4 * q + 2 : 0] = u.z;
            o.av[O::HAS_MIN ? 4 * q + 3 : 0] = u.w;
        }
    }
}

// MFMA of column piece j: D = the bits of 1.5 * 2^23 + each block dot.
template <int FMT, int CF>
__device__ __forceinline__ void mfma_piece(const Ops<FMT, CF> &o, int j, const v16i &cmag, v16i &D, v16i &Dh) {
    D = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.b[j], cmag, 0, 0, 0);
    if (Ops<FMT, CF>::DUAL) Dh = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, o.bh[Ops<FMT, CF>::DUAL ? j : 0], cmag, 0, 0, 0);
}

// Epilogue of column piece j: SLOW is the reference's exact operation order.
template <int FMT, int CF, bool SLOW>
__device__ __forceinline__ void epilogue_piece(const Ops<FMT, CF> &o, int j, const v16i &D, const v16i &Dh,
                                               float (&acc)[CF][16]) {
    using O = Ops<FMT, CF>;
    const float wd = o.wd[j];
    const float wmn = O::HAS_MIN ? o.wm[O::HAS_MIN ? j : 0] : 0.0f;
    const float wdh = O::DUAL ? o.wdh[O::DUAL ? j : 0] : 0.0f;
    if (!SLOW) {
        const float cd = -kMagic * wd, cdh = -kMagic * wdh;  // exact: 2 significant bits x an f16
#pragma unroll
        for (int v = 0; v < 16; v++) {
            float t = __builtin_fmaf(__int_as_float(D[v]), wd, cd);
            if (O::HAS_MIN) t = __builtin_fmaf(__int_as_float(o.av[O::HAS_MIN ? v : 0]), wmn, t);
            if (O::DUAL) t = t + __builtin_fmaf(__int_as_float(Dh[v]), wdh, cdh);
            acc[j][v] = __builtin_fmaf(t, o.xv[v], acc[j][v]);
        }
    } else {
        // the reference's operation order (no contraction)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float dot = __int_as_float(D[v]) - kMagic;  // exact
            if (FMT == SLLM_Q8_0 || FMT == SLLM_Q4_0) {
                // q8q8.go:193-195 + vnni_amd64.s:70-73; q4q8.go:37-43
                const float cmb = wd * o.xv[v];
                const float term = cmb * dot;
                acc[j][v] = acc[j][v] + term;
            } else {
                // q41q8_row_amd64.s:65-71
                const float t1 = dot * wd;
                const float t2 = __int_as_float(o.av[O::HAS_MIN ? v : 0]) * wmn;
                float tt = t1 + t2;
                tt = tt * o.xv[v];
                acc[j][v] = acc[j][v] + tt;
                if (O::DUAL) {
                    // the high block's min is +0 (convertQ5KToTwoQ41): its term is float(dot) * dh * xs
                    const float h1 = (__int_as_float(Dh[v]) - kMagic) * wdh;
                    const float hh = h1 * o.xv[v];
                    acc[j][v] = acc[j][v] + hh;
                }
            }
        }
    }
}

// Debug: every block dot of column piece j to dots[((m * N + n) * G + g) * (1 | 2) + part].
template <int FMT, int CF>
__device__ __forceinline__ void dots_piece(int j, const v16i &D, const v16i &Dh, int *dots, int m0, int n0, int wm,
                                           int wn, int lane, int M, int N, int G, int g) {
    const int r32 = lane & 31, h = lane >> 5;
    const int n = n0 + wn * 32 * CF + 32 * j + r32;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int m = m0 + wm * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < M && n < N) {
            const size_t o = ((size_t)m * N + n) * G + g;
            if (FMT == SLLM_Q5K1) {
                dots[2 * o] = D[v] - kMagicBits;
                dots[2 * o + 1] = Dh[v] - kMagicBits;
            } else {
                dots[o] = D[v] - kMagicBits;
            }
        }
    }
}

// The NB blocks blk0, blk0 + WK, ... of one K stage for one wave, software-
// pipelined: block i+1's LDS operands are read before block i's epilogue, and
// its MFMA for piece j is issued as soon as block i's epilogue has consumed
// piece j's results, so the LDS and MFMA latencies of the next block overlap
// the current block's VALU work.
template <int FMT, int KB, int BM, int BN, int CF, int NB, int WK, bool PIPE, bool DBG>
__device__ __forceinline__ void stage_fast(const Stage<FMT, KB, BM, BN> &S, int blk0, int wm, int wn, int lane,
                                           const v16i &cmag, float (&acc)[CF][16], int *dots, int m0, int n0, int M,
                                           int N, int G, int g0) {
    if (!PIPE) {
        // one block at a time (fewer registers: leaves room for a deeper global prefetch)
#pragma unroll 1
        for (int i = 0; i < NB; i++) {
            Ops<FMT, CF> o;
            load_ops<FMT, KB, BM, BN, CF>(o, S, blk0 + i * WK, wm, wn, lane);
            v16i D[CF], Dh[CF];
#pragma unroll
            for (int j = 0; j < CF; j++) mfma_piece<FMT, CF>(o, j, cmag, D[j], Dh[j]);
#pragma unroll
            for (int j = 0; j < CF; j++) {
                if (DBG) dots_piece<FMT, CF>(j, D[j], Dh[j], dots, m0, n0, wm, wn, lane, M, N, G, g0 + blk0 + i * WK);
                epilogue_piece<FMT, CF, false>(o, j, D[j], Dh[j], acc);
            }
        }
        return;
    }
    Ops<FMT, CF> ops[2];
    v16i D[CF], Dh[CF];
    load_ops<FMT, KB, BM, BN, CF>(ops[0], S, blk0, wm, wn, lane);
#pragma unroll
    for (int j = 0; j < CF; j++) mfma_piece<FMT, CF>(ops[0], j, cmag, D[j], Dh[j]);
#pragma unroll
    for (int i = 0; i < NB; i++) {
        Ops<FMT, CF> &cur = ops[i & 1];
        Ops<FMT, CF> &nxt = ops[(i + 1) & 1];
        if (i + 1 < NB) load_ops<FMT, KB, BM, BN, CF>(nxt, S, blk0 + (i + 1) * WK, wm, wn, lane);
        // keep the next block's LDS reads ahead of this block's epilogue
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < CF; j++) {
            if (DBG) dots_piece<FMT, CF>(j, D[j], Dh[j], dots, m0, n0, wm, wn, lane, M, N, G, g0 + blk0 + i * WK);
            epilogue_piece<FMT, CF, false>(cur, j, D[j], Dh[j], acc);
            if (i + 1 < NB) mfma_piece<FMT, CF>(nxt, j, cmag, D[j], Dh[j]);
        }
    }
}

// The same blocks in the reference's exact operation order, one at a time.
template <int FMT, int KB, int BM, int BN, int CF, int NB, int WK, bool DBG>
__device__ __forceinline__ void stage_slow(const Stage<FMT, KB, BM, BN> &S, int blk0, int wm, int wn, int lane,
                                           const v16i &cmag, float (&acc)[CF][16], int *dots, int m0, int n0, int M,
                                           int N, int G, int g0) {
#pragma unroll 1
    for (int i = 0; i < NB; i++) {
        Ops<FMT, CF> o;
        load_ops<FMT, KB, BM, BN, CF>(o, S, blk0 + i * WK, wm, wn, lane);
#pragma unroll
        for (int j = 0; j < CF; j++) {
            v16i D, Dh;
            mfma_piece<FMT, CF>(o, j, cmag, D, Dh);
            if (DBG) dots_piece<FMT, CF>(j, D, Dh, dots, m0, n0, wm, wn, lane, M, N, G, g0 + blk0 + i * WK);
            epilogue_piece<FMT, CF, true>(o, j, D, Dh, acc);
        }
    }
}

// Workgroup = WM x WN x WK waves; tile (32 WM) x (32 CF WN); K stages [st0, st1).
// DBG: also write every block dot to dots[((m * N + n) * G + g) * (1 | 2) + part].
// PIPE: software-pipelined blocks (stage_fast); PF: K stages of global loads
// in flight (1: the next stage while this one is computed; 2: the next two).
template <int FMT, int WM, int WN, int CF, int WK, int KB, bool PIPE, int PF, bool DBG>
__global__ void __launch_bounds__(64 * WM * WN * WK) __attribute__((amdgpu_waves_per_eu(2))) gemm_kernel(
    Planes P, const int8_t *__restrict__ xq, const float *__restrict__ xs, const int *__restrict__ sx,
    float *__restrict__ out, int M, int N, int G, int mtiles, int ntiles, int splits, int sps,
    int *__restrict__ dots) {
    constexpr int BM = 32 * WM, BN = 32 * CF * WN, T = 64 * WM * WN * WK;
    static_assert(KB % WK == 0, "every wave takes the same number of blocks per stage");
    static_assert(CF % 2 == 0, "column pieces go in pairs");
    using St = Stage<FMT, KB, BM, BN>;
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
    St *stages = (St *)lds_raw;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wk = wave / (WM * WN), wmn = wave % (WM * WN);
    const int wm = wmn % WM, wn = wmn / WM;
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
    const int m0 = mt * BM, n0 = nt * BN;
    const int nst = G / KB;
    const int st0 = sp * sps, st1 = min(nst, st0 + sps);

    float acc[CF][16];
#pragma unroll
    for (int j = 0; j < CF; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;
    v16i cmag;
#pragma unroll
    for (int v = 0; v < 16; v++) cmag[v] = kMagicBits;

    if (threadIdx.x == 0) stages[0].tag = stages[1].tag = -1;
    __syncthreads();
    auto compute = [&](int st) {
        const St &S = stages[(st - st0) & 1];
        if (S.tag != st)
            stage_fast<FMT, KB, BM, BN, CF, KB / WK, WK, PIPE, DBG>(S, wk, wm, wn, lane, cmag, acc, dots, m0, n0, M,
                                                                    N, G, st * KB);
        else
            stage_slow<FMT, KB, BM, BN, CF, KB / WK, WK, DBG>(S, wk, wm, wn, lane, cmag, acc, dots, m0, n0, M, N, G,
                                                              st * KB);
    };
    using Fe = Fetch<FMT, KB, BM, BN, T>;
    if (PF == 1) {
        Fe f;
        if (st0 < st1) {
            fetch_stage<FMT, KB, BM, BN, T>(f, P, xq, xs, sx, m0, n0, M, N, G, st0 * KB);
            store_stage<FMT, KB, BM, BN, T>(f, stages[0], st0);
        }
        __syncthreads();
        for (int s = st0; s < st1; s++) {
            if (s + 1 < st1) fetch_stage<FMT, KB, BM, BN, T>(f, P, xq, xs, sx, m0, n0, M, N, G, (s + 1) * KB);
            compute(s);
            if (s + 1 < st1) store_stage<FMT, KB, BM, BN, T>(f, stages[(s + 1 - st0) & 1], s + 1);
            __syncthreads();
        }
    } else {
        // two fetch register sets, filled alternately two stages ahead
        Fe fa, fb;
        if (st0 < st1) {
            fetch_stage<FMT, KB, BM, BN, T>(fa, P, xq, xs, sx, m0, n0, M, N, G, st0 * KB);
            if (st0 + 1 < st1) fetch_stage<FMT, KB, BM, BN, T>(fb, P, xq, xs, sx, m0, n0, M, N, G, (st0 + 1) * KB);
            store_stage<FMT, KB, BM, BN, T>(fa, stages[0], st0);
        }
        __syncthreads();
        for (int s = st0; s < st1; s += 2) {
            // stage s: fb holds stage s + 1
            if (s + 2 < st1) fetch_stage<FMT, KB, BM, BN, T>(fa, P, xq, xs, sx, m0, n0, M, N, G, (s + 2) * KB);
            compute(s);
            if (s + 1 < st1) store_stage<FMT, KB, BM, BN, T>(fb, stages[(s + 1 - st0) & 1], s + 1);
            __syncthreads();
            if (s + 1 >= st1) break;
            // stage s + 1: fa holds stage s + 2
            if (s + 3 < st1) fetch_stage<FMT, KB, BM, BN, T>(fb, P, xq, xs, sx, m0, n0, M, N, G, (s + 3) * KB);
            compute(s + 1);
            if (s + 2 < st1) store_stage<FMT, KB, BM, BN, T>(fa, stages[(s + 2 - st0) & 1], s + 2);
            __syncthreads();
        }
    }

    // add the WK partial tiles: wk + step into wk, step = WK/2 .. 1 (fixed tree order)
    if (WK > 1) {
        float *red = (float *)lds_raw;  // [WK/2][WM*WN][16 * CF][64]
#pragma unroll
        for (int step = WK / 2; step >= 1; step /= 2) {
            if (wk >= step && wk < 2 * step) {
                float *r = red + ((size_t)((wk - step) * WM * WN + wmn) * 16 * CF) * 64;
#pragma unroll
                for (int j = 0; j < CF; j++)
#pragma unroll
                    for (int v = 0; v < 16; v++) r[(j * 16 + v) * 64 + lane] = acc[j][v];
            }
            __syncthreads();
            if (wk < step) {
                const float *r = red + ((size_t)(wk * WM * WN + wmn) * 16 * CF) * 64;
#pragma unroll
                for (int j = 0; j < CF; j++)
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[j][v] = acc[j][v] + r[(j * 16 + v) * 64 + lane];
            }
            __syncthreads();
        }
        if (wk != 0) return;
    }

    const int r32 = lane & 31, h = lane >> 5;
    float *o = out + (size_t)sp * M * N;  // splits > 1: partial tile of split sp
#pragma unroll
    for (int j = 0; j < CF; j++) {
        const int n = n0 + wn * 32 * CF + 32 * j + r32;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + wm * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
            if (m < M && n < N) o[(size_t)m * N + n] = acc[j][v];
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

// Workgroup shapes of the int8 GEMM (4 waves of 32 x 64, 4-block K stages).
// kWide: 64 x 128 tiles, the blocks of a stage software-pipelined, one stage
// of global loads in flight. kDeep: 64 x 64 tiles, two waves per 32 x 64
// taking alternate blocks of each stage, pipelined. kDeepS: kDeep computing
// one block at a time, two stages of global loads in flight. kDeepS32: 32 x 64
// tiles whose 4 waves take one block of each 4-block stage each (one block at
// a time, two stages in flight), for Q5K1 with up to 32 activation rows (the
// other formats measure faster on 64-row tiles even then: Q8_0 4096x14336 at
// M = 32 on 32 x 256 tiles 46.8 us against 34.7 at M = 33 on kWide).
enum GemmShape { kWide = 0, kDeep = 1, kDeepS = 2, kDeepS32 = 3 };

struct GemmPlan {
    int shape, bm, bn, kb, splits, sps, mtiles, ntiles;
};

GemmPlan plan_gemm_q5(int M, int N, int G) {
    const int cus = 256;
    GemmPlan p{};
    p.shape = 0;
    p.mtiles = (M + kQ5Tile - 1) / kQ5Tile;
    p.ntiles = (N + kQ5Tile - 1) / kQ5Tile;
    int S = 1;
    while ((int64_t)p.mtiles * p.ntiles * S < 2 * cus && G / (S * 2) >= 4) S *= 2;
    p.splits = S;
    p.sps = (G + S - 1) / S;  // blocks per split
    return p;
}

constexpr int shape_bm(int shape) { return shape == kDeepS32 ? 32 : 64; }
constexpr int shape_bn(int shape) { return shape == kWide ? 128 : 64; }
constexpr int shape_kb(int shape) { return 4; }

GemmPlan plan_gemm(int fmt, int M, int N, int G) {
    if (fmt == SLLM_Q5_0) return plan_gemm_q5(M, N, G);
    const int cus = 256;
    GemmPlan p{};
    // Q5K1 (two MFMAs and a longer epilogue per block, so twice the registers
    // per output) on the narrow tiles, the other formats on the wide ones.
    // Measured at M = 64 / 128 / 512 (us): Q4_1 14336x4096 wide 37 / 57 / 172,
    // deep 41 / 62 / 212; Q8_0 4096x14336 wide 37 / 52 / 148, deep 39 / 59 /
    // 180; Q5K1 14336x4096 kDeepS 52 / 85 / 276, kDeep 54 / 84 / 306, wide
    // 100 / 168 / 575 (its wide tiles spill).
    // (Q5K1 with up to 32 activation rows: 32-row tiles; Q5K1 4096x4096 at M
    // = 32 19.1 us against 23.2 at M = 33 on 64-row ones.)
    p.shape = fmt == SLLM_Q5K1 ? (M <= 32 ? kDeepS32 : kDeepS) : kWide;
    if (tuning().gemm_shape >= 1 && tuning().gemm_shape <= 4) p.shape = tuning().gemm_shape - 1;
    p.bm = shape_bm(p.shape);
    p.bn = shape_bn(p.shape);
    p.kb = shape_kb(p.shape);
    p.mtiles = (M + p.bm - 1) / p.bm;
    p.ntiles = (N + p.bn - 1) / p.bn;
    const int nst = G / p.kb;
    // K splits double until there are 1.5 workgroups per CU, each split keeping >= 2 stages
    int S = 1;
    while ((int64_t)p.mtiles * p.ntiles * S * 2 < 3 * cus && nst / (S * 2) >= 2) S *= 2;
    if (tuning().gemm_splits) S = tuning().gemm_splits < nst ? tuning().gemm_splits : nst;
    p.splits = S;
    p.sps = (nst + S - 1) / S;
    return p;
}

template <int FMT, int WM, int WN, int CF, int WK, int KB, bool PIPE, int PF, bool DBG>
sllm_status launch_shape(const Planes &P, const int8_t *xq, const float *xsp, const int *sxp, float *out, int M,
                         int N, int G, const GemmPlan &p, int *dots, hipStream_t s) {
    const int total = p.mtiles * p.ntiles * p.splits;
    const int grid = ((total + 7) / 8) * 8;
    constexpr size_t stages = 2 * sizeof(Stage<FMT, KB, 32 * WM, 32 * CF * WN>);
    constexpr size_t red = (size_t)(WK / 2) * WM * WN * 16 * CF * 64 * sizeof(float);
    constexpr size_t lds = stages > red ? stages : red;
    static_assert(lds <= 160 * 1024, "LDS");
    hipLaunchKernelGGL((gemm_kernel<FMT, WM, WN, CF, WK, KB, PIPE, PF, DBG>), dim3(grid), dim3(64 * WM * WN * WK), lds, s, P, xq,
                       xsp, sxp, out, M, N, G, p.mtiles, p.ntiles, p.splits, p.sps, dots);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

template <int FMT, bool DBG>
sllm_status launch_fmt(const Planes &P, const int8_t *xq, const float *xsp, const int *sxp, float *out, int M,
                       int N, int G, const GemmPlan &p, int *dots, hipStream_t s) {
    switch (p.shape) {
    case kDeep: return launch_shape<FMT, 2, 1, 2, 2, 4, true, 1, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
    case kDeepS: return launch_shape<FMT, 2, 1, 2, 2, 4, false, 2, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
    case kDeepS32: return launch_shape<FMT, 1, 1, 2, 4, 4, false, 2, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
    default: return launch_shape<FMT, 2, 2, 2, 1, 4, true, 1, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
    }
}

template <bool DBG>
sllm_status launch_int8(int fmt, const Planes &P, const int8_t *xq, const float *xsp, const int *sxp, float *out,
                        int M, int N, int G, const GemmPlan &p, int *dots, hipStream_t s) {
    switch (fmt) {
    case SLLM_Q8_0: return launch_fmt<SLLM_Q8_0, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
    case SLLM_Q4_0: return launch_fmt<SLLM_Q4_0, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
    case SLLM_Q4_1: return launch_fmt<SLLM_Q4_1, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
    case SLLM_Q5K1: return launch_fmt<SLLM_Q5K1, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
    }
    return set_error(SLLM_ERR_QTYPE, "gemm: format has no int8 MFMA path");
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

sllm_status gemm_impl(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M, void *ws,
                      size_t ws_bytes, int *dots, hipStream_t s) {
    if (ws_bytes < gemm_workspace_bytes(fmt, N, G, M)) return set_error(SLLM_ERR_ARG, "gemm: workspace too small");
    if (!gemm_supported(fmt, G)) return set_error(SLLM_ERR_SHAPE, "gemm: format or cols not supported");
    const GemmPlan p = plan_gemm(fmt, M, N, G);
    sllm_status st = SLLM_OK;
    float *part;
    if (fmt == SLLM_Q5_0) {
        if (dots) return set_error(SLLM_ERR_QTYPE, "gemm block dots: Q5_0 has no int8 GEMM");
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
        st = dots ? launch_int8<true>(fmt, P, xq, xsp, sxp, out, M, N, G, p, dots, s)
                  : launch_int8<false>(fmt, P, xq, xsp, sxp, out, M, N, G, p, nullptr, s);
    }
    if (st != SLLM_OK || p.splits == 1) return st;
    const size_t n = (size_t)M * N;
    int grid = (int)((n + 255) / 256);
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(reduce_splits_kernel, dim3(grid), dim3(256), 0, s, part, dst, n, p.splits);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

}  // namespace

bool gemm_supported(int fmt, int G) {
    if (kq_native(fmt)) return false;  // the GEMV takes every row count
    return fmt == SLLM_Q5_0 ? G >= 1 : G % shape_kb(kWide) == 0;
}

size_t gemm_workspace_bytes(int fmt, int N, int G, int M) {
    const GemmPlan p = plan_gemm(fmt, M, N, G);
    const size_t parts = p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
    if (fmt == SLLM_Q5_0) return align256(parts);
    return align256((size_t)M * G * 32) + 2 * align256((size_t)M * G * 4) + align256(parts);
}

sllm_status launch_gemm(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M, void *ws,
                        size_t ws_bytes, hipStream_t s) {
    return gemm_impl(fmt, P, x, dst, N, G, M, ws, ws_bytes, nullptr, s);
}

sllm_status launch_gemm_dots(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M, void *ws,
                             size_t ws_bytes, int32_t *dots, hipStream_t s) {
    if (!dots) return set_error(SLLM_ERR_ARG, "gemm block dots: null output");
    return gemm_impl(fmt, P, x, dst, N, G, M, ws, ws_bytes, dots, s);
}

}  // namespace sllm
