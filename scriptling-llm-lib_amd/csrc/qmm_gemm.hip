// Prefill GEMM (xRows >= 8 or 16): int8 matrix cores for Q8_0 / Q4_0 / Q4_1 /
// Q5K1, and bf16 matrix cores for Q5_0 (fp32 activations split exactly into
// three bf16 parts; see gemm_q5_kernel below).
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
//      Q5K1: t = t + round(dot_high * d_high)               (high block)
//      acc = fma(t, xs, acc)
//    The min term of Q4_1 / Q5K1, float(Σxq) * m * xs per block, factors into
//    a plain product over blocks, sum_g (float(Σxq) * xs)[m][g] * m[n][g]:
//    v_mfma_f32_32x32x2_f32 adds it two blocks at a time into the same
//    accumulator (min_piece), so the per-block VALU
//    work is two multiply-adds for Q4_1 (three in the reference's order).
//    Each part of a per-block term is rounded about as often as in the
//    reference's own order (cmb = d * xs, term = cmb * float(dot), acc +=
//    term; Q4_1: (dot * d + Σxq * m) * xs), so every output differs from the
//    reference's sequential sum by a few ulp of sum |term| at most (|term|
//    here counting the dot and min parts apart); the tests hold it to 1e-5 *
//    sum |term|.
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
// 4 q + r for i = 8 q + 4 h + r. A block's 32 codes are stored in LDS in
// element order and lane half h reads elements 16 h .. 16 h + 15 with one
// ds_read_b128, for both operands: whatever k each byte position stands for
// inside the instruction, both operands pair the same elements, and an int32
// dot does not depend on the order of its products.
#include <hip/hip_runtime.h>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

namespace sllm {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kMagicBits = 0x4B400000;  // 1.5 * 2^23
constexpr float kMagic = 12582912.0f;
constexpr float kHugeXs = 0x1p90f;      // activation scales from here on take the exact path

__host__ __device__ constexpr int row_bytes(int KB) { return KB * 32 + 16; }  // padded: conflict-free b128 reads

// Format traits. SLLM_Q5K1F is a Q5K1 weight with dh = 16 d in every block:
// its codes are staged as q5 = nib + 16 bit, so one MFMA gives dot5 = dot +
// 16 dot_h and dot5 * d = dot * d + dot_h * dh exactly; its dh plane is not
// read (the exact path splits the codes back into the two halves and takes
// 16 d for dh).
__host__ __device__ constexpr bool has_min(int f) { return f == SLLM_Q4_1 || f == SLLM_Q5K1 || f == SLLM_Q5K1F; }
__host__ __device__ constexpr bool two_mfma(int f) { return f == SLLM_Q5K1; }
__host__ __device__ constexpr bool has_dh(int f) { return f == SLLM_Q5K1; }
__host__ __device__ constexpr bool has_hb(int f) { return f == SLLM_Q5K1 || f == SLLM_Q5K1F; }

template <int FMT, int KB, int BM, int BN>
struct alignas(16) Stage {
    static constexpr bool HAS_MIN = has_min(FMT);
    static constexpr bool DUAL = two_mfma(FMT);
    int8_t a[BM * row_bytes(KB)];                          // activation codes
    int8_t b[BN * row_bytes(KB)];  // weight codes (Q4_0: nib - 8, Q4_1 / Q5K1: nib, Q5K1F: nib + 16 bit)
    int8_t bh[(DUAL ? BN : 1) * row_bytes(KB)];            // Q5K1 high bits as 0 / 1 bytes
    float xs[KB][BM];                                      // activation scales
    int aux[HAS_MIN ? KB : 1][BM];                         // float(Σxq) bits (exact, |Σxq| < 2^24)
    float d[KB][BN];                                       // weight scales (Q8_0: the reference's f16 table)
    float m[HAS_MIN ? KB : 1][BN];                         // mins
    float dh[has_dh(FMT) ? KB : 1][BN];                    // Q5K1 high-block scales
    int tag;  // the K stage index whose data needs the exact epilogue (any thread that sees it writes it)
};

// Global -> register staging of one K stage, T threads; unit e of each kind is
// (row e / KB, block e % KB).
template <int FMT, int KB, int BM, int BN, int T>
struct Fetch {
    static constexpr int A_N = BM * KB, B_N = BN * KB;
    static constexpr int A_PER = (A_N + T - 1) / T, B_PER = (B_N + T - 1) / T;
    static constexpr bool Q8 = FMT == SLLM_Q8_0;
    // native vectors: an array of HIP's int4 (a union) copied whole is kept in scratch memory
    v4i a[A_PER][2];
    v4i b[B_PER][Q8 ? 2 : 1];
    float xs[A_PER];
    int sx[A_PER];
    uint16_t d[B_PER], m[B_PER], dh[B_PER];
    uint32_t hb[B_PER];
};

// Which part of a stage a fetch / store moves: both, the activations only or
// the weights only.
enum StagePart { kBoth = 0, kActs = 1, kWeights = 2 };

template <int FMT, int KB, int BM, int BN, int T, int PART = kBoth>
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
        if (PART != kWeights && (F::A_N % T == 0 || e < F::A_N)) {
            const int m = min(m0 + e / KB, M - 1);  // rows past M reload the last row; never stored
            const v4i *p = (const v4i *)(xq + (size_t)m * K + (size_t)(g0 + e % KB) * 32);
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
        if (PART != kActs && (F::B_N % T == 0 || e < F::B_N)) {
            const int n = min(n0 + e / KB, N - 1);
            const size_t idx = (size_t)n * G + g0 + e % KB;
            f.b[i][0] = *(const v4i *)(P.qs + idx);
            if (F::Q8) f.b[i][F::Q8 ? 1 : 0] = *(const v4i *)(P.qs2 + idx);
            f.d[i] = P.d[idx];
            if (has_min(FMT)) f.m[i] = P.m[idx];
            if (has_dh(FMT)) f.dh[i] = P.dh[idx];
            if (has_hb(FMT)) f.hb[i] = P.qh[idx];
        }
    }
}

__device__ __forceinline__ bool f16_nonfinite(uint16_t h) { return (h & 0x7c00u) == 0x7c00u; }

// Stores the fetched stage `stage` into LDS in the MFMA's element order; a
// thread that sees a scale needing the exact epilogue writes `stage` to S.tag.
template <int FMT, int KB, int BM, int BN, int T, int PART = kBoth>
__device__ __forceinline__ void store_stage(const Fetch<FMT, KB, BM, BN, T> &f, Stage<FMT, KB, BM, BN> &S,
                                            int stage) {
    using F = Fetch<FMT, KB, BM, BN, T>;
    constexpr int RB = row_bytes(KB);
    const int tid = threadIdx.x;
    bool slow = false;
#pragma unroll
    for (int i = 0; i < F::A_PER; i++) {
        const int e = tid + T * i;
        if (PART != kWeights && (F::A_N % T == 0 || e < F::A_N)) {
            const int r = e / KB, blk = e % KB;
            v4i *p = (v4i *)(S.a + r * RB + blk * 32);
            p[0] = f.a[i][0];  // elements 0..15
            p[1] = f.a[i][1];  // elements 16..31
            S.xs[blk][r] = f.xs[i];
            if (has_min(FMT)) S.aux[blk][r] = __float_as_int((float)f.sx[i]);
            slow |= !(f.xs[i] < kHugeXs);
        }
    }
#pragma unroll
    for (int i = 0; i < F::B_PER; i++) {
        const int e = tid + T * i;
        if (PART != kActs && (F::B_N % T == 0 || e < F::B_N)) {
            const int r = e / KB, blk = e % KB;
            v4i *p = (v4i *)(S.b + r * RB + blk * 32);
            if (F::Q8) {
                p[0] = f.b[i][0];
                p[1] = f.b[i][F::Q8 ? 1 : 0];
            } else {
                // byte j holds element j (low nibble) and element j + 16 (high nibble)
                const v4i v = f.b[i][0];
                int c[8] = {v.x & 0x0f0f0f0f,        v.y & 0x0f0f0f0f,        v.z & 0x0f0f0f0f,
                            v.w & 0x0f0f0f0f,        (v.x >> 4) & 0x0f0f0f0f, (v.y >> 4) & 0x0f0f0f0f,
                            (v.z >> 4) & 0x0f0f0f0f, (v.w >> 4) & 0x0f0f0f0f};
                if (FMT == SLLM_Q4_0) {
                    // the signed code nib - 8 per byte (q4q8.go:37-43): 0x80 + nib - 8 never
                    // borrows across bytes, and ^ 0x80 gives (nib - 8) mod 256
#pragma unroll
                    for (int k = 0; k < 8; k++) c[k] = ((c[k] | (int)0x80808080) - 0x08080808) ^ (int)0x80808080;
                }
                if (FMT == SLLM_Q5K1F) {
                    // + 16 x the high bit; bits in group order: (hb >> k) & 0x01010101
                    // are elements 4k .. 4k + 3, the elements of c[k]
                    const int hb = (int)f.hb[i];
#pragma unroll
                    for (int k = 0; k < 8; k++) c[k] |= ((hb >> k) & 0x01010101) << 4;
                }
                p[0] = v4i{c[0], c[1], c[2], c[3]};
                p[1] = v4i{c[4], c[5], c[6], c[7]};
            }
            S.d[blk][r] = (FMT == SLLM_Q8_0) ? f16_lut(f.d[i]) : f16_exact(f.d[i]);
            slow |= f16_nonfinite(f.d[i]);
            if (has_min(FMT)) {
                S.m[has_min(FMT) ? blk : 0][r] = f16_exact(f.m[i]);
                slow |= f16_nonfinite(f.m[i]);
            }
            if (has_dh(FMT)) {
                S.dh[has_dh(FMT) ? blk : 0][r] = f16_exact(f.dh[i]);
                slow |= f16_nonfinite(f.dh[i]);
            }
            if (FMT == SLLM_Q5K1) {
                // high bits in group order: (hb >> k) & 0x01010101 = elements 4k .. 4k + 3
                const int hb = (int)f.hb[i];
                constexpr int m = 0x01010101;
                v4i *q = (v4i *)(S.bh + r * RB + blk * 32);
                q[0] = v4i{hb & m, (hb >> 1) & m, (hb >> 2) & m, (hb >> 3) & m};
                q[1] = v4i{(hb >> 4) & m, (hb >> 5) & m, (hb >> 6) & m, (hb >> 7) & m};
            }
        }
    }
    if (slow) S.tag = stage;
}

// The LDS operands of one 32-element block for one wave's 32 x (32 CF) tile:
// the MFMA operands and the scales the epilogue applies.
template <int FMT, int CF>
struct Ops {
    static constexpr bool DUAL = two_mfma(FMT);
    static constexpr bool HAS_MIN = has_min(FMT);
    v4i a;
    v4i b[CF], bh[DUAL ? CF : 1];
    float xv[16];                   // activation scales of the lane's 16 rows
    int av[HAS_MIN ? 16 : 1];       // float(Σxq) of those rows
    float wd[CF], wm[HAS_MIN ? CF : 1], wdh[DUAL ? CF : 1];
};

// AV: also the rows' float(Σxq) (only the exact epilogue adds the min term
// per block; the fast path adds it on the fp32 matrix cores, see min_piece).
template <int FMT, int KB, int BM, int BN, int CF, bool AV = false>
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
        if (O::HAS_MIN && AV) {
            const int4 u = *(const int4 *)&S.aux[O::HAS_MIN ? blk : 0][wm * 32 + 8 * q + 4 * h];
            o.av[O::HAS_MIN ? 4 * q : 0] = u.x;
            o.av[O::HAS_MIN ? 4 * q + 1 : 0] = u.y;
            o.av[O::HAS_MIN ? 4 * q + 2 : 0] = u.z;
            o.av[O::HAS_MIN ? 4 * q + 3 : 0] = u.w;
        }
    }
}

// The min term of Q4_1 / Q5K1 on the fp32 matrix cores: sum over blocks g of
// float(Σxq[m][g]) * xs[m][g] * m[n][g] is a plain product of an M x G and a
// G x N matrix, so v_mfma_f32_32x32x2_f32 adds it two blocks at a time into
// the tile's accumulator (A: row m's fl(float(Σxq) * xs) in lane m % 32, of
// block blkA in lanes 0..31 and blkB in lanes 32..63; B: the mins of the same
// blocks for column n), and the per-block epilogue keeps one multiply-add
// fewer. blkB < 0: the upper k slot is zero.
template <int CF>
struct MinOps {
    float a;
    float b[CF];
};

template <int FMT, int KB, int BM, int BN, int CF>
__device__ __forceinline__ void load_min(MinOps<CF> &o, const Stage<FMT, KB, BM, BN> &S, int blkA, int blkB, int wm,
                                         int wn, int lane) {
    constexpr bool HAS_MIN = has_min(FMT);
    const int r32 = lane & 31, h = lane >> 5;
    const int blk = h ? blkB : blkA;
    const bool live = blk >= 0;
    const int bi = HAS_MIN && live ? blk : 0;
    const int row = wm * 32 + r32;
    o.a = live ? __int_as_float(S.aux[HAS_MIN ? bi : 0][row]) * S.xs[bi][row] : 0.0f;
#pragma unroll
    for (int j = 0; j < CF; j++) o.b[j] = live ? S.m[HAS_MIN ? bi : 0][wn * 32 * CF + 32 * j + r32] : 0.0f;
}

template <int CF>
__device__ __forceinline__ void min_piece(const MinOps<CF> &o, int j, v16f &acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(o.a, o.b[j], acc, 0, 0, 0);
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
                                               v16f (&acc)[CF]) {
    using O = Ops<FMT, CF>;
    const float wd = o.wd[j];
    const float wmn = O::HAS_MIN ? o.wm[O::HAS_MIN ? j : 0] : 0.0f;
    const float wdh = O::DUAL ? o.wdh[O::DUAL ? j : 0] : 0.0f;
    if (!SLOW) {
        const float cd = -kMagic * wd, cdh = -kMagic * wdh;  // exact: 2 significant bits x an f16
#pragma unroll
        for (int v = 0; v < 16; v++) {
            float t = __builtin_fmaf(__int_as_float(D[v]), wd, cd);
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

// Debug: the block dots of column piece j as dots_piece writes them. Q5K1F:
// the two halves' dots of the Q5K1 layout, from the MFMA the epilogue scales
// (dot5 = dot + 16 dot_h) and one more of the high bits alone: dot = dot5 - 16
// dot_h.
template <int FMT, int CF>
__device__ __forceinline__ void dbg_dots(const Ops<FMT, CF> &o, int j, const v16i &cmag, const v16i &D,
                                         const v16i &Dh, int *dots, int m0, int n0, int wm, int wn, int lane, int M,
                                         int N, int G, int g) {
    if constexpr (FMT == SLLM_Q5K1F) {
        const v16i H = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, (o.b[j] >> 4) & 0x01010101, cmag, 0, 0, 0);
        v16i L;
#pragma unroll
        for (int v = 0; v < 16; v++) L[v] = D[v] - 16 * (H[v] - kMagicBits);
        dots_piece<SLLM_Q5K1, CF>(j, L, H, dots, m0, n0, wm, wn, lane, M, N, G, g);
    } else {
        dots_piece<FMT, CF>(j, D, Dh, dots, m0, n0, wm, wn, lane, M, N, G, g);
    }
}

// The NB blocks blk0, blk0 + WK, ... of one K stage for one wave, software-
// pipelined: block i+1's LDS operands are read before block i's epilogue, and
// its MFMA for piece j is issued as soon as block i's epilogue has consumed
// piece j's results, so the LDS and MFMA latencies of the next block overlap
// the current block's VALU work. Q4_1 / Q5K1: the min terms of blocks i and
// i + 1 go into acc (min_piece) at every even i.
template <int FMT, int KB, int BM, int BN, int CF, int NB, int WK, bool PIPE, bool DBG>
__device__ __forceinline__ void stage_fast(const Stage<FMT, KB, BM, BN> &S, int blk0, int wm, int wn, int lane,
                                           const v16i &cmag, v16f (&acc)[CF], int *dots,
                                           int m0, int n0, int M, int N, int G, int g0) {
    constexpr bool HAS_MIN = has_min(FMT);
    auto min_pair = [&](int i, MinOps<CF> &mo) {
        load_min<FMT, KB, BM, BN, CF>(mo, S, blk0 + i * WK, i + 1 < NB ? blk0 + (i + 1) * WK : -1, wm, wn, lane);
    };
    if (!PIPE) {
        // one block at a time (fewer registers: leaves room for a deeper global prefetch)
#pragma unroll 1
        for (int i = 0; i < NB; i++) {
            Ops<FMT, CF> o;
            load_ops<FMT, KB, BM, BN, CF>(o, S, blk0 + i * WK, wm, wn, lane);
            MinOps<CF> mo;
            if (HAS_MIN && (i & 1) == 0) min_pair(i, mo);
            v16i D[CF], Dh[CF];
#pragma unroll
            for (int j = 0; j < CF; j++) mfma_piece<FMT, CF>(o, j, cmag, D[j], Dh[j]);
            if (HAS_MIN && (i & 1) == 0) {
#pragma unroll
                for (int j = 0; j < CF; j++) min_piece<CF>(mo, j, acc[j]);
            }
#pragma unroll
            for (int j = 0; j < CF; j++) {
                if (DBG) dbg_dots<FMT, CF>(o, j, cmag, D[j], Dh[j], dots, m0, n0, wm, wn, lane, M, N, G, g0 + blk0 + i * WK);
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
        MinOps<CF> mo;
        if (HAS_MIN && (i & 1) == 0) min_pair(i, mo);
        // keep the next block's LDS reads ahead of this block's epilogue
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < CF; j++) {
            if (DBG) dbg_dots<FMT, CF>(cur, j, cmag, D[j], Dh[j], dots, m0, n0, wm, wn, lane, M, N, G, g0 + blk0 + i * WK);
            epilogue_piece<FMT, CF, false>(cur, j, D[j], Dh[j], acc);
            // fence the MFMA between two epilogue pieces: left to itself the
            // scheduler sinks all of the next block's MFMAs below the last
            // piece, and the next epilogue then waits out their latency
            __builtin_amdgcn_sched_barrier(0);
            if (i + 1 < NB) mfma_piece<FMT, CF>(nxt, j, cmag, D[j], Dh[j]);
            if (HAS_MIN && (i & 1) == 0) min_piece<CF>(mo, j, acc[j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// The same blocks in the reference's exact operation order, one at a time.
template <int FMT, int KB, int BM, int BN, int CF, int NB, int WK, bool DBG>
__device__ __forceinline__ void stage_slow(const Stage<FMT, KB, BM, BN> &S, int blk0, int wm, int wn, int lane,
                                           const v16i &cmag, v16f (&acc)[CF], int *dots, int m0, int n0, int M,
                                           int N, int G, int g0) {
#pragma unroll 1
    for (int i = 0; i < NB; i++) {
        const int blk = blk0 + i * WK;
        Ops<FMT, CF> o;
        load_ops<FMT, KB, BM, BN, CF, true>(o, S, blk, wm, wn, lane);
        if constexpr (FMT == SLLM_Q5K1F) {
            // the two halves apart, as Q5K1: low nibbles and high bits of the
            // 5-bit codes, each half with its own scale
            Ops<SLLM_Q5K1, CF> q;
            q.a = o.a;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                q.xv[v] = o.xv[v];
                q.av[v] = o.av[v];
            }
#pragma unroll
            for (int j = 0; j < CF; j++) {
                q.b[j] = o.b[j] & 0x0f0f0f0f;
                q.bh[j] = (o.b[j] >> 4) & 0x01010101;
                q.wd[j] = o.wd[j];
                q.wm[j] = o.wm[j];
                q.wdh[j] = 16.0f * o.wd[j];  // dh, exactly
            }
#pragma unroll
            for (int j = 0; j < CF; j++) {
                v16i D, Dh;
                mfma_piece<SLLM_Q5K1, CF>(q, j, cmag, D, Dh);
                if (DBG) dots_piece<SLLM_Q5K1, CF>(j, D, Dh, dots, m0, n0, wm, wn, lane, M, N, G, g0 + blk);
                epilogue_piece<SLLM_Q5K1, CF, true>(q, j, D, Dh, acc);
            }
        } else {
#pragma unroll
            for (int j = 0; j < CF; j++) {
                v16i D, Dh;
                mfma_piece<FMT, CF>(o, j, cmag, D, Dh);
                if (DBG) dots_piece<FMT, CF>(j, D, Dh, dots, m0, n0, wm, wn, lane, M, N, G, g0 + blk);
                epilogue_piece<FMT, CF, true>(o, j, D, Dh, acc);
            }
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

    v16f acc[CF];
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
    if constexpr (PF == 1) {
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
    } else if constexpr (FMT == SLLM_Q4_1) {
        // The weights two stages ahead in two register sets filled alternately,
        // the activations (mostly L2 hits) one stage ahead in a third. Each
        // stage's activations are issued before the weights of the stage after
        // it, so waiting for them leaves those weights in flight. Q4_1 only:
        // with whole stages in both sets its 64 x 128 kernel spills, and the
        // reloads wait for every load in flight (14336x4096 at M = 512 / 1024:
        // 164-166 / 287-292 -> 160-161 / 277-280 us); Q8_0 and Q5K1 fit and
        // gain nothing from it.
        Fe fa, fb, xa;
        auto put = [&](const Fe &w, int s) {
            store_stage<FMT, KB, BM, BN, T, kActs>(xa, stages[(s - st0) & 1], s);
            store_stage<FMT, KB, BM, BN, T, kWeights>(w, stages[(s - st0) & 1], s);
        };
        if (st0 < st1) {
            fetch_stage<FMT, KB, BM, BN, T>(fa, P, xq, xs, sx, m0, n0, M, N, G, st0 * KB);
            if (st0 + 1 < st1)
                fetch_stage<FMT, KB, BM, BN, T, kWeights>(fb, P, xq, xs, sx, m0, n0, M, N, G, (st0 + 1) * KB);
            store_stage<FMT, KB, BM, BN, T>(fa, stages[0], st0);
        }
        __syncthreads();
        for (int s = st0; s < st1; s += 2) {
            // stage s: fb holds the weights of stage s + 1
            if (s + 1 < st1) fetch_stage<FMT, KB, BM, BN, T, kActs>(xa, P, xq, xs, sx, m0, n0, M, N, G, (s + 1) * KB);
            if (s + 2 < st1) fetch_stage<FMT, KB, BM, BN, T, kWeights>(fa, P, xq, xs, sx, m0, n0, M, N, G, (s + 2) * KB);
            compute(s);
            if (s + 1 < st1) put(fb, s + 1);
            __syncthreads();
            if (s + 1 >= st1) break;
            // stage s + 1: fa holds the weights of stage s + 2
            if (s + 2 < st1) fetch_stage<FMT, KB, BM, BN, T, kActs>(xa, P, xq, xs, sx, m0, n0, M, N, G, (s + 2) * KB);
            if (s + 3 < st1) fetch_stage<FMT, KB, BM, BN, T, kWeights>(fb, P, xq, xs, sx, m0, n0, M, N, G, (s + 3) * KB);
            compute(s + 1);
            if (s + 2 < st1) put(fa, s + 2);
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
// Q5_0 keeps fp32 activations (no int8 operand, float32_ops.go:427-436): each
// block's sum is sum_j v_j x_j over its 32 elements (v = q5 - 16, the pairs j
// and j + 16 added in j order by q5DotGroupXF32, float32_ops.go:335-367), then
// term = d * sum. On the matrix cores:
// * a pre-pass splits every activation exactly into three bf16 parts, x = hi
//   + mid + lo: hi the top 8 significand bits (truncated), mid the next 8 of
//   the remainder, lo the remainder itself, which has at most 8 significant
//   bits left and so is a bf16 (a non-finite x: hi = x, mid = lo = 0);
// * v is a small integer, exact in bf16, so v_mfma_f32_32x32x16_bf16 over the
//   three parts forms every product v * part exactly and each block's sum in
//   fp32 (summed in the matrix core's order instead of the reference's j
//   order: reassociation only);
// * the epilogue adds the block term with one fused multiply-add,
//   acc = fma(f16lut(d), sum, acc) (the reference rounds d * sum first).
// A workgroup of 4 waves owns a 64 x 128 tile (each wave 32 x 64: two 32 x 32
// MFMA tiles); one block per K stage through LDS, double-buffered; split-K
// with the fixed-order reduction when tiles are few.

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kQ5BM = 64;
constexpr int kQ5Pieces = kQ5BM * 12;  // 16-byte pieces of a block-stage's activation parts
constexpr int kQ5Row = 40;  // bf16 per LDS row of one block: 32 + 8 pad (80 B: conflict-free b128 reads)

// x [M][K] fp32 -> xs3 [M][G][3][32] bf16: the hi, mid and lo parts of each block.
__global__ void split_act_kernel(const float *__restrict__ x, size_t nblocks, uint16_t *__restrict__ xs3) {
    // one thread per 8 elements (two float4)
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nblocks * 4;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t blk = i >> 2;
        const int c = (int)(i & 3);
        const float4 *src = (const float4 *)(x + blk * 32 + 8 * c);
        const float4 u0 = src[0], u1 = src[1];
        const float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
        uint32_t hi[4], mid[4], lo[4];
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            uint32_t ph[2], pm[2], pl[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const float f = v[k + e];
                const uint32_t ub = __float_as_uint(f);
                if ((ub & 0x7f800000u) == 0x7f800000u) {  // Inf / NaN: the value itself, no remainder
                    ph[e] = ub >> 16;
                    pm[e] = pl[e] = 0;
                    continue;
                }
                const float h = __uint_as_float(ub & 0xffff0000u);
                const float r1 = f - h;  // exact
                const float m = __uint_as_float(__float_as_uint(r1) & 0xffff0000u);
                const float r2 = r1 - m;  // exact, and a bf16
                ph[e] = ub >> 16;
                pm[e] = __float_as_uint(m) >> 16;
                pl[e] = __float_as_uint(r2) >> 16;
            }
            hi[k >> 1] = ph[0] | (ph[1] << 16);
            mid[k >> 1] = pm[0] | (pm[1] << 16);
            lo[k >> 1] = pl[0] | (pl[1] << 16);
        }
        uint16_t *dst = xs3 + blk * 96 + 8 * c;
        *(uint4 *)dst = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4 *)(dst + 32) = make_uint4(mid[0], mid[1], mid[2], mid[3]);
        *(uint4 *)(dst + 64) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
}

template <int BN>
struct alignas(16) Q5Stage {
    uint16_t a[3][kQ5BM][kQ5Row];  // activation parts (bf16), elements in block order
    uint16_t b[BN][kQ5Row];        // weights q5 - 16 (bf16, exact)
    float d[BN];                   // f16lut(d) (the reference's table decode)
};

// One thread's share of one block-stage (T = 2 BN threads): pieces t, t + T,
// ... of the activation parts (64 rows x 3 parts x 4 pieces of 16 bytes), and
// half a weight row's block (row t / 2, elements 8 h .. 8 h + 7 and their + 16
// partners, h = t % 2).
template <int T>
struct Q5Fetch {
    static constexpr int A_PER = (kQ5Pieces + T - 1) / T;
    v4i a[A_PER];  // a native vector: an array of HIP's int4 (a union) is kept in scratch memory
    uint2 qs;
    uint32_t qh;
    uint16_t d;
};

template <int T>
__device__ __forceinline__ void q5m_fetch(Q5Fetch<T> &f, const Planes &P, const uint16_t *__restrict__ xs3, int M,
                                          int N, int G, int m0, int n0, int g) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < Q5Fetch<T>::A_PER; i++) {
        // piece e: row e / 12, part (e % 12) / 4, 16 bytes e % 4; a thread past
        // the last piece reloads it (never stored): the loads stay unconditional,
        // so the array stays in registers
        const int e = min(t + T * i, kQ5Pieces - 1);
        const int m = min(m0 + e / 12, M - 1);  // rows past M reload the last row; never stored
        const int rem = e % 12;
        f.a[i] = *(const v4i *)(xs3 + ((size_t)m * G + g) * 96 + (rem >> 2) * 32 + (rem & 3) * 8);
    }
    const int n = min(n0 + (t >> 1), N - 1);
    const size_t idx = (size_t)n * G + g;
    f.qs = ((const uint2 *)(P.qs + idx))[t & 1];
    f.qh = P.qh[idx];
    f.d = P.d[idx];
}

// bf16 bits of the small integer v (exact).
__device__ __forceinline__ uint32_t bf16_of_int(int v) { return __float_as_uint((float)v) >> 16; }

template <int T>
__device__ __forceinline__ void q5m_store(const Q5Fetch<T> &f, Q5Stage<T / 2> &S) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < Q5Fetch<T>::A_PER; i++) {
        const int e = t + T * i;
        if (kQ5Pieces % T == 0 || e < kQ5Pieces) {
            const int rem = e % 12;
            *(v4i *)&S.a[rem >> 2][e / 12][(rem & 3) * 8] = f.a[i];
        }
    }
    // weight row t / 2: nibble bytes 8 h .. 8 h + 7 hold elements j (low) and
    // j + 16 (high); bit e of qh is bit 4 of element e (gguf.go:472-490)
    const int row = t >> 1, h = t & 1;
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        uint32_t pl[2], ph[2];
#pragma unroll
        for (int e2 = 0; e2 < 2; e2++) {
            const int k2 = k + e2;
            const uint32_t byte = ((k2 < 4 ? f.qs.x : f.qs.y) >> (8 * (k2 & 3))) & 0xffu;
            const int j = 8 * h + k2;
            const int q0 = (int)((byte & 0x0fu) | (((f.qh >> j) & 1u) << 4));
            const int q1 = (int)((byte >> 4) | (((f.qh >> (j + 16)) & 1u) << 4));
            pl[e2] = bf16_of_int(q0 - 16);
            ph[e2] = bf16_of_int(q1 - 16);
        }
        lo[k >> 1] = pl[0] | (pl[1] << 16);
        hi[k >> 1] = ph[0] | (ph[1] << 16);
    }
    *(uint4 *)&S.b[row][8 * h] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *(uint4 *)&S.b[row][16 + 8 * h] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    if (h == 0) S.d[row] = f16_lut(f.d);
}

// One block's MFMAs and epilogue for one wave's 32 x 64 tile.
template <int BN>
__device__ __forceinline__ void q5m_block(const Q5Stage<BN> &S, int wm, int wn, int r32, int h, float (&acc)[2][16]) {
    // operands of one step at a time (step s: elements 16 s .. 16 s + 15, lane
    // half h 8 of them): the whole block's would hold 40 registers, and at 4
    // waves per SIMD the global prefetch then spills
    v16f sum[2] = {};
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
        v8bf a[3], b[2];
#pragma unroll
        for (int part = 0; part < 3; part++)
            a[part] = __builtin_bit_cast(v8bf, *(const int4 *)&S.a[part][wm * 32 + r32][16 * s2 + 8 * h]);
#pragma unroll
        for (int j = 0; j < 2; j++)
            b[j] = __builtin_bit_cast(v8bf, *(const int4 *)&S.b[wn * 64 + 32 * j + r32][16 * s2 + 8 * h]);
#pragma unroll
        for (int part = 0; part < 3; part++)
#pragma unroll
            for (int j = 0; j < 2; j++) sum[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[part], b[j], sum[j], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const float dd = S.d[wn * 64 + 32 * j + r32];
#pragma unroll
        for (int v = 0; v < 16; v++) acc[j][v] = __builtin_fmaf(dd, sum[j][v], acc[j][v]);
    }
}

// Tile (mt, nt) of split sp; blocks [sp * bps, min(G, (sp + 1) * bps)); a
// workgroup of 2 x WN waves owns a 64 x 64 WN tile. PF: blocks of global loads
// in flight (two register sets filled alternately).
template <int WN, int PF>
__global__ void __launch_bounds__(128 * WN) gemm_q5_kernel(Planes P, const uint16_t *__restrict__ xs3,
                                                      float *__restrict__ out, int M, int N, int G, int mtiles,
                                                      int ntiles, int splits, int bps) {
    constexpr int BN = 64 * WN, T = 128 * WN;
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
    Q5Stage<BN> *st = (Q5Stage<BN> *)lds_raw;
    // XCD-aware order, as in gemm_kernel: the M-tiles of one weight tile and
    // split run on one XCD, so the weight tile is read from HBM once into its
    // L2 (measured against the other way round, one activation tile per XCD:
    // 14336x4096 at M = 512 648 against 853 us)
    const int total = mtiles * ntiles * splits;
    const int per_xcd = (total + 7) / 8;
    const int lin = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (lin >= total) return;
    const int mt = lin % mtiles;
    const int rest = lin / mtiles;
    const int sp = rest % splits, nt = rest / splits;
    const int m0 = mt * kQ5BM, n0 = nt * BN;
    const int g0 = sp * bps, g1 = min(G, g0 + bps);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int r32 = lane & 31, h = lane >> 5;

    float acc[2][16];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;

    if constexpr (PF == 1) {
        Q5Fetch<T> f;
        if (g0 < g1) {
            q5m_fetch(f, P, xs3, M, N, G, m0, n0, g0);
            q5m_store(f, st[0]);
        }
        __syncthreads();
        for (int g = g0; g < g1; g++) {
            const int cur = (g - g0) & 1;
            if (g + 1 < g1) q5m_fetch(f, P, xs3, M, N, G, m0, n0, g + 1);
            q5m_block(st[cur], wm, wn, r32, h, acc);
            if (g + 1 < g1) q5m_store(f, st[cur ^ 1]);
            __syncthreads();
        }
    } else {
        Q5Fetch<T> fa, fb;
        if (g0 < g1) {
            q5m_fetch(fa, P, xs3, M, N, G, m0, n0, g0);
            if (g0 + 1 < g1) q5m_fetch(fb, P, xs3, M, N, G, m0, n0, g0 + 1);
            q5m_store(fa, st[0]);
        }
        __syncthreads();
        for (int g = g0; g < g1; g += 2) {
            // block g: fb holds block g + 1
            if (g + 2 < g1) q5m_fetch(fa, P, xs3, M, N, G, m0, n0, g + 2);
            q5m_block(st[(g - g0) & 1], wm, wn, r32, h, acc);
            if (g + 1 < g1) q5m_store(fb, st[(g + 1 - g0) & 1]);
            __syncthreads();
            if (g + 1 >= g1) break;
            // block g + 1: fa holds block g + 2
            if (g + 3 < g1) q5m_fetch(fb, P, xs3, M, N, G, m0, n0, g + 3);
            q5m_block(st[(g + 1 - g0) & 1], wm, wn, r32, h, acc);
            if (g + 2 < g1) q5m_store(fa, st[(g + 2 - g0) & 1]);
            __syncthreads();
        }
    }

    float *o = out + (size_t)sp * M * N;  // splits > 1: partial tile of split sp
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = n0 + wn * 64 + 32 * j + r32;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + wm * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
            if (m < M && n < N) o[(size_t)m * N + n] = acc[j][v];
        }
    }
}

// dst = part[0] + part[1] + ... + part[S-1], added in split order. V floats
// per thread (V = 4: float4 loads and stores, n a multiple of 4 and dst 16-byte
// aligned); the loads of up to eight splits are issued before their adds (a
// load-add chain waited for every split's load in turn).
template <int V>
__global__ void reduce_splits_kernel(const float *__restrict__ part, float *__restrict__ dst, size_t n, int S) {
    typedef float vec __attribute__((ext_vector_type(V)));
    const size_t nv = n / V;
    const vec *pv = (const vec *)part;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += (size_t)gridDim.x * blockDim.x) {
        vec v = pv[i];
        for (int s0 = 1; s0 < S; s0 += 8) {
            vec p[8];
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (s0 + k < S) p[k] = pv[(size_t)(s0 + k) * nv + i];
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (s0 + k < S) v = v + p[k];
        }
        ((vec *)dst)[i] = v;
    }
}

// Workgroup shapes of the int8 GEMM (4 waves of 32 x 64, 4-block K stages).
// kWide: 64 x 128 tiles, the blocks of a stage software-pipelined, one stage
// of global loads in flight; kWide2: the same with two stages in flight, for
// more than 128 rows (Q8_0 4096x14336 at M = 256 / 512 / 1024 79.6 / 139.1 /
// 245.6 us against 82.8 / 143.8 / 254.9, Q4_1 14336x4096 89.9 / 162.4 /
// 289.7 against 91.0 / 167.1 / 287.7; at M = 64 35.1 against 33.6 and 37.3
// against 34.5). kDeep: 64 x 64 tiles, two waves per 32 x 64
// taking alternate blocks of each stage, pipelined. kDeepS: kDeep computing
// one block at a time, two stages of global loads in flight. kDeepS32: 32 x 64
// tiles whose 4 waves take one block of each 4-block stage each (one block at
// a time, two stages in flight), for Q5K1 with up to 32 activation rows (the
// other formats measure faster on 64-row tiles even then: Q8_0 4096x14336 at
// M = 32 on 32 x 256 tiles 46.8 us against 34.7 at M = 33 on kWide).
enum GemmShape { kWide = 0, kDeep = 1, kDeepS = 2, kDeepS32 = 3, kWide2 = 4 };

struct GemmPlan {
    int shape, bm, bn, kb, splits, sps, mtiles, ntiles;
};

GemmPlan plan_gemm_q5(int M, int N, int G) {
    const int cus = 256;
    GemmPlan p{};
    p.shape = 0;
    p.bm = kQ5BM;
    // 64 x 256 tiles (8 waves) halve the activation parts' re-reads across
    // N-tiles: 14336x4096 at M = 16 / 64 / 128 / 512 54.7 / 60.9 / 106.5 /
    // 357.3 us against 58.5 / 65.3 / 119.8 / 397.3 on 64 x 128 tiles (4
    // waves), which stay ahead up to 4096 weight rows at few activation rows
    // (4096x4096 at M = 16 / 64 / 128: 26.1 / 30.2 / 38.9 against 30.0 / 33.3
    // / 39.5; 1024x4096: 20.8 / 25.2 / 27.4 against 22.3 / 26.2 / 31.6)
    p.bn = (N > 4096 || M > 128) ? 256 : 128;
    if (tuning().gemm_shape == 1) p.bn = 256;
    if (tuning().gemm_shape == 2) p.bn = 128;
    p.kb = 1;
    p.mtiles = (M + kQ5BM - 1) / kQ5BM;
    p.ntiles = (N + p.bn - 1) / p.bn;
    // K splits double until there are 1.5 workgroups per CU, each split keeping >= 4 blocks
    int S = 1;
    while ((int64_t)p.mtiles * p.ntiles * S * 2 < 3 * cus && G / (S * 2) >= 4) S *= 2;
    if (tuning().gemm_splits) S = tuning().gemm_splits < G ? tuning().gemm_splits : G;
    p.splits = S;
    p.sps = (G + S - 1) / S;  // blocks per split
    return p;
}

constexpr int shape_bm(int shape) { return shape == kDeepS32 ? 32 : 64; }
constexpr int shape_bn(int shape) { return shape == kWide || shape == kWide2 ? 128 : 64; }
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
    // = 32 19.1 us against 23.2 at M = 33 on 64-row ones.) Q5K1F (one MFMA
    // per block): 32-row tiles up to 32 rows, 64 x 64 up to 128, then 64 x
    // 128 with one stage in flight (its two-stage kernel spills). Measured
    // (us, kDeepS32 / kDeep / kWide): 14336x4096 at M = 16 28.7 / 31.5 / 30.3,
    // M = 64 44.0 / 35.8 / 35.9, M = 512 264.9 / 187.4 / 175.4 (kWide2 208);
    // 4096x4096 at M = 64 21.3 / 21.0 / 25.4, M = 512 85.3 / 61.8 / 60.0.
    if (fmt == SLLM_Q5K1F)
        p.shape = M <= 32 ? kDeepS32 : (M <= 128 ? kDeep : kWide);
    else
        p.shape = fmt == SLLM_Q5K1 ? (M <= 32 ? kDeepS32 : kDeepS) : (M > 128 ? kWide2 : kWide);
    if (tuning().gemm_shape >= 1 && tuning().gemm_shape <= 5) p.shape = tuning().gemm_shape - 1;
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
    case kWide2: return launch_shape<FMT, 2, 2, 2, 1, 4, true, 2, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
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
    case SLLM_Q5K1F: return launch_fmt<SLLM_Q5K1F, DBG>(P, xq, xsp, sxp, out, M, N, G, p, dots, s);
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
        uint16_t *xs3 = (uint16_t *)ws;
        part = (float *)((char *)ws + align256((size_t)M * G * 96 * sizeof(uint16_t)));
        const size_t nblocks = (size_t)M * G;
        int sgrid = (int)((nblocks * 4 + 255) / 256);
        if (sgrid > 4096) sgrid = 4096;
        hipLaunchKernelGGL(split_act_kernel, dim3(sgrid), dim3(256), 0, s, x, nblocks, xs3);
        SLLM_HIP(hipGetLastError());
        const int total = p.mtiles * p.ntiles * p.splits;
        dim3 grid(((total + 7) / 8) * 8);
        float *o = p.splits > 1 ? part : dst;
        if (p.bn == 256)
            hipLaunchKernelGGL((gemm_q5_kernel<4, 1>), grid, dim3(512), 2 * sizeof(Q5Stage<256>), s, P, xs3, o, M, N,
                               G, p.mtiles, p.ntiles, p.splits, p.sps);
        else
            hipLaunchKernelGGL((gemm_q5_kernel<2, 1>), grid, dim3(256), 2 * sizeof(Q5Stage<128>), s, P, xs3, o, M, N,
                               G, p.mtiles, p.ntiles, p.splits, p.sps);
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
    const bool v4 = n % 4 == 0 && ((uintptr_t)dst & 15) == 0;
    int grid = (int)((n / (v4 ? 4 : 1) + 255) / 256);
    if (grid > 4096) grid = 4096;
    if (v4)
        hipLaunchKernelGGL(reduce_splits_kernel<4>, dim3(grid), dim3(256), 0, s, part, dst, n, p.splits);
    else
        hipLaunchKernelGGL(reduce_splits_kernel<1>, dim3(grid), dim3(256), 0, s, part, dst, n, p.splits);
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
    if (fmt == SLLM_Q5_0) return align256((size_t)M * G * 96 * sizeof(uint16_t)) + align256(parts);
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
