// Decode GEMV kernel templates, shared by the per-format translation units
// (qmm_gemv_<fmt>.hip instantiate the launch chain for one weight format each,
// so they compile in parallel) and by the planner in qmm_gemv.hip.
//
// Decode GEMV (xRows < 64) for every weight format.
//
// Persistent launch (at most gemv_wg_per_cu workgroups per CU). Each wave owns
// RPW rows (consecutive ones for an odd RPW, else rows wv, wv + TW, ...) and
// streams them as units of NB blocks per lane (one K-chunk of a row), keeping
// D units in flight in a register ring.
//   1. threads that own an activation block issue its loads first, then every
//      wave issues its first unit of weight loads, the owners quantize their
//      block into LDS with the bit-exact Q8_0 quantizer (Q5_0: stage the fp32
//      block), then the waves issue the rest of their first D units - the
//      weight stream is in flight during the prologue;
//   2. main loop: lane l owns blocks l + 64 i of each K-chunk; it reads the
//      block's activation codes from LDS, forms the reference's per-block term
//      exactly and accumulates; at a row's end the wave reduces across lanes
//      (fixed order) and parks the sum in lane (row ordinal); results are
//      stored once at the end, one coalesced store per wave.
// The per-block term equals the reference's bit for bit; only the order in
// which a row's terms are added differs from the reference's sequential loop
// (reassociation), and that order is fixed, so results are reproducible.
#pragma once

#include <hip/hip_runtime.h>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"
#include "qmm_q6k.hpp"

namespace sllm {
namespace gemv {


typedef int v4i __attribute__((ext_vector_type(4)));

// Weight planes are read once per GEMV: non-temporal loads keep them from
// displacing the activations and other reused data in L2 / MALL.
__device__ __forceinline__ int4 ld_nt(const int4 *p) {
    const v4i t = __builtin_nontemporal_load((const v4i *)p);
    return make_int4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint16_t ld_nt(const uint16_t *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ uint32_t ld_nt(const uint32_t *p) { return __builtin_nontemporal_load(p); }
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ld_nt(const uint2 *p) {
    const v2u t = __builtin_nontemporal_load((const v2u *)p);
    return make_uint2(t.x, t.y);
}

// LDS image of the prologue for MT activation rows of G blocks.
struct ActView {
    int4 *xl;   // [MT][G] elements 0..15 of each block (int8)
    int4 *xh;   // [MT][G] elements 16..31
    float *xs;  // [MT][G] activation scale
    int *sx;    // [MT][G] Σxq
    float *xf;  // fp32-activation formats: [MT][G][kXfStride] fp32 activations
};

__host__ __device__ inline size_t act_lds_bytes(int fmt, int MT, int G) {
    if (act_f32(fmt)) return (size_t)MT * G * kXfStride * sizeof(float);
    return (size_t)MT * G * (2 * sizeof(int4) + sizeof(float) + sizeof(int));
}

__device__ inline ActView carve_act(unsigned char *lds, int fmt, int MT, int G) {
    ActView v{};
    if (act_f32(fmt)) {
        v.xf = (float *)lds;
    } else {
        v.xl = (int4 *)lds;
        v.xh = v.xl + (size_t)MT * G;
        v.xs = (float *)(v.xh + (size_t)MT * G);
        v.sx = (int *)(v.xs + (size_t)MT * G);
    }
    return v;
}

// Writes one lane's part (8/TPB float4 = 32/TPB elements) of activation block
// blk into LDS: quantized codes + scale + Σq, or (fp32-activation formats)
// the fp32 values.
template <int FMT, int TPB>
__device__ __forceinline__ void stage_part(const float4 *v, int blk, int sub, const ActView &A) {
    constexpr int NV = 8 / TPB;
    if (act_f32(FMT)) {
        float4 *d = (float4 *)(A.xf + (size_t)blk * kXfStride) + sub * NV;
#pragma unroll
        for (int k = 0; k < NV; k++) d[k] = v[k];
    } else {
        int w[NV];
        float s;
        int sm;
        quantize_part<TPB>(v, w, s, sm);
        // word j of the block (j = sub*NV + k): words 0..3 -> xl, 4..7 -> xh
        int *lo = (int *)(A.xl + blk), *hi = (int *)(A.xh + blk);
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int j = sub * NV + k;
            if (j < 4) lo[j] = w[k];
            else hi[j - 4] = w[k];
        }
        if (sub == 0) {
            A.xs[blk] = s;
            A.sx[blk] = sm;
        }
    }
}

// Per-lane register image of one weight block.
struct BlockRegs {
    int4 q, q2;
    uint16_t d, m, dh;
    uint32_t qh;
    uint2 c2;      // native k-quants: the 2-bit codes; Q6_K streamed: the top code bits
    uint32_t sbw;  // native k-quants: the super-block's scale word
    int4 hq;       // Q4_K streamed: the super-block's GGUF header
    uint32_t jj;   // Q4_K streamed: the block's index in its super-block
};
// Q6_K streamed uses q (low nibbles), c2 (top bits), qh (the m6 word) and d
// (the super-block's d).

template <class T>
__device__ __forceinline__ const T *at(const T *base, uint32_t idx) {
    // base + 32-bit byte offset: lets the loads use the SGPR-base + VGPR-offset form
    return (const T *)((const char *)base + (uint64_t)(idx * (uint32_t)sizeof(T)));
}

template <int FMT>
__device__ __forceinline__ void load_block(const Planes &P, uint32_t idx, BlockRegs &b) {
    if (kq_native(FMT)) {
        b.c2 = ld_nt(at(P.q2, idx));
        b.d = ld_nt(at(P.d, idx));
        b.sbw = ld_nt(at(P.sb, idx >> 3));  // rows hold whole super-blocks (G % 8 == 0)
        if (FMT == SLLM_Q3K) b.qh = ld_nt(at(P.qh, idx));
        return;
    }
    if (FMT == SLLM_Q6K_STREAM) {
        b.q = ld_nt(at(P.l6, idx));
        b.c2 = ld_nt(at(P.h6, idx));
        b.qh = ld_nt(at(P.m6, idx));
        b.d = ld_nt(at(P.d6, idx >> 3));  // rows hold whole super-blocks (G % 8 == 0)
        return;
    }
    b.q = ld_nt(at(P.qs, idx));
    if (FMT == SLLM_Q4K_STREAM) {
        b.hq = ld_nt(at(P.hdr, idx >> 3));  // rows hold whole super-blocks (G % 8 == 0)
        b.jj = idx & 7u;
        return;
    }
    b.d = ld_nt(at(P.d, idx));
    if (FMT == SLLM_Q8_0) b.q2 = ld_nt(at(P.qs2, idx));
    if (FMT == SLLM_Q4_1 || FMT == SLLM_Q5K1) b.m = ld_nt(at(P.m, idx));
    if (FMT == SLLM_Q5K1) b.dh = ld_nt(at(P.dh, idx));
    if (FMT == SLLM_Q5_0 || FMT == SLLM_Q5K1) b.qh = ld_nt(at(P.qh, idx));
}

// Blocks lane + 64 i (i < NB) of one unit, starting at plane index `base`.
template <int FMT, int NB>
__device__ __forceinline__ void load_unit(const Planes &P, BlockRegs (&u)[NB], uint32_t base) {
#pragma unroll
    for (int i = 0; i < NB; i++) load_block<FMT>(P, base + 64u * i, u[i]);
}

// Activation operands of one block, read from LDS.
struct ActRegs {
    int4 xl, xh;
    float xs;
    int sx;
    float4 xf[8];
};

template <int FMT>
__device__ __forceinline__ void load_act(const ActView &A, size_t a, ActRegs &r) {
    if (act_f32(FMT)) {
        const float4 *src = (const float4 *)(A.xf + a * kXfStride);
#pragma unroll
        for (int k = 0; k < 8; k++) r.xf[k] = src[k];
    } else {
        r.xl = A.xl[a];
        r.xh = A.xh[a];
        r.xs = A.xs[a];
        r.sx = A.sx[a];
    }
}

// Adds one block's term to acc (acc2: the Q5K1 high half), in the reference's
// operation order for that format.
// Element e (0..31) of a block's fp32 activations (e a compile-time constant).
__device__ __forceinline__ float elem(const float4 *v, int e) {
    const float4 t = v[e >> 2];
    return (e & 3) == 0 ? t.x : ((e & 3) == 1 ? t.y : ((e & 3) == 2 ? t.z : t.w));
}

template <int FMT>
__device__ __forceinline__ void block_term(const BlockRegs &b, const ActRegs &x, float &acc, float &acc2,
                                           const unsigned char *q5tab = nullptr) {
    if (FMT == SLLM_Q2K) {
        // dequantizeQ2KNative (kquants.go:147-180) gives w = float32(d*sc*q -
        // dmin*m); here both products are exact in float32 and the difference
        // is rounded once, to the same float32. Then the dense loop's product
        // x * w (modelMatmulFloatIntoF32, float32_ops.go:475-477), summed per block.
        const float d = f16_exact((uint16_t)(b.sbw & 0xffffu)), dm = f16_exact((uint16_t)(b.sbw >> 16));
        float sum = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t sc = ((uint32_t)b.d >> (8 * h)) & 0xffu;
            const float dl = d * (float)(sc & 0xfu), ml = dm * (float)(sc >> 4);
            const uint32_t w = h ? b.c2.y : b.c2.x;
            // codes l, l+4, l+8, l+12 as the bytes of sp[l & 3]: each converts
            // with one byte-to-float instruction (no per-code bit extract; the
            // empty asm keeps the compiler from folding the masks back into
            // one extract per code)
            uint32_t sp[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sp[j] = (w >> (2 * j)) & 0x03030303u;
                asm volatile("" : "+v"(sp[j]));
            }
#pragma unroll
            for (int l = 0; l < 16; l++) {
                const float q = (float)((sp[l & 3] >> (8 * (l >> 2))) & 0xffu);
                // dl * q is exact (at most 17 significant bits), so one fused
                // multiply-add rounds the difference exactly as mul + sub does
                const float wt = __builtin_fmaf(dl, q, -ml);
                sum = sum + elem(x.xf, 16 * h + l) * wt;
            }
        }
        acc = acc + sum;
    } else if (FMT == SLLM_Q3K) {
        // dequantizeQ3KNative (kquants.go:183-245): w = float32(d*(sc-32)*(q -
        // sub)), sub 4 unless the element's high-mask bit is set - an exact
        // float32 product here. Then x * w as above.
        const float d = f16_exact((uint16_t)(b.sbw & 0xffffu));
        float sum = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float dl = d * (float)(int)(int8_t)(((uint32_t)b.d >> (8 * h)) & 0xffu);
            const float ndl4 = -4.0f * dl;
            const uint32_t w = h ? b.c2.y : b.c2.x;
            const uint32_t hb = b.qh >> (16 * h);  // 0: subtract 4
            // q + 4 = code + 4 * (high bit), in 0..7, for elements l, l+4,
            // l+8, l+12 as the bytes of sp[l & 3] (the high bits moved from
            // stride 4 to bit 2 of each byte), each converted with one
            // byte-to-float instruction; the empty asm keeps the compiler from
            // folding the masks back into one extract per element
            uint32_t sp[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t t = (hb >> j) & 0x1111u;                   // bits 0, 4, 8, 12
                t = (t & 0x0011u) | ((t & 0x1100u) << 8);           // bits 0, 4, 16, 20
                t = (t & 0x00010001u) | ((t & 0x00100010u) << 4);   // bits 0, 8, 16, 24
                sp[j] = ((w >> (2 * j)) & 0x03030303u) | (t << 2);
                asm volatile("" : "+v"(sp[j]));
            }
            if (__all(__builtin_isfinite(dl))) {
#pragma unroll
                for (int l = 0; l < 16; l++) {
                    const float q4 = (float)((sp[l & 3] >> (8 * (l >> 2))) & 0xffu);
                    // dl * (q + 4) is exact (at most 20 significant bits) and so
                    // is dl * q, so one fused multiply-add gives dl * q exactly
                    // (a zero as +0 where dl * q can be -0: the sum starts at +0
                    // and, rounded to nearest, is never -0, so adding either zero
                    // leaves it). An infinite dl would make it inf - inf: waves
                    // holding one take the plain product below.
                    const float wt = __builtin_fmaf(dl, q4, ndl4);
                    sum = sum + elem(x.xf, 16 * h + l) * wt;
                }
            } else {
#pragma unroll
                for (int l = 0; l < 16; l++) {
                    const float q = (float)((sp[l & 3] >> (8 * (l >> 2))) & 0xffu) - 4.0f;
                    const float wt = dl * q;
                    sum = sum + elem(x.xf, 16 * h + l) * wt;
                }
            }
        }
        acc = acc + sum;
    } else if (FMT == SLLM_Q4K_STREAM) {
        // convertQ4KToQ41 (kquant_kernels.go:30-63) for this block: scale / min
        // pair jj of getScaleMinK4 (kquants.go:62-71), d' = float64ToFloat16(d *
        // sc), m' = float64ToFloat16(-dmin * m) - both products exact in float32,
        // so the truncating encode sees the fp64 value - then the Q4_1 term.
        const uint32_t jj = b.jj, k8 = 8 * (jj & 3u);
        const uint32_t A = ((uint32_t)b.hq.y >> k8) & 0xffu;  // scale byte jj & 3
        const uint32_t B = ((uint32_t)b.hq.z >> k8) & 0xffu;  // byte (jj & 3) + 4
        const uint32_t C = ((uint32_t)b.hq.w >> k8) & 0xffu;  // byte (jj & 3) + 8
        const bool lo = jj < 4;
        const uint32_t sc = lo ? (A & 63u) : ((C & 15u) | ((A >> 6) << 4));
        const uint32_t mn = lo ? (B & 63u) : ((C >> 4) | ((B >> 6) << 4));
        const float d = f16_exact((uint16_t)((uint32_t)b.hq.x & 0xffffu));
        const float dmin = f16_exact((uint16_t)((uint32_t)b.hq.x >> 16));
        const float dq = f16_trunc_value(d * (float)sc);
        const float mq = f16_trunc_value(-dmin * (float)mn);
        // q41q8_row_amd64.s:65-71: ((float(qsum)*d) + (float(Σxq)*m)) * xs
        const float fsx = (float)x.sx;
        const int qsum = nib_isum(b.q, x.xl, x.xh);
        const float t1 = (float)qsum * dq;
        const float t2 = fsx * mq;
        float t = t1 + t2;
        t = t * x.xs;
        acc = acc + t;
    } else if (FMT == SLLM_Q5_0) {
        const float sum = q5_block_sum_tab(b.q, b.qh, x.xf, q5tab);
        const float grp = f16_lut(b.d) * sum;  // float32_ops.go:366 `s * sum`
        acc = acc + grp;
    } else if (FMT == SLLM_Q8_0) {
        // q8q8.go:187-195 + vnni_amd64.s:70-73: cmb = ws*xs, term = float(isum)*cmb
        const int isum = q8_isum(b.q, b.q2, x.xl, x.xh);
        const float cmb = f16_lut(b.d) * x.xs;
        const float term = cmb * (float)isum;
        acc = acc + term;
    } else if (FMT == SLLM_Q4_0) {
        // q4q8.go:37-43: ws*xs*float(Σ(nib-8)·xq); Σ(nib-8)xq = Σnib·xq - 8Σxq exactly
        const int isum = nib_isum(b.q, x.xl, x.xh) - 8 * x.sx;
        const float cmb = f16_exact(b.d) * x.xs;
        const float term = cmb * (float)isum;
        acc = acc + term;
    } else {
        // q41q8_row_amd64.s:65-71: ((float(qsum)*d) + (float(Σxq)*m)) * xs
        const float fsx = (float)x.sx;
        const int qsum = nib_isum(b.q, x.xl, x.xh);
        const float t1 = (float)qsum * f16_exact(b.d);
        const float t2 = fsx * f16_exact(b.m);
        float t = t1 + t2;
        t = t * x.xs;
        acc = acc + t;
        if (FMT == SLLM_Q5K1) {
            // high Q4_1 block of convertQ5KToTwoQ41: scale dh, min +0, 0/1 codes.
            // Its min term float(Σxq) * +0 is a zero, and adding it changes h1
            // only from -0 to +0; acc2 starts at +0 and, rounded to nearest, is
            // never -0, so adding either zero leaves it - the term is left out,
            // as in the GEMM (bit-identical)
            const int hsum = bits_isum(b.qh, x.xl, x.xh);
            float h = (float)hsum * f16_exact(b.dh);
            h = h * x.xs;
            acc2 = acc2 + h;
        }
    }
}


template <int FMT, int NB, int D, int TPB, class Issue>
__device__ __forceinline__ void prologue(BlockRegs (&buf)[D][NB], const float *__restrict__ x, int M, int G,
                                         const ActView &A, Issue &issue) {
    constexpr int NV = 8 / TPB;  // float4 per thread per block
    const int nblk = M * G;
    const int per_pass = blockDim.x / TPB;
    const int blk = threadIdx.x / TPB, sub = threadIdx.x % TPB;
    // One unit goes out with the activation loads, the rest of the ring once
    // this thread's first block is staged: the activations share the HBM
    // queues with every weight load already issued device-wide, so fewer of
    // those ahead of them shorten the prologue (measured: 1-2 % per launch).
    if (blk < nblk) {
        float4 xv[NV];
        const float4 *src = (const float4 *)(x + (size_t)blk * 32) + sub * NV;
#pragma unroll
        for (int k = 0; k < NV; k++) xv[k] = src[k];
        __builtin_amdgcn_sched_barrier(0);
        issue(buf[0]);
        __builtin_amdgcn_sched_barrier(0);
        stage_part<FMT, TPB>(xv, blk, sub, A);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 1; d < D; d++) issue(buf[d]);
    } else {
#pragma unroll
        for (int d = 0; d < D; d++) issue(buf[d]);
    }
    for (int b = blk + per_pass; b < nblk; b += per_pass) {
        float4 v[NV];
        const float4 *src = (const float4 *)(x + (size_t)b * 32) + sub * NV;
#pragma unroll
        for (int k = 0; k < NV; k++) v[k] = src[k];
        stage_part<FMT, TPB>(v, b, sub, A);
    }
}

// rmsNormFlatF32 (float32_ops.go:159-172) statistics of one K-element row,
// called by every thread of a workgroup of >= 256 threads: the sum of squares
// over a fixed partition - slot s (s < 256) adds v*v for v = xr[s], xr[s+256],
// ... in that order, then the 256 slot sums are added by wave_sum within each
// of the first four waves and the four results left to right - so every launch
// shape gives the same value. Then inv = 1 / float32(sqrt(float64(ss) /
// float64(K) + float64(eps))), as the reference computes it. The reference
// adds the squares in one sequential loop; only that association differs.
//
// Split in two so that a caller can issue other loads between them: rms_load
// issues slot t's next RB loads (past the row's end they read as 0, and adding
// 0*0 leaves a non-negative sum unchanged), rms_finish adds them and the rest.
template <int RB>
__device__ __forceinline__ void rms_load(const float *__restrict__ xr, int K, int i, float (&v)[RB]) {
#pragma unroll
    for (int k = 0; k < RB; k++) v[k] = i + k * 256 < K ? xr[i + k * 256] : 0.0f;
}
template <int RB>
__device__ __forceinline__ float rms_finish(const float *__restrict__ xr, int K, float eps, float *red,
                                            float (&v)[RB]) {
    const int t = threadIdx.x;
    float p = 0.0f;
    if (t < 256) {
        for (int i = t;;) {
#pragma unroll
            for (int k = 0; k < RB; k++) p = p + v[k] * v[k];
            i += RB * 256;
            if (i >= K) break;
            rms_load<RB>(xr, K, i, v);
        }
    }
    const float w = wave_sum(p);
    if (t < 256 && (t & 63) == 0) red[t >> 6] = w;
    __syncthreads();
    const float ss = ((red[0] + red[1]) + red[2]) + red[3];
    // float64(ss) / float64(K): for a power-of-two K the quotient is exact, and
    // so is the product with the exact reciprocal, without the division's
    // iterations. red is written once per launch by each caller, so no barrier
    // guards it after these reads.
    const double q = (K & (K - 1)) == 0 ? (double)ss * (1.0 / (double)K) : (double)ss / (double)K;
    const double ms = q + (double)eps;
    return 1.0f / (float)sqrt(ms);
}
template <int RB = 16>
__device__ __forceinline__ float rms_inv(const float *__restrict__ xr, int K, float eps, float *red) {
    float v[RB];
    if (threadIdx.x < 256) rms_load<RB>(xr, K, threadIdx.x, v);
    return rms_finish<RB>(xr, K, eps, red, v);
}

// The prologue with the RMSNorm in front of the quantizer, for one activation
// row: the row's statistics loads go out first, then this thread's first
// block of x and of the norm weight, then the wave's first weight unit; the
// statistics are then reduced, each block of (x * inv) * w quantized into
// LDS, and the rest of the ring issued. (Loads return in order: anything
// issued after weight units would wait for them, and the activation loads
// queue in HBM behind every weight load issued before them device-wide:
// measured, 10 % off the q/k/v launch.)
template <int FMT, int NB, int D, int TPB, class Issue>
__device__ __forceinline__ void prologue_norm(BlockRegs (&buf)[D][NB], const float *__restrict__ x,
                                              const float *__restrict__ nw, float eps, int G, const ActView &A,
                                              Issue &issue) {
    __shared__ float red[4];
    constexpr int NV = 8 / TPB;
    // fewer statistics loads in flight where the weight ring holds many registers
    constexpr int RB = NB * D >= 6 ? 4 : 16;
    // the first block's operands are preloaded where they are few registers
    // and the ring leaves room for them
    constexpr bool PRE = NV <= 2 && NB * D < 6;
    const int K = G * 32;
    float v[RB];
    if (threadIdx.x < 256) rms_load<RB>(x, K, threadIdx.x, v);
    const int sub = threadIdx.x % TPB;
    const int blk0 = threadIdx.x / TPB;
    float4 xa[PRE ? NV : 1], wa[PRE ? NV : 1];
    if (PRE) {
        const int bc = blk0 < G ? blk0 : 0;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            xa[PRE ? k : 0] = ((const float4 *)(x + (size_t)bc * 32) + sub * NV)[k];
            wa[PRE ? k : 0] = ((const float4 *)(nw + (size_t)bc * 32) + sub * NV)[k];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    issue(buf[0]);  // the rest of the ring after the quantization (as in prologue())
    __builtin_amdgcn_sched_barrier(0);
    const float inv = rms_finish<RB>(x, K, eps, red, v);
    const int per_pass = blockDim.x / TPB;
    for (int b = blk0; b < G; b += per_pass) {
        float4 q[NV];
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const float4 a = PRE && b == blk0 ? xa[PRE ? k : 0] : ((const float4 *)(x + (size_t)b * 32) + sub * NV)[k];
            const float4 c = PRE && b == blk0 ? wa[PRE ? k : 0] : ((const float4 *)(nw + (size_t)b * 32) + sub * NV)[k];
            // float32_ops.go:169: out = x * inv * w, left to right
            q[k] = make_float4((a.x * inv) * c.x, (a.y * inv) * c.y, (a.z * inv) * c.z, (a.w * inv) * c.w);
        }
        stage_part<FMT, TPB>(q, b, sub, A);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 1; d < D; d++) issue(buf[d]);
}

// The weights of one launch (same format, same K, same activation rows).
// Segment s owns the waves [wave0[s], wave0[s + 1]) of the grid; wave0[n] is
// the grid's wave count, so the last segment also takes the spare waves.
// Paired launch (gate / up of one FFN): a single segment of row waves; P[1]
// holds the up planes, dst[0] receives SwiGLU(gate, up), dst[1] / dst[2]
// (optional) the gate / up outputs themselves.
// Greedy argmax of a one-row, one-weight launch (argmaxF32, float32_ops.go:
// 812-822): amax_key != null turns it on. key / cnt are per-stream scratch
// that every launch leaves at zero; out receives the index.
struct SegTable {
    Planes P[kMaxSegs];
    float *dst[kMaxSegs];
    int N[kMaxSegs];
    int wave0[kMaxSegs + 1];
    int n;
    const float *norm_w;  // non-null: RMSNorm the activation rows first (weight vector, eps)
    float norm_eps;
    unsigned long long *amax_key;
    unsigned int *amax_cnt;  // [0] workgroups done, [1] row 0 is NaN
    int *amax_out;
    int accum;  // non-zero: dst += result (the residual add after o / down)
};

// Order-preserving key of a non-NaN value and its row: larger values give
// larger keys, and among equal values the lowest row the largest (the first
// maximum wins, as with the reference's strict `>`). -0 and +0 are equal.
__device__ __forceinline__ unsigned long long argmax_key(float v, int row) {
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)~(uint32_t)row;
}

// Argmax over the launch's outputs: each wave takes the largest key of its
// rows (NaN rows never win), the workgroup's waves meet in LDS, one atomic
// max per workgroup; the last workgroup to finish writes the index and
// clears the scratch for the next launch. If row 0 is NaN the answer is 0
// (no value compares greater than the reference's starting NaN).
//
// Ordering without fences: device-scope read-modify-write atomics are
// performed at the device's coherence point (every XCD's workgroups count on
// the one counter), and one that has returned its old value has been
// performed. Thread 0 issues the count only once its max (and NaN flag) have
// returned - the count's operand is passed through an empty asm that takes
// their results as inputs, so the wave waits for them first - and the last
// workgroup reads and clears the scratch with atomic exchanges, which see
// every max that was performed before the counts it observed. A fence here
// would write back and invalidate the XCD's L2 (buffer_wbl2 / buffer_inv):
// measured, several microseconds over a launch's workgroups.
__device__ __forceinline__ void argmax_tail(const SegTable &S, float v, bool mine, int row) {
    __shared__ unsigned long long slot[16];
    __shared__ int nan_row0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    if (threadIdx.x == 0) nan_row0 = 0;
    unsigned long long k = (mine && !__builtin_isnan(v)) ? argmax_key(v, row) : 0ull;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(k, off, 64);
        k = o > k ? o : k;
    }
    __syncthreads();  // nan_row0 cleared before any wave sets it
    if (mine && row == 0 && __builtin_isnan(v)) nan_row0 = 1;
    if (lane == 0) slot[wave] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long best = 0;
        for (int w = 0; w < W; w++) best = slot[w] > best ? slot[w] : best;
        unsigned long long r1 = 0;
        unsigned int r2 = 0;
        if (best) r1 = __hip_atomic_fetch_max(S.amax_key, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (nan_row0) r2 = __hip_atomic_fetch_or(&S.amax_cnt[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        unsigned int one = 1u;
        asm volatile("" : "+v"(one) : "v"(r1), "v"(r2));  // waits for both to return
        if (__hip_atomic_fetch_add(&S.amax_cnt[0], one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            gridDim.x - 1) {
            const unsigned long long fin =
                __hip_atomic_exchange(S.amax_key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned int nan0 =
                __hip_atomic_exchange(&S.amax_cnt[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *S.amax_out = (nan0 || fin == 0) ? 0 : (int)~(uint32_t)fin;
            (void)__hip_atomic_exchange(&S.amax_cnt[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// A wave's work is a stream of units: unit t is K-chunk (t % KCH) of its row
// number (t / KCH), rows being base, base + step, ... of its segment's weight
// (at most RPW of them; consecutive rows for an odd RPW, rows strided by the
// segment's wave count otherwise). A unit is NB blocks per lane. The wave keeps D units in
// flight in a register ring: it computes unit t, then issues the loads of
// unit t + D into the registers it just consumed. PAIR: the first half of a
// workgroup's waves stream gate rows, the second half the same rows of up
// (each wave RPW consecutive rows of one weight, as an unpaired launch
// streams them), and the two sums of a row meet in LDS for the SwiGLU.
// NORM: the activation row (M == 1) is RMSNormed (S.norm_w, S.norm_eps) on the way in.
template <int FMT, int NB, int D, int MT, bool HOIST, bool PAIR, bool NORM>
__global__ void __launch_bounds__(1024) gemv_kernel(SegTable S, const float *__restrict__ x, int G, int M,
                                                    int KCH, int RPW, int tpb) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const ActView A = carve_act(lds, FMT, MT, G);
    const int lane = threadIdx.x & 63;
    const int W = blockDim.x >> 6;
    // this wave's segment (wave-uniform, so the selection stays in scalar registers)
    const int wg = __builtin_amdgcn_readfirstlane(blockIdx.x * W + (threadIdx.x >> 6));
    Planes P = S.P[0];
    float *__restrict__ dst = S.dst[0];
    int N = S.N[0], w0 = 0, w1 = S.wave0[1];
#pragma unroll
    for (int s = 1; s < kMaxSegs; s++) {
        if (s < S.n && wg >= S.wave0[s]) {
            P = S.P[s];
            dst = S.dst[s];
            N = S.N[s];
            w0 = S.wave0[s];
            w1 = S.wave0[s + 1];
        }
    }
    const Planes P2 = S.P[PAIR ? 1 : 0];  // PAIR: the up planes
    const int wv = wg - w0;
    // PAIR: this wave's half of the workgroup (gate or up) and its place in it
    const int H = W >> 1, wi = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool upw = PAIR && wi >= H;
    const int U = RPW * KCH;
    constexpr int CH = 64 * NB;  // blocks per K-chunk

    // Load-stream position (row ordinal lq, chunk lk; lt units issued). Every
    // wave runs U units; one with fewer than RPW rows re-reads its last real
    // unit for the rest (the data is still in flight or in cache, and no two
    // waves pile onto the same lines); those rows' sums land in lanes >=
    // real_rows and are not stored.
    // The wave's rows are base + q step, q < RPW: an odd RPW takes RPW
    // consecutive rows (one contiguous stretch of the planes per wave), an
    // even one the rows wv, wv + TW, ... strided by the segment's wave count.
    // Measured (same box, bit-identical): the fused C3 gate+up (RPW 7) 13.24
    // against 13.55-13.65 µs with strided rows; the RMSNorm + head + argmax
    // (RPW 32) 87.0-87.7 strided against 90.8-91.3 consecutive: with an even
    // RPW the waves' stretches start a power-of-two multiple of the 2 KB plane
    // rows apart, and their concurrent loads share HBM channels.
    // PAIR: rows blockIdx.x * H * RPW + (wi % H) * RPW, ... (RPW consecutive;
    // C3: 7 on 16 waves per CU, as the unpaired gate + up). Against each wave
    // streaming 4 rows' gate and up halves in turn on 14 waves per CU (rows
    // strided): RMSNorm + gate/up + SwiGLU 15.00 -> 14.57 µs, without the
    // norm 14.38 -> 13.87.
    const int TW = w1 - w0;
    const bool consec = PAIR || (RPW & 1) != 0;
    const int base = PAIR ? ((int)blockIdx.x * H + wi % H) * RPW : (consec ? wv * RPW : wv), step = consec ? 1 : TW;
    const int real_rows = base < N ? min((N - 1 - base) / step + 1, RPW) : 0;
    const int U_real = real_rows * KCH;
    int lq = 0, lk = 0, lt = 0;
    const bool lup = upw;  // the units read the up planes
    uint32_t last = (uint32_t)min(base, N - 1) * (uint32_t)G + (uint32_t)lane;
    auto next_base = [&]() -> uint32_t {
        if (lt >= U_real) return last;
        const int row = base + lq * step;
        last = (uint32_t)row * (uint32_t)G + (uint32_t)(lk * CH + lane);
        ++lt;
        if (++lk == KCH) {
            lk = 0;
            ++lq;
        }
        return last;
    };
    auto issue = [&](BlockRegs (&u)[NB]) {
        const uint32_t base = next_base();
        load_unit<FMT, NB>(lup ? P2 : P, u, base);
    };

    // The residual add (o / down): each lane's dst value is loaded before
    // anything else, so the add at the end does not wait a memory round trip
    // (dst is only written there).
    float pre[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) {
        pre[m] = 0.0f;
        if (!PAIR && S.accum && m < M && lane < real_rows) pre[m] = dst[(size_t)m * N + base + lane * step];
    }
    __builtin_amdgcn_sched_barrier(0);

    // Q5_0: the high-bit table of q5_block_sum_tab (16 entries, 16 B apart),
    // written before the prologue's barrier
    __shared__ __attribute__((aligned(16))) unsigned char q5tab_lds[FMT == SLLM_Q5_0 ? 256 : 16];
    const unsigned char *q5tab = q5tab_lds;
    if constexpr (FMT == SLLM_Q5_0) {
        if (threadIdx.x < 16) *(uint32_t *)(q5tab_lds + 16 * threadIdx.x) = q5_hi_mask(threadIdx.x);
    }
    BlockRegs buf[D][NB];
    // Prologue: the activation rows (M x G blocks) are quantized by all
    // threads, TPB lanes per block. Each thread issues its activation loads
    // and its wave's first unit of weights, quantizes (waiting only for its
    // activation loads while that unit is in flight), then issues the rest of
    // the wave's first D units.
    if constexpr (NORM) {
        // 8 or 4 lanes per block (the launch passes tpb >= 4): fewer would hold
        // x, w and the normed values of a whole block per lane beside the ring
        if (tpb == 8) prologue_norm<FMT, NB, D, 8>(buf, x, S.norm_w, S.norm_eps, G, A, issue);
        else prologue_norm<FMT, NB, D, 4>(buf, x, S.norm_w, S.norm_eps, G, A, issue);
    } else {
        switch (tpb) {
        case 8: prologue<FMT, NB, D, 8>(buf, x, M, G, A, issue); break;
        case 4: prologue<FMT, NB, D, 4>(buf, x, M, G, A, issue); break;
        case 2: prologue<FMT, NB, D, 2>(buf, x, M, G, A, issue); break;
        default: prologue<FMT, NB, D, 1>(buf, x, M, G, A, issue); break;
        }
    }
    __syncthreads();

    float acc[MT], acc2[MT], res[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) acc[m] = acc2[m] = res[m] = 0.0f;
    int cq = 0, ck = 0;  // compute-stream position (row ordinal, chunk)

    // HOIST (a row is one K-chunk): every unit uses the same blocks, so the
    // activation operands are read from LDS once, before the loop.
    ActRegs xh[HOIST ? NB : 1][HOIST ? MT : 1];
    if (HOIST) {
#pragma unroll
        for (int i = 0; i < NB; i++)
#pragma unroll
            for (int m = 0; m < MT; m++)
                if (m < M) load_act<FMT>(A, (size_t)m * G + min(lane + 64 * i, G - 1), xh[HOIST ? i : 0][HOIST ? m : 0]);
    }

    // the terms of one block (all MT activation rows)
    auto block_terms = [&](const BlockRegs &b, int g, int i) {
        if constexpr (FMT == SLLM_Q6K_STREAM) {
            // the Q8_0 codes and scale, rebuilt once for every activation row,
            // then the Q8_0 term (q8q8.go:187-195 + vnni_amd64.s:70-73)
            int4 wl, wh;
            float sv;
            q6s::requant(b.q, b.c2, b.qh, b.d, wl, wh, sv);
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m >= M) continue;
                ActRegs xa;
                if (HOIST) xa = xh[HOIST ? i : 0][HOIST ? m : 0];
                else load_act<FMT>(A, (size_t)m * G + g, xa);
                const int isum = q8_isum(wl, wh, xa.xl, xa.xh);
                const float cmb = sv * xa.xs;
                const float term = cmb * (float)isum;
                acc[m] = acc[m] + term;
            }
            return;
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
            if (m >= M) continue;
            if (HOIST) {
                block_term<FMT>(b, xh[HOIST ? i : 0][HOIST ? m : 0], acc[m], acc2[m], q5tab);
            } else {
                ActRegs xa;
                load_act<FMT>(A, (size_t)m * G + g, xa);
                block_term<FMT>(b, xa, acc[m], acc2[m], q5tab);
            }
        }
    };
    // consume one unit from ring slot d; only a row's last, partial chunk
    // needs the per-lane block guard (the branch on ck is wave-uniform)
    auto compute = [&](BlockRegs (&u)[NB]) {
        if ((ck + 1) * CH <= G) {
#pragma unroll
            for (int i = 0; i < NB; i++) block_terms(u[i], ck * CH + lane + 64 * i, i);
        } else {
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const int g = ck * CH + lane + 64 * i;
                if (g < G) block_terms(u[i], g, i);
            }
        }
        if (++ck == KCH) {
            // row done: reduce across the wave (fixed order), park it in lane cq
#pragma unroll
            for (int m = 0; m < MT; m++) {
                float v = wave_sum(acc[m]);
                if (FMT == SLLM_Q5K1) v = v + wave_sum(acc2[m]);
                res[m] = (lane == cq) ? v : res[m];
                acc[m] = acc2[m] = 0.0f;
            }
            ck = 0;
            ++cq;
        }
    };

    // Steady state: consume unit t, then issue unit t + D into the slot it
    // freed. These loads are unconditional, so the compiler waits exactly for
    // the unit being consumed. The last ring refills only the units that are
    // left (rem < D of them); D <= U, so the prologue's D units all exist.
    int t0 = 0;
    for (; t0 + 2 * D <= U; t0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            compute(buf[d]);
            issue(buf[d]);
        }
    }
    const int rem = U - t0 - D;
#pragma unroll
    for (int d = 0; d < D; d++) {
        compute(buf[d]);
        if (d < rem) issue(buf[d]);
    }
#pragma unroll
    for (int d = 0; d < D; d++)
        if (d < rem) compute(buf[d]);

    const int row = base + lane * step;  // lane q holds the sum of row ordinal q
    if constexpr (PAIR) {
        // the up waves hand their sums to the gate waves of the same rows; the
        // gate waves form the gate part of the SwiGLU while they wait
        __shared__ float ups[8][64][4];  // [gate wave][row ordinal][activation row]
        float t[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) t[m] = 0.0f;
        if (upw && lane < real_rows) {
#pragma unroll
            for (int m = 0; m < MT; m++) ups[wi - H][lane][m] = res[m];
        } else if (!upw && lane < real_rows) {
#pragma unroll
            for (int m = 0; m < MT; m++)
                if (m < M) t[m] = swiglu_gate(res[m]);
        }
        __syncthreads();
        if (lane < real_rows) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m >= M) continue;
                const size_t o = (size_t)m * N + row;
                if (!upw) {
                    dst[o] = t[m] * ups[wi][lane][m];  // swiglu(gate, up)
                    if (S.dst[1]) S.dst[1][o] = res[m];
                } else if (S.dst[2]) {
                    S.dst[2][o] = res[m];
                }
            }
        }
        return;
    }
    if (lane < real_rows) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            if (m >= M) continue;
            const size_t o = (size_t)m * N + row;
            if (dst) {
                // model_f32.go:472-474 / 495-497: x[i] += o[i], one float32 add
                dst[o] = S.accum ? pre[m] + res[m] : res[m];
            }
        }
    }
    if (!PAIR && S.amax_key) argmax_tail(S, res[0], lane < real_rows, row);
}

template <int FMT, int NB, int D, int MT, bool PAIR>
sllm_status launch_t(const SegTable &S, const float *x, int G, int M, int KCH, int RPW, int W, int grid,
                     size_t lds, hipStream_t s) {
    // hoisting needs room for the operands: fp32-activation formats hold 32
    // floats per block
    constexpr bool kCanHoist = act_f32(FMT) ? ((kq_native(FMT) || FMT == SLLM_Q5_0) && NB * MT <= 2 &&
                                               NB * D <= (FMT == SLLM_Q5_0 ? 4 : 2))
                                            : NB * MT <= 4;
    // lanes per activation block in the prologue: 8 where the workgroup allows,
    // 4 with the RMSNorm in front and where a wave streams at most two units
    // (the waves left without an activation block issue their whole ring at
    // once). Measured (one row, K = 4096; same box, back-to-back launches):
    // o 5.23 -> 5.03 µs, RMSNorm + head + argmax 87.5 -> 87.0, C1 / C2 shapes
    // 5-15 % faster; 4 lanes for the fused gate + up (7 units per wave) cost it
    // 0.1 µs
    int tpb = (S.norm_w || RPW * KCH <= 2) ? 4 : 8;
    while (tpb > (S.norm_w ? 4 : 1) && (int64_t)M * G * tpb > W * 64) tpb >>= 1;
    const bool hoist = kCanHoist && KCH == 1;
    if (S.norm_w) {
        // the fused RMSNorm prologue exists for one-row tiles (decode)
        if constexpr (MT == 1) {
            if (hoist)
                hipLaunchKernelGGL((gemv_kernel<FMT, NB, D, MT, kCanHoist, PAIR, true>), dim3(grid), dim3(W * 64), lds,
                                   s, S, x, G, M, KCH, RPW, tpb);
            else
                hipLaunchKernelGGL((gemv_kernel<FMT, NB, D, MT, false, PAIR, true>), dim3(grid), dim3(W * 64), lds, s,
                                   S, x, G, M, KCH, RPW, tpb);
        } else {
            return set_error(SLLM_ERR_SHAPE, "gemv: the fused RMSNorm takes one activation row");
        }
    } else if (hoist) {
        hipLaunchKernelGGL((gemv_kernel<FMT, NB, D, MT, kCanHoist, PAIR, false>), dim3(grid), dim3(W * 64), lds, s, S,
                           x, G, M, KCH, RPW, tpb);
    } else {
        hipLaunchKernelGGL((gemv_kernel<FMT, NB, D, MT, false, PAIR, false>), dim3(grid), dim3(W * 64), lds, s, S, x,
                           G, M, KCH, RPW, tpb);
    }
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

// D units in flight; NB * D * MT <= 8 blocks per lane.
template <int FMT, int NB, int MT, bool PAIR>
sllm_status launch_d(int D, const SegTable &S, const float *x, int G, int M, int KCH, int RPW, int W, int grid,
                     size_t lds, hipStream_t s) {
    constexpr int DMAX = 8 / (NB * MT) >= 8 ? 8 : (8 / (NB * MT) >= 4 ? 4 : (8 / (NB * MT) >= 2 ? 2 : 1));
    if (D >= 8 && DMAX >= 8) return launch_t<FMT, NB, (DMAX >= 8 ? 8 : 1), MT, PAIR>(S, x, G, M, KCH, RPW, W, grid, lds, s);
    if (D >= 4 && DMAX >= 4) return launch_t<FMT, NB, (DMAX >= 4 ? 4 : 1), MT, PAIR>(S, x, G, M, KCH, RPW, W, grid, lds, s);
    if (D >= 2 && DMAX >= 2) return launch_t<FMT, NB, (DMAX >= 2 ? 2 : 1), MT, PAIR>(S, x, G, M, KCH, RPW, W, grid, lds, s);
    return launch_t<FMT, NB, 1, MT, PAIR>(S, x, G, M, KCH, RPW, W, grid, lds, s);
}

template <int FMT, int MT, bool PAIR>
sllm_status launch_nb(int NB, int D, const SegTable &S, const float *x, int G, int M, int KCH, int RPW, int W,
                      int grid, size_t lds, hipStream_t s) {
    switch (NB) {
    case 1: return launch_d<FMT, 1, MT, PAIR>(D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 2: return launch_d<FMT, 2, MT, PAIR>(D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 3: return launch_d<FMT, 3, MT, PAIR>(D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 4: return launch_d<FMT, 4, MT, PAIR>(D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 5: return launch_d<FMT, 5, MT, PAIR>(D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 6: return launch_d<FMT, 6, MT, PAIR>(D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 7: return launch_d<FMT, 7, MT, PAIR>(D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 8: return launch_d<FMT, 8, MT, PAIR>(D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    }
    return set_error(SLLM_ERR_SHAPE, "gemv: unsupported blocks-per-lane");
}

template <int FMT, bool PAIR>
sllm_status launch_mt(int MT, int NB, int D, const SegTable &S, const float *x, int G, int M, int KCH, int RPW,
                      int W, int grid, size_t lds, hipStream_t s) {
    switch (MT) {
    case 1: return launch_nb<FMT, 1, PAIR>(NB, D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 2: return launch_nb<FMT, 2, PAIR>(NB, D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    case 4: return launch_nb<FMT, 4, PAIR>(NB, D, S, x, G, M, KCH, RPW, W, grid, lds, s);
    }
    return set_error(SLLM_ERR_SHAPE, "gemv: unsupported row tile");
}

}  // namespace gemv
}  // namespace sllm
