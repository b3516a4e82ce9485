// Q6_K weights streamed natively (layout SLLM_Q6K_STREAM, opt-in): the Q8_0
// codes the reference computes at load are rebuilt in registers from the
// 6-bit codes.
//
// The reference re-quantizes Q6_K to Q8_0 at load: dequantizeQ6KBlock
// (gguf.go:988-1015) gives v = d * sc * q in fp64 (q = 6-bit code - 32, sc the
// sub-block's int8 scale), then quantizeQ8Rows (gguf.go:1098-1125) codes each
// 32-element block with scale = maxAbs / 127, inv = 1 / scale, code =
// round(clamp(v * inv)) (half away from zero) and stores
// float64ToFloat16(scale).
//
// Every product d * sc * q is exact in fp64, so maxAbs = |d| Mi with Mi =
// max |sc q| over the block (an integer <= 4096) and the exact value of v *
// inv is 127 sc q sgn(d) / Mi up to the relative rounding errors of scale and
// inv (< 2^-52). Wherever that quotient is not a half-integer it lies at least
// 1 / (2 Mi) >= 2^-13 from one, so any computation within 2^-14 of it rounds
// the same way. Where it is exactly k + 1/2 (an element whose |sc q| is an odd
// multiple of Mi / 254, e.g. half the block maximum) the reference's fp64
// product lands just above or just below the half, and which depends on the
// block's scale and inv. The load-time pack records that direction per
// 16-element sub-block (dec bit), and the kernel computes
//   x = q R, R = 127 (1 +- 2^-21) sc sgn(d) / Mi  (fp32; + for ties away from 0)
//   code = the integer nearest to x
// The nudge (8 * 2^-24 relative) exceeds the fp32 rounding errors of R and x
// (at most 5 * 2^-24: the reciprocal's ulp and three roundings) and, on values
// of at most 127, stays below the 2^-13 by which every other quotient misses a
// half; the pack checks every block regardless. The scale: |d| Mi is exact
// in fp32, and float64ToFloat16's truncation of maxAbs / 127 equals the
// truncation of the correctly rounded fp32 quotient (no f16 value lies within
// half an fp32 ulp of |d| Mi / 127 unless the quotient is that value).
//
// A sub-block whose ties go both ways (about one block in 10^4 on random
// data) has no such R. The pack computes every block both ways - the
// reference's fp64 arithmetic and this rule - and marks each block where they
// differ (X bit); the kernel recomputes marked blocks with the reference's
// fp64 arithmetic (codes_exact), in a branch that only waves holding one take.
//
// Planes, per 32-element block (elements e = 0..31 of the Q8_0 block):
//   l6  int4   byte i of word j: low nibble of e = 4j + i | that of 16 + 4j + i << 4
//   h6  uint2  byte i of word h: bits 2j, 2j + 1 = the top two bits of e = 16h + 4j + i
//   m6  u32    sc0 (int8) | sc1 << 8 | Mi << 16 (13 bits) | dec0 << 29 | dec1 << 30 | X << 31
//              (Mi stored as 0 where d is zero or not finite: every code is then 0)
//   d6  u16    per super-block: the GGUF d (f16 bits)
// 28.25 B per 32 weights, against the Q8_0 planes' 34.
#pragma once

#include <hip/hip_runtime.h>

#include "qmm_device.hpp"

namespace sllm {
namespace q6s {

constexpr float kTieUp = 127.0f + 0x1p-14f;    // 127 (1 + 2^-21.0)
constexpr float kTieDown = 127.0f - 0x1p-14f;  // 127 (1 - 2^-21.0)

// The block's 32 codes u = q + 32 (0..63) as bytes: word j < 4 holds elements
// 4j .. 4j + 3, word 4 + j elements 16 + 4j ..
__device__ __forceinline__ void unpack(int4 l6, uint2 h6, uint32_t (&u)[8]) {
    const uint32_t L[4] = {(uint32_t)l6.x, (uint32_t)l6.y, (uint32_t)l6.z, (uint32_t)l6.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        // the top two bits of byte i's elements sit at bits 2j, 2j + 1: move them to bits 4, 5
        const uint32_t a = j < 2 ? h6.x << (4 - 2 * j) : h6.x >> (2 * j - 4);
        const uint32_t b = j < 2 ? h6.y << (4 - 2 * j) : h6.y >> (2 * j - 4);
        u[j] = (L[j] & 0x0f0f0f0fu) | (a & 0x30303030u);
        u[4 + j] = ((L[j] >> 4) & 0x0f0f0f0fu) | (b & 0x30303030u);
    }
}

// The nearest integer to x = u * r + b as the low byte of the result (x is
// never within the rounding margin of a half, so the tie rule of the rounding
// does not matter): adding 1.5 * 2^23 rounds |x| < 2^22 to an integer in the
// low mantissa bits, two's complement in the low byte - one add, where a
// float-to-int conversion issues at half the rate on this part.
__device__ __forceinline__ int code_of(float uf, float r, float b) {
    const float x = __builtin_fmaf(uf, r, b);
    return __builtin_bit_cast(int, x + 12582912.0f);
}
__device__ __forceinline__ int codes4(uint32_t w, float r, float b) {
    return pack4(code_of((float)(w & 0xffu), r, b), code_of((float)((w >> 8) & 0xffu), r, b),
                 code_of((float)((w >> 16) & 0xffu), r, b), code_of((float)(w >> 24), r, b));
}

// The Q8_0 codes by the per-sub-block rule (lo: elements 0..15, hi: 16..31,
// as the Q8_0 planes hold them).
__device__ __forceinline__ void codes_fast(const uint32_t (&u)[8], uint32_t m6, uint16_t d6, int4 &lo, int4 &hi) {
    const uint32_t mi = (m6 >> 16) & 0x1fffu;
    const float rc = mi ? __builtin_amdgcn_rcpf((float)mi) : 0.0f;
    const float sg = (d6 & 0x8000u) ? -rc : rc;
    const float r0 = (((m6 >> 29) & 1u) ? kTieDown : kTieUp) * (float)(int)(int8_t)(m6 & 0xffu) * sg;
    const float r1 = (((m6 >> 30) & 1u) ? kTieDown : kTieUp) * (float)(int)(int8_t)((m6 >> 8) & 0xffu) * sg;
    const float b0 = -32.0f * r0, b1 = -32.0f * r1;  // x = (u - 32) r, one rounding
    lo = make_int4(codes4(u[0], r0, b0), codes4(u[1], r0, b0), codes4(u[2], r0, b0), codes4(u[3], r0, b0));
    hi = make_int4(codes4(u[4], r1, b1), codes4(u[5], r1, b1), codes4(u[6], r1, b1), codes4(u[7], r1, b1));
}

// f16LUT(float64ToFloat16(|d| Mi / 127)): the block's Q8_0 scale as the Q8_0
// term reads it.
__device__ __forceinline__ float scale_fast(uint32_t m6, uint16_t d6) {
    const float y = __builtin_fabsf(f16_exact(d6)) * (float)((m6 >> 16) & 0x1fffu);
    return f16_trunc_value(y / 127.0f);
}

// Word j (0..7, known at run time) of unpack(l6, h6).
__device__ __forceinline__ uint32_t word_of(int4 l6, uint2 h6, int j) {
    const int jj = j & 3;
    const uint32_t L = jj == 0 ? (uint32_t)l6.x : (jj == 1 ? (uint32_t)l6.y : (jj == 2 ? (uint32_t)l6.z : (uint32_t)l6.w));
    const uint32_t H = j < 4 ? h6.x : h6.y;
    return ((j < 4 ? L : L >> 4) & 0x0f0f0f0fu) | (((H >> (2 * jj)) & 0x03030303u) << 4);
}

// The reference's own arithmetic for one block, in fp64 (dequantizeQ6KBlock's
// v = (d * sc) * q, then quantizeQ8Rows: the NaN-skipping maximum, scale,
// inv, v * inv clamped and rounded half away from zero, Go's int8 conversion),
// going over the 32 values twice instead of holding them. Rolled loops: this
// runs for a few blocks in 10^4, and a small body keeps the GEMV's register
// ring unrolled.
__device__ __forceinline__ void codes_exact(int4 l6, uint2 h6, uint32_t m6, uint16_t d6, int4 &lo, int4 &hi,
                                            float &sv) {
    const double d = (double)f16_exact(d6);
    const double ds0 = d * (double)(int)(int8_t)(m6 & 0xffu);
    const double ds1 = d * (double)(int)(int8_t)((m6 >> 8) & 0xffu);
    double maxAbs = 0.0;
#pragma unroll 1
    for (int j = 0; j < 8; j++) {
        const uint32_t w = word_of(l6, h6, j);
        const double ds = j < 4 ? ds0 : ds1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const double v = ds * (double)((int)((w >> (8 * k)) & 0xffu) - 32);
            const double a = __builtin_fabs(v);
            if (a > maxAbs) maxAbs = a;
        }
    }
    double scale = 0.0;
    if (maxAbs > 0) scale = maxAbs / 127.0;
    sv = f16_lut(f64_to_f16_trunc(scale));
    const double inv = 1.0 / scale;
#pragma unroll 1
    for (int j = 0; j < 8; j++) {
        const uint32_t w = word_of(l6, h6, j);
        const double ds = j < 4 ? ds0 : ds1;
        uint32_t c = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const double v = ds * (double)((int)((w >> (8 * k)) & 0xffu) - 32);
            double val = v * inv;
            if (val > 127) val = 127;
            else if (val < -128) val = -128;
            c |= f64_to_i8_byte(round(val)) << (8 * k);
        }
        lo.x = j == 0 ? (int)c : lo.x;
        lo.y = j == 1 ? (int)c : lo.y;
        lo.z = j == 2 ? (int)c : lo.z;
        lo.w = j == 3 ? (int)c : lo.w;
        hi.x = j == 4 ? (int)c : hi.x;
        hi.y = j == 5 ? (int)c : hi.y;
        hi.z = j == 6 ? (int)c : hi.z;
        hi.w = j == 7 ? (int)c : hi.w;
    }
}

// One streamed block's Q8_0 codes and scale value.
__device__ __forceinline__ void requant(int4 l6, uint2 h6, uint32_t m6, uint16_t d6, int4 &lo, int4 &hi,
                                        float &sv) {
    uint32_t u[8];
    unpack(l6, h6, u);
    codes_fast(u, m6, d6, lo, hi);
    sv = scale_fast(m6, d6);
    if (m6 >> 31) codes_exact(l6, h6, m6, d6, lo, hi, sv);
}

}  // namespace q6s
}  // namespace sllm
