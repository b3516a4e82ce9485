// Device-side building blocks shared by the GEMV, GEMM and verification kernels:
// f16 codecs, the bit-exact Q8_0 activation quantizer and the per-block integer
// dots of each weight format. Compiled with -ffp-contract=off: every float
// expression below rounds each operation separately, in the order written,
// which is the order the reference evaluates it in.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sllm {

// ------------------------------------------------------------------ f16 ----

// Exact IEEE half -> float (v_cvt_f32_f16; f16 denormals are kept). This is the
// decode the reference's fused Q4_0 / Q4_1 kernels perform with VCVTPH2PS
// (q4q8_row_amd64.s:36-38, q41q8_row_amd64.s:58-63).
__device__ __forceinline__ float f16_exact(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// The reference's table decode f16ToF32 / f16LUT (dot_scalar.go:46-64,
// q8q8.go:60-62), used for Q8_0 and Q5_0 scales: identical to the exact decode
// except that every f16 subnormal becomes a signed zero (the Go code divides a
// float32 denormal by 2^24, which underflows).
__device__ __forceinline__ float f16_lut(uint16_t h) {
    float f = f16_exact(h);
    return (h & 0x7c00u) ? f : __builtin_copysignf(0.0f, f);
}

// float64ToFloat16 (quantize.go:133-159): NaN/Inf -> 0, mantissa truncated,
// values below the f16 normal range flush to a signed zero.
__device__ __forceinline__ uint16_t f64_to_f16_trunc(double f) {
    uint64_t bits = __builtin_bit_cast(uint64_t, f);
    uint64_t exp64 = (bits >> 52) & 0x7ffu;
    if (exp64 == 0x7ffu) return 0;  // NaN or Inf
    uint16_t sign = (uint16_t)((bits >> 48) & 0x8000u);
    if (exp64 == 0) return sign;
    int exp16 = (int)exp64 - 1023 + 15;
    if (exp16 <= 0) return sign;
    if (exp16 >= 0x1f) return sign | 0x7c00u;
    return sign | (uint16_t)(exp16 << 10) | (uint16_t)((bits >> 42) & 0x3ffu);
}

// float64ToFloat16 of a value that float32 holds exactly (so its top mantissa
// bits and exponent are the fp64 value's): the same truncating encode.
__device__ __forceinline__ uint16_t f32_to_f16_trunc(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = (int)((u >> 23) & 0xffu);
    if (e == 0xff) return 0;  // NaN or Inf
    const int e16 = e - 127 + 15;
    if (e == 0 || e16 <= 0) return (uint16_t)sign;
    if (e16 >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | ((u >> 13) & 0x3ffu));
}

// Go's byte(int8(f64)) on amd64 (CVTTSD2SL, low byte): NaN -> 0.
__device__ __forceinline__ uint32_t f64_to_i8_byte(double v) {
    if (!(v >= -2147483648.0 && v < 2147483648.0)) return 0;
    return (uint32_t)(int8_t)(int32_t)v & 0xffu;
}

// f16_exact(f32_to_f16_trunc(f)) without the round trip: the f16 normal range
// keeps the top 10 mantissa bits, below it a signed zero, above it a signed
// Inf, NaN / Inf give +0.
__device__ __forceinline__ float f16_trunc_value(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    const uint32_t e = (u >> 23) & 0xffu;
    const uint32_t sign = u & 0x80000000u;
    uint32_t r = (e >= 113u && e <= 142u) ? (u & 0xffffe000u) : (e > 142u ? (sign | 0x7f800000u) : sign);
    r = e == 0xffu ? 0u : r;
    return __builtin_bit_cast(float, r);
}

// ------------------------------------------------- activation quantizer ----

// Combine a value across the TPB consecutive, aligned lanes that share a block
// (TPB = 1, 2, 4 or 8) with DPP moves; every lane of the group receives it.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
template <int TPB>
__device__ __forceinline__ float group_max(float a) {
    // max of non-NaN magnitudes (a is never NaN here): order-independent
    float o;
    if (TPB >= 2) { o = __builtin_bit_cast(float, dpp_mov<0xb1>(__builtin_bit_cast(int, a))); a = o > a ? o : a; }
    if (TPB >= 4) { o = __builtin_bit_cast(float, dpp_mov<0x4e>(__builtin_bit_cast(int, a))); a = o > a ? o : a; }
    if (TPB >= 8) { o = __builtin_bit_cast(float, dpp_mov<0x141>(__builtin_bit_cast(int, a))); a = o > a ? o : a; }
    return a;
}
template <int TPB>
__device__ __forceinline__ int group_sum(int v) {
    if (TPB >= 2) v += dpp_mov<0xb1>(v);   // lane ^ 1
    if (TPB >= 4) v += dpp_mov<0x4e>(v);   // lane ^ 2
    if (TPB >= 8) v += dpp_mov<0x141>(v);  // other quad of the 8
    return v;
}

// quantizeActivationsQ8 (q8q8.go:96-125) for one 32-element block spread over
// TPB lanes, each holding 8/TPB float4 (elements 32/TPB * sub ...). Every lane
// returns its 8/TPB packed code words; scale and Σq are the block's. maxAbs
// over |x| (NaN never wins the `>` compare), scale = maxAbs/127 and inv =
// 1/scale in IEEE fp32 (0 for an all-zero block), q = clamp(int32(x*inv)).
// The maximum and the integer sum do not depend on how the lanes combine.
//
// Per element the reference computes Go's int32(float32) on amd64
// (CVTTSS2SL: truncation toward zero; NaN, +-Inf and values outside int32
// become INT32_MIN) and clamps that to [-128, 127]. Here the product is
// clamped in float first (fmaxf returns -128 for a NaN product, and
// trunc(clamp(t)) == clamp(trunc(t)) for every finite or infinite t), then
// truncated. The one case where the two differ is a +Inf product, which Go
// sends to INT32_MIN and so to -128: x * inv is +Inf only when inv itself is
// +Inf (the block's scale underflowed to 0 or below 1/FLT_MAX), and then every
// product of the block is +-Inf or NaN, so the whole block codes to -128.
__device__ __forceinline__ int quant_clamped(float p) {
    const float t = __builtin_fminf(__builtin_fmaxf(p, -128.0f), 127.0f);
    return (int)t;
}
// Low bytes of four ints packed into one word (element 0 in byte 0).
__device__ __forceinline__ int pack4(int q0, int q1, int q2, int q3) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q1, (uint32_t)q0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q3, (uint32_t)q2, 0x0c0c0400u);
    return (int)__builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

template <int TPB>
__device__ __forceinline__ void quantize_part(const float4 *v, int *w, float &scale, int &sum) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 8 / TPB; k++) {
        float t;
        t = __builtin_fabsf(v[k].x); a = t > a ? t : a;
        t = __builtin_fabsf(v[k].y); a = t > a ? t : a;
        t = __builtin_fabsf(v[k].z); a = t > a ? t : a;
        t = __builtin_fabsf(v[k].w); a = t > a ? t : a;
    }
    a = group_max<TPB>(a);
    float s = 0.0f, inv = 0.0f;
    if (a > 0.0f) {
        s = a / 127.0f;
        inv = 1.0f / s;
    }
    const bool inf_inv = inv == __builtin_inff();
    int sm = 0;
#pragma unroll
    for (int k = 0; k < 8 / TPB; k++) {
        w[k] = pack4(quant_clamped(v[k].x * inv), quant_clamped(v[k].y * inv), quant_clamped(v[k].z * inv),
                     quant_clamped(v[k].w * inv));
        w[k] = inf_inv ? (int)0x80808080u : w[k];
        sm = __builtin_amdgcn_sdot4(w[k], 0x01010101, sm, false);
    }
    scale = s;
    sum = group_sum<TPB>(sm);
}

// ------------------------------------------------------------- SwiGLU ----

// forwardBlock's FFN activation (model_f32.go:486-489), in its operation order:
// s = float32(1.0 / (1.0 + exp(-float64(gate)))) in fp64, then (gate * s) * up
// in fp32. exp is the device's fp64 exp (faithfully rounded), where the
// reference calls Go's math.Exp.
// swiglu_gate is the part that depends on gate alone: swiglu(g, u) is
// swiglu_gate(g) * u, operation for operation.
__device__ __forceinline__ float swiglu_gate(float gate) {
    const double e = exp(-(double)gate);
    const float s = (float)(1.0 / (1.0 + e));
    return gate * s;
}
__device__ __forceinline__ float swiglu(float gate, float up) {
    const float t = swiglu_gate(gate);
    return t * up;
}

// ---------------------------------------------------------- block dots ----

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Σ w·xq over a Q8_0 block: w halves (elements 0..15, 16..31), xq halves likewise.
__device__ __forceinline__ int q8_isum(int4 wl, int4 wh, int4 xl, int4 xh) {
    int s = dot4(wl.x, xl.x, 0);
    s = dot4(wl.y, xl.y, s);
    s = dot4(wl.z, xl.z, s);
    s = dot4(wl.w, xl.w, s);
    s = dot4(wh.x, xh.x, s);
    s = dot4(wh.y, xh.y, s);
    s = dot4(wh.z, xh.z, s);
    s = dot4(wh.w, xh.w, s);
    return s;
}

// Σ nib·xq over a 4-bit block (16 GGUF nibble bytes: low nibbles are elements
// 0..15, high nibbles 16..31).
__device__ __forceinline__ int nib_isum(int4 q, int4 xl, int4 xh) {
    const int lo = 0x0f0f0f0f;
    int s = dot4(q.x & lo, xl.x, 0);
    s = dot4(q.y & lo, xl.y, s);
    s = dot4(q.z & lo, xl.z, s);
    s = dot4(q.w & lo, xl.w, s);
    s = dot4((q.x >> 4) & lo, xh.x, s);
    s = dot4((q.y >> 4) & lo, xh.y, s);
    s = dot4((q.z >> 4) & lo, xh.z, s);
    s = dot4((q.w >> 4) & lo, xh.w, s);
    return s;
}

// Four bits (b0..b3 of t) -> four bytes holding 0 or 1.
__device__ __forceinline__ int spread4(uint32_t t) { return (int)(((t & 0xfu) * 0x00204081u) & 0x01010101u); }

// The Q5K1 high-bit word is kept in group order: bit 8 i + k holds the high
// bit of element 4 k + i (i < 4, k < 8), so (w >> k) & 0x01010101 spreads the
// four elements of group k to bytes with one shift and one mask.
__host__ __device__ inline uint32_t q5k1_bits_to_groups(uint32_t bits) {
    uint32_t g = 0;
    for (int k = 0; k < 8; k++)
        for (int i = 0; i < 4; i++) g |= ((bits >> (4 * k + i)) & 1u) << (8 * i + k);
    return g;
}
__host__ __device__ inline uint32_t q5k1_groups_to_bits(uint32_t g) {
    uint32_t bits = 0;
    for (int k = 0; k < 8; k++)
        for (int i = 0; i < 4; i++) bits |= ((g >> (8 * i + k)) & 1u) << (4 * k + i);
    return bits;
}

// Σ bit_e·xq_e over a block's 32 elements, the high bits in group order: the
// Q5K1 high block.
__device__ __forceinline__ int bits_isum(uint32_t hb, int4 xl, int4 xh) {
    constexpr uint32_t m = 0x01010101u;
    int s = dot4((int)(hb & m), xl.x, 0);
    s = dot4((int)((hb >> 1) & m), xl.y, s);
    s = dot4((int)((hb >> 2) & m), xl.z, s);
    s = dot4((int)((hb >> 3) & m), xl.w, s);
    s = dot4((int)((hb >> 4) & m), xh.x, s);
    s = dot4((int)((hb >> 5) & m), xh.y, s);
    s = dot4((int)((hb >> 6) & m), xh.z, s);
    s = dot4((int)((hb >> 7) & m), xh.w, s);
    return s;
}

// Signed Q5_0 codes q5 - 16 of four elements as bytes: the nibble (low four
// bits of each byte of nib), with 0xf0 above it where the element's high bit
// is clear (bits b0..b3 of clear4), i.e. the nibble - 16. 255 t (t: 0 / 1
// bytes) is formed as (t << 8) - t: a 32-bit multiply runs at a quarter of
// the VALU rate.
__device__ __forceinline__ uint32_t q5_codes(uint32_t nib, uint32_t clear4) {
    const uint32_t t = (uint32_t)spread4(clear4);
    uint32_t t8 = t << 8;
    asm("" : "+v"(t8));
    return (nib & 0x0f0f0f0fu) | ((t8 - t) & 0xf0f0f0f0u);
}

// Q5_0 in-block fp32 partial sum in the reference order (q5DotGroupXF32,
// float32_ops.go:335-367): sum += v0*x[j] + v1*x[j+16] for j = 0..15, with
// v = float(q5) - 16 and q5 = nibble | (bit e of qh) << 4. xb holds the block's
// 32 activations (8 float4).
__device__ __forceinline__ float q5_block_sum(int4 q, uint32_t qh, const float4 *xb) {
    const uint32_t w[4] = {(uint32_t)q.x, (uint32_t)q.y, (uint32_t)q.z, (uint32_t)q.w};
    float sum = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        float4 a = xb[jj];      // elements 4jj .. 4jj+3
        float4 b = xb[jj + 4];  // elements 16+4jj ..
        const float av[4] = {a.x, a.y, a.z, a.w};
        const float bv[4] = {b.x, b.y, b.z, b.w};
        // q5 - 16 of elements 4jj+k (lo) and 16+4jj+k (hi) as signed bytes k:
        // the nibble, with 0xf0 above it where the high bit is clear (the
        // nibble - 16), so each converts with one sign-extending byte-to-float
        // instruction; float(q5 - 16) is float(q5) - 16 exactly (+0 for 16)
        const uint32_t lo = q5_codes(w[jj], ~qh >> (4 * jj));
        const uint32_t hi = q5_codes(w[jj] >> 4, ~qh >> (16 + 4 * jj));
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float v0 = (float)(int)(int8_t)((lo >> (8 * k)) & 0xffu);
            float v1 = (float)(int)(int8_t)((hi >> (8 * k)) & 0xffu);
            float p0 = v0 * av[k];
            float p1 = v1 * bv[k];
            float pair = p0 + p1;
            sum = sum + pair;
        }
    }
    return sum;
}

// The same block sum reassociated for the GEMV: the products of elements j
// and j + 16 go into two fused multiply-add chains (16 steps each, one
// rounding per step) that are added at the end - about 2 VALU operations per
// weight instead of 3, the two chains overlapping. The products v * x are
// the reference's; only the order of the additions and their rounding differ
// (each partial is within a few ulp of the block's sum |v x|). The codes are
// q5_codes', with their high-bit half read from a table in LDS: entry t (16 B
// apart, so the 16 entries sit in distinct banks) holds 0xf0 in byte k where
// bit k of t is clear, and a group's entry is addressed by its four qh bits
// times 16 (about three operations and a read per four codes, where the
// multiply-spread took six: C4 Q5_0 14336x4096 at M = 1 13.4-13.5 -> 12.1-12.2
// us).
__device__ __forceinline__ uint32_t q5_hi_mask(uint32_t t) {
    uint32_t m = 0;
    for (int k = 0; k < 4; k++)
        if (!((t >> k) & 1u)) m |= 0xf0u << (8 * k);
    return m;
}
__device__ __forceinline__ float q5_block_sum_tab(int4 q, uint32_t qh, const float4 *xb, const unsigned char *tab) {
    const uint32_t w[4] = {(uint32_t)q.x, (uint32_t)q.y, (uint32_t)q.z, (uint32_t)q.w};
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        float4 a = xb[jj];
        float4 b = xb[jj + 4];
        const float av[4] = {a.x, a.y, a.z, a.w};
        const float bv[4] = {b.x, b.y, b.z, b.w};
        // byte offsets 16 * (four qh bits) of elements 4jj.. and 16 + 4jj..
        const uint32_t ol = jj == 1 ? (qh & 0xf0u) : (jj == 0 ? (qh << 4) : (qh >> (4 * jj - 4))) & 0xf0u;
        const uint32_t oh = (qh >> (12 + 4 * jj)) & 0xf0u;
        const uint32_t lo = (w[jj] & 0x0f0f0f0fu) | *(const uint32_t *)(tab + ol);
        const uint32_t hi = ((w[jj] >> 4) & 0x0f0f0f0fu) | *(const uint32_t *)(tab + oh);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s0 = __builtin_fmaf((float)(int)(int8_t)((lo >> (8 * k)) & 0xffu), av[k], s0);
            s1 = __builtin_fmaf((float)(int)(int8_t)((hi >> (8 * k)) & 0xffu), bv[k], s1);
        }
    }
    return s0 + s1;
}

// ------------------------------------------------------ wave reduction ----

// Sum over the 64 lanes of a wave with DPP moves (no LDS round trips), in a
// fixed order: pairs, quads, 8-lane and 16-lane rows within each row of 16
// lanes, then the four row sums (lanes 0, 16, 32, 48) added left to right.
// Every lane receives the result.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    const int m = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false);
    return v + __builtin_bit_cast(float, m);
}
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0xb1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    v = dpp_add<0x4e>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    v = dpp_add<0x141>(v);  // row_half_mirror: the other quad of each 8 lanes
    v = dpp_add<0x140>(v);  // row_mirror: the other 8 lanes of each row of 16
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return ((r0 + r1) + r2) + r3;
}

// Padded LDS stride (floats) of one 32-element fp32 activation block, chosen so
// that 16 lanes reading 16 B from consecutive blocks hit distinct banks.
constexpr int kXfStride = 36;

}  // namespace sllm
