// Load-time weight preparation on the GPU: GGUF / QuantWeight block bytes ->
// HBM planes. One thread per output 32-element block. Covers the repack of
// native blocks and the remaps the reference performs in gguf.go:818-934:
//   Q4_K -> Q4_1            (convertQ4KToQ41, kquant_kernels.go:30-63)
//   Q5_K -> two Q4_1 halves (convertQ5KToTwoQ41, kquant_kernels.go:110-154)
//   Q6_K, IQ4_NL -> Q8_0    (fp64 dequant gguf.go:988-1015 / kquants.go:14-27,
//                            then quantizeQ8Rows gguf.go:1080-1134)
//   fp32 -> Q8_0            (quantizeQ8RowsF32, gguf.go:1136-1186)
//   Q2_K, Q3_K kept native  (codes in element order, scale bytes, d / dmin),
//                           where the reference goes to dense fp32 (gguf.go:907-911)
// All arithmetic is the reference's: fp64 products (exact for these inputs),
// IEEE fp64/fp32 division, round-half-away-from-zero, truncating f16 encode.
#include <hip/hip_runtime.h>

#include <cstring>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"
#include "qmm_q6k.hpp"

namespace sllm {

size_t carve_planes(int fmt, int64_t nb, void *base, MutPlanes *out) {
    size_t off = 0;
    auto take = [&](size_t bytes) -> void * {
        off = (off + 255) & ~(size_t)255;
        void *p = base ? (void *)((char *)base + off) : nullptr;
        off += bytes;
        return p;
    };
    // kPlanePadBlocks spare entries per plane: a GEMV lane may read up to one
    // K-chunk past a row's last block (the values are ignored), so the last row
    // of a plane must not run off the allocation.
    const size_t n = (size_t)nb + kPlanePadBlocks;
    MutPlanes p;
    if (kq_native(fmt)) {
        p.q2 = (uint2 *)take(n * 8);
        if (fmt == SLLM_Q3K) p.qh = (uint32_t *)take(n * 4);
        p.d = (uint16_t *)take(n * 2);
        p.sb = (uint32_t *)take(n / 8 * 4);
        if (out) *out = p;
        return (off + 255) & ~(size_t)255;
    }
    p.qs = (int4 *)take(n * 16);
    if (fmt == SLLM_Q8_0 || fmt == SLLM_Q6K_STREAM) p.qs2 = (int4 *)take(n * 16);
    if (fmt == SLLM_Q6K_STREAM) {
        p.d = (uint16_t *)take(n * 2);
        p.l6 = (int4 *)take(n * 16);
        p.h6 = (uint2 *)take(n * 8);
        p.m6 = (uint32_t *)take(n * 4);
        p.d6 = (uint16_t *)take(n / 8 * 2);
        p.q6stat = (uint32_t *)take(2 * sizeof(uint32_t));
        if (out) *out = p;
        return (off + 255) & ~(size_t)255;
    }
    if (fmt == SLLM_Q5_0 || fmt == SLLM_Q5K1) p.qh = (uint32_t *)take(n * 4);
    p.d = (uint16_t *)take(n * 2);
    if (fmt == SLLM_Q4_1 || fmt == SLLM_Q5K1 || fmt == SLLM_Q4K_STREAM) p.m = (uint16_t *)take(n * 2);
    if (fmt == SLLM_Q4K_STREAM) p.hdr = (int4 *)take(n / 8 * 16);
    if (fmt == SLLM_Q5K1) p.dh = (uint16_t *)take(n * 2);
    if (out) *out = p;
    return (off + 255) & ~(size_t)255;
}

namespace {

__device__ __forceinline__ uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
__device__ __forceinline__ int4 ld_int4(const uint8_t *p) {
    int4 v;
    v.x = (int)ld32(p);
    v.y = (int)ld32(p + 4);
    v.z = (int)ld32(p + 8);
    v.w = (int)ld32(p + 12);
    return v;
}
__device__ __forceinline__ double f16_to_f64(uint16_t h) { return (double)f16_exact(h); }

// quantizeQ8Rows (gguf.go:1098-1125) for one block of 32 fp64 values.
__device__ void q8_from_f64(const double *v, int4 &lo, int4 &hi, uint16_t &d) {
    double maxAbs = 0.0;
    for (int i = 0; i < 32; i++) {
        double a = __builtin_fabs(v[i]);
        if (a > maxAbs) maxAbs = a;
    }
    double scale = 0.0;
    if (maxAbs > 0) scale = maxAbs / 127.0;
    d = f64_to_f16_trunc(scale);
    const double inv = 1.0 / scale;
    uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < 32; i++) {
        double val = v[i] * inv;
        if (val > 127) val = 127;
        else if (val < -128) val = -128;
        w[i >> 2] |= f64_to_i8_byte(round(val)) << (8 * (i & 3));
    }
    lo = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
    hi = make_int4((int)w[4], (int)w[5], (int)w[6], (int)w[7]);
}

// getScaleMinK4 (kquants.go:62-71).
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// Sub-block jj of a Q4_K / Q5_K super-block as a Q4_1 block (kquant_kernels.go:41-59).
__device__ __forceinline__ void kquant_low_block(const uint8_t *sb, const uint8_t *qs, int jj, int4 &q,
                                                 uint16_t &d, uint16_t &m, double &dsc) {
    const double dd = f16_to_f64(ld16(sb));
    const double dmin = f16_to_f64(ld16(sb + 2));
    int sc, mm;
    scale_min_k4(jj, sb + 4, sc, mm);
    dsc = dd * (double)sc;
    d = f64_to_f16_trunc(dsc);
    m = f64_to_f16_trunc((-dmin) * (double)mm);
    const int k = (jj / 2) * 32;
    uint32_t w[4] = {0, 0, 0, 0};
    for (int i = 0; i < 16; i++) {
        uint32_t b = (jj & 1) ? (uint32_t)((qs[k + i] >> 4) | ((qs[k + i + 16] >> 4) << 4))
                              : (uint32_t)((qs[k + i] & 0x0f) | ((qs[k + i + 16] & 0x0f) << 4));
        w[i >> 2] |= (b & 0xffu) << (8 * (i & 3));
    }
    q = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
}

// Native QuantWeight.Raw blocks -> planes. For q5k1 the Raw is [low][high];
// the high half must be in the form convertQ5KToTwoQ41 writes (min 0, 0/1
// nibbles), otherwise *err is set.
__global__ void pack_raw_kernel(int fmt, const uint8_t *__restrict__ raw, int64_t nb, MutPlanes P,
                                int *__restrict__ err) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        switch (fmt) {
        case SLLM_Q8_0: {
            const uint8_t *p = raw + b * 34;
            P.d[b] = ld16(p);
            P.qs[b] = ld_int4(p + 2);
            P.qs2[b] = ld_int4(p + 18);
            break;
        }
        case SLLM_Q4_0: {
            const uint8_t *p = raw + b * 18;
            P.d[b] = ld16(p);
            P.qs[b] = ld_int4(p + 2);
            break;
        }
        case SLLM_Q4_1: {
            const uint8_t *p = raw + b * 20;
            P.d[b] = ld16(p);
            P.m[b] = ld16(p + 2);
            P.qs[b] = ld_int4(p + 4);
            break;
        }
        case SLLM_Q5_0: {
            const uint8_t *p = raw + b * 22;
            P.d[b] = ld16(p);
            P.qh[b] = ld32(p + 2);
            P.qs[b] = ld_int4(p + 6);
            break;
        }
        case SLLM_Q5K1: {
            const uint8_t *lo = raw + b * 20;
            const uint8_t *hi = raw + (nb + b) * 20;
            P.d[b] = ld16(lo);
            P.m[b] = ld16(lo + 2);
            P.qs[b] = ld_int4(lo + 4);
            P.dh[b] = ld16(hi);
            uint32_t bits = 0;
            bool bad = ld16(hi + 2) != 0;
            for (int i = 0; i < 16; i++) {
                uint32_t v = hi[4 + i];
                bad |= (v & 0xeeu) != 0;
                bits |= (v & 1u) << i;
                bits |= ((v >> 4) & 1u) << (i + 16);
            }
            P.qh[b] = q5k1_bits_to_groups(bits);
            if (bad) *err = 1;
            break;
        }
        }
    }
}

// Q4_K (144 B / 256) -> Q4_1 planes; block b = (row, super-block, jj).
__global__ void pack_q4k_kernel(const uint8_t *__restrict__ raw, int64_t nb, MutPlanes P) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t *sb = raw + (b >> 3) * 144;
        double dsc;
        kquant_low_block(sb, sb + 16, (int)(b & 7), P.qs[b], P.d[b], P.m[b], dsc);
        if (P.hdr && (b & 7) == 0) P.hdr[b >> 3] = ld_int4(sb);  // d, dmin, scales[12]
    }
}

// Q5_K (176 B / 256) -> Q5K1 planes (low Q4_1 block + high-bit block).
__global__ void pack_q5k_kernel(const uint8_t *__restrict__ raw, int64_t nb, MutPlanes P) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t *sb = raw + (b >> 3) * 176;
        const int jj = (int)(b & 7);
        double dsc;
        kquant_low_block(sb, sb + 48, jj, P.qs[b], P.d[b], P.m[b], dsc);
        P.dh[b] = f64_to_f16_trunc(16 * dsc);
        const uint8_t *qh = sb + 16;
        uint32_t bits = 0;
        for (int i = 0; i < 16; i++) {
            bits |= (uint32_t)((qh[i] >> jj) & 1) << i;
            bits |= (uint32_t)((qh[i + 16] >> jj) & 1) << (i + 16);
        }
        P.qh[b] = q5k1_bits_to_groups(bits);
    }
}

// The GEMM's one-MFMA form of a Q5K1 weight (SLLM_Q5K1F) needs every block's
// high-block scale to equal 16 times its low scale. convertQ5KToTwoQ41 writes
// f16(16 d sc) and f16(d sc) (kquant_kernels.go:127-144): equal to 16 times
// the latter unless 16 d sc overflows f16 (d sc is a multiple of 2^-24, exact
// in f16 below its normal range); a "q5k1" QuantWeight may hold any scales. *bad (cleared by the caller) is
// set when some block differs (a NaN never equals).
__global__ void q5k1_scale_check_kernel(const uint16_t *__restrict__ d, const uint16_t *__restrict__ dh, int64_t nb,
                                        int *bad) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x)
        if (!(f16_exact(dh[b]) == 16.0f * f16_exact(d[b]))) *bad = 1;
}

// Q6_K (210 B / 256) -> Q8_0 planes. Q8 block b of a super-block covers
// elements 32*(b%8) ..: half n = (b%8)/4, quarter k = (b%8)%4 of dequantizeQ6KBlock.
__global__ void pack_q6k_kernel(const uint8_t *__restrict__ raw, int64_t nb, MutPlanes P) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t *sb = raw + (b >> 3) * 210;
        const int j = (int)(b & 7), n = j >> 2, k = j & 3;
        const double d = f16_to_f64(ld16(sb + 208));
        const uint8_t *ql = sb + n * 64 + (k & 1) * 32;
        const uint8_t *qh = sb + 128 + n * 32;
        const uint8_t *sc = sb + 192 + n * 8 + 2 * k;
        double v[32];
        for (int l = 0; l < 32; l++) {
            int nib = (k < 2) ? (ql[l] & 0x0f) : (ql[l] >> 4);
            int q = (int)(int8_t)(nib | (((qh[l] >> (2 * k)) & 3) << 4)) - 32;
            double s = (double)(int8_t)sc[l / 16];
            v[l] = d * s * (double)q;
        }
        int4 lo, hi;
        uint16_t dd;
        q8_from_f64(v, lo, hi, dd);
        P.qs[b] = lo;
        P.qs2[b] = hi;
        P.d[b] = dd;
    }
}

// Q6_K (210 B / 256) -> the Q8_0 planes (as pack_q6k_kernel) and the streamed
// Q6_K planes (qmm_q6k.hpp). Per block: the 6-bit codes, Mi = max |sc q|, and
// per sub-block the direction the reference rounded its ties in - a tie is an
// element with 127 |sc q| / Mi = k + 1/2 exactly, i.e. 254 |sc q| an odd
// multiple of Mi, and it went toward zero when its Q8_0 code is k. Then the
// GEMV's rule is evaluated on the stored planes and compared with the Q8_0
// codes and scale: a block where they differ gets the X bit (the GEMV redoes
// it in fp64) and is counted in q6stat[0]; a block where the GEMV's fp64 path
// differs would be a defect and is counted in q6stat[1] (the load then fails).
__global__ void pack_q6k_stream_kernel(const uint8_t *__restrict__ raw, int64_t nb, MutPlanes P) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t *sb = raw + (b >> 3) * 210;
        const int j = (int)(b & 7), n = j >> 2, k = j & 3;
        const uint16_t dbits = ld16(sb + 208);
        const double d = f16_to_f64(dbits);
        const uint8_t *ql = sb + n * 64 + (k & 1) * 32;
        const uint8_t *qh = sb + 128 + n * 32;
        const uint8_t *sc = sb + 192 + n * 8 + 2 * k;
        const int s[2] = {(int)(int8_t)sc[0], (int)(int8_t)sc[1]};
        int u[32];
        double v[32];
        int mi = 0;
        for (int l = 0; l < 32; l++) {
            const int nib = (k < 2) ? (ql[l] & 0x0f) : (ql[l] >> 4);
            u[l] = nib | (((qh[l] >> (2 * k)) & 3) << 4);
            const int q = u[l] - 32;
            v[l] = d * (double)s[l / 16] * (double)q;
            const int a = s[l / 16] * q < 0 ? -(s[l / 16] * q) : s[l / 16] * q;
            mi = a > mi ? a : mi;
        }
        int4 lo, hi;
        uint16_t dd;
        q8_from_f64(v, lo, hi, dd);
        P.qs[b] = lo;
        P.qs2[b] = hi;
        P.d[b] = dd;

        const uint32_t cw[8] = {(uint32_t)lo.x, (uint32_t)lo.y, (uint32_t)lo.z, (uint32_t)lo.w,
                                (uint32_t)hi.x, (uint32_t)hi.y, (uint32_t)hi.z, (uint32_t)hi.w};
        uint32_t l6[4] = {0, 0, 0, 0}, h6[2] = {0, 0}, dec = 0;
        for (int e = 0; e < 32; e++) {
            const int jw = (e & 15) >> 2, i = e & 3;  // word jw, byte i of its half
            l6[jw] |= (uint32_t)(u[e] & 15) << (8 * i + (e >= 16 ? 4 : 0));
            h6[e >> 4] |= (uint32_t)(u[e] >> 4) << (8 * i + 2 * jw);
            const int sq = s[e / 16] * (u[e] - 32);
            const int a = sq < 0 ? -sq : sq;
            if (mi > 0 && (254 * a) % mi == 0 && ((254 * a / mi) & 1)) {
                const int c = (int)(int8_t)((cw[e >> 2] >> (8 * (e & 3))) & 0xffu);
                if ((c < 0 ? -c : c) == (254 * a / mi - 1) / 2) dec |= 1u << (e / 16);
            }
        }
        const bool finite_nonzero = (dbits & 0x7fffu) != 0 && (dbits & 0x7c00u) != 0x7c00u;
        uint32_t m6 = (uint32_t)(s[0] & 0xff) | ((uint32_t)(s[1] & 0xff) << 8) |
                      ((uint32_t)(finite_nonzero ? mi : 0) << 16) | (dec << 29);
        const int4 l6v = make_int4((int)l6[0], (int)l6[1], (int)l6[2], (int)l6[3]);
        const uint2 h6v = make_uint2(h6[0], h6[1]);
        uint32_t uu[8];
        q6s::unpack(l6v, h6v, uu);
        const float ref_sv = f16_lut(dd);
        int4 flo, fhi;
        q6s::codes_fast(uu, m6, dbits, flo, fhi);
        const float fsv = q6s::scale_fast(m6, dbits);
        const bool fast_ok = flo.x == lo.x && flo.y == lo.y && flo.z == lo.z && flo.w == lo.w && fhi.x == hi.x &&
                             fhi.y == hi.y && fhi.z == hi.z && fhi.w == hi.w &&
                             __float_as_uint(fsv) == __float_as_uint(ref_sv);
        if (!fast_ok) {
            m6 |= 1u << 31;
            atomicAdd(&P.q6stat[0], 1u);
        }
        int4 elo, ehi;
        float esv;
        q6s::codes_exact(l6v, h6v, m6, dbits, elo, ehi, esv);
        const bool exact_ok = elo.x == lo.x && elo.y == lo.y && elo.z == lo.z && elo.w == lo.w && ehi.x == hi.x &&
                              ehi.y == hi.y && ehi.z == hi.z && ehi.w == hi.w &&
                              __float_as_uint(esv) == __float_as_uint(ref_sv);
        if (!exact_ok) atomicAdd(&P.q6stat[1], 1u);
        P.l6[b] = l6v;
        P.h6[b] = h6v;
        P.m6[b] = m6;
        if (j == 0) P.d6[b >> 3] = dbits;
    }
}

// IQ4_NL (18 B / 32) -> Q8_0 planes (kquants.go:7-27 then quantizeQ8Rows).
__constant__ int8_t kIQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

__global__ void pack_iq4nl_kernel(const uint8_t *__restrict__ raw, int64_t nb, MutPlanes P) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t *p = raw + b * 18;
        const double d = f16_to_f64(ld16(p));
        double v[32];
        for (int j = 0; j < 16; j++) {
            v[j] = d * (double)kIQ4NL[p[2 + j] & 0x0f];
            v[j + 16] = d * (double)kIQ4NL[p[2 + j] >> 4];
        }
        int4 lo, hi;
        uint16_t dd;
        q8_from_f64(v, lo, hi, dd);
        P.qs[b] = lo;
        P.qs2[b] = hi;
        P.d[b] = dd;
    }
}

// fp32 rows -> Q8_0 planes (quantizeQ8RowsF32, gguf.go:1143-1176).
__global__ void pack_f32_kernel(const float *__restrict__ w, int64_t nb, MutPlanes P) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const float *v = w + b * 32;
        float maxAbs = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = __builtin_fabsf(v[i]);
            if (a > maxAbs) maxAbs = a;
        }
        float scale = 0.0f;
        if (maxAbs > 0) scale = maxAbs / 127.0f;
        P.d[b] = f64_to_f16_trunc((double)scale);
        const float inv = 1.0f / scale;
        uint32_t q[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int i = 0; i < 32; i++) {
            double val = (double)(v[i] * inv);
            if (val > 127) val = 127;
            else if (val < -128) val = -128;
            q[i >> 2] |= f64_to_i8_byte(round(val)) << (8 * (i & 3));
        }
        P.qs[b] = make_int4((int)q[0], (int)q[1], (int)q[2], (int)q[3]);
        P.qs2[b] = make_int4((int)q[4], (int)q[5], (int)q[6], (int)q[7]);
    }
}

// The 2-bit codes of block bi (0..7) of a Q2_K / Q3_K super-block, from its
// 64 code bytes: sub-block pair bi covers elements 32 bi .. 32 bi + 31, half
// n = bi / 4 of the bytes at bit pair 2 (bi % 4) - the element order of
// dequantizeQ2KNative / dequantizeQ3KNative (kquants.go:147-245).
__device__ __forceinline__ uint2 kq_codes(const uint8_t *qs, int bi) {
    const int n = bi >> 2, sh = 2 * (bi & 3);
    const uint8_t *q = qs + 32 * n;
    uint32_t x = 0, y = 0;
    for (int l = 0; l < 16; l++) {
        x |= (uint32_t)((q[l] >> sh) & 3) << (2 * l);
        y |= (uint32_t)((q[16 + l] >> sh) & 3) << (2 * l);
    }
    return make_uint2(x, y);
}

// Q2_K (84 B / 256: scales[16], qs[64], d, dmin) kept native.
__global__ void pack_q2k_kernel(const uint8_t *__restrict__ raw, int64_t nb, MutPlanes P) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t *sb = raw + (b >> 3) * 84;
        const int bi = (int)(b & 7);
        P.q2[b] = kq_codes(sb + 16, bi);
        P.d[b] = (uint16_t)(sb[2 * bi] | (sb[2 * bi + 1] << 8));
        if (bi == 0) P.sb[b >> 3] = (uint32_t)ld16(sb + 80) | ((uint32_t)ld16(sb + 82) << 16);
    }
}

// The 6-bit scale s (0..15) of a Q3_K super-block from its 12 packed bytes:
// the unpacking of dequantizeQ3KNative (kquants.go:195-210) for one scale.
__host__ __device__ inline int q3k_scale(const uint8_t *scb, int s) {
    const int k = s >> 2, i = s & 3;
    const int hi = (scb[8 + i] >> (2 * k)) & 3;
    const int lo = (k & 1) ? scb[4 + i] : scb[i];
    return ((k < 2) ? (lo & 0x0f) : (lo >> 4)) | (hi << 4);
}

// Q3_K (110 B / 256: hmask[32], qs[64], scales[12], d) kept native.
__global__ void pack_q3k_kernel(const uint8_t *__restrict__ raw, int64_t nb, MutPlanes P) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t *sb = raw + (b >> 3) * 110;
        const int bi = (int)(b & 7);
        P.q2[b] = kq_codes(sb + 32, bi);
        const int bit = 4 * (bi >> 2) + (bi & 3);  // the hmask bit of this block (m in the reference)
        uint32_t h = 0;
        for (int e = 0; e < 32; e++) h |= (uint32_t)((sb[e] >> bit) & 1) << e;
        P.qh[b] = h;
        const int s0 = q3k_scale(sb + 96, 2 * bi) - 32, s1 = q3k_scale(sb + 96, 2 * bi + 1) - 32;
        P.d[b] = (uint16_t)((s0 & 0xff) | ((s1 & 0xff) << 8));
        if (bi == 0) P.sb[b >> 3] = ld16(sb + 108);
    }
}

inline int grid_for(int64_t nb) {
    int64_t g = (nb + 255) / 256;
    return g > 65536 ? 65536 : (int)(g < 1 ? 1 : g);
}

}  // namespace

sllm_status pack_from_raw(int fmt, const uint8_t *raw_dev, int rows, int G, const MutPlanes &P, int *err_dev,
                          hipStream_t s) {
    const int64_t nb = (int64_t)rows * G;
    hipLaunchKernelGGL(pack_raw_kernel, dim3(grid_for(nb)), dim3(256), 0, s, fmt, raw_dev, nb, P, err_dev);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

sllm_status pack_from_gguf(uint32_t t, const uint8_t *raw_dev, int rows, int cols, const MutPlanes &P,
                           hipStream_t s) {
    const int64_t nb = (int64_t)rows * (cols / 32);
    switch (t) {
    case 12: hipLaunchKernelGGL(pack_q4k_kernel, dim3(grid_for(nb)), dim3(256), 0, s, raw_dev, nb, P); break;
    case 13: hipLaunchKernelGGL(pack_q5k_kernel, dim3(grid_for(nb)), dim3(256), 0, s, raw_dev, nb, P); break;
    case 14: hipLaunchKernelGGL(pack_q6k_kernel, dim3(grid_for(nb)), dim3(256), 0, s, raw_dev, nb, P); break;
    case 20: hipLaunchKernelGGL(pack_iq4nl_kernel, dim3(grid_for(nb)), dim3(256), 0, s, raw_dev, nb, P); break;
    case 10: hipLaunchKernelGGL(pack_q2k_kernel, dim3(grid_for(nb)), dim3(256), 0, s, raw_dev, nb, P); break;
    case 11: hipLaunchKernelGGL(pack_q3k_kernel, dim3(grid_for(nb)), dim3(256), 0, s, raw_dev, nb, P); break;
    default: return set_error(SLLM_ERR_QTYPE, "pack_from_gguf: not a remapped type");
    }
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

void export_kq_native(int fmt, const MutPlanes &p, int64_t nb, uint8_t *o) {
    // inverse of pack_q2k_kernel / pack_q3k_kernel, one super-block at a time
    const int per = fmt == SLLM_Q2K ? 84 : 110;
    for (int64_t s = 0; s < nb / 8; s++) {
        uint8_t *sb = o + s * per;
        std::memset(sb, 0, (size_t)per);
        uint8_t *qs = sb + (fmt == SLLM_Q2K ? 16 : 32);
        int v[16];
        for (int bi = 0; bi < 8; bi++) {
            const int64_t b = s * 8 + bi;
            const int n = bi >> 2, sh = 2 * (bi & 3);
            for (int l = 0; l < 16; l++) {
                qs[32 * n + l] |= (uint8_t)(((p.q2[b].x >> (2 * l)) & 3) << sh);
                qs[32 * n + 16 + l] |= (uint8_t)(((p.q2[b].y >> (2 * l)) & 3) << sh);
            }
            if (fmt == SLLM_Q2K) {
                sb[2 * bi] = (uint8_t)(p.d[b] & 0xff);
                sb[2 * bi + 1] = (uint8_t)(p.d[b] >> 8);
            } else {
                const int bit = 4 * n + (bi & 3);
                for (int e = 0; e < 32; e++) sb[e] |= (uint8_t)(((p.qh[b] >> e) & 1) << bit);
                v[2 * bi] = (int)(int8_t)(p.d[b] & 0xff) + 32;
                v[2 * bi + 1] = (int)(int8_t)(p.d[b] >> 8) + 32;
            }
        }
        if (fmt == SLLM_Q2K) {
            sb[80] = (uint8_t)(p.sb[s] & 0xff);
            sb[81] = (uint8_t)((p.sb[s] >> 8) & 0xff);
            sb[82] = (uint8_t)((p.sb[s] >> 16) & 0xff);
            sb[83] = (uint8_t)(p.sb[s] >> 24);
        } else {
            uint8_t *scb = sb + 96;
            for (int i = 0; i < 4; i++) {
                scb[i] = (uint8_t)((v[i] & 0x0f) | ((v[8 + i] & 0x0f) << 4));
                scb[4 + i] = (uint8_t)((v[4 + i] & 0x0f) | ((v[12 + i] & 0x0f) << 4));
                scb[8 + i] = (uint8_t)((v[i] >> 4) | ((v[4 + i] >> 4) << 2) | ((v[8 + i] >> 4) << 4) |
                                       ((v[12 + i] >> 4) << 6));
            }
            sb[108] = (uint8_t)(p.sb[s] & 0xff);
            sb[109] = (uint8_t)((p.sb[s] >> 8) & 0xff);
        }
    }
}

sllm_status check_q5k1_one_mfma(const MutPlanes &P, int64_t nb, int *bad_dev, hipStream_t s) {
    hipLaunchKernelGGL(q5k1_scale_check_kernel, dim3(grid_for(nb)), dim3(256), 0, s, P.d, P.dh, nb, bad_dev);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

sllm_status pack_q6k_stream(const uint8_t *raw_dev, int rows, int cols, const MutPlanes &P, hipStream_t s) {
    const int64_t nb = (int64_t)rows * (cols / 32);
    hipLaunchKernelGGL(pack_q6k_stream_kernel, dim3(grid_for(nb)), dim3(256), 0, s, raw_dev, nb, P);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

sllm_status pack_from_f32(const float *w_dev, int rows, int cols, const MutPlanes &P, hipStream_t s) {
    const int64_t nb = (int64_t)rows * (cols / 32);
    hipLaunchKernelGGL(pack_f32_kernel, dim3(grid_for(nb)), dim3(256), 0, s, w_dev, nb, P);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

}  // namespace sllm
