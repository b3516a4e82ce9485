/*
 * refcpu.c — scalar restatement of scriptling-llm-lib's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle). The product library never links or
 * calls this file. Built with: gcc -O2 -ffp-contract=off -fno-fast-math.
 *
 * Each function restates the reference function named in its comment from the
 * Go source, keeping the evaluation order and the precision of every step:
 *   - Go evaluates `a * b * c` left to right, each op rounded in the operand
 *     type (float32 ops stay float32; no FMA contraction on amd64 GOAMD64=v1);
 *   - float32 -> int32 conversion truncates toward zero; on amd64 (CVTTSS2SL)
 *     NaN and out-of-range values give INT32_MIN ("integer indefinite");
 *   - float -> int8 of a NaN keeps the low byte of INT32_MIN, i.e. 0.
 *
 * How each part is pinned independently of this file (tests/test_oracle_*.py):
 * the reference tests' own known answers and pattern vectors, exhaustive f16
 * tables against an independent decoder, brute-force integer sums, closed-form
 * requantization, and dequant(remap) == dequant(source) identities.
 */
#include "refcpu.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- f16 ---- */

static inline float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t f64_bits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

/*
 * dot_scalar.go:46-64 f16ToF32 (and the f16LUT built from it, q8q8.go:60-62;
 * readF16F32 float32_ops.go:87-106 is the same function). For a subnormal half
 * the Go code builds the float32 whose bit pattern is frac<<13 (itself a float32
 * denormal, value frac*2^-136) and divides it by 2^24, so every f16 subnormal
 * decodes to a signed zero. This is reproduced literally.
 */
float ref_f16_to_f32_lut(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t frac = h & 0x3ffu;
    if (exp == 0) {
        if (frac == 0) return f32_from_bits(sign);
        volatile float f32 = f32_from_bits(sign | (frac << 13));
        return f32 / (float)(1 << 24);
    }
    if (exp == 31) {
        if (frac == 0) return f32_from_bits(sign | 0x7f800000u);
        return f32_from_bits(sign | 0x7fc00000u);
    }
    return f32_from_bits(sign | ((exp + 112) << 23) | (frac << 13));
}

/*
 * VCVTPH2PS (used in-kernel by q4q8_row_amd64.s:36-38 and q41q8_row_amd64.s:58-63):
 * exact IEEE half -> single, subnormals normalised, NaN quietened with payload.
 */
float ref_f16_to_f32_cvtph(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t frac = h & 0x3ffu;
    if (exp == 0) {
        if (frac == 0) return f32_from_bits(sign);
        int e = 113; /* 127 - 14 */
        while (!(frac & 0x400u)) { frac <<= 1; e--; }
        frac &= 0x3ffu;
        return f32_from_bits(sign | ((uint32_t)e << 23) | (frac << 13));
    }
    if (exp == 31) return f32_from_bits(sign | 0x7f800000u | (frac << 13) | (frac ? 0x400000u : 0));
    return f32_from_bits(sign | ((exp + 112) << 23) | (frac << 13));
}

/* llm_primitives.go:698-717 float16ToFloat64 (exact; NaN -> NaN). */
double ref_f16_to_f64(uint16_t h) {
    double sign = (h & 0x8000u) ? -1.0 : 1.0;
    int exp = (h >> 10) & 0x1f;
    double frac = (double)(h & 0x3ffu);
    if (exp == 0 && frac == 0) return sign * 0.0;
    if (exp == 0) return sign * ldexp(frac / 1024.0, -14);
    if (exp == 31 && frac == 0) return sign * INFINITY;
    if (exp == 31) return NAN;
    return sign * ldexp(1.0 + frac / 1024.0, exp - 15);
}

/*
 * quantize.go:133-159 float64ToFloat16: NaN/Inf -> 0; mantissa TRUNCATED to 10
 * bits; results below the f16 normal range flush to a signed zero; overflow
 * to signed infinity.
 */
uint16_t ref_f64_to_f16(double f) {
    if (isnan(f) || isinf(f)) return 0;
    uint64_t bits = f64_bits(f);
    uint16_t sign = (uint16_t)((bits >> 48) & 0x8000u);
    uint64_t exp64 = (bits >> 52) & 0x7ffu;
    uint64_t mant64 = bits & 0x000fffffffffffffull;
    if (exp64 == 0) return sign;
    if (exp64 == 0x7ff) return sign | 0x7c00u;
    int exp16 = (int)(int16_t)exp64 - 1023 + 15;
    if (exp16 <= 0) return sign;
    if (exp16 >= 0x1f) return sign | 0x7c00u;
    uint16_t mant16 = (uint16_t)((mant64 >> 42) & 0x3ffu);
    return sign | (uint16_t)(exp16 << 10) | mant16;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* Go's int32(float32) on amd64: CVTTSS2SL (truncate; NaN/out of range -> INT32_MIN). */
static inline int32_t go_f32_to_i32(float v) {
    if (isnan(v) || v >= 2147483648.0f || v < -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

/* Go's byte(int8(f64)) on amd64: CVTTSD2SL then the low byte (NaN -> 0x00). */
static inline uint8_t go_f64_to_i8_byte(double v) {
    if (isnan(v) || v >= 2147483648.0 || v < -2147483648.0) return 0;
    return (uint8_t)(int8_t)(int32_t)v;
}

/* ----------------------------------------------------------- quantizers ---- */

/* q8q8.go:96-125 quantizeActivationsQ8. */
void ref_quantize_act_q8(const float *x, int groups, int8_t *q, float *s) {
    for (int g = 0; g < groups; g++) {
        const float *xb = x + (size_t)g * 32;
        float maxAbs = 0.0f;
        for (int i = 0; i < 32; i++) {
            float v = xb[i];
            if (v < 0) v = -v;
            if (v > maxAbs) maxAbs = v;
        }
        float scale = 0.0f, inv = 0.0f;
        if (maxAbs > 0) {
            scale = maxAbs / 127.0f;
            inv = 1.0f / scale;
        }
        s[g] = scale;
        for (int i = 0; i < 32; i++) {
            int32_t v = go_f32_to_i32(xb[i] * inv);
            if (v > 127) v = 127;
            else if (v < -128) v = -128;
            q[(size_t)g * 32 + i] = (int8_t)v;
        }
    }
}

/* gguf.go:1136-1186 quantizeQ8RowsF32 (fp32 absmax/scale/inv, round half away). */
int ref_quantize_q8_rows_f32(const float *w, int rows, int cols, uint8_t *out) {
    if (cols % 32 != 0 || rows <= 0 || cols <= 0) return -1;
    int gpr = cols / 32;
    uint8_t *o = out;
    for (int r = 0; r < rows; r++) {
        for (int g = 0; g < gpr; g++) {
            const float *b = w + (size_t)r * cols + (size_t)g * 32;
            float maxAbs = 0.0f;
            for (int i = 0; i < 32; i++) {
                float v = b[i];
                if (v < 0) v = -v;
                if (v > maxAbs) maxAbs = v;
            }
            float scale = 0.0f;
            if (maxAbs > 0) scale = maxAbs / 127.0f;
            wr16(o, ref_f64_to_f16((double)scale));
            volatile float one = 1.0f;
            float inv = one / scale; /* +Inf for an all-zero block */
            for (int i = 0; i < 32; i++) {
                double val = (double)(b[i] * inv);
                if (val > 127) val = 127;
                else if (val < -128) val = -128;
                o[2 + i] = go_f64_to_i8_byte(round(val));
            }
            o += 34;
        }
    }
    return 0;
}

/* gguf.go:1080-1134 quantizeQ8Rows (fp64 throughout; stored scale is f16-truncated,
 * but inv uses the unrounded fp64 scale). */
int ref_quantize_q8_rows_f64(const double *w, int rows, int cols, uint8_t *out) {
    if (cols % 32 != 0 || rows <= 0 || cols <= 0) return -1;
    int gpr = cols / 32;
    uint8_t *o = out;
    for (int r = 0; r < rows; r++) {
        for (int g = 0; g < gpr; g++) {
            const double *b = w + (size_t)r * cols + (size_t)g * 32;
            double maxAbs = 0.0;
            for (int i = 0; i < 32; i++) {
                double v = fabs(b[i]);
                if (v > maxAbs) maxAbs = v;
            }
            double scale = 0.0;
            if (maxAbs > 0) scale = maxAbs / 127.0;
            wr16(o, ref_f64_to_f16(scale));
            volatile double one = 1.0;
            double inv = one / scale;
            for (int i = 0; i < 32; i++) {
                double val = b[i] * inv;
                if (val > 127) val = 127;
                else if (val < -128) val = -128;
                o[2 + i] = go_f64_to_i8_byte(round(val));
            }
            o += 34;
        }
    }
    return 0;
}

/* --------------------------------------------------------- dequantizers ---- */

void ref_dequant_q8_0(const uint8_t *raw, int64_t n, double *out) {
    for (int64_t g = 0; g < n / 32; g++) {
        const uint8_t *b = raw + g * 34;
        double scale = ref_f16_to_f64(rd16(b));
        for (int i = 0; i < 32; i++) out[g * 32 + i] = (double)(int8_t)b[2 + i] * scale;
    }
}

void ref_dequant_q4_0(const uint8_t *raw, int64_t n, double *out) {
    for (int64_t g = 0; g < n / 32; g++) {
        const uint8_t *b = raw + g * 18;
        double scale = ref_f16_to_f64(rd16(b));
        for (int i = 0; i < 16; i++) {
            uint8_t v = b[2 + i];
            out[g * 32 + i] = (double)((int)(v & 0x0f) - 8) * scale;
            out[g * 32 + 16 + i] = (double)((int)((v >> 4) & 0x0f) - 8) * scale;
        }
    }
}

void ref_dequant_q4_1(const uint8_t *raw, int64_t n, double *out) {
    for (int64_t g = 0; g < n / 32; g++) {
        const uint8_t *b = raw + g * 20;
        double d = ref_f16_to_f64(rd16(b));
        double m = ref_f16_to_f64(rd16(b + 2));
        for (int i = 0; i < 16; i++) {
            uint8_t v = b[4 + i];
            out[g * 32 + i] = (double)(v & 0x0f) * d + m;
            out[g * 32 + 16 + i] = (double)((v >> 4) & 0x0f) * d + m;
        }
    }
}

void ref_dequant_q5_0(const uint8_t *raw, int64_t n, double *out) {
    for (int64_t g = 0; g < n / 32; g++) {
        const uint8_t *b = raw + g * 22;
        double d = ref_f16_to_f64(rd16(b));
        uint32_t qh = rd32(b + 2);
        for (int j = 0; j < 16; j++) {
            uint8_t q = b[6 + j];
            int32_t xh0 = (int32_t)((qh >> j) << 4) & 0x10;
            int32_t xh1 = (int32_t)(qh >> (j + 12)) & 0x10;
            out[g * 32 + j] = (double)(((int32_t)(q & 0x0f) | xh0) - 16) * d;
            out[g * 32 + j + 16] = (double)(((int32_t)(q >> 4) | xh1) - 16) * d;
        }
    }
}

/* kquants.go:62-71 getScaleMinK4. */
void ref_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void ref_dequant_q4_k(const uint8_t *raw, int64_t n, double *out) {
    int64_t oi = 0;
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *base = raw + b * 144;
        double d = ref_f16_to_f64(rd16(base));
        double dmin = ref_f16_to_f64(rd16(base + 2));
        const uint8_t *scales = base + 4, *qs = base + 16;
        int is = 0, qo = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t sc, m;
            ref_scale_min_k4(is, scales, &sc, &m);
            double d1 = d * (double)sc, m1 = dmin * (double)m;
            ref_scale_min_k4(is + 1, scales, &sc, &m);
            double d2 = d * (double)sc, m2 = dmin * (double)m;
            for (int l = 0; l < 32; l++) out[oi++] = d1 * (double)(qs[qo + l] & 0x0f) - m1;
            for (int l = 0; l < 32; l++) out[oi++] = d2 * (double)(qs[qo + l] >> 4) - m2;
            qo += 32;
            is += 2;
        }
    }
}

void ref_dequant_q5_k(const uint8_t *raw, int64_t n, double *out) {
    int64_t oi = 0;
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *base = raw + b * 176;
        double d = ref_f16_to_f64(rd16(base));
        double dmin = ref_f16_to_f64(rd16(base + 2));
        const uint8_t *scales = base + 4, *qh = base + 16, *qs = base + 48;
        int is = 0, qo = 0;
        uint8_t u1 = 1, u2 = 2;
        for (int j = 0; j < 256; j += 64) {
            uint8_t sc, m;
            ref_scale_min_k4(is, scales, &sc, &m);
            double d1 = d * (double)sc, m1 = dmin * (double)m;
            ref_scale_min_k4(is + 1, scales, &sc, &m);
            double d2 = d * (double)sc, m2 = dmin * (double)m;
            for (int l = 0; l < 32; l++) {
                double hi = (qh[l] & u1) ? 16.0 : 0.0;
                out[oi++] = d1 * ((double)(qs[qo + l] & 0x0f) + hi) - m1;
            }
            for (int l = 0; l < 32; l++) {
                double hi = (qh[l] & u2) ? 16.0 : 0.0;
                out[oi++] = d2 * ((double)(qs[qo + l] >> 4) + hi) - m2;
            }
            qo += 32;
            is += 2;
            u1 = (uint8_t)(u1 << 2);
            u2 = (uint8_t)(u2 << 2);
        }
    }
}

/* gguf.go:988-1015 dequantizeQ6KBlock (products are exact in fp64). */
static void dequant_q6k_block(const uint8_t *raw, double *out) {
    double d = ref_f16_to_f64(rd16(raw + 208));
    const uint8_t *ql = raw, *qh = raw + 128;
    const uint8_t *sc = raw + 192;
    int oo = 0;
    for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            double q1 = (double)((int)(int8_t)((ql[l] & 0xf) | (((qh[l] >> 0) & 3) << 4)) - 32);
            double q2 = (double)((int)(int8_t)((ql[l + 32] & 0xf) | (((qh[l] >> 2) & 3) << 4)) - 32);
            double q3 = (double)((int)(int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
            double q4 = (double)((int)(int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
            double sc0 = (double)(int8_t)sc[is + 0];
            double sc2 = (double)(int8_t)sc[is + 2];
            double sc4 = (double)(int8_t)sc[is + 4];
            double sc6 = (double)(int8_t)sc[is + 6];
            out[oo + l + 0] = d * sc0 * q1;
            out[oo + l + 32] = d * sc2 * q2;
            out[oo + l + 64] = d * sc4 * q3;
            out[oo + l + 96] = d * sc6 * q4;
        }
        oo += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

void ref_dequant_q6_k(const uint8_t *raw, int64_t n, double *out) {
    for (int64_t b = 0; b < n / 256; b++) dequant_q6k_block(raw + b * 210, out + b * 256);
}

/* kquants.go:7 iq4nlValues, kquants.go:14-27 dequantizeIQ4NLNative. */
static const int8_t kIQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1, 13, 25, 38, 53, 69, 89, 113};

void ref_dequant_iq4_nl(const uint8_t *raw, int64_t n, double *out) {
    for (int64_t b = 0; b < n / 32; b++) {
        const uint8_t *base = raw + b * 18;
        double d = ref_f16_to_f64(rd16(base));
        const uint8_t *qs = base + 2;
        for (int j = 0; j < 16; j++) {
            out[b * 32 + j] = d * (double)kIQ4NL[qs[j] & 0x0f];
            out[b * 32 + 16 + j] = d * (double)kIQ4NL[qs[j] >> 4];
        }
    }
}

/* ---------------------------------------------------------------- remaps ---- */

/* kquant_kernels.go:30-63 convertQ4KToQ41. */
void ref_convert_q4k_to_q41(const uint8_t *src, int rows, int cols, uint8_t *out) {
    int nSB = cols / 256;
    uint8_t *o = out;
    for (int r = 0; r < rows; r++) {
        for (int sb = 0; sb < nSB; sb++) {
            const uint8_t *b = src + ((size_t)r * nSB + sb) * 144;
            double d = ref_f16_to_f64(rd16(b));
            double dmin = ref_f16_to_f64(rd16(b + 2));
            const uint8_t *scales = b + 4, *qs = b + 16;
            for (int jj = 0; jj < 8; jj++) {
                uint8_t sc, m;
                ref_scale_min_k4(jj, scales, &sc, &m);
                wr16(o, ref_f64_to_f16(d * (double)sc));
                wr16(o + 2, ref_f64_to_f16(-dmin * (double)m));
                int k = (jj / 2) * 32;
                for (int i = 0; i < 16; i++) {
                    if ((jj & 1) == 0)
                        o[4 + i] = (uint8_t)((qs[k + i] & 0x0f) | ((qs[k + i + 16] & 0x0f) << 4));
                    else
                        o[4 + i] = (uint8_t)((qs[k + i] >> 4) | ((qs[k + i + 16] >> 4) << 4));
                }
                o += 20;
            }
        }
    }
}

/* kquant_kernels.go:110-154 convertQ5KToTwoQ41. */
void ref_convert_q5k_to_two_q41(const uint8_t *src, int rows, int cols, uint8_t *out) {
    int nSB = cols / 256;
    size_t half = (size_t)rows * (cols / 32) * 20;
    uint8_t *lo = out, *hi = out + half;
    for (int r = 0; r < rows; r++) {
        for (int sb = 0; sb < nSB; sb++) {
            const uint8_t *b = src + ((size_t)r * nSB + sb) * 176;
            double d = ref_f16_to_f64(rd16(b));
            double dmin = ref_f16_to_f64(rd16(b + 2));
            const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
            for (int jj = 0; jj < 8; jj++) {
                uint8_t sc, m;
                ref_scale_min_k4(jj, scales, &sc, &m);
                double dsc = d * (double)sc;
                wr16(lo, ref_f64_to_f16(dsc));
                wr16(lo + 2, ref_f64_to_f16(-dmin * (double)m));
                int k = (jj / 2) * 32;
                for (int i = 0; i < 16; i++) {
                    if ((jj & 1) == 0)
                        lo[4 + i] = (uint8_t)((qs[k + i] & 0x0f) | ((qs[k + i + 16] & 0x0f) << 4));
                    else
                        lo[4 + i] = (uint8_t)((qs[k + i] >> 4) | ((qs[k + i + 16] >> 4) << 4));
                }
                lo += 20;
                wr16(hi, ref_f64_to_f16(16 * dsc));
                wr16(hi + 2, 0);
                for (int i = 0; i < 16; i++)
                    hi[4 + i] = (uint8_t)(((qh[i] >> jj) & 1) | (((qh[i + 16] >> jj) & 1) << 4));
                hi += 20;
            }
        }
    }
}

int ref_block_bytes(const char *qtype) {
    if (!strcmp(qtype, "q8")) return 34;
    if (!strcmp(qtype, "q4")) return 18;
    if (!strcmp(qtype, "q4_1")) return 20;
    if (!strcmp(qtype, "q5")) return 22;
    if (!strcmp(qtype, "q5k1")) return 40;
    return -1;
}

/* gguf.go:818-934 loadWeightF32Direct, int8-kernel branches (useInt8Q8/Q41 on). */
int64_t ref_load_weight(uint32_t t, const uint8_t *raw, int rows, int cols,
                        char *qtype, uint8_t *out, int64_t out_cap) {
    int64_t n = (int64_t)rows * cols;
    int64_t G = n / 32;
    const char *qt = NULL;
    int64_t bytes = -1;
    switch (t) {
    case 8: qt = "q8"; bytes = G * 34; break;
    case 2: qt = "q4"; bytes = G * 18; break;
    case 3: qt = "q4_1"; bytes = G * 20; break;
    case 6: qt = "q5"; bytes = G * 22; break;
    default: break;
    }
    if (qt) {
        if (cols % 32 || bytes > out_cap) return -1;
        memcpy(out, raw, (size_t)bytes);
        strcpy(qtype, qt);
        return bytes;
    }
    if (t == 12 && cols % 256 == 0) {
        bytes = G * 20;
        if (bytes > out_cap) return -1;
        ref_convert_q4k_to_q41(raw, rows, cols, out);
        strcpy(qtype, "q4_1");
        return bytes;
    }
    if (t == 13 && cols % 256 == 0) {
        bytes = G * 40;
        if (bytes > out_cap) return -1;
        ref_convert_q5k_to_two_q41(raw, rows, cols, out);
        strcpy(qtype, "q5k1");
        return bytes;
    }
    if ((t == 14 || t == 20) && cols % 32 == 0) {
        bytes = G * 34;
        if (bytes > out_cap) return -1;
        double *flat = (double *)malloc((size_t)n * sizeof(double));
        if (!flat) return -1;
        if (t == 14) ref_dequant_q6_k(raw, n, flat);
        else ref_dequant_iq4_nl(raw, n, flat);
        ref_quantize_q8_rows_f64(flat, rows, cols, out);
        free(flat);
        strcpy(qtype, "q8");
        return bytes;
    }
    return -1;
}

/* -------------------------------------------------------------- dots ---- */

/* q8q8.go:83-91 int8DotScalar. */
int32_t ref_int8_dot(const int8_t *a, const int8_t *b, int n) {
    int32_t s = 0;
    for (int i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

/* Q8_0 block: Σ w·xq over the 32 int8 (q8q8_row_amd64.s:25-40). */
static int32_t q8_block_isum(const uint8_t *blk, const int8_t *xq) {
    return ref_int8_dot((const int8_t *)(blk + 2), xq, 32);
}

/* Q4_0 block: Σ(nib-8)·xq (q4q8.go:37-43; equals Σnib·xq − 8Σxq of the fused kernel). */
static int32_t q4_block_isum(const uint8_t *blk, const int8_t *xq) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        uint8_t b = blk[2 + j];
        s += ((int32_t)(b & 0x0f) - 8) * xq[j] + ((int32_t)(b >> 4) - 8) * xq[j + 16];
    }
    return s;
}

/* Q4_1 block: Σ nib·xq (q41q8_vnni_amd64.go:31-35). qs at blk+4. */
static int32_t q41_block_qsum(const uint8_t *blk, const int8_t *xq) {
    int32_t s = 0;
    for (int i = 0; i < 16; i++) {
        uint8_t b = blk[4 + i];
        s += (int32_t)(b & 0x0f) * xq[i] + (int32_t)(b >> 4) * xq[16 + i];
    }
    return s;
}

/* Q5_0 in-block fp32 partial sum in the reference order (float32_ops.go:340-365). */
static float q5_block_sum(const uint8_t *blk, const float *x) {
    uint32_t qh = rd32(blk + 2);
    const uint8_t *qs = blk + 6;
    float sum = 0.0f;
    for (int j = 0; j < 16; j++) {
        uint8_t xh0 = (uint8_t)((qh >> j) << 4) & 0x10;
        uint8_t xh1 = (uint8_t)(qh >> (j + 12)) & 0x10;
        float v0 = (float)(int32_t)((qs[j] & 0x0f) | xh0) - 16;
        float v1 = (float)(int32_t)((qs[j] >> 4) | xh1) - 16;
        float p0 = v0 * x[j];
        float p1 = v1 * x[j + 16];
        float pair = p0 + p1;
        sum = sum + pair;
    }
    return sum;
}

static int32_t sum_xq32(const int8_t *xq) {
    int32_t s = 0;
    for (int k = 0; k < 32; k++) s += xq[k];
    return s;
}

/* q8q8.go:131-141 q8q8RowDot; identical per-group term and sequential sum in the
 * fused AVX2 (q8q8_row_amd64.s:16-58) and VNNI (vnni_amd64.s:41-84) kernels. */
float ref_q8q8_row(const uint8_t *w, const int8_t *xq, const float *xs, int groups) {
    float total = 0.0f;
    for (int g = 0; g < groups; g++) {
        const uint8_t *b = w + (size_t)g * 34;
        float ws = ref_f16_to_f32_lut(rd16(b));
        int32_t isum = q8_block_isum(b, xq + (size_t)g * 32);
        float cmb = ws * xs[g];
        float term = cmb * (float)isum;
        total = total + term;
    }
    return total;
}

/*
 * q4q8.go:29-45 q4q8RowDotScalarDecode structure (ws·xs·float(isum), sequential).
 * The scale is decoded with VCVTPH2PS as in the fused kernel that runs on amd64
 * (q4q8_row_amd64.s:36-38); the two decodes differ only for subnormal halves.
 */
float ref_q4q8_row(const uint8_t *w, const int8_t *xq, const float *xs, int groups) {
    float total = 0.0f;
    for (int g = 0; g < groups; g++) {
        const uint8_t *b = w + (size_t)g * 18;
        float ws = ref_f16_to_f32_cvtph(rd16(b));
        int32_t isum = q4_block_isum(b, xq + (size_t)g * 32);
        float cmb = ws * xs[g];
        float term = cmb * (float)isum;
        total = total + term;
    }
    return total;
}

/* q41q8_row_amd64.s:55-71 (and the VNNI twin q41q8_vnni_amd64.s:52-68):
 * term = ((float(qsum)·d) + (float(sumXq)·m))·xs, accumulated sequentially. */
float ref_q41q8_row(const uint8_t *w, const int8_t *xq, const float *xs,
                    const int32_t *sum_xq, int groups) {
    float acc = 0.0f;
    for (int g = 0; g < groups; g++) {
        const uint8_t *b = w + (size_t)g * 20;
        float d = ref_f16_to_f32_cvtph(rd16(b));
        float m = ref_f16_to_f32_cvtph(rd16(b + 2));
        int32_t qsum = q41_block_qsum(b, xq + (size_t)g * 32);
        float t1 = (float)qsum * d;
        float t2 = (float)sum_xq[g] * m;
        float t = t1 + t2;
        t = t * xs[g];
        acc = acc + t;
    }
    return acc;
}

/* float32_ops.go:507-513 q5DotRowsF32 over q5DotGroupXF32 (:335-367). */
float ref_q5_row(const uint8_t *w, const float *x, int groups) {
    float total = 0.0f;
    for (int g = 0; g < groups; g++) {
        const uint8_t *b = w + (size_t)g * 22;
        float s = ref_f16_to_f32_lut(rd16(b));
        float sum = q5_block_sum(b, x + (size_t)g * 32);
        float grp = s * sum;
        total = total + grp;
    }
    return total;
}

/* ------------------------------------------------------------- drivers ---- */

typedef struct { int8_t *xq; float *xs; int32_t *sxq; } act_t;

static int act_quantize(const float *x, int M, int G, act_t *a) {
    int K = G * 32;
    a->xq = (int8_t *)malloc((size_t)M * K);
    a->xs = (float *)malloc((size_t)M * G * sizeof(float));
    a->sxq = (int32_t *)malloc((size_t)M * G * sizeof(int32_t));
    if (!a->xq || !a->xs || !a->sxq) return -1;
    for (int r = 0; r < M; r++) {
        ref_quantize_act_q8(x + (size_t)r * K, G, a->xq + (size_t)r * K, a->xs + (size_t)r * G);
        for (int g = 0; g < G; g++) a->sxq[(size_t)r * G + g] = sum_xq32(a->xq + (size_t)r * K + (size_t)g * 32);
    }
    return 0;
}

static void act_free(act_t *a) { free(a->xq); free(a->xs); free(a->sxq); }

void ref_q8q8_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst) {
    act_t a;
    if (act_quantize(x, M, G, &a)) { act_free(&a); return; }
    int K = G * 32;
    for (int j = 0; j < N; j++)
        for (int xi = 0; xi < M; xi++)
            dst[(size_t)xi * N + j] = ref_q8q8_row(raw + (size_t)j * G * 34, a.xq + (size_t)xi * K,
                                                   a.xs + (size_t)xi * G, G);
    act_free(&a);
}

void ref_q4q8_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst) {
    act_t a;
    if (act_quantize(x, M, G, &a)) { act_free(&a); return; }
    int K = G * 32;
    for (int xi = 0; xi < M; xi++)
        for (int j = 0; j < N; j++)
            dst[(size_t)xi * N + j] = ref_q4q8_row(raw + (size_t)j * G * 18, a.xq + (size_t)xi * K,
                                                   a.xs + (size_t)xi * G, G);
    act_free(&a);
}

void ref_q41q8_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst) {
    act_t a;
    if (act_quantize(x, M, G, &a)) { act_free(&a); return; }
    int K = G * 32;
    for (int xi = 0; xi < M; xi++)
        for (int j = 0; j < N; j++)
            dst[(size_t)xi * N + j] = ref_q41q8_row(raw + (size_t)j * G * 20, a.xq + (size_t)xi * K,
                                                    a.xs + (size_t)xi * G, a.sxq + (size_t)xi * G, G);
    act_free(&a);
}

void ref_q5k1_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst) {
    size_t half = (size_t)N * G * 20;
    ref_q41q8_matmul(raw, N, G, x, M, dst);
    float *tmp = (float *)malloc((size_t)M * N * sizeof(float));
    if (!tmp) return;
    ref_q41q8_matmul(raw + half, N, G, x, M, tmp);
    for (size_t i = 0; i < (size_t)M * N; i++) dst[i] = dst[i] + tmp[i];
    free(tmp);
}

void ref_q5_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst) {
    int K = G * 32;
    for (int xi = 0; xi < M; xi++)
        for (int j = 0; j < N; j++)
            dst[(size_t)xi * N + j] = ref_q5_row(raw + (size_t)j * G * 22, x + (size_t)xi * K, G);
}

int ref_matmul_quant(const char *qtype, const uint8_t *raw, int N, int K,
                     const float *x, int M, float *dst) {
    if (K % 32) return -1;
    int G = K / 32;
    if (!strcmp(qtype, "q8")) ref_q8q8_matmul(raw, N, G, x, M, dst);
    else if (!strcmp(qtype, "q4")) ref_q4q8_matmul(raw, N, G, x, M, dst);
    else if (!strcmp(qtype, "q4_1")) ref_q41q8_matmul(raw, N, G, x, M, dst);
    else if (!strcmp(qtype, "q5")) ref_q5_matmul(raw, N, G, x, M, dst);
    else if (!strcmp(qtype, "q5k1")) ref_q5k1_matmul(raw, N, G, x, M, dst);
    else return -1;
    return 0;
}

int ref_block_dots(const char *qtype, const uint8_t *raw, int N, int G,
                   const int8_t *xq, const float *x, int M, int32_t *out) {
    int K = G * 32;
    int isq5k1 = !strcmp(qtype, "q5k1");
    size_t half = (size_t)N * G * 20;
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            for (int g = 0; g < G; g++) {
                size_t o = ((size_t)m * N + n) * G + g;
                const int8_t *q = xq + (size_t)m * K + (size_t)g * 32;
                if (!strcmp(qtype, "q8")) out[o] = q8_block_isum(raw + ((size_t)n * G + g) * 34, q);
                else if (!strcmp(qtype, "q4")) out[o] = q4_block_isum(raw + ((size_t)n * G + g) * 18, q);
                else if (!strcmp(qtype, "q4_1")) out[o] = q41_block_qsum(raw + ((size_t)n * G + g) * 20, q);
                else if (isq5k1) {
                    out[2 * o] = q41_block_qsum(raw + ((size_t)n * G + g) * 20, q);
                    out[2 * o + 1] = q41_block_qsum(raw + half + ((size_t)n * G + g) * 20, q);
                } else if (!strcmp(qtype, "q5")) {
                    float s = q5_block_sum(raw + ((size_t)n * G + g) * 22, x + (size_t)m * K + (size_t)g * 32);
                    memcpy(&out[o], &s, 4);
                } else return -1;
            }
        }
    }
    return 0;
}

int ref_argmax(const float *v, int n) {
    int best = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

/* forwardBlock's SwiGLU loop (model_f32.go:486-489):
 *   g := float64(gateData[i]); s := float32(1.0 / (1.0 + math.Exp(-g)))
 *   siluData[i] = gateData[i] * s * upData[i]      (float32, left to right)
 * math.Exp is Go's; libm's exp stands in for it here (both are faithfully
 * rounded; they can differ in the last bit of the float64, which changes the
 * float32 s only when that value lies within one float64 ulp of a float32
 * rounding boundary). */
float ref_swiglu(float gate, float up) {
    double e = exp(-(double)gate);
    float s = (float)(1.0 / (1.0 + e));
    float t = gate * s;
    return t * up;
}

void ref_swiglu_n(const float *gate, const float *up, float *h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = ref_swiglu(gate[i], up[i]);
}

/* rmsNormFlatF32 (float32_ops.go:159-172), per row:
 *   ss += v*v (float32, sequential); inv := 1.0 / float32(math.Sqrt(float64(ss)/float64(cols)+float64(eps)))
 *   out[j] = x[j] * inv * w[j]  (float32, left to right) */
static void rms_apply(const float *x, const float *w, float ss, float eps, int cols, float *out) {
    float inv = 1.0f / (float)sqrt((double)ss / (double)cols + (double)eps);
    for (int j = 0; j < cols; j++) {
        float t = x[j] * inv;
        out[j] = t * w[j];
    }
}

void ref_rmsnorm(const float *x, const float *w, float eps, int rows, int cols, float *out) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * cols;
        float ss = 0.0f;
        for (int j = 0; j < cols; j++) {
            float sq = xr[j] * xr[j];
            ss = ss + sq;
        }
        rms_apply(xr, w, ss, eps, cols, out + (size_t)r * cols);
    }
}

/* The same norm with the sum of squares in the library's association (its
 * fused GEMV prologue and prefill pre-pass): 256 slot sums, slot s adding
 * x[s]^2, x[s+256]^2, ... in order; each group of 64 slots added as a wave
 * reduction does it (pairs, quads, groups of 8 and of 16 as balanced trees,
 * then the four 16-slot sums left to right); the four 64-slot sums left to
 * right. Test infrastructure: it lets the GPU path be checked bit for bit;
 * ref_rmsnorm above is the reference's order. */
static float tree16(const float *v) {
    float a[16];
    for (int i = 0; i < 16; i++) a[i] = v[i];
    for (int w = 1; w < 16; w *= 2)
        for (int i = 0; i < 16; i += 2 * w) a[i] = a[i] + a[i + w];
    return a[0];
}

void ref_rmsnorm_lib(const float *x, const float *w, float eps, int rows, int cols, float *out) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * cols;
        float slot[256];
        for (int s = 0; s < 256; s++) {
            float p = 0.0f;
            for (int i = s; i < cols; i += 256) {
                float sq = xr[i] * xr[i];
                p = p + sq;
            }
            slot[s] = p;
        }
        float waves[4];
        for (int q = 0; q < 4; q++) {
            float r16[4];
            for (int k = 0; k < 4; k++) r16[k] = tree16(slot + 64 * q + 16 * k);
            waves[q] = ((r16[0] + r16[1]) + r16[2]) + r16[3];
        }
        float ss = ((waves[0] + waves[1]) + waves[2]) + waves[3];
        rms_apply(xr, w, ss, eps, cols, out + (size_t)r * cols);
    }
}

/* ---- the decode step around the matmuls --------------------------------- */

/* applyRopeInPlaceF32, float32_ops.go:174-188. The angle is a float32
 * product, cos / sin are taken in float64 and rounded to float32. */
void ref_rope(float *data, int rows, int d_k, int start_pos, const float *freqs, int half_dim) {
    for (int r = 0; r < rows; r++) {
        const int pos = start_pos + r;
        float *row = data + (size_t)r * d_k;
        for (int i = 0; i < half_dim; i++) {
            const float angle = freqs[i] * (float)pos;
            const float c = (float)cos((double)angle);
            const float s = (float)sin((double)angle);
            const float x0 = row[2 * i], x1 = row[2 * i + 1];
            row[2 * i] = x0 * c - x1 * s;
            row[2 * i + 1] = x0 * s + x1 * c;
        }
    }
}

/* fusedAttentionHeadF32, float32_ops.go:190-235: sequential float32 dot,
 * scale, causal -Inf mask, max (first score, then strict >), float32(exp(
 * float64(score - max))), sequential float32 sum, invSum = 1 / sum, and
 * out[d] = sum over ki of (exps[ki] * invSum) * v[ki][d], sequentially. */
void ref_attention_head(const float *q, const float *k, const float *v, int q_rows, int d_k, int k_rows,
                        int causal, int cache_len, float *out, int out_off) {
    const float scale = 1.0f / (float)sqrt((double)d_k);
    float *scores = (float *)malloc(sizeof(float) * (size_t)(k_rows > 0 ? k_rows : 1));
    float *exps = (float *)malloc(sizeof(float) * (size_t)(k_rows > 0 ? k_rows : 1));
    for (int qi = 0; qi < q_rows; qi++) {
        const float *qr = q + (size_t)qi * d_k;
        for (int ki = 0; ki < k_rows; ki++) {
            const float *kr = k + (size_t)ki * d_k;
            float dot = 0.0f;
            for (int d = 0; d < d_k; d++) dot += qr[d] * kr[d];
            scores[ki] = dot * scale;
        }
        if (causal) {
            for (int ki = cache_len + qi + 1; ki < k_rows; ki++) scores[ki] = -INFINITY;
        }
        float mx = scores[0];
        for (int ki = 1; ki < k_rows; ki++)
            if (scores[ki] > mx) mx = scores[ki];
        float sum = 0.0f;
        for (int ki = 0; ki < k_rows; ki++) {
            const float e = (float)exp((double)(scores[ki] - mx));
            exps[ki] = e;
            sum += e;
        }
        const float inv = 1.0f / sum;
        float *o = out + out_off + (size_t)qi * d_k;
        for (int d = 0; d < d_k; d++) {
            float val = 0.0f;
            for (int ki = 0; ki < k_rows; ki++) {
                const float t = exps[ki] * inv;
                val += t * v[(size_t)ki * d_k + d];
            }
            o[d] = val;
        }
    }
    free(scores);
    free(exps);
}

/* forwardBlock, model_f32.go:398-466: bias adds (:398-420), splitHeadsDataF32
 * (float32_ops.go:237-250), per-head QK RMSNorm (:424-435), RoPE (:437-443),
 * KV append (:445-448), repeatKVDataF32 (float32_ops.go:252-260: q head h reads kv head h / nRep,
 * :455-458), fusedAttentionHeadF32 with causal masking (:460-466) and
 * mergeHeadsDataF32 (float32_ops.go:262-273). */
void ref_attention_layer(float *q, float *k, float *v, int seq_len, int n_heads, int n_kv, int d_k,
                         const float *q_bias, int q_bias_len, const float *k_bias, int k_bias_len,
                         const float *v_bias, int v_bias_len, const float *q_norm_w, const float *k_norm_w,
                         float eps, int lib_norm, const float *freqs, int half_dim, int start_pos,
                         float *cache_k, float *cache_v, int cap, int cache_len, float *out, float *q_rot) {
    const int qc = n_heads * d_k, kc = n_kv * d_k;
    for (int s = 0; s < seq_len; s++) {
        if (q_bias)
            for (int j = 0; j < q_bias_len && j < qc; j++) q[(size_t)s * qc + j] += q_bias[j];
        if (k_bias)
            for (int j = 0; j < k_bias_len && j < kc; j++) k[(size_t)s * kc + j] += k_bias[j];
        if (v_bias)
            for (int j = 0; j < v_bias_len && j < kc; j++) v[(size_t)s * kc + j] += v_bias[j];
    }
    const size_t hs = (size_t)seq_len * d_k;
    float *qh = (float *)malloc(sizeof(float) * hs * (size_t)n_heads);
    float *kh = (float *)malloc(sizeof(float) * hs * (size_t)n_kv);
    float *vh = (float *)malloc(sizeof(float) * hs * (size_t)n_kv);
    for (int s = 0; s < seq_len; s++) {
        for (int h = 0; h < n_heads; h++)
            memcpy(qh + h * hs + (size_t)s * d_k, q + (size_t)s * qc + (size_t)h * d_k, sizeof(float) * d_k);
        for (int g = 0; g < n_kv; g++) {
            memcpy(kh + g * hs + (size_t)s * d_k, k + (size_t)s * kc + (size_t)g * d_k, sizeof(float) * d_k);
            memcpy(vh + g * hs + (size_t)s * d_k, v + (size_t)s * kc + (size_t)g * d_k, sizeof(float) * d_k);
        }
    }
    void (*norm)(const float *, const float *, float, int, int, float *) = lib_norm ? ref_rmsnorm_lib : ref_rmsnorm;
    if (q_norm_w)
        for (int h = 0; h < n_heads; h++) norm(qh + h * hs, q_norm_w, eps, seq_len, d_k, qh + h * hs);
    if (k_norm_w)
        for (int g = 0; g < n_kv; g++) norm(kh + g * hs, k_norm_w, eps, seq_len, d_k, kh + g * hs);
    for (int h = 0; h < n_heads; h++) ref_rope(qh + h * hs, seq_len, d_k, start_pos, freqs, half_dim);
    for (int g = 0; g < n_kv; g++) ref_rope(kh + g * hs, seq_len, d_k, start_pos, freqs, half_dim);
    for (int g = 0; g < n_kv; g++) {
        memcpy(cache_k + ((size_t)g * cap + cache_len) * d_k, kh + g * hs, sizeof(float) * hs);
        memcpy(cache_v + ((size_t)g * cap + cache_len) * d_k, vh + g * hs, sizeof(float) * hs);
    }
    const int kv_len = cache_len + seq_len, rep = n_heads / n_kv;
    float *att = (float *)malloc(sizeof(float) * hs * (size_t)n_heads);
    for (int h = 0; h < n_heads; h++) {
        const int g = h / rep;
        ref_attention_head(qh + h * hs, cache_k + (size_t)g * cap * d_k, cache_v + (size_t)g * cap * d_k, seq_len,
                           d_k, kv_len, 1, cache_len, att, (int)(h * hs));
    }
    for (int s = 0; s < seq_len; s++)
        for (int h = 0; h < n_heads; h++) {
            memcpy(out + (size_t)s * qc + (size_t)h * d_k, att + h * hs + (size_t)s * d_k, sizeof(float) * d_k);
            if (q_rot)
                memcpy(q_rot + (size_t)s * qc + (size_t)h * d_k, qh + h * hs + (size_t)s * d_k, sizeof(float) * d_k);
        }
    free(qh);
    free(kh);
    free(vh);
    free(att);
}

/* ---- native k-quants and the dense fp32 path ---------------------------- */

/* kquants.go:147-180 dequantizeQ2KNative: per 16-element sub-block the scale
 * byte gives dl = d * (sc & 15) and ml = dmin * (sc >> 4); w = dl * q - ml in
 * fp64, q the 2-bit code at bit pair `shift` of the code bytes. */
void ref_dequant_q2_k(const uint8_t *raw, int64_t n, double *out) {
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *base = raw + b * 84;
        const uint8_t *scales = base, *qs = base + 16;
        const double d = ref_f16_to_f64(rd16(base + 80)), dmin = ref_f16_to_f64(rd16(base + 82));
        double *o = out + b * 256;
        int is = 0, qo = 0;
        for (int half = 0; half < 2; half++) {
            for (int j = 0, shift = 0; j < 4; j++, shift += 2) {
                for (int sub = 0; sub < 2; sub++) {
                    const uint8_t sc = scales[is++];
                    const double dl = d * (double)(sc & 0x0f), ml = dmin * (double)(sc >> 4);
                    for (int l = 0; l < 16; l++) *o++ = dl * (double)((qs[qo + 16 * sub + l] >> shift) & 3) - ml;
                }
            }
            qo += 32;
        }
    }
}

/* kquants.go:183-245 dequantizeQ3KNative: the 16 six-bit scales unpacked from
 * their 12 bytes (low nibbles in bytes 0..7, high bit pairs in bytes 8..11),
 * dl = d * (scale - 32); w = dl * (q - sub) with sub = 0 where the element's
 * high-mask bit (bit m, m = 1, 2, 4, ... per sub-block pair) is set, else 4. */
void ref_dequant_q3_k(const uint8_t *raw, int64_t n, double *out) {
    for (int64_t b = 0; b < n / 256; b++) {
        const uint8_t *base = raw + b * 110;
        const uint8_t *hmask = base, *qs = base + 32, *scb = base + 96;
        const double d = ref_f16_to_f64(rd16(base + 108));
        int scales[16];
        for (int i = 0; i < 4; i++) {
            scales[i] = (scb[i] & 0x0f) | (((scb[8 + i] >> 0) & 3) << 4);
            scales[4 + i] = (scb[4 + i] & 0x0f) | (((scb[8 + i] >> 2) & 3) << 4);
            scales[8 + i] = (scb[i] >> 4) | (((scb[8 + i] >> 4) & 3) << 4);
            scales[12 + i] = (scb[4 + i] >> 4) | (((scb[8 + i] >> 6) & 3) << 4);
        }
        double *o = out + b * 256;
        int is = 0, qo = 0;
        uint8_t m = 1;
        for (int half = 0; half < 2; half++) {
            for (int j = 0, shift = 0; j < 4; j++, shift += 2, m = (uint8_t)(m << 1)) {
                for (int sub = 0; sub < 2; sub++) {
                    const double dl = d * (double)(scales[is++] - 32);
                    for (int l = 0; l < 16; l++) {
                        const double s = (hmask[16 * sub + l] & m) ? 0.0 : 4.0;
                        *o++ = dl * ((double)((qs[qo + 16 * sub + l] >> shift) & 3) - s);
                    }
                }
            }
            qo += 32;
        }
    }
}

/* modelMatmulFloatIntoF32 (float32_ops.go:462-482): dst[i][j] = sequential
 * float32 sum over l of x[i][l] * w[j][l]. */
void ref_matmul_dense(const float *w, int N, int K, const float *x, int M, float *dst) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float sum = 0.0f;
            const float *xr = x + (size_t)i * K, *wr = w + (size_t)j * K;
            for (int l = 0; l < K; l++) sum += xr[l] * wr[l];
            dst[(size_t)i * N + j] = sum;
        }
}

/* The same products summed per 32-element block, each from zero in element
 * order: out[i][j][g] (float32). */
void ref_dense_block_sums(const float *w, int N, int K, const float *x, int M, float *out) {
    const int G = K / 32;
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++)
            for (int g = 0; g < G; g++) {
                float sum = 0.0f;
                const float *xr = x + (size_t)i * K + 32 * g, *wr = w + (size_t)j * K + 32 * g;
                for (int l = 0; l < 32; l++) sum += xr[l] * wr[l];
                out[((size_t)i * N + j) * G + g] = sum;
            }
}
