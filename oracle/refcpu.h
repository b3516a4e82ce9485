/*
 * refcpu — scalar CPU restatement of scriptling-llm-lib's quantized-matmul
 * arithmetic, used ONLY as a test oracle and as the CPU baseline in bench.py.
 *
 * TEST INFRASTRUCTURE. Nothing in the product library links, loads or calls
 * this code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may use it, and then only as the checker / the timed CPU baseline.
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the reference repository root). Semantics that matter for
 * bit-exactness are reproduced literally: operation order, float32 vs float64
 * evaluation, truncation vs rounding, and the f16 decode each path uses.
 * The file must be compiled with -ffp-contract=off and without fast-math.
 */
#ifndef SLLM_REFCPU_H
#define SLLM_REFCPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 codecs -------------------------------------------------------- */
float    ref_f16_to_f32_lut(uint16_t h);    /* dot_scalar.go:46-64 (f16LUT q8q8.go:52,60-62) */
float    ref_f16_to_f32_cvtph(uint16_t h);  /* VCVTPH2PS semantics, q4q8_row_amd64.s:36-38 */
double   ref_f16_to_f64(uint16_t h);        /* llm_primitives.go:698-717 */
uint16_t ref_f64_to_f16(double f);          /* quantize.go:133-159 */

/* ---- quantizers -------------------------------------------------------- */
/* q8q8.go:96-125: per-32-block absmax, scale=maxAbs/127, q=trunc(x*inv) */
void ref_quantize_act_q8(const float *x, int groups, int8_t *q, float *s);
/* gguf.go:1136-1186 (fp32 weights -> Q8_0 raw, 34 B/block). returns 0 on ok */
int ref_quantize_q8_rows_f32(const float *w, int rows, int cols, uint8_t *out);
/* gguf.go:1080-1134 (fp64 weights -> Q8_0 raw). returns 0 on ok */
int ref_quantize_q8_rows_f64(const double *w, int rows, int cols, uint8_t *out);

/* ---- dequantizers (fp64, as the loader computes them) -------------------- */
void ref_dequant_q8_0(const uint8_t *raw, int64_t n, double *out);  /* gguf.go:424-435 */
void ref_dequant_q4_0(const uint8_t *raw, int64_t n, double *out);  /* gguf.go:437-452 */
void ref_dequant_q4_1(const uint8_t *raw, int64_t n, double *out);  /* gguf.go:454-470 */
void ref_dequant_q5_0(const uint8_t *raw, int64_t n, double *out);  /* gguf.go:472-490 */
void ref_dequant_q4_k(const uint8_t *raw, int64_t n, double *out);  /* kquants.go:73-102 */
void ref_dequant_q5_k(const uint8_t *raw, int64_t n, double *out);  /* kquants.go:104-145 */
void ref_dequant_q6_k(const uint8_t *raw, int64_t n, double *out);  /* gguf.go:979-1015 */
void ref_dequant_iq4_nl(const uint8_t *raw, int64_t n, double *out);/* kquants.go:7-27 */
void ref_dequant_q2_k(const uint8_t *raw, int64_t n, double *out);  /* kquants.go:147-180 */
void ref_dequant_q3_k(const uint8_t *raw, int64_t n, double *out);  /* kquants.go:183-245 */
/* float32_ops.go:462-482 modelMatmulFloatIntoF32 (dense float32 weights). */
void ref_matmul_dense(const float *w, int N, int K, const float *x, int M, float *dst);
/* Its products summed per 32-element block from zero, element order. */
void ref_dense_block_sums(const float *w, int N, int K, const float *x, int M, float *out);

/* ---- load-time remaps / requantization ---------------------------------- */
void ref_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m); /* kquants.go:62-71 */
/* kquant_kernels.go:30-63: Q4_K rows -> Q4_1 rows (rows*cols/32*20 bytes) */
void ref_convert_q4k_to_q41(const uint8_t *src, int rows, int cols, uint8_t *out);
/* kquant_kernels.go:110-154: Q5_K rows -> [low Q4_1 half][high Q4_1 half] */
void ref_convert_q5k_to_two_q41(const uint8_t *src, int rows, int cols, uint8_t *out);
/*
 * gguf.go:818-934 (loadWeightF32Direct, the int8-kernel branches): turns a
 * GGUF tensor of type ggml_type into the QuantWeight the matmul consumes.
 * Writes the QType name into qtype (>= 8 bytes) and the Raw bytes into out
 * (capacity out_cap). Returns Raw size in bytes, or -1 for a type the int8
 * path does not take (the reference then builds a dense fp32 weight).
 */
int64_t ref_load_weight(uint32_t ggml_type, const uint8_t *raw, int rows, int cols,
                        char *qtype, uint8_t *out, int64_t out_cap);

/* ---- integer block dots -------------------------------------------------- */
int32_t ref_int8_dot(const int8_t *a, const int8_t *b, int n); /* q8q8.go:83-91 */
/*
 * Per-(activation row m, weight row n, block g) integer block dots as the
 * reference's kernels form them (see ref_block_dots in refcpu.c for each
 * format's definition). Output int32 [M][N][G] (x2 for q5k1: [..][G][2]);
 * for q5 the fp32 in-block partial sum (before the d scale) is written as
 * its bit pattern. Returns 0, or -1 for an unknown qtype.
 */
int ref_block_dots(const char *qtype, const uint8_t *raw, int N, int G,
                   const int8_t *xq, const float *x, int M, int32_t *out);

/* ---- row dots (one weight row x one quantized activation row) ---------- */
float ref_q8q8_row(const uint8_t *w, const int8_t *xq, const float *xs, int groups);      /* q8q8.go:131-141, q8q8_row_amd64.s:16-58 */
float ref_q4q8_row(const uint8_t *w, const int8_t *xq, const float *xs, int groups);      /* q4q8.go:29-45 (d via VCVTPH2PS) */
float ref_q41q8_row(const uint8_t *w, const int8_t *xq, const float *xs, const int32_t *sum_xq, int groups); /* q41q8_row_amd64.s:25-83 */
float ref_q5_row(const uint8_t *w, const float *x, int groups);                           /* float32_ops.go:335-367,507-513 */

/* ---- matmul drivers (dst[xi*N + j]) -------------------------------------- */
void ref_q8q8_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst);  /* q8q8.go:147-246 */
void ref_q4q8_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst);  /* q4q8.go:49-101 */
void ref_q41q8_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst); /* q41q8.go:20-60 */
void ref_q5k1_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst);  /* kquant_kernels.go:159-174 */
void ref_q5_matmul(const uint8_t *raw, int N, int G, const float *x, int M, float *dst);    /* float32_ops.go:427-436 */
/*
 * float32_ops.go:379-460 (modelMatmulQuantIntoF32) dispatch on QType.
 * Returns 0, or -1 for an unknown qtype (the reference then leaves dst unfilled).
 */
int ref_matmul_quant(const char *qtype, const uint8_t *raw, int N, int K,
                     const float *x, int M, float *dst);
/* float32_ops.go:812-822: first index of the maximum (strict >). */
int ref_argmax(const float *v, int n);

/* Bytes per 32-element block of a QType's Raw ("q5k1" counts both halves). */
int ref_block_bytes(const char *qtype);

/* model_f32.go:486-489 SwiGLU, one element and n elements. */
float ref_swiglu(float gate, float up);
void ref_swiglu_n(const float *gate, const float *up, float *h, int64_t n);

/* rmsNormFlatF32 (float32_ops.go:159-172) in the reference's order, and with
 * the library's sum-of-squares association. */
void ref_rmsnorm(const float *x, const float *w, float eps, int rows, int cols, float *out);
void ref_rmsnorm_lib(const float *x, const float *w, float eps, int rows, int cols, float *out);

/* ---- the decode step around the matmuls --------------------------------- */
/* applyRopeInPlaceF32 (float32_ops.go:174-188): rows x d_k, pairs (2i, 2i+1),
 * i < half_dim, at positions start_pos + r. */
void ref_rope(float *data, int rows, int d_k, int start_pos, const float *freqs, int half_dim);
/* fusedAttentionHeadF32 (float32_ops.go:190-235): q q_rows x d_k, k / v
 * k_rows x d_k; out rows at out + out_off. */
void ref_attention_head(const float *q, const float *k, const float *v, int q_rows, int d_k, int k_rows,
                        int causal, int cache_len, float *out, int out_off);
/*
 * forwardBlock's attention section (model_f32.go:398-466) for one layer:
 * q / k / v are the matmul outputs (seq_len x n_heads*d_k, seq_len x
 * n_kv*d_k); bias vectors (length q_bias_len ... or NULL), per-head QK RMSNorm
 * weights (d_k, or NULL; lib_norm: the library's sum-of-squares association),
 * RoPE at start_pos, then the rows are appended to the cache (cache_k /
 * cache_v: n_kv x cap x d_k, holding cache_len rows per head) and the causal
 * GQA attention of every head is written merged (seq_len x n_heads*d_k).
 * The bias adds modify q, k and v in place, as the reference's do; the
 * normed and rotated heads are copies, as the reference's split heads are.
 * q_rot (or NULL) receives the normed, rotated q heads (seq_len x
 * n_heads*d_k).
 */
void ref_attention_layer(float *q, float *k, float *v, int seq_len, int n_heads, int n_kv, int d_k,
                         const float *q_bias, int q_bias_len, const float *k_bias, int k_bias_len,
                         const float *v_bias, int v_bias_len, const float *q_norm_w, const float *k_norm_w,
                         float eps, int lib_norm, const float *freqs, int half_dim, int start_pos,
                         float *cache_k, float *cache_v, int cap, int cache_len, float *out, float *q_rot);

#ifdef __cplusplus
}
#endif

#endif
