/*
 * sllm_qmm.h — C ABI of the MI355X (gfx950) quantized-matmul library that
 * replaces scriptling-llm-lib's int8 matmul path.
 *
 * Every entry point names the reference function it stands in for
 * (paths relative to the reference repository root). All functions return an
 * sllm_status; on failure sllm_last_error() gives a message for the calling
 * thread. Nothing here aborts the process, and no entry point falls back to a
 * CPU path: a missing GPU is an error (SLLM_ERR_DEVICE).
 *
 * Threading: weight handles are immutable after creation and may be shared by
 * any number of threads; every matmul call is independent (the host-pointer
 * entry points draw a private HIP stream and staging buffers from a pool).
 *
 * Layout conventions (same as the reference): x is xRows x xCols fp32
 * row-major, dst is xRows x rows fp32 row-major (dst[xi*rows + j]), weights
 * are [rows][cols/32 blocks] with rows = GGUF Dims[1], cols = Dims[0].
 */
#ifndef SLLM_QMM_H
#define SLLM_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    SLLM_OK = 0,
    SLLM_ERR_ARG = 1,         /* null pointer, bad size, shape mismatch */
    SLLM_ERR_QTYPE = 2,       /* QType / GGUF type this path does not take */
    SLLM_ERR_SHAPE = 3,       /* cols not a multiple of the block size, or beyond limits */
    SLLM_ERR_DEVICE = 4,      /* no usable gfx950 device, or a HIP runtime error */
    SLLM_ERR_OOM = 5,         /* device or pinned-host allocation failed */
    SLLM_ERR_FORMAT = 6       /* Raw bytes not in the form the QType requires */
} sllm_status;

/* QType of a weight, as in QuantWeight.QType (gguf.go:73-79). */
typedef enum {
    SLLM_Q8_0 = 0,  /* "q8"   34 B / 32: f16 d, int8 q[32]                          */
    SLLM_Q4_0 = 1,  /* "q4"   18 B / 32: f16 d, 16 nibble bytes, w = d*(nib-8)        */
    SLLM_Q4_1 = 2,  /* "q4_1" 20 B / 32: f16 d, f16 m, 16 nibble bytes, w = d*nib+m   */
    SLLM_Q5_0 = 3,  /* "q5"   22 B / 32: f16 d, u32 qh, 16 nibble bytes, w = d*(q5-16)*/
    SLLM_Q5K1 = 4,  /* "q5k1" Q5_K as two summed Q4_1 tensors (kquant_kernels.go:103-154) */
    SLLM_Q2K = 5,   /* GGUF Q2_K kept native (84 B / 256); the reference loads it as dense fp32 */
    SLLM_Q3K = 6    /* GGUF Q3_K kept native (110 B / 256); the reference loads it as dense fp32 */
} sllm_qtype;

typedef struct sllm_weight sllm_weight;

/* Library set-up on the current HIP device; idempotent. Optional: every other
 * entry point initialises on first use. */
sllm_status sllm_init(void);

/* Message for the last failing call on this thread ("" if none). */
const char *sllm_last_error(void);

/*
 * The per-stream device workspace (no counterpart in the reference, whose
 * scratch comes from sync.Pools, q8q8.go:12-13): the _dev entry points keep
 * the prefill GEMM's activation codes and split partials, the attention's
 * q rows and split states and multi-row normed rows in a buffer owned by
 * (device, stream), grown on demand. Growth allocates, so it cannot happen
 * while the stream is being captured into a HIP graph (the call returns
 * SLLM_ERR_ARG, naming the size it needed): reserve at least that many bytes
 * with this call before capturing. A buffer that is outgrown is kept, not
 * freed, until the process ends, so graphs captured before a growth stay
 * valid. Growth at least doubles the buffer.
 */
sllm_status sllm_workspace_reserve(void *stream, size_t bytes);

/* Static description: arch, plane layout version, kernel configuration. */
const char *sllm_kernel_info(void);

/* --------------------------------------------------------------------------
 * Weight creation (load time). Each call repacks the block bytes once into
 * HBM-resident planes: quant plane(s), f16 scale plane, f16 min plane (Q4_1,
 * Q5K1), high-bit plane (Q5_0, Q5K1). The call is synchronous.
 * ------------------------------------------------------------------------ */

/*
 * From a QuantWeight as the reference holds it (gguf.go:73-79): qtype is the
 * QType string ("q8", "q4", "q4_1", "q5", "q5k1"), raw/raw_bytes its Raw bytes
 * in host memory, groups/rows/cols its fields. Replaces keeping QuantWeight.Raw
 * on the host for modelMatmulQuantIntoF32 (float32_ops.go:379).
 * "q5k1" Raw must be what convertQ5KToTwoQ41 produces (high half: min 0 and
 * 0/1 nibbles), else SLLM_ERR_FORMAT.
 */
sllm_status sllm_weight_from_quant(const char *qtype, const void *raw, size_t raw_bytes,
                                   int groups, int rows, int cols, sllm_weight **out);

/*
 * From a GGUF tensor (type id and its block bytes in host memory): the
 * int8-kernel branches of loadWeightF32Direct (gguf.go:818-934), run on the GPU.
 *   8 Q8_0, 2 Q4_0, 3 Q4_1, 6 Q5_0: repacked as is;
 *   12 Q4_K -> Q4_1 (convertQ4KToQ41, kquant_kernels.go:30-63);
 *   13 Q5_K -> Q5K1 (convertQ5KToTwoQ41, kquant_kernels.go:110-154);
 *   14 Q6_K, 20 IQ4_NL -> Q8_0 (dequantize in fp64 + quantizeQ8Rows,
 *      gguf.go:889-894,912-921,979-1015,1080-1134);
 *   10 Q2_K, 11 Q3_K -> kept native (SLLM_Q2K / SLLM_Q3K). The reference
 *      dequantizes these to dense fp32 (gguf.go:907-911, dequantizeQ2KNative /
 *      dequantizeQ3KNative kquants.go:147-245) and multiplies with the plain
 *      float32 loop (modelMatmulFloatIntoF32, float32_ops.go:462-482); the
 *      matmuls here rebuild each of those float32 weights exactly from the
 *      native blocks and multiply fp32 activations by them, so only the order
 *      of the row sums differs (no int8 activation codes for these types).
 * Other types return SLLM_ERR_QTYPE (the reference's dense-fp32 branch).
 */
sllm_status sllm_weight_from_gguf(uint32_t ggml_type, const void *raw, size_t raw_bytes,
                                  int rows, int cols, sllm_weight **out);

/*
 * From dense fp32 weights (host memory, rows x cols): Q8_0 via
 * quantizeQ8RowsF32 (gguf.go:1136-1186), as the tied output head is built
 * (model_f32.go:150-152).
 */
sllm_status sllm_weight_from_f32(const float *w, int rows, int cols, sllm_weight **out);

void sllm_weight_destroy(sllm_weight *w);

/* QuantWeight fields of a handle. */
sllm_status sllm_weight_info(const sllm_weight *w, int *qtype, int *groups, int *rows, int *cols,
                             size_t *raw_bytes);

/*
 * Bytes one decode GEMV of this weight streams from HBM (its planes as the
 * kernel reads them: the algorithmic weight bytes of a matmul). Q4_K weights
 * loaded while the load option "gemv_q4k_stream" is set keep the GGUF Q4_K
 * headers beside the Q4_1 planes (2 B more per 256 weights) and their decode
 * GEMV streams the Q4_1 nibbles and the headers, 18 B per 32 weights,
 * rebuilding each block's Q4_1 scale and min as convertQ4KToQ41 computes
 * them (kquant_kernels.go:30-63); other Q4_K weights stream the Q4_1 planes
 * (20 B), which measures faster (C3 gate + up: 15.7-16.6 against 14.2-14.6
 * us). No counterpart in the reference.
 */
sllm_status sllm_weight_stream_bytes(const sllm_weight *w, size_t *bytes);

/*
 * GGUF Q6_K weights loaded while the load option "gemv_q6k_stream" is set
 * keep their 6-bit codes beside the Q8_0 planes, so such a weight holds both
 * plane sets (about 62 B per 32 weights, 83 % more device memory than the
 * Q8_0 planes alone); for the life of the weight its decode GEMV streams the
 * 6-bit planes (28.25 B per 32 weights, against 34) and rebuilds the Q8_0
 * codes and scale in registers (VALU-bound: C3 down 24.2 against 12.4 us,
 * the 128256 x 4096 head 136 against 85 us), bit-identical to the Q8_0
 * planes the reference's load computes (dequantizeQ6KBlock + quantizeQ8Rows,
 * gguf.go:988-1015, 1080-1134). *blocks: the 32-element blocks it recomputes
 * with the reference's fp64 arithmetic (where the fast per-sub-block rule
 * cannot reproduce the rounding of exact ties), or -1 for a weight loaded
 * without those planes. No counterpart in the reference.
 */
sllm_status sllm_weight_q6k_exact_blocks(const sllm_weight *w, int64_t *blocks);

/*
 * *yes = 1 when the prefill GEMM computes this Q5K1 weight with one int8 MFMA
 * per block: every block's high-block scale is exactly 16 times its low scale
 * (convertQ5KToTwoQ41, kquant_kernels.go:127-144, writes f16(16 d sc) and
 * f16(d sc), so this holds unless 16 d sc overflows f16: d sc is a multiple of
 * 2^-24, exact in f16 below its normal range), and the two halves' terms of a
 * block are then one dot of
 * the 5-bit codes scaled by the low scale. 0 otherwise and for every other
 * format (the halves take one MFMA each). Decided at load. No counterpart in
 * the reference.
 */
sllm_status sllm_weight_q5k1_one_mfma(const sllm_weight *w, int *yes);

/*
 * Rebuild the reference Raw bytes (QuantWeight.Raw layout) from the device
 * planes into host memory (cap >= raw_bytes). Bit-exact inverse of the repack.
 * SLLM_Q2K / SLLM_Q3K: the GGUF super-block bytes the weight was made from.
 */
sllm_status sllm_weight_export(const sllm_weight *w, void *raw, size_t cap);

/* --------------------------------------------------------------------------
 * Matmul (decode GEMV for xRows < 64 tokens, int8-MFMA GEMM for xRows >= 64).
 * ------------------------------------------------------------------------ */

/*
 * modelMatmulQuantIntoF32 (float32_ops.go:379-460) for a handle: host x and
 * dst, synchronous (dst is filled when it returns). Covers q8q8MatmulInto
 * (q8q8.go:147), q4q8MatmulInto (q4q8.go:49), q41q8MatmulInto (q41q8.go:20),
 * q5k1MatmulInto (kquant_kernels.go:159) and the Q5_0 branch (:427-436).
 */
sllm_status sllm_matmul_quant_into_f32(const sllm_weight *w, const float *x, int x_rows, int x_cols,
                                       float *dst);

/* modelMatmulRowQuantIntoF32 (float32_ops.go:620-707): one activation row. */
sllm_status sllm_matmul_row_quant_into_f32(const sllm_weight *w, const float *normed, float *dst);

/*
 * Device-resident variant: x and dst are device pointers, work is enqueued on
 * `stream` (a hipStream_t; NULL = the default stream) and the call returns
 * without synchronising. May allocate device scratch on first use of a larger
 * shape (the stream's workspace, see sllm_workspace_reserve).
 */
sllm_status sllm_matmul_dev(const sllm_weight *w, const float *x_dev, int x_rows, int x_cols,
                            float *dst_dev, void *stream);

/*
 * Several weights applied to the same activation rows: the consecutive
 * modelMatmulIntoF32 calls of forwardBlock that share one input (q, k, v on
 * b.normed, model_f32.go:391-396; gate, up on b.ffnNormed, model_f32.go:479-482).
 * Equivalent to count calls of sllm_matmul_quant_into_f32 (dst[i] receives
 * x_rows x Rows(ws[i]) floats, bit-identical to the single call's result),
 * but decode GEMVs of weights with the same QType share one launch (up to
 * four weights each) and x is staged once. Every ws[i] must have
 * Cols == x_cols.
 */
sllm_status sllm_matmul_multi_quant_into_f32(const sllm_weight *const *ws, int count, const float *x,
                                             int x_rows, int x_cols, float *const *dst);

/* Device-resident form of sllm_matmul_multi_quant_into_f32 (see sllm_matmul_dev). */
sllm_status sllm_matmul_multi_dev(const sllm_weight *const *ws, int count, const float *x_dev, int x_rows,
                                  int x_cols, float *const *dst_dev, void *stream);

/*
 * forwardBlock's FFN input in one call (model_f32.go:479-490): gate = Wgate x,
 * up = Wup x (modelMatmulIntoF32 on b.ffnNormed) and then, elementwise,
 * h = gate * float32(1 / (1 + exp(-float64(gate)))) * up, the reference's
 * SwiGLU loop in its operation order. h receives x_rows x Rows floats. Below
 * the GEMM's row threshold (gemm_min_rows) and for weights of one QType this
 * is a single GEMV launch (half of each workgroup's waves stream gate rows,
 * the other half the same rows of up, and they meet in LDS) that writes h
 * directly; gate and up are not written unless gate_dev / up_dev are given
 * (each may be NULL). Wgate and Wup must have the same Rows and Cols == x_cols.
 */
sllm_status sllm_matmul_swiglu_dev(const sllm_weight *w_gate, const sllm_weight *w_up, const float *x_dev,
                                   int x_rows, int x_cols, float *h_dev, float *gate_dev, float *up_dev,
                                   void *stream);

/*
 * The RMSNorm in front of a layer's matmuls, fused into the GEMV prologue:
 * rmsNormFlatF32 (float32_ops.go:159-172) of each activation row with weight
 * vector norm_w_dev (x_cols floats) and eps, then the matmuls of
 * sllm_matmul_multi_dev / sllm_matmul_swiglu_dev / sllm_matmul_argmax_dev on
 * the normed rows (forwardBlock: model_f32.go:388-396 and 476-490;
 * outputLogits: model_f32.go:502-527). For one row (decode) the GEMV launch
 * computes the row statistic itself, so no normed vector goes through memory;
 * several rows are normed into the workspace first by a standalone kernel
 * with the same statistics. inv = 1 / float32(sqrt(
 * float64(ss) / cols + float64(eps))) and normed = (x * inv) * w as in the
 * reference; the sum of squares ss is added in a fixed order of the library's
 * (256 strided partial sums, then a fixed tree) rather than the reference's
 * single sequential loop, so only its association differs. x_dev and
 * norm_w_dev must be 16-byte aligned.
 */
sllm_status sllm_rmsnorm_matmul_multi_dev(const sllm_weight *const *ws, int count, const float *x_dev,
                                          const float *norm_w_dev, float eps, int x_rows, int x_cols,
                                          float *const *dst_dev, void *stream);
sllm_status sllm_rmsnorm_matmul_swiglu_dev(const sllm_weight *w_gate, const sllm_weight *w_up, const float *x_dev,
                                           const float *norm_w_dev, float eps, int x_rows, int x_cols,
                                           float *h_dev, void *stream);
sllm_status sllm_rmsnorm_matmul_argmax_dev(const sllm_weight *w, const float *x_dev, const float *norm_w_dev,
                                           float eps, int x_cols, float *logits_dev, int *argmax_dev,
                                           void *stream);

/*
 * The matmul followed by the residual add: dst += x W^T (device buffers,
 * dst x_rows x Rows). Replaces modelMatmulIntoF32(WO) + `xData[i] +=
 * oData[i]` (model_f32.go:469-474) and modelMatmulIntoF32(WDown) + `xData[i]
 * += downData[i]` (model_f32.go:492-497): the product is the one
 * sllm_matmul_dev computes, then one float32 add per element, as in the
 * reference. Decode adds in the GEMV's epilogue.
 */
sllm_status sllm_matmul_add_dev(const sllm_weight *w, const float *x_dev, int x_rows, int x_cols,
                                float *dst_dev, void *stream);

/* --------------------------------------------------------------------------
 * The attention section of a step (forwardBlock, model_f32.go:398-466) on
 * the device, with every layer's KV cache resident in HBM.
 * ------------------------------------------------------------------------ */

/*
 * KVCacheF32 (float32_ops.go:11-14) for n_layers layers: K and V rows of
 * n_kv_heads heads, d_k floats each, up to max_seq positions per layer
 * (InferenceModelF32.KVCaches, initKVCaches model_f32.go:310-318; the
 * reference appends without bound, MaxSeqLen caps the context,
 * model_f32.go:599-602). Layout: layer-major, then head, position, d_k
 * (fp32, as the reference keeps it). d_k: a multiple of 4, at most 256;
 * max_seq x d_k x 4 bytes (one kv head of one layer) below 4 GiB.
 */
typedef struct sllm_kv_cache sllm_kv_cache;
sllm_status sllm_kv_cache_create(int n_layers, int n_kv_heads, int d_k, int max_seq, sllm_kv_cache **out);
void sllm_kv_cache_destroy(sllm_kv_cache *kv);
/* Rows held by a layer (len(cache.K[h]) / dK in the reference). */
sllm_status sllm_kv_cache_length(const sllm_kv_cache *kv, int layer, int *len);
/* Every layer back to (or forward to) len rows: 0 starts a new sequence, as
 * initKVCaches does when Generate starts at kvStartPos 0
 * (model_f32.go:589-591). Rows beyond len keep their contents. */
sllm_status sllm_kv_cache_set_length(sllm_kv_cache *kv, int len);
/* Device addresses of layer's K and V (n_kv_heads x max_seq x d_k each). */
sllm_status sllm_kv_cache_data(const sllm_kv_cache *kv, int layer, float **k_dev, float **v_dev);

/* The model constants of the attention section (device pointers to the
 * model's own tensors; NULL / 0 where the model has none). */
typedef struct sllm_attn_params {
    int n_heads;            /* m.nHeads */
    int n_kv_heads;         /* m.nKVHeads (n_heads = n_kv_heads * nRep, nRep <= 8) */
    int d_k;                /* m.dK */
    int rope_half_dim;      /* m.ropeHalfDim (<= d_k / 2) */
    const float *rope_freqs; /* m.ropeFreqs, rope_half_dim floats (model_f32.go:256-260) */
    const float *q_bias;    /* block.QBias */
    int q_bias_len;
    const float *k_bias;    /* block.KBias */
    int k_bias_len;
    const float *v_bias;    /* block.VBias */
    int v_bias_len;
    const float *q_norm_w;  /* block.QNormW (d_k floats) */
    const float *k_norm_w;  /* block.KNormW (d_k floats) */
    float norm_eps;         /* Config.NormEps */
} sllm_attn_params;

/*
 * forwardBlock's attention section for `layer` (model_f32.go:398-466): q_dev
 * (seq_len x n_heads*d_k), k_dev and v_dev (seq_len x n_kv_heads*d_k) are the
 * q/k/v matmul outputs. Adds the biases, RMSNorms each q / k head with
 * QNormW / KNormW, applies RoPE at positions start_pos + r
 * (applyRopeInPlaceF32, float32_ops.go:174-188), appends the k / v rows to
 * the layer's cache, and writes the causal attention of every q head over
 * the cache (q head h reads kv head h / nRep; fusedAttentionHeadF32,
 * float32_ops.go:190-235) to out_dev, heads merged (seq_len x n_heads*d_k,
 * mergeHeadsDataF32 float32_ops.go:262-273). q/k/v are not modified.
 * Scores are the reference's sequential float32 dots; the softmax sums and
 * the weighted sum of values are reassociated (split over the positions and
 * combined), and the per-head RMSNorm sums its squares in the library's
 * fixed order. One row (decode): two launches (the attention over splits of
 * the cached positions, which also prepares the row, then the combine of the
 * splits); several rows: three (the row preparation first). Asynchronous on
 * `stream`; allocates nothing once the stream's workspace has grown to the
 * call's size.
 */
sllm_status sllm_attention_dev(sllm_kv_cache *kv, int layer, const sllm_attn_params *p, const float *q_dev,
                               const float *k_dev, const float *v_dev, int seq_len, int start_pos,
                               float *out_dev, void *stream);

/*
 * No counterpart in the reference. For callers that cannot allocate device
 * memory: code under HIP graph capture (without a warm-up call on the
 * stream), serving loops and harnesses that forbid hipMalloc. The same
 * attention as sllm_attention_dev (same kernels, bit-identical outputs), but
 * its scratch - the rotated q rows and the split states - lives in a static
 * 8 MiB device array per GPU, held until the process ends, so the call
 * allocates nothing and never touches the stream's workspace. Calls that
 * need more scratch than that (about seq_len x n_heads x (d_k x 4 bytes) for
 * the q rows, plus the split states of long caches; a decode step of a
 * 64-head model at 8K positions needs about 2 MiB) return SLLM_ERR_SHAPE.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (different streams, or graph replays running concurrently) race and
 * give wrong results; serialize them.
 */
sllm_status sllm_attention_noalloc_dev(sllm_kv_cache *kv, int layer, const sllm_attn_params *p,
                                       const float *q_dev, const float *k_dev, const float *v_dev, int seq_len,
                                       int start_pos, float *out_dev, void *stream);

/* Host-buffer form of sllm_matmul_swiglu_dev (synchronous; h only). */
sllm_status sllm_matmul_swiglu_into_f32(const sllm_weight *w_gate, const sllm_weight *w_up, const float *x,
                                        int x_rows, int x_cols, float *h);

/*
 * The output head and greedy sampling in one launch: modelMatmulRowQuantIntoF32
 * of one activation row (outputLogits, model_f32.go:521) followed by argmaxF32
 * (float32_ops.go:812-822) of the logits: the first index of the maximum, NaN
 * values never winning, and 0 if logits[0] is NaN. *argmax_dev (device int)
 * receives the index; logits_dev (may be NULL) the logits. Needs
 * x_cols == Cols. Launches on the same stream are serialized; launches on
 * different streams each use their own 64-byte scratch (allocated by the
 * first call on a stream, which therefore must not be under capture). A HIP
 * graph captured on stream S keeps S's scratch wherever it is replayed: a
 * replay must not overlap an argmax launch on S, nor a replay of another
 * graph captured on S (the shared counter would misfire).
 * Ordering assumption: the workgroups combine their maxima with device-scope
 * relaxed atomics and no fence (a fence writes back and invalidates the L2 of
 * each XCD). The last workgroup to count reads every maximum because a
 * device-scope read-modify-write whose old value has returned has been
 * performed at the device's coherence point, and each workgroup counts only
 * after its maximum has returned. This holds on gfx950 (the argmax tests
 * check ties, NaN rules, repeated launches, two streams and graph replays)
 * but is not promised by the HIP memory model for relaxed atomics.
 */
sllm_status sllm_matmul_argmax_dev(const sllm_weight *w, const float *x_dev, int x_cols, float *logits_dev,
                                   int *argmax_dev, void *stream);

/* Host-buffer form: normed in, the greedy token out (4 bytes read back, not the logits). */
sllm_status sllm_matmul_argmax(const sllm_weight *w, const float *normed, int *token);

/* argmaxF32 (float32_ops.go:812-822) over n device floats; result to host. */
sllm_status sllm_argmax_dev(const float *v_dev, int n, int *out, void *stream);

/* --------------------------------------------------------------------------
 * Verification entry points (bit-exact checks; not on the hot path).
 * ------------------------------------------------------------------------ */

/* quantizeActivationsQ8 (q8q8.go:96-125) on the GPU, with the same device
 * routine the matmul prologue uses. Host buffers: x [rows*cols], xq
 * [rows*cols], xs [rows*cols/32], sum_xq [rows*cols/32] (may be NULL). */
sllm_status sllm_debug_quantize_act(const float *x, int rows, int cols, int8_t *xq, float *xs,
                                    int32_t *sum_xq);

/*
 * Per-(activation row, weight row, block) integer dots computed by the same
 * device block routines as the matmul: out is int32 [x_rows][rows][groups]
 * (x2 in the last dimension for Q5K1: low, high). For Q5_0 (fp32 activations)
 * each entry is the fp32 in-block partial sum's bit pattern.
 */
sllm_status sllm_debug_block_dots(const sllm_weight *w, const float *x, int x_rows, int x_cols,
                                  int32_t *out);

/*
 * The prefill GEMM's own block dots: runs the int8 matrix-core GEMM (the
 * kernel sllm_matmul uses from gemm_min_rows activation rows on) on x_rows
 * (>= 1) rows against weight rows [row0, row0 + n_rows), and writes every
 * int32 block dot its MFMA instructions returned, from the registers its
 * epilogue scales: out int32 [x_rows][n_rows][groups] (x2 for Q5K1: low,
 * high). Q4_0 entries include the -8 Σxq zero-point term, as
 * sllm_debug_block_dots. Formats Q8_0, Q4_0, Q4_1, Q5K1 (cols a multiple of
 * 64); others SLLM_ERR_QTYPE. Replaces no reference interface: the
 * reference forms the same per-(row, block) dots in q8q8.go:156-195,
 * q4q8.go:58-77 and q41q8.go:31-52.
 */
sllm_status sllm_debug_gemm_block_dots(const sllm_weight *w, const float *x, int x_rows, int x_cols,
                                       int row0, int n_rows, int32_t *out);

/*
 * Launch-shape knobs (no counterpart in the reference: its matmuls have no
 * launch shapes). Process-wide; set them before the calls they should
 * affect, not while other threads are launching. Results do not depend on
 * any of them except where noted. Unknown names or values: SLLM_ERR_ARG.
 *   gemv_waves          4, 8, 16   most waves per GEMV workgroup (16)
 *   gemv_wg_per_cu      1..8       GEMV workgroups per CU (1)
 *   gemv_max_nb         1..8       most 32-element blocks per lane per unit (8)
 *   gemv_inflight_kb    >= 64      weight bytes in flight over the device (32768)
 *   gemv_q4k_stream     0, 1       load option: Q4_K weights created while it is 1 keep
 *                                  their GGUF headers and their GEMV streams them (0; see
 *                                  sllm_weight_stream_bytes)
 *   gemv_q6k_stream     0, 1       load option: Q6_K weights created while it is 1 keep
 *                                  their 6-bit codes and their GEMV streams them (0; see
 *                                  sllm_weight_q6k_exact_blocks)
 *                                  (a weight's plane layout, and so its GEMV kernel, is
 *                                  fixed when it is created: these two never act on the
 *                                  call path)
 *   gemm_min_rows       >= 0       activation rows from which the GEMM is used (0: 8 for
 *                                  weights of 2^24 elements or more, 16 for smaller ones;
 *                                  the GEMM and GEMV sum a row's blocks in different
 *                                  orders, so a row's last bits can change with it)
 *   gemm_shape          0..5       GEMM workgroups: 1 = 64 x 128 tiles, 2 = 64 x 64 tiles with
 *                                  each K stage split over two waves, 3 = as 2 with two
 *                                  stages of loads in flight, 4 = 32 x 64 tiles with each
 *                                  stage split over four waves, 5 = as 1 with two stages of
 *                                  loads in flight (0: 1, above 128 rows 5; for Q5K1 3,
 *                                  and 4 up to 32 rows; for Q5K1 in one MFMA per block,
 *                                  see sllm_weight_q5k1_one_mfma, 4 up to 32 rows, 2 up
 *                                  to 128, else 1); Q5_0: 1 = 64 x 256
 *                                  tiles, 2 = 64 x 128 (0: 2 up to 4096 weight rows and
 *                                  128 activation rows, else 1). The shape moves the fp32
 *                                  summation splits
 *   gemm_splits         0..64      GEMM K splits, added in split order (0: by tile count;
 *                                  the split count moves the fp32 summation splits)
 *   attn_target_blocks  1..65536   attention: about this many workgroups when splitting (512)
 *   attn_tile_groups    1..4       attention: most tile groups per workgroup (4)
 *   attn_head_slices    0..64      attention: workgroups sharing a kv head's q heads
 *                                  (0: while the grid has fewer workgroups than CUs)
 * The attention knobs move the summation splits of the softmax except
 * attn_head_slices, whose results are bit-identical for any value.
 */
sllm_status sllm_set_param(const char *name, int value);

#ifdef __cplusplus
}
#endif
#endif
