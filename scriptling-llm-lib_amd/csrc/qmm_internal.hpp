// Host-side definitions shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "sllm_qmm.h"

namespace sllm {

// Device planes of one weight. Every plane is [rows][groups] in block order,
// rows contiguous, each plane 256-byte aligned inside one allocation.
//   qs   16 B / block: Q8_0 elements 0..15 (int8); Q4_0 / Q4_1 / Q5_0 / Q5K1 the
//        16 GGUF nibble bytes (byte i = element i low nibble | element i+16 high)
//   qs2  16 B / block: Q8_0 elements 16..31
//   d    f16 scale bits           (all formats)
//   m    f16 min bits             (Q4_1, Q5K1 low block)
//   dh   f16 scale of the Q5K1 high block (16 * d*sc, truncated separately)
//   qh   u32 high bits, bit e = bit 4 of element e (Q5_0, Q5K1); Q3K: bit e =
//        the high-mask bit of element e
// Native k-quants (Q2K, Q3K), per 32-element block b of a super-block (two
// 16-element sub-blocks):
//   q2   8 B: the 2-bit codes in element order (x: elements 0..15, y: 16..31,
//        element l at bits 2l)
//   d    u16: the two sub-blocks' scale bytes (Q2K: sc | m << 4 as stored;
//        Q3K: the decoded 6-bit scales minus 32, as int8)
//   sb   u32 per super-block: Q2K d | dmin << 16, Q3K d (f16 bits)
//   hdr  16 B per super-block (Q4_K streamed natively): the GGUF Q4_K header
//        (d, dmin, the 12 packed scale bytes), next to the Q4_1 planes
// Q6_K streamed natively (SLLM_Q6K_STREAM), next to the Q8_0 planes: l6 / h6
// the 6-bit codes (16 + 8 B), m6 the block's scales, code maximum and flags,
// d6 the super-block's f16 d (qmm_q6k.hpp has the layout); q6stat two
// counters the pack fills: blocks left to the fp64 path, self-check failures.
struct Planes {
    const int4 *qs = nullptr;
    const int4 *qs2 = nullptr;
    const uint16_t *d = nullptr;
    const uint16_t *m = nullptr;
    const uint16_t *dh = nullptr;
    const uint32_t *qh = nullptr;
    const uint2 *q2 = nullptr;
    const uint32_t *sb = nullptr;
    const int4 *hdr = nullptr;
    const int4 *l6 = nullptr;
    const uint2 *h6 = nullptr;
    const uint32_t *m6 = nullptr;
    const uint16_t *d6 = nullptr;
};

struct MutPlanes {
    int4 *qs = nullptr;
    int4 *qs2 = nullptr;
    uint16_t *d = nullptr;
    uint16_t *m = nullptr;
    uint16_t *dh = nullptr;
    uint32_t *qh = nullptr;
    uint2 *q2 = nullptr;
    uint32_t *sb = nullptr;
    int4 *hdr = nullptr;
    int4 *l6 = nullptr;
    uint2 *h6 = nullptr;
    uint32_t *m6 = nullptr;
    uint16_t *d6 = nullptr;
    uint32_t *q6stat = nullptr;
};

// Kernel format of a Q4_K weight streamed natively: the Q4_1 nibble plane plus
// the GGUF header per super-block (18 B / 32 weights); the Q4_1 scale and min
// of each block are rebuilt in the kernel (convertQ4KToQ41's arithmetic).
// Internal only: such a weight is a "q4_1" QuantWeight at the ABI (its d / m
// planes serve the GEMM and the export).
constexpr int SLLM_Q4K_STREAM = 7;
// Kernel format of a Q6_K weight streamed natively: the 6-bit codes and the
// per-block scale data, the Q8_0 codes rebuilt in registers (qmm_q6k.hpp).
// Internal only: such a weight is a "q8" QuantWeight at the ABI, and its Q8_0
// planes, kept beside the stream's, serve the GEMM and the export.
constexpr int SLLM_Q6K_STREAM = 8;
// GEMM format of a Q5K1 weight whose high-block scale is 16 times its low
// scale in every block (as convertQ5KToTwoQ41 writes them unless 16 d sc
// overflows f16): its codes are staged as the 5-bit q5 = nib + 16 *
// bit, one MFMA per block, whose dot scaled by the low scale is the two halves'
// terms together. Internal only (the weight is a "q5k1" QuantWeight).
constexpr int SLLM_Q5K1F = 9;

// Formats whose activations stay fp32 (no Q8_0 codes): Q5_0 and the native k-quants.
__host__ __device__ constexpr bool act_f32(int fmt) {
    return fmt == SLLM_Q5_0 || fmt == SLLM_Q2K || fmt == SLLM_Q3K;
}
// Native k-quant formats (256-element super-blocks).
__host__ __device__ constexpr bool kq_native(int fmt) { return fmt == SLLM_Q2K || fmt == SLLM_Q3K; }

// Bytes each format streams per 32-element block from the planes.
inline int plane_block_bytes(int fmt) {
    switch (fmt) {
    case SLLM_Q8_0: return 34;
    case SLLM_Q4_0: return 18;
    case SLLM_Q4_1: return 20;
    case SLLM_Q5_0: return 22;
    case SLLM_Q5K1: return 26;
    case SLLM_Q4K_STREAM: return 18;  // 16 + 16 / 8
    case SLLM_Q6K_STREAM: return 29;  // 28.25: 16 + 8 + 4 + 2 / 8 (rounded up)
    case SLLM_Q2K: return 11;  // 10.5: 8 + 2 + 4 / 8 (rounded up)
    case SLLM_Q3K: return 15;  // 14.5: 8 + 4 + 2 + 4 / 8 (rounded up)
    }
    return 0;
}

// Bytes one GEMV streams from the planes of nb blocks (the algorithmic weight bytes).
inline size_t stream_bytes_of(int fmt, int64_t nb) {
    if (fmt == SLLM_Q2K) return (size_t)nb * 10 + (size_t)(nb / 8) * 4;
    if (fmt == SLLM_Q3K) return (size_t)nb * 14 + (size_t)(nb / 8) * 4;
    if (fmt == SLLM_Q4K_STREAM) return (size_t)nb * 16 + (size_t)(nb / 8) * 16;
    if (fmt == SLLM_Q6K_STREAM) return (size_t)nb * 28 + (size_t)(nb / 8) * 2;
    return (size_t)nb * plane_block_bytes(fmt);
}

// Bytes the reference's Raw (or, native k-quants, the GGUF blocks) takes for
// nb 32-element blocks.
inline size_t raw_bytes_of(int fmt, int64_t nb) {
    if (fmt == SLLM_Q2K) return (size_t)(nb / 8) * 84;
    if (fmt == SLLM_Q3K) return (size_t)(nb / 8) * 110;
    switch (fmt) {
    case SLLM_Q8_0: return (size_t)nb * 34;
    case SLLM_Q4_0: return (size_t)nb * 18;
    case SLLM_Q4_1: return (size_t)nb * 20;
    case SLLM_Q5_0: return (size_t)nb * 22;
    case SLLM_Q5K1: return (size_t)nb * 40;
    }
    return 0;
}

// Bytes per block of the reference Raw layout (QuantWeight.Raw).
inline int raw_block_bytes(int fmt) {
    switch (fmt) {
    case SLLM_Q8_0: return 34;
    case SLLM_Q4_0: return 18;
    case SLLM_Q4_1: return 20;
    case SLLM_Q5_0: return 22;
    case SLLM_Q5K1: return 40;
    }
    return 0;
}

// Spare blocks at the end of every plane (the GEMV reads whole 64-block lane
// groups and may run up to 8 x 64 blocks past the last row's end).
constexpr int kPlanePadBlocks = 8 * 64;

// Carve the planes of a (rows x groups) weight of format fmt out of `base`
// (nullptr: only compute the size). Returns the total allocation size.
size_t carve_planes(int fmt, int64_t nblocks, void *base, MutPlanes *out);

inline Planes as_const(const MutPlanes &p) {
    Planes c;
    c.qs = p.qs; c.qs2 = p.qs2; c.d = p.d; c.m = p.m; c.dh = p.dh; c.qh = p.qh;
    c.q2 = p.q2; c.sb = p.sb; c.hdr = p.hdr;
    c.l6 = p.l6; c.h6 = p.h6; c.m6 = p.m6; c.d6 = p.d6;
    return c;
}

// Thread-local error message plumbing.
sllm_status set_error(sllm_status st, const std::string &msg);
sllm_status hip_error(hipError_t e, const char *what);

#define SLLM_HIP(call)                                             \
    do {                                                           \
        hipError_t e_ = (call);                                    \
        if (e_ != hipSuccess) return ::sllm::hip_error(e_, #call); \
    } while (0)

// Kernel launch helpers implemented in the .hip files.
sllm_status launch_gemv(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M,
                        hipStream_t s);
// One GEMV launch over up to kMaxSegs weights of one format and one K that
// share the activation rows x: weight i (N[i] rows) writes dst[i] (M x N[i]).
constexpr int kMaxSegs = 4;
// norm_w (optional): RMSNorm each activation row first (rmsNormFlatF32,
// float32_ops.go:159-172, with weight vector norm_w and eps), fused into the
// GEMV prologue.
sllm_status launch_gemv_multi(int fmt, const Planes *P, float *const *dst, const int *N, int nseg,
                              const float *x, int G, int M, hipStream_t s, const float *norm_w = nullptr,
                              float eps = 0.0f);
// Paired gate / up GEMV of one FFN: h = SwiGLU(Wg x, Wu x) (model_f32.go:479-490);
// gate / up (may be null) also receive the two matmul outputs. Both weights
// have the same format, N rows and G blocks per row.
sllm_status launch_gemv_swiglu(int fmt, const Planes &Pg, const Planes &Pu, const float *x, float *h,
                               float *gate, float *up, int N, int G, int M, hipStream_t s,
                               const float *norm_w = nullptr, float eps = 0.0f);
// One-row GEMV that also writes the greedy argmax of its outputs to *out
// (device). logits may be null. key / cnt: 16 bytes of zeroed per-stream
// scratch, left zeroed again by every launch.
sllm_status launch_gemv_argmax(int fmt, const Planes &P, const float *x, float *logits, int N, int G,
                               unsigned long long *key, unsigned int *cnt, int *out, hipStream_t s,
                               const float *norm_w = nullptr, float eps = 0.0f);
// dst (M x N) += the GEMV's result: the residual add that follows the o and
// down matmuls (model_f32.go:472-474, 495-497), in the GEMV epilogue.
sllm_status launch_gemv_add(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M,
                            hipStream_t s);
// dst[i] += src[i] for n elements (the GEMM path of the residual add).
sllm_status launch_add(float *dst, const float *src, size_t n, hipStream_t s);
// rmsNormFlatF32 of rows x K into out (the prefill path of the fused-norm
// entry points; same statistics as the GEMV prologue).
sllm_status launch_rmsnorm(const float *x, const float *norm_w, float eps, int rows, int K, float *out,
                           hipStream_t s);
// h[i] = SwiGLU(gate[i], up[i]) for n elements (the prefill path and mixed formats).
sllm_status launch_swiglu(const float *gate, const float *up, float *h, size_t n, hipStream_t s);
sllm_status launch_gemm(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M,
                        void *ws, size_t ws_bytes, hipStream_t s);
// The same GEMM that also writes every int32 block dot its matrix cores
// produce to dots [M][N][G] (x2 for Q5K1: low, high); int8 formats only.
sllm_status launch_gemm_dots(int fmt, const Planes &P, const float *x, float *dst, int N, int G, int M,
                             void *ws, size_t ws_bytes, int32_t *dots, hipStream_t s);
size_t gemm_workspace_bytes(int fmt, int N, int G, int M);
bool gemm_supported(int fmt, int G);  // Q5_0 and K not a multiple of 128 stay on the GEMV
sllm_status launch_quantize_act(const float *x, int rows, int G, int8_t *xq, float *xs, int32_t *sx,
                                hipStream_t s);
sllm_status launch_block_dots(int fmt, const Planes &P, const float *x, int N, int G, int M,
                              int32_t *out, hipStream_t s);
sllm_status launch_argmax(const float *v, int n, int *out_dev, hipStream_t s);

// Weight creation kernels: raw (device) -> planes.
sllm_status pack_from_raw(int fmt, const uint8_t *raw_dev, int rows, int G, const MutPlanes &P,
                          int *err_flag_dev, hipStream_t s);
sllm_status pack_from_gguf(uint32_t ggml_type, const uint8_t *raw_dev, int rows, int cols,
                           const MutPlanes &P, hipStream_t s);
sllm_status pack_from_f32(const float *w_dev, int rows, int cols, const MutPlanes &P, hipStream_t s);
// GGUF Q6_K -> the Q8_0 planes and the streamed Q6_K planes (P.q6stat zeroed
// by the caller; the pack counts into it).
sllm_status pack_q6k_stream(const uint8_t *raw_dev, int rows, int cols, const MutPlanes &P, hipStream_t s);
// *bad_dev (cleared by the caller) set unless every block of a Q5K1 weight's
// planes has dh = 16 d: the condition for the GEMM's one-MFMA form.
sllm_status check_q5k1_one_mfma(const MutPlanes &P, int64_t nb, int *bad_dev, hipStream_t s);
// GGUF super-block bytes of a native k-quant weight from its (host copy of the) planes.
void export_kq_native(int fmt, const MutPlanes &p, int64_t nb, uint8_t *out);

// The attention section of one layer (forwardBlock, model_f32.go:398-466) on
// device buffers; launch_attention checks nothing (the C entry does).
struct AttnArgs {
    const float *q, *k, *v;  // matmul outputs: seq x n_heads*d_k, seq x n_kv*d_k
    int seq, n_heads, n_kv, d_k, rep;
    const float *q_bias, *k_bias, *v_bias;  // or null
    int qb_len, kb_len, vb_len;
    const float *q_norm, *k_norm;  // per-head RMSNorm weights (d_k) or null
    float eps;
    const float *freqs;  // RoPE frequencies (half_dim)
    int half_dim, start_pos;
    float *cache_k, *cache_v;  // this layer: n_kv x cap x d_k
    int cap, cache_len;        // rows held before this call
    float scale;               // 1 / float32(sqrt(float64(d_k)))
    float *out;                // seq x n_heads*d_k (merged heads)
    float *qrot;               // workspace: seq x n_heads x d_k
    float *part;               // workspace: seq x n_heads x splits x (d_k + 2)
    int splits, tps, tw;       // splits per (row, kv head); tile groups per split; tiles of 64 positions per group
    int hs;                    // head slices: workgroups per (split, row, kv head), rep / hs q heads each
    int row0;                  // first query row of a split-kernel launch (long prefills run in row chunks)
};
// Split plan and workspace bytes (qrot + partials) of an attention call.
void attention_plan(int seq, int n_heads, int n_kv, int d_k, int kv_len, int *splits, int *tps, int *tw, int *hs,
                    size_t *ws_bytes);
sllm_status launch_attention(const AttnArgs &a, hipStream_t s);

// Tuning parameters (launch shapes), settable through sllm_set_param.
struct Tuning {
    int gemv_waves = 16;       // waves per GEMV workgroup (4, 8 or 16); fewer for small row counts
    int gemv_wg_per_cu = 1;    // GEMV workgroups per CU (persistent grid = CUs x this)
    int gemv_max_nb = 8;       // max blocks per lane in one GEMV unit (K-chunk)
    int gemv_inflight_kb = 32768;  // weight bytes in flight over the device (ring depth)
    int gemm_min_rows = 0;     // xRows at which the MFMA GEMM takes over (0: 8, or 16 below 2^24 weights)
    int gemm_shape = 0;        // GEMM workgroup shape (1..5; 0: by format and rows)
    int gemm_splits = 0;       // GEMM K splits (0: by tile count)
    int gemv_q4k_stream = 0;   // load option: Q4_K weights keep (and stream) the GGUF headers (1) or not (0, faster)
    int gemv_q6k_stream = 0;   // load option: Q6_K weights keep (and stream) the native 6-bit planes (1) or not (0)
    int attn_target_blocks = 512;  // attention: splits chosen to give about this many workgroups
    int attn_tile_groups = 4;      // attention: most tile groups (of max(4, rep) waves) per workgroup
    int attn_head_slices = 0;      // attention: workgroups sharing one kv head's q heads (0: by workgroup count)
};
Tuning &tuning();

}  // namespace sllm
