// The attention section of a decode / prefill step (forwardBlock,
// model_f32.go:398-466) on device buffers: bias adds, per-head QK RMSNorm,
// RoPE, the KV-cache append and the causal GQA attention with merged heads.
//
// attn_prep_kernel: one wave per (row, head) - bias, norm and RoPE of a q
//   head into the workspace, of a kv head into the cache (v: bias only).
// attn_kernel: one workgroup per (split, row, kv head). A split is a range
//   of cached positions in tiles of 64 (one per lane); the workgroup stages a
//   tile's K rows in LDS once for all q heads of the group (GQA: the kv head
//   is read from HBM once), each wave owns one or two q heads. Scores are the
//   reference's sequential float32 dots; the softmax runs online over the
//   tiles; the last workgroup of a (row, kv head) combines the splits.
#include <hip/hip_runtime.h>

#include <cmath>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

namespace sllm {

namespace {

constexpr int kTile = 64;     // positions per tile: one per lane
constexpr int kChunk = 128;   // K columns staged per pass (LDS: 64 x 132 floats)
constexpr int kMaxDk = 256;   // head size limit (o: 4 values per lane)
constexpr int kTargetBlocks = 512;

__device__ __forceinline__ float lane_bcast(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Bias (model_f32.go:398-420), per-head RMSNorm (:424-435; rmsNormFlatF32,
// float32_ops.go:159-172, the sum of squares in the library's association:
// slot s < 256 adds x[s]^2, x[s+256]^2, ..., the four groups of 64 slots are
// wave sums added left to right), RoPE (applyRopeInPlaceF32, float32_ops.go:
// 174-188) and the cache append (:445-448).
__global__ void __launch_bounds__(64) attn_prep_kernel(AttnArgs a) {
    __shared__ float row[kMaxDk];
    const int s = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const bool isq = t < a.n_heads;
    const int h = isq ? t : t - a.n_heads;
    const int dk = a.d_k;
    const int cols = (isq ? a.n_heads : a.n_kv) * dk;
    const float *src = (isq ? a.q : a.k) + (size_t)s * cols + (size_t)h * dk;
    const float *bias = isq ? a.q_bias : a.k_bias;
    const int blen = isq ? a.qb_len : a.kb_len;
    const float *nw = isq ? a.q_norm : a.k_norm;
    for (int d = lane; d < dk; d += 64) {
        float x = src[d];
        const int j = h * dk + d;
        if (bias && j < blen) x = x + bias[j];
        row[d] = x;
    }
    __syncthreads();
    if (nw) {
        float w[4];
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            float p = 0.0f;
            for (int i = q4 * 64 + lane; i < dk; i += 256) p = p + row[i] * row[i];
            w[q4] = wave_sum(p);
        }
        const float ss = ((w[0] + w[1]) + w[2]) + w[3];
        const float inv = 1.0f / (float)sqrt((double)ss / (double)dk + (double)a.eps);
        __syncthreads();
        for (int d = lane; d < dk; d += 64) row[d] = (row[d] * inv) * nw[d];
        __syncthreads();
    }
    const int pos = a.start_pos + s;
    for (int i = lane; i < a.half_dim; i += 64) {
        const float ang = a.freqs[i] * (float)pos;
        double sd, cd;
        sincos((double)ang, &sd, &cd);
        const float c = (float)cd, sn = (float)sd;
        const float x0 = row[2 * i], x1 = row[2 * i + 1];
        row[2 * i] = x0 * c - x1 * sn;
        row[2 * i + 1] = x0 * sn + x1 * c;
    }
    __syncthreads();
    if (isq) {
        float *dst = a.qrot + ((size_t)s * a.n_heads + h) * dk;
        for (int d = lane; d < dk; d += 64) dst[d] = row[d];
    } else {
        const size_t at = ((size_t)h * a.cap + (size_t)(a.cache_len + s)) * dk;
        const float *vs = a.v + (size_t)s * cols + (size_t)h * dk;
        for (int d = lane; d < dk; d += 64) {
            a.cache_k[at + d] = row[d];
            float x = vs[d];
            const int j = h * dk + d;
            if (a.v_bias && j < a.vb_len) x = x + a.v_bias[j];
            a.cache_v[at + d] = x;
        }
    }
}

// fusedAttentionHeadF32 (float32_ops.go:190-235) for the q heads of one kv
// head (repeatKVDataF32, float32_ops.go:252-260: q head g*rep + r reads kv
// head g) and one query row, over one split of the positions the causal mask
// leaves (0 .. cache_len + qi). Score = (sequential float32 dot) * scale, as
// the reference computes it; the exponentials are float32(exp(float64(score
// - running max))), rescaled by the same form when the running max grows, and
// the splits are combined with weights float32(exp(float64(m_split - max))).
// Against the reference's single pass (exps relative to the global max, one
// sequential sum, terms (e * invSum) * v) only the association of the sums
// and these rescalings differ.
__global__ void __launch_bounds__(256) attn_kernel(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) float kt[];  // kTile x (kChunk + 4)
    __shared__ int last;
    constexpr int ks = kChunk + 4;
    const int split = blockIdx.x;
    const int qi = blockIdx.y / a.n_kv, g = blockIdx.y - qi * a.n_kv;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int dk = a.d_k;
    const int limit = a.cache_len + qi + 1;
    const int p0 = split * a.tps * kTile;
    const int p1 = min(p0 + a.tps * kTile, limit);
    const float *kb = a.cache_k + (size_t)g * a.cap * dk;
    const float *vb = a.cache_v + (size_t)g * a.cap * dk;
    const float *qg = a.qrot + ((size_t)qi * a.n_heads + (size_t)g * a.rep) * dk;

    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
    float o[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    for (int t0 = p0; t0 < p1; t0 += kTile) {
        const int n = min(kTile, p1 - t0);  // valid positions of this tile (lanes < n)
        float dot[2] = {0.0f, 0.0f};
        for (int c0 = 0; c0 < dk; c0 += kChunk) {
            const int cw = min(kChunk, dk - c0);
            const int q4 = cw / 4;
            __syncthreads();  // the previous chunk's readers are done
            for (int i = threadIdx.x; i < n * q4; i += 256) {
                const int p = i / q4, c = (i - p * q4) * 4;
                *(float4 *)(kt + p * ks + c) = *(const float4 *)(kb + (size_t)(t0 + p) * dk + c0 + c);
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int r = wave + 4 * j;
                if (r >= a.rep || lane >= n) continue;
                const float *qr = qg + (size_t)r * dk + c0;
                const float *kr = kt + lane * ks;
                float acc = dot[j];
                for (int d = 0; d < cw; d += 4) {
                    const float4 k4 = *(const float4 *)(kr + d);
                    const float4 q = *(const float4 *)(qr + d);
                    acc += q.x * k4.x;
                    acc += q.y * k4.y;
                    acc += q.z * k4.z;
                    acc += q.w * k4.w;
                }
                dot[j] = acc;
            }
        }
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int r = wave + 4 * j;
            if (r >= a.rep) continue;  // wave-uniform
            const float s = lane < n ? dot[j] * a.scale : -INFINITY;
            float mt = s;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
            const float mn = fmaxf(m[j], mt);
            const float alpha = (float)exp((double)(m[j] - mn));
            const float e = lane < n ? (float)exp((double)(s - mn)) : 0.0f;
            l[j] = l[j] * alpha + wave_sum(e);
#pragma unroll
            for (int jj = 0; jj < 4; jj++) o[j][jj] = o[j][jj] * alpha;
#pragma unroll 4
            for (int p = 0; p < n; p++) {
                const float ep = lane_bcast(e, p);
                const float *vr = vb + (size_t)(t0 + p) * dk;
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int d = lane + 64 * jj;
                    if (d < dk) o[j][jj] = o[j][jj] + ep * vr[d];
                }
            }
            m[j] = mn;
        }
    }

    // this split's partial of each head: running max, sum, weighted values
    const size_t stride = (size_t)dk + 2;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = wave + 4 * j;
        if (r >= a.rep) continue;
        const int h = g * a.rep + r;
        float *pp = a.part + (((size_t)qi * a.n_heads + h) * a.splits + split) * stride;
        if (lane == 0) {
            pp[0] = m[j];
            pp[1] = l[j];
        }
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const int d = lane + 64 * jj;
            if (d < dk) pp[2 + d] = o[j][jj];
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(&a.cnt[blockIdx.y], 1u) == (unsigned int)(a.splits - 1);
    __syncthreads();
    if (!last) return;
    // the last workgroup of this (row, kv head): every other split's partials
    // were written before its count (fence, then count)
    __threadfence();
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = wave + 4 * j;
        if (r >= a.rep) continue;
        const int h = g * a.rep + r;
        const float *pb = a.part + ((size_t)qi * a.n_heads + h) * a.splits * stride;
        float M = -INFINITY;
        for (int t = 0; t < a.splits; t++) M = fmaxf(M, pb[t * stride]);
        float L = 0.0f, O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int t = 0; t < a.splits; t++) {
            const float w = (float)exp((double)(pb[t * stride] - M));
            L = L + pb[t * stride + 1] * w;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int d = lane + 64 * jj;
                if (d < dk) O[jj] = O[jj] + pb[t * stride + 2 + d] * w;
            }
        }
        const float inv = 1.0f / L;
        float *dst = a.out + ((size_t)qi * a.n_heads + h) * dk;  // mergeHeadsDataF32 layout
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const int d = lane + 64 * jj;
            if (d < dk) dst[d] = O[jj] * inv;
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(&a.cnt[blockIdx.y], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

void attention_plan(int seq, int n_heads, int n_kv, int d_k, int kv_len, int *splits, int *tps,
                    size_t *ws_bytes) {
    const int tiles = (kv_len + kTile - 1) / kTile;
    const int pairs = seq * n_kv;
    int S = (kTargetBlocks + pairs - 1) / pairs;
    S = S < 1 ? 1 : (S > tiles ? tiles : S);
    const int t = (tiles + S - 1) / S;
    S = (tiles + t - 1) / t;
    *splits = S;
    *tps = t;
    const size_t qrot = (size_t)seq * n_heads * d_k * sizeof(float);
    const size_t part = (size_t)seq * n_heads * S * (d_k + 2) * sizeof(float);
    *ws_bytes = ((qrot + 255) & ~(size_t)255) + part;
}

sllm_status launch_attention(const AttnArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(attn_prep_kernel, dim3(a.seq, a.n_heads + a.n_kv), dim3(64), 0, s, a);
    SLLM_HIP(hipGetLastError());
    const size_t lds = (size_t)kTile * (kChunk + 4) * sizeof(float);
    hipLaunchKernelGGL(attn_kernel, dim3(a.splits, a.seq * a.n_kv), dim3(256), lds, s, a);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

}  // namespace sllm
