// The attention section of a decode / prefill step (forwardBlock,
// model_f32.go:398-466) on device buffers: bias adds, per-head QK RMSNorm,
// RoPE, the KV-cache append and the causal GQA attention with merged heads.
//
// attn_split_kernel: one workgroup per (split, row, kv head). A split is a
//   range of cached positions in tiles of 64 (one per lane); the workgroup
//   stages a tile's K and V rows in LDS once for all q heads of the group
//   (GQA: the kv head is read from HBM once), each wave owns one q head,
//   and the split's partial softmax state goes to the workspace.
//   Scores are the reference's sequential float32 dots. For one query row
//   (decode) it also does the bias / norm / RoPE / append work itself.
// attn_prep_kernel (several rows): that work, one wave per (row, head).
// attn_combine_kernel: one wave per (row, head) merges the splits. Separate
//   launches instead of a last-workgroup combine: on this multi-XCD part a
//   device-scope fence writes back and invalidates the L2, which costs more
//   than the launch.
#include <hip/hip_runtime.h>

#include <cmath>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

namespace sllm {

namespace {

constexpr int kTile = 64;     // positions per tile: one per lane
constexpr int kChunk = 128;   // K columns staged per pass (LDS: 64 x 132 floats)
constexpr int kMaxDk = 256;   // head size limit (o: 4 values per lane)

// Native 4-float vector: arrays of it stay in registers (HIP's float4, a
// union type, can keep a register array in scratch memory).
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lane_bcast(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Bias (model_f32.go:398-420), per-head RMSNorm (:424-435; rmsNormFlatF32,
// float32_ops.go:159-172, the sum of squares in the library's association:
// slot s < 256 adds x[s]^2, x[s+256]^2, ..., the four groups of 64 slots are
// wave sums added left to right) and RoPE (applyRopeInPlaceF32,
// float32_ops.go:174-188) of one head row, by one wave, into row (LDS).
// j0: the row's offset in the full q / k row (the bias index).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}
__device__ void prep_row(float *row, const float *src, int dk, const float *bias, int j0, int blen,
                         const float *nw, float eps, const float *freqs, int half, int pos, int lane) {
    // this lane's first rotation frequency, loaded with the row (half <= 64 in one pass)
    const float f0 = lane < half ? freqs[lane] : 0.0f;
    for (int d = lane; d < dk; d += 64) {
        float x = src[d];
        if (bias && j0 + d < blen) x = x + bias[j0 + d];
        row[d] = x;
    }
    wave_lds_sync();
    if (nw) {
        float w[4];
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            float p = 0.0f;
            for (int i = q4 * 64 + lane; i < dk; i += 256) p = p + row[i] * row[i];
            w[q4] = wave_sum(p);
        }
        const float ss = ((w[0] + w[1]) + w[2]) + w[3];
        const float inv = 1.0f / (float)sqrt((double)ss / (double)dk + (double)eps);
        wave_lds_sync();
        for (int d = lane; d < dk; d += 64) row[d] = (row[d] * inv) * nw[d];
        wave_lds_sync();
    }
    for (int i = lane; i < half; i += 64) {
        const float ang = (i == lane ? f0 : freqs[i]) * (float)pos;
        double sd, cd;
        sincos((double)ang, &sd, &cd);
        const float c = (float)cd, sn = (float)sd;
        const float x0 = row[2 * i], x1 = row[2 * i + 1];
        row[2 * i] = x0 * c - x1 * sn;
        row[2 * i + 1] = x0 * sn + x1 * c;
    }
    wave_lds_sync();
}

// Several rows (prefill): one wave per (row, head) - q heads into the
// workspace, kv heads into the cache (k: bias, norm, RoPE; v: bias) at
// rows cache_len + s (the append, model_f32.go:445-448).
__global__ void __launch_bounds__(64) attn_prep_kernel(AttnArgs a) {
    __shared__ float row[kMaxDk];
    const int s = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const bool isq = t < a.n_heads;
    const int h = isq ? t : t - a.n_heads;
    const int dk = a.d_k;
    const int cols = (isq ? a.n_heads : a.n_kv) * dk;
    prep_row(row, (isq ? a.q : a.k) + (size_t)s * cols + (size_t)h * dk, dk, isq ? a.q_bias : a.k_bias, h * dk,
             isq ? a.qb_len : a.kb_len, isq ? a.q_norm : a.k_norm, a.eps, a.freqs, a.half_dim, a.start_pos + s,
             lane);
    if (isq) {
        float *dst = a.qrot + ((size_t)s * a.n_heads + h) * dk;
        for (int d = lane; d < dk; d += 64) dst[d] = row[d];
    } else {
        const size_t at = ((size_t)h * a.cap + (size_t)(a.cache_len + s)) * dk;
        const float *vs = a.v + (size_t)s * cols + (size_t)h * dk;
        for (int d = lane; d < dk; d += 64) {
            a.cache_k[at + d] = row[d];
            float x = vs[d];
            if (a.v_bias && h * dk + d < a.vb_len) x = x + a.v_bias[h * dk + d];
            a.cache_v[at + d] = x;
        }
    }
}

// fusedAttentionHeadF32 (float32_ops.go:190-235) for the q heads of one kv
// head (repeatKVDataF32, float32_ops.go:252-260: q head g*rep + r reads kv
// head g) and one query row, over one split of the positions the causal mask
// leaves (0 .. cache_len + qi): writes the split's running max, sum of
// exponentials and exponential-weighted sum of values per head. Score =
// (sequential float32 dot) * scale, as the reference computes it; the
// exponentials are float32(exp(float64(score - running max))), rescaled by
// the same form when the running max grows.
//
// Wave r owns q head r of the group (max(4, rep) waves); lane l holds the
// values d = l + 64 j, j < DKL (DKL = d_k / 64 rounded up). PREP (one query
// row): the waves first build their q heads (bias, norm, RoPE) in LDS, and
// the workgroup whose range holds the new position builds the new k / v row,
// appends it to the cache and uses it from LDS; otherwise attn_prep_kernel
// has done both. Per tile the K and V rows are loaded together (K straight
// to LDS, V to registers while the scores are computed, then to the same LDS
// buffer): one memory latency per tile, overlapped with the q preparation
// for the first. LDS reads are issued in groups of eight.
template <bool PREP, int DKL>
__global__ void __launch_bounds__(512) attn_split_kernel(AttnArgs a) {

    extern __shared__ __attribute__((aligned(16))) float lds[];
    constexpr int ks = kChunk + 4;
    float *kt = lds;                   // kTile x ks: a K chunk, then a V chunk
    float *qs = lds + kTile * ks;      // rep x d_k: the group's rotated q heads
    float *nk = qs + a.rep * a.d_k;    // PREP: the new k and v rows (2 x d_k)
    const int nt = blockDim.x;
    const int split = blockIdx.x;
    const int qi = blockIdx.y / a.n_kv, g = blockIdx.y - qi * a.n_kv;
    const int tid = threadIdx.x, lane = tid & 63;
    const int r = __builtin_amdgcn_readfirstlane(tid >> 6);  // this wave's q head in the group
    const bool head = r < a.rep;
    const int dk = a.d_k;
    const int limit = a.cache_len + qi + 1;
    const int p0 = split * a.tps * kTile;
    const int p1 = min(p0 + a.tps * kTile, limit);
    // rows read from the cache: PREP builds the new one (position cache_len) itself
    const int have = PREP ? a.cache_len : limit;
    const bool owns_new = PREP && a.cache_len >= p0 && a.cache_len < p1;
    const float *kb = a.cache_k + (size_t)g * a.cap * dk;
    const float *vb = a.cache_v + (size_t)g * a.cap * dk;
    constexpr bool one_chunk = DKL <= 2;  // d_k <= kChunk

    v4f kreg[8], vreg[8];
    auto load_chunk = [&](int t0, int n, int c0, bool k_too, bool v_too) {
        const int q4 = min(kChunk, dk - c0) / 4;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = tid + nt * u;
            if (i < n * q4) {
                const int p = i / q4, c = (i - p * q4) * 4;
                if (t0 + p < have) {
                    const size_t at = (size_t)(t0 + p) * dk + c0 + c;
                    if (k_too) kreg[u] = *(const v4f *)(kb + at);
                    if (v_too) vreg[u] = *(const v4f *)(vb + at);
                }
            }
        }
    };
    auto store_chunk = [&](const v4f *reg, int n, int c0, int newp, const float *newrow) {
        const int q4 = min(kChunk, dk - c0) / 4;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = tid + nt * u;
            if (i < n * q4) {
                const int p = i / q4, c = (i - p * q4) * 4;
                *(v4f *)(kt + p * ks + c) = (p == newp) ? *(const v4f *)(newrow + c0 + c) : reg[u];
            }
        }
    };
    // the first tile's K (and V) rows: issued before anything waits
    if (p0 < p1) load_chunk(p0, min(kTile, p1 - p0), 0, true, one_chunk);

    if (PREP) {
        const int pos = a.start_pos + qi;
        if (head) {
            const int h = g * a.rep + r;
            prep_row(qs + r * dk, a.q + (size_t)qi * a.n_heads * dk + (size_t)h * dk, dk, a.q_bias, h * dk, a.qb_len,
                     a.q_norm, a.eps, a.freqs, a.half_dim, pos, lane);
        }
        if (owns_new && r == (nt >> 6) - 1) {  // the last wave: no q head unless rep fills the workgroup
            const size_t off = (size_t)qi * a.n_kv * dk + (size_t)g * dk;
            prep_row(nk, a.k + off, dk, a.k_bias, g * dk, a.kb_len, a.k_norm, a.eps, a.freqs, a.half_dim, pos, lane);
            const size_t at = ((size_t)g * a.cap + (size_t)a.cache_len) * dk;
            for (int d = lane; d < dk; d += 64) {
                float x = a.v[off + d];
                if (a.v_bias && g * dk + d < a.vb_len) x = x + a.v_bias[g * dk + d];
                nk[dk + d] = x;
                a.cache_k[at + d] = nk[d];
                a.cache_v[at + d] = x;
            }
        }
    } else {
        const float4 *qg = (const float4 *)(a.qrot + ((size_t)qi * a.n_heads + (size_t)g * a.rep) * dk);
        for (int i = tid; i < a.rep * dk / 4; i += nt) ((float4 *)qs)[i] = qg[i];
    }

    float m = -INFINITY, l = 0.0f, o[DKL];
#pragma unroll
    for (int j = 0; j < DKL; j++) o[j] = 0.0f;
    for (int t0 = p0; t0 < p1; t0 += kTile) {
        const int n = min(kTile, p1 - t0);  // valid positions of this tile (lanes < n)
        const int newp = owns_new ? a.cache_len - t0 : -1;  // row of the new position in this tile
        float dot = 0.0f;
        for (int c0 = 0; c0 < dk; c0 += kChunk) {
            const int cw = min(kChunk, dk - c0);
            if (t0 != p0 || c0 != 0) load_chunk(t0, n, c0, true, one_chunk);
            __syncthreads();  // the previous users of kt are done (and qs / nk are written)
            store_chunk(kreg, n, c0, newp, nk);
            __syncthreads();
            if (head && lane < n) {
                const float *qr = qs + r * dk + c0;
                const float *kr = kt + lane * ks;
                for (int d0 = 0; d0 < cw; d0 += 32) {
                    // eight 4-element steps: their LDS reads issue together, the
                    // products are added one by one in element order
                    v4f kv[8], qv[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        kv[u] = *(const v4f *)(kr + d0 + 4 * u);
                        qv[u] = *(const v4f *)(qr + d0 + 4 * u);
                    }
                    const int steps = min(8, (cw - d0) / 4);
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        if (u < steps) {
                            dot += qv[u].x * kv[u].x;
                            dot += qv[u].y * kv[u].y;
                            dot += qv[u].z * kv[u].z;
                            dot += qv[u].w * kv[u].w;
                        }
                    }
                }
            }
        }
        // online softmax of this tile
        float e = 0.0f;
        if (head) {
            const float sc = lane < n ? dot * a.scale : -INFINITY;
            float mt = sc;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
            const float mn = fmaxf(m, mt);
            const float alpha = (float)exp((double)(m - mn));
            e = lane < n ? (float)exp((double)(sc - mn)) : 0.0f;
            l = l * alpha + wave_sum(e);
            m = mn;
#pragma unroll
            for (int j = 0; j < DKL; j++) o[j] = o[j] * alpha;
        }
        // o += sum over the tile's positions of e_p * V[p], V chunk by chunk in LDS
        for (int c0 = 0; c0 < dk; c0 += kChunk) {
            const int cw = min(kChunk, dk - c0);
            if (!one_chunk) load_chunk(t0, n, c0, false, true);
            __syncthreads();  // the score readers of kt are done
            store_chunk(vreg, n, c0, newp, nk + dk);
            __syncthreads();
            if (head) {
                for (int q0 = 0; q0 < n; q0 += 8) {
                    // eight positions' values read together, then added in order
                    float vv[8][DKL];
#pragma unroll
                    for (int pp = 0; pp < 8; pp++) {
                        const float *vr = kt + (q0 + pp) * ks - c0;
#pragma unroll
                        for (int j = 0; j < DKL; j++) {
                            const int d = lane + 64 * j;
                            // rows past the tile's end hold stale LDS data: zero, not
                            // a zero weight times whatever is there (NaN * 0 is NaN)
                            vv[pp][j] = (q0 + pp < n && d >= c0 && d < c0 + cw) ? vr[d] : 0.0f;
                        }
                    }
#pragma unroll
                    for (int pp = 0; pp < 8; pp++) {
                        const float ep = lane_bcast(e, q0 + pp);  // 0 past the tile's end
#pragma unroll
                        for (int j = 0; j < DKL; j++) {
                            const int d = lane + 64 * j;
                            if (d >= c0 && d < c0 + cw) o[j] = o[j] + ep * vv[pp][j];
                        }
                    }
                }
            }
        }
    }

    // this split's partial of the head: running max, sum, weighted values
    if (head) {
        const size_t stride = (size_t)dk + 2;
        const int h = g * a.rep + r;
        float *pp = a.part + (((size_t)qi * a.n_heads + h) * a.splits + split) * stride;
        if (lane == 0) {
            pp[0] = m;
            pp[1] = l;
        }
#pragma unroll
        for (int j = 0; j < DKL; j++) {
            const int d = lane + 64 * j;
            if (d < dk) pp[2 + d] = o[j];
        }
    }
}

// The splits of one (row, head), one wave each: M = max of the split maxima,
// weights w_t = float32(exp(float64(m_t - M))), L = sum of l_t * w_t (fixed
// lane order), out[d] = (sum over t of o_t[d] * w_t) * (1 / L), written in
// mergeHeadsDataF32's layout (float32_ops.go:262-273).
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs a) {
    const int lane = threadIdx.x & 63;
    const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);  // qi * n_heads + h
    if (pair >= a.seq * a.n_heads) return;                 // wave-uniform
    const int dk = a.d_k;
    const size_t stride = (size_t)dk + 2;
    const float *pb = a.part + (size_t)pair * a.splits * stride;
    // splits in groups of 16: lane t holds m_t and l_t of its group, every
    // lane the values of its d for the whole group - all loaded together
    // (a group's missing splits weigh 0 and add exact zeros)
    float M = -INFINITY;
    for (int t = lane; t < a.splits; t += 64) M = fmaxf(M, pb[t * stride]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    float Lp = 0.0f;
    float O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int t0 = 0; t0 < a.splits; t0 += 16) {
        const int nt = min(16, a.splits - t0);
        const int tl = t0 + (lane & 15);
        const bool mine = lane < 16 && tl < a.splits;
        const float ml = mine ? pb[tl * stride] : -INFINITY;
        const float ll = mine ? pb[tl * stride + 1] : 0.0f;
        float ov[16][4];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const float *ob = pb + (size_t)(t0 + u) * stride + 2;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int d = lane + 64 * jj;
                ov[u][jj] = (u < nt && d < dk) ? ob[d] : 0.0f;
            }
        }
        const float wl = mine ? (float)exp((double)(ml - M)) : 0.0f;
        Lp = Lp + ll * wl;
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const float w = lane_bcast(wl, u);  // 0 past the group's end
#pragma unroll
            for (int jj = 0; jj < 4; jj++) O[jj] = O[jj] + ov[u][jj] * w;
        }
    }
    const float L = wave_sum(Lp);
    const float inv = 1.0f / L;
    float *dst = a.out + (size_t)pair * dk;  // mergeHeadsDataF32 layout
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const int d = lane + 64 * jj;
        if (d < dk) dst[d] = O[jj] * inv;
    }
}

}  // namespace

void attention_plan(int seq, int n_heads, int n_kv, int d_k, int kv_len, int *splits, int *tps,
                    size_t *ws_bytes) {
    const int tiles = (kv_len + kTile - 1) / kTile;
    const int pairs = seq * n_kv;
    const int target = tuning().attn_target_blocks;
    int S = (target + pairs - 1) / pairs;
    S = S < 1 ? 1 : (S > tiles ? tiles : S);
    const int t = (tiles + S - 1) / S;
    S = (tiles + t - 1) / t;
    *splits = S;
    *tps = t;
    const size_t qrot = (size_t)seq * n_heads * d_k * sizeof(float);
    const size_t part = (size_t)seq * n_heads * S * (d_k + 2) * sizeof(float);
    *ws_bytes = ((qrot + 255) & ~(size_t)255) + part;
}

template <bool PREP>
void launch_split(const AttnArgs &a, dim3 grid, size_t lds, hipStream_t s) {
    const dim3 block(64 * (a.rep > 4 ? a.rep : 4));
    switch ((a.d_k + 63) / 64) {
    case 1: hipLaunchKernelGGL((attn_split_kernel<PREP, 1>), grid, block, lds, s, a); break;
    case 2: hipLaunchKernelGGL((attn_split_kernel<PREP, 2>), grid, block, lds, s, a); break;
    case 3: hipLaunchKernelGGL((attn_split_kernel<PREP, 3>), grid, block, lds, s, a); break;
    default: hipLaunchKernelGGL((attn_split_kernel<PREP, 4>), grid, block, lds, s, a); break;
    }
}

sllm_status launch_attention(const AttnArgs &a, hipStream_t s) {
    const size_t lds = ((size_t)kTile * (kChunk + 4) + (size_t)(a.rep + 2) * a.d_k) * sizeof(float);
    if (a.seq == 1) {
        launch_split<true>(a, dim3(a.splits, a.n_kv), lds, s);
    } else {
        hipLaunchKernelGGL(attn_prep_kernel, dim3(a.seq, a.n_heads + a.n_kv), dim3(64), 0, s, a);
        SLLM_HIP(hipGetLastError());
        launch_split<false>(a, dim3(a.splits, a.seq * a.n_kv), lds, s);
    }
    SLLM_HIP(hipGetLastError());
    hipLaunchKernelGGL(attn_combine_kernel, dim3((a.seq * a.n_heads + 3) / 4), dim3(256), 0, s, a);
    SLLM_HIP(hipGetLastError());
    return SLLM_OK;
}

}  // namespace sllm
