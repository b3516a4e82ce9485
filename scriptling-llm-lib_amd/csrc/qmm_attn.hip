// The attention section of a decode / prefill step (forwardBlock,
// model_f32.go:398-466) on device buffers: bias adds, per-head QK RMSNorm,
// RoPE, the KV-cache append and the causal GQA attention with merged heads.
//
// attn_split_kernel: one workgroup per (split, row, kv head, head slice). A
//   split is a range of cached positions in tiles of 64 (one per lane),
//   shared by up to three tile groups of waves that run side by side; a group
//   stages its tile's K and V rows in LDS once for the q heads of its slice
//   (GQA: the kv head is read from HBM once, through L2 by each slice) and
//   each owning wave takes one q head. The groups' softmax states are merged in LDS; with one split the
//   workgroup writes the attention output itself, otherwise the split's
//   state goes to the workspace. Scores are the reference's sequential
//   float32 dots. For one query row (decode) it also does the bias / norm /
//   RoPE / append work itself.
// attn_prep_kernel (several rows): that work, one wave per (row, head).
// attn_combine_kernel (more than one split): one wave per (row, head) merges
//   the splits. Separate launches instead of a last-workgroup combine: on
//   this multi-XCD part a device-scope fence writes back and invalidates the
//   L2, which costs more than the launch.
#include <hip/hip_runtime.h>

#include <cmath>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

namespace sllm {

namespace {

constexpr int kTile = 64;     // positions per tile: one per lane
constexpr int kChunk = 128;   // K columns staged per pass (LDS: 64 x 132 floats)
constexpr int kMaxDk = 256;   // head size limit (o: 4 values per lane)
constexpr int kMaxWaves = 12; // split workgroup: up to three tile groups of four waves (168 VGPRs each)
constexpr int kDotSteps = 4;  // 4-element steps of a score's LDS reads issued together

// Native 4-float vector: arrays of it stay in registers (HIP's float4, a
// union type, can keep a register array in scratch memory).
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

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
    // this lane's first rotation frequency and its norm weights (d = lane +
    // 64 j, dk <= 256), loaded with the row: one memory round trip in all
    const float f0 = lane < half ? freqs[lane] : 0.0f;
    float wv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) wv[j] = nw && lane + 64 * j < dk ? nw[lane + 64 * j] : 0.0f;
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
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int d = lane + 64 * j;
            if (d < dk) row[d] = (row[d] * inv) * wv[j];
        }
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
// leaves (0 .. cache_len + qi). Score = (sequential float32 dot) * scale, as
// the reference computes it; the exponentials are float32(exp(float64(score
// - running max))), rescaled by the same form when the running max grows.
//
// The split is a.tw tile groups of nh = max(4, rep) waves (at most
// kMaxWaves waves in all); group t takes a.tps consecutive tiles of the
// split's range (every group runs the same number of steps, so the
// workgroup barriers line up; a tile past the range has no positions). The
// kv group's q heads are shared by a.hs workgroups (head slices) of hp =
// rep / hs heads each; in group t, wave r owns slice head hr = (r - t hp)
// mod nh if hr < hp (the owning waves of successive groups start on
// successive SIMDs), and keeps the value sums of d_k / 64 (rounded up)
// dimensions per lane: d = 2 lane + j when d_k is 128 (one 8-byte LDS read
// per position), d = lane + 64 j otherwise. FULL: d_k is exactly 64 DKL.
// Every head's arithmetic is the same whatever hs is.
// PREP (one query row): group 0's waves first build the q heads (bias, norm,
// RoPE) in LDS, and in the workgroup whose range holds the new position the
// last wave builds the new k / v row, appends it to the cache and the groups
// use it from LDS; otherwise attn_prep_kernel has done both. Per tile the K
// and V rows are loaded together (K straight to LDS, V to registers while
// the scores are computed, then to the same LDS buffer): one memory latency
// per tile, overlapped with the q preparation for the first tile (FULL; the
// other head sizes issue its V rows after the preparation, whose registers
// they would share). LDS reads are issued in groups. At the end each wave
// leaves its (max, sum, values) state in LDS and group 0 merges the groups'
// states in group order exactly as attn_combine_kernel merges splits.
template <bool PREP, int DKL, bool FULL>
__global__ void __launch_bounds__(kMaxWaves * 64) attn_split_kernel(AttnArgs a) {

    extern __shared__ __attribute__((aligned(16))) float lds[];
    constexpr int ks = kChunk + 4;
    const int dk = FULL ? 64 * DKL : a.d_k;
    // o[j] of a lane holds value dof(j): d = 2 lane + j (PAIRED: one 8-byte
    // LDS read per position) or d = lane + 64 j
    constexpr bool PAIRED = FULL && DKL == 2;
    const int nh = a.rep > 4 ? a.rep : 4;  // waves per tile group
    const int hp = a.rep / a.hs;           // q heads per workgroup
    const int ng = 64 * nh;                // threads per tile group
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave / nh;
    const int r = wave - grp * nh;
    const int hr = (r + nh - (grp * hp) % nh) % nh;  // this wave's q head in the slice, if < hp
    const int tg = tid - grp * ng;                   // thread index within the group
    const bool head = hr < hp;
    auto dof = [&](int j) { return PAIRED ? 2 * lane + j : lane + 64 * j; };
    float *kt = lds + (size_t)grp * kTile * ks;  // kTile x ks: a K chunk, then a V chunk
    float *qs = lds + (size_t)a.tw * kTile * ks; // hp x d_k: the slice's rotated q heads
    float *nk = qs + hp * dk;                    // PREP: the new k and v rows (2 x d_k)
    float *mg = nk + 2 * dk;                     // hp x tw x (d_k + 2): the groups' states
    float *ew = mg + (size_t)hp * a.tw * (dk + 2) + (size_t)wave * kTile;  // this wave's tile weights
    const int split = blockIdx.x;
    const int ys = blockIdx.y / a.hs, sl = blockIdx.y - ys * a.hs;  // (row, kv head), head slice
    const int qi = a.row0 + ys / a.n_kv, g = ys - (ys / a.n_kv) * a.n_kv;
    const int h0 = g * a.rep + sl * hp;  // the slice's first q head
    const int limit = a.cache_len + qi + 1;
    const int w0 = split * a.tw * a.tps * kTile;  // the workgroup's range [w0, w1)
    const int w1 = min(w0 + a.tw * a.tps * kTile, limit);
    const int p0 = w0 + grp * a.tps * kTile;      // this group's range [p0, p1) (may be empty)
    const int p1 = min(p0 + a.tps * kTile, limit);
    // rows read from the cache: PREP builds the new one (position cache_len) itself
    const int have = PREP ? a.cache_len : limit;
    const bool owns_new = PREP && a.cache_len >= w0 && a.cache_len < w1;
    const float *kb = a.cache_k + (size_t)g * a.cap * dk;
    const float *vb = a.cache_v + (size_t)g * a.cap * dk;
    constexpr bool one_chunk = DKL <= 2;  // d_k <= kChunk

    v4f kreg[8], vreg[8];
    auto load_chunk = [&](int t0, int n, int c0, bool k_too, bool v_too) {
        const int q4 = FULL ? 16 * DKL : min(kChunk, dk - c0) / 4;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = tg + ng * u;
            if (i < n * q4) {
                const int p = (int)((unsigned)i / (unsigned)q4), c = (i - p * q4) * 4;
                if (t0 + p < have) {
                    // 32-bit byte offset from the head's base (SGPR base + VGPR offset)
                    const uint32_t at = ((uint32_t)(t0 + p) * (uint32_t)dk + (uint32_t)(c0 + c)) * 4u;
                    if (k_too) kreg[u] = *(const v4f *)((const char *)kb + at);
                    if (v_too) vreg[u] = *(const v4f *)((const char *)vb + at);
                }
            }
        }
    };
    // rows n .. n rounded up to 8 are written as zeros (the value loop reads
    // whole groups of eight rows)
    auto store_chunk = [&](const v4f *reg, int n, int c0, int newp, const float *newrow) {
        const int q4 = FULL ? 16 * DKL : min(kChunk, dk - c0) / 4;
        const int n8 = (n + 7) & ~7;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = tg + ng * u;
            if (i < n8 * q4) {
                const int p = (int)((unsigned)i / (unsigned)q4), c = (i - p * q4) * 4;
                const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
                *(v4f *)(kt + p * ks + c) = p >= n ? z : ((p == newp) ? *(const v4f *)(newrow + c0 + c) : reg[u]);
            }
        }
    };
    // the first tile's K rows (FULL: and V rows) are issued before anything
    // waits; otherwise its V rows after the q preparation, whose registers
    // they would share
    if (p0 < p1) load_chunk(p0, min(kTile, p1 - p0), 0, true, FULL && one_chunk);

    if (PREP) {
        const int pos = a.start_pos + qi;
        if (head && grp == 0) {
            const int h = h0 + hr;
            prep_row(qs + hr * dk, a.q + (size_t)qi * a.n_heads * dk + (size_t)h * dk, dk, a.q_bias, h * dk, a.qb_len,
                     a.q_norm, a.eps, a.freqs, a.half_dim, pos, lane);
        }
        // the first wave of group 0 that prepares no q head (waves 0 .. nh - 1
        // start first; with every group-0 wave on a q head, the workgroup's
        // last wave); every head slice builds the row for itself, slice 0
        // appends it to the cache
        const int kwave = hp < nh ? hp : (int)(blockDim.x >> 6) - 1;
        if (owns_new && wave == kwave) {
            const size_t off = (size_t)qi * a.n_kv * dk + (size_t)g * dk;
            // the v row (d = lane + 64 j, dk <= 256) is loaded before the k
            // row is prepared, so its memory round trip overlaps that work
            float vv[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = lane + 64 * j;
                vv[j] = 0.0f;
                if (d < dk) {
                    vv[j] = a.v[off + d];
                    if (a.v_bias && g * dk + d < a.vb_len) vv[j] = vv[j] + a.v_bias[g * dk + d];
                }
            }
            prep_row(nk, a.k + off, dk, a.k_bias, g * dk, a.kb_len, a.k_norm, a.eps, a.freqs, a.half_dim, pos, lane);
            const size_t at = ((size_t)g * a.cap + (size_t)a.cache_len) * dk;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = lane + 64 * j;
                if (d < dk) {
                    nk[dk + d] = vv[j];
                    if (sl == 0) {
                        a.cache_k[at + d] = nk[d];
                        a.cache_v[at + d] = vv[j];
                    }
                }
            }
        }
    } else {
        const float4 *qq = (const float4 *)(a.qrot + ((size_t)qi * a.n_heads + (size_t)h0) * dk);
        for (int i = tid; i < hp * dk / 4; i += (int)blockDim.x) ((float4 *)qs)[i] = qq[i];
    }

    if (!FULL && one_chunk && p0 < p1) load_chunk(p0, min(kTile, p1 - p0), 0, false, true);

    float m = -INFINITY, l = 0.0f, o[DKL];
#pragma unroll
    for (int j = 0; j < DKL; j++) o[j] = 0.0f;
    for (int it = 0; it < a.tps; it++) {
        const int t0 = p0 + it * kTile;
        const int n = max(0, min(kTile, p1 - t0));  // valid positions of this tile (lanes < n)
        const int newp = owns_new ? a.cache_len - t0 : -1;  // row of the new position in this tile
        float dot = 0.0f;
        for (int c0 = 0; c0 < dk; c0 += kChunk) {
            const int cw = min(kChunk, dk - c0);
            if (it != 0 || c0 != 0) load_chunk(t0, n, c0, true, one_chunk);
            __syncthreads();  // the previous users of kt are done (and qs / nk are written)
            store_chunk(kreg, n, c0, newp, nk);
            __syncthreads();
            if (head && lane < n) {
                const float *qr = qs + hr * dk + c0;
                const float *kr = kt + lane * ks;
                for (int d0 = 0; d0 < cw; d0 += 4 * kDotSteps) {
                    // kDotSteps 4-element steps: their LDS reads issue together,
                    // the products are added one by one in element order
                    v4f kv[kDotSteps], qv[kDotSteps];
#pragma unroll
                    for (int u = 0; u < kDotSteps; u++) {
                        kv[u] = *(const v4f *)(kr + d0 + 4 * u);
                        qv[u] = *(const v4f *)(qr + d0 + 4 * u);
                    }
                    const int steps = min(kDotSteps, (cw - d0) / 4);
#pragma unroll
                    for (int u = 0; u < kDotSteps; u++) {
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
        // online softmax of this tile (a tile without positions changes nothing)
        float e = 0.0f;
        if (head && n > 0) {
            const float sc = lane < n ? dot * a.scale : -INFINITY;
            float mt = sc;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
            const float mn = fmaxf(m, mt);
            // a group's first tile (running max still -inf) against a finite
            // max: exp(-inf) = 0 exactly, without the fp64 exp on the chain
            const float alpha = (m == -INFINITY && mn > -INFINITY && mn < INFINITY) ? 0.0f
                                                                                  : (float)exp((double)(m - mn));
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
                // the weights go through LDS: eight per group of positions in two
                // broadcast reads (0 past the tile's end, where the rows are zeros)
                if (c0 == 0) {
                    ew[lane] = e;
                    wave_lds_sync();
                }
                for (int q0 = 0; q0 < n; q0 += 8) {
                    const v4f ea = *(const v4f *)(ew + q0), eb = *(const v4f *)(ew + q0 + 4);
                    const float ev[8] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
                    if (PAIRED) {
                        // eight positions' values read together, then accumulated in
                        // order (fused multiply-add: one rounding per step)
                        v2f vv[8];
#pragma unroll
                        for (int pp = 0; pp < 8; pp++) vv[pp] = *(const v2f *)(kt + (q0 + pp) * ks + 2 * lane);
#pragma unroll
                        for (int pp = 0; pp < 8; pp++) {
                            o[0] = __builtin_fmaf(ev[pp], vv[pp].x, o[0]);
                            o[PAIRED ? 1 : 0] = __builtin_fmaf(ev[pp], vv[pp].y, o[PAIRED ? 1 : 0]);
                        }
                    } else {
                        float vv[8][DKL];
#pragma unroll
                        for (int pp = 0; pp < 8; pp++) {
                            const float *vr = kt + (q0 + pp) * ks - c0;
#pragma unroll
                            for (int j = 0; j < DKL; j++) {
                                const int d = dof(j);
                                vv[pp][j] = (d >= c0 && d < c0 + cw) ? vr[d] : 0.0f;
                            }
                        }
#pragma unroll
                        for (int pp = 0; pp < 8; pp++) {
#pragma unroll
                            for (int j = 0; j < DKL; j++) {
                                const int d = dof(j);
                                if (d >= c0 && d < c0 + cw) o[j] = __builtin_fmaf(ev[pp], vv[pp][j], o[j]);
                            }
                        }
                    }
                }
            }
        }
    }

    // the groups' states meet in LDS; group 0 merges them (M = max, weights
    // w_t = float32(exp(float64(m_t - M))), L = wave_sum over lanes t of
    // l_t * w_t, O = sum over t in order of o_t * w_t), as attn_combine_kernel does
    const int sst = dk + 2;
    if (head) {
        float *st = mg + ((size_t)hr * a.tw + grp) * sst;
        if (lane == 0) {
            st[0] = m;
            st[1] = l;
        }
#pragma unroll
        for (int j = 0; j < DKL; j++) {
            const int d = dof(j);
            if (d < dk) st[2 + d] = o[j];
        }
    }
    __syncthreads();
    if (!head || grp != 0) return;
    const float *sb = mg + (size_t)hr * a.tw * sst;
    float M = -INFINITY;
    for (int t = 0; t < a.tw; t++) M = fmaxf(M, sb[t * sst]);
    const bool mine = lane < a.tw;
    const float ml = mine ? sb[lane * sst] : -INFINITY;
    const float ll = mine ? sb[lane * sst + 1] : 0.0f;
    // a group without positions weighs 0 (also when no group has any: a split
    // of a causal row can lie wholly past it, and then leaves (-inf, 0, 0))
    const float wl = (mine && ml != -INFINITY) ? (float)exp((double)(ml - M)) : 0.0f;
    const float L = wave_sum(0.0f + ll * wl);
    float O[DKL];
#pragma unroll
    for (int j = 0; j < DKL; j++) O[j] = 0.0f;
    for (int t = 0; t < a.tw; t++) {
        const float w = lane_bcast(wl, t);
#pragma unroll
        for (int j = 0; j < DKL; j++) {
            const int d = dof(j);
            O[j] = O[j] + (d < dk ? sb[t * sst + 2 + d] : 0.0f) * w;
        }
    }
    const int h = h0 + hr;
    if (a.splits == 1) {
        const float inv = 1.0f / L;
        float *dst = a.out + ((size_t)qi * a.n_heads + h) * dk;  // mergeHeadsDataF32 layout
#pragma unroll
        for (int j = 0; j < DKL; j++) {
            const int d = dof(j);
            if (d < dk) dst[d] = O[j] * inv;
        }
    } else {
        // this split's partial of the head: running max, sum, weighted values
        float *pp = a.part + (((size_t)qi * a.n_heads + h) * a.splits + split) * sst;
        if (lane == 0) {
            pp[0] = M;
            pp[1] = L;
        }
#pragma unroll
        for (int j = 0; j < DKL; j++) {
            const int d = dof(j);
            if (d < dk) pp[2 + d] = O[j];
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
    // (a group's missing splits weigh 0 and add exact zeros). With at most 16
    // splits the maximum comes from the same loads (one memory round);
    // otherwise from a first pass over the maxima.
    const bool one = a.splits <= 16;
    float M = -INFINITY;
    if (!one) {
        for (int t = lane; t < a.splits; t += 64) M = fmaxf(M, pb[t * stride]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    }
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
        if (one) {
            M = ml;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        }
        // a split without positions (-inf) weighs 0
        const float wl = (mine && ml != -INFINITY) ? (float)exp((double)(ml - M)) : 0.0f;
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

namespace {
// hp: q heads per workgroup (rep / head slices)
size_t attn_lds_bytes(int tw, int rep, int hp, int d_k) {
    const int nh = rep > 4 ? rep : 4;
    return ((size_t)tw * kTile * (kChunk + 4) + (size_t)(hp + 2) * d_k + (size_t)tw * hp * (d_k + 2) +
            (size_t)tw * nh * kTile) *
           sizeof(float);
}
// the device's LDS per workgroup (read once)
size_t lds_per_block() {
    static const size_t v = [] {
        int dev = 0, b = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&b, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || b <= 0)
            return (size_t)64 * 1024;
        return (size_t)b;
    }();
    return v;
}
// the device's CU count (read once)
int cus_per_device() {
    static const int v = [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            return 256;
        return c;
    }();
    return v;
}
}  // namespace

void attention_plan(int seq, int n_heads, int n_kv, int d_k, int kv_len, int *splits, int *tps, int *tw, int *hs,
                    size_t *ws_bytes) {
    const int tiles = (kv_len + kTile - 1) / kTile;
    const int pairs = seq * n_kv;
    const int rep = n_heads / n_kv, nh = rep > 4 ? rep : 4;
    const Tuning &T = tuning();
    // tile groups per workgroup: at most kMaxWaves waves, and what LDS holds
    int G = kMaxWaves / nh;
    G = G < T.attn_tile_groups ? G : T.attn_tile_groups;
    G = G < tiles ? G : tiles;
    while (G > 1 && attn_lds_bytes(G, rep, rep, d_k) > lds_per_block()) G--;
    G = G < 1 ? 1 : G;
    int S, t;
    if (tiles <= G) {
        // one workgroup per (row, kv head), a tile per group: no combine launch
        S = 1;
        t = 1;
        G = tiles;
    } else {
        // splits of at most two groups (waves that share a SIMD share its
        // VALU), about attn_target_blocks workgroups over the (row, kv head)
        // pairs; more tiles per group only past that
        G = G < 2 ? G : 2;
        S = (T.attn_target_blocks + pairs - 1) / pairs;
        const int smax = (tiles + G - 1) / G;
        S = S < 1 ? 1 : (S > smax ? smax : S);
        t = (tiles + S * G - 1) / (S * G);
        S = (tiles + t * G - 1) / (t * G);
    }
    // head slices (the plan above does not depend on them, so neither do the
    // results): while there are fewer workgroups than CUs, the q heads of a
    // kv head are spread over up to rep / 2 workgroups (two heads or more
    // each), every one reading the kv head's rows for its own heads; a
    // divisor of rep. Measured (decode, 32 q / 8 kv heads, d_k 128): KV 128
    // 10.2 -> 8.8 µs, KV 2047 15.4 -> 14.8 µs; one head per workgroup was
    // slower (9.1 and 21.4 µs)
    int H = T.attn_head_slices;
    if (H <= 0) {
        const int64_t wgs = (int64_t)pairs * S;
        H = (int)((cus_per_device() + wgs - 1) / wgs);
        H = H < rep / 2 ? H : rep / 2;
    }
    H = H < 1 ? 1 : (H > rep ? rep : H);
    while (H > 1 && (rep % H || (int64_t)pairs * H > 65535)) H--;  // grid y: pairs x H
    *splits = S;
    *tps = t;
    *tw = G;
    *hs = H;
    const size_t qrot = (size_t)seq * n_heads * d_k * sizeof(float);
    const size_t part = S > 1 ? (size_t)seq * n_heads * S * (d_k + 2) * sizeof(float) : 0;
    *ws_bytes = ((qrot + 255) & ~(size_t)255) + part;
}

template <bool PREP>
void launch_split(const AttnArgs &a, dim3 grid, size_t lds, hipStream_t s) {
    const dim3 block(64 * (a.rep > 4 ? a.rep : 4) * a.tw);
    switch ((a.d_k + 63) / 64) {
    case 1:
        if (a.d_k == 64) hipLaunchKernelGGL((attn_split_kernel<PREP, 1, true>), grid, block, lds, s, a);
        else hipLaunchKernelGGL((attn_split_kernel<PREP, 1, false>), grid, block, lds, s, a);
        break;
    case 2:
        if (a.d_k == 128) hipLaunchKernelGGL((attn_split_kernel<PREP, 2, true>), grid, block, lds, s, a);
        else hipLaunchKernelGGL((attn_split_kernel<PREP, 2, false>), grid, block, lds, s, a);
        break;
    case 3: hipLaunchKernelGGL((attn_split_kernel<PREP, 3, false>), grid, block, lds, s, a); break;
    default: hipLaunchKernelGGL((attn_split_kernel<PREP, 4, false>), grid, block, lds, s, a); break;
    }
}

sllm_status launch_attention(const AttnArgs &a, hipStream_t s) {
    if (a.hs < 1 || a.rep % a.hs) return set_error(SLLM_ERR_ARG, "attention: head slices must divide rep");
    const size_t lds = attn_lds_bytes(a.tw, a.rep, a.rep / a.hs, a.d_k);
    if (a.seq == 1) {
        AttnArgs b = a;
        b.row0 = 0;
        launch_split<true>(b, dim3(a.splits, a.n_kv * a.hs), lds, s);
        SLLM_HIP(hipGetLastError());
    } else {
        hipLaunchKernelGGL(attn_prep_kernel, dim3(a.seq, a.n_heads + a.n_kv), dim3(64), 0, s, a);
        SLLM_HIP(hipGetLastError());
        // grid y is (row, kv head, head slice), at most 65535: long prefills
        // run in chunks of rows (every row's k / v is already in the cache)
        const int per = 65535 / (a.n_kv * a.hs);
        if (per < 1) return set_error(SLLM_ERR_SHAPE, "attention: n_kv_heads x head slices exceeds the grid");
        for (int r0 = 0; r0 < a.seq; r0 += per) {
            AttnArgs b = a;
            b.row0 = r0;
            const int rows = a.seq - r0 < per ? a.seq - r0 : per;
            launch_split<false>(b, dim3(a.splits, rows * a.n_kv * a.hs), lds, s);
            SLLM_HIP(hipGetLastError());
        }
    }
    if (a.splits > 1) {
        hipLaunchKernelGGL(attn_combine_kernel, dim3((a.seq * a.n_heads + 3) / 4), dim3(256), 0, s, a);
        SLLM_HIP(hipGetLastError());
    }
    return SLLM_OK;
}

}  // namespace sllm
