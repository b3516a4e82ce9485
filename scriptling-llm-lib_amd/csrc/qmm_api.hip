// C ABI (include/sllm_qmm.h): weight handles, the matmul entry points that
// stand in for the reference's Go matmul functions, and verification hooks.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "qmm_device.hpp"
#include "qmm_internal.hpp"

struct sllm_weight {
    int fmt = 0;     // the QType at the ABI
    int layout = 0;  // the plane layout (SLLM_Q4K_STREAM: Q4_1 planes + the Q4_K headers;
                     // SLLM_Q6K_STREAM: Q8_0 planes + the streamed Q6_K planes)
    int64_t q6_exceptions = 0;  // SLLM_Q6K_STREAM: blocks the GEMV recomputes in fp64
    bool q5_one_mfma = false;   // Q5K1 with dh = 16 d in every block: the GEMM's SLLM_Q5K1F form
    int groups = 0, rows = 0, cols = 0;
    int device = 0;
    void *base = nullptr;
    size_t bytes = 0;
    sllm::MutPlanes planes;
};

// KVCacheF32 (float32_ops.go:11-14) of every layer on the device: K and V of
// layer l, kv head g, position p at ((l * n_kv + g) * cap + p) * d_k.
struct sllm_kv_cache {
    int n_layers = 0, n_kv = 0, d_k = 0, cap = 0;
    int device = 0;
    float *k = nullptr, *v = nullptr;
    std::vector<int> len;  // rows held per layer
};

namespace sllm {

namespace {

thread_local std::string g_err;

std::mutex g_mu;
bool g_init_done = false;
sllm_status g_init_status = SLLM_ERR_DEVICE;
std::string g_init_msg;

// Per-call resources for the host-pointer entry points: a stream, device
// staging buffers and pinned host bounce buffers, pooled so concurrent
// callers never share one.
struct Ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    void *buf = nullptr;
    size_t cap = 0;
    void *hbuf = nullptr;  // pinned host memory (hipHostMalloc, cacheable by the GPU): inputs and copies
    size_t hcap = 0;
    void *obuf = nullptr;  // coherent pinned host memory (kDirectOutBytes): outputs the kernels write directly

    unsigned *flag = nullptr;  // coherent pinned word: the stream writes seq there when a call's work is done
    unsigned seq = 0;
};
std::vector<Ctx *> g_pool;

// Host transfers of a call at most this large go through the context's
// pinned bounce buffer (a host memcpy plus a DMA from / to pinned memory,
// instead of the runtime staging pageable memory itself); larger ones are
// copied from / to the caller's pageable memory directly. The buffer grows
// geometrically up to this size, so each pooled context (one per caller
// running concurrently on a device) holds at most kMaxPinnedBytes +
// kDirectOutBytes of pinned host memory for the life of the process.
constexpr size_t kMaxPinnedBytes = (size_t)64 << 20;
// Outputs of a call at most this large (together) are written by the kernels
// straight into the context's coherent pinned buffer (fine-grained host
// memory: the kernels' stores reach host memory before the kernels complete,
// so they are visible once the completion word below is), without a
// device-to-host copy.
constexpr size_t kDirectOutBytes = (size_t)1 << 20;
// Inputs of at most this size are read by the kernels from the pinned bounce
// buffer (no upload enqueue); larger ones are uploaded first.
constexpr size_t kDirectInBytes = (size_t)64 << 10;
// How long a call spins on its completion word before it blocks in
// hipStreamSynchronize instead (long calls, or a stream in error).
constexpr double kSpinSeconds = 2e-3;

// Workspace per (device, stream) (GEMM activation codes and split partials,
// attention q rows and split states, normed rows), grown on demand. A buffer
// that is outgrown is retired, never freed while the library is loaded: a HIP
// graph captured on the stream before the growth still holds its address and
// may be replayed later.
struct Ws {
    void *p = nullptr;
    size_t cap = 0;
    std::vector<void *> retired;
};
std::unordered_map<uint64_t, Ws> g_ws;

bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Argmax scratch per (device, stream): a 64-bit key and two counters, zeroed
// once at allocation; every argmax launch leaves them zeroed again.
std::unordered_map<uint64_t, void *> g_amax;
constexpr size_t kLaunchScratchBytes = 64;

sllm_status amax_scratch(hipStream_t stream, void **out) {
    int dev = 0;
    SLLM_HIP(hipGetDevice(&dev));
    const uint64_t key = ((uint64_t)(uintptr_t)stream << 8) ^ (uint64_t)dev;
    std::lock_guard<std::mutex> lk(g_mu);
    void *&p = g_amax[key];
    if (!p) {
        if (capturing(stream))
            return set_error(SLLM_ERR_ARG, "argmax: the first call on a stream allocates its scratch; "
                                           "make one call on the stream before capturing it");
        if (hipMalloc(&p, kLaunchScratchBytes) != hipSuccess) {
            p = nullptr;
            return set_error(SLLM_ERR_OOM, "argmax scratch allocation failed");
        }
        // cleared on the stream that uses it: a non-blocking stream is not
        // ordered after the null stream, where hipMemset would run
        SLLM_HIP(hipMemsetAsync(p, 0, kLaunchScratchBytes, stream));
    }
    *out = p;
    return SLLM_OK;
}

// The workspace of `stream` on the current device, grown to at least `need`
// bytes (to at least twice its size, so retired buffers total less than the
// live one). The old buffer is retired, not freed (work queued on the stream
// and graphs captured on it may still use it). A stream under capture cannot
// grow its workspace: the caller reserves it first (sllm_workspace_reserve).
sllm_status workspace(hipStream_t stream, size_t need, void **out, size_t *cap) {
    int dev = 0;
    SLLM_HIP(hipGetDevice(&dev));
    const uint64_t key = ((uint64_t)(uintptr_t)stream << 8) ^ (uint64_t)dev;
    std::lock_guard<std::mutex> lk(g_mu);
    Ws &w = g_ws[key];
    if (w.cap < need) {
        if (capturing(stream))
            return set_error(SLLM_ERR_ARG, "the stream's workspace must grow to " + std::to_string(need) +
                                               " bytes while the stream is capturing; call "
                                               "sllm_workspace_reserve on it before the capture");
        size_t want = need < ((size_t)4 << 20) ? ((size_t)4 << 20) : need;
        want = want < 2 * w.cap ? 2 * w.cap : want;
        void *p = nullptr;
        if (hipMalloc(&p, want) != hipSuccess) return set_error(SLLM_ERR_OOM, "workspace allocation failed");
        if (w.p) w.retired.push_back(w.p);
        w.p = p;
        w.cap = want;
    }
    *out = w.p;
    *cap = w.cap;
    return SLLM_OK;
}

// The scratch of sllm_attention_noalloc_dev: the attention's rotated q rows
// and split states, which sllm_attention_dev keeps in the stream's
// workspace, in a static device array so that the call allocates nothing.
// Every GPU holds its own copy until the process ends. In host code
// `scratch` only names the array (its host shadow): its device address on
// each GPU comes from hipGetSymbolAddress, looked up once per device with
// that device current, and kept in g_scratch. Nothing in it needs to start at
// zero: every call writes the q rows and split states it reads.
constexpr size_t kStaticScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];
std::unordered_map<int, void *> g_scratch;  // device -> address of its scratch

// The current device's scratch address; g_mu held.
sllm_status static_scratch_locked(int dev, void **out) {
    auto it = g_scratch.find(dev);
    if (it == g_scratch.end()) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
        if (!p) return set_error(SLLM_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned no address");
        it = g_scratch.emplace(dev, p).first;
    }
    *out = it->second;
    return SLLM_OK;
}

sllm_status static_scratch(void **out) {
    int dev = 0;
    SLLM_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_mu);
    return static_scratch_locked(dev, out);
}

sllm_status ensure_init() {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_init_done) {
        if (g_init_status != SLLM_OK) return set_error(g_init_status, g_init_msg);
        return SLLM_OK;
    }
    g_init_done = true;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        g_init_status = SLLM_ERR_DEVICE;
        g_init_msg = "no HIP device available (this library needs an MI355X / gfx950 GPU)";
        return set_error(g_init_status, g_init_msg);
    }
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) {
        g_init_status = SLLM_ERR_DEVICE;
        g_init_msg = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e);
        return set_error(g_init_status, g_init_msg);
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_init_status = SLLM_ERR_DEVICE;
        g_init_msg = std::string("device is ") + prop.gcnArchName + ", this build targets gfx950 only";
        return set_error(g_init_status, g_init_msg);
    }
    // (the static scratch's address is looked up by the first no-allocation
    // call on each device, whose error stays that call's)
    g_init_status = SLLM_OK;
    return SLLM_OK;
}

sllm_status acquire(Ctx **out, size_t bytes) {
    int dev = 0;
    SLLM_HIP(hipGetDevice(&dev));
    Ctx *c = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        for (size_t i = 0; i < g_pool.size(); i++) {
            if (g_pool[i]->device == dev) {
                c = g_pool[i];
                g_pool.erase(g_pool.begin() + (long)i);
                break;
            }
        }
    }
    if (!c) {
        c = new Ctx();
        c->device = dev;
        hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete c;
            return hip_error(e, "hipStreamCreateWithFlags");
        }
    }
    if (c->cap < bytes) {
        if (c->buf) (void)hipFree(c->buf);
        c->buf = nullptr;
        c->cap = 0;
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        hipError_t e = hipMalloc(&c->buf, want);
        if (e != hipSuccess) {
            std::lock_guard<std::mutex> lk(g_mu);
            g_pool.push_back(c);
            return set_error(SLLM_ERR_OOM, "device staging allocation failed");
        }
        c->cap = want;
    }
    *out = c;
    return SLLM_OK;
}

void release(Ctx *c) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_pool.push_back(c);
}

int parse_qtype(const char *q) {
    if (!q) return -1;
    if (!std::strcmp(q, "q8")) return SLLM_Q8_0;
    if (!std::strcmp(q, "q4")) return SLLM_Q4_0;
    if (!std::strcmp(q, "q4_1")) return SLLM_Q4_1;
    if (!std::strcmp(q, "q5")) return SLLM_Q5_0;
    if (!std::strcmp(q, "q5k1")) return SLLM_Q5K1;
    return -1;
}

sllm_status alloc_weight(int fmt, int rows, int cols, sllm_weight **out, int layout = -1) {
    // the GEMV addresses a plane with 32-bit byte offsets (16-byte entries at most)
    if ((int64_t)rows * (cols / 32) >= ((int64_t)1 << 28))
        return set_error(SLLM_ERR_SHAPE, "weight too large: at most 2^28 blocks of 32 weights");
    auto *w = new sllm_weight();
    w->fmt = fmt;
    w->layout = layout < 0 ? fmt : layout;
    w->rows = rows;
    w->cols = cols;
    w->groups = cols / 32;
    (void)hipGetDevice(&w->device);
    const int64_t nb = (int64_t)rows * w->groups;
    w->bytes = carve_planes(w->layout, nb, nullptr, nullptr);
    hipError_t e = hipMalloc(&w->base, w->bytes);
    if (e != hipSuccess) {
        delete w;
        return set_error(SLLM_ERR_OOM, "weight plane allocation failed");
    }
    carve_planes(w->layout, nb, w->base, &w->planes);
    *out = w;
    return SLLM_OK;
}

// The context's pinned buffer, grown to at least `bytes` (false: larger than
// kMaxPinnedBytes, or pinned memory is not available).
bool pinned(Ctx *c, size_t bytes) {
    if (bytes > kMaxPinnedBytes) return false;
    if (c->hcap >= bytes) return true;
    if (c->hbuf) (void)hipHostFree(c->hbuf);
    c->hbuf = nullptr;
    size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    if (want < 2 * c->hcap) want = 2 * c->hcap;  // geometric growth: rising sizes reallocate rarely
    if (want > kMaxPinnedBytes) want = kMaxPinnedBytes;
    c->hcap = 0;
    if (hipHostMalloc(&c->hbuf, want, hipHostMallocDefault) != hipSuccess) {
        c->hbuf = nullptr;
        return false;
    }
    c->hcap = want;
    return true;
}

// The context's coherent output buffer (kDirectOutBytes), allocated once.
bool coherent_out(Ctx *c) {
    if (c->obuf) return true;
    if (hipHostMalloc(&c->obuf, kDirectOutBytes, hipHostMallocCoherent) != hipSuccess) {
        c->obuf = nullptr;
        return false;
    }
    return true;
}

// Wait for everything enqueued on the context's stream. The stream writes
// the next sequence number into the context's coherent pinned word once all
// earlier work on it has completed (hipStreamWriteValue32) and the caller
// spins on that word: about 4 µs less per call than hipStreamSynchronize.
// Past kSpinSeconds, or when the word cannot be used, the call blocks in
// hipStreamSynchronize, which also reports a failed stream.
hipError_t wait_stream(Ctx *c) {
    if (!c->flag) {
        if (hipHostMalloc((void **)&c->flag, 64, hipHostMallocCoherent) != hipSuccess) {
            c->flag = nullptr;
        } else {
            // the allocation's contents are unspecified: start the sequence from a known value
            __atomic_store_n(c->flag, 0u, __ATOMIC_RELEASE);
            c->seq = 0;
        }
    }
    if (c->flag) {
        const unsigned want = ++c->seq;
        if (hipStreamWriteValue32(c->stream, c->flag, want, 0) == hipSuccess) {
            const auto t0 = std::chrono::steady_clock::now();
            for (unsigned it = 1;; it++) {
                if (__atomic_load_n(c->flag, __ATOMIC_ACQUIRE) == want) return hipSuccess;
                if ((it & 1023) == 0 &&
                    std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > kSpinSeconds)
                    break;
            }
        }
    }
    return hipStreamSynchronize(c->stream);
}

// One host-buffer call: copy the inputs (host -> device staging), run
// `launch` on the context's stream, bring the outputs back and wait for the
// stream. Small transfers bounce through pinned memory; small inputs are read
// by the kernels from the pinned buffer itself (no upload enqueue) and small
// outputs are written into the coherent pinned buffer. launch(iaddr, oaddr) gets the device-visible
// address each input is to be read from and each output is to be written to.
struct HostIn {
    const void *src;
    void *dev;
    size_t bytes;
};
struct HostOut {
    void *dst;
    void *dev;  // device staging for the output (used unless it is written to pinned memory)
    size_t bytes;
};
template <class F>
sllm_status host_call(Ctx *c, const HostIn *in, int nin, const HostOut *out, int nout, F launch) {
    size_t tin = 0, tout = 0;
    for (int i = 0; i < nin; i++) tin += (in[i].bytes + 255) & ~(size_t)255;
    for (int i = 0; i < nout; i++) tout += (out[i].bytes + 255) & ~(size_t)255;
    const bool pin = pinned(c, tin + tout);
    const bool direct_in = pin && tin <= kDirectInBytes;
    const bool direct = pin && tout <= kDirectOutBytes && coherent_out(c);
    char *hb = (char *)c->hbuf;
    char *ob = (char *)c->obuf;
    hipError_t e = hipSuccess;
    size_t off = 0;
    void *i1[4];
    std::vector<void *> inv(nin > 4 ? (size_t)nin : 0);
    void **iaddr = nin > 4 ? inv.data() : i1;
    for (int i = 0; i < nin && e == hipSuccess; i++) {
        iaddr[i] = in[i].dev;
        if (pin) {
            std::memcpy(hb + off, in[i].src, in[i].bytes);
            if (direct_in) iaddr[i] = hb + off;
            else e = hipMemcpyAsync(in[i].dev, hb + off, in[i].bytes, hipMemcpyHostToDevice, c->stream);
            off += (in[i].bytes + 255) & ~(size_t)255;
        } else {
            e = hipMemcpyAsync(in[i].dev, in[i].src, in[i].bytes, hipMemcpyHostToDevice, c->stream);
        }
    }
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(c->stream);  // copies enqueued before the failure still read the bounce buffer
        return hip_error(e, "host-to-device copy");
    }
    const size_t obase = off;
    void *o1[4];  // the usual case; more outputs take a vector
    std::vector<void *> on(nout > 4 ? (size_t)nout : 0);
    void **oaddr = nout > 4 ? on.data() : o1;
    size_t doff = 0;
    for (int i = 0; i < nout; i++) {
        oaddr[i] = direct ? (void *)(ob + doff) : out[i].dev;
        doff += (out[i].bytes + 255) & ~(size_t)255;
    }
    sllm_status st = launch((void *const *)iaddr, (void *const *)oaddr);
    if (st != SLLM_OK) {
        (void)hipStreamSynchronize(c->stream);  // the inputs' copies or kernels still read the bounce buffer
        return st;
    }
    off = obase;
    for (int i = 0; i < nout && e == hipSuccess && !direct; i++) {
        if (pin) {
            e = hipMemcpyAsync(hb + off, out[i].dev, out[i].bytes, hipMemcpyDeviceToHost, c->stream);
            off += (out[i].bytes + 255) & ~(size_t)255;
        } else {
            e = hipMemcpyAsync(out[i].dst, out[i].dev, out[i].bytes, hipMemcpyDeviceToHost, c->stream);
        }
    }
    const hipError_t es = wait_stream(c);
    if (e == hipSuccess) e = es;
    if (e != hipSuccess) return hip_error(e, "device-to-host copy");
    if (pin) {
        off = direct ? 0 : obase;
        const char *src = direct ? ob : hb;
        for (int i = 0; i < nout; i++) {
            std::memcpy(out[i].dst, src + off, out[i].bytes);
            off += (out[i].bytes + 255) & ~(size_t)255;
        }
    }
    return SLLM_OK;
}

// Upload `bytes` of host memory into the context buffer and run `fn` on it.
template <class F>
sllm_status with_upload(const void *host, size_t bytes, size_t extra, F fn) {
    Ctx *c = nullptr;
    sllm_status st = acquire(&c, bytes + extra + 256);
    if (st != SLLM_OK) return st;
    hipError_t e = hipMemcpyAsync(c->buf, host, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        st = fn(c);
        if (st == SLLM_OK) e = hipStreamSynchronize(c->stream);
    }
    release(c);
    if (e != hipSuccess) return hip_error(e, "upload");
    return st;
}

bool uses_gemm(const sllm_weight *w, int x_rows) {
    // 0 (the default): the GEMM from 8 activation rows for weights of at least
    // 2^24 elements, from 16 for smaller ones. The GEMV takes up to 4 rows per
    // launch and streams the weight once per launch; the GEMM streams it once.
    // Measured (us, GEMV at M = 8 / GEMM at M = 8): Q4_1 14336x4096 36.0 /
    // 28.3, Q8_0 4096x14336 54.6 / 42.4, Q5K1 4096x4096 20.2 / 17.7; Q4_1
    // 1024x4096 at M = 8 13.7 / 20.1 and M = 16 27.2 / 19.1, Q4_0 8192x2048 at
    // M = 16 30.5 / 17.9.
    int min_rows = tuning().gemm_min_rows;
    if (min_rows == 0) min_rows = (int64_t)w->rows * w->cols >= ((int64_t)1 << 24) ? 8 : 16;
    return x_rows >= min_rows && gemm_supported(w->fmt, w->groups);
}

// The GEMV kernel format of a weight, fixed by its plane layout at load: Q4_K
// / Q6_K weights loaded with their native planes stream those, every other
// weight its QType's planes.
int gemv_fmt(const sllm_weight *w) {
    if (w->layout == SLLM_Q4K_STREAM || w->layout == SLLM_Q6K_STREAM) return w->layout;
    return w->fmt;
}

// The GEMM kernel format of a weight: a Q5K1 weight whose high-block scales are
// 16 times its low ones runs as one MFMA per block (SLLM_Q5K1F).
int gemm_fmt(const sllm_weight *w) { return w->fmt == SLLM_Q5K1 && w->q5_one_mfma ? SLLM_Q5K1F : w->fmt; }

// One weight's matmul on device buffers: the GEMV, or the GEMM with the given
// activation workspace (at least gemm_workspace_bytes).
sllm_status run_matmul(const sllm_weight *w, const float *x, int x_rows, float *dst, hipStream_t s, void *ws,
                       size_t cap) {
    const Planes P = as_const(w->planes);
    if (!uses_gemm(w, x_rows)) return launch_gemv(gemv_fmt(w), P, x, dst, w->rows, w->groups, x_rows, s);
    return launch_gemm(gemm_fmt(w), P, x, dst, w->rows, w->groups, x_rows, ws, cap, s);
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// GEMM activation workspace the GEMM-bound weights of a set need (the largest).
size_t multi_gemm_ws(const sllm_weight *const *ws, int count, int x_rows) {
    size_t need = 0;
    for (int i = 0; i < count; i++)
        if (uses_gemm(ws[i], x_rows)) {
            const size_t b = gemm_workspace_bytes(gemm_fmt(ws[i]), ws[i]->rows, ws[i]->groups, x_rows);
            need = b > need ? b : need;
        }
    return align256(need);
}

// Weights sharing the activation rows x. GEMV weights are grouped by format,
// up to kMaxSegs per launch (with the RMSNorm prologue when nw is given);
// GEMM-bound weights run one by one with the workspace [gws, gws + gcap).
sllm_status multi_impl(const sllm_weight *const *ws, int count, const float *x, int x_rows, float *const *dst,
                       hipStream_t s, void *gws, size_t gcap, const float *nw, float eps) {
    sllm_status st = SLLM_OK;
    std::vector<char> done((size_t)count, 0);
    for (int i = 0; i < count; i++) {
        if (done[(size_t)i]) continue;
        const sllm_weight *w = ws[i];
        if (uses_gemm(w, x_rows)) {
            done[(size_t)i] = 1;
            if ((st = run_matmul(w, x, x_rows, dst[i], s, gws, gcap)) != SLLM_OK) return st;
            continue;
        }
        Planes P[kMaxSegs];
        float *D[kMaxSegs];
        int N[kMaxSegs];
        int n = 0;
        for (int j = i; j < count && n < kMaxSegs; j++) {
            if (done[(size_t)j] || gemv_fmt(ws[j]) != gemv_fmt(w) || uses_gemm(ws[j], x_rows)) continue;
            P[n] = as_const(ws[j]->planes);
            D[n] = dst[j];
            N[n] = ws[j]->rows;
            n++;
            done[(size_t)j] = 1;
        }
        if ((st = launch_gemv_multi(gemv_fmt(w), P, D, N, n, x, w->groups, x_rows, s, nw, eps)) != SLLM_OK) return st;
    }
    return SLLM_OK;
}

// Whether gate / up fit the one paired GEMV launch.
bool swiglu_paired(const sllm_weight *wg, const sllm_weight *wu, int x_rows) {
    return !uses_gemm(wg, x_rows) && !uses_gemm(wu, x_rows) && gemv_fmt(wg) == gemv_fmt(wu);
}

// Workspace the unpaired SwiGLU path needs: the GEMM workspace, then gate / up
// buffers the caller did not provide.
size_t swiglu_ws_bytes(const sllm_weight *wg, const sllm_weight *wu, int x_rows, const float *gate,
                       const float *up) {
    if (swiglu_paired(wg, wu, x_rows)) return 0;
    const sllm_weight *pair[2] = {wg, wu};
    const size_t mm = align256((size_t)x_rows * wg->rows * sizeof(float));
    return multi_gemm_ws(pair, 2, x_rows) + (gate ? 0 : mm) + (up ? 0 : mm);
}

sllm_status swiglu_impl(const sllm_weight *wg, const sllm_weight *wu, const float *x, int x_rows, float *h,
                        float *gate, float *up, hipStream_t s, void *ws, const float *nw, float eps) {
    const int N = wg->rows;
    if (swiglu_paired(wg, wu, x_rows))
        return launch_gemv_swiglu(gemv_fmt(wg), as_const(wg->planes), as_const(wu->planes), x, h, gate, up, N,
                                  wg->groups, x_rows, s, nw, eps);
    // Prefill or mixed formats: the two matmuls, then the elementwise SwiGLU;
    // x is already normed here (nw is only passed for the paired launch).
    const sllm_weight *pair[2] = {wg, wu};
    const size_t gw = multi_gemm_ws(pair, 2, x_rows);
    const size_t mm = align256((size_t)x_rows * N * sizeof(float));
    char *tail = (char *)ws + gw;
    float *g = gate ? gate : (float *)tail;
    float *u = up ? up : (float *)(tail + (gate ? 0 : mm));
    sllm_status st;
    if ((st = run_matmul(wg, x, x_rows, g, s, ws, gw)) != SLLM_OK) return st;
    if ((st = run_matmul(wu, x, x_rows, u, s, ws, gw)) != SLLM_OK) return st;
    return launch_swiglu(g, u, h, (size_t)x_rows * N, s);
}

sllm_status check_multi(const sllm_weight *const *ws, int count, const float *x, int x_rows, int x_cols,
                        float *const *dst) {
    if (!ws || !x || !dst) return set_error(SLLM_ERR_ARG, "null pointer");
    if (count <= 0) return set_error(SLLM_ERR_ARG, "count must be positive");
    if (x_rows <= 0) return set_error(SLLM_ERR_ARG, "xRows must be positive");
    for (int i = 0; i < count; i++) {
        if (!ws[i] || !dst[i]) return set_error(SLLM_ERR_ARG, "null weight or dst");
        if (ws[i]->cols != x_cols) return set_error(SLLM_ERR_ARG, "xCols does not match a weight's Cols");
    }
    return SLLM_OK;
}

sllm_status check_swiglu(const sllm_weight *wg, const sllm_weight *wu, const float *x, int x_rows, int x_cols,
                         const float *h) {
    if (!wg || !wu || !x || !h) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_rows <= 0) return set_error(SLLM_ERR_ARG, "xRows must be positive");
    if (wg->cols != x_cols || wu->cols != x_cols) return set_error(SLLM_ERR_ARG, "xCols does not match Cols");
    if (wg->rows != wu->rows) return set_error(SLLM_ERR_ARG, "gate and up have different Rows");
    return SLLM_OK;
}

bool check_shape(int rows, int cols, sllm_status *st) {
    if (rows <= 0 || cols <= 0) {
        *st = set_error(SLLM_ERR_ARG, "rows and cols must be positive");
        return false;
    }
    if (cols % 32) {
        *st = set_error(SLLM_ERR_SHAPE, "cols must be a multiple of 32");
        return false;
    }
    return true;
}

// sllm_attention_dev and, noalloc, sllm_attention_noalloc_dev: the same
// checks, plan and kernels; the scratch is the stream's workspace or the
// device's static array.
sllm_status attention_impl(sllm_kv_cache *kv, int layer, const sllm_attn_params *p, const float *q, const float *k,
                           const float *v, int seq_len, int start_pos, float *out, hipStream_t s, bool noalloc) {
    if (!kv || !p || !q || !k || !v || !out) return set_error(SLLM_ERR_ARG, "null pointer");
    if (layer < 0 || layer >= kv->n_layers) return set_error(SLLM_ERR_ARG, "layer out of range");
    if (seq_len <= 0) return set_error(SLLM_ERR_ARG, "seq_len must be positive");
    if (start_pos < 0) return set_error(SLLM_ERR_ARG, "start_pos must not be negative");
    if (p->n_kv_heads != kv->n_kv || p->d_k != kv->d_k)
        return set_error(SLLM_ERR_ARG, "n_kv_heads / d_k differ from the KV cache's");
    if (p->n_heads <= 0 || p->n_heads % p->n_kv_heads != 0 || p->n_heads / p->n_kv_heads > 8)
        return set_error(SLLM_ERR_SHAPE, "n_heads must be a multiple of n_kv_heads, at most 8 times it");
    if (p->rope_half_dim < 0 || 2 * p->rope_half_dim > p->d_k)
        return set_error(SLLM_ERR_ARG, "rope_half_dim outside 0 .. d_k / 2");
    if (p->rope_half_dim > 0 && !p->rope_freqs) return set_error(SLLM_ERR_ARG, "null rope_freqs");
    if (p->q_bias_len < 0 || p->k_bias_len < 0 || p->v_bias_len < 0)
        return set_error(SLLM_ERR_ARG, "negative bias length");
    const int cl = kv->len[(size_t)layer];
    if ((int64_t)cl + seq_len > kv->cap) return set_error(SLLM_ERR_SHAPE, "KV cache full (max_seq rows)");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    int splits = 0, tps = 0, tw = 0, hs = 1;
    size_t wsb = 0;
    attention_plan(seq_len, p->n_heads, kv->n_kv, kv->d_k, cl + seq_len, &splits, &tps, &tw, &hs, &wsb);
    void *ws = nullptr;
    size_t cap = 0;
    if (noalloc) {
        if (wsb > kStaticScratchBytes)
            return set_error(SLLM_ERR_SHAPE, "attention needs " + std::to_string(wsb) +
                                                 " bytes of scratch, more than the static scratch's " +
                                                 std::to_string(kStaticScratchBytes) +
                                                 " (fewer rows per call, or sllm_attention_dev)");
        if ((st = static_scratch(&ws)) != SLLM_OK) return st;
    } else if ((st = workspace(s, wsb, &ws, &cap)) != SLLM_OK) {
        return st;
    }
    AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.seq = seq_len;
    a.n_heads = p->n_heads;
    a.n_kv = kv->n_kv;
    a.d_k = kv->d_k;
    a.rep = p->n_heads / kv->n_kv;
    a.q_bias = p->q_bias_len ? p->q_bias : nullptr;
    a.k_bias = p->k_bias_len ? p->k_bias : nullptr;
    a.v_bias = p->v_bias_len ? p->v_bias : nullptr;
    a.qb_len = p->q_bias_len;
    a.kb_len = p->k_bias_len;
    a.vb_len = p->v_bias_len;
    a.q_norm = p->q_norm_w;
    a.k_norm = p->k_norm_w;
    a.eps = p->norm_eps;
    a.freqs = p->rope_freqs;
    a.half_dim = p->rope_half_dim;
    a.start_pos = start_pos;
    const size_t loff = (size_t)layer * kv->n_kv * kv->cap * kv->d_k;
    a.cache_k = kv->k + loff;
    a.cache_v = kv->v + loff;
    a.cap = kv->cap;
    a.cache_len = cl;
    a.scale = 1.0f / (float)std::sqrt((double)kv->d_k);  // fusedAttentionHeadF32, float32_ops.go:191
    a.out = out;
    a.qrot = (float *)ws;
    a.part = (float *)((char *)ws + align256((size_t)seq_len * p->n_heads * kv->d_k * sizeof(float)));
    a.splits = splits;
    a.tps = tps;
    a.tw = tw;
    a.hs = hs;
    if ((st = launch_attention(a, s)) != SLLM_OK) return st;
    kv->len[(size_t)layer] = cl + seq_len;
    return SLLM_OK;
}

}  // namespace

sllm_status set_error(sllm_status st, const std::string &msg) {
    g_err = msg;
    return st;
}

sllm_status hip_error(hipError_t e, const char *what) {
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return SLLM_ERR_DEVICE;
}

Tuning &tuning() {
    static Tuning t;
    return t;
}

}  // namespace sllm

using namespace sllm;

extern "C" {

sllm_status sllm_init(void) { return ensure_init(); }

const char *sllm_last_error(void) { return g_err.c_str(); }

const char *sllm_kernel_info(void) {
    static std::string info;
    const Tuning &t = tuning();
    char buf[512];
    std::snprintf(buf, sizeof buf,
                  "sllm_qmm gfx950 planes-v1 | gemv: persistent, <=%d waves/WG, %d WG/CU, fused Q8_0 LDS "
                  "prologue, non-temporal weight stream | gemm: int8 MFMA from xRows>=%s",
                  t.gemv_waves, t.gemv_wg_per_cu,
                  t.gemm_min_rows ? std::to_string(t.gemm_min_rows).c_str() : "8 (16 below 2^24 weights)");
    info = buf;
    return info.c_str();
}

sllm_status sllm_set_param(const char *name, int value) {
    if (!name) return set_error(SLLM_ERR_ARG, "null name");
    Tuning &t = tuning();
    if (!std::strcmp(name, "gemv_waves") && (value == 4 || value == 8 || value == 16)) t.gemv_waves = value;
    else if (!std::strcmp(name, "gemv_wg_per_cu") && value >= 1 && value <= 8) t.gemv_wg_per_cu = value;
    else if (!std::strcmp(name, "gemv_max_nb") && value >= 1 && value <= 8) t.gemv_max_nb = value;
    else if (!std::strcmp(name, "gemv_inflight_kb") && value >= 64) t.gemv_inflight_kb = value;
    else if (!std::strcmp(name, "attn_target_blocks") && value >= 1 && value <= 65536) t.attn_target_blocks = value;
    else if (!std::strcmp(name, "attn_tile_groups") && value >= 1 && value <= 4) t.attn_tile_groups = value;
    else if (!std::strcmp(name, "attn_head_slices") && value >= 0 && value <= 64) t.attn_head_slices = value;
    else if (!std::strcmp(name, "gemm_shape") && value >= 0 && value <= 5) t.gemm_shape = value;
    else if (!std::strcmp(name, "gemm_min_rows") && value >= 0) t.gemm_min_rows = value;
    else if (!std::strcmp(name, "gemm_splits") && value >= 0 && value <= 64) t.gemm_splits = value;
    else if (!std::strcmp(name, "gemv_q4k_stream") && (value == 0 || value == 1)) t.gemv_q4k_stream = value;
    else if (!std::strcmp(name, "gemv_q6k_stream") && (value == 0 || value == 1)) t.gemv_q6k_stream = value;
    else return set_error(SLLM_ERR_ARG, std::string("unknown parameter or value: ") + name);
    return SLLM_OK;
}

sllm_status sllm_workspace_reserve(void *stream, size_t bytes) {
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    void *p = nullptr;
    size_t cap = 0;
    return workspace((hipStream_t)stream, bytes, &p, &cap);
}

sllm_status sllm_weight_from_quant(const char *qtype, const void *raw, size_t raw_bytes, int groups, int rows,
                                   int cols, sllm_weight **out) {
    if (!out || !raw) return set_error(SLLM_ERR_ARG, "null pointer");
    *out = nullptr;
    const int fmt = parse_qtype(qtype);
    if (fmt < 0) return set_error(SLLM_ERR_QTYPE, std::string("unknown QType ") + (qtype ? qtype : "(null)"));
    sllm_status st = SLLM_OK;
    if (!check_shape(rows, cols, &st)) return st;
    if (groups != cols / 32) return set_error(SLLM_ERR_ARG, "groups must equal cols/32");
    const size_t need = (size_t)rows * groups * raw_block_bytes(fmt);
    if (raw_bytes < need) return set_error(SLLM_ERR_ARG, "Raw is shorter than rows*groups blocks");
    if ((st = ensure_init()) != SLLM_OK) return st;
    sllm_weight *w = nullptr;
    if ((st = alloc_weight(fmt, rows, cols, &w)) != SLLM_OK) return st;
    int flag[2] = {0, 0};  // malformed high half; a block with dh != 16 d
    st = with_upload(raw, need, 256, [&](Ctx *c) -> sllm_status {
        int *err = (int *)((char *)c->buf + ((need + 255) & ~(size_t)255));
        SLLM_HIP(hipMemsetAsync(err, 0, 2 * sizeof(int), c->stream));
        sllm_status s2 = pack_from_raw(fmt, (const uint8_t *)c->buf, rows, groups, w->planes, err, c->stream);
        if (s2 != SLLM_OK) return s2;
        if (fmt == SLLM_Q5K1 &&
            (s2 = check_q5k1_one_mfma(w->planes, (int64_t)rows * groups, err + 1, c->stream)) != SLLM_OK)
            return s2;
        SLLM_HIP(hipMemcpyAsync(flag, err, 2 * sizeof(int), hipMemcpyDeviceToHost, c->stream));
        return SLLM_OK;
    });
    w->q5_one_mfma = fmt == SLLM_Q5K1 && flag[1] == 0;
    if (st == SLLM_OK && flag[0])
        st = set_error(SLLM_ERR_FORMAT, "q5k1 high half is not in convertQ5KToTwoQ41 form (min 0, 0/1 nibbles)");
    if (st != SLLM_OK) {
        sllm_weight_destroy(w);
        return st;
    }
    *out = w;
    return SLLM_OK;
}

sllm_status sllm_weight_from_gguf(uint32_t t, const void *raw, size_t raw_bytes, int rows, int cols,
                                  sllm_weight **out) {
    if (!out || !raw) return set_error(SLLM_ERR_ARG, "null pointer");
    *out = nullptr;
    sllm_status st = SLLM_OK;
    if (!check_shape(rows, cols, &st)) return st;
    int fmt = -1, layout = -1;
    size_t per = 0, blk = 32;
    switch (t) {
    case 8: fmt = SLLM_Q8_0; per = 34; break;
    case 2: fmt = SLLM_Q4_0; per = 18; break;
    case 3: fmt = SLLM_Q4_1; per = 20; break;
    case 6: fmt = SLLM_Q5_0; per = 22; break;
    case 12:
        fmt = SLLM_Q4_1; per = 144; blk = 256;
        if (tuning().gemv_q4k_stream) layout = SLLM_Q4K_STREAM;
        break;
    case 13: fmt = SLLM_Q5K1; per = 176; blk = 256; break;
    case 14:
        fmt = SLLM_Q8_0; per = 210; blk = 256;
        if (tuning().gemv_q6k_stream) layout = SLLM_Q6K_STREAM;
        break;
    case 20: fmt = SLLM_Q8_0; per = 18; break;
    case 10: fmt = SLLM_Q2K; per = 84; blk = 256; break;
    case 11: fmt = SLLM_Q3K; per = 110; blk = 256; break;
    default:
        return set_error(SLLM_ERR_QTYPE, "GGUF type " + std::to_string(t) +
                                             " has no int8 kernel (the reference loads it as dense fp32)");
    }
    if (cols % blk) return set_error(SLLM_ERR_SHAPE, "cols must be a multiple of the super-block size 256");
    const size_t need = (size_t)rows * (cols / blk) * per;
    if (raw_bytes < need) return set_error(SLLM_ERR_ARG, "raw is shorter than the tensor's blocks");
    if ((st = ensure_init()) != SLLM_OK) return st;
    sllm_weight *w = nullptr;
    if ((st = alloc_weight(fmt, rows, cols, &w, layout)) != SLLM_OK) return st;
    uint32_t q6stat[2] = {0, 0};
    int q5bad = 1;
    st = with_upload(raw, need, 256, [&](Ctx *c) -> sllm_status {
        const uint8_t *dev = (const uint8_t *)c->buf;
        if (t == 8 || t == 2 || t == 3 || t == 6) return pack_from_raw(fmt, dev, rows, cols / 32, w->planes, nullptr, c->stream);
        if (t == 13) {
            int *bad = (int *)((char *)c->buf + ((need + 255) & ~(size_t)255));
            SLLM_HIP(hipMemsetAsync(bad, 0, sizeof(int), c->stream));
            sllm_status ps = pack_from_gguf(t, dev, rows, cols, w->planes, c->stream);
            if (ps == SLLM_OK) ps = check_q5k1_one_mfma(w->planes, (int64_t)rows * (cols / 32), bad, c->stream);
            if (ps != SLLM_OK) return ps;
            SLLM_HIP(hipMemcpyAsync(&q5bad, bad, sizeof(int), hipMemcpyDeviceToHost, c->stream));
            return SLLM_OK;
        }
        if (w->layout != SLLM_Q6K_STREAM) return pack_from_gguf(t, dev, rows, cols, w->planes, c->stream);
        SLLM_HIP(hipMemsetAsync(w->planes.q6stat, 0, sizeof(q6stat), c->stream));
        sllm_status ps = pack_q6k_stream(dev, rows, cols, w->planes, c->stream);
        if (ps != SLLM_OK) return ps;
        SLLM_HIP(hipMemcpyAsync(q6stat, w->planes.q6stat, sizeof(q6stat), hipMemcpyDeviceToHost, c->stream));
        return SLLM_OK;
    });
    if (st == SLLM_OK && q6stat[1] != 0)
        st = set_error(SLLM_ERR_DEVICE, "Q6_K stream pack: the fp64 requantization disagrees with the Q8_0 planes");
    w->q6_exceptions = q6stat[0];
    w->q5_one_mfma = t == 13 && q5bad == 0;
    if (st != SLLM_OK) {
        sllm_weight_destroy(w);
        return st;
    }
    *out = w;
    return SLLM_OK;
}

sllm_status sllm_weight_from_f32(const float *wf, int rows, int cols, sllm_weight **out) {
    if (!out || !wf) return set_error(SLLM_ERR_ARG, "null pointer");
    *out = nullptr;
    sllm_status st = SLLM_OK;
    if (!check_shape(rows, cols, &st)) return st;
    if ((st = ensure_init()) != SLLM_OK) return st;
    sllm_weight *w = nullptr;
    if ((st = alloc_weight(SLLM_Q8_0, rows, cols, &w)) != SLLM_OK) return st;
    st = with_upload(wf, (size_t)rows * cols * sizeof(float), 0, [&](Ctx *c) -> sllm_status {
        return pack_from_f32((const float *)c->buf, rows, cols, w->planes, c->stream);
    });
    if (st != SLLM_OK) {
        sllm_weight_destroy(w);
        return st;
    }
    *out = w;
    return SLLM_OK;
}

void sllm_weight_destroy(sllm_weight *w) {
    if (!w) return;
    if (w->base) (void)hipFree(w->base);
    delete w;
}

sllm_status sllm_weight_info(const sllm_weight *w, int *qtype, int *groups, int *rows, int *cols,
                             size_t *raw_bytes) {
    if (!w) return set_error(SLLM_ERR_ARG, "null weight");
    if (qtype) *qtype = w->fmt;
    if (groups) *groups = w->groups;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (raw_bytes) *raw_bytes = raw_bytes_of(w->fmt, (int64_t)w->rows * w->groups);
    return SLLM_OK;
}

sllm_status sllm_weight_stream_bytes(const sllm_weight *w, size_t *bytes) {
    if (!w || !bytes) return set_error(SLLM_ERR_ARG, "null pointer");
    *bytes = stream_bytes_of(gemv_fmt(w), (int64_t)w->rows * w->groups);
    return SLLM_OK;
}

sllm_status sllm_weight_q6k_exact_blocks(const sllm_weight *w, int64_t *blocks) {
    if (!w || !blocks) return set_error(SLLM_ERR_ARG, "null pointer");
    *blocks = w->layout == SLLM_Q6K_STREAM ? w->q6_exceptions : -1;
    return SLLM_OK;
}

sllm_status sllm_weight_q5k1_one_mfma(const sllm_weight *w, int *yes) {
    if (!w || !yes) return set_error(SLLM_ERR_ARG, "null pointer");
    *yes = gemm_fmt(w) == SLLM_Q5K1F ? 1 : 0;
    return SLLM_OK;
}

sllm_status sllm_weight_export(const sllm_weight *w, void *raw, size_t cap) {
    if (!w || !raw) return set_error(SLLM_ERR_ARG, "null pointer");
    const int64_t nb = (int64_t)w->rows * w->groups;
    const size_t need = raw_bytes_of(w->fmt, nb);
    if (cap < need) return set_error(SLLM_ERR_ARG, "export buffer too small");
    std::vector<unsigned char> img(w->bytes);
    SLLM_HIP(hipMemcpy(img.data(), w->base, w->bytes, hipMemcpyDeviceToHost));
    MutPlanes p;
    carve_planes(w->layout, nb, img.data(), &p);
    if (kq_native(w->fmt)) {
        export_kq_native(w->fmt, p, nb, (uint8_t *)raw);
        return SLLM_OK;
    }
    unsigned char *o = (unsigned char *)raw;
    auto put16 = [](unsigned char *dst, uint16_t v) { dst[0] = (unsigned char)v; dst[1] = (unsigned char)(v >> 8); };
    for (int64_t b = 0; b < nb; b++) {
        switch (w->fmt) {
        case SLLM_Q8_0:
            put16(o + b * 34, p.d[b]);
            std::memcpy(o + b * 34 + 2, &p.qs[b], 16);
            std::memcpy(o + b * 34 + 18, &p.qs2[b], 16);
            break;
        case SLLM_Q4_0:
            put16(o + b * 18, p.d[b]);
            std::memcpy(o + b * 18 + 2, &p.qs[b], 16);
            break;
        case SLLM_Q4_1:
            put16(o + b * 20, p.d[b]);
            put16(o + b * 20 + 2, p.m[b]);
            std::memcpy(o + b * 20 + 4, &p.qs[b], 16);
            break;
        case SLLM_Q5_0:
            put16(o + b * 22, p.d[b]);
            std::memcpy(o + b * 22 + 2, &p.qh[b], 4);
            std::memcpy(o + b * 22 + 6, &p.qs[b], 16);
            break;
        case SLLM_Q5K1: {
            unsigned char *lo = o + b * 20, *hi = o + (nb + b) * 20;
            put16(lo, p.d[b]);
            put16(lo + 2, p.m[b]);
            std::memcpy(lo + 4, &p.qs[b], 16);
            put16(hi, p.dh[b]);
            put16(hi + 2, 0);
            const uint32_t bits = q5k1_groups_to_bits(p.qh[b]);  // bit e = element e
            for (int i = 0; i < 16; i++)
                hi[4 + i] = (unsigned char)(((bits >> i) & 1u) | (((bits >> (i + 16)) & 1u) << 4));
            break;
        }
        }
    }
    return SLLM_OK;
}

sllm_status sllm_matmul_dev(const sllm_weight *w, const float *x, int x_rows, int x_cols, float *dst,
                            void *stream) {
    if (!w || !x || !dst) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_rows <= 0) return set_error(SLLM_ERR_ARG, "xRows must be positive");
    if (x_cols != w->cols) return set_error(SLLM_ERR_ARG, "xCols does not match the weight's Cols");
    if (((uintptr_t)x & 15) != 0) return set_error(SLLM_ERR_ARG, "x must be 16-byte aligned");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    void *ws = nullptr;
    size_t cap = 0;
    if (uses_gemm(w, x_rows) && (st = workspace(s, gemm_workspace_bytes(gemm_fmt(w), w->rows, w->groups, x_rows), &ws,
                                                 &cap)) != SLLM_OK)
        return st;
    return run_matmul(w, x, x_rows, dst, s, ws, cap);
}

sllm_status sllm_matmul_argmax_dev(const sllm_weight *w, const float *x, int x_cols, float *logits, int *argmax,
                                   void *stream) {
    if (!w || !x || !argmax) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_cols != w->cols) return set_error(SLLM_ERR_ARG, "xCols does not match the weight's Cols");
    if (((uintptr_t)x & 15) != 0) return set_error(SLLM_ERR_ARG, "x must be 16-byte aligned");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    void *scr = nullptr;
    if ((st = amax_scratch(s, &scr)) != SLLM_OK) return st;
    return launch_gemv_argmax(gemv_fmt(w), as_const(w->planes), x, logits, w->rows, w->groups,
                              (unsigned long long *)scr, (unsigned int *)((char *)scr + 8), argmax, s);
}

sllm_status sllm_matmul_argmax(const sllm_weight *w, const float *normed, int *token) {
    if (!w || !normed || !token) return set_error(SLLM_ERR_ARG, "null pointer");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    const size_t xb = (size_t)w->cols * sizeof(float);
    const size_t ooff = (xb + 255) & ~(size_t)255;
    Ctx *c = nullptr;
    if ((st = acquire(&c, ooff + 256)) != SLLM_OK) return st;
    float *dx = (float *)c->buf;
    int *dout = (int *)((char *)c->buf + ooff);
    const HostIn in{normed, dx, xb};
    const HostOut out{token, dout, sizeof(int)};
    st = host_call(c, &in, 1, &out, 1, [&](void *const *i, void *const *o) {
        return sllm_matmul_argmax_dev(w, (const float *)i[0], w->cols, nullptr, (int *)o[0], c->stream);
    });
    release(c);
    return st;
}

sllm_status sllm_matmul_swiglu_dev(const sllm_weight *wg, const sllm_weight *wu, const float *x, int x_rows,
                                   int x_cols, float *h, float *gate, float *up, void *stream) {
    sllm_status st = check_swiglu(wg, wu, x, x_rows, x_cols, h);
    if (st != SLLM_OK) return st;
    if (((uintptr_t)x & 15) != 0) return set_error(SLLM_ERR_ARG, "x must be 16-byte aligned");
    if ((st = ensure_init()) != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    void *ws = nullptr;
    size_t cap = 0;
    const size_t need = swiglu_ws_bytes(wg, wu, x_rows, gate, up);
    if (need && (st = workspace(s, need, &ws, &cap)) != SLLM_OK) return st;
    return swiglu_impl(wg, wu, x, x_rows, h, gate, up, s, ws, nullptr, 0.0f);
}

sllm_status sllm_rmsnorm_matmul_swiglu_dev(const sllm_weight *wg, const sllm_weight *wu, const float *x,
                                           const float *norm_w, float eps, int x_rows, int x_cols, float *h,
                                           void *stream) {
    sllm_status st = check_swiglu(wg, wu, x, x_rows, x_cols, h);
    if (st != SLLM_OK) return st;
    if (!norm_w) return set_error(SLLM_ERR_ARG, "null norm weight");
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)norm_w & 15) != 0)
        return set_error(SLLM_ERR_ARG, "x and the norm weight must be 16-byte aligned");
    if ((st = ensure_init()) != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    // one row (decode) with a paired gate / up: the norm is the GEMV's prologue
    if (x_rows == 1 && swiglu_paired(wg, wu, x_rows))
        return swiglu_impl(wg, wu, x, x_rows, h, nullptr, nullptr, s, nullptr, norm_w, eps);
    // several rows / mixed formats: normed rows into the workspace first
    const size_t nb = align256((size_t)x_rows * x_cols * sizeof(float));
    void *ws = nullptr;
    size_t cap = 0;
    if ((st = workspace(s, nb + swiglu_ws_bytes(wg, wu, x_rows, nullptr, nullptr), &ws, &cap)) != SLLM_OK) return st;
    float *normed = (float *)ws;
    if ((st = launch_rmsnorm(x, norm_w, eps, x_rows, x_cols, normed, s)) != SLLM_OK) return st;
    return swiglu_impl(wg, wu, normed, x_rows, h, nullptr, nullptr, s, (char *)ws + nb, nullptr, 0.0f);
}

sllm_status sllm_matmul_swiglu_into_f32(const sllm_weight *wg, const sllm_weight *wu, const float *x, int x_rows,
                                        int x_cols, float *h) {
    if (!wg || !wu || !x || !h) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_rows <= 0) return set_error(SLLM_ERR_ARG, "xRows must be positive");
    if (wg->cols != x_cols || wu->cols != x_cols) return set_error(SLLM_ERR_ARG, "xCols does not match Cols");
    if (wg->rows != wu->rows) return set_error(SLLM_ERR_ARG, "gate and up have different Rows");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    const size_t xb = (size_t)x_rows * x_cols * sizeof(float);
    const size_t hb = (size_t)x_rows * wg->rows * sizeof(float);
    const size_t hoff = (xb + 255) & ~(size_t)255;
    Ctx *c = nullptr;
    if ((st = acquire(&c, hoff + hb)) != SLLM_OK) return st;
    float *dx = (float *)c->buf;
    float *dh = (float *)((char *)c->buf + hoff);
    const HostIn in{x, dx, xb};
    const HostOut out{h, dh, hb};
    st = host_call(c, &in, 1, &out, 1, [&](void *const *i, void *const *o) {
        return sllm_matmul_swiglu_dev(wg, wu, (const float *)i[0], x_rows, x_cols, (float *)o[0], nullptr, nullptr,
                                      c->stream);
    });
    release(c);
    return st;
}

sllm_status sllm_matmul_quant_into_f32(const sllm_weight *w, const float *x, int x_rows, int x_cols, float *dst) {
    if (!w || !x || !dst) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_rows <= 0) return set_error(SLLM_ERR_ARG, "xRows must be positive");
    if (x_cols != w->cols) return set_error(SLLM_ERR_ARG, "xCols does not match the weight's Cols");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    const size_t xb = (size_t)x_rows * x_cols * sizeof(float);
    const size_t yb = (size_t)x_rows * w->rows * sizeof(float);
    const size_t yoff = (xb + 255) & ~(size_t)255;
    Ctx *c = nullptr;
    if ((st = acquire(&c, yoff + yb)) != SLLM_OK) return st;
    float *dx = (float *)c->buf;
    float *dy = (float *)((char *)c->buf + yoff);
    const HostIn in{x, dx, xb};
    const HostOut out{dst, dy, yb};
    st = host_call(c, &in, 1, &out, 1, [&](void *const *i, void *const *o) {
        return sllm_matmul_dev(w, (const float *)i[0], x_rows, x_cols, (float *)o[0], c->stream);
    });
    release(c);
    return st;
}

sllm_status sllm_matmul_multi_dev(const sllm_weight *const *ws, int count, const float *x, int x_rows, int x_cols,
                                  float *const *dst, void *stream) {
    sllm_status st = check_multi(ws, count, x, x_rows, x_cols, dst);
    if (st != SLLM_OK) return st;
    if (((uintptr_t)x & 15) != 0) return set_error(SLLM_ERR_ARG, "x must be 16-byte aligned");
    if ((st = ensure_init()) != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    void *gws = nullptr;
    size_t cap = 0;
    const size_t need = multi_gemm_ws(ws, count, x_rows);
    if (need && (st = workspace(s, need, &gws, &cap)) != SLLM_OK) return st;
    return multi_impl(ws, count, x, x_rows, dst, s, gws, need, nullptr, 0.0f);
}

sllm_status sllm_rmsnorm_matmul_multi_dev(const sllm_weight *const *ws, int count, const float *x,
                                          const float *norm_w, float eps, int x_rows, int x_cols,
                                          float *const *dst, void *stream) {
    sllm_status st = check_multi(ws, count, x, x_rows, x_cols, dst);
    if (st != SLLM_OK) return st;
    if (!norm_w) return set_error(SLLM_ERR_ARG, "null norm weight");
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)norm_w & 15) != 0)
        return set_error(SLLM_ERR_ARG, "x and the norm weight must be 16-byte aligned");
    if ((st = ensure_init()) != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    const size_t gneed = multi_gemm_ws(ws, count, x_rows);
    // one row (decode): the norm is the GEMV's prologue
    if (x_rows == 1 && gneed == 0) return multi_impl(ws, count, x, x_rows, dst, s, nullptr, 0, norm_w, eps);
    // several rows: normed rows into the workspace first, then every weight
    // reads them (GEMV and GEMM alike)
    const size_t nb = align256((size_t)x_rows * x_cols * sizeof(float));
    void *ws_ = nullptr;
    size_t cap = 0;
    if ((st = workspace(s, nb + gneed, &ws_, &cap)) != SLLM_OK) return st;
    float *normed = (float *)ws_;
    if ((st = launch_rmsnorm(x, norm_w, eps, x_rows, x_cols, normed, s)) != SLLM_OK) return st;
    return multi_impl(ws, count, normed, x_rows, dst, s, (char *)ws_ + nb, gneed, nullptr, 0.0f);
}

sllm_status sllm_rmsnorm_matmul_argmax_dev(const sllm_weight *w, const float *x, const float *norm_w, float eps,
                                           int x_cols, float *logits, int *argmax, void *stream) {
    if (!w || !x || !norm_w || !argmax) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_cols != w->cols) return set_error(SLLM_ERR_ARG, "xCols does not match the weight's Cols");
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)norm_w & 15) != 0)
        return set_error(SLLM_ERR_ARG, "x and the norm weight must be 16-byte aligned");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    void *scr = nullptr;
    if ((st = amax_scratch(s, &scr)) != SLLM_OK) return st;
    return launch_gemv_argmax(gemv_fmt(w), as_const(w->planes), x, logits, w->rows, w->groups,
                              (unsigned long long *)scr, (unsigned int *)((char *)scr + 8), argmax, s, norm_w, eps);
}

sllm_status sllm_matmul_multi_quant_into_f32(const sllm_weight *const *ws, int count, const float *x, int x_rows,
                                             int x_cols, float *const *dst) {
    if (!ws || !x || !dst) return set_error(SLLM_ERR_ARG, "null pointer");
    if (count <= 0) return set_error(SLLM_ERR_ARG, "count must be positive");
    if (x_rows <= 0) return set_error(SLLM_ERR_ARG, "xRows must be positive");
    for (int i = 0; i < count; i++) {
        if (!ws[i] || !dst[i]) return set_error(SLLM_ERR_ARG, "null weight or dst");
        if (ws[i]->cols != x_cols) return set_error(SLLM_ERR_ARG, "xCols does not match a weight's Cols");
    }
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    // staging: x, then each output, 256-byte aligned
    const size_t xb = (size_t)x_rows * x_cols * sizeof(float);
    std::vector<size_t> off((size_t)count);
    size_t total = (xb + 255) & ~(size_t)255;
    for (int i = 0; i < count; i++) {
        off[(size_t)i] = total;
        total += ((size_t)x_rows * ws[i]->rows * sizeof(float) + 255) & ~(size_t)255;
    }
    Ctx *c = nullptr;
    if ((st = acquire(&c, total)) != SLLM_OK) return st;
    std::vector<float *> dd((size_t)count);
    std::vector<HostOut> outs((size_t)count);
    for (int i = 0; i < count; i++) {
        dd[(size_t)i] = (float *)((char *)c->buf + off[(size_t)i]);
        outs[(size_t)i] = HostOut{dst[i], dd[(size_t)i], (size_t)x_rows * ws[i]->rows * sizeof(float)};
    }
    const HostIn in{x, c->buf, xb};
    st = host_call(c, &in, 1, outs.data(), count, [&](void *const *xi, void *const *o) {
        for (int i = 0; i < count; i++) dd[(size_t)i] = (float *)o[i];
        return sllm_matmul_multi_dev(ws, count, (const float *)xi[0], x_rows, x_cols, dd.data(), c->stream);
    });
    release(c);
    return st;
}

sllm_status sllm_matmul_row_quant_into_f32(const sllm_weight *w, const float *normed, float *dst) {
    if (!w) return set_error(SLLM_ERR_ARG, "null weight");
    return sllm_matmul_quant_into_f32(w, normed, 1, w->cols, dst);
}

sllm_status sllm_argmax_dev(const float *v, int n, int *out, void *stream) {
    if (!v || !out || n <= 0) return set_error(SLLM_ERR_ARG, "bad argument");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    Ctx *c = nullptr;
    if ((st = acquire(&c, 256)) != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    st = launch_argmax(v, n, (int *)c->buf, s);
    hipError_t e = hipSuccess;
    if (st == SLLM_OK) {
        e = hipMemcpyAsync(out, c->buf, sizeof(int), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    release(c);
    if (e != hipSuccess) return hip_error(e, "argmax");
    return st;
}

sllm_status sllm_debug_quantize_act(const float *x, int rows, int cols, int8_t *xq, float *xs, int32_t *sum_xq) {
    if (!x || !xq || !xs) return set_error(SLLM_ERR_ARG, "null pointer");
    sllm_status st = SLLM_OK;
    if (!check_shape(rows, cols, &st)) return st;
    if ((st = ensure_init()) != SLLM_OK) return st;
    const int G = cols / 32;
    const size_t xb = (size_t)rows * cols * 4, qb = (size_t)rows * cols, sb = (size_t)rows * G * 4;
    const size_t oq = (xb + 255) & ~(size_t)255, os = oq + ((qb + 255) & ~(size_t)255), ox = os + ((sb + 255) & ~(size_t)255);
    Ctx *c = nullptr;
    if ((st = acquire(&c, ox + sb)) != SLLM_OK) return st;
    char *b = (char *)c->buf;
    hipError_t e = hipMemcpyAsync(b, x, xb, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        st = launch_quantize_act((float *)b, rows, G, (int8_t *)(b + oq), (float *)(b + os), (int32_t *)(b + ox), c->stream);
        if (st == SLLM_OK) {
            e = hipMemcpyAsync(xq, b + oq, qb, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess) e = hipMemcpyAsync(xs, b + os, sb, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess && sum_xq) e = hipMemcpyAsync(sum_xq, b + ox, sb, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        }
    }
    release(c);
    if (e != hipSuccess) return hip_error(e, "debug_quantize_act");
    return st;
}

sllm_status sllm_debug_block_dots(const sllm_weight *w, const float *x, int x_rows, int x_cols, int32_t *out) {
    if (!w || !x || !out) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_rows <= 0 || x_cols != w->cols) return set_error(SLLM_ERR_ARG, "bad activation shape");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    const size_t xb = (size_t)x_rows * x_cols * 4;
    const size_t ob = (size_t)x_rows * w->rows * w->groups * 4 * (w->fmt == SLLM_Q5K1 ? 2 : 1);
    const size_t oo = (xb + 255) & ~(size_t)255;
    Ctx *c = nullptr;
    if ((st = acquire(&c, oo + ob)) != SLLM_OK) return st;
    char *b = (char *)c->buf;
    hipError_t e = hipMemcpyAsync(b, x, xb, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        st = launch_block_dots(w->fmt, as_const(w->planes), (const float *)b, w->rows, w->groups, x_rows,
                               (int32_t *)(b + oo), c->stream);
        if (st == SLLM_OK) {
            e = hipMemcpyAsync(out, b + oo, ob, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        }
    }
    release(c);
    if (e != hipSuccess) return hip_error(e, "debug_block_dots");
    return st;
}

sllm_status sllm_debug_gemm_block_dots(const sllm_weight *w, const float *x, int x_rows, int x_cols, int row0,
                                       int n_rows, int32_t *out) {
    if (!w || !x || !out) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_rows <= 0 || x_cols != w->cols) return set_error(SLLM_ERR_ARG, "bad activation shape");
    if (row0 < 0 || n_rows <= 0 || row0 > w->rows - n_rows) return set_error(SLLM_ERR_ARG, "bad weight row range");
    if (w->fmt != SLLM_Q8_0 && w->fmt != SLLM_Q4_0 && w->fmt != SLLM_Q4_1 && w->fmt != SLLM_Q5K1)
        return set_error(SLLM_ERR_QTYPE, "gemm block dots: the format has no int8 GEMM");
    if (!gemm_supported(w->fmt, w->groups)) return set_error(SLLM_ERR_SHAPE, "gemm block dots: cols not supported");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    // the weight rows [row0, row0 + n_rows) as a weight of their own: every plane is [rows][groups]
    Planes P = as_const(w->planes);
    const size_t off = (size_t)row0 * w->groups;
    P.qs += off;
    if (P.qs2) P.qs2 += off;
    P.d += off;
    if (P.m) P.m += off;
    if (P.dh) P.dh += off;
    if (P.qh) P.qh += off;
    const int G = w->groups;
    const size_t xb = align256((size_t)x_rows * x_cols * 4);
    const size_t gb = align256(gemm_workspace_bytes(gemm_fmt(w), n_rows, G, x_rows));
    const size_t db = align256((size_t)x_rows * n_rows * 4);
    const size_t ob = (size_t)x_rows * n_rows * G * 4 * (w->fmt == SLLM_Q5K1 ? 2 : 1);
    Ctx *c = nullptr;
    if ((st = acquire(&c, xb + gb + db + ob)) != SLLM_OK) return st;
    char *b = (char *)c->buf;
    hipError_t e = hipMemcpyAsync(b, x, (size_t)x_rows * x_cols * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        st = launch_gemm_dots(gemm_fmt(w), P, (const float *)b, (float *)(b + xb + gb), n_rows, G, x_rows, b + xb, gb,
                              (int32_t *)(b + xb + gb + db), c->stream);
        if (st == SLLM_OK) {
            e = hipMemcpyAsync(out, b + xb + gb + db, ob, hipMemcpyDeviceToHost, c->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        } else {
            (void)hipStreamSynchronize(c->stream);
        }
    }
    release(c);
    if (e != hipSuccess) return hip_error(e, "debug_gemm_block_dots");
    return st;
}

sllm_status sllm_matmul_add_dev(const sllm_weight *w, const float *x, int x_rows, int x_cols, float *dst,
                                void *stream) {
    if (!w || !x || !dst) return set_error(SLLM_ERR_ARG, "null pointer");
    if (x_rows <= 0) return set_error(SLLM_ERR_ARG, "xRows must be positive");
    if (x_cols != w->cols) return set_error(SLLM_ERR_ARG, "xCols does not match the weight's Cols");
    if (((uintptr_t)x & 15) != 0) return set_error(SLLM_ERR_ARG, "x must be 16-byte aligned");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    const Planes P = as_const(w->planes);
    if (!uses_gemm(w, x_rows)) return launch_gemv_add(gemv_fmt(w), P, x, dst, w->rows, w->groups, x_rows, s);
    // GEMM: the product into the workspace behind the GEMM's own, then dst += it
    const size_t gb = align256(gemm_workspace_bytes(gemm_fmt(w), w->rows, w->groups, x_rows));
    const size_t n = (size_t)x_rows * w->rows;
    void *ws = nullptr;
    size_t cap = 0;
    if ((st = workspace(s, gb + n * sizeof(float), &ws, &cap)) != SLLM_OK) return st;
    float *tmp = (float *)((char *)ws + gb);
    if ((st = launch_gemm(gemm_fmt(w), P, x, tmp, w->rows, w->groups, x_rows, ws, gb, s)) != SLLM_OK) return st;
    return launch_add(dst, tmp, n, s);
}

sllm_status sllm_kv_cache_create(int n_layers, int n_kv_heads, int d_k, int max_seq, sllm_kv_cache **out) {
    if (!out) return set_error(SLLM_ERR_ARG, "null pointer");
    *out = nullptr;
    if (n_layers <= 0 || n_kv_heads <= 0 || max_seq <= 0 || d_k <= 0)
        return set_error(SLLM_ERR_ARG, "KV cache dimensions must be positive");
    if (d_k % 4 != 0 || d_k > 256) return set_error(SLLM_ERR_SHAPE, "d_k must be a multiple of 4, at most 256");
    // the attention kernels address one kv head's rows with 32-bit byte offsets
    if ((int64_t)max_seq * d_k * (int64_t)sizeof(float) >= ((int64_t)1 << 32))
        return set_error(SLLM_ERR_SHAPE, "max_seq x d_k x 4 bytes must stay below 4 GiB per kv head");
    sllm_status st = ensure_init();
    if (st != SLLM_OK) return st;
    auto *kv = new sllm_kv_cache();
    kv->n_layers = n_layers;
    kv->n_kv = n_kv_heads;
    kv->d_k = d_k;
    kv->cap = max_seq;
    kv->len.assign((size_t)n_layers, 0);
    (void)hipGetDevice(&kv->device);
    const size_t bytes = (size_t)n_layers * n_kv_heads * max_seq * d_k * sizeof(float);
    if (hipMalloc(&kv->k, bytes) != hipSuccess || hipMalloc(&kv->v, bytes) != hipSuccess) {
        (void)hipFree(kv->k);
        (void)hipFree(kv->v);
        delete kv;
        return set_error(SLLM_ERR_OOM, "KV cache allocation failed");
    }
    hipError_t e = hipMemsetAsync(kv->k, 0, bytes, nullptr);
    if (e == hipSuccess) e = hipMemsetAsync(kv->v, 0, bytes, nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        (void)hipFree(kv->k);
        (void)hipFree(kv->v);
        delete kv;
        return hip_error(e, "KV cache clear");
    }
    *out = kv;
    return SLLM_OK;
}

void sllm_kv_cache_destroy(sllm_kv_cache *kv) {
    if (!kv) return;
    (void)hipFree(kv->k);
    (void)hipFree(kv->v);
    delete kv;
}

sllm_status sllm_kv_cache_length(const sllm_kv_cache *kv, int layer, int *len) {
    if (!kv || !len) return set_error(SLLM_ERR_ARG, "null pointer");
    if (layer < 0 || layer >= kv->n_layers) return set_error(SLLM_ERR_ARG, "layer out of range");
    *len = kv->len[(size_t)layer];
    return SLLM_OK;
}

sllm_status sllm_kv_cache_set_length(sllm_kv_cache *kv, int len) {
    if (!kv) return set_error(SLLM_ERR_ARG, "null pointer");
    if (len < 0 || len > kv->cap) return set_error(SLLM_ERR_ARG, "length outside 0 .. max_seq");
    for (int &l : kv->len) l = len;
    return SLLM_OK;
}

sllm_status sllm_kv_cache_data(const sllm_kv_cache *kv, int layer, float **k_dev, float **v_dev) {
    if (!kv || !k_dev || !v_dev) return set_error(SLLM_ERR_ARG, "null pointer");
    if (layer < 0 || layer >= kv->n_layers) return set_error(SLLM_ERR_ARG, "layer out of range");
    const size_t off = (size_t)layer * kv->n_kv * kv->cap * kv->d_k;
    *k_dev = kv->k + off;
    *v_dev = kv->v + off;
    return SLLM_OK;
}

sllm_status sllm_attention_dev(sllm_kv_cache *kv, int layer, const sllm_attn_params *p, const float *q,
                               const float *k, const float *v, int seq_len, int start_pos, float *out,
                               void *stream) {
    return attention_impl(kv, layer, p, q, k, v, seq_len, start_pos, out, (hipStream_t)stream, false);
}

sllm_status sllm_attention_noalloc_dev(sllm_kv_cache *kv, int layer, const sllm_attn_params *p, const float *q,
                                       const float *k, const float *v, int seq_len, int start_pos, float *out,
                                       void *stream) {
    return attention_impl(kv, layer, p, q, k, v, seq_len, start_pos, out, (hipStream_t)stream, true);
}

}  // extern "C"
