// rac_capi.hip — the C ABI of librac_amd.so.
//
// Three surfaces, all extern "C", plain pointers and sizes:
//  1. rac.h (reference rac.h:85-346): synchronous, void, pointer-agnostic.
//     Each pointer is classified per call; host buffers are staged through
//     device memory, device buffers are used in place; the call returns once
//     the result is in the caller's buffer.  Errors leave the output
//     untouched and are reported through rac_last_error().
//  2. rac_ext.h: device pointers, an explicit HIP stream, asynchronous,
//     returning a status (0 = ok, <0 = rac_status-style error).  This is
//     what the Python layer and hot loops call.
//  3. The kernel-library launcher ABI of rac_kernels.hip:822-909
//     (rac_launch_{nn,nt,tn}[_iters]), which rac_torch_bind.cpp binds.
// Process-wide knobs: RAC_CORDIC_ITERS (default RAC_ITERS = 16, rac.h:41)
// and RAC_CORDIC_MODE (default "cordic") seed rac_{set,get}_cordic_{iters,mode}.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <atomic>
#include <mutex>
#include <string>
#include <utility>
#include <vector>
#include "rac_internal.hpp"
#include "rac_tables.hpp"

#define RAC_EXPORT extern "C" __attribute__((visibility("default")))

namespace rac {

// ── constants computed once on the host ──────────────────────────────────

static double hyp_gain(int steps) {
    double k = 1.0;
    for (int j = 0; j < steps; j++) k *= sqrt(1.0 - ldexp(1.0, -2 * hyp_shift(j)));
    return k;
}

const HostConsts& host_consts() {
    static const HostConsts c = [] {
        HostConsts h{};
        h.exp_khinv[0] = 1.0f;
        for (int n = 1; n <= 24; n++) h.exp_khinv[n] = (float)(1.0 / hyp_gain(n));
        h.rsqrt_khinv = (float)(1.0 / hyp_gain(kRsqrtSteps));
        return h;
    }();
    return c;
}

}  // namespace rac

using namespace rac;

enum {
    RAC_OK = 0,
    RAC_ERR_NULL_PTR = -1,     // rac_cpu.h:54-59
    RAC_ERR_INVALID_DIM = -2,
    RAC_ERR_ALLOC = -3,
    RAC_ERR_DEVICE = -4,
};

// ── error channel ────────────────────────────────────────────────────────

static thread_local char g_last_error[512] = "";

static int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}

static int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return RAC_OK;
    (void)hipGetLastError();
    return fail(RAC_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

namespace rac {
int report(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}
int report_hip(hipError_t e, const char* what) { return check_hip(e, what); }
}  // namespace rac

RAC_EXPORT const char* rac_last_error(void) { return g_last_error; }
RAC_EXPORT void rac_clear_error(void) { g_last_error[0] = '\0'; }

// ── process knobs ────────────────────────────────────────────────────────

static std::atomic<int> g_iters{0};     // 0 = not yet read from the environment
static std::atomic<int> g_mode{-1};

static int mode_from_string(const char* s) {
    if (!s) return -1;
    if (!strcmp(s, "fast") || !strcmp(s, "0")) return kModeFast;
    if (!strcmp(s, "cordic") || !strcmp(s, "1")) return kModeCordic;
    if (!strcmp(s, "shiftadd") || !strcmp(s, "2")) return kModeShiftAdd;
    return -1;
}

RAC_EXPORT void rac_set_cordic_iters(int iters) {
    // rac_torch_bind.cpp:205-210: <= 0 means the default, clamp to [1, 24]
    g_iters.store(iters <= 0 ? 16 : clamp_iters(iters));
}

RAC_EXPORT int rac_get_cordic_iters(void) {
    int v = g_iters.load();
    if (v == 0) {
        const char* e = getenv("RAC_CORDIC_ITERS");
        v = e ? clamp_iters(atoi(e)) : 16;
        if (e && atoi(e) <= 0) v = 16;
        int expected = 0;
        g_iters.compare_exchange_strong(expected, v);
        v = g_iters.load();
    }
    return v;
}

RAC_EXPORT void rac_set_cordic_mode(int mode) {
    // rac_torch_bind.cpp:216-219: out-of-range modes select FAST
    g_mode.store((mode < 0 || mode > 2) ? kModeFast : mode);
}

RAC_EXPORT int rac_get_cordic_mode(void) {
    int v = g_mode.load();
    if (v < 0) {
        int m = mode_from_string(getenv("RAC_CORDIC_MODE"));
        if (m < 0) m = kModeCordic;
        int expected = -1;
        g_mode.compare_exchange_strong(expected, m);
        v = g_mode.load();
    }
    return v;
}

// Stream used by the synchronous rac.h entry points (default: null stream).
static std::atomic<hipStream_t> g_stream{nullptr};
RAC_EXPORT void rac_set_stream(void* stream) { g_stream.store((hipStream_t)stream); }
RAC_EXPORT void* rac_get_stream(void) { return (void*)g_stream.load(); }

RAC_EXPORT int rac_version(void) { return 10000; }   // 1.0.0

RAC_EXPORT int rac_cordic_direction_bits(int iters, int* d) {
    if (!d) return fail(RAC_ERR_NULL_PTR, "rac_cordic_direction_bits: null output");
    const int n = clamp_iters(iters);
    for (int i = 0; i < n; i++) d[i] = cordic_dir(i);
    return n;
}

RAC_EXPORT float rac_exp_gain_inverse(int iters) { return host_consts().exp_khinv[clamp_iters(iters)]; }
RAC_EXPORT float rac_rsqrt_gain_inverse(void) { return host_consts().rsqrt_khinv; }

// ── pointer staging for the synchronous API ──────────────────────────────

namespace rac {
bool is_device_ptr(const void* p) {
    if (!p) return false;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}
}  // namespace rac
static bool is_device_pointer(const void* p) { return is_device_ptr(p); }

// Device staging buffers of the synchronous API come from a per-device
// cache instead of a hipMalloc / hipFree pair per call (hipFree also waits
// for the whole device, and a scalar call such as rac_rotate would otherwise
// pay for up to five of each).  Every synchronous call synchronises its
// stream before its Staged objects are destroyed, so a buffer is back in the
// cache only once no work of the call can touch it.  At most
// stage_cache_cap() bytes stay cached per device (RAC_STAGE_CACHE_MB, 512 by
// default; 0 disables caching); a release beyond that is freed.
// rac_release_cached_memory() frees every cached buffer, for processes where
// another allocator (torch's) needs the memory back.  Buffers cached at
// process exit are left to the runtime's teardown.
namespace {
struct StageCache {
    std::mutex mu;
    std::vector<std::pair<void*, size_t>> free_list[64];
    size_t cached[64] = {};
};
StageCache g_stage_cache;
constexpr size_t kStageGranule = 64u << 10;

size_t stage_cache_cap() {
    static const size_t cap = [] {
        const char* e = getenv("RAC_STAGE_CACHE_MB");
        if (!e || !*e) return (size_t)512 << 20;
        char* end = nullptr;
        const long mb = strtol(e, &end, 10);
        if (end == e || mb < 0) return (size_t)512 << 20;
        return (size_t)mb << 20;
    }();
    return cap;
}

void* stage_take(int dev, size_t want, size_t* got) {
    {
        std::lock_guard<std::mutex> lock(g_stage_cache.mu);
        auto& fl = g_stage_cache.free_list[dev];
        int best = -1;
        for (int i = 0; i < (int)fl.size(); i++)
            if (fl[i].second >= want && (best < 0 || fl[i].second < fl[best].second)) best = i;
        if (best >= 0) {
            void* p = fl[best].first;
            *got = fl[best].second;
            g_stage_cache.cached[dev] -= *got;
            fl.erase(fl.begin() + best);
            return p;
        }
    }
    const size_t sz = (want + kStageGranule - 1) / kStageGranule * kStageGranule;
    void* p = nullptr;
    if (hipMalloc(&p, sz) != hipSuccess) {
        (void)hipGetLastError();
        // out of memory with buffers cached: release them and try once more
        std::vector<std::pair<void*, size_t>> drop;
        {
            std::lock_guard<std::mutex> lock(g_stage_cache.mu);
            drop.swap(g_stage_cache.free_list[dev]);
            g_stage_cache.cached[dev] = 0;
        }
        if (drop.empty()) return nullptr;
        for (auto& e : drop) (void)hipFree(e.first);
        if (hipMalloc(&p, sz) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    *got = sz;
    return p;
}

void stage_give(int dev, void* p, size_t sz) {
    {
        std::lock_guard<std::mutex> lock(g_stage_cache.mu);
        if (g_stage_cache.cached[dev] + sz <= stage_cache_cap()) {
            g_stage_cache.free_list[dev].push_back({p, sz});
            g_stage_cache.cached[dev] += sz;
            return;
        }
    }
    (void)hipFree(p);
}
}  // namespace

// Frees every staging buffer the synchronous API keeps cached, on every
// device; returns the bytes released.  Cached buffers are idle by
// construction (each call synchronises before returning its buffers).
RAC_EXPORT long rac_release_cached_memory(void) {
    std::vector<std::pair<void*, size_t>> drop;
    {
        std::lock_guard<std::mutex> lock(g_stage_cache.mu);
        for (int d = 0; d < 64; d++) {
            for (auto& e : g_stage_cache.free_list[d]) drop.push_back(e);
            g_stage_cache.free_list[d].clear();
            g_stage_cache.cached[d] = 0;
        }
    }
    long bytes = 0;
    for (auto& e : drop) {
        (void)hipFree(e.first);
        bytes += (long)e.second;
    }
    (void)hipGetLastError();
    return bytes;
}

struct Staged {
    void* host = nullptr;     // caller's host pointer (null when device)
    void* dev = nullptr;      // pointer the kernel uses
    size_t bytes = 0;
    bool owned = false;
    int cache_dev = -1;       // device whose stage cache owns `dev` (-1: plain hipMalloc)
    size_t cap = 0;
    Staged() = default;
    Staged(const Staged&) = delete;
    Staged& operator=(const Staged&) = delete;
    ~Staged() {
        if (!owned || !dev) return;
        if (cache_dev >= 0) stage_give(cache_dev, dev, cap);
        else (void)hipFree(dev);
    }
    // Device memory of at least nbytes owned by this object.
    int alloc(size_t nbytes, const char* what) {
        int d = -1;
        if (hipGetDevice(&d) != hipSuccess) {
            (void)hipGetLastError();
            d = -1;
        }
        if (d >= 0 && d < 64) {
            dev = stage_take(d, nbytes, &cap);
            if (dev) cache_dev = d;
        } else if (hipMalloc(&dev, nbytes) != hipSuccess) {
            (void)hipGetLastError();
            dev = nullptr;
        }
        if (!dev) return fail(RAC_ERR_ALLOC, "%s of %zu bytes failed", what, nbytes);
        owned = true;
        return RAC_OK;
    }
    // Make `p` (bytes long) visible to the device; copy host contents in when
    // `copy_in`.
    int bind(const void* p, size_t nbytes, bool copy_in, hipStream_t s) {
        bytes = nbytes;
        if (!p) return RAC_OK;
        if (is_device_pointer(p)) {
            dev = const_cast<void*>(p);
            return RAC_OK;
        }
        host = const_cast<void*>(p);
        if (nbytes == 0) return RAC_OK;
        const int rc = alloc(nbytes, "device staging allocation");
        if (rc) return rc;
        if (copy_in)
            return check_hip(hipMemcpyAsync(dev, p, nbytes, hipMemcpyHostToDevice, s), "staging copy in");
        return RAC_OK;
    }
    int copy_out(hipStream_t s) {
        if (!owned || !host || bytes == 0) return RAC_OK;
        return check_hip(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, s), "staging copy out");
    }
    float* f() const { return static_cast<float*>(dev); }
};

static int finish_sync(hipStream_t s, int rc) {
    const int rc2 = check_hip(hipStreamSynchronize(s), "stream synchronize");
    return rc != RAC_OK ? rc : rc2;
}

// ── argument checks shared by both API styles ────────────────────────────

static int check_gemm(const void* A, const void* B, const void* C, long M, long N, long K) {
    if (!A || !B || !C) return fail(RAC_ERR_NULL_PTR, "rac_matmul: null operand");
    if (M <= 0 || N <= 0 || K <= 0) return fail(RAC_ERR_INVALID_DIM, "rac_matmul: M, N, K must be > 0 (got %ld, %ld, %ld)", M, N, K);
    if ((N + 15) / 16 > 2147483647L || (M + 15) / 16 > 65535L * 64)
        return fail(RAC_ERR_INVALID_DIM, "rac_matmul: shape too large for one launch");
    return RAC_OK;
}

static int check_rows(const char* who, const void* x, const void* y, long rows, long n) {
    if (!x || !y) return fail(RAC_ERR_NULL_PTR, "%s: null buffer", who);
    if (rows <= 0 || n <= 0) return fail(RAC_ERR_INVALID_DIM, "%s: rows and row length must be > 0", who);
    if (rows > 16777215L) return fail(RAC_ERR_INVALID_DIM, "%s: at most 16777215 rows per call", who);
    return RAC_OK;
}

static int check_rope(const void* x, const void* c, const void* s, long b, long h, long t, long d) {
    if (!x || !c || !s) return fail(RAC_ERR_NULL_PTR, "rac_rope_apply: null buffer");
    if (b <= 0 || h <= 0 || t <= 0 || d <= 0 || (d & 1))
        return fail(RAC_ERR_INVALID_DIM, "rac_rope_apply: dims must be > 0 and head_dim even");
    return RAC_OK;
}

// ═════════════════════════ rac_ext.h: device API ══════════════════════════

RAC_EXPORT int rac_gemm_dev(const float* A, const float* B, float* C, int M, int N, int K,
                            int trans_a, int trans_b, float alpha, float beta, int iters,
                            int mode, void* stream) {
    int rc = check_gemm(A, B, C, M, N, K);
    if (rc) return rc;
    if (mode < 0 || mode > 2) return fail(RAC_ERR_INVALID_DIM, "rac_gemm_dev: mode must be 0, 1 or 2");
    return check_hip(gemm_launch(trans_a != 0, trans_b != 0, A, B, C, M, N, K, alpha, beta,
                                 clamp_iters(iters), mode, (hipStream_t)stream),
                     "rac_gemm_dev launch");
}

RAC_EXPORT int rac_gemm_batched_dev(const float* A, const float* B, float* C, int M, int N, int K,
                                    int trans_a, int trans_b, float alpha, float beta, int iters,
                                    int mode, int batch, long stride_a, long stride_b, long stride_c,
                                    void* stream) {
    int rc = check_gemm(A, B, C, M, N, K);
    if (rc) return rc;
    if (mode < 0 || mode > 2) return fail(RAC_ERR_INVALID_DIM, "rac_gemm_batched_dev: mode must be 0, 1 or 2");
    if (batch <= 0 || batch > 65535) return fail(RAC_ERR_INVALID_DIM, "rac_gemm_batched_dev: batch must be in [1, 65535]");
    if (stride_a < 0 || stride_b < 0 || stride_c < 0)
        return fail(RAC_ERR_INVALID_DIM, "rac_gemm_batched_dev: negative stride");
    return check_hip(gemm_launch(trans_a != 0, trans_b != 0, A, B, C, M, N, K, alpha, beta,
                                 clamp_iters(iters), mode, (hipStream_t)stream, batch, stride_a, stride_b,
                                 stride_c),
                     "rac_gemm_batched_dev launch");
}

// output[M,N] = act(input[M,K] weight[N,K]^T + bias) in one launch
// (rac_torch.cu:705-780 with the RAC MAC of `mode`); pre, when not null,
// receives the pre-activation (what the backward pass needs).
RAC_EXPORT int rac_fused_linear_dev(const float* input, const float* weight, const float* bias, float* out,
                                    float* pre, int M, int N, int K, int act, int iters, int mode,
                                    void* stream) {
    int rc = check_gemm(input, weight, out, M, N, K);
    if (rc) return rc;
    if (mode < 0 || mode > 2) return fail(RAC_ERR_INVALID_DIM, "rac_fused_linear_dev: mode must be 0, 1 or 2");
    if (act < 0 || act > 3) return fail(RAC_ERR_INVALID_DIM, "rac_fused_linear_dev: act must be 0..3");
    GemmEpilogue ep;
    ep.bias = bias;
    ep.pre = pre;
    ep.act = act;
    ep.khinv = host_consts().exp_khinv[clamp_iters(iters)];
    return check_hip(gemm_fused_launch(input, weight, out, M, N, K, ep, iters, mode, (hipStream_t)stream),
                     "rac_fused_linear_dev launch");
}

// d[i] = g[i] * act'(pre[i]) for the activation ids of rac_fused_linear_dev.
RAC_EXPORT int rac_act_grad_dev(const float* g, const float* pre, float* d, long count, int act, int iters,
                                void* stream) {
    if (!g || !pre || !d) return fail(RAC_ERR_NULL_PTR, "rac_act_grad_dev: null buffer");
    if (count < 0) return fail(RAC_ERR_INVALID_DIM, "rac_act_grad_dev: negative count");
    if (act < 0 || act > 3) return fail(RAC_ERR_INVALID_DIM, "rac_act_grad_dev: act must be 0..3");
    if (count == 0) return RAC_OK;
    return check_hip(act_grad_launch(g, pre, d, count, act, iters, (hipStream_t)stream),
                     "rac_act_grad_dev launch");
}

// Row softmax with attention masking of rows laid out as [.., seq, seq]:
// causal and/or an additive [seq, seq] mask (either may be off); in place
// when x == y.
RAC_EXPORT int rac_softmax_masked_dev(const float* x, float* y, long rows, long seq, const float* mask,
                                      int is_causal, int iters, void* stream) {
    int rc = check_rows("rac_softmax_masked_dev", x, y, rows, seq);
    if (rc) return rc;
    if (rows % seq) return fail(RAC_ERR_INVALID_DIM, "rac_softmax_masked_dev: rows must be a multiple of seq");
    SoftmaxMask mk;
    mk.mask = mask;
    mk.causal = is_causal != 0;
    mk.seq = seq;
    mk.zero_guard = 1;
    return check_hip(softmax_launch(x, y, rows, seq, iters, (hipStream_t)stream, mk),
                     "rac_softmax_masked_dev launch");
}

RAC_EXPORT int rac_softmax_dev(const float* x, float* y, long rows, long n, int iters, void* stream) {
    int rc = check_rows("rac_softmax_dev", x, y, rows, n);
    if (rc) return rc;
    return check_hip(softmax_launch(x, y, rows, n, iters, (hipStream_t)stream), "rac_softmax_dev launch");
}

// ── decode step (bench_rac_transformer.c decoder_forward_kv, T_new = 1) ──

// Grouped-query attention of one token over positions 0 .. *pos of the
// cache (bench_rac_transformer.c:508-548, query head h on key/value head
// h / (n_heads / n_kv_heads)).
RAC_EXPORT int rac_decode_attention_dev(const float* q, const float* k_cache, const float* v_cache, float* out,
                                        int n_heads, int n_kv_heads, int d_head, long t_cap, const int* pos,
                                        float scale, int iters, void* stream) {
    if (!q || !k_cache || !v_cache || !out || !pos)
        return fail(RAC_ERR_NULL_PTR, "rac_decode_attention_dev: null buffer");
    if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads)
        return fail(RAC_ERR_INVALID_DIM, "rac_decode_attention_dev: n_heads must be a positive multiple of n_kv_heads");
    if (n_heads > 65535) return fail(RAC_ERR_INVALID_DIM, "rac_decode_attention_dev: at most 65535 heads");
    if (d_head <= 0 || d_head > kDecodeMaxHead)
        return fail(RAC_ERR_INVALID_DIM, "rac_decode_attention_dev: d_head must be in [1, %d]", kDecodeMaxHead);
    if (t_cap <= 0 || t_cap > kDecodeMaxLen)
        return fail(RAC_ERR_INVALID_DIM, "rac_decode_attention_dev: t_cap must be in [1, %d]", kDecodeMaxLen);
    return check_hip(decode_attention_launch(q, k_cache, v_cache, out, n_heads, n_kv_heads, d_head, t_cap, pos,
                                             scale, iters, (hipStream_t)stream),
                     "rac_decode_attention_dev launch");
}

// The new token's keys and values into the cache at *pos
// (bench_rac_transformer.c:569-574).
RAC_EXPORT int rac_kv_append_dev(const float* kv, float* k_cache, float* v_cache, int n_kv_heads, int d_head,
                                 long t_cap, const int* pos, void* stream) {
    if (!kv || !k_cache || !v_cache || !pos) return fail(RAC_ERR_NULL_PTR, "rac_kv_append_dev: null buffer");
    if (n_kv_heads <= 0 || d_head <= 0 || t_cap <= 0)
        return fail(RAC_ERR_INVALID_DIM, "rac_kv_append_dev: sizes must be positive");
    return check_hip(kv_append_launch(kv, k_cache, v_cache, n_kv_heads, d_head, t_cap, pos, (hipStream_t)stream),
                     "rac_kv_append_dev launch");
}

// The decode step's fused one-row GEMVs: x is normalised inside the GEMV
// (rac_rmsnorm_dev's arithmetic and order), so K must take the row kernel's
// 16-byte form (K % 4 == 0, K <= 16384) and the GEMV its fast layout
// (K % 256 == 0); x, norm_weight and the weights 16-byte aligned.
static int check_fused_gemv(const char* who, const float* x, const float* g, const void* w, long rows, int K) {
    if (!x || !g || !w) return fail(RAC_ERR_NULL_PTR, "%s: null buffer", who);
    if (rows <= 0 || rows > 2147483647L) return fail(RAC_ERR_INVALID_DIM, "%s: bad row count", who);
    if (K <= 0 || K % 256 || K > 16384)
        return fail(RAC_ERR_INVALID_DIM, "%s: K must be a multiple of 256 and at most 16384", who);
    const uintptr_t a = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(g) |
                        reinterpret_cast<uintptr_t>(w);
    if (a & 15) return fail(RAC_ERR_INVALID_DIM, "%s: x, norm_weight and weight must be 16-byte aligned", who);
    return RAC_OK;
}

// out = act(W rmsnorm(x) * norm_weight + bias) for one row
// (bench_rac_transformer.c:566-567 / :605-606, norm then projection).
RAC_EXPORT int rac_q8_0_gemv_rmsnorm_dev(const float* x, const float* norm_weight, float eps, const void* weight,
                                         const float* bias, float* out, int N, int K, int act, void* stream) {
    int rc = check_fused_gemv("rac_q8_0_gemv_rmsnorm_dev", x, norm_weight, weight, N, K);
    if (rc) return rc;
    if (!out) return fail(RAC_ERR_NULL_PTR, "rac_q8_0_gemv_rmsnorm_dev: null output");
    if (act < 0 || act > 3) return fail(RAC_ERR_INVALID_DIM, "rac_q8_0_gemv_rmsnorm_dev: act must be 0..3");
    return check_hip(q8_rmsnorm_gemv_launch(x, norm_weight, eps, static_cast<const uint8_t*>(weight), bias, out, N,
                                            K, act, (hipStream_t)stream),
                     "rac_q8_0_gemv_rmsnorm_dev launch");
}

// Q, K and V of the new token (:566-574): weight rows (n_heads + 2
// n_kv_heads) * d_head over K = d_model; the queries to q_out, keys and
// values into the caches at *pos.
RAC_EXPORT int rac_decode_qkv_dev(const float* x, const float* norm_weight, float eps, const void* weight,
                                  float* q_out, float* k_cache, float* v_cache, int n_heads, int n_kv_heads,
                                  int d_head, int K, long t_cap, const int* pos, void* stream) {
    if (!q_out || !k_cache || !v_cache || !pos) return fail(RAC_ERR_NULL_PTR, "rac_decode_qkv_dev: null buffer");
    if (n_heads <= 0 || n_kv_heads <= 0 || d_head <= 0 || t_cap <= 0)
        return fail(RAC_ERR_INVALID_DIM, "rac_decode_qkv_dev: sizes must be positive");
    const long rows = (long)(n_heads + 2L * n_kv_heads) * d_head;
    int rc = check_fused_gemv("rac_decode_qkv_dev", x, norm_weight, weight, rows, K);
    if (rc) return rc;
    return check_hip(q8_decode_qkv_launch(x, norm_weight, eps, static_cast<const uint8_t*>(weight), q_out,
                                          n_heads * d_head, k_cache, v_cache, n_kv_heads * d_head, d_head, t_cap,
                                          pos, K, (hipStream_t)stream),
                     "rac_decode_qkv_dev launch");
}

// Gate and up of the SwiGLU feed-forward (:605-611) in one GEMV: weight
// rows interleave gate_0, up_0, gate_1, up_1, ...; out[i] = silu(gate_i)
// * up_i over h = rmsnorm(x) * norm_weight.
RAC_EXPORT int rac_decode_swiglu_gemv_dev(const float* x, const float* norm_weight, float eps, const void* weight,
                                          float* out, int n_ff, int K, int iters, void* stream) {
    if (!out) return fail(RAC_ERR_NULL_PTR, "rac_decode_swiglu_gemv_dev: null output");
    if (n_ff <= 0 || n_ff > 1073741823) return fail(RAC_ERR_INVALID_DIM, "rac_decode_swiglu_gemv_dev: bad n_ff");
    int rc = check_fused_gemv("rac_decode_swiglu_gemv_dev", x, norm_weight, weight, 2L * n_ff, K);
    if (rc) return rc;
    return check_hip(q8_decode_swiglu_launch(x, norm_weight, eps, static_cast<const uint8_t*>(weight), out, n_ff, K,
                                             iters, (hipStream_t)stream),
                     "rac_decode_swiglu_gemv_dev launch");
}

// *pos += by on the stream (full_model_forward's cur_len += T_new, :624).
RAC_EXPORT int rac_position_advance_dev(int* pos, int by, void* stream) {
    if (!pos) return fail(RAC_ERR_NULL_PTR, "rac_position_advance_dev: null buffer");
    return check_hip(position_advance_launch(pos, by, (hipStream_t)stream), "rac_position_advance_dev launch");
}

// out[i] = silu(gu[i]) * gu[n + i] (bench_rac_transformer.c:607-611, SiLU
// by the CORDIC exp).
RAC_EXPORT int rac_swiglu_dev(const float* gu, float* out, long n, int iters, void* stream) {
    if (!gu || !out) return fail(RAC_ERR_NULL_PTR, "rac_swiglu_dev: null buffer");
    if (n < 0) return fail(RAC_ERR_INVALID_DIM, "rac_swiglu_dev: negative count");
    if (n == 0) return RAC_OK;
    return check_hip(swiglu_launch(gu, out, n, iters, (hipStream_t)stream), "rac_swiglu_dev launch");
}

static int elt_dev(const char* who, int op, const float* x, float* y, long count, int iters, void* stream) {
    if (!x || !y) return fail(RAC_ERR_NULL_PTR, "%s: null buffer", who);
    if (count < 0) return fail(RAC_ERR_INVALID_DIM, "%s: negative count", who);
    if (count == 0) return RAC_OK;
    return check_hip(eltwise_launch(op, x, y, count, iters, (hipStream_t)stream), who);
}

RAC_EXPORT int rac_exp_dev(const float* x, float* y, long count, int iters, void* stream) {
    return elt_dev("rac_exp_dev", kEltExp, x, y, count, iters, stream);
}
RAC_EXPORT int rac_silu_dev(const float* x, float* y, long count, int iters, void* stream) {
    return elt_dev("rac_silu_dev", kEltSilu, x, y, count, iters, stream);
}
RAC_EXPORT int rac_sigmoid_dev(const float* x, float* y, long count, int iters, void* stream) {
    return elt_dev("rac_sigmoid_dev", kEltSigmoid, x, y, count, iters, stream);
}
RAC_EXPORT int rac_tanh_dev(const float* x, float* y, long count, int iters, void* stream) {
    return elt_dev("rac_tanh_dev", kEltTanh, x, y, count, iters, stream);
}
RAC_EXPORT int rac_gelu_dev(const float* x, float* y, long count, void* stream) {
    return elt_dev("rac_gelu_dev", kEltGelu, x, y, count, 0, stream);
}
RAC_EXPORT int rac_relu_dev(const float* x, float* y, long count, void* stream) {
    return elt_dev("rac_relu_dev", kEltRelu, x, y, count, 0, stream);
}

RAC_EXPORT int rac_rsqrt_dev(const float* x, float* y, long count, void* stream) {
    if (!x || !y) return fail(RAC_ERR_NULL_PTR, "rac_rsqrt_dev: null buffer");
    if (count < 0) return fail(RAC_ERR_INVALID_DIM, "rac_rsqrt_dev: negative count");
    if (count == 0) return RAC_OK;
    return check_hip(rsqrt_launch(x, y, count, (hipStream_t)stream), "rac_rsqrt_dev launch");
}

RAC_EXPORT int rac_sincos_dev(const float* theta, float* s, float* c, long count, void* stream) {
    if (!theta || !s || !c) return fail(RAC_ERR_NULL_PTR, "rac_sincos_dev: null buffer");
    if (count < 0) return fail(RAC_ERR_INVALID_DIM, "rac_sincos_dev: negative count");
    if (count == 0) return RAC_OK;
    return check_hip(sincos_launch(theta, s, c, count, (hipStream_t)stream), "rac_sincos_dev launch");
}

RAC_EXPORT int rac_rmsnorm_dev(const float* x, float* y, const float* gamma, float eps, long rows,
                               long d, void* stream) {
    int rc = check_rows("rac_rmsnorm_dev", x, y, rows, d);
    if (rc) return rc;
    return check_hip(rmsnorm_launch(x, y, gamma, eps, rows, d, (hipStream_t)stream), "rac_rmsnorm_dev launch");
}

RAC_EXPORT int rac_layernorm_dev(const float* x, float* y, const float* gamma, const float* beta,
                                 float eps, long rows, long d, void* stream) {
    int rc = check_rows("rac_layernorm_dev", x, y, rows, d);
    if (rc) return rc;
    return check_hip(layernorm_launch(x, y, gamma, beta, eps, rows, d, (hipStream_t)stream),
                     "rac_layernorm_dev launch");
}

// inv_freq[i] = 1.0f / powf(base, (2.0f*i)/head_dim) on the host, as
// rac_cpu.c:588-589 computes it (glibc powf; the angle p*inv_freq and the
// CORDIC rotation run on the device).
static void rope_inv_freq(float* inv, int head_dim, float base) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        const float exponent = (2.0f * (float)i) / (float)head_dim;
        inv[i] = 1.0f / powf(base, exponent);
    }
}

RAC_EXPORT int rac_rope_cache_dev(float* cos_out, float* sin_out, int max_seq, int head_dim,
                                  float base, const float* inv_freq_dev, void* stream) {
    // inv_freq_dev: device buffer of head_dim/2 floats filled by
    // rac_rope_inv_freq (the caller owns it, so no allocation happens here).
    if (!cos_out || !sin_out || !inv_freq_dev) return fail(RAC_ERR_NULL_PTR, "rac_rope_cache_dev: null buffer");
    if (max_seq <= 0 || head_dim <= 0 || (head_dim & 1))
        return fail(RAC_ERR_INVALID_DIM, "rac_rope_cache_dev: max_seq > 0 and even head_dim > 0 required");
    (void)base;
    return check_hip(rope_cache_launch(cos_out, sin_out, inv_freq_dev, max_seq, head_dim / 2,
                                       (hipStream_t)stream),
                     "rac_rope_cache_dev launch");
}

RAC_EXPORT int rac_rope_inv_freq(float* inv_freq_host, int head_dim, float base) {
    if (!inv_freq_host) return fail(RAC_ERR_NULL_PTR, "rac_rope_inv_freq: null buffer");
    if (head_dim <= 0 || (head_dim & 1)) return fail(RAC_ERR_INVALID_DIM, "rac_rope_inv_freq: even head_dim > 0 required");
    rope_inv_freq(inv_freq_host, head_dim, base);
    return RAC_OK;
}

RAC_EXPORT int rac_rope_apply_dev(float* x, const float* cos_tab, const float* sin_tab, int batch,
                                  int n_heads, int seq, int head_dim, long stride_b, long stride_h,
                                  long stride_t, void* stream) {
    int rc = check_rope(x, cos_tab, sin_tab, batch, n_heads, seq, head_dim);
    if (rc) return rc;
    return check_hip(rope_apply_launch(x, cos_tab, sin_tab, batch, n_heads, seq, head_dim, stride_b,
                                       stride_h, stride_t, (hipStream_t)stream),
                     "rac_rope_apply_dev launch");
}

// rac_rope_apply (rac_cpu.c:600-635) out of place: rows read at x with
// strides (stride_b, stride_h, stride_t), the rotated rows written at y with
// (out_b, out_h, out_t); x and y must not overlap.  One read and one write
// per element, where a copy followed by the in-place call moves twice that.
RAC_EXPORT int rac_rope_apply_out_dev(const float* x, float* y, const float* cos_tab, const float* sin_tab,
                                      int batch, int n_heads, int seq, int head_dim, long stride_b,
                                      long stride_h, long stride_t, long out_b, long out_h, long out_t,
                                      void* stream) {
    int rc = check_rope(x, cos_tab, sin_tab, batch, n_heads, seq, head_dim);
    if (rc) return rc;
    if (!y) return fail(RAC_ERR_NULL_PTR, "rac_rope_apply_out_dev: null output");
    return check_hip(rope_apply_out_launch(x, y, cos_tab, sin_tab, batch, n_heads, seq, head_dim, stride_b,
                                           stride_h, stride_t, out_b, out_h, out_t, (hipStream_t)stream),
                     "rac_rope_apply_out_dev launch");
}

// ── vector primitives on device buffers ──────────────────────────────────

// Which operands each primitive op reads / writes (see PrimOp).
static bool prim_needs_b(int op) {
    return op == kPrimDot || op == kPrimCoherence || op == kPrimComplexMul || op == kPrimInnerTerm;
}
static bool prim_needs_theta(int op) {
    return op == kPrimRotate || op == kPrimRotateRaw || op == kPrimProject || op == kPrimRotateN ||
           op == kPrimProjectN;
}
static bool prim_writes_pair(int op) {
    return op == kPrimRotate || op == kPrimRotateRaw || op == kPrimCompensate || op == kPrimPolar ||
           op == kPrimNormalize || op == kPrimComplexMul || op == kPrimRotateN;
}

static int check_prim(int op, long n, const void* a, const void* b, const void* th, const void* o2,
                      const void* o1) {
    if (op < kPrimRotate || op > kPrimInnerTerm) return fail(RAC_ERR_INVALID_DIM, "rac_vec2_dev: unknown op %d", op);
    if (n < 0) return fail(RAC_ERR_INVALID_DIM, "rac_vec2_dev: negative count");
    if (n > 2147483647L * 128L) return fail(RAC_ERR_INVALID_DIM, "rac_vec2_dev: count too large for one launch");
    if (!a || (prim_needs_b(op) && !b) || (prim_needs_theta(op) && !th) ||
        (prim_writes_pair(op) ? !o2 : !o1))
        return fail(RAC_ERR_NULL_PTR, "rac_vec2_dev: null operand for op %d", op);
    return RAC_OK;
}

RAC_EXPORT int rac_vec2_dev(int op, long n, const float* a, const float* b, const float* theta,
                            int iarg, float* out2, float* out1, void* stream) {
    int rc = check_prim(op, n, a, b, theta, out2, out1);
    if (rc || n == 0) return rc;
    return check_hip(prim_launch(op, n, reinterpret_cast<const float2*>(a), reinterpret_cast<const float2*>(b),
                                 theta, iarg, reinterpret_cast<float2*>(out2), out1, (hipStream_t)stream),
                     "rac_vec2_dev launch");
}

RAC_EXPORT int rac_inner_dev(const float* a, const float* b, long n, float* out, void* stream) {
    if (!a || !b || !out) return fail(RAC_ERR_NULL_PTR, "rac_inner_dev: null buffer");
    if (n < 0) return fail(RAC_ERR_INVALID_DIM, "rac_inner_dev: negative count");
    return check_hip(inner_launch(reinterpret_cast<const float2*>(a), reinterpret_cast<const float2*>(b), n, out,
                                  (hipStream_t)stream),
                     "rac_inner_dev launch");
}

RAC_EXPORT int rac_outer_dev(const float* a, const float* b, float* C, int m, int n, void* stream) {
    if (!a || !b || !C) return fail(RAC_ERR_NULL_PTR, "rac_outer_dev: null buffer");
    if (m < 0 || n < 0) return fail(RAC_ERR_INVALID_DIM, "rac_outer_dev: negative dimension");
    if ((long)m * n > 2147483647L * 128L) return fail(RAC_ERR_INVALID_DIM, "rac_outer_dev: too large for one launch");
    if ((long)m * n == 0) return RAC_OK;
    return check_hip(outer_launch(reinterpret_cast<const float2*>(a), reinterpret_cast<const float2*>(b), C, m, n,
                                  (hipStream_t)stream),
                     "rac_outer_dev launch");
}

RAC_EXPORT int rac_dct_dev(const float* x, float* X, int n, void* stream) {
    if (!x || !X) return fail(RAC_ERR_NULL_PTR, "rac_dct_dev: null buffer");
    if (n < 0) return fail(RAC_ERR_INVALID_DIM, "rac_dct_dev: negative length");
    if (n == 0) return RAC_OK;
    return check_hip(dct_launch(x, X, n, (hipStream_t)stream), "rac_dct_dev launch");
}

// ── scaled dot-product attention (rac.h:323-335) ────────────────────────

static int check_attention(const void* q, const void* k, const void* v, const void* out, long b,
                           long h, long t, long d) {
    if (!q || !k || !v || !out) return fail(RAC_ERR_NULL_PTR, "rac_attention: null buffer");
    if (b <= 0 || h <= 0 || t <= 0 || d <= 0) return fail(RAC_ERR_INVALID_DIM, "rac_attention: dims must be > 0");
    if (b * h > 65535L) return fail(RAC_ERR_INVALID_DIM, "rac_attention: batch*n_heads must be <= 65535");
    // one softmax workgroup per score row: at most 16777215 rows per launch
    if (b * h * t > 16777215L || t > 2147483647L / 16)
        return fail(RAC_ERR_INVALID_DIM, "rac_attention: batch*n_heads*seq must be <= 16777215");
    return RAC_OK;
}

// The attention core runs over chunks of `chunk` query rows: per chunk the
// scores of those rows against every key, [batch*n_heads, chunk, seq] in the
// workspace, the masked softmax of those full-length rows in place, and
// their P V rows.  Every score, probability and output element is computed
// exactly as with one chunk of all seq rows (each score row keeps its full
// length, so the softmax's row sum has the same order), so the chunk size
// never changes a result; it only bounds the workspace by
// 4 * batch*n_heads * chunk * seq bytes instead of 4 * batch*n_heads * seq^2.
// The workspace ends with 256 bytes for a device flag.
static constexpr long kAttnChunkBudget = 128L << 20;

static long attention_scores_bytes(long bh, long seq, long chunk) {
    return (long)sizeof(float) * bh * chunk * seq;
}

// Query rows per chunk for a workspace budget: all seq rows when their
// scores fit it, else the largest multiple of 64 rows that does (64 at
// least, or seq when shorter).
static long attention_chunk_rows(long bh, long seq, long budget) {
    const long per_row = attention_scores_bytes(bh, seq, 1);
    long c = budget / per_row;
    if (c >= seq) return seq;
    c = (c / 64) * 64;
    return c >= 64 ? c : (seq < 64 ? seq : 64);
}

RAC_EXPORT long rac_attention_workspace_bytes(int batch, int n_heads, int seq) {
    if (batch <= 0 || n_heads <= 0 || seq <= 0) return 0;
    const long bh = (long)batch * n_heads;
    return attention_scores_bytes(bh, seq, attention_chunk_rows(bh, seq, kAttnChunkBudget)) + 256;
}

// The workspace of rac_attention_probs_dev: all [batch*n_heads, seq, seq]
// probabilities (what the backward pass reads) plus the flag.
RAC_EXPORT long rac_attention_probs_workspace_bytes(int batch, int n_heads, int seq) {
    if (batch <= 0 || n_heads <= 0 || seq <= 0) return 0;
    return attention_scores_bytes((long)batch * n_heads, seq, seq) + 256;
}

// scores = (Q K^T) / sqrt(D) by the RAC matmul (batched over b*h), masked
// row softmax with CORDIC exp in place, out = P V by the RAC matmul; over
// query chunks of `chunk` rows (see above).
// Probabilities of query rows t0 .. t0+c-1 of every head into P [bh, c, t]
// (scores, then the masked softmax in place).  Each score is one
// accumulator over d in order and each softmax row the full row, so P does
// not depend on the chunk: these are rows t0.. of the one-chunk P, bit for
// bit.
static int attention_probs_chunk(const float* q, const float* k, const float* mask, int causal, float* P,
                                 int bh, int t, int d, long t0, int c, int iters, int mode, hipStream_t s) {
    const long td = (long)t * d;
    const float scale = 1.0f / sqrtf((float)d);
    // causal: score tiles wholly above the diagonal are masked by the
    // softmax regardless of their contents, so the scores GEMM schedules
    // only the tiles on or below it (the whole sequence: the square
    // triangular schedule; a chunk: its trapezoid).  Both products keep the
    // literal-chain recompute of the public GEMM (exact_specials): operands
    // outside the strength-reduced chain's range (in P V, the probabilities
    // below 2^-105 of a peaked softmax row) are rotated as the reference
    // does, so every output equals the reference composition bit for bit.
    // Cost, measured at [1, 32, 2048, 128] causal n = 16: ~3-6% of the
    // attention core on unscaled inputs, ~2x when Q and K are scaled by 4.
    const int ssched = !causal ? 0 : ((c == t && t0 == 0) ? 1 : 3);
    int rc = check_hip(gemm_launch(0, 1, q + t0 * d, k, P, c, t, d, scale, 0.0f, iters, mode, s, bh, td, td,
                                   (long)c * t, ssched, nullptr, true, (int)t0),
                       "rac_attention scores launch");
    if (rc) return rc;
    SoftmaxMask mk;
    mk.mask = mask;
    mk.causal = causal != 0;
    mk.seq = c;
    mk.row0 = t0;
    mk.mask_ld = t;
    mk.zero_guard = 1;
    return check_hip(softmax_launch(P, P, (long)bh * c, t, iters, s, mk), "rac_attention softmax launch");
}

static int attention_launch(const float* q, const float* k, const float* v, const float* mask, int causal,
                            float* out, int b, int h, int t, int d, float* ws, long chunk, int iters, int mode,
                            hipStream_t s) {
    const int bh = b * h;
    const long td = (long)t * d;
    // causal: P is exactly 0 above the diagonal, so P V may stop each row
    // tile's K loop at its last query position -- when V is finite (0 * inf
    // is NaN); the flag lives in the workspace tail, evaluated on the device
    int* flag = nullptr;
    int rc = RAC_OK;
    if (causal) {
        flag = reinterpret_cast<int*>(reinterpret_cast<char*>(ws) + attention_scores_bytes(bh, t, chunk));
        rc = check_hip(all_finite_launch(v, (long)bh * td, flag, s), "rac_attention finite check");
        if (rc) return rc;
    }
    for (long t0 = 0; t0 < t; t0 += chunk) {
        const int c = (int)(chunk < t - t0 ? chunk : t - t0);
        const long ct = (long)c * t;
        rc = attention_probs_chunk(q, k, mask, causal, ws, bh, t, d, t0, c, iters, mode, s);
        if (rc) return rc;
        // causal: row tiles paired for balance (the GEMM falls back to the
        // plain schedule where pairing leaves too few workgroups)
        const int psched = causal ? 2 : 0;
        rc = check_hip(gemm_launch(0, 0, ws, v, out + t0 * d, c, d, t, 1.0f, 0.0f, iters, mode, s, bh, ct, td, td,
                                   psched, flag, true, (int)t0),
                       "rac_attention output launch");
        if (rc) return rc;
    }
    return RAC_OK;
}

RAC_EXPORT int rac_attention_dev(const float* q, const float* k, const float* v, const float* mask,
                                 int is_causal, float* out, int batch, int n_heads, int seq,
                                 int head_dim, float* workspace, int iters, int mode, void* stream) {
    int rc = check_attention(q, k, v, out, batch, n_heads, seq, head_dim);
    if (rc) return rc;
    if (!workspace) return fail(RAC_ERR_NULL_PTR, "rac_attention_dev: null workspace");
    if (mode < 0 || mode > 2) return fail(RAC_ERR_INVALID_DIM, "rac_attention_dev: mode must be 0, 1 or 2");
    const long bh = (long)batch * n_heads;
    return attention_launch(q, k, v, mask, is_causal, out, batch, n_heads, seq, head_dim, workspace,
                            attention_chunk_rows(bh, seq, kAttnChunkBudget), clamp_iters(iters), mode,
                            (hipStream_t)stream);
}

// Query rows per chunk that a workspace of `bytes` holds: all seq rows when
// they fit, else the largest multiple of 64 rows that fits, else as many
// rows as fit (0 when not even one row does).
static long attention_chunk_for_bytes(long bh, long seq, long bytes) {
    const long per_row = attention_scores_bytes(bh, seq, 1);
    const long c = (bytes - 256) / per_row;
    if (c >= seq) return seq;
    if (c >= 64) return (c / 64) * 64;
    return c > 0 ? c : 0;
}

// rac_attention_dev with the workspace size given: the chunk is the largest
// the workspace holds (results do not depend on it).
RAC_EXPORT int rac_attention_ws_dev(const float* q, const float* k, const float* v, const float* mask,
                                    int is_causal, float* out, int batch, int n_heads, int seq, int head_dim,
                                    float* workspace, long workspace_bytes, int iters, int mode, void* stream) {
    int rc = check_attention(q, k, v, out, batch, n_heads, seq, head_dim);
    if (rc) return rc;
    if (!workspace) return fail(RAC_ERR_NULL_PTR, "rac_attention_ws_dev: null workspace");
    if (mode < 0 || mode > 2) return fail(RAC_ERR_INVALID_DIM, "rac_attention_ws_dev: mode must be 0, 1 or 2");
    const long bh = (long)batch * n_heads;
    const long chunk = attention_chunk_for_bytes(bh, seq, workspace_bytes);
    if (chunk < 1)
        return fail(RAC_ERR_INVALID_DIM, "rac_attention_ws_dev: workspace of %ld bytes is below the %ld one query "
                    "row of every head needs", workspace_bytes, attention_scores_bytes(bh, seq, 1) + 256);
    return attention_launch(q, k, v, mask, is_causal, out, batch, n_heads, seq, head_dim, workspace, chunk,
                            clamp_iters(iters), mode, (hipStream_t)stream);
}

// ── allocation-free attention ────────────────────────────────────────────
//
// For callers that cannot allocate device memory (code under stream or
// graph capture, serving loops that forbid allocation): the chunk workspace
// lives in this file-scope device array, kScratchBytes (64 MiB + 256 B) per
// GPU, held by each GPU the library runs on until the process ends.  It
// holds 256 query rows of every head at [1, 32, 2048, 128] (smaller chunks
// leave the causal P V launches too few workgroups: 64-row chunks took
// 16.3 ms there against 10.0 ms), and one query row of every head for every
// shape the argument check accepts (batch*n_heads*seq <= 16777215).  Every
// call on one GPU shares that GPU's array: calls that overlap on one GPU
// (other streams, other host threads) race and must be serialised by the
// caller.
// The array's device address is looked up once per device (the host-side
// name is only a stand-in for it) and used from then on.  The lookup is set
// up outside any stream capture: rac_create_context does it for the current
// device, and so does the first call of rac_attention_noalloc_dev on a device
// when its stream is not capturing.  A first call that arrives under
// capture is refused (-4) instead of querying the runtime there (the lookup
// may load the library's code object, which allocates the array).
static constexpr long kScratchBytes = (64L << 20) + 256;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[64];

static int scratch_for_current_device(hipStream_t stream, void** out) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= 64) return fail(RAC_ERR_DEVICE, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        if (stream) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            rc = check_hip(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing");
            if (rc) return rc;
            if (cs != hipStreamCaptureStatusNone)
                return fail(RAC_ERR_DEVICE, "rac_attention_noalloc_dev: the first call on device %d is under stream "
                            "capture; call rac_create_context (or make one call) outside capture first", dev);
        }
        void* p = nullptr;
        rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "scratch address");
        if (rc) return rc;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return RAC_OK;
}

// rac_attention_dev without a workspace argument and without allocating:
// the chunks of query rows are sized to the library's scratch array
// (results equal rac_attention_dev's).  Shapes beyond the argument check's
// limit (batch*n_heads*seq > 16777215, whose one query row of every head
// would not fit the array either) are refused before any device work.
RAC_EXPORT int rac_attention_noalloc_dev(const float* q, const float* k, const float* v, const float* mask,
                                         int is_causal, float* out, int batch, int n_heads, int seq,
                                         int head_dim, int iters, int mode, void* stream) {
    int rc = check_attention(q, k, v, out, batch, n_heads, seq, head_dim);
    if (rc) return rc;
    if (mode < 0 || mode > 2) return fail(RAC_ERR_INVALID_DIM, "rac_attention_noalloc_dev: mode must be 0, 1 or 2");
    const long bh = (long)batch * n_heads;
    const long chunk = attention_chunk_for_bytes(bh, seq, kScratchBytes);
    if (chunk < 1)
        return fail(RAC_ERR_INVALID_DIM, "rac_attention_noalloc_dev: batch*n_heads*seq = %ld exceeds the %ld the "
                    "%ld-byte scratch holds", bh * seq, (kScratchBytes - 256) / (long)sizeof(float), kScratchBytes);
    void* ws = nullptr;
    rc = scratch_for_current_device((hipStream_t)stream, &ws);
    if (rc) return rc;
    return attention_launch(q, k, v, mask, is_causal, out, batch, n_heads, seq, head_dim, static_cast<float*>(ws),
                            chunk, clamp_iters(iters), mode, (hipStream_t)stream);
}

// rac_attention_dev in one chunk: the workspace (of
// rac_attention_probs_workspace_bytes) keeps every probability P [batch,
// n_heads, seq, seq] in its first batch*n_heads*seq*seq floats.
RAC_EXPORT int rac_attention_probs_dev(const float* q, const float* k, const float* v, const float* mask,
                                       int is_causal, float* out, int batch, int n_heads, int seq,
                                       int head_dim, float* workspace, int iters, int mode, void* stream) {
    int rc = check_attention(q, k, v, out, batch, n_heads, seq, head_dim);
    if (rc) return rc;
    if (!workspace) return fail(RAC_ERR_NULL_PTR, "rac_attention_probs_dev: null workspace");
    if (mode < 0 || mode > 2) return fail(RAC_ERR_INVALID_DIM, "rac_attention_probs_dev: mode must be 0, 1 or 2");
    return attention_launch(q, k, v, mask, is_causal, out, batch, n_heads, seq, head_dim, workspace, seq,
                            clamp_iters(iters), mode, (hipStream_t)stream);
}

// The probabilities of query rows row0 .. row0+rows-1 of every head,
// P [batch*n_heads, rows, seq], equal to those rows of rac_attention_probs_dev's
// P: for a backward pass that recomputes P a chunk at a time instead of
// keeping the [batch*n_heads, seq, seq] matrix.
RAC_EXPORT int rac_attention_probs_rows_dev(const float* q, const float* k, const float* mask, int is_causal,
                                            float* P, int batch, int n_heads, int seq, int head_dim, int row0,
                                            int rows, int iters, int mode, void* stream) {
    int rc = check_attention(q, k, k, P, batch, n_heads, seq, head_dim);
    if (rc) return rc;
    if (mode < 0 || mode > 2) return fail(RAC_ERR_INVALID_DIM, "rac_attention_probs_rows_dev: mode must be 0, 1 or 2");
    if (row0 < 0 || rows <= 0 || (long)row0 + rows > seq)
        return fail(RAC_ERR_INVALID_DIM, "rac_attention_probs_rows_dev: rows %d .. %ld outside 0 .. %d", row0,
                    (long)row0 + rows - 1, seq - 1);
    return attention_probs_chunk(q, k, mask, is_causal, P, batch * n_heads, seq, head_dim, row0, rows,
                                 clamp_iters(iters), mode, (hipStream_t)stream);
}

// ── Q8_0 weights and decode GEMV (lib/c/rac_q8_0.h) ─────────────────────

static int check_q8(const char* who, const void* a, const void* b, long rows, long K) {
    if (!a || !b) return fail(RAC_ERR_NULL_PTR, "%s: null buffer", who);
    if (rows <= 0 || K <= 0 || K % 32) return fail(RAC_ERR_INVALID_DIM, "%s: rows > 0 and K a positive multiple of 32 required", who);
    if (rows * (K / 32) > 2147483647L * 128L) return fail(RAC_ERR_INVALID_DIM, "%s: too many blocks", who);
    return RAC_OK;
}

RAC_EXPORT int rac_q8_0_gemv_dev(const float* x, const void* weight, const float* bias, float* out, int M, int N,
                                 int K, int act, void* stream) {
    int rc = check_q8("rac_q8_0_gemv_dev", x, weight, N, K);
    if (rc) return rc;
    if (!out) return fail(RAC_ERR_NULL_PTR, "rac_q8_0_gemv_dev: null output");
    if (M <= 0) return fail(RAC_ERR_INVALID_DIM, "rac_q8_0_gemv_dev: M must be > 0");
    if (act < 0 || act > 3) return fail(RAC_ERR_INVALID_DIM, "rac_q8_0_gemv_dev: act must be 0..3");
    if ((long)M * N > 2147483647L * 2L) return fail(RAC_ERR_INVALID_DIM, "rac_q8_0_gemv_dev: M*N too large");
    return check_hip(q8_gemv_launch(x, static_cast<const uint8_t*>(weight), bias, out, M, N, K, act,
                                    (hipStream_t)stream),
                     "rac_q8_0_gemv_dev launch");
}

RAC_EXPORT int rac_q8_0_quantize_dev(const float* src, void* dst, long rows, int K, void* stream) {
    int rc = check_q8("rac_q8_0_quantize_dev", src, dst, rows, K);
    if (rc) return rc;
    return check_hip(q8_quantize_launch(src, static_cast<uint8_t*>(dst), rows * (K / 32), (hipStream_t)stream),
                     "rac_q8_0_quantize_dev launch");
}

RAC_EXPORT int rac_q8_0_dequantize_dev(const void* src, float* dst, long rows, int K, void* stream) {
    int rc = check_q8("rac_q8_0_dequantize_dev", src, dst, rows, K);
    if (rc) return rc;
    return check_hip(q8_dequantize_launch(static_cast<const uint8_t*>(src), dst, rows * (K / 32),
                                          (hipStream_t)stream),
                     "rac_q8_0_dequantize_dev launch");
}

// ── RAC-DSP integer CORDIC engine (sim/rac_dsp_core.h) ──────────────────

// ROM contents: generated by the rule of rtl/gen_coarse_lut.py:27-123 (LUT
// entry k = direction bits of a 10-step double-precision circular CORDIC
// driving (k - 512 + 0.5) pi / 1024 to zero; atan / atanh constants
// round(v / pi * 2^63)), or replaced by rac_load_all_roms.  A copy lives
// in device memory per GPU, refreshed when the host contents change.
static std::mutex g_dsp_mutex;
static DspRoms g_dsp_roms;
static int g_dsp_version = 0;            // 0: not generated yet
struct DspDeviceRoms {
    DspRoms* ptr = nullptr;
    int version = -1;
};
static DspDeviceRoms g_dsp_dev[64];

static int64_t q063_frac_pi(double v) { return (int64_t)nearbyint(v / M_PI * 9223372036854775808.0); }

static void dsp_derive(DspRoms& r);

static void dsp_generate_roms(DspRoms& r) {
    for (int k = 0; k < kDspLut; k++) {
        double z = (k - kDspLut / 2 + 0.5) * M_PI / kDspLut;
        unsigned bits = 0;
        for (int i = 0; i < kDspLutBits; i++) {
            const double step = atan(ldexp(1.0, -i));
            if (z >= 0.0) { z -= step; bits |= 1u << i; }
            else z += step;
        }
        r.lut[k] = (uint16_t)bits;
    }
    for (int i = 0; i < kDspAtan; i++) r.atan_rom[i] = q063_frac_pi(atan(ldexp(1.0, -i)));
    for (int i = 0; i < kDspRes; i++) r.atanh_rom[i] = q063_frac_pi(atanh(ldexp(1.0, -(kDspResStart + i))));
    dsp_derive(r);
}

// The coarse stage's z bookkeeping depends only on the LUT word and the atan
// ROM; sums wrap modulo 2^64, so the table equals the step-by-step update.
static void dsp_derive(DspRoms& r) {
    for (int k = 0; k < kDspLut; k++) {
        uint64_t za = 0;
        for (int i = 0; i < kDspLutBits; i++)
            za = ((r.lut[k] >> i) & 1u) ? za + (uint64_t)r.atan_rom[i] : za - (uint64_t)r.atan_rom[i];
        r.coarse_z[k] = (int64_t)za;
    }
}

// Device copy of the current ROMs for the current device (allocated once per
// device and kept for the life of the process).
static int dsp_device_roms(const DspRoms** out, hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_dsp_mutex);
    if (g_dsp_version == 0) {
        dsp_generate_roms(g_dsp_roms);
        g_dsp_version = 1;
    }
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= 64) return fail(RAC_ERR_DEVICE, "RAC-DSP: device index %d out of range", dev);
    DspDeviceRoms& d = g_dsp_dev[dev];
    if (!d.ptr) {
        if (hipMalloc(&d.ptr, sizeof(DspRoms)) != hipSuccess) {
            (void)hipGetLastError();
            d.ptr = nullptr;
            return fail(RAC_ERR_ALLOC, "RAC-DSP: ROM buffer allocation failed");
        }
    }
    if (d.version != g_dsp_version) {
        // The buffer is rewritten in place: RAC-DSP kernels queued earlier on
        // any stream of this device must finish reading the old ROMs first.
        rc = check_hip(hipDeviceSynchronize(), "RAC-DSP ROM upload (wait for earlier users)");
        if (rc) return rc;
        rc = check_hip(hipMemcpyAsync(d.ptr, &g_dsp_roms, sizeof(DspRoms), hipMemcpyHostToDevice, s),
                       "RAC-DSP ROM upload");
        if (!rc) rc = check_hip(hipStreamSynchronize(s), "RAC-DSP ROM upload");
        if (rc) return rc;
        d.version = g_dsp_version;
    }
    *out = d.ptr;
    return RAC_OK;
}

// rac_load_hex_lut (sim/rac_dsp_core.c:56-72): $readmemh-style lines; blank
// lines and // comments skipped; returns the count parsed or -1.
RAC_EXPORT int rac_load_hex_lut(const char* path, uint64_t* out, int expected) {
    if (!path || !out) return fail(RAC_ERR_NULL_PTR, "rac_load_hex_lut: null argument");
    FILE* f = fopen(path, "r");
    if (!f) return fail(-1, "rac_load_hex_lut: cannot open %s", path);
    char line[256];
    int n = 0;
    while (fgets(line, sizeof(line), f)) {
        const char* p = line;
        while (*p == ' ' || *p == '\t') p++;
        if (*p == '\0' || *p == '\n' || (*p == '/' && p[1] == '/')) continue;
        unsigned long long v = 0;
        if (sscanf(p, "%llx", &v) != 1) continue;
        if (n < expected) out[n++] = (uint64_t)v;
    }
    fclose(f);
    return n;
}

// rac_load_all_roms (sim/rac_dsp_core.c:74-89): replaces the ROMs used by
// every later RAC-DSP call; 0 on success, 1/2/3 for the LUT/atan/atanh file.
// As in the reference the three files are applied one after the other: a
// file that cannot be opened stops the load with the earlier ROMs already
// replaced, and a file with fewer entries than its ROM replaces only those
// entries.  (The reference keeps the previous entries for a short LUT file
// but copies uninitialised stack words for a short atan or atanh file; here
// every short file keeps the previous entries.)
RAC_EXPORT int rac_load_all_roms(const char* coarse_lut_path, const char* atan_path, const char* atanh_path) {
    std::lock_guard<std::mutex> lock(g_dsp_mutex);
    if (g_dsp_version == 0) {
        dsp_generate_roms(g_dsp_roms);
        g_dsp_version = 1;
    }
    auto publish = [] {
        dsp_derive(g_dsp_roms);
        g_dsp_version = g_dsp_version + 1;
    };
    uint64_t words[kDspLut];
    for (int i = 0; i < kDspLut; i++) words[i] = g_dsp_roms.lut[i];
    if (rac_load_hex_lut(coarse_lut_path, words, kDspLut) < 0) return 1;
    for (int i = 0; i < kDspLut; i++) g_dsp_roms.lut[i] = (uint16_t)(words[i] & 0x3ffu);
    publish();
    for (int i = 0; i < kDspAtan; i++) words[i] = (uint64_t)g_dsp_roms.atan_rom[i];
    if (rac_load_hex_lut(atan_path, words, kDspAtan) < 0) return 2;
    for (int i = 0; i < kDspAtan; i++) g_dsp_roms.atan_rom[i] = (int64_t)words[i];
    publish();
    for (int i = 0; i < kDspRes; i++) words[i] = (uint64_t)g_dsp_roms.atanh_rom[i];
    if (rac_load_hex_lut(atanh_path, words, kDspRes) < 0) return 3;
    for (int i = 0; i < kDspRes; i++) g_dsp_roms.atanh_rom[i] = (int64_t)words[i];
    publish();
    return 0;
}

// Replaces the ROMs from memory (the reference lets callers assign its ROM
// globals directly, sim/rac_dsp_core.h:23-27).  Any pointer may be null to
// keep that ROM.
RAC_EXPORT void rac_dsp_set_roms(const uint64_t* lut, const int64_t* atan_rom, const int64_t* atanh_rom) {
    std::lock_guard<std::mutex> lock(g_dsp_mutex);
    if (g_dsp_version == 0) dsp_generate_roms(g_dsp_roms);
    if (lut) for (int i = 0; i < kDspLut; i++) g_dsp_roms.lut[i] = (uint16_t)(lut[i] & 0x3ffu);
    if (atan_rom) for (int i = 0; i < kDspAtan; i++) g_dsp_roms.atan_rom[i] = atan_rom[i];
    if (atanh_rom) for (int i = 0; i < kDspRes; i++) g_dsp_roms.atanh_rom[i] = atanh_rom[i];
    dsp_derive(g_dsp_roms);
    g_dsp_version = g_dsp_version + 1 + (g_dsp_version == 0);
}

// Host copy of the ROMs in use (generated ones unless replaced).
RAC_EXPORT void rac_dsp_get_roms(uint64_t* lut, int64_t* atan_rom, int64_t* atanh_rom) {
    std::lock_guard<std::mutex> lock(g_dsp_mutex);
    if (g_dsp_version == 0) {
        dsp_generate_roms(g_dsp_roms);
        g_dsp_version = 1;
    }
    if (lut) for (int i = 0; i < kDspLut; i++) lut[i] = g_dsp_roms.lut[i];
    if (atan_rom) for (int i = 0; i < kDspAtan; i++) atan_rom[i] = g_dsp_roms.atan_rom[i];
    if (atanh_rom) for (int i = 0; i < kDspRes; i++) atanh_rom[i] = g_dsp_roms.atanh_rom[i];
}

RAC_EXPORT int rac_dsp_eval_dev(int op, long n, const int64_t* x, const int64_t* y, const int64_t* z, int64_t* xo,
                                int64_t* yo, int64_t* zo, void* stream) {
    if (!x || !z || !xo) return fail(RAC_ERR_NULL_PTR, "rac_dsp_eval_dev: x, z and xo are required");
    if (n < 0) return fail(RAC_ERR_INVALID_DIM, "rac_dsp_eval_dev: negative count");
    if (n == 0) return RAC_OK;
    const DspRoms* roms = nullptr;
    int rc = dsp_device_roms(&roms, (hipStream_t)stream);
    if (rc) return rc;
    return check_hip(dsp_eval_launch(op, n, x, y, z, xo, yo, zo, roms, (hipStream_t)stream),
                     "rac_dsp_eval_dev launch");
}

RAC_EXPORT int rac_dsp_systolic_dev(int N, int K, const int64_t* W, const int64_t* X, int64_t* Y, void* stream) {
    if (!W || !X || !Y) return fail(RAC_ERR_NULL_PTR, "rac_dsp_systolic_dev: null buffer");
    if (N <= 0 || K <= 0 || (long)N * N > 2147483647L || (long)N * K > 2147483647L)
        return fail(RAC_ERR_INVALID_DIM, "rac_dsp_systolic_dev: need N, K > 0 and N*N, N*K < 2^31");
    const DspRoms* roms = nullptr;
    int rc = dsp_device_roms(&roms, (hipStream_t)stream);
    if (rc) return rc;
    return check_hip(dsp_systolic_launch(N, K, W, X, Y, roms, (hipStream_t)stream), "rac_dsp_systolic_dev launch");
}

// ═════════════════ reference launcher ABI (rac_kernels.hip) ═══════════════

RAC_EXPORT void rac_launch_nn_iters(const float* A, const float* B, float* C, int M, int N, int K,
                                    float alpha, float beta, int iters, int mode, void* stream) {
    (void)rac_gemm_dev(A, B, C, M, N, K, 0, 0, alpha, beta, iters, mode, stream);
}
RAC_EXPORT void rac_launch_nt_iters(const float* A, const float* B, float* C, int M, int N, int K,
                                    float alpha, float beta, int iters, int mode, void* stream) {
    (void)rac_gemm_dev(A, B, C, M, N, K, 0, 1, alpha, beta, iters, mode, stream);
}
RAC_EXPORT void rac_launch_tn_iters(const float* A, const float* B, float* C, int M, int N, int K,
                                    float alpha, float beta, int iters, int mode, void* stream) {
    (void)rac_gemm_dev(A, B, C, M, N, K, 1, 0, alpha, beta, iters, mode, stream);
}
RAC_EXPORT void rac_launch_nn(const float* A, const float* B, float* C, int M, int N, int K,
                              float alpha, float beta, void* stream) {
    rac_launch_nn_iters(A, B, C, M, N, K, alpha, beta, 24, kModeFast, stream);
}
RAC_EXPORT void rac_launch_nt(const float* A, const float* B, float* C, int M, int N, int K,
                              float alpha, float beta, void* stream) {
    rac_launch_nt_iters(A, B, C, M, N, K, alpha, beta, 24, kModeFast, stream);
}
RAC_EXPORT void rac_launch_tn(const float* A, const float* B, float* C, int M, int N, int K,
                              float alpha, float beta, void* stream) {
    rac_launch_tn_iters(A, B, C, M, N, K, alpha, beta, 24, kModeFast, stream);
}

// ══════════════════════ rac.h: synchronous API ════════════════════════════

RAC_EXPORT void rac_matmul(float* A, float* B, float* C, int M, int N, int K) {
    if (check_gemm(A, B, C, M, N, K)) return;
    hipStream_t s = g_stream.load();
    Staged a, b, c;
    int rc = a.bind(A, sizeof(float) * (size_t)M * K, true, s);
    if (!rc) rc = b.bind(B, sizeof(float) * (size_t)K * N, true, s);
    if (!rc) rc = c.bind(C, sizeof(float) * (size_t)M * N, false, s);
    if (!rc) rc = check_hip(gemm_launch(0, 0, a.f(), b.f(), c.f(), M, N, K, 1.0f, 0.0f,
                                        rac_get_cordic_iters(), rac_get_cordic_mode(), s),
                            "rac_matmul launch");
    if (!rc) rc = c.copy_out(s);
    (void)finish_sync(s, rc);
}

static void softmax_sync(const float* x, float* out, long rows, long n) {
    if (check_rows("rac_softmax", x, out, rows, n)) return;
    hipStream_t s = g_stream.load();
    const size_t bytes = sizeof(float) * (size_t)rows * n;
    Staged a, b;
    int rc = a.bind(x, bytes, true, s);
    if (!rc) rc = b.bind(out, bytes, false, s);
    if (!rc) rc = check_hip(softmax_launch(a.f(), b.f(), rows, n, rac_get_cordic_iters(), s), "rac_softmax launch");
    if (!rc) rc = b.copy_out(s);
    (void)finish_sync(s, rc);
}

RAC_EXPORT void rac_softmax(float* x, float* out, int n) { softmax_sync(x, out, 1, n); }

// rac_cpu.h:172 signature
RAC_EXPORT void rac_softmax_batch(const float* x, float* out, int batch, int n) {
    softmax_sync(x, out, batch, n);
}

static void elt_sync(const char* who, int op, const float* x, float* out, long n, int iters) {
    if (!x || !out) { fail(RAC_ERR_NULL_PTR, "%s: null buffer", who); return; }
    if (n <= 0) return;
    hipStream_t s = g_stream.load();
    Staged a, b;
    int rc = a.bind(x, sizeof(float) * (size_t)n, true, s);
    if (!rc) rc = b.bind(out, sizeof(float) * (size_t)n, false, s);
    if (!rc) rc = check_hip(eltwise_launch(op, a.f(), b.f(), n, iters, s), who);
    if (!rc) rc = b.copy_out(s);
    (void)finish_sync(s, rc);
}

// rac_cpu.h:169-171 batch activations
RAC_EXPORT void rac_relu(const float* x, float* out, int n) { elt_sync("rac_relu", kEltRelu, x, out, n, 0); }
RAC_EXPORT void rac_gelu(const float* x, float* out, int n) { elt_sync("rac_gelu", kEltGelu, x, out, n, 0); }
RAC_EXPORT void rac_silu(const float* x, float* out, int n) {
    elt_sync("rac_silu", kEltSilu, x, out, n, rac_get_cordic_iters());
}

static float scalar_elt(int op, float x) {
    float y = 0.0f;
    elt_sync("rac scalar op", op, &x, &y, 1, rac_get_cordic_iters());
    return y;
}

RAC_EXPORT float rac_exp(float x) { return scalar_elt(kEltExp, x); }
RAC_EXPORT float rac_tanh(float x) { return scalar_elt(kEltTanh, x); }
RAC_EXPORT float rac_sigmoid(float x) { return scalar_elt(kEltSigmoid, x); }

RAC_EXPORT float rac_rsqrt(float x) {
    hipStream_t s = g_stream.load();
    Staged a, b;
    float y = 0.0f;
    int rc = a.bind(&x, sizeof(float), true, s);
    if (!rc) rc = b.bind(&y, sizeof(float), false, s);
    if (!rc) rc = check_hip(rsqrt_launch(a.f(), b.f(), 1, s), "rac_rsqrt launch");
    if (!rc) rc = b.copy_out(s);
    (void)finish_sync(s, rc);
    return y;
}

RAC_EXPORT void rac_sincos(float theta, float* sp, float* cp) {
    if (!sp || !cp) { fail(RAC_ERR_NULL_PTR, "rac_sincos: null output"); return; }
    hipStream_t s = g_stream.load();
    float sv = 0.0f, cv = 0.0f;
    Staged a, b, c;
    int rc = a.bind(&theta, sizeof(float), true, s);
    if (!rc) rc = b.bind(&sv, sizeof(float), false, s);
    if (!rc) rc = c.bind(&cv, sizeof(float), false, s);
    if (!rc) rc = check_hip(sincos_launch(a.f(), b.f(), c.f(), 1, s), "rac_sincos launch");
    if (!rc) rc = b.copy_out(s);
    if (!rc) rc = c.copy_out(s);
    if (finish_sync(s, rc) == RAC_OK) { *sp = sv; *cp = cv; }
}

RAC_EXPORT void rac_rmsnorm(const float* x, float* y, const float* gamma, float eps, int rows, int d) {
    if (check_rows("rac_rmsnorm", x, y, rows, d)) return;
    hipStream_t s = g_stream.load();
    const size_t bytes = sizeof(float) * (size_t)rows * d;
    Staged a, b, g;
    int rc = a.bind(x, bytes, true, s);
    if (!rc) rc = b.bind(y, bytes, false, s);
    if (!rc) rc = g.bind(gamma, sizeof(float) * (size_t)d, true, s);
    if (!rc) rc = check_hip(rmsnorm_launch(a.f(), b.f(), g.f(), eps, rows, d, s), "rac_rmsnorm launch");
    if (!rc) rc = b.copy_out(s);
    (void)finish_sync(s, rc);
}

RAC_EXPORT void rac_layernorm(const float* x, float* y, const float* gamma, const float* beta,
                              float eps, int rows, int d) {
    if (check_rows("rac_layernorm", x, y, rows, d)) return;
    hipStream_t s = g_stream.load();
    const size_t bytes = sizeof(float) * (size_t)rows * d;
    Staged a, b, g, bt;
    int rc = a.bind(x, bytes, true, s);
    if (!rc) rc = b.bind(y, bytes, false, s);
    if (!rc) rc = g.bind(gamma, sizeof(float) * (size_t)d, true, s);
    if (!rc) rc = bt.bind(beta, sizeof(float) * (size_t)d, true, s);
    if (!rc) rc = check_hip(layernorm_launch(a.f(), b.f(), g.f(), bt.f(), eps, rows, d, s), "rac_layernorm launch");
    if (!rc) rc = b.copy_out(s);
    (void)finish_sync(s, rc);
}

RAC_EXPORT void rac_rope_cache(float* cos_out, float* sin_out, int max_seq, int head_dim, float base) {
    if (!cos_out || !sin_out) { fail(RAC_ERR_NULL_PTR, "rac_rope_cache: null buffer"); return; }
    if (max_seq <= 0 || head_dim <= 0 || (head_dim & 1)) {
        fail(RAC_ERR_INVALID_DIM, "rac_rope_cache: max_seq > 0 and even head_dim > 0 required");
        return;
    }
    hipStream_t s = g_stream.load();
    const int half = head_dim / 2;
    const size_t bytes = sizeof(float) * (size_t)max_seq * half;
    std::string inv_host(sizeof(float) * (size_t)half, '\0');
    rope_inv_freq(reinterpret_cast<float*>(&inv_host[0]), head_dim, base);
    Staged c, sn, inv;
    int rc = c.bind(cos_out, bytes, false, s);
    if (!rc) rc = sn.bind(sin_out, bytes, false, s);
    if (!rc) rc = inv.bind(&inv_host[0], inv_host.size(), true, s);
    if (!rc) rc = check_hip(rope_cache_launch(c.f(), sn.f(), inv.f(), max_seq, half, s), "rac_rope_cache launch");
    if (!rc) rc = c.copy_out(s);
    if (!rc) rc = sn.copy_out(s);
    (void)finish_sync(s, rc);
}

RAC_EXPORT void rac_rope_apply(float* x, const float* cos_tab, const float* sin_tab, int batch,
                               int n_heads, int seq, int head_dim) {
    if (check_rope(x, cos_tab, sin_tab, batch, n_heads, seq, head_dim)) return;
    hipStream_t s = g_stream.load();
    const size_t xbytes = sizeof(float) * (size_t)batch * n_heads * seq * head_dim;
    const size_t tbytes = sizeof(float) * (size_t)seq * (head_dim / 2);
    Staged a, c, sn;
    int rc = a.bind(x, xbytes, true, s);
    if (!rc) rc = c.bind(cos_tab, tbytes, true, s);
    if (!rc) rc = sn.bind(sin_tab, tbytes, true, s);
    const long st = head_dim, sh = (long)seq * head_dim, sb = (long)n_heads * sh;
    if (!rc) rc = check_hip(rope_apply_launch(a.f(), c.f(), sn.f(), batch, n_heads, seq, head_dim, sb, sh, st, s),
                            "rac_rope_apply launch");
    if (!rc) rc = a.copy_out(s);
    (void)finish_sync(s, rc);
}

// ── vector primitives (rac.h:101-250, 345-346) ───────────────────────────
// A pair {float x, y} passed and returned by value: the C layout of the
// reference's float2 (rac.h:31), classified the same way by the host ABI.
struct RacVec2 {
    float x, y;
};

// Runs one primitive op over n items in caller memory (host or device).
static int prim_sync(int op, long n, const void* a, const void* b, const float* th, int iarg, void* o2,
                     float* o1) {
    if (n <= 0) return RAC_OK;
    hipStream_t s = g_stream.load();
    Staged sa, sb, st, so2, so1;
    const size_t n2 = sizeof(float) * 2 * (size_t)n, n1 = sizeof(float) * (size_t)n;
    int rc = sa.bind(a, n2, true, s);
    if (!rc && prim_needs_b(op)) rc = sb.bind(b, n2, true, s);
    if (!rc && prim_needs_theta(op)) rc = st.bind(th, n1, true, s);
    if (!rc && prim_writes_pair(op)) rc = so2.bind(o2, n2, false, s);
    if (!rc && !prim_writes_pair(op)) rc = so1.bind(o1, n1, false, s);
    if (!rc) rc = rac_vec2_dev(op, n, sa.f(), sb.f(), st.f(), iarg, so2.f(), so1.f(), s);
    if (!rc) rc = so2.copy_out(s);
    if (!rc) rc = so1.copy_out(s);
    return finish_sync(s, rc);
}

static RacVec2 prim_pair(int op, RacVec2 a, RacVec2 b, float theta, int iarg) {
    RacVec2 r = {0.0f, 0.0f};
    RacVec2 out = {0.0f, 0.0f};
    if (prim_sync(op, 1, &a, &b, &theta, iarg, &out, nullptr) == RAC_OK) r = out;
    return r;
}
static float prim_scalar(int op, RacVec2 a, RacVec2 b, float theta, int iarg) {
    float out = 0.0f;
    if (prim_sync(op, 1, &a, &b, &theta, iarg, nullptr, &out) != RAC_OK) return 0.0f;
    return out;
}

RAC_EXPORT RacVec2 rac_rotate(RacVec2 v, float theta) { return prim_pair(kPrimRotate, v, v, theta, 0); }
RAC_EXPORT RacVec2 rac_rotate_raw(RacVec2 v, float theta) { return prim_pair(kPrimRotateRaw, v, v, theta, 0); }
RAC_EXPORT RacVec2 rac_compensate(RacVec2 v, int chain_length) {
    return prim_pair(kPrimCompensate, v, v, 0.0f, chain_length);
}
RAC_EXPORT float rac_project(RacVec2 v, float theta) { return prim_scalar(kPrimProject, v, v, theta, 0); }
RAC_EXPORT void rac_polar(RacVec2 v, float* mag, float* angle) {
    if (!mag || !angle) { fail(RAC_ERR_NULL_PTR, "rac_polar: null output"); return; }
    RacVec2 out = {0.0f, 0.0f};
    if (prim_sync(kPrimPolar, 1, &v, nullptr, nullptr, 0, &out, nullptr) == RAC_OK) {
        *mag = out.x;
        *angle = out.y;
    }
}
RAC_EXPORT float rac_norm(RacVec2 v) {
    float m = 0.0f, a = 0.0f;
    rac_polar(v, &m, &a);
    return m;
}
RAC_EXPORT RacVec2 rac_normalize(RacVec2 v) { return prim_pair(kPrimNormalize, v, v, 0.0f, 0); }
RAC_EXPORT float rac_dot(RacVec2 a, RacVec2 b) { return prim_scalar(kPrimDot, a, b, 0.0f, 0); }
RAC_EXPORT float rac_coherence(RacVec2 a, RacVec2 b) { return prim_scalar(kPrimCoherence, a, b, 0.0f, 0); }
RAC_EXPORT RacVec2 rac_complex_mul(RacVec2 a, RacVec2 b) { return prim_pair(kPrimComplexMul, a, b, 0.0f, 0); }
RAC_EXPORT RacVec2 rac_rotate_precision(RacVec2 v, float theta, int iters) {
    return prim_pair(kPrimRotateN, v, v, theta, iters);
}
RAC_EXPORT float rac_project_precision(RacVec2 v, float theta, int iters) {
    return prim_scalar(kPrimProjectN, v, v, theta, iters);
}

RAC_EXPORT void rac_rotate_batch(RacVec2* v, float* theta, RacVec2* out, int n) {
    if (!v || !theta || !out) { fail(RAC_ERR_NULL_PTR, "rac_rotate_batch: null buffer"); return; }
    (void)prim_sync(kPrimRotate, n, v, nullptr, theta, 0, out, nullptr);
}

RAC_EXPORT float rac_inner(RacVec2* a, RacVec2* b, int n) {
    if (!a || !b) { fail(RAC_ERR_NULL_PTR, "rac_inner: null buffer"); return 0.0f; }
    if (n <= 0) return 0.0f;
    hipStream_t s = g_stream.load();
    float result = 0.0f;
    Staged sa, sb, so;
    int rc = sa.bind(a, sizeof(float) * 2 * (size_t)n, true, s);
    if (!rc) rc = sb.bind(b, sizeof(float) * 2 * (size_t)n, true, s);
    if (!rc) rc = so.bind(&result, sizeof(float), false, s);
    if (!rc) rc = rac_inner_dev(sa.f(), sb.f(), n, so.f(), s);
    if (!rc) rc = so.copy_out(s);
    return finish_sync(s, rc) == RAC_OK ? result : 0.0f;
}

RAC_EXPORT void rac_outer(RacVec2* a, RacVec2* b, float* C, int m, int n) {
    if (!a || !b || !C) { fail(RAC_ERR_NULL_PTR, "rac_outer: null buffer"); return; }
    if (m <= 0 || n <= 0) return;
    hipStream_t s = g_stream.load();
    Staged sa, sb, sc;
    int rc = sa.bind(a, sizeof(float) * 2 * (size_t)m, true, s);
    if (!rc) rc = sb.bind(b, sizeof(float) * 2 * (size_t)n, true, s);
    if (!rc) rc = sc.bind(C, sizeof(float) * (size_t)m * n, false, s);
    if (!rc) rc = rac_outer_dev(sa.f(), sb.f(), sc.f(), m, n, s);
    if (!rc) rc = sc.copy_out(s);
    (void)finish_sync(s, rc);
}

RAC_EXPORT void rac_dct(float* x, float* X, int n) {
    if (!x || !X) { fail(RAC_ERR_NULL_PTR, "rac_dct: null buffer"); return; }
    if (n <= 0) return;
    hipStream_t s = g_stream.load();
    Staged sx, sX;
    int rc = sx.bind(x, sizeof(float) * (size_t)n, true, s);
    if (!rc) rc = sX.bind(X, sizeof(float) * (size_t)n, false, s);
    if (!rc) rc = rac_dct_dev(sx.f(), sX.f(), n, s);
    if (!rc) rc = sX.copy_out(s);
    (void)finish_sync(s, rc);
}

RAC_EXPORT void rac_attention(const float* q, const float* k, const float* v, const float* mask,
                              int is_causal, float* out, int batch, int n_heads, int seq, int head_dim) {
    if (check_attention(q, k, v, out, batch, n_heads, seq, head_dim)) return;
    hipStream_t s = g_stream.load();
    const size_t xb = sizeof(float) * (size_t)batch * n_heads * seq * head_dim;
    Staged sq, sk, sv, sm, so, ws;
    int rc = sq.bind(q, xb, true, s);
    if (!rc) rc = sk.bind(k, xb, true, s);
    if (!rc) rc = sv.bind(v, xb, true, s);
    if (!rc) rc = sm.bind(mask, sizeof(float) * (size_t)seq * seq, true, s);
    if (!rc) rc = so.bind(out, xb, false, s);
    const long bh = (long)batch * n_heads;
    const long chunk = attention_chunk_rows(bh, seq, kAttnChunkBudget);
    if (!rc) rc = ws.alloc((size_t)attention_scores_bytes(bh, seq, chunk) + 256, "rac_attention: score workspace");
    if (!rc) rc = attention_launch(sq.f(), sk.f(), sv.f(), sm.f(), is_causal, so.f(), batch, n_heads, seq,
                                   head_dim, ws.f(), chunk, rac_get_cordic_iters(), rac_get_cordic_mode(), s);
    if (!rc) rc = so.copy_out(s);
    (void)finish_sync(s, rc);
}

// ── Q8_0 with the rac_q8_0.h signatures (host or device buffers) ────────

// rac_fp16_to_fp32 / rac_fp32_to_fp16 (rac_q8_0.h:47-48): scalar format
// helpers of the block layout, evaluated on the host.
RAC_EXPORT float rac_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu, bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            int e = -14;
            while ((mant & 0x400u) == 0) { mant <<= 1; e--; }
            mant &= 0x3ffu;
            bits = (sign << 31) | ((uint32_t)(e + 127) << 23) | (mant << 13);
        }
    } else if (ex == 31) {
        bits = (sign << 31) | (0xffu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((ex - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

RAC_EXPORT uint16_t rac_fp32_to_fp16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int ex = (int)((b >> 23) & 0xffu) - 127 + 15;
    uint32_t mant = b & 0x7fffffu;
    if (ex <= 0) {
        if (ex < -10) return (uint16_t)sign;
        mant = (mant | 0x800000u) >> (1 - ex);
        return (uint16_t)(sign | (mant >> 13));
    }
    if (ex >= 31) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    return (uint16_t)(sign | ((uint32_t)ex << 10) | (mant >> 13));
}

static void q8_quantize_sync(const char* who, const float* src, void* dst, long rows, int K) {
    if (check_q8(who, src, dst, rows, K)) return;
    hipStream_t s = g_stream.load();
    const long nblk = rows * (K / 32);
    Staged a, b;
    int rc = a.bind(src, sizeof(float) * (size_t)rows * K, true, s);
    if (!rc) rc = b.bind(dst, 34 * (size_t)nblk, false, s);
    if (!rc) rc = check_hip(q8_quantize_launch(a.f(), static_cast<uint8_t*>(b.dev), nblk, s), who);
    if (!rc) rc = b.copy_out(s);
    (void)finish_sync(s, rc);
}

RAC_EXPORT void rac_q8_0_quantize_row(const float* src, void* dst, int N) {
    q8_quantize_sync("rac_q8_0_quantize_row", src, dst, 1, N);
}
RAC_EXPORT void rac_q8_0_quantize_matrix(const float* src, void* dst, int rows, int K) {
    q8_quantize_sync("rac_q8_0_quantize_matrix", src, dst, rows, K);
}

RAC_EXPORT void rac_q8_0_dequantize_row(const void* src, float* dst, int N) {
    if (check_q8("rac_q8_0_dequantize_row", src, dst, 1, N)) return;
    hipStream_t s = g_stream.load();
    Staged a, b;
    int rc = a.bind(src, 34 * (size_t)(N / 32), true, s);
    if (!rc) rc = b.bind(dst, sizeof(float) * (size_t)N, false, s);
    if (!rc) rc = check_hip(q8_dequantize_launch(static_cast<const uint8_t*>(a.dev), b.f(), N / 32, s),
                            "rac_q8_0_dequantize_row launch");
    if (!rc) rc = b.copy_out(s);
    (void)finish_sync(s, rc);
}

// rac_q8_0_gemv (rac_q8_0.h:94-100): returns the rac_status code.
RAC_EXPORT int rac_q8_0_gemv(const float* input, const void* weight, const float* bias, float* output, int N,
                             int K, int act) {
    int rc = check_q8("rac_q8_0_gemv", input, weight, N, K);
    if (rc) return rc;
    if (!output) return fail(RAC_ERR_NULL_PTR, "rac_q8_0_gemv: null output");
    hipStream_t s = g_stream.load();
    Staged a, w, bb, o;
    rc = a.bind(input, sizeof(float) * (size_t)K, true, s);
    if (!rc) rc = w.bind(weight, 34 * (size_t)N * (K / 32), true, s);
    if (!rc) rc = bb.bind(bias, sizeof(float) * (size_t)N, true, s);
    if (!rc) rc = o.bind(output, sizeof(float) * (size_t)N, false, s);
    if (!rc) rc = rac_q8_0_gemv_dev(a.f(), w.dev, bb.f(), o.f(), 1, N, K, act, s);
    if (!rc) rc = o.copy_out(s);
    return finish_sync(s, rc);
}

// ── RAC-DSP with the sim/rac_dsp_core.h signatures (host or device) ─────

static int dsp_sync(int op, long n, const int64_t* x, const int64_t* y, const int64_t* z, int64_t* xo, int64_t* yo,
                    int64_t* zo) {
    if (n <= 0) return RAC_OK;
    hipStream_t s = g_stream.load();
    const size_t b = sizeof(int64_t) * (size_t)n;
    Staged sx, sy, sz, ox, oy, oz;
    int rc = sx.bind(x, b, true, s);
    if (!rc) rc = sy.bind(y, b, true, s);
    if (!rc) rc = sz.bind(z, b, true, s);
    if (!rc) rc = ox.bind(xo, b, false, s);
    if (!rc) rc = oy.bind(yo, b, false, s);
    if (!rc) rc = oz.bind(zo, b, false, s);
    if (!rc) rc = rac_dsp_eval_dev(op, n, static_cast<const int64_t*>(sx.dev), static_cast<const int64_t*>(sy.dev),
                                   static_cast<const int64_t*>(sz.dev), static_cast<int64_t*>(ox.dev),
                                   static_cast<int64_t*>(oy.dev), static_cast<int64_t*>(oz.dev), s);
    if (!rc) rc = ox.copy_out(s);
    if (!rc) rc = oy.copy_out(s);
    if (!rc) rc = oz.copy_out(s);
    return finish_sync(s, rc);
}

// sim/rac_dsp_core.h:41-42
RAC_EXPORT void rac_dsp_eval(int64_t x_in, int64_t y_in, int64_t z_in, int op, int64_t* x_out, int64_t* y_out,
                             int64_t* z_out) {
    if (!x_out || !y_out || !z_out) { fail(RAC_ERR_NULL_PTR, "rac_dsp_eval: null output"); return; }
    int64_t xo = 0, yo = 0, zo = 0;
    if (dsp_sync(op, 1, &x_in, &y_in, &z_in, &xo, &yo, &zo) == RAC_OK) {
        *x_out = xo;
        *y_out = yo;
        *z_out = zo;
    }
}

// sim/rac_dsp_core.h:48-50: x_out[i] = project(xs[i], 0, zs[i]).x
RAC_EXPORT void rac_dsp_project_batch(int n, const int64_t* xs, const int64_t* zs, int64_t* x_out) {
    if (!xs || !zs || !x_out) { fail(RAC_ERR_NULL_PTR, "rac_dsp_project_batch: null buffer"); return; }
    (void)dsp_sync(1, n, xs, nullptr, zs, x_out, nullptr, nullptr);
}

// sim/rac_dsp_core.h:57-58: sum of the n projections (wrapping int64)
RAC_EXPORT int64_t rac_dsp_project_sum(int n, const int64_t* xs, const int64_t* zs) {
    if (!xs || !zs) { fail(RAC_ERR_NULL_PTR, "rac_dsp_project_sum: null buffer"); return 0; }
    if (n <= 0) return 0;
    hipStream_t s = g_stream.load();
    const size_t b = sizeof(int64_t) * (size_t)n;
    // the n projections run on the GPU; their wrapping sum is taken here
    std::string buf(b, '\0');
    Staged sx, sz, ox;
    int rc = sx.bind(xs, b, true, s);
    if (!rc) rc = sz.bind(zs, b, true, s);
    if (!rc) rc = ox.bind(&buf[0], b, false, s);
    if (!rc) rc = rac_dsp_eval_dev(1, n, static_cast<const int64_t*>(sx.dev), nullptr,
                                   static_cast<const int64_t*>(sz.dev), static_cast<int64_t*>(ox.dev), nullptr,
                                   nullptr, s);
    if (!rc) rc = ox.copy_out(s);
    if (finish_sync(s, rc) != RAC_OK) return 0;
    uint64_t sum = 0;
    const int64_t* v = reinterpret_cast<const int64_t*>(buf.data());
    for (int i = 0; i < n; i++) sum += (uint64_t)v[i];
    return (int64_t)sum;
}

// ── context (rac.h:85-88; the reference's HIP backend is a stub,
//    rac_hip.cpp:416-435: every op but RAC_OP_EXTENDED is "supported") ────

struct rac_context_t {
    int backend;
};

// The reference's context is a malloc'd stub (rac_hip.cpp:416-435); here it
// is also the library's set-up call: it resolves the allocation-free
// attention's scratch address for the current device, outside any capture
// (a missing device is not an error for the stub).
RAC_EXPORT rac_context_t* rac_create_context(int backend) {
    rac_context_t* c = (rac_context_t*)malloc(sizeof(rac_context_t));
    if (c) c->backend = backend;
    int n = 0;
    if (hipGetDeviceCount(&n) == hipSuccess && n > 0) {
        void* p = nullptr;
        (void)scratch_for_current_device(nullptr, &p);
    }
    (void)hipGetLastError();
    return c;
}
RAC_EXPORT void rac_destroy_context(rac_context_t* ctx) { free(ctx); }
RAC_EXPORT int rac_query_capability(rac_context_t* ctx, int op) {
    (void)ctx;
    return op == 0xFF ? 0 : 1;
}
RAC_EXPORT int rac_execute(rac_context_t* ctx, int op, void* desc) {
    (void)ctx; (void)op; (void)desc;
    return 0;
}
