// rac_safetensors.hip — safetensors weights into HBM (the reader of
// bench/safetensors_reader.h, with the element conversion on the GPU).
//
// Host: the file is mapped read-only and its JSON header parsed into the
// reference's st_file / st_tensor records.  Device: a tensor streams from
// the mapping through two pinned staging buffers (host threads copy chunk
// c+1 out of the page cache while chunk c crosses PCIe) into a device
// staging buffer, where one kernel widens it to fp32 (F16 / BF16 / F64; F32
// goes straight to its destination) or quantizes it to Q8_0 blocks in the
// same pass.  Conversions are bit-exact with the reference's host loops
// (safetensors_reader.c:375-425) and, for Q8_0, with its quantizer applied
// to those fp32 values.
#include <hip/hip_runtime.h>
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <algorithm>
#include <mutex>
#include <thread>
#include <vector>
#include "rac_internal.hpp"
#include "rac_q8.hpp"
#include "../../include/rac_safetensors.h"

#define RAC_EXPORT extern "C" __attribute__((visibility("default")))

extern "C" void* rac_get_stream(void);

namespace rac {

// Element size of the dtypes st_to_f32 converts (0 for the others).
static int st_float_size(int dt) {
    switch (dt) {
    case ST_F32: return 4;
    case ST_F16: return 2;
    case ST_BF16: return 2;
    case ST_F64: return 8;
    default: return 0;
    }
}

// Element size of every known dtype (0 for ST_UNKNOWN).
static int st_elem_size(int dt) {
    switch (dt) {
    case ST_I8: case ST_U8: case ST_BOOL: return 1;
    case ST_I16: return 2;
    case ST_I32: return 4;
    case ST_I64: return 8;
    default: return st_float_size(dt);
    }
}

// ── device conversion ────────────────────────────────────────────────────

// (float)d as x86-64's cvtsd2ss produces it: round to nearest even, and a
// NaN keeps its sign and top 22 payload bits with the quiet bit set.
__device__ __forceinline__ float f64_bits_to_float(uint64_t b) {
    if (((b >> 52) & 0x7ffu) == 0x7ffu && (b & 0xfffffffffffffull)) {
        const uint32_t r = ((uint32_t)(b >> 32) & 0x80000000u) | 0x7fc00000u | (uint32_t)((b >> 29) & 0x3fffffu);
        return __uint_as_float(r);
    }
    return (float)__longlong_as_double((long long)b);
}

template <int DT>
__device__ __forceinline__ float st_load(const uint8_t* p, long i) {
    if constexpr (DT == ST_F32) return reinterpret_cast<const float*>(p)[i];
    else if constexpr (DT == ST_F16) return half_bits_to_float(reinterpret_cast<const uint16_t*>(p)[i]);
    else if constexpr (DT == ST_BF16) return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
    else return f64_bits_to_float(reinterpret_cast<const uint64_t*>(p)[i]);
}

template <int DT>
constexpr int st_size() { return DT == ST_F32 ? 4 : DT == ST_F64 ? 8 : 2; }

// 8 consecutive elements from 16-byte loads.
template <int DT>
__device__ __forceinline__ void st_load8(const uint8_t* p, long i0, float (&v)[8]) {
    using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
    constexpr int W = st_size<DT>() * 8 / 16;                 // 16-byte words per 8 elements
    const u32x4* q = reinterpret_cast<const u32x4*>(p + i0 * st_size<DT>());
    u32x4 w[W];
#pragma unroll
    for (int k = 0; k < W; k++) w[k] = __builtin_nontemporal_load(q + k);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        if constexpr (DT == ST_F32) {
            v[e] = __uint_as_float(w[e / 4][e % 4]);
        } else if constexpr (DT == ST_F64) {
            const uint64_t b = (uint64_t)w[e / 2][(e % 2) * 2] | ((uint64_t)w[e / 2][(e % 2) * 2 + 1] << 32);
            v[e] = f64_bits_to_float(b);
        } else {
            const uint32_t h = (w[0][e / 2] >> (16 * (e % 2))) & 0xffffu;
            v[e] = (DT == ST_F16) ? half_bits_to_float(h) : __uint_as_float(h << 16);
        }
    }
}

// n elements -> fp32, 8 per lane per trip; `vec`: src and dst 16-byte aligned.
template <int DT>
__global__ __launch_bounds__(256) void st_convert_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                         long n, int vec) {
    const long groups = (n + 7) / 8;
    const long stride = (long)gridDim.x * blockDim.x;
    for (long g = (long)blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += stride) {
        const long i0 = g * 8;
        if (vec && i0 + 8 <= n) {
            float v[8];
            st_load8<DT>(src, i0, v);
            using f32x4 = float __attribute__((ext_vector_type(4)));
            f32x4* o = reinterpret_cast<f32x4*>(dst + i0);
            __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, o);
            __builtin_nontemporal_store(f32x4{v[4], v[5], v[6], v[7]}, o + 1);
        } else {
            for (long i = i0; i < n && i < i0 + 8; i++) dst[i] = st_load<DT>(src, i);
        }
    }
}

// One lane per Q8_0 block: 32 elements widened to fp32, then quantized as
// rac_q8_0_quantize_row does.
template <int DT>
__global__ __launch_bounds__(256) void st_quantize_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                          long nblocks, int vec) {
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    float v[kQ8Block];
    if (vec) {
#pragma unroll
        for (int k = 0; k < kQ8Block / 8; k++) {
            float w[8];
            st_load8<DT>(src, b * kQ8Block + k * 8, w);
#pragma unroll
            for (int e = 0; e < 8; e++) v[k * 8 + e] = w[e];
        }
    } else {
#pragma unroll
        for (int i = 0; i < kQ8Block; i++) v[i] = st_load<DT>(src, b * kQ8Block + i);
    }
    q8_quantize_block(v, dst + b * kQ8Bytes);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

hipError_t st_convert_launch(int dtype, const void* src, long n, float* dst, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long blocks = ((n + 7) / 8 + 255) / 256;
    blocks = std::min(blocks, 256L * 64);
    const dim3 g((unsigned)blocks), b(256);
    const int vec = aligned16(src) && aligned16(dst);
    const uint8_t* p = static_cast<const uint8_t*>(src);
    switch (dtype) {
    case ST_F32: hipLaunchKernelGGL(st_convert_kernel<ST_F32>, g, b, 0, s, p, dst, n, vec); break;
    case ST_F16: hipLaunchKernelGGL(st_convert_kernel<ST_F16>, g, b, 0, s, p, dst, n, vec); break;
    case ST_BF16: hipLaunchKernelGGL(st_convert_kernel<ST_BF16>, g, b, 0, s, p, dst, n, vec); break;
    case ST_F64: hipLaunchKernelGGL(st_convert_kernel<ST_F64>, g, b, 0, s, p, dst, n, vec); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t st_quantize_launch(int dtype, const void* src, long nblocks, uint8_t* dst, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    const dim3 g((unsigned)((nblocks + 255) / 256)), b(256);
    const int vec = aligned16(src);
    const uint8_t* p = static_cast<const uint8_t*>(src);
    switch (dtype) {
    case ST_F32: hipLaunchKernelGGL(st_quantize_kernel<ST_F32>, g, b, 0, s, p, dst, nblocks, vec); break;
    case ST_F16: hipLaunchKernelGGL(st_quantize_kernel<ST_F16>, g, b, 0, s, p, dst, nblocks, vec); break;
    case ST_BF16: hipLaunchKernelGGL(st_quantize_kernel<ST_BF16>, g, b, 0, s, p, dst, nblocks, vec); break;
    case ST_F64: hipLaunchKernelGGL(st_quantize_kernel<ST_F64>, g, b, 0, s, p, dst, nblocks, vec); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ── header parsing (JSON subset: objects, arrays, strings, numbers, literals) ──

namespace {

struct Scan {
    const char* p;
    const char* end;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) {
            p++;
            return true;
        }
        return false;
    }
    bool peek(char c) {
        ws();
        return p < end && *p == c;
    }
    // Quoted string; the raw bytes between the quotes (escapes left as is).
    bool str(const char** s, size_t* n) {
        ws();
        if (p >= end || *p != '"') return false;
        const char* q = ++p;
        while (p < end && *p != '"') p += (*p == '\\') ? 2 : 1;
        if (p >= end) return false;
        *s = q;
        *n = (size_t)(p - q);
        p++;
        return true;
    }
    bool integer(int64_t* v) {
        ws();
        const char* q = p;
        if (p < end && (*p == '-' || *p == '+')) p++;
        const char* digits = p;
        while (p < end && *p >= '0' && *p <= '9') p++;
        if (p == digits || p - q > 20) return false;
        char buf[24];
        memcpy(buf, q, (size_t)(p - q));
        buf[p - q] = '\0';
        errno = 0;
        *v = strtoll(buf, nullptr, 10);
        return errno == 0;
    }
    // Skip one value of any kind.
    bool skip(int depth = 0) {
        ws();
        if (p >= end || depth > 64) return false;
        if (*p == '"') {
            const char* s;
            size_t n;
            return str(&s, &n);
        }
        if (*p == '{' || *p == '[') {
            const char close = (*p == '{') ? '}' : ']';
            const bool obj = (*p == '{');
            p++;
            if (eat(close)) return true;
            for (;;) {
                if (obj) {
                    const char* s;
                    size_t n;
                    if (!str(&s, &n) || !eat(':')) return false;
                }
                if (!skip(depth + 1)) return false;
                if (eat(close)) return true;
                if (!eat(',')) return false;
            }
        }
        const char* q = p;   // number or literal
        while (p < end && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\t' && *p != '\n' &&
               *p != '\r')
            p++;
        return p > q;
    }
};

st_dtype dtype_of(const char* s, size_t n) {
    static const struct { const char* name; st_dtype dt; } kNames[] = {
        {"F32", ST_F32}, {"F16", ST_F16}, {"BF16", ST_BF16}, {"F64", ST_F64}, {"I8", ST_I8},
        {"U8", ST_U8},   {"I16", ST_I16}, {"I32", ST_I32},   {"I64", ST_I64}, {"BOOL", ST_BOOL},
    };
    for (const auto& k : kNames)
        if (strlen(k.name) == n && !memcmp(k.name, s, n)) return k.dt;
    return ST_UNKNOWN;
}

bool key_is(const char* s, size_t n, const char* k) { return strlen(k) == n && !memcmp(s, k, n); }

}  // namespace

static int st_fail(st_file* f, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
static int st_fail(st_file* f, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(f->err, sizeof f->err, fmt, ap);
    va_end(ap);
    return -1;
}

// One tensor record {"dtype": ..., "shape": [...], "data_offsets": [a, b]}.
static int parse_tensor(st_file* f, Scan& sc, st_tensor* t, size_t data_len) {
    if (!sc.eat('{')) return st_fail(f, "tensor '%s': expected an object", t->name);
    bool have_dtype = false, have_shape = false, have_offsets = false;
    int64_t a = 0, b = 0;
    if (!sc.eat('}')) {
        for (;;) {
            const char* k;
            size_t kn;
            if (!sc.str(&k, &kn) || !sc.eat(':')) return st_fail(f, "tensor '%s': malformed field", t->name);
            if (key_is(k, kn, "dtype")) {
                const char* v;
                size_t vn;
                if (!sc.str(&v, &vn)) return st_fail(f, "tensor '%s': dtype is not a string", t->name);
                t->dtype = dtype_of(v, vn);
                have_dtype = true;
            } else if (key_is(k, kn, "shape")) {
                if (!sc.eat('[')) return st_fail(f, "tensor '%s': shape is not an array", t->name);
                t->ndim = 0;
                if (!sc.eat(']')) {
                    for (;;) {
                        int64_t d;
                        if (!sc.integer(&d) || d < 0) return st_fail(f, "tensor '%s': bad dimension", t->name);
                        if (t->ndim == ST_MAX_NDIM)
                            return st_fail(f, "tensor '%s': more than %d dimensions", t->name, ST_MAX_NDIM);
                        t->shape[t->ndim++] = d;
                        if (sc.eat(']')) break;
                        if (!sc.eat(',')) return st_fail(f, "tensor '%s': bad shape", t->name);
                    }
                }
                have_shape = true;
            } else if (key_is(k, kn, "data_offsets")) {
                if (!sc.eat('[') || !sc.integer(&a) || !sc.eat(',') || !sc.integer(&b) || !sc.eat(']'))
                    return st_fail(f, "tensor '%s': data_offsets must be [begin, end]", t->name);
                have_offsets = true;
            } else if (!sc.skip()) {
                return st_fail(f, "tensor '%s': malformed value", t->name);
            }
            if (sc.eat('}')) break;
            if (!sc.eat(',')) return st_fail(f, "tensor '%s': expected ',' or '}'", t->name);
        }
    }
    if (!have_dtype || !have_shape || !have_offsets)
        return st_fail(f, "tensor '%s': dtype, shape and data_offsets are required", t->name);
    if (a < 0 || b < a || (uint64_t)b > data_len)
        return st_fail(f, "tensor '%s': data_offsets [%lld, %lld] outside the %zu-byte data segment", t->name,
                       (long long)a, (long long)b, data_len);
    t->offset = (size_t)a;
    t->nbytes = (size_t)(b - a);
    const int es = st_elem_size(t->dtype);
    if (es) {
        unsigned __int128 want = (unsigned __int128)es;
        for (int i = 0; i < t->ndim; i++) want *= (uint64_t)t->shape[i];
        if (want != (unsigned __int128)t->nbytes)
            return st_fail(f, "tensor '%s': %zu bytes do not hold its shape", t->name, t->nbytes);
    }
    return 0;
}

static int parse_header(st_file* f, const char* json, size_t len, size_t data_len) {
    Scan sc{json, json + len};
    if (!sc.eat('{')) return st_fail(f, "header is not a JSON object");
    if (sc.eat('}')) return 0;
    for (;;) {
        const char* k;
        size_t kn;
        if (!sc.str(&k, &kn) || !sc.eat(':'))
            return st_fail(f, "expected a key at header byte %ld", (long)(sc.p - json));
        if (key_is(k, kn, "__metadata__")) {   // informational
            if (!sc.skip()) return st_fail(f, "malformed __metadata__");
        } else {
            if (f->n_tensors >= ST_MAX_TENSORS) return st_fail(f, "more than %d tensors", ST_MAX_TENSORS);
            st_tensor* t = &f->tensors[f->n_tensors];
            const size_t c = std::min(kn, (size_t)ST_MAX_NAME - 1);
            memcpy(t->name, k, c);
            t->name[c] = '\0';
            if (parse_tensor(f, sc, t, data_len)) return -1;
            f->n_tensors++;
        }
        if (sc.eat('}')) return 0;
        if (!sc.eat(',')) return st_fail(f, "expected ',' or '}' at header byte %ld", (long)(sc.p - json));
    }
}

// ── staging pool: two pinned + two device chunk buffers per device ────────

constexpr size_t kStChunk = 32u << 20;

struct StPool {
    uint8_t* pinned[2] = {nullptr, nullptr};
    uint8_t* draw[2] = {nullptr, nullptr};
    hipEvent_t h2d[2] = {nullptr, nullptr};   // pinned[b] has been read by its copy
    hipEvent_t kern[2] = {nullptr, nullptr};  // draw[b] has been read by its kernel
};

static std::mutex g_st_mutex;
static StPool g_st_pool[64];
static int g_st_open = 0;

static void pool_release_all() {
    for (int d = 0; d < 64; d++) {
        StPool& P = g_st_pool[d];
        if (!P.pinned[0] && !P.draw[0] && !P.h2d[0]) continue;
        int cur = 0;
        (void)hipGetDevice(&cur);
        (void)hipSetDevice(d);
        for (int b = 0; b < 2; b++) {
            if (P.h2d[b]) (void)hipEventSynchronize(P.h2d[b]);
            if (P.kern[b]) (void)hipEventSynchronize(P.kern[b]);
            if (P.pinned[b]) (void)hipHostFree(P.pinned[b]);
            if (P.draw[b]) (void)hipFree(P.draw[b]);
            if (P.h2d[b]) (void)hipEventDestroy(P.h2d[b]);
            if (P.kern[b]) (void)hipEventDestroy(P.kern[b]);
        }
        P = StPool();
        (void)hipSetDevice(cur);
    }
}

static int pool_get(StPool** out) {
    int dev = 0;
    int rc = report_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= 64) return report(-4, "safetensors: device index %d out of range", dev);
    StPool& P = g_st_pool[dev];
    for (int b = 0; b < 2; b++) {
        if (!P.pinned[b] && hipHostMalloc((void**)&P.pinned[b], kStChunk, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            P.pinned[b] = nullptr;
            return report(-3, "safetensors: pinned staging allocation failed");
        }
        if (!P.draw[b] && hipMalloc((void**)&P.draw[b], kStChunk) != hipSuccess) {
            (void)hipGetLastError();
            P.draw[b] = nullptr;
            return report(-3, "safetensors: device staging allocation failed");
        }
        if (!P.h2d[b] && (rc = report_hip(hipEventCreateWithFlags(&P.h2d[b], hipEventDisableTiming), "event")))
            return rc;
        if (!P.kern[b] && (rc = report_hip(hipEventCreateWithFlags(&P.kern[b], hipEventDisableTiming), "event")))
            return rc;
    }
    *out = &P;
    return 0;
}

// memcpy out of the mapping with a few threads (page-cache reads fault in
// parallel).
static void par_copy(uint8_t* dst, const uint8_t* src, size_t n) {
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned T = (n >= (8u << 20)) ? std::min(8u, hw) : 1u;
    if (T <= 1) {
        memcpy(dst, src, n);
        return;
    }
    const size_t slice = ((n + T - 1) / T + 4095) & ~(size_t)4095;
    std::vector<std::thread> th;
    for (unsigned i = 1; i < T; i++) {
        const size_t o = slice * i;
        if (o >= n) break;
        th.emplace_back([=] { memcpy(dst + o, src + o, std::min(slice, n - o)); });
    }
    memcpy(dst, src, std::min(slice, n));
    for (auto& x : th) x.join();
}

enum StSink { kSinkF32 = 0, kSinkQ8 = 1 };

// Stream n elements of `dtype` from host memory `src` into `out` (fp32 or
// Q8_0 blocks) on stream s.
static int st_stream(const uint8_t* src, long n, int dtype, StSink sink, void* out, hipStream_t s) {
    const int es = st_float_size(dtype);
    std::lock_guard<std::mutex> lock(g_st_mutex);
    StPool* P = nullptr;
    int rc = pool_get(&P);
    if (rc) return rc;
    const long chunk = (long)(kStChunk / (size_t)es) & ~31L;
    long c = 0;
    for (long e0 = 0; e0 < n; e0 += chunk, c++) {
        const int b = (int)(c & 1);
        const long ne = std::min(chunk, n - e0);
        const size_t nb = (size_t)ne * (size_t)es;
        if ((rc = report_hip(hipEventSynchronize(P->h2d[b]), "safetensors staging wait"))) return rc;
        par_copy(P->pinned[b], src + (size_t)e0 * es, nb);
        if (sink == kSinkF32 && dtype == ST_F32) {
            rc = report_hip(hipMemcpyAsync(static_cast<float*>(out) + e0, P->pinned[b], nb, hipMemcpyHostToDevice, s),
                            "safetensors upload");
            if (!rc) rc = report_hip(hipEventRecord(P->h2d[b], s), "event record");
            if (rc) return rc;
            continue;
        }
        rc = report_hip(hipStreamWaitEvent(s, P->kern[b], 0), "stream wait");
        if (!rc) rc = report_hip(hipMemcpyAsync(P->draw[b], P->pinned[b], nb, hipMemcpyHostToDevice, s),
                                 "safetensors upload");
        if (!rc) rc = report_hip(hipEventRecord(P->h2d[b], s), "event record");
        if (rc) return rc;
        if (sink == kSinkF32)
            rc = report_hip(st_convert_launch(dtype, P->draw[b], ne, static_cast<float*>(out) + e0, s),
                            "safetensors convert");
        else
            rc = report_hip(st_quantize_launch(dtype, P->draw[b], ne / kQ8Block,
                                               static_cast<uint8_t*>(out) + (size_t)(e0 / kQ8Block) * kQ8Bytes, s),
                            "safetensors quantize");
        if (!rc) rc = report_hip(hipEventRecord(P->kern[b], s), "event record");
        if (rc) return rc;
    }
    return 0;
}

static bool owns(const st_file* f, const st_tensor* t) {
    return f && t && t >= f->tensors && t < f->tensors + f->n_tensors;
}

}  // namespace rac

using namespace rac;

// ── the reader's API (bench/safetensors_reader.h:73-96) ────────────────────

RAC_EXPORT void st_close(st_file* f) {
    if (!f) return;
    if (f->mmap_base) munmap(f->mmap_base, f->mmap_len);
    if (f->fd >= 0) close(f->fd);
    free(f->header_copy);
    free(f->tensors);
    free(f);
    std::lock_guard<std::mutex> lock(g_st_mutex);
    if (g_st_open > 0 && --g_st_open == 0) pool_release_all();
}

RAC_EXPORT st_file* st_open(const char* path, char errout[256]) {
    st_file* f = static_cast<st_file*>(calloc(1, sizeof(st_file)));
    if (!f) {
        if (errout) snprintf(errout, 256, "out of memory");
        report(-3, "st_open: out of memory");
        return nullptr;
    }
    f->fd = -1;
    {
        std::lock_guard<std::mutex> lock(g_st_mutex);
        g_st_open++;
    }
    auto bail = [&]() -> st_file* {
        if (errout) snprintf(errout, 256, "%s", f->err);
        report(-1, "st_open: %s", f->err);
        st_close(f);
        return nullptr;
    };
    if (!path) {
        st_fail(f, "null path");
        return bail();
    }
    f->tensors = static_cast<st_tensor*>(calloc(ST_MAX_TENSORS, sizeof(st_tensor)));
    if (!f->tensors) {
        st_fail(f, "out of memory");
        return bail();
    }
    f->fd = open(path, O_RDONLY);
    if (f->fd < 0) {
        st_fail(f, "open(%s): %s", path, strerror(errno));
        return bail();
    }
    struct stat sb;
    if (fstat(f->fd, &sb) != 0) {
        st_fail(f, "fstat(%s): %s", path, strerror(errno));
        return bail();
    }
    f->mmap_len = (size_t)sb.st_size;
    if (f->mmap_len < 8) {
        st_fail(f, "file too small (%zu bytes)", f->mmap_len);
        return bail();
    }
    void* m = mmap(nullptr, f->mmap_len, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) {
        st_fail(f, "mmap: %s", strerror(errno));
        return bail();
    }
    f->mmap_base = m;
    uint64_t hl = 0;
    memcpy(&hl, m, 8);   // little-endian u64
    if (hl > f->mmap_len - 8) {
        st_fail(f, "header length %llu exceeds the file", (unsigned long long)hl);
        return bail();
    }
    f->data_offset = 8 + (size_t)hl;
    f->header_copy = static_cast<char*>(malloc((size_t)hl + 1));
    if (!f->header_copy) {
        st_fail(f, "out of memory");
        return bail();
    }
    memcpy(f->header_copy, static_cast<const char*>(m) + 8, (size_t)hl);
    f->header_copy[hl] = '\0';
    if (parse_header(f, f->header_copy, (size_t)hl, f->mmap_len - f->data_offset)) return bail();
    return f;
}

RAC_EXPORT const st_tensor* st_find(const st_file* f, const char* name) {
    if (!f || !name) return nullptr;
    for (int i = 0; i < f->n_tensors; i++)
        if (!strcmp(f->tensors[i].name, name)) return &f->tensors[i];
    return nullptr;
}

RAC_EXPORT const void* st_data(const st_file* f, const st_tensor* t) {
    if (!f || !t) return nullptr;
    return static_cast<const char*>(f->mmap_base) + f->data_offset + t->offset;
}

RAC_EXPORT size_t st_numel(const st_tensor* t) {
    if (!t) return 0;
    size_t n = 1;
    for (int i = 0; i < t->ndim; i++) n *= (size_t)t->shape[i];
    return n;
}

RAC_EXPORT const char* st_dtype_name(st_dtype d) {
    switch (d) {
    case ST_F32: return "F32";
    case ST_F16: return "F16";
    case ST_BF16: return "BF16";
    case ST_F64: return "F64";
    case ST_I8: return "I8";
    case ST_U8: return "U8";
    case ST_I16: return "I16";
    case ST_I32: return "I32";
    case ST_I64: return "I64";
    case ST_BOOL: return "BOOL";
    default: return "UNKNOWN";
    }
}

RAC_EXPORT void st_dump(const st_file* f) {
    if (!f) {
        printf("(null st_file)\n");
        return;
    }
    printf("%d tensors, data segment at byte %zu\n", f->n_tensors, f->data_offset);
    for (int i = 0; i < f->n_tensors; i++) {
        const st_tensor* t = &f->tensors[i];
        printf("  %4d  %-48s %-7s [", i, t->name, st_dtype_name(t->dtype));
        for (int d = 0; d < t->ndim; d++) printf(d ? ", %lld" : "%lld", (long long)t->shape[d]);
        printf("]  %zu bytes at +%zu\n", t->nbytes, t->offset);
    }
    fflush(stdout);
}

// ── device forms ─────────────────────────────────────────────────────────

RAC_EXPORT int rac_st_convert_dev(int dtype, const void* src, long n, float* out, void* stream) {
    if (!src || !out) return report(-1, "rac_st_convert_dev: null buffer");
    if (n < 0) return report(-2, "rac_st_convert_dev: negative count");
    if (!st_float_size(dtype))
        return report(RAC_ST_ERR_DTYPE, "rac_st_convert_dev: dtype %s is not a float type",
                      st_dtype_name((st_dtype)dtype));
    return report_hip(st_convert_launch(dtype, src, n, out, (hipStream_t)stream), "rac_st_convert_dev launch");
}

RAC_EXPORT int rac_st_quantize_dev(int dtype, const void* src, long n_blocks, void* out_blocks, void* stream) {
    if (!src || !out_blocks) return report(-1, "rac_st_quantize_dev: null buffer");
    if (n_blocks < 0 || n_blocks > 2147483647L * 256L)
        return report(-2, "rac_st_quantize_dev: bad block count %ld", n_blocks);
    if (!st_float_size(dtype))
        return report(RAC_ST_ERR_DTYPE, "rac_st_quantize_dev: dtype %s is not a float type",
                      st_dtype_name((st_dtype)dtype));
    return report_hip(st_quantize_launch(dtype, src, n_blocks, static_cast<uint8_t*>(out_blocks), (hipStream_t)stream),
                      "rac_st_quantize_dev launch");
}

RAC_EXPORT int rac_st_to_f32_dev(const st_file* f, const st_tensor* t, float* out, void* stream) {
    if (!f || !t || !out) return report(-1, "rac_st_to_f32_dev: null argument");
    if (!owns(f, t)) return report(-1, "rac_st_to_f32_dev: tensor does not belong to this file");
    if (!st_float_size(t->dtype))
        return report(RAC_ST_ERR_DTYPE, "rac_st_to_f32_dev: '%s' is %s, not a float type", t->name,
                      st_dtype_name(t->dtype));
    const long n = (long)st_numel(t);
    if (n == 0) return 0;
    return st_stream(static_cast<const uint8_t*>(st_data(f, t)), n, t->dtype, kSinkF32, out, (hipStream_t)stream);
}

RAC_EXPORT int rac_st_to_q8_0_dev(const st_file* f, const st_tensor* t, void* out_blocks, void* stream) {
    if (!f || !t || !out_blocks) return report(-1, "rac_st_to_q8_0_dev: null argument");
    if (!owns(f, t)) return report(-1, "rac_st_to_q8_0_dev: tensor does not belong to this file");
    if (!st_float_size(t->dtype))
        return report(RAC_ST_ERR_DTYPE, "rac_st_to_q8_0_dev: '%s' is %s, not a float type", t->name,
                      st_dtype_name(t->dtype));
    if (t->ndim < 1 || t->shape[t->ndim - 1] % kQ8Block != 0)
        return report(-2, "rac_st_to_q8_0_dev: '%s' needs a last dimension that is a multiple of 32", t->name);
    const long n = (long)st_numel(t);
    if (n == 0) return 0;
    return st_stream(static_cast<const uint8_t*>(st_data(f, t)), n, t->dtype, kSinkQ8, out_blocks,
                     (hipStream_t)stream);
}

// safetensors_reader.h:87 — synchronous; `out` host or device memory.
RAC_EXPORT int st_to_f32(const st_file* f, const st_tensor* t, float* out) {
    if (!f || !t || !out) {
        report(-1, "st_to_f32: null argument");
        return -1;
    }
    if (!st_float_size(t->dtype)) {
        report(RAC_ST_ERR_DTYPE, "st_to_f32: '%s' is %s, not a float type", t->name, st_dtype_name(t->dtype));
        return -1;
    }
    const size_t n = st_numel(t);
    if (n == 0) return 0;
    hipStream_t s = (hipStream_t)rac_get_stream();
    float* dst = out;
    const bool host = !is_device_ptr(out);
    if (host && hipMalloc((void**)&dst, n * sizeof(float)) != hipSuccess) {
        (void)hipGetLastError();
        report(-3, "st_to_f32: device staging allocation failed");
        return -1;
    }
    int rc = rac_st_to_f32_dev(f, t, dst, s);
    if (!rc && host)
        rc = report_hip(hipMemcpyAsync(out, dst, n * sizeof(float), hipMemcpyDeviceToHost, s), "st_to_f32 copy out");
    const int rc2 = report_hip(hipStreamSynchronize(s), "st_to_f32 synchronize");
    if (host) (void)hipFree(dst);
    return (rc || rc2) ? -1 : 0;
}
