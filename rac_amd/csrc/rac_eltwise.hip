// rac_eltwise.hip — streaming kernels for gfx950: RoPE table build and
// application (circular CORDIC / Givens rotation), hyperbolic-CORDIC
// activations (exp, SiLU, sigmoid, tanh), GELU, ReLU, and batch rsqrt /
// sin-cos used by the scalar C entry points.
//
// RoPE apply (rac_cpu.c:600-635) is pure HBM streaming: each (b, h, t) row of
// head_dim floats is rotated pairwise by the table row t.  A workgroup owns a
// fixed block of positions t and a slice of kRopeRslice (b, h) rows, so its
// cos/sin values are loaded once into registers and reused; each lane moves
// 16 bytes per row with one non-temporal load and store (1 read + 1 write per
// element, the HBM minimum), and consecutive lanes touch consecutive
// addresses.
#include <hip/hip_runtime.h>
#include "rac_act.hpp"

namespace rac {

// ── elementwise ──────────────────────────────────────────────────────────

// One pass, no grid-stride loop: workgroup b (64 lanes) owns float4 groups
// 256 b .. 256 b + 255, lane l the groups 256 b + l + 64 f, f = 0..3 (each
// coalesced), so sixteen CORDIC chains interleave per lane; groups past the
// end compute on zeros and are not stored.  The grid covers the array once
// and the hardware dispatcher starts a new workgroup as soon as one
// retires, which keeps loads in flight better than resident workgroups
// walking the array (measured on SiLU 16384 x 11008: 216 / 254 / 311 us at
// n = 8 / 16 / 24 against 258-274 / 277-298 / 331-365 us for a grid-stride
// loop over a capped grid, and slower still for a grid of resident
// workgroups, with or without prefetching each next trip into LDS).  With
// the loads at raised priority (below), 4 float4 per lane on 64-lane
// workgroups measured 0.6-1% faster than 2 on 128 (n = 16: 247.7 vs 249.1
// and 252.6 vs 255.2 us on two boxes; 1 float4 per lane 3-4% slower).
constexpr int kEltThreads = 64;
constexpr int kEltF4 = 4;                            // float4 groups per lane
constexpr int kEltGroups = kEltF4 * kEltThreads;     // float4 groups per workgroup

template <int OP, int NITER>
__global__ __launch_bounds__(kEltThreads) void eltwise_vec_kernel(
    const float4* __restrict__ x, float4* __restrict__ y, long n4, int iters, float khinv)
{
    // A new workgroup's address arithmetic and loads issue at raised wave
    // priority, ahead of the CORDIC chains of older waves on the SIMD, so
    // its HBM requests leave early and the chains hide their latency
    // (SiLU 16384 x 11008, n = 16: 260.2 -> 256.6 us median, same bits).
    __builtin_amdgcn_s_setprio(3);
    const long i0 = (long)blockIdx.x * kEltGroups + threadIdx.x;
    float4 r[kEltF4];
#pragma unroll
    for (int f = 0; f < kEltF4; f++) {
        const long i = i0 + (long)f * kEltThreads;
        r[f] = (i < n4) ? ld4_stream(&x[i]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    __builtin_amdgcn_s_setprio(0);
    float v[4 * kEltF4];
#pragma unroll
    for (int f = 0; f < kEltF4; f++) {
        v[4 * f] = r[f].x; v[4 * f + 1] = r[f].y; v[4 * f + 2] = r[f].z; v[4 * f + 3] = r[f].w;
    }
    elt_vec<OP, NITER, 4 * kEltF4>(v, iters, khinv);
#pragma unroll
    for (int f = 0; f < kEltF4; f++) {
        const long i = i0 + (long)f * kEltThreads;
        if (i < n4) st4_stream(&y[i], make_float4(v[4 * f], v[4 * f + 1], v[4 * f + 2], v[4 * f + 3]));
    }
}

template <int OP, int NITER>
__global__ __launch_bounds__(256) void eltwise_scalar_kernel(
    const float* __restrict__ x, float* __restrict__ y, long n, int iters, float khinv)
{
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        y[i] = elt<OP, NITER>(x[i], iters, khinv);
}

static unsigned stream_grid(long items) {
    // enough waves to cover HBM latency on 256 CUs; grid-stride beyond that
    long blocks = (items + 255) / 256;
    const long cap = 256L * 64;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    return (unsigned)blocks;
}

__global__ __launch_bounds__(256) void act_grad_kernel(const float* __restrict__ g,
                                                       const float* __restrict__ pre,
                                                       float* __restrict__ d, long n, int act,
                                                       int iters, float khinv) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        d[i] = act_grad(g[i], pre[i], act, iters, khinv);
}

hipError_t act_grad_launch(const float* g, const float* pre, float* d, long count, int act, int iters,
                           hipStream_t s) {
    iters = clamp_iters(iters);
    hipLaunchKernelGGL(act_grad_kernel, dim3(stream_grid(count)), dim3(256), 0, s, g, pre, d, count, act,
                       iters, host_consts().exp_khinv[iters]);
    return hipGetLastError();
}

template <int OP, int NITER>
static hipError_t elt_launch2(const float* x, float* y, long count, int iters, float khinv,
                              hipStream_t s) {
    const bool vec_ok = (count % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0) &&
                        ((reinterpret_cast<uintptr_t>(y) & 15) == 0);
    if (vec_ok) {
        // at most 2^24 workgroups (2^31 work-items) per launch
        constexpr long kChunk = (1L << 24) * kEltGroups;
        const long n4 = count / 4;
        for (long off = 0; off < n4; off += kChunk) {
            const long len = n4 - off < kChunk ? n4 - off : kChunk;
            hipLaunchKernelGGL((eltwise_vec_kernel<OP, NITER>), dim3((unsigned)((len + kEltGroups - 1) / kEltGroups)),
                               dim3(kEltThreads), 0, s, reinterpret_cast<const float4*>(x) + off,
                               reinterpret_cast<float4*>(y) + off, len, iters, khinv);
        }
    } else {
        hipLaunchKernelGGL((eltwise_scalar_kernel<OP, NITER>), dim3(stream_grid(count)), dim3(256),
                           0, s, x, y, count, iters, khinv);
    }
    return hipGetLastError();
}

template <int OP>
static hipError_t elt_launch_iters(const float* x, float* y, long count, int iters, hipStream_t s) {
    iters = clamp_iters(iters);
    const float khinv = host_consts().exp_khinv[iters];
    switch (iters) {
        case 8: return elt_launch2<OP, 8>(x, y, count, iters, khinv, s);
        case 16: return elt_launch2<OP, 16>(x, y, count, iters, khinv, s);
        case 24: return elt_launch2<OP, 24>(x, y, count, iters, khinv, s);
        default: return elt_launch2<OP, 0>(x, y, count, iters, khinv, s);
    }
}

hipError_t eltwise_launch(int op, const float* x, float* y, long count, int iters, hipStream_t s) {
    switch (op) {
        case kEltExp: return elt_launch_iters<kEltExp>(x, y, count, iters, s);
        case kEltSilu: return elt_launch_iters<kEltSilu>(x, y, count, iters, s);
        case kEltSigmoid: return elt_launch_iters<kEltSigmoid>(x, y, count, iters, s);
        case kEltTanh: return elt_launch_iters<kEltTanh>(x, y, count, iters, s);
        case kEltGelu: return elt_launch2<kEltGelu, 0>(x, y, count, 0, 0.0f, s);
        case kEltRelu: return elt_launch2<kEltRelu, 0>(x, y, count, 0, 0.0f, s);
        default: return hipErrorInvalidValue;
    }
}

// ── rsqrt / sincos batches (scalar C entry points run through these) ─────

__global__ void rsqrt_kernel(const float* __restrict__ x, float* __restrict__ y, long n, float k) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = rsqrt_cordic(x[i], k);
}

hipError_t rsqrt_launch(const float* x, float* y, long count, hipStream_t s) {
    hipLaunchKernelGGL(rsqrt_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, x, y,
                       count, host_consts().rsqrt_khinv);
    return hipGetLastError();
}

__global__ void sincos_kernel(const float* __restrict__ th, float* __restrict__ so,
                              float* __restrict__ co, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float s, c;
        sincos_cordic(th[i], s, c);
        so[i] = s;
        co[i] = c;
    }
}

hipError_t sincos_launch(const float* theta, float* s_out, float* c_out, long count, hipStream_t s) {
    hipLaunchKernelGGL(sincos_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, theta,
                       s_out, c_out, count);
    return hipGetLastError();
}

// ── RoPE table (rac_cpu.c:576-598) ───────────────────────────────────────

__global__ void rope_cache_kernel(float* __restrict__ cos_out, float* __restrict__ sin_out,
                                  const float* __restrict__ inv_freq, int max_seq, int half) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)max_seq * half) return;
    const int p = (int)(idx / half), i = (int)(idx % half);
    float s, c;
    sincos_cordic((float)p * inv_freq[i], s, c);
    cos_out[idx] = c;
    sin_out[idx] = s;
}

hipError_t rope_cache_launch(float* cos_out, float* sin_out, const float* inv_freq, int max_seq,
                             int half, hipStream_t s) {
    const long n = (long)max_seq * half;
    hipLaunchKernelGGL(rope_cache_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       cos_out, sin_out, inv_freq, max_seq, half);
    return hipGetLastError();
}

// ── RoPE apply (rac_cpu.c:600-635) ───────────────────────────────────────
//
// Row (b, h, t) starts at x + b*sb + h*sh + t*st (element strides; the
// contiguous [B,H,T,D] layout is sb = H*T*D, sh = T*D, st = D).
// Vector path: head_dim % 4 == 0 and every row 16-byte aligned; each lane
// owns one float4 (two pairs) of a row.  A block covers RPB positions and
// RSLICE consecutive (b, h) rows.

// (b, h) rows per lane: 2 measured best on MI355X (335 us for Q+K
// [8,32,4096,128], ~the 1:1 streaming-copy rate); more rows per lane cut
// the number of workgroups in flight and lost bandwidth (16 rows: 394 us).
constexpr int kRopeRslice = 2;

// Row (b, h, t) is read at x + b*sb + h*sh + t*st and written at
// y + b*ob + h*oh + t*ot: in place when y == x with the same strides,
// out of place otherwise (the two must then not overlap).
struct RopeOut {
    float* y;
    long ob, oh, ot;
};

template <int LPR>   // lanes per row = head_dim / 4, a power of two <= 256
__global__ __launch_bounds__(256) void rope_apply_vec_kernel(
    const float* x, const float* __restrict__ cos_tab, const float* __restrict__ sin_tab,
    int heads, int seq, int head_dim, long sb, long sh, long st, long bh_total, RopeOut out)
{
    constexpr int RPB = 256 / LPR;
    const int lane_in_row = threadIdx.x % LPR;
    const int t = blockIdx.x * RPB + threadIdx.x / LPR;
    if (t >= seq) return;
    const int half = head_dim / 2;
    // pairs 2*lane_in_row and 2*lane_in_row+1 of position t
    const float2 c = *reinterpret_cast<const float2*>(cos_tab + (long)t * half + 2 * lane_in_row);
    const float2 sn = *reinterpret_cast<const float2*>(sin_tab + (long)t * half + 2 * lane_in_row);
    const long bh0 = (long)blockIdx.y * kRopeRslice;
    long bh_end = bh0 + kRopeRslice;
    if (bh_end > bh_total) bh_end = bh_total;
    float4 v[kRopeRslice];
    float4* p[kRopeRslice];
#pragma unroll
    for (int r = 0; r < kRopeRslice; r++) {
        const long bh = bh0 + r;
        if (bh < bh_end) {
            const long b = bh / heads, h = bh % heads;
            v[r] = ld4_stream(reinterpret_cast<const float4*>(x + b * sb + h * sh + (long)t * st) + lane_in_row);
            p[r] = reinterpret_cast<float4*>(out.y + b * out.ob + h * out.oh + (long)t * out.ot) + lane_in_row;
        }
    }
#pragma unroll
    for (int r = 0; r < kRopeRslice; r++) {
        if (bh0 + r < bh_end) {
            float4 o;
            o.x = __builtin_fmaf(v[r].x, c.x, -(v[r].y * sn.x));
            o.y = __builtin_fmaf(v[r].x, sn.x, v[r].y * c.x);
            o.z = __builtin_fmaf(v[r].z, c.y, -(v[r].w * sn.y));
            o.w = __builtin_fmaf(v[r].z, sn.y, v[r].w * c.y);
            st4_stream(p[r], o);
        }
    }
}

__global__ __launch_bounds__(256) void rope_apply_scalar_kernel(
    const float* x, const float* __restrict__ cos_tab, const float* __restrict__ sin_tab,
    int heads, int seq, int head_dim, long sb, long sh, long st, long total_pairs, RopeOut out)
{
    const int half = head_dim / 2;
    const long stride = (long)gridDim.x * blockDim.x;
    for (long q = (long)blockIdx.x * blockDim.x + threadIdx.x; q < total_pairs; q += stride) {
        const long i = q % half;
        long r = q / half;
        const long t = r % seq;
        r /= seq;
        const long h = r % heads, b = r / heads;
        const float* row = x + b * sb + h * sh + t * st;
        float* orow = out.y + b * out.ob + h * out.oh + t * out.ot;
        const float a = row[2 * i], b2 = row[2 * i + 1];
        const float c = cos_tab[t * half + i], s = sin_tab[t * half + i];
        orow[2 * i] = __builtin_fmaf(a, c, -(b2 * s));
        orow[2 * i + 1] = __builtin_fmaf(a, s, b2 * c);
    }
}

hipError_t rope_apply_launch(float* x, const float* cos_tab, const float* sin_tab, int batch,
                             int heads, int seq, int head_dim, long sb, long sh, long st,
                             hipStream_t s) {
    return rope_apply_out_launch(x, x, cos_tab, sin_tab, batch, heads, seq, head_dim, sb, sh, st, sb, sh, st, s);
}

hipError_t rope_apply_out_launch(const float* x, float* y, const float* cos_tab, const float* sin_tab, int batch,
                                 int heads, int seq, int head_dim, long sb, long sh, long st, long ob, long oh,
                                 long ot, hipStream_t s) {
    const long bh_total = (long)batch * heads;
    const int lpr = head_dim / 4;
    const RopeOut out{y, ob, oh, ot};
    const bool pow2_lpr = (head_dim % 4 == 0) && lpr >= 1 && lpr <= 256 && (lpr & (lpr - 1)) == 0;
    const bool aligned = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (sb % 4 == 0) &&
                         (sh % 4 == 0) && (st % 4 == 0) &&
                         ((reinterpret_cast<uintptr_t>(y) & 15) == 0) && (ob % 4 == 0) &&
                         (oh % 4 == 0) && (ot % 4 == 0) &&
                         ((reinterpret_cast<uintptr_t>(cos_tab) & 7) == 0) &&
                         ((reinterpret_cast<uintptr_t>(sin_tab) & 7) == 0);
    const long grid_y = (bh_total + kRopeRslice - 1) / kRopeRslice;
    if (pow2_lpr && aligned && grid_y <= 65535) {
        const int rpb = 256 / lpr;
        dim3 grid((unsigned)((seq + rpb - 1) / rpb), (unsigned)grid_y);
#define RAC_ROPE_CASE(L)                                                                          \
    case L:                                                                                       \
        hipLaunchKernelGGL((rope_apply_vec_kernel<L>), grid, dim3(256), 0, s, x, cos_tab, sin_tab, \
                           heads, seq, head_dim, sb, sh, st, bh_total, out);                     \
        break;
        switch (lpr) {
            RAC_ROPE_CASE(1) RAC_ROPE_CASE(2) RAC_ROPE_CASE(4) RAC_ROPE_CASE(8)
            RAC_ROPE_CASE(16) RAC_ROPE_CASE(32) RAC_ROPE_CASE(64) RAC_ROPE_CASE(128)
            RAC_ROPE_CASE(256)
            default: return hipErrorInvalidValue;
        }
#undef RAC_ROPE_CASE
    } else {
        const long pairs = bh_total * seq * (head_dim / 2);
        hipLaunchKernelGGL(rope_apply_scalar_kernel, dim3(stream_grid(pairs)), dim3(256), 0, s, x,
                           cos_tab, sin_tab, heads, seq, head_dim, sb, sh, st, pairs, out);
    }
    return hipGetLastError();
}

}  // namespace rac
