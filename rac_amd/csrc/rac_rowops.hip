// rac_rowops.hip — row-wise softmax (hyperbolic-CORDIC exp), RMSNorm and
// LayerNorm (CORDIC-vectoring rsqrt) for gfx950.
//
// One 256-lane workgroup (4 wave64) per row.  When the row length is a
// multiple of 4 and the row fits in registers (<= 16 float4 per lane), the
// row is read from HBM exactly once into registers with 16-byte loads, the
// reductions run as wave64 butterflies (ds_swizzle/DPP via __shfl_xor) plus a
// 4-entry LDS exchange, and the result is written once: 1 read + 1 write per
// element, the HBM minimum.  Other shapes take a strided loop that re-reads
// the row (from L2 for rows up to a few MB).
//
// Arithmetic follows rac_cpu.c:258-271 (softmax), :548-574 (RMSNorm) and
// :507-546 (LayerNorm) rounding for rounding, except the order of the row
// sums: each lane adds its own values in order (the register path's lane l
// holds the float4 groups l, l + 256, ...; the strided loop's, the elements
// l, l + 256, ...), lanes combine by a wave64 XOR butterfly (offsets 32 ..
// 1) and the four wave partials in order, instead of one left-to-right sum
// (differences O(1e-7) relative).  That order is fixed, so results do not
// depend on scheduling and a CPU model of it matches bit for bit.
#include <hip/hip_runtime.h>
#include <atomic>
#include <type_traits>
#include "rac_math.hpp"
#include "rac_internal.hpp"
#include "rac_rowred.hpp"

namespace rac {

template <int NITER>
__device__ __forceinline__ float exp_n(float x, int iters, float khinv) {
    if constexpr (NITER > 0) return exp_cordic<NITER>(x, khinv);
    else return exp_cordic_rt(x, iters, khinv);
}

// ── softmax ──────────────────────────────────────────────────────────────

// Attention masking of score x at (query position t, key column j), in the
// order of rac_cpu.c:668-670: causal sets -inf above the diagonal, then the
// additive mask is added (mask_ld set by the dispatcher).
__device__ __forceinline__ float mask_score(float x, long t, long j, const SoftmaxMask& mk) {
    if (mk.causal && j > t) x = -__builtin_inff();
    if (mk.mask) x += mk.mask[t * mk.mask_ld + j];
    return x;
}

// 1/sum, or 0 for a non-positive sum when the guard of rac_cpu.c:687 is on.
__device__ __forceinline__ float inv_sum(float s, int zero_guard) {
    return (zero_guard && !(s > 0.0f)) ? 0.0f : 1.0f / s;
}

// Exps of the E = 4*VPT row elements a lane holds.  Compile-time step
// counts use the step-major form (all elements advance one step at a time:
// independent chains interleave and constants are shared); bit-identical
// to one exp_cordic call per element.
template <int NITER, int E, int OPT = kExpFull>
__device__ __forceinline__ void exp_lane(float* v, int iters, float khinv) {
    if constexpr (NITER > 0) {
        constexpr int G = E < 16 ? E : 16;
#pragma unroll
        for (int b = 0; b < E; b += G) exp_cordic_vec<NITER, G, OPT>(v + b, khinv);
    } else {
#pragma unroll
        for (int e = 0; e < E; e++) v[e] = exp_cordic_rt(v[e], iters, khinv);
    }
}

// Softmax of the row a workgroup holds in registers: lane l holds the float4
// groups l, l + 256, ... of the row (E = 4 VPT values, -inf past the row
// end, whose exp is +0, so the max, the lane sums (s + 0 == s) and the
// outputs are those of the elements that exist).  On return v holds the
// outputs.  t is the row's query position (masked rows only).
// First stage: masking (masked rows) and the lane's maximum.
template <int VPT, bool MASKED, bool FULL>
__device__ __forceinline__ float softmax_lane_max(float* v, long n4, long t, const SoftmaxMask& mk) {
    if constexpr (MASKED) {
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const long idx = threadIdx.x + (long)i * kRowThreads;
            if (FULL || idx < n4) {
#pragma unroll
                for (int c = 0; c < 4; c++) v[4 * i + c] = mask_score(v[4 * i + c], t, 4 * idx + c, mk);
            }
        }
    }
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < VPT; i++)
        m = fmaxf(fmaxf(fmaxf(m, v[4 * i]), fmaxf(v[4 * i + 1], v[4 * i + 2])), v[4 * i + 3]);
    return m;
}

// The lane's first zero (zero_key) in the register layout: group i of lane l
// is the row's float4 group l + 256 i, so the lane's values run in index
// order.
template <int VPT>
__device__ __forceinline__ uint32_t lane_first_zero(const float* v) {
    uint32_t key = ~0u;
#pragma unroll
    for (int e = 4 * VPT - 1; e >= 0; e--)
        if (v[e] == 0.0f) key = zero_key<uint32_t>(4 * (threadIdx.x + kRowThreads * (e / 4)) + e % 4, v[e]);
    return key;
}

// Exps of the lane's values against the row maximum m, and the lane's sum
// of them (masked rows, and rows whose step count is known only at run time).
template <int VPT, int NITER, bool MASKED>
__device__ __forceinline__ float softmax_lane_exps(float* v, float m, int iters, float khinv) {
    constexpr int E = 4 * VPT;
#pragma unroll
    for (int e = 0; e < E; e++) v[e] = v[e] - m;
    exp_lane<NITER, E>(v, iters, khinv);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < E; e++) s += v[e];
    return s;
}

// Unmasked rows with a compile-time step count.  Every x - max is <= 0 or
// NaN, and a NaN anywhere, or a maximum of +-inf, makes the reference's row
// sum NaN and with it every output (rac_cpu.c:258-271).  So:
//  - the row maximum is the NaN-propagating IEEE maximum (v_maximum3, no
//    canonicalisation of the loaded values; -0 < +0 as for v_max_f32, so
//    the maximum and every x - max equal the general path's), and a
//    non-finite maximum forces the row sum to NaN instead of a per-element
//    NaN test;
//  - the exps skip the sign-dependent rounding bias (kExpNonPos);
//  - when every x - max of the wave is >= -86 (then k >= -124), the exp's
//    (p / K_h) 2^k is p * (1/K_h 2^k) with the scale built in the exponent
//    field: one rounding of the same exact product, every intermediate
//    normal, so the bits of ldexp(p / K_h, k); otherwise ldexp and the
//    k <= -127 flush.
// Bit-identical to softmax_lane_exps<VPT, NITER, false> with kExpFlush |
// kExpNonPos exps and a NaN pass; ~5% fewer VALU instructions per element.
struct RowExtent {
    float max;   // row maximum (every lane)
    float min;   // the lane's minimum
};

// row_lds: the row in LDS in the same layout (the prefetching kernel), read
// instead of v for the rare zero-maximum scan, so that scan holds no
// registers of its own; null: scan v.
template <int VPT, bool LDS_ONLY>
__device__ __forceinline__ RowExtent unmasked_row_extent(const float* v, float* red, uint32_t* zred,
                                                         const float* row_lds = nullptr) {
    constexpr int E = 4 * VPT;
    float mx = v[0], mn = v[0];
#pragma unroll
    for (int e = 1; e < E; e++) {
        mx = maximum(mx, v[e]);
        mn = fminf(mn, v[e]);
    }
    mx = block_maximum<false, LDS_ONLY>(mx, red);
    if (mx == 0.0f) {
        uint32_t key = ~0u;
        if (row_lds) {
            for (int e = 0; e < E && key == ~0u; e++) {
                const int idx = 4 * (threadIdx.x + kRowThreads * (e / 4)) + e % 4;
                if (row_lds[idx] == 0.0f) key = zero_key<uint32_t>(idx, row_lds[idx]);
            }
        } else {
            key = lane_first_zero<VPT>(v);
        }
        mx = first_zero_max<LDS_ONLY>(key, zred);
    }
    return {mx, mn};
}

template <int N, int G>
__device__ __forceinline__ void unmasked_exp_group(float* v, float khinv, bool fused) {
    int k[G];
    float p[G], z[G];
#pragma unroll
    for (int e = 0; e < G; e++) {
        k[e] = cvt_i32_sat(__builtin_fmaf(v[e], kInvLn2, -0.5f));
        z[e] = __builtin_fmaf(-(float)k[e], kLn2, v[e]);
        p[e] = 1.0f;
    }
    HypStepV<N, 0, G>::run(p, z);
    if (fused) {
#pragma unroll
        for (int e = 0; e < G; e++) v[e] = p[e] * as_f(as_u(khinv) + ((uint32_t)k[e] << 23));
    } else {
#pragma unroll
        for (int e = 0; e < G; e++) {
            const float res = __builtin_ldexpf(p[e] * khinv, k[e]);
            v[e] = (k[e] <= -127) ? 0.0f : res;
        }
    }
}

template <int NITER, int E>
__device__ __forceinline__ float unmasked_lane_exps(float* v, RowExtent r, float khinv) {
    const bool fused = __all((r.min - r.max) >= -86.0f);
#pragma unroll
    for (int e = 0; e < E; e++) v[e] = v[e] - r.max;
    constexpr int G = E < 16 ? E : 16;
#pragma unroll
    for (int b = 0; b < E; b += G) unmasked_exp_group<NITER, G>(v + b, khinv, fused);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < E; e++) s += v[e];
    if (!(__builtin_fabsf(r.max) < __builtin_inff())) s = __builtin_nanf("");
    return s;
}

// Second stage: row max, exps, row sum, scaling (m: the lane's maximum).
// red: 2 kRowWaves floats (max and sum partials apart, so neither reduction
// needs a trailing barrier; a kernel handles one row per workgroup).
template <int VPT, int NITER, bool MASKED>
__device__ __forceinline__ void softmax_row_finish(float* v, float m, int iters, float khinv,
                                                   const SoftmaxMask& mk, float* red, uint32_t* zred) {
    constexpr int E = 4 * VPT;
    m = block_max<false>(m, red);
    if (m == 0.0f) m = first_zero_max<false>(lane_first_zero<VPT>(v), zred);
    float s = softmax_lane_exps<VPT, NITER, MASKED>(v, m, iters, khinv);
    s = block_sum<false>(s, red + kRowWaves);
    const float inv = inv_sum(s, MASKED ? mk.zero_guard : 0);
#pragma unroll
    for (int e = 0; e < E; e++) v[e] = v[e] * inv;
}

template <int VPT, int NITER, bool MASKED, bool FULL>
__device__ __forceinline__ void softmax_row_regs(float* v, long n4, long t, int iters, float khinv,
                                                 const SoftmaxMask& mk, float* red, uint32_t* zred) {
    if constexpr (!MASKED && NITER > 0) {
        const RowExtent r = unmasked_row_extent<VPT, false>(v, red, zred);
        float s = unmasked_lane_exps<NITER, 4 * VPT>(v, r, khinv);
        s = block_sum<false>(s, red + kRowWaves);
        const float inv = inv_sum(s, 0);
#pragma unroll
        for (int e = 0; e < 4 * VPT; e++) v[e] = v[e] * inv;
        return;
    }
    const float m = softmax_lane_max<VPT, MASKED, FULL>(v, n4, t, mk);
    softmax_row_finish<VPT, NITER, MASKED>(v, m, iters, khinv, mk, red, zred);
}

template <int VPT, bool FULL>
__device__ __forceinline__ void load_row_regs(const float* xrow, long n4, float* v) {
    const float4* xr = reinterpret_cast<const float4*>(xrow);
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const long idx = threadIdx.x + (long)i * kRowThreads;
        float4 t = make_float4(-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff());
        if (FULL || idx < n4) t = ld4_stream(&xr[idx]);
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

template <int VPT, bool FULL>
__device__ __forceinline__ void store_row_regs(float* yrow, long n4, const float* v) {
    float4* yr = reinterpret_cast<float4*>(yrow);
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const long idx = threadIdx.x + (long)i * kRowThreads;
        if (FULL || idx < n4) st4_stream(&yr[idx], make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]));
    }
}

// One workgroup per row: the row is read once into registers (16-byte
// loads), reduced, exponentiated and written once.
// FULL: n == 1024 * VPT exactly, so no lane needs a bounds check.
template <int VPT, int NITER, bool MASKED, bool FULL>
__global__ __launch_bounds__(kRowThreads) void softmax_reg_kernel(
    const float* x, float* y, long n, int iters, float khinv,
    SoftmaxMask mk)
{
    __shared__ float red[2 * kRowWaves];
    __shared__ uint32_t zred[kRowWaves];
    const long row = blockIdx.x;
    const long n4 = n / 4;
    float v[4 * VPT];
    load_row_regs<VPT, FULL>(x + row * n, n4, v);
    softmax_row_regs<VPT, NITER, MASKED, FULL>(v, n4, MASKED ? mk.row0 + row % mk.seq : 0, iters, khinv, mk,
                                               red, zred);
    store_row_regs<VPT, FULL>(y + row * n, n4, v);
}

// Unmasked rows of exactly 1024 VPT floats, persistent: workgroup g takes
// rows g, g + G, g + 2G, ... (G = gridDim.x).  While a row's exps run, the
// next row is already on its way from HBM into LDS (global_load_lds, which
// holds no VGPRs), so each workgroup keeps one row of loads in flight
// through its whole lifetime instead of waiting for its row at start-up.
// The row reductions use LDS-only barriers (lds_barrier): the previous
// row's stores stay in flight across them; the barrier of the row sum
// waits for the prefetch (an LDS write), which has had the exps to land.
// Same arithmetic as softmax_reg_kernel<VPT, NITER, false, true>, so the
// same bits.  Used where the exps are short (n = 8): at 16 and 24 steps the
// one-row-per-workgroup kernel is faster (measured on 4096 x 4096: n = 8
// 23.6 -> 22.2 us; n = 16 25.0 against 26.3, n = 24 31.1 against 32.2).
template <int VPT, int NITER>
__global__ __launch_bounds__(kRowThreads, 6) void softmax_prefetch_kernel(
    const float* x, float* y, long rows, float khinv)
{
    constexpr long n = 1024L * VPT;
    constexpr int E = 4 * VPT;
    __shared__ __attribute__((aligned(16))) float row_lds[n];
    __shared__ float red[2 * kRowWaves];
    __shared__ uint32_t zred[kRowWaves];
    const int t = threadIdx.x, w = t >> 6;
    const long G = gridDim.x;
    long row = blockIdx.x;
    // lane t of wave w copies the float4 groups t + 256 i of row r to the
    // same group index in row_lds; each instruction fills 1 KB at the
    // wave's base (64 lanes x 16 bytes)
    auto prefetch = [&](long r) {
        const float* src = x + r * n;
#pragma unroll
        for (int i = 0; i < VPT; i++)
            __builtin_amdgcn_global_load_lds(src + 4 * (t + kRowThreads * i),
                                             (__attribute__((address_space(3))) void*)(row_lds + 4 * (kRowThreads * i + 64 * w)),
                                             16, 0, 0);
    };
    prefetch(row);
    lds_barrier();
    for (; row < rows; row += G) {
        float v[E];
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const float4 q = *reinterpret_cast<const float4*>(row_lds + 4 * (t + kRowThreads * i));
            v[4 * i] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
        }
        // every wave has read row_lds (its lane maximum needs the values)
        // once the barrier inside block_maximum is passed
        const RowExtent r = unmasked_row_extent<VPT, true>(v, red, zred, row_lds);
        if (row + G < rows) prefetch(row + G);
        float s = unmasked_lane_exps<NITER, E>(v, r, khinv);
        // the prefetch has landed before the barrier below (the LDS fence
        // waits for it too; this states it, and the operand keeps the wait
        // after the exps)
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(s));
        s = block_sum<false, true>(s, red + kRowWaves);
        const float inv = inv_sum(s, 0);
#pragma unroll
        for (int e = 0; e < E; e++) v[e] = v[e] * inv;
        store_row_regs<VPT, true>(y + row * n, n / 4, v);
    }
}

// Workgroups of softmax_prefetch_kernel<VPT, NITER> resident per CU.
template <int VPT, int NITER>
static int softmax_prefetch_occupancy() {
    static std::atomic<int> cached{0};
    int v = cached.load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, softmax_prefetch_kernel<VPT, NITER>, kRowThreads, 0) !=
                hipSuccess || v < 1) {
            (void)hipGetLastError();
            v = 1;
        }
        cached.store(v, std::memory_order_relaxed);
    }
    return v;
}

template <int NITER, bool MASKED>
__global__ __launch_bounds__(kRowThreads) void softmax_loop_kernel(
    const float* x, float* y, long n, int iters, float khinv,
    SoftmaxMask mk)
{
    __shared__ float red[kRowWaves];
    const long row = blockIdx.x;
    const long t = MASKED ? mk.row0 + row % mk.seq : 0;
    const float* xr = x + row * n;
    float* yr = y + row * n;
    float m = -__builtin_inff();
    for (long i = threadIdx.x; i < n; i += kRowThreads) {
        float v = xr[i];
        if constexpr (MASKED) v = mask_score(v, t, i, mk);
        m = fmaxf(m, v);
    }
    m = block_max(m, red);
    if (m == 0.0f) {
        __shared__ uint64_t zred[kRowWaves];
        uint64_t key = ~0ull;
        for (long i = threadIdx.x; i < n; i += kRowThreads) {
            float v = xr[i];
            if constexpr (MASKED) v = mask_score(v, t, i, mk);
            if (v == 0.0f) {
                key = zero_key<uint64_t>(i, v);
                break;
            }
        }
        m = first_zero_max<false>(key, zred);
    }
    float s = 0.0f;
    for (long i = threadIdx.x; i < n; i += kRowThreads) {
        float v = xr[i];
        if constexpr (MASKED) v = mask_score(v, t, i, mk);
        const float e = exp_n<NITER>(v - m, iters, khinv);
        yr[i] = e;
        s += e;
    }
    s = block_sum(s, red);
    const float inv = inv_sum(s, MASKED ? mk.zero_guard : 0);
    for (long i = threadIdx.x; i < n; i += kRowThreads) yr[i] = yr[i] * inv;
}

// Workgroups per CU of the unmasked register kernel with compile-time steps.
// Its leaner arithmetic needs fewer VGPRs than the general form (59 / 82 /
// 113 at VPT 4 / 8 / 16 against 74 / 120 / 137), which would raise
// residency from 6 / 4 / 3 to 8 / 5 / 4 workgroups per CU.  At VPT 4 that
// was measured slower (softmax 4096 x 4096, n = 16: 8 per CU ran 29.2 µs
// median against 25.4 at 6 on one box, 0.97x on another; 6 per CU with the
// lean arithmetic: 0.95-0.99x of the general form), so the launch keeps the
// general form's residency by requesting unused dynamic LDS: 160 KB / cap
// minus 1 KB lets exactly `cap` workgroups share a CU's 160 KB.
constexpr long kCuLdsBytes = 160L * 1024;
constexpr int unmasked_reg_cap(int vpt) { return vpt <= 2 ? 0 : vpt == 4 ? 6 : vpt == 8 ? 4 : 3; }

template <int VPT, int NITER, bool MASKED>
static void softmax_reg_launch(dim3 grid, hipStream_t s, const float* x, float* y, long n, int iters,
                               float khinv, const SoftmaxMask& mk) {
    constexpr int cap = (!MASKED && NITER > 0) ? unmasked_reg_cap(VPT) : 0;
    constexpr size_t lds = cap ? (size_t)(kCuLdsBytes / cap - 1024) : 0;
    if (n == 4L * VPT * kRowThreads)
        hipLaunchKernelGGL((softmax_reg_kernel<VPT, NITER, MASKED, true>), grid, dim3(kRowThreads), lds, s, x, y,
                           n, iters, khinv, mk);
    else
        hipLaunchKernelGGL((softmax_reg_kernel<VPT, NITER, MASKED, false>), grid, dim3(kRowThreads), lds, s, x,
                           y, n, iters, khinv, mk);
}

template <int NITER, bool MASKED>
static hipError_t softmax_dispatch(const float* x, float* y, long rows, long n, int iters,
                                   float khinv, hipStream_t s, const SoftmaxMask& mk) {
    const bool vec_ok = (n % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0) &&
                        ((reinterpret_cast<uintptr_t>(y) & 15) == 0);
    const long n4 = n / 4;
    dim3 grid((unsigned)rows), block(kRowThreads);
    if constexpr (!MASKED && NITER > 0 && NITER <= 8) {
        // short exps: the persistent prefetching kernel, where every
        // workgroup gets at least two rows
        auto prefetch_launch = [&](auto vpt) -> bool {
            constexpr int VPT = decltype(vpt)::value;
            if (n != 1024L * VPT) return false;
            const long g = (long)softmax_prefetch_occupancy<VPT, NITER>() * device_cus();
            if (rows < 2 * g) return false;
            hipLaunchKernelGGL((softmax_prefetch_kernel<VPT, NITER>), dim3((unsigned)g), block, 0, s, x, y, rows,
                               khinv);
            return true;
        };
        if (vec_ok && (prefetch_launch(std::integral_constant<int, 1>{}) ||
                       prefetch_launch(std::integral_constant<int, 2>{}) ||
                       prefetch_launch(std::integral_constant<int, 4>{})))
            return hipGetLastError();
    }
    if (vec_ok && n4 <= 1 * kRowThreads)
        softmax_reg_launch<1, NITER, MASKED>(grid, s, x, y, n, iters, khinv, mk);
    else if (vec_ok && n4 <= 2 * kRowThreads)
        softmax_reg_launch<2, NITER, MASKED>(grid, s, x, y, n, iters, khinv, mk);
    else if (vec_ok && n4 <= 4 * kRowThreads)
        softmax_reg_launch<4, NITER, MASKED>(grid, s, x, y, n, iters, khinv, mk);
    else if (vec_ok && n4 <= 8 * kRowThreads)
        softmax_reg_launch<8, NITER, MASKED>(grid, s, x, y, n, iters, khinv, mk);
    else if (vec_ok && n4 <= 16 * kRowThreads)
        softmax_reg_launch<16, NITER, MASKED>(grid, s, x, y, n, iters, khinv, mk);
    else
        hipLaunchKernelGGL((softmax_loop_kernel<NITER, MASKED>), grid, block, 0, s, x, y, n, iters, khinv, mk);
    return hipGetLastError();
}

template <int NITER>
static hipError_t softmax_mask_dispatch(const float* x, float* y, long rows, long n, int iters,
                                        float khinv, hipStream_t s, const SoftmaxMask& mk) {
    if (mk.mask || mk.causal || mk.zero_guard) {
        SoftmaxMask m2 = mk;
        if (m2.seq <= 0) m2.seq = n;   // square scores: row length = sequence length
        if (m2.mask_ld <= 0) m2.mask_ld = n;
        return softmax_dispatch<NITER, true>(x, y, rows, n, iters, khinv, s, m2);
    }
    return softmax_dispatch<NITER, false>(x, y, rows, n, iters, khinv, s, mk);
}

hipError_t softmax_launch(const float* x, float* y, long rows, long n, int iters, hipStream_t s,
                          const SoftmaxMask& mk) {
    iters = clamp_iters(iters);
    const float khinv = host_consts().exp_khinv[iters];
    switch (iters) {
        case 8: return softmax_mask_dispatch<8>(x, y, rows, n, iters, khinv, s, mk);
        case 16: return softmax_mask_dispatch<16>(x, y, rows, n, iters, khinv, s, mk);
        case 24: return softmax_mask_dispatch<24>(x, y, rows, n, iters, khinv, s, mk);
        default: return softmax_mask_dispatch<0>(x, y, rows, n, iters, khinv, s, mk);
    }
}

// ── RMSNorm / LayerNorm ──────────────────────────────────────────────────

template <int VPT>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_reg_kernel(
    const float* __restrict__ x, float* __restrict__ y, const float* __restrict__ gamma,
    float eps, long d, float khinv16)
{
    __shared__ float red[kRowWaves];
    const long row = blockIdx.x;
    const float4* xr = reinterpret_cast<const float4*>(x + row * d);
    float4* yr = reinterpret_cast<float4*>(y + row * d);
    const float4* g4 = reinterpret_cast<const float4*>(gamma);
    const long d4 = d / 4;
    float4 v[VPT];
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const long idx = threadIdx.x + (long)i * kRowThreads;
        v[i] = (idx < d4) ? ld4_stream(&xr[idx]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        ss = __builtin_fmaf(v[i].x, v[i].x, ss);
        ss = __builtin_fmaf(v[i].y, v[i].y, ss);
        ss = __builtin_fmaf(v[i].z, v[i].z, ss);
        ss = __builtin_fmaf(v[i].w, v[i].w, ss);
    }
    const float ms = block_sum(ss, red) / (float)d;
    const float inv = rsqrt_cordic(ms + eps, khinv16);
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const long idx = threadIdx.x + (long)i * kRowThreads;
        if (idx < d4) {
            const float4 g = gamma ? g4[idx] : make_float4(1.f, 1.f, 1.f, 1.f);
            float4 o;
            o.x = v[i].x * inv * g.x; o.y = v[i].y * inv * g.y;
            o.z = v[i].z * inv * g.z; o.w = v[i].w * inv * g.w;
            st4_stream(&yr[idx], o);
        }
    }
}

__global__ __launch_bounds__(kRowThreads) void rmsnorm_loop_kernel(
    const float* __restrict__ x, float* __restrict__ y, const float* __restrict__ gamma,
    float eps, long d, float khinv16)
{
    __shared__ float red[kRowWaves];
    const long row = blockIdx.x;
    const float* xr = x + row * d;
    float* yr = y + row * d;
    float ss = 0.0f;
    for (long i = threadIdx.x; i < d; i += kRowThreads) ss = __builtin_fmaf(xr[i], xr[i], ss);
    const float ms = block_sum(ss, red) / (float)d;
    const float inv = rsqrt_cordic(ms + eps, khinv16);
    for (long i = threadIdx.x; i < d; i += kRowThreads) {
        const float g = gamma ? gamma[i] : 1.0f;
        yr[i] = xr[i] * inv * g;
    }
}

template <int VPT>
__global__ __launch_bounds__(kRowThreads) void layernorm_reg_kernel(
    const float* __restrict__ x, float* __restrict__ y, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, long d, float khinv16)
{
    __shared__ float red[kRowWaves];
    const long row = blockIdx.x;
    const float4* xr = reinterpret_cast<const float4*>(x + row * d);
    float4* yr = reinterpret_cast<float4*>(y + row * d);
    const float4* g4 = reinterpret_cast<const float4*>(gamma);
    const float4* b4 = reinterpret_cast<const float4*>(beta);
    const long d4 = d / 4;
    float4 v[VPT];
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const long idx = threadIdx.x + (long)i * kRowThreads;
        v[i] = (idx < d4) ? ld4_stream(&xr[idx]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float sm = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; i++) { sm += v[i].x; sm += v[i].y; sm += v[i].z; sm += v[i].w; }
    const float mean = block_sum(sm, red) / (float)d;
    float sv = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const long idx = threadIdx.x + (long)i * kRowThreads;
        if (idx < d4) {
            float z;
            z = v[i].x - mean; sv = __builtin_fmaf(z, z, sv);
            z = v[i].y - mean; sv = __builtin_fmaf(z, z, sv);
            z = v[i].z - mean; sv = __builtin_fmaf(z, z, sv);
            z = v[i].w - mean; sv = __builtin_fmaf(z, z, sv);
        }
    }
    const float var = block_sum(sv, red) / (float)d;
    const float inv = rsqrt_cordic(var + eps, khinv16);
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const long idx = threadIdx.x + (long)i * kRowThreads;
        if (idx < d4) {
            const float4 g = gamma ? g4[idx] : make_float4(1.f, 1.f, 1.f, 1.f);
            const float4 b = beta ? b4[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 o;
            o.x = __builtin_fmaf(g.x, (v[i].x - mean) * inv, b.x);
            o.y = __builtin_fmaf(g.y, (v[i].y - mean) * inv, b.y);
            o.z = __builtin_fmaf(g.z, (v[i].z - mean) * inv, b.z);
            o.w = __builtin_fmaf(g.w, (v[i].w - mean) * inv, b.w);
            st4_stream(&yr[idx], o);
        }
    }
}

__global__ __launch_bounds__(kRowThreads) void layernorm_loop_kernel(
    const float* __restrict__ x, float* __restrict__ y, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, long d, float khinv16)
{
    __shared__ float red[kRowWaves];
    const long row = blockIdx.x;
    const float* xr = x + row * d;
    float* yr = y + row * d;
    float sm = 0.0f;
    for (long i = threadIdx.x; i < d; i += kRowThreads) sm += xr[i];
    const float mean = block_sum(sm, red) / (float)d;
    float sv = 0.0f;
    for (long i = threadIdx.x; i < d; i += kRowThreads) {
        const float z = xr[i] - mean;
        sv = __builtin_fmaf(z, z, sv);
    }
    const float var = block_sum(sv, red) / (float)d;
    const float inv = rsqrt_cordic(var + eps, khinv16);
    for (long i = threadIdx.x; i < d; i += kRowThreads) {
        const float g = gamma ? gamma[i] : 1.0f;
        const float b = beta ? beta[i] : 0.0f;
        yr[i] = __builtin_fmaf(g, (xr[i] - mean) * inv, b);
    }
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

hipError_t rmsnorm_launch(const float* x, float* y, const float* gamma, float eps,
                          long rows, long d, hipStream_t s) {
    const float k = host_consts().rsqrt_khinv;
    const bool vec_ok = (d % 4 == 0) && aligned16(x) && aligned16(y) && (!gamma || aligned16(gamma));
    const long d4 = d / 4;
    dim3 grid((unsigned)rows), block(kRowThreads);
    if (vec_ok && d4 <= kRowThreads)
        hipLaunchKernelGGL((rmsnorm_reg_kernel<1>), grid, block, 0, s, x, y, gamma, eps, d, k);
    else if (vec_ok && d4 <= 2 * kRowThreads)
        hipLaunchKernelGGL((rmsnorm_reg_kernel<2>), grid, block, 0, s, x, y, gamma, eps, d, k);
    else if (vec_ok && d4 <= 4 * kRowThreads)
        hipLaunchKernelGGL((rmsnorm_reg_kernel<4>), grid, block, 0, s, x, y, gamma, eps, d, k);
    else if (vec_ok && d4 <= 8 * kRowThreads)
        hipLaunchKernelGGL((rmsnorm_reg_kernel<8>), grid, block, 0, s, x, y, gamma, eps, d, k);
    else if (vec_ok && d4 <= 16 * kRowThreads)
        hipLaunchKernelGGL((rmsnorm_reg_kernel<16>), grid, block, 0, s, x, y, gamma, eps, d, k);
    else
        hipLaunchKernelGGL(rmsnorm_loop_kernel, grid, block, 0, s, x, y, gamma, eps, d, k);
    return hipGetLastError();
}

hipError_t layernorm_launch(const float* x, float* y, const float* gamma, const float* beta,
                            float eps, long rows, long d, hipStream_t s) {
    const float k = host_consts().rsqrt_khinv;
    const bool vec_ok = (d % 4 == 0) && aligned16(x) && aligned16(y) &&
                        (!gamma || aligned16(gamma)) && (!beta || aligned16(beta));
    const long d4 = d / 4;
    dim3 grid((unsigned)rows), block(kRowThreads);
    if (vec_ok && d4 <= kRowThreads)
        hipLaunchKernelGGL((layernorm_reg_kernel<1>), grid, block, 0, s, x, y, gamma, beta, eps, d, k);
    else if (vec_ok && d4 <= 2 * kRowThreads)
        hipLaunchKernelGGL((layernorm_reg_kernel<2>), grid, block, 0, s, x, y, gamma, beta, eps, d, k);
    else if (vec_ok && d4 <= 4 * kRowThreads)
        hipLaunchKernelGGL((layernorm_reg_kernel<4>), grid, block, 0, s, x, y, gamma, beta, eps, d, k);
    else if (vec_ok && d4 <= 8 * kRowThreads)
        hipLaunchKernelGGL((layernorm_reg_kernel<8>), grid, block, 0, s, x, y, gamma, beta, eps, d, k);
    else if (vec_ok && d4 <= 16 * kRowThreads)
        hipLaunchKernelGGL((layernorm_reg_kernel<16>), grid, block, 0, s, x, y, gamma, beta, eps, d, k);
    else
        hipLaunchKernelGGL(layernorm_loop_kernel, grid, block, 0, s, x, y, gamma, beta, eps, d, k);
    return hipGetLastError();
}

}  // namespace rac
