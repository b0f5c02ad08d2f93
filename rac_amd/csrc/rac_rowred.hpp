// rac_rowred.hpp — the fixed-order reductions of the row kernels (softmax,
// RMSNorm, LayerNorm) and of the decode attention, which must sum a row in
// the same order as the softmax kernel.  A 256-lane workgroup (4 wave64)
// reduces one row: each lane's partial, a wave64 XOR butterfly (offsets 32
// .. 1; after it every lane holds the same value, since each step adds a
// pair in either order), then the four wave partials in order.
#pragma once
#include <hip/hip_runtime.h>

namespace rac {

constexpr int kRowThreads = 256;
constexpr int kRowWaves = kRowThreads / 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// IEEE maximum (NaN-propagating; -0 < +0 like v_max_f32): no operand
// canonicalisation, and a NaN anywhere reaches every lane.
__device__ __forceinline__ float maximum(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float wave_maximum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = maximum(v, __shfl_xor(v, off, 64));
    return v;
}

// Workgroup barrier that orders LDS only.  __syncthreads() also releases
// global memory, which makes every wave wait for its outstanding global
// stores; a kernel that keeps stores in flight across its row reductions
// uses this instead (LDS writes issued by global_load_lds count as LDS
// writes, so the release still waits for those).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <bool LDS_ONLY>
__device__ __forceinline__ void red_barrier() {
    if constexpr (LDS_ONLY) lds_barrier();
    else __syncthreads();
}

// Block-wide reductions; `red` holds kRowWaves floats.  The result is the
// same value in every lane (fixed combination order).  TRAIL: end with a
// barrier, so that `red` may be rewritten at once; callers that give each
// reduction of a row its own `red` leave it off.  LDS_ONLY: the barriers
// order LDS only (lds_barrier).
template <bool TRAIL = true, bool LDS_ONLY = false>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    red_barrier<LDS_ONLY>();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kRowWaves; i++) r += red[i];
    if constexpr (TRAIL) red_barrier<LDS_ONLY>();
    return r;
}
// The reference's row maximum (rac_cpu.c:258-262: m = x[0], replaced only
// by a strictly greater x[i]) is the first element, in index order, of
// those equal to the maximum value.  A parallel maximum finds the value, and
// can differ from that element only in the sign of a zero maximum (+0 and -0
// compare equal).  x - max then differs in the sign of zero for the -0
// entries, which the CORDIC exp's first direction sees (a zero query row in
// attention gives such rows).  So when the maximum is zero, the row takes
// the sign of its first zero.  key: the lane's first zero as (element index
// << 1) | sign bit, all ones if it holds none (K: uint32_t where indices
// stay below 2^31, else uint64_t).  Returns the signed zero; every lane must
// call it (it holds barriers); zred: kRowWaves keys of LDS used by nothing
// else.
template <class K>
__device__ __forceinline__ K zero_key(long index, float v) {
    return ((K)index << 1) | (K)(__float_as_uint(v) >> 31);
}
template <bool LDS_ONLY, class K>
__device__ __forceinline__ float first_zero_max(K key, K* zred);

// block_max with the NaN-propagating maximum throughout.
template <bool TRAIL = true, bool LDS_ONLY = false>
__device__ __forceinline__ float block_maximum(float v, float* red) {
    v = wave_maximum(v);
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    red_barrier<LDS_ONLY>();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kRowWaves; i++) r = maximum(r, red[i]);
    if constexpr (TRAIL) red_barrier<LDS_ONLY>();
    return r;
}
template <bool TRAIL = true, bool LDS_ONLY = false>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    red_barrier<LDS_ONLY>();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kRowWaves; i++) r = fmaxf(r, red[i]);
    if constexpr (TRAIL) red_barrier<LDS_ONLY>();
    return r;
}

template <bool LDS_ONLY, class K>
__device__ __forceinline__ float first_zero_max(K key, K* zred) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const K o = __shfl_xor(key, off, 64);
        key = o < key ? o : key;
    }
    if ((threadIdx.x & 63) == 0) zred[threadIdx.x / 64] = key;
    red_barrier<LDS_ONLY>();
    K k = zred[0];
#pragma unroll
    for (int i = 1; i < kRowWaves; i++) k = zred[i] < k ? zred[i] : k;
    red_barrier<LDS_ONLY>();
    return (k & 1) ? -0.0f : 0.0f;
}

}  // namespace rac
