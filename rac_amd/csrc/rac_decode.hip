// rac_decode.hip — the per-token pieces of a decoder layer's decode step
// that are not GEMVs or row norms (bench/bench_rac_transformer.c
// decoder_forward_kv :557-616 with T_new = 1): the key/value cache append,
// grouped-query attention of the new token over the cache, SiLU(gate) * up,
// and the cache position's advance.
//
// The token's position lives in device memory (one int) and every kernel
// here reads it there, so the launches of a whole decode step have fixed
// arguments: the step can be recorded once as a HIP graph and replayed per
// token, the position advancing inside the graph.
//
// Attention is one workgroup (256 lanes) per query head h, reading key /
// value head g = h / rep of a cache laid out [n_kv_heads, t_cap, d_head]
// (each head's keys a row-major matrix).  Its arithmetic is that of the
// composition  scores = alpha * (q K^T) (FAST MAC: one fmaf chain over
// d_head in order, from +0), softmax by the row kernel, out = P V (one fmaf
// chain over the positions in order)  with the softmax row padded with -inf
// to a multiple of 4 (the row kernel's 16-byte form: lane l sums the
// elements 4 g .. 4 g + 3 of its groups g = l, l + 256, ... in order, then
// the fixed wave and block combination); P V over the padded length equals
// the unpadded one, since the padded probabilities are +0.  So the output
// is bit-identical to bmm -> softmax -> bmm on the padded scores.
#include <hip/hip_runtime.h>
#include "rac_act.hpp"
#include "rac_internal.hpp"
#include "rac_math.hpp"
#include "rac_rowred.hpp"

namespace rac {

// softmax exps of 4 values x - max (<= 0 or NaN), as the row kernel's
// unmasked form: step-major CORDIC for compile-time step counts (kLean:
// NaN is forced into the row sum separately), the runtime loop otherwise
template <int NITER>
__device__ __forceinline__ void dec_exp4(float* v, int iters, float khinv) {
    if constexpr (NITER > 0) {
        exp_cordic_vec<NITER, 4, kExpFlush | kExpNonPos>(v, khinv);
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = exp_cordic_rt(v[e], iters, khinv);
    }
}

// V tile staged in LDS for the P V chains: kDecTile floats (16 KB)
constexpr int kDecTile = 4096;

// Scores: lane t computes positions t, t + 256, ... (one fmaf chain each;
// DH > 0: the row's DH / 4 16-byte loads are issued together).  Softmax:
// lane l takes the groups l, l + 256, ... as the row kernel.  P V: the
// value rows pass through LDS a tile at a time (every lane loads, the next
// tile's loads are in flight during the chains), and lane c < d_head runs
// output column c's chain over the tile.
template <int NITER, int DH>
__global__ __launch_bounds__(kRowThreads) void decode_attention_kernel(
    const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc,
    float* __restrict__ out, int rep, int dh_rt, long t_cap, const int* __restrict__ pos_dev, float scale,
    int iters, float khinv)
{
    __shared__ __attribute__((aligned(16))) float sq[kDecodeMaxHead];
    __shared__ __attribute__((aligned(16))) float sp[kDecodeMaxLen];
    __shared__ __attribute__((aligned(16))) float sv[kDecTile];
    __shared__ float red[2 * kRowWaves];
    const int dh = DH > 0 ? DH : dh_rt;
    const int tid = threadIdx.x;
    const int h = blockIdx.x;
    const long g = h / rep;
    const int pos = *pos_dev;
    float* o = out + (long)h * dh;
    if (pos < 0 || pos >= t_cap || pos >= kDecodeMaxLen) {
        // a position outside the cache: NaN output, nothing read
        for (int c = tid; c < dh; c += kRowThreads) o[c] = __builtin_nanf("");
        return;
    }
    const int n = pos + 1;                 // positions 0 .. pos, the new token's included
    const int n4 = (n + 3) / 4;
    const float* K = kc + g * t_cap * dh;
    const float* V = vc + g * t_cap * dh;
    for (int c = tid; c < dh; c += kRowThreads) sq[c] = q[(long)h * dh + c];
    __syncthreads();

    for (int j = tid; j < n; j += kRowThreads) {
        const float* kr = K + (long)j * dh;
        float acc = 0.0f;
        if constexpr (DH > 0) {
            float4 kv[DH / 4];
#pragma unroll
            for (int k = 0; k < DH / 4; k++) kv[k] = reinterpret_cast<const float4*>(kr)[k];
#pragma unroll
            for (int k = 0; k < DH / 4; k++) {
                const float4 a = reinterpret_cast<const float4*>(sq)[k];
                acc = __builtin_fmaf(a.x, kv[k].x, acc);
                acc = __builtin_fmaf(a.y, kv[k].y, acc);
                acc = __builtin_fmaf(a.z, kv[k].z, acc);
                acc = __builtin_fmaf(a.w, kv[k].w, acc);
            }
        } else {
            for (int k = 0; k < dh; k++) acc = __builtin_fmaf(sq[k], kr[k], acc);
        }
        sp[j] = scale * acc;
    }
    if (tid < 4 * n4 - n) sp[n + tid] = -__builtin_inff();       // the row's -inf padding
    __syncthreads();

    // the lane's maximum, exps and sum over its groups, in group order
    float m = -__builtin_inff();
    for (int gi = tid; gi < n4; gi += kRowThreads) {
#pragma unroll
        for (int c = 0; c < 4; c++) m = fmaxf(m, sp[4 * gi + c]);
    }
    m = block_max<false>(m, red);
    if (m == 0.0f) {
        // the signed zero the reference's scan ends on (first_zero_max)
        __shared__ uint32_t zred[kRowWaves];
        uint32_t key = ~0u;
        for (int gi = tid; gi < n4 && key == ~0u; gi += kRowThreads) {
#pragma unroll
            for (int c = 3; c >= 0; c--)
                if (sp[4 * gi + c] == 0.0f) key = zero_key<uint32_t>(4 * gi + c, sp[4 * gi + c]);
        }
        m = first_zero_max<false>(key, zred);
    }
    constexpr bool kLean = NITER > 0;
    float nanp = -__builtin_inff();
    float s = 0.0f;
    for (int gi = tid; gi < n4; gi += kRowThreads) {
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            v[c] = sp[4 * gi + c] - m;
            if constexpr (kLean) nanp = __builtin_elementwise_maximum(nanp, v[c]);
        }
        dec_exp4<NITER>(v, iters, khinv);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            s += v[c];
            sp[4 * gi + c] = v[c];
        }
    }
    if constexpr (kLean) {
        if (nanp != nanp) s = __builtin_nanf("");
    }
    s = block_sum<false>(s, red + kRowWaves);
    const float inv = 1.0f / s;
    for (int gi = tid; gi < n4; gi += kRowThreads) {
#pragma unroll
        for (int c = 0; c < 4; c++) sp[4 * gi + c] = sp[4 * gi + c] * inv;
    }

    // out[c] = sum_j p_j V[j][c], one chain per output column in j order
    const int tj = kDecTile / dh;                        // value rows per tile
    constexpr int kF4 = kDecTile / 4 / kRowThreads;      // tile float4 per lane
    const bool vec = DH > 0;
    float4 pre[kF4];
    auto fetch = [&](int j0) {                           // rows j0 .. of the tile into registers
        const int cnt = (n - j0 < tj ? n - j0 : tj) * dh;
        const float* src = V + (long)j0 * dh;
#pragma unroll
        for (int i = 0; i < kF4; i++) {
            const int e = (tid + i * kRowThreads) * 4;
            if (vec) {
                pre[i] = e < cnt ? *reinterpret_cast<const float4*>(src + e) : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                pre[i].x = e < cnt ? src[e] : 0.0f;
                pre[i].y = e + 1 < cnt ? src[e + 1] : 0.0f;
                pre[i].z = e + 2 < cnt ? src[e + 2] : 0.0f;
                pre[i].w = e + 3 < cnt ? src[e + 3] : 0.0f;
            }
        }
    };
    float acc = 0.0f;
    fetch(0);
    for (int j0 = 0; j0 < n; j0 += tj) {
        __syncthreads();                                 // previous tile's chains done (and sp final)
#pragma unroll
        for (int i = 0; i < kF4; i++) reinterpret_cast<float4*>(sv)[tid + i * kRowThreads] = pre[i];
        __syncthreads();
        if (j0 + tj < n) fetch(j0 + tj);                 // in flight during the chains
        const int cnt = n - j0 < tj ? n - j0 : tj;
        if (tid < dh) {
            int u = 0;
            for (; u + 8 <= cnt; u += 8) {
#pragma unroll
                for (int w = 0; w < 8; w++) acc = __builtin_fmaf(sp[j0 + u + w], sv[(u + w) * dh + tid], acc);
            }
            for (; u < cnt; u++) acc = __builtin_fmaf(sp[j0 + u], sv[u * dh + tid], acc);
        }
    }
    if (tid < dh) o[tid] = acc;
}

template <int NITER>
static hipError_t decode_attention_dh(int dh, bool vec, const float* q, const float* kc, const float* vc,
                                      float* out, int n_heads, int rep, long t_cap, const int* pos, float scale,
                                      int iters, float khinv, hipStream_t s) {
#define RAC_DEC_ATT(D)                                                                                         \
    hipLaunchKernelGGL((decode_attention_kernel<NITER, D>), dim3(n_heads), dim3(kRowThreads), 0, s, q, kc, vc, \
                       out, rep, dh, t_cap, pos, scale, iters, khinv)
    if (vec && dh == 64) RAC_DEC_ATT(64);
    else if (vec && dh == 128) RAC_DEC_ATT(128);
    else if (vec && dh == 32) RAC_DEC_ATT(32);
    else RAC_DEC_ATT(0);
#undef RAC_DEC_ATT
    return hipGetLastError();
}

hipError_t decode_attention_launch(const float* q, const float* kc, const float* vc, float* out, int n_heads,
                                   int n_kv_heads, int dh, long t_cap, const int* pos, float scale, int iters,
                                   hipStream_t s) {
    iters = clamp_iters(iters);
    const float khinv = host_consts().exp_khinv[iters];
    const int rep = n_heads / n_kv_heads;
    // 16-byte loads of key and value rows: rows on 16-byte boundaries
    const bool vec = dh % 4 == 0 && (reinterpret_cast<uintptr_t>(kc) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(vc) & 15) == 0;
    switch (iters) {
        case 8: return decode_attention_dh<8>(dh, vec, q, kc, vc, out, n_heads, rep, t_cap, pos, scale, iters, khinv, s);
        case 16: return decode_attention_dh<16>(dh, vec, q, kc, vc, out, n_heads, rep, t_cap, pos, scale, iters, khinv, s);
        case 24: return decode_attention_dh<24>(dh, vec, q, kc, vc, out, n_heads, rep, t_cap, pos, scale, iters, khinv, s);
        default: return decode_attention_dh<0>(dh, vec, q, kc, vc, out, n_heads, rep, t_cap, pos, scale, iters, khinv, s);
    }
}

// ── cache append ─────────────────────────────────────────────────────────

// kv = [k (n_kv_heads * d_head) | v (n_kv_heads * d_head)] of the new token
// (the K and V projections' outputs, adjacent); written at the position
// *pos of every head's rows.  A position outside the cache writes nothing.
__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ kv, float* __restrict__ kc,
                                                       float* __restrict__ vc, long w, int dh, long t_cap,
                                                       const int* __restrict__ pos_dev) {
    const int pos = *pos_dev;
    if (pos < 0 || pos >= t_cap) return;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < 2 * w; i += (long)gridDim.x * 256) {
        const long r = i < w ? i : i - w;
        const long g = r / dh, c = r - g * dh;
        (i < w ? kc : vc)[(g * t_cap + pos) * dh + c] = kv[i];
    }
}

hipError_t kv_append_launch(const float* kv, float* kc, float* vc, int n_kv_heads, int dh, long t_cap,
                            const int* pos, hipStream_t s) {
    const long w = (long)n_kv_heads * dh;
    const long blocks = (2 * w + 255) / 256;
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, s, kv, kc,
                       vc, w, dh, t_cap, pos);
    return hipGetLastError();
}

__global__ void position_advance_kernel(int* pos, int by) {
    if (blockIdx.x == 0 && threadIdx.x == 0) *pos += by;
}

hipError_t position_advance_launch(int* pos, int by, hipStream_t s) {
    hipLaunchKernelGGL(position_advance_kernel, dim3(1), dim3(64), 0, s, pos, by);
    return hipGetLastError();
}

// ── SiLU(gate) * up ──────────────────────────────────────────────────────

// out[i] = silu(gu[i]) * gu[n + i]: the gate and up projections stacked in
// one vector; SiLU by the CORDIC exp of the elementwise kernels (same bits).
template <int NITER>
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gu, float* __restrict__ out, long n,
                                                    int iters, float khinv) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
        out[i] = elt<kEltSilu, NITER>(gu[i], iters, khinv) * gu[n + i];
}

hipError_t swiglu_launch(const float* gu, float* out, long n, int iters, hipStream_t s) {
    iters = clamp_iters(iters);
    const float khinv = host_consts().exp_khinv[iters];
    const long blocks = (n + 255) / 256;
    const dim3 grid((unsigned)(blocks < 4096 ? blocks : 4096));
    switch (iters) {
        case 8: hipLaunchKernelGGL((swiglu_kernel<8>), grid, dim3(256), 0, s, gu, out, n, iters, khinv); break;
        case 16: hipLaunchKernelGGL((swiglu_kernel<16>), grid, dim3(256), 0, s, gu, out, n, iters, khinv); break;
        case 24: hipLaunchKernelGGL((swiglu_kernel<24>), grid, dim3(256), 0, s, gu, out, n, iters, khinv); break;
        default: hipLaunchKernelGGL((swiglu_kernel<0>), grid, dim3(256), 0, s, gu, out, n, iters, khinv); break;
    }
    return hipGetLastError();
}

}  // namespace rac
