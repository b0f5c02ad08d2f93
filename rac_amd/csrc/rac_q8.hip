// rac_q8.hip — Q8_0 weights (lib/c/rac_q8_0.h: blocks of 32 int8 with one
// fp16 scale, 34 bytes) and the decode GEMV out = act(W x + bias) on gfx950.
//
// The GEMV is HBM-bound: every weight byte is read once (34 bytes per 32
// weights, 3.8x less than fp32).  Results are bit-identical to the
// reference's AVX2 build (rac_q8_0.c:128-211): each block's 32 products
// combine in the order of its 8-lane vector tree, and the block terms of a
// row accumulate in block order as acc = fma(d_b, dot_b, acc).  The fast
// kernel keeps that serial order while the loads of a whole chunk (16 or 32
// rows x 32 blocks) are in flight at once; shapes it does not cover
// (K % 256 != 0, unaligned weights) take a generic kernel with the same
// arithmetic.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include "rac_act.hpp"
#include "rac_internal.hpp"
#include "rac_math.hpp"
#include "rac_q8.hpp"
#include "rac_rowred.hpp"

namespace rac {

// One block's dot product, in the AVX2 kernel's order: lane l of 8 sums
// q[l] x[l], then fma with q[l+8] x[l+8], q[l+16] x[l+16], q[l+24] x[l+24];
// the 8 sums combine as ((a0+a4) + (a1+a5)) + ((a2+a6) + (a3+a7)).
template <typename QP, typename XP>
__device__ __forceinline__ float q8_block_dot(QP q, XP x) {
    float a[8];
#pragma unroll
    for (int l = 0; l < 8; l++) {
        float s = (float)q[l] * x[l];
        s = __builtin_fmaf((float)q[l + 8], x[l + 8], s);
        s = __builtin_fmaf((float)q[l + 16], x[l + 16], s);
        s = __builtin_fmaf((float)q[l + 24], x[l + 24], s);
        a[l] = s;
    }
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s1) + (s2 + s3);
}

// act(acc + bias) as rac_q8_0.c:167-174, 205-207 (erff / expf of the device
// math library).
__device__ __forceinline__ float q8_finish(float acc, const float* bias, long j, int act) {
    if (bias) acc += bias[j];
    switch (act) {
    case 1: return acc > 0.0f ? acc : 0.0f;
    case 2: return 0.5f * acc * (1.0f + erff(acc * 0.7071067811865f));
    case 3: return acc / (1.0f + expf(-acc));
    default: return acc;
    }
}

// Fast path (K % 256 == 0, K >= 32 CB, 16-byte aligned buffers).  A
// workgroup owns R consecutive weight rows and walks K in chunks of CB
// blocks (R x CB x 34 bytes, all requested at once, so the whole chunk is
// in flight before any of it is used):
//   1. 16-byte loads of the chunk (contiguous per row) -> registers -> LDS;
//   2. every lane computes block dots, lane-fast along a row (consecutive
//      lanes read consecutive blocks, the x slice is padded to 33 floats
//      per block, so LDS reads do not collide), and stores (d, dot);
//   3. lane (m, r) folds its row's terms in block order.
// Every chunk is a full CB blocks: when CB does not divide the row, the
// last chunk starts CB blocks before the row end and its first blocks,
// already folded, are skipped.  So the loads' placement is one fixed
// pattern per lane, computed once, and no code depends on a run-time chunk
// width.  The next chunk's loads are issued before the current chunk's
// math.  Up to 4 input rows (batched decode) share one pass over the
// weights, 5-8 rows one pass of the 8-row kernel (at K >= 1024).  The shape
// only decides which lane computes what; every output
// is the same serial fold, so all shapes give identical bits.
// One input row asks for 4 workgroups per CU (at most 128 VGPRs; the
// kernel needs 123), several rows for 2.
// A block's 32 x floats sit in LDS rows of 36 (16-byte rows): the dot
// phase reads them with 8 ds_read_b128 at immediate offsets from one
// address, and a lane's k-stride of 36 dwords keeps every 16-lane pass on
// distinct banks.
constexpr int kQ8XPad = 36;                                 // x floats per block in LDS

// Fusions of a decoder layer's decode step into the one-row GEMV:
//   NORM   x is replaced by rmsnorm(x) * gamma with the row kernel's
//          arithmetic and sum order (lane l's float4 groups l, l + 256, ...,
//          fmaf of the squares in order, the fixed block combination, the
//          CORDIC rsqrt of mean + eps, then (x * inv) * gamma), computed by
//          every workgroup while its first chunk's loads are in flight.
//   EPI 1  rows come in gate / up pairs (2i, 2i + 1): out[i] =
//          silu(gate) * up, SiLU by the runtime-step CORDIC exp.
//   EPI 2  rows [split, split + kvw) are the token's keys, [split + kvw,
//          split + 2 kvw) its values: written into kc / vc [heads, t_cap,
//          dh] at position *pos (nothing for a position outside the cache);
//          rows below split go to out.
// Each output's fold is the plain kernel's, so its bits are unchanged.
struct Q8Fuse {
    const float* gamma = nullptr;
    float eps = 0.0f, rs_khinv = 0.0f;
    int iters = 0;
    float khinv = 0.0f;
    int split = 0, kvw = 0, dh = 1;
    long t_cap = 0;
    const int* pos = nullptr;
    float* kc = nullptr;
    float* vc = nullptr;
};

template <int MX, int CB, int R, bool NORM = false, int EPI = 0>
__global__ __launch_bounds__(256, MX == 1 ? 4 : 2) void q8_gemv_kernel(const float* __restrict__ x,
                                                      const uint8_t* __restrict__ w,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ out, int M, int N, int K,
                                                      int act, Q8Fuse fz = Q8Fuse()) {
    static_assert(256 % CB == 0 && CB % 8 == 0 && R * CB >= 256 && MX * R <= 256, "chunk shape");
    static_assert((!NORM && EPI == 0) || MX == 1, "decode fusions take one input row");
    static_assert(EPI != 1 || R % 2 == 0, "gate / up pairs stay in one workgroup");
    constexpr int kRowLds = CB * kQ8Bytes + 16;                       // row stride in LDS (16-byte multiple)
    constexpr int kVrow = CB * kQ8Bytes / 16;                         // 16-byte vectors per row and chunk
    constexpr int kVPT = (R * kVrow + 255) / 256;                     // weight vectors per lane
    constexpr int kXF4 = MX * CB * kQ8Block / 4;                      // x float4 per chunk
    constexpr int kXPT = (kXF4 + 255) / 256;                          // x float4 per lane
    constexpr int kRPT = R * CB / 256;                                // rows per lane in the dot phase
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) uint8_t sw[R * kRowLds];
    __shared__ __attribute__((aligned(16))) float sx[MX][CB * kQ8XPad];
    constexpr int kTermLd = CB + 4;                                    // 16-byte rows: the fold reads float4
    __shared__ __attribute__((aligned(16))) float sdot[MX][R][kTermLd];
    __shared__ __attribute__((aligned(16))) float sd[R][kTermLd];

    const int tid = threadIdx.x;
    const long j0 = (long)blockIdx.x * R;
    const int nrows = (int)min((long)R, (long)N - j0);
    const int nb = K / kQ8Block;                     // >= CB, multiple of 8
    const long rowB = (long)nb * kQ8Bytes;
    const int nch = (nb + CB - 1) / CB;

    // Vector placement, fixed for every chunk: byte offset of this lane's
    // vector i from the chunk start (rows past the last re-read row 0: every
    // load is unconditional, so a chunk's loads are all in flight together)
    // and its LDS offset (-1: nothing to store).  The byte offset is 64-bit:
    // R rows of a very long K (R rowB >= 2^32 from K ~ 2.5e8 at R = 16)
    // would wrap a 32-bit one.
    long goff[kVPT];
    int soff[kVPT];
#pragma unroll
    for (int i = 0; i < kVPT; i++) {
        const int v = tid + i * 256;
        const bool in = v < R * kVrow;
        const int r = in ? v / kVrow : 0, o = in ? v % kVrow : 0;
        goff[i] = (long)(r < nrows ? r : 0) * rowB + o * 16;
        soff[i] = (in && r < nrows) ? r * kRowLds + o * 16 : -1;
    }
    u4 rw[kVPT];
    float4 rx[kXPT];
    float4 rg[NORM ? kXPT : 1];
    auto chunk_start = [&](int c) { return min(c * CB, nb - CB); };
    auto fetch = [&](int b0) {
        const uint8_t* base = w + j0 * rowB + (long)b0 * kQ8Bytes;
#pragma unroll
        for (int i = 0; i < kVPT; i++)
            rw[i] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(base + goff[i]));
#pragma unroll
        for (int i = 0; i < kXPT; i++) {
            const int e = min(tid + i * 256, kXF4 - 1) * 4;           // float index in [MX][CB*32]
            const int m = e / (CB * kQ8Block), q = e % (CB * kQ8Block);
            rx[i] = *reinterpret_cast<const float4*>(x + (long)min(m, M - 1) * K + (long)b0 * kQ8Block + q);
            if constexpr (NORM) rg[i] = *reinterpret_cast<const float4*>(fz.gamma + (long)b0 * kQ8Block + q);
        }
    };

    float acc = 0.0f;          // lane tid < MX * R owns output (tid / R, j0 + tid % R)
    fetch(chunk_start(0));
    float inv = 1.0f;
    if constexpr (NORM) {
        __shared__ float red[kRowWaves];
        const float4* x4 = reinterpret_cast<const float4*>(x);
        float ss = 0.0f;
        for (int i = tid; i < K / 4; i += 256) {
            const float4 v = x4[i];
            ss = __builtin_fmaf(v.x, v.x, ss);
            ss = __builtin_fmaf(v.y, v.y, ss);
            ss = __builtin_fmaf(v.z, v.z, ss);
            ss = __builtin_fmaf(v.w, v.w, ss);
        }
        const float ms = block_sum(ss, red) / (float)K;
        inv = rsqrt_cordic(ms + fz.eps, fz.rs_khinv);
    }
    for (int c = 0; c < nch; c++) {
        const int b0 = chunk_start(c);
        const int k0 = c * CB - b0;                  // blocks of this chunk already folded
        __syncthreads();                             // previous chunk's LDS consumed
#pragma unroll
        for (int i = 0; i < kVPT; i++)
            if (soff[i] >= 0) *reinterpret_cast<u4*>(&sw[soff[i]]) = rw[i];
#pragma unroll
        for (int i = 0; i < kXPT; i++) {
            const int e = (tid + i * 256) * 4;
            if (kXF4 % 256 == 0 || e < kXF4 * 4) {
                const int m = e / (CB * kQ8Block), q = e % (CB * kQ8Block);
                // stored component by component: a whole-float4 copy of rx[i]
                // sends the staging array to scratch memory
                float4* dst = reinterpret_cast<float4*>(&sx[m][(q / kQ8Block) * kQ8XPad + q % kQ8Block]);
                if constexpr (NORM) {
                    *dst = make_float4(rx[i].x * inv * rg[i].x, rx[i].y * inv * rg[i].y,
                                       rx[i].z * inv * rg[i].z, rx[i].w * inv * rg[i].w);
                } else {
                    *dst = make_float4(rx[i].x, rx[i].y, rx[i].z, rx[i].w);
                }
            }
        }
        __syncthreads();
        if (c + 1 < nch) fetch(chunk_start(c + 1));  // in flight during the math
        // block dots: lane owns block k = tid % CB of rows tid / CB + (256 / CB) i
        const int k = tid % CB;
        if (k < k0) {
            // already folded: (0, 0) terms leave the fold unchanged, since
            // fma(0, 0, acc) == acc for every acc the fold can hold (it
            // starts at +0 and a sum rounds to -0 only from -0 + -0)
#pragma unroll
            for (int i = 0; i < kRPT; i++) {
                const int r = tid / CB + (256 / CB) * i;
                sd[r][k] = 0.0f;
#pragma unroll
                for (int m = 0; m < MX; m++) sdot[m][r][k] = 0.0f;
            }
        } else {
            float xr[kQ8Block];
            if constexpr (MX == 1) {
#pragma unroll
                for (int i = 0; i < kQ8Block / 4; i++) {
                    const float4 v = *reinterpret_cast<const float4*>(&sx[0][k * kQ8XPad + 4 * i]);
                    xr[4 * i] = v.x; xr[4 * i + 1] = v.y; xr[4 * i + 2] = v.z; xr[4 * i + 3] = v.w;
                }
            }
#pragma unroll
            for (int i = 0; i < kRPT; i++) {
                const int r = tid / CB + (256 / CB) * i;
                const int A = r * kRowLds + k * kQ8Bytes;     // block start (2-byte aligned)
                const uint32_t* dw = reinterpret_cast<const uint32_t*>(&sw[A & ~3]);
                uint32_t d0[10];
#pragma unroll
                for (int t = 0; t < 10; t++) d0[t] = dw[t];
                // the block's dwords: shifted down 16 bits when it starts 2
                // bytes into its first dword (a shift of 0 returns d0[t])
                uint32_t wd[9];
#pragma unroll
                for (int t = 0; t < 9; t++) wd[t] = __builtin_amdgcn_alignbit(d0[t + 1], d0[t], (A & 2) * 8);
                float qf[kQ8Block];
#pragma unroll
                for (int t = 0; t < kQ8Block; t++) qf[t] = (float)(int8_t)(wd[(2 + t) / 4] >> (8 * ((2 + t) % 4)));
                sd[r][k] = half_bits_to_float_cvt(wd[0] & 0xffffu);
                if constexpr (MX == 1) {
                    sdot[0][r][k] = q8_block_dot(qf, xr);
                } else {
#pragma unroll
                    for (int m = 0; m < MX; m++)
                        if (m < M) sdot[m][r][k] = q8_block_dot(qf, &sx[m][k * kQ8XPad]);
                }
            }
        }
        __syncthreads();
        // ordered fold of this chunk's terms
        if (tid < MX * R) {
            const int m = tid / R, r = tid % R;
            if (m < M && r < nrows) {
                // 16 terms per LDS round trip (float4 reads of both rows)
                constexpr int kB = CB < 16 ? CB : 16;
#pragma unroll
                for (int kk = 0; kk < CB; kk += kB) {
                    float4 dv[kB / 4], tv[kB / 4];
#pragma unroll
                    for (int u = 0; u < kB / 4; u++) {
                        dv[u] = *reinterpret_cast<const float4*>(&sd[r][kk + 4 * u]);
                        tv[u] = *reinterpret_cast<const float4*>(&sdot[m][r][kk + 4 * u]);
                    }
#pragma unroll
                    for (int u = 0; u < kB / 4; u++) {
                        acc = __builtin_fmaf(dv[u].x, tv[u].x, acc);
                        acc = __builtin_fmaf(dv[u].y, tv[u].y, acc);
                        acc = __builtin_fmaf(dv[u].z, tv[u].z, acc);
                        acc = __builtin_fmaf(dv[u].w, tv[u].w, acc);
                    }
                }
            }
        }
    }
    if constexpr (EPI == 1) {
        // lanes 2i and 2i + 1 (wave 0) hold a pair's gate and up
        const float up = __shfl_down(acc, 1, 64);
        if (tid < R && tid % 2 == 0 && tid < nrows)
            out[(j0 + tid) / 2] = elt<kEltSilu, 0>(acc, fz.iters, fz.khinv) * up;
    } else if constexpr (EPI == 2) {
        if (tid < R && tid < nrows) {
            const long j = j0 + tid;
            const float v = bias ? acc + bias[j] : acc;
            if (j < fz.split) {
                out[j] = v;
            } else {
                const int p = *fz.pos;
                const long r = j - fz.split;
                const bool is_v = r >= fz.kvw;
                const long rr = is_v ? r - fz.kvw : r;
                const long hh = rr / fz.dh, c = rr - hh * fz.dh;
                if (p >= 0 && p < fz.t_cap) (is_v ? fz.vc : fz.kc)[(hh * fz.t_cap + p) * fz.dh + c] = v;
            }
        }
    } else {
        if (tid < MX * R) {
            const int m = tid / R, r = tid % R;
            if (m < M && r < nrows) out[(long)m * N + j0 + r] = q8_finish(acc, bias, j0 + r, act);
        }
    }
}

// Generic path (any K % 32 == 0, any alignment): one wave per output
// (m, j); lane l computes the dot of block b0 + l straight from global
// memory, then every lane folds the 64 terms in block order through
// broadcasts (the accumulator is wave-uniform).
__global__ __launch_bounds__(256) void q8_gemv_generic_kernel(const float* __restrict__ x,
                                                              const uint8_t* __restrict__ w,
                                                              const float* __restrict__ bias,
                                                              float* __restrict__ out, int M, int N,
                                                              int K, int act) {
    const int lane = threadIdx.x % 64;
    const long o = (long)blockIdx.x * 4 + threadIdx.x / 64;
    if (o >= (long)M * N) return;      // the whole wave leaves together
    const long m = o / N, j = o % N;
    const int nb = K / kQ8Block;
    const uint8_t* row = w + j * (long)nb * kQ8Bytes;
    const float* xm = x + m * K;
    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += 64) {
        const int b = b0 + lane;
        float dot = 0.0f, d = 0.0f;
        if (b < nb) {
            const uint8_t* blk = row + (long)b * kQ8Bytes;
            dot = q8_block_dot(reinterpret_cast<const int8_t*>(blk + 2), xm + (long)b * kQ8Block);
            d = half_bits_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        }
        const int cnt = min(64, nb - b0);
        for (int i = 0; i < cnt; i++) acc = __builtin_fmaf(__shfl(d, i, 64), __shfl(dot, i, 64), acc);
    }
    if (lane == 0) out[m * N + j] = q8_finish(acc, bias, j, act);
}

// One input row on the fast path: the workgroup shape by the number of
// rows.  16 rows per workgroup while that still gives two workgroups per
// CU; below, 4 rows (8 when a row has fewer than 64 blocks) so that small
// matrices spread over every CU (measured on MI355X with weights streamed
// from HBM: 2560 x 2048 in 4.6 us instead of 5.2, 2048 x 5632 in 7.1
// instead of 10.3).  The shape only changes which lane computes what.
template <bool NORM, int EPI>
static void q8_launch_row(const float* x, const uint8_t* w, const float* bias, float* out, int N, int K, int act,
                          const Q8Fuse& fz, hipStream_t s) {
    const int nb = K / kQ8Block;
    const long cus = device_cus();
#define RAC_Q8_ROW(CB, R)                                                                                   \
    hipLaunchKernelGGL((q8_gemv_kernel<1, CB, R, NORM, EPI>), dim3((unsigned)((N + R - 1) / R)), dim3(256), 0, \
                       s, x, w, bias, out, 1, N, K, act, fz)
    if (nb < 32) RAC_Q8_ROW(8, 32);
    else if ((N + 15) / 16 >= 2 * cus) RAC_Q8_ROW(32, 16);
    else if (nb >= 64) RAC_Q8_ROW(64, 4);
    else RAC_Q8_ROW(32, 8);
#undef RAC_Q8_ROW
}

static bool q8_fast_ok(const uint8_t* w, int K) {
    return (K % (8 * kQ8Block) == 0) && ((reinterpret_cast<uintptr_t>(w) & 15) == 0);
}

hipError_t q8_rmsnorm_gemv_launch(const float* x, const float* gamma, float eps, const uint8_t* w,
                                  const float* bias, float* out, int N, int K, int act, hipStream_t s) {
    if (!q8_fast_ok(w, K)) return hipErrorInvalidValue;
    Q8Fuse fz;
    fz.gamma = gamma;
    fz.eps = eps;
    fz.rs_khinv = host_consts().rsqrt_khinv;
    q8_launch_row<true, 0>(x, w, bias, out, N, K, act, fz, s);
    return hipGetLastError();
}

hipError_t q8_decode_qkv_launch(const float* x, const float* gamma, float eps, const uint8_t* w, float* q_out,
                                int split, float* kc, float* vc, int kvw, int dh, long t_cap, const int* pos,
                                int K, hipStream_t s) {
    if (!q8_fast_ok(w, K)) return hipErrorInvalidValue;
    Q8Fuse fz;
    fz.gamma = gamma;
    fz.eps = eps;
    fz.rs_khinv = host_consts().rsqrt_khinv;
    fz.split = split;
    fz.kvw = kvw;
    fz.dh = dh;
    fz.t_cap = t_cap;
    fz.pos = pos;
    fz.kc = kc;
    fz.vc = vc;
    q8_launch_row<true, 2>(x, w, nullptr, q_out, split + 2 * kvw, K, 0, fz, s);
    return hipGetLastError();
}

hipError_t q8_decode_swiglu_launch(const float* x, const float* gamma, float eps, const uint8_t* w, float* out,
                                   int n_ff, int K, int iters, hipStream_t s) {
    if (!q8_fast_ok(w, K)) return hipErrorInvalidValue;
    Q8Fuse fz;
    fz.gamma = gamma;
    fz.eps = eps;
    fz.rs_khinv = host_consts().rsqrt_khinv;
    fz.iters = clamp_iters(iters);
    fz.khinv = host_consts().exp_khinv[fz.iters];
    q8_launch_row<true, 1>(x, w, nullptr, out, 2 * n_ff, K, 0, fz, s);
    return hipGetLastError();
}

hipError_t q8_gemv_launch(const float* x, const uint8_t* w, const float* bias, float* out, int M, int N,
                          int K, int act, hipStream_t s) {
    const bool fast = q8_fast_ok(w, K);
    if (fast && M == 1) {
        q8_launch_row<false, 0>(x, w, bias, out, N, K, act, Q8Fuse(), s);
    } else if (fast) {
        // chunks of 32 blocks, 16 rows per workgroup; rows of fewer than 32
        // blocks (K < 1024) in chunks of 8 blocks, 32 rows per workgroup
        const int nb = K / kQ8Block;
        const dim3 g16((unsigned)((N + 15) / 16)), g32((unsigned)((N + 31) / 32));
        // passes of up to 8 rows where more than 4 remain (K >= 1024): one
        // pass of the 8-row kernel (162 VGPRs, 75 KB of LDS: 2 workgroups
        // per CU) reads the weights once for them, against two 4-row passes;
        // bit-identical, M = 8: 4096x4096 20.9 -> 16.6 us, 11008x4096 35.0
        // -> 32.4, 32000x4096 79.5 -> 71.7
        for (int m0 = 0; m0 < M;) {
            const int left = M - m0;
            const float* xg = x + (long)m0 * K;
            float* og = out + (long)m0 * N;
            if (left > 4 && nb >= 32) {
                const int mm = min(8, left);
                hipLaunchKernelGGL((q8_gemv_kernel<8, 32, 16>), g16, dim3(256), 0, s, xg, w, bias, og, mm, N, K, act,
                                   Q8Fuse());
                m0 += mm;
                continue;
            }
            const int mm = min(4, left);
            m0 += mm;
            if (nb < 32) {
                if (mm > 1)
                    hipLaunchKernelGGL((q8_gemv_kernel<4, 8, 32>), g32, dim3(256), 0, s, xg, w, bias, og, mm, N, K, act, Q8Fuse());
                else
                    hipLaunchKernelGGL((q8_gemv_kernel<1, 8, 32>), g32, dim3(256), 0, s, xg, w, bias, og, mm, N, K, act, Q8Fuse());
            } else if (mm > 1) {
                hipLaunchKernelGGL((q8_gemv_kernel<4, 32, 16>), g16, dim3(256), 0, s, xg, w, bias, og, mm, N, K, act, Q8Fuse());
            } else {
                hipLaunchKernelGGL((q8_gemv_kernel<1, 32, 16>), g16, dim3(256), 0, s, xg, w, bias, og, mm, N, K, act, Q8Fuse());
            }
        }
    } else {
        const long outs = (long)M * N;
        hipLaunchKernelGGL(q8_gemv_generic_kernel, dim3((unsigned)((outs + 3) / 4)), dim3(256), 0, s, x, w,
                           bias, out, M, N, K, act);
    }
    return hipGetLastError();
}

// rac_q8_0_quantize_matrix (rac_q8_0.c:68-100): one lane per block.
__global__ __launch_bounds__(256) void q8_quantize_kernel(const float* __restrict__ src,
                                                          uint8_t* __restrict__ dst, long nblocks) {
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float* blk = src + b * kQ8Block;
    float v[kQ8Block];
#pragma unroll
    for (int i = 0; i < kQ8Block; i++) v[i] = blk[i];
    q8_quantize_block(v, dst + b * kQ8Bytes);
}

// rac_q8_0_dequantize_row (rac_q8_0.c:102-111): one lane per block.
__global__ __launch_bounds__(256) void q8_dequantize_kernel(const uint8_t* __restrict__ src,
                                                            float* __restrict__ dst, long nblocks) {
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* blk = src + b * kQ8Bytes;
    const float d = half_bits_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const int8_t* q = reinterpret_cast<const int8_t*>(blk + 2);
#pragma unroll
    for (int i = 0; i < kQ8Block; i++) dst[b * kQ8Block + i] = d * (float)q[i];
}

hipError_t q8_quantize_launch(const float* src, uint8_t* dst, long nblocks, hipStream_t s) {
    hipLaunchKernelGGL(q8_quantize_kernel, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, s, src, dst,
                       nblocks);
    return hipGetLastError();
}

hipError_t q8_dequantize_launch(const uint8_t* src, float* dst, long nblocks, hipStream_t s) {
    hipLaunchKernelGGL(q8_dequantize_kernel, dim3((unsigned)((nblocks + 255) / 256)), dim3(256), 0, s, src, dst,
                       nblocks);
    return hipGetLastError();
}

}  // namespace rac
