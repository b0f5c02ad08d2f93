// rac_gemm_skinny.hip — the RAC GEMM for products with few rows of op(A)
// (M <= 16: decode-time linears, one token or a few) or few columns
// (N <= 16: a matrix-vector product, a classifier head), all three MACs.
//
// Each output is ONE accumulator over k = 0..K-1 in order (rac_fma_iters,
// rac_kernels.hip:204-219), so such a product has only M * N serial chains.
// The block tiles of gemm_kernel give it few workgroups with most of their
// rows or columns empty (1 x 4096 x 4096 NT ran ~200 us in FAST mode and ~1
// ms in CORDIC mode n = 16; 4096 x 1 x 4096 alike).  Here the per-MAC work
// and the serial fold are separated:
//   * a workgroup owns an RB x CB block of outputs: RB = M (<= 16) rows by
//     16 columns, the grid over N (few rows), or 16 rows by CB = N (<= 16)
//     columns, the grid over M (few columns); it walks K in tiles of KT;
//   * A's RB x KT and B's KT x CB slices go global -> registers -> LDS (the
//     next tile's loads in flight during the current tile's work);
//   * the lanes compute the per-MAC terms of the tile, 4 consecutive k at a
//     time: CORDIC the rotation of (a ^ sign(b), 0) and its gain correction
//     p = R_n(.) * (1/K-hat(n)) (rac_kernels.hip:140-185; the literal chain
//     for inputs outside the strength-reduced one's range, as gemm_kernel),
//     SHIFTADD the shift-add product (rac_kernels.hip:85-122); FAST has no
//     term to prepare;
//   * lane m * CB + n folds output (m, n) over the tile's k in order:
//     fma(p, |b|, acc), acc + prod or fma(a, b, acc), exactly the MAC of
//     gemm_kernel, so every result has the same bits as there and in the
//     reference.
// Every MAC's rotation or shift-add product is still computed, per MAC.
#include <hip/hip_runtime.h>
#include "rac_act.hpp"

namespace rac {

// Where the per-MAC terms are computed.  FAST has none.  With 256 outputs
// per workgroup (one per lane) each lane computes its own MACs' terms and
// folds them at once ("own"); with fewer, every lane computes terms for the
// tile into LDS and the lanes owning outputs fold them ("shared").  k per
// tile keeps the workgroup's LDS under 64 KB.  (512-k FAST tiles on grids
// of one workgroup per CU were faster with the looped fold, 42 -> 31 us at
// 1x4096x4096; with the read-ahead fold the 256-k tile is: 32.2 -> 29.9 us,
// 4096x1x4096 31.8 -> 29.3 us, bit-identical.)
template <int MODE, int OUTS>
struct SkCfg {
    static constexpr bool kShared = MODE != kModeFast && OUTS < 256;
    static constexpr bool kOwn = MODE != kModeFast && OUTS == 256;
    static constexpr int kKT = MODE == kModeFast ? 256
                               : kOwn ? 128 : (OUTS == 16 ? 256 : (OUTS <= 64 ? 128 : 64));
    static constexpr int kRow = kKT + 4;        // LDS row stride (16 rows cover all banks)
};

// The CORDIC term of one MAC: the rotation of (a ^ sign(b), 0) times the
// gain correction, for E consecutive k; inputs outside the strength-reduced
// chain's range take the literal chain when `lit` (rac_kernels.hip:152-163).
template <int NITER, int E = 4>
__device__ __forceinline__ void sk_cordic_terms(const float* a, const float* b, float* p, int iters, float kinv,
                                                bool lit) {
#pragma unroll
    for (int e = 0; e < E; e++) p[e] = as_f(as_u(a[e]) ^ (as_u(b[e]) & 0x80000000u));
    if constexpr (NITER > 0) {
        cordic_rot_x_vec<NITER, E>(p);
#pragma unroll
        for (int e = 0; e < E; e++) p[e] = p[e] * cordic_kinv(NITER);
    } else {
#pragma unroll
        for (int e = 0; e < E; e++) p[e] = cordic_rot_x_rt(p[e], iters) * kinv;
    }
    if (lit) {
#pragma unroll
        for (int e = 0; e < E; e++)
            if (cordic_needs_literal(a[e]))
                p[e] = cordic_rot_x_literal_rt(as_f(as_u(a[e]) ^ (as_u(b[e]) & 0x80000000u)),
                                               NITER > 0 ? NITER : iters) *
                       (NITER > 0 ? cordic_kinv(NITER > 0 ? NITER : 1) : kinv);
    }
}

// Global -> registers: element (m0 + m, k) of A (row-major M x K) and
// (k, n0 + n) of op(B) for the K-tile at k0, zero outside the matrices,
// spread over lanes L0 .. L0 + NL - 1 (the others return: with L0 = 64 the
// folding wave 0 issues no loads).
template <int RB, int CB, int KT, bool TB, int L0 = 0, int NL = 256>
__device__ __forceinline__ void sk_load(const float* __restrict__ A, const float* __restrict__ B, int M, int N,
                                        int K, long m0, long n0, int k0, float* ra, float* rb) {
    if ((int)threadIdx.x < L0) return;
    const int tid = (int)threadIdx.x - L0;
#pragma unroll
    for (int r = 0; r < (RB * KT + NL - 1) / NL; r++) {
        const int idx = tid + r * NL, kk = idx % KT;
        const long gm = m0 + idx / KT, gk = (long)k0 + kk;
        ra[r] = (idx < RB * KT && gm < M && gk < K) ? A[gm * K + gk] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < (CB * KT + NL - 1) / NL; r++) {
        const int idx = tid + r * NL;
        int nn, kk;
        if constexpr (TB) { nn = idx / KT; kk = idx % KT; }      // W[n][k]: k contiguous
        else { kk = idx / CB; nn = idx % CB; }                   // B[k][n]: n contiguous
        const long gn = n0 + nn, gk = (long)k0 + kk;
        rb[r] = (idx < CB * KT && gn < N && gk < K) ? (TB ? B[gn * K + gk] : B[gk * N + gn]) : 0.0f;
    }
}

// Registers -> LDS (A as [RB][ROW], B as [CB][ROW], k contiguous) by the
// lanes that loaded them; true when this lane staged a CORDIC input outside
// the strength-reduced chain's range.
template <int MODE, int RB, int CB, int KT, int ROW, bool TB, int L0 = 0, int NL = 256>
__device__ __forceinline__ bool sk_store(float* sA, float* sB, const float* ra, const float* rb) {
    if ((int)threadIdx.x < L0) return false;
    const int tid = (int)threadIdx.x - L0;
    bool special = false;
#pragma unroll
    for (int r = 0; r < (RB * KT + NL - 1) / NL; r++) {
        const int idx = tid + r * NL;
        if (idx < RB * KT) sA[(idx / KT) * ROW + idx % KT] = ra[r];
        if constexpr (MODE == kModeCordic) special |= cordic_needs_literal(ra[r]);
    }
#pragma unroll
    for (int r = 0; r < (CB * KT + NL - 1) / NL; r++) {
        const int idx = tid + r * NL;
        if (idx < CB * KT) {
            if constexpr (TB) sB[(idx / KT) * ROW + idx % KT] = rb[r];
            else sB[(idx % CB) * ROW + idx / CB] = rb[r];
        }
    }
    return special;
}

// The tile's per-MAC terms into sP (row m * CB + n) for the outputs inside
// the matrix (m < mv, n < nv), 4 consecutive k of one (m, n) per step,
// spread over lanes L0 .. L0 + NL - 1 (the others return).
template <int MODE, int NITER, int RB, int CB, int KT, int ROW, int L0 = 0, int NL = 256>
__device__ __forceinline__ void sk_terms(const float* sA, const float* sB, float* sP, int mv, int nv, int iters,
                                         float kinv, bool lit) {
    constexpr int kQuads = RB * CB * KT / 4;
    if ((int)threadIdx.x < L0) return;
#pragma unroll 2
    for (int q = (int)threadIdx.x - L0; q < kQuads; q += NL) {
        const int kk = (q % (KT / 4)) * 4, mn = q / (KT / 4), m = mn / CB, n = mn % CB;
        if (m >= mv || n >= nv) continue;
        const float4 a4 = *reinterpret_cast<const float4*>(&sA[m * ROW + kk]);
        const float4 b4 = *reinterpret_cast<const float4*>(&sB[n * ROW + kk]);
        const float a[4] = {a4.x, a4.y, a4.z, a4.w}, b[4] = {b4.x, b4.y, b4.z, b4.w};
        float p[4];
        if constexpr (MODE == kModeCordic) {
            sk_cordic_terms<NITER>(a, b, p, iters, kinv, lit);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) p[e] = shiftadd_mul(a[e], b[e], iters);
        }
        *reinterpret_cast<float4*>(&sP[mn * ROW + kk]) = make_float4(p[0], p[1], p[2], p[3]);
    }
}

// The serial fold of output (om, on) over kn k of a tile, in order: the
// terms from sP row `prow` (SHARED), or computed here from sA row om (own
// terms; FAST: the A element itself).  Zero k-padding leaves acc as is.
template <int MODE, int NITER, int ROW, bool SHARED, bool RING>
__device__ __forceinline__ float sk_fold(const float* sA, const float* sB, const float* sP, int om, int on,
                                         int prow, int kn, float acc, int iters, float kinv, bool lit) {
    if constexpr (!SHARED && MODE == kModeCordic) {
        // own terms: 8 k per step, so 8 rotation chains interleave (the k
        // past kn are zero padding or, in a causal P V, zeros of P)
        for (int kk = 0; kk < kn; kk += 8) {
            const float4 a0 = *reinterpret_cast<const float4*>(&sA[om * ROW + kk]);
            const float4 a1 = *reinterpret_cast<const float4*>(&sA[om * ROW + kk + 4]);
            const float4 b0 = *reinterpret_cast<const float4*>(&sB[on * ROW + kk]);
            const float4 b1 = *reinterpret_cast<const float4*>(&sB[on * ROW + kk + 4]);
            const float a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            float t8[8];
            sk_cordic_terms<NITER, 8>(a, b, t8, iters, kinv, lit);
#pragma unroll
            for (int e = 0; e < 8; e++) acc = __builtin_fmaf(t8[e], __builtin_fabsf(b[e]), acc);
        }
        return acc;
    }
    if constexpr (RING && (SHARED || MODE == kModeFast)) {
        // Terms (or FAST's A elements) come from LDS, so the chain is fed by
        // reads alone.  A full tile's fold is unrolled completely and its
        // reads run D 4-k steps ahead of the FMAs through a ring of D
        // register pairs: step j folds pair j and reads pair j + D, and a
        // scheduling barrier after each step keeps that order (left to
        // itself the scheduler read one step ahead and waited on LDS every
        // 8 k; a dependent fmaf costs ~4.6 cycles on one wave).  2 D reads
        // in flight stay within the 15 the LDS counter tracks.  RING is set
        // where it measured faster (sk_block): FAST blocks of at most 64
        // outputs, and larger ones on grids of at most two workgroups per CU
        // (the ring's VGPRs cost a wave per SIMD on wider ones), and the
        // CORDIC pipeline on 512 lanes or with 64-output blocks.
        constexpr int KT = ROW - 4, D = 6;
        if (kn == KT) {
            const float* rowb = &sB[on * ROW];
            const float* rowt = SHARED ? &sP[prow * ROW] : &sA[om * ROW];
            float4 rb[D], rt[D];
#pragma unroll
            for (int j = 0; j < D; j++) {
                rb[j] = *reinterpret_cast<const float4*>(rowb + 4 * j);
                rt[j] = *reinterpret_cast<const float4*>(rowt + 4 * j);
            }
#pragma unroll
            for (int j = 0; j < KT / 4; j++) {
                const float b[4] = {rb[j % D].x, rb[j % D].y, rb[j % D].z, rb[j % D].w};
                const float t[4] = {rt[j % D].x, rt[j % D].y, rt[j % D].z, rt[j % D].w};
                if (j + D < KT / 4) {
                    rb[j % D] = *reinterpret_cast<const float4*>(rowb + 4 * (j + D));
                    rt[j % D] = *reinterpret_cast<const float4*>(rowt + 4 * (j + D));
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if constexpr (MODE == kModeCordic) acc = __builtin_fmaf(t[e], __builtin_fabsf(b[e]), acc);
                    else if constexpr (MODE == kModeShiftAdd) acc = acc + t[e];
                    else acc = __builtin_fmaf(t[e], b[e], acc);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            return acc;
        }
    }
    // a partial tile (and own SHIFTADD terms): 4-k steps, unrolled so the
    // LDS reads of 32 k run ahead of the dependent chain of FMAs
#pragma unroll 8
    for (int kk = 0; kk < kn; kk += 4) {
        const float4 b4 = *reinterpret_cast<const float4*>(&sB[on * ROW + kk]);
        const float b[4] = {b4.x, b4.y, b4.z, b4.w};
        float t4[4];
        if constexpr (SHARED) {
            const float4 p4 = *reinterpret_cast<const float4*>(&sP[prow * ROW + kk]);
            t4[0] = p4.x; t4[1] = p4.y; t4[2] = p4.z; t4[3] = p4.w;
        } else {
            const float4 a4 = *reinterpret_cast<const float4*>(&sA[om * ROW + kk]);
            const float a[4] = {a4.x, a4.y, a4.z, a4.w};
            if constexpr (MODE == kModeCordic) {
                sk_cordic_terms<NITER>(a, b, t4, iters, kinv, lit);
            } else if constexpr (MODE == kModeShiftAdd) {
#pragma unroll
                for (int e = 0; e < 4; e++) t4[e] = shiftadd_mul(a[e], b[e], iters);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) t4[e] = a[e];
            }
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if constexpr (MODE == kModeCordic) acc = __builtin_fmaf(t4[e], __builtin_fabsf(b[e]), acc);
            else if constexpr (MODE == kModeShiftAdd) acc = acc + t4[e];
            else acc = __builtin_fmaf(t4[e], b[e], acc);
        }
    }
    return acc;
}

// alpha / beta, bias and activation of output (gm, gn), as gemm_kernel's
template <bool FUSED>
__device__ __forceinline__ void sk_epilogue(float* C, int N, long gm, long gn, float acc, float alpha, float beta,
                                            const GemmEpilogue& ep, int iters) {
    float* cp = C + gm * N + gn;
    // rac_kernels.hip:267-272
    float v = (beta != 0.0f) ? __builtin_fmaf(alpha, acc, beta * *cp) : alpha * acc;
    if constexpr (FUSED) {
        // rac_torch.cu:770-775
        if (ep.bias) v = v + ep.bias[gn];
        if (ep.pre) ep.pre[gm * N + gn] = v;
        v = act_rt(v, ep.act, iters, ep.khinv);
    }
    *cp = v;
}

// The block of outputs a workgroup owns: rows m0 .. m0 + mv - 1, columns
// n0 .. n0 + nv - 1; the causal P V limit of those rows (rows past a query
// position's key range are exactly 0 in P and, with every v finite,
// fma(0, v, acc) == acc: acc starts at +0 and never becomes -0).
template <int RB, int CB, bool FEWCOL>
struct SkBlock {
    long m0, n0;
    int mv, nv, kend;
    __device__ SkBlock(int M, int N, int K, const int* k_causal, int row0) {
        m0 = FEWCOL ? (long)blockIdx.x * RB : 0;
        n0 = FEWCOL ? 0 : (long)blockIdx.x * CB;
        mv = (int)min((long)RB, (long)M - m0);
        nv = (int)min((long)CB, (long)N - n0);
        kend = K;
        if (k_causal && *k_causal == 1) kend = (int)min((long)K, (long)row0 + m0 + mv);
    }
};

template <int MODE, int NITER, bool TB, bool FUSED, int RB, int CB, bool FEWCOL, bool RING>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    float alpha, float beta, int iters, float kinv, long sa, long sb, long sc, GemmEpilogue ep,
    const int* k_causal, int exact_specials, int row0)
{
    using Cfg = SkCfg<MODE, RB * CB>;
    constexpr int KT = Cfg::kKT, ROW = Cfg::kRow;
    constexpr bool kShared = Cfg::kShared;
    __shared__ __attribute__((aligned(16))) float sA[RB * ROW];
    __shared__ __attribute__((aligned(16))) float sB[CB * ROW];
    __shared__ __attribute__((aligned(16))) float sP[kShared ? RB * CB * ROW : 4];
    // CORDIC: lit[t & 1] is set when tile t's A slice holds an input outside
    // the strength-reduced chain's range; two flags, so the next tile's is
    // cleared while no lane reads it
    __shared__ int lit[2];

    const int tid = threadIdx.x;
    A += (long)blockIdx.z * sa;
    B += (long)blockIdx.z * sb;
    C += (long)blockIdx.z * sc;
    const SkBlock<RB, CB, FEWCOL> blk(M, N, K, k_causal, row0);
    if (tid == 0) lit[0] = lit[1] = 0;               // ordered before any set by the loop's first barrier

    const int om = tid / CB, on = tid % CB;           // output owned by lanes tid < RB * CB
    const bool owner = tid < RB * CB && om < blk.mv && on < blk.nv;
    // FAST with one row (or column) of 16 outputs: wave 0 only folds, and
    // waves 1-3 load and stage the tiles, so the next tile's loads are
    // issued while wave 0 folds this one (per tile at 1x4096x4096 wave 0
    // spent ~950 of 4300 cycles issuing its share of the loads before its
    // fold).  Measured, bit-identical: 1x4096x4096 29.9 -> 29.3 us,
    // 1x4096x11008 72.5 -> 66.6, 4096x1x4096 29.4 -> 28.4; with 4 rows it
    // lost (30.3 -> 31.8 us), and the CORDIC pipeline, whose waves 1-3
    // compute the terms, lost too (1x4096x4096 54.3 -> 63.7 us).
    constexpr int L0 = (MODE == kModeFast && RB * CB <= 16) ? 64 : 0, NL = 256 - L0;
    float ra[(RB * KT + NL - 1) / NL], rb[(CB * KT + NL - 1) / NL];
    float acc = 0.0f;
    sk_load<RB, CB, KT, TB, L0, NL>(A, B, M, N, K, blk.m0, blk.n0, 0, ra, rb);
    for (int k0 = 0, t = 0; k0 < blk.kend; k0 += KT, t++) {
        __syncthreads();                                // previous tile's fold done with LDS
        if (sk_store<MODE, RB, CB, KT, ROW, TB, L0, NL>(sA, sB, ra, rb) && exact_specials) lit[t & 1] = 1;
        __syncthreads();
        if (k0 + KT < blk.kend) sk_load<RB, CB, KT, TB, L0, NL>(A, B, M, N, K, blk.m0, blk.n0, k0 + KT, ra, rb);
        const bool lit_tile = MODE == kModeCordic && lit[t & 1] != 0;
        if constexpr (kShared) {
            sk_terms<MODE, NITER, RB, CB, KT, ROW>(sA, sB, sP, blk.mv, blk.nv, iters, kinv, lit_tile);
            __syncthreads();
        }
        if (tid == 0) lit[(t + 1) & 1] = 0;            // tile t+1's flag: set after the loop-top barrier
        if (owner)
            acc = sk_fold<MODE, NITER, ROW, kShared, RING>(sA, sB, sP, om, on, tid, min(KT, blk.kend - k0), acc, iters,
                                                     kinv, lit_tile);
    }
    if (owner) sk_epilogue<FUSED>(C, N, blk.m0 + om, blk.n0 + on, acc, alpha, beta, ep, iters);
}

// The shared terms pipelined (CORDIC, <= 64 outputs): B slices and terms
// in two LDS buffers, so waves 1-3 compute tile t+1's terms while wave 0's
// output lanes fold tile t (in the form above the fold, a serial chain of
// KT dependent operations per output, waited for the terms and the terms
// for the fold).  Tile t+1's A slice has one buffer: only the terms read it.
// The prologue's terms of tile 0 use every lane.
// NT = 512 (grids of at most one workgroup per CU): 7 waves compute the
// terms and also load and stage the tiles, wave 0 only folds (read-ahead
// fold); 256-k tiles for 16 outputs, 128-k for 64.  128 outputs (8 x 16
// blocks) fold on waves 0-1, their terms on waves 2-7, in 64-k tiles
// (8x4096x4096 175.8 -> 160.4 us against 8 x 8 blocks on 256 lanes,
// 2048x10x4096 243.6 -> 179.8).  With 256 lanes a tile
// of 1x4096x4096 took ~4300 cycles, ~3200 of them the three term waves
// (one wave per SIMD issues slowly), while the fold waited ~1300.
// Measured, bit-identical, n = 16: 1x4096x4096 54.0 -> 36.4 us,
// 1x4096x11008 139.4 -> 86.7, 4096x1x4096 56.6 -> 35.5, 4x4096x4096 158.5
// -> 85.3.
template <int MODE, int NITER, bool TB, bool FUSED, int RB, int CB, bool FEWCOL, int NT>
__global__ __launch_bounds__(NT) void gemm_skinny_pipe_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    float alpha, float beta, int iters, float kinv, long sa, long sb, long sc, GemmEpilogue ep,
    const int* k_causal, int exact_specials, int row0)
{
    static_assert(NT == 256 || NT == 512, "block size");
    static_assert(RB * CB <= (NT == 512 ? 128 : 64), "the fold lanes are wave 0 (and 1)");
    constexpr int FL = RB * CB <= 64 ? 64 : 128;              // lanes of the folding waves
    constexpr int KT = NT == 512 ? (RB * CB == 16 ? 256 : (RB * CB == 64 ? 128 : 64)) : (RB * CB == 16 ? 128 : 64);
    constexpr int ROW = KT + 4;
    constexpr int L0 = NT == 512 ? FL : 0, NL = NT - L0;      // the loading lanes
    constexpr bool kRing = NT == 512 || RB * CB == 64;
    __shared__ __attribute__((aligned(16))) float sA[RB * ROW];
    __shared__ __attribute__((aligned(16))) float sB[2][CB * ROW];
    __shared__ __attribute__((aligned(16))) float sP[2][RB * CB * ROW];
    // lit[t & 1]: tile t's A slice holds an input outside the strength-
    // reduced chain's range (set when the tile is staged, read by its terms,
    // cleared two tiles later)
    __shared__ int lit[2];

    const int tid = threadIdx.x;
    A += (long)blockIdx.z * sa;
    B += (long)blockIdx.z * sb;
    C += (long)blockIdx.z * sc;
    const SkBlock<RB, CB, FEWCOL> blk(M, N, K, k_causal, row0);
    if (tid == 0) lit[0] = lit[1] = 0;

    const int om = tid / CB, on = tid % CB;
    const bool owner = tid < RB * CB && om < blk.mv && on < blk.nv;
    float ra[(RB * KT + NL - 1) / NL], rb[(CB * KT + NL - 1) / NL];
    float acc = 0.0f;
    // prologue: tile 0 staged and its terms computed, tile 1 in flight
    sk_load<RB, CB, KT, TB, L0, NL>(A, B, M, N, K, blk.m0, blk.n0, 0, ra, rb);
    __syncthreads();                                     // flags cleared
    if (sk_store<MODE, RB, CB, KT, ROW, TB, L0, NL>(sA, sB[0], ra, rb) && exact_specials) lit[0] = 1;
    __syncthreads();
    if (KT < blk.kend) sk_load<RB, CB, KT, TB, L0, NL>(A, B, M, N, K, blk.m0, blk.n0, KT, ra, rb);
    sk_terms<MODE, NITER, RB, CB, KT, ROW, 0, NT>(sA, sB[0], sP[0], blk.mv, blk.nv, iters, kinv,
                                                  MODE == kModeCordic && lit[0] != 0);
    for (int k0 = 0, t = 0; k0 < blk.kend; k0 += KT, t++) {
        const int cur = t & 1, nxt = cur ^ 1;
        const bool more = k0 + KT < blk.kend;
        __syncthreads();                                 // tile t's terms written; tile t-1 folded
        if (more && sk_store<MODE, RB, CB, KT, ROW, TB, L0, NL>(sA, sB[nxt], ra, rb) && exact_specials) lit[nxt] = 1;
        __syncthreads();                                 // tile t+1 staged
        if (k0 + 2 * KT < blk.kend)
            sk_load<RB, CB, KT, TB, L0, NL>(A, B, M, N, K, blk.m0, blk.n0, k0 + 2 * KT, ra, rb);
        if (more)
            sk_terms<MODE, NITER, RB, CB, KT, ROW, FL, NT - FL>(sA, sB[nxt], sP[nxt], blk.mv, blk.nv, iters, kinv,
                                                                MODE == kModeCordic && lit[nxt] != 0);
        if (tid == 0) lit[cur] = 0;                      // tile t+2's flag (tile t's was read a phase ago)
        if (owner)
            acc = sk_fold<MODE, NITER, ROW, true, kRing>(sA, sB[cur], sP[cur], om, on, tid, min(KT, blk.kend - k0),
                                                         acc, iters, kinv, false);
    }
    if (owner) sk_epilogue<FUSED>(C, N, blk.m0 + om, blk.n0 + on, acc, alpha, beta, ep, iters);
}

template <int MODE, int NITER, bool TB, bool FUSED, int RB, int CB, bool FEWCOL, bool PIPE,
          bool RING = (MODE == kModeFast && RB * CB <= 64), int NT = 256>
static hipError_t sk_launch(const SkinnyArgs& g, hipStream_t s) {
    const unsigned wgs = FEWCOL ? (unsigned)((g.M + RB - 1) / RB) : (unsigned)((g.N + CB - 1) / CB);
    const dim3 grid(wgs, 1, (unsigned)g.batch);
    if constexpr (PIPE) {
        hipLaunchKernelGGL((gemm_skinny_pipe_kernel<MODE, NITER, TB, FUSED, RB, CB, FEWCOL, NT>), grid, dim3(NT), 0, s,
                           g.A, g.B, g.C, g.M, g.N, g.K, g.alpha, g.beta, g.iters, cordic_kinv(g.iters), g.sa, g.sb,
                           g.sc, g.ep, g.k_causal, g.exact_specials, g.row0);
    } else {
        hipLaunchKernelGGL((gemm_skinny_kernel<MODE, NITER, TB, FUSED, RB, CB, FEWCOL, RING>), grid, dim3(256), 0, s,
                           g.A, g.B, g.C, g.M, g.N, g.K, g.alpha, g.beta, g.iters, cordic_kinv(g.iters), g.sa, g.sb,
                           g.sc, g.ep, g.k_causal, g.exact_specials, g.row0);
    }
    return hipGetLastError();
}

// One output block shape (RB x CB): CORDIC takes the pipelined terms (<= 64
// outputs); SHIFTADD's
// terms (a shift-add product each) outweigh its fold and keep all four
// waves (pipelined on three: 1x4096x4096 213 -> 297 us).  The read-ahead
// fold (RING), measured against the looped one, bit-identical: FAST
// 1x11008x4096 50.7 -> 43.8 us, 8x4096x4096 34.0 -> 32.0, 16x4096x4096
// 38.6 -> 36.4, 2048x10x4096 55.2 -> 43.2; CORDIC n = 16 4x4096x4096 175.7
// -> 158.3.  With 2.7 workgroups per CU its VGPRs cost a wave per SIMD
// (FAST 16x11008x4096 77.7 -> 83.2 us), and one-row CORDIC and SHIFTADD
// gained nothing (CORDIC 1x4096x4096 54.3 -> 55.1, SHIFTADD 1x11008x4096
// 271.7 -> 279.7 us), so they keep the loop.
template <int MODE, int NITER, bool TB, bool FUSED, int RB, int CB, bool FEWCOL>
static hipError_t sk_block(const SkinnyArgs& g, hipStream_t s) {
    const long wgs = (FEWCOL ? (long)((g.M + RB - 1) / RB) : (long)((g.N + CB - 1) / CB)) * g.batch;
    if constexpr (MODE == kModeCordic && RB * CB == 128) {
        if (wgs <= device_cus()) return sk_launch<MODE, NITER, TB, FUSED, RB, CB, FEWCOL, true, false, 512>(g, s);
    }
    if constexpr (RB * CB <= 64) {
        if constexpr (MODE == kModeCordic) {
            if (wgs <= device_cus()) return sk_launch<MODE, NITER, TB, FUSED, RB, CB, FEWCOL, true, false, 512>(g, s);
            return sk_launch<MODE, NITER, TB, FUSED, RB, CB, FEWCOL, true>(g, s);
        }
    } else if constexpr (MODE == kModeFast) {
        if (wgs <= 2 * device_cus()) return sk_launch<MODE, NITER, TB, FUSED, RB, CB, FEWCOL, false, true>(g, s);
    }
    return sk_launch<MODE, NITER, TB, FUSED, RB, CB, FEWCOL, false>(g, s);
}

// The output block.  Few rows: RB = M rounded up (1, 4, 8, 16) by 16
// columns; few columns: 16 rows by CB = N rounded up.  With 5-16 rows (or
// columns), when the 16-wide grid would leave at most one workgroup per CU,
// half as wide blocks double the workgroups (two waves per SIMD instead of
// one): measured, bit-identical, 8x4096x4096 CORDIC n = 16 218 -> 177 us,
// 16x4096x4096 330 -> 225 us, SHIFTADD 1.54 -> 0.85 ms and 2.97 -> 1.69
// ms, FAST 16 rows 52 -> 37 us; on wider grids (N = 11008) the narrow
// blocks lost 6-29% (CORDIC, FAST), and FAST lost with 8 rows everywhere.
// SHIFTADD, bound by its terms, takes them at 9-16 rows on any grid.  CORDIC
// with 5-8 rows (or columns) now keeps 8 x 16 blocks on such grids, which
// the 512-lane pipeline runs (8 x 8 blocks on 256 lanes: 175.8 us, 8 x 16
// on 512: 160.4 us at 8x4096x4096 n = 16).  One
// FAST row (or column) takes 8-wide blocks on such grids too: its fold is
// one wave per workgroup, so twice the workgroups fold on twice the SIMDs
// (1x4096x4096 29.1 -> 26.4 us, 1x4096x11008 66.7 -> 62.2; on the wider
// 1x11008x4096 grid 43.9 -> 51.9, so that keeps 16).
template <int MODE, int NITER, bool TB, bool FUSED>
static hipError_t sk_shape(const SkinnyArgs& g, hipStream_t s) {
    const long cus = device_cus();
    if (g.M <= kSkinnyMaxRows) {                         // few rows, the grid over N
        const bool one_per_cu = (long)((g.N + 15) / 16) * g.batch <= cus;
        if (g.M == 1) {
            if (MODE == kModeFast && one_per_cu) return sk_block<MODE, NITER, TB, FUSED, 1, 8, false>(g, s);
            return sk_block<MODE, NITER, TB, FUSED, 1, 16, false>(g, s);
        }
        if (g.M <= 4) return sk_block<MODE, NITER, TB, FUSED, 4, 16, false>(g, s);
        if (g.M <= 8) {
            // CORDIC keeps 8 x 16 blocks there: the 512-lane pipeline takes them
            if (MODE == kModeShiftAdd && one_per_cu) return sk_block<MODE, NITER, TB, FUSED, 8, 8, false>(g, s);
            return sk_block<MODE, NITER, TB, FUSED, 8, 16, false>(g, s);
        }
        if (MODE == kModeShiftAdd || one_per_cu) return sk_block<MODE, NITER, TB, FUSED, 16, 8, false>(g, s);
        return sk_block<MODE, NITER, TB, FUSED, 16, 16, false>(g, s);
    }
    // few columns, the grid over M
    const bool one_per_cu = (long)((g.M + 15) / 16) * g.batch <= cus;
    if (g.N == 1) {
        if (MODE == kModeFast && one_per_cu) return sk_block<MODE, NITER, TB, FUSED, 8, 1, true>(g, s);
        return sk_block<MODE, NITER, TB, FUSED, 16, 1, true>(g, s);
    }
    if (g.N <= 4) return sk_block<MODE, NITER, TB, FUSED, 16, 4, true>(g, s);
    if (g.N <= 8) {
        if (MODE != kModeFast && one_per_cu) return sk_block<MODE, NITER, TB, FUSED, 8, 8, true>(g, s);
        return sk_block<MODE, NITER, TB, FUSED, 16, 8, true>(g, s);
    }
    if (MODE == kModeShiftAdd || one_per_cu) return sk_block<MODE, NITER, TB, FUSED, 8, 16, true>(g, s);
    return sk_block<MODE, NITER, TB, FUSED, 16, 16, true>(g, s);
}

template <int MODE, int NITER>
static hipError_t sk_layout(const SkinnyArgs& g, hipStream_t s) {
    if (g.fused) return sk_shape<MODE, NITER, true, true>(g, s);
    if (g.tb) return sk_shape<MODE, NITER, true, false>(g, s);
    return sk_shape<MODE, NITER, false, false>(g, s);
}

hipError_t gemm_skinny_launch(const SkinnyArgs& g, int mode, hipStream_t s) {
    if (mode == kModeFast) return sk_layout<kModeFast, 0>(g, s);
    if (mode == kModeShiftAdd) return sk_layout<kModeShiftAdd, 0>(g, s);
    switch (g.iters) {
        case 8: return sk_layout<kModeCordic, 8>(g, s);
        case 16: return sk_layout<kModeCordic, 16>(g, s);
        case 24: return sk_layout<kModeCordic, 24>(g, s);
        default: return sk_layout<kModeCordic, 0>(g, s);
    }
}

}  // namespace rac
