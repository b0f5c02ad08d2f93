// rac_gemm.hip — rotate-project-accumulate GEMM for gfx950 (VALU; FAST mode
// on the FP32 matrix cores where the launch is large enough).
//
// C[M,N] = alpha * op(A) @ op(B) (+ beta * C), row-major, with the MAC of
// rac_fma_iters (rac_kernels.hip:204-219):
//   FAST     fmaf(a ^ sign(b), |b|, acc)                  == fmaf(a, b, acc)
//   CORDIC   n circular micro-rotations of (a ^ sign(b), 0), x * 1/K-hat(n),
//            projected on |b| and accumulated               (rac_math.hpp)
//   SHIFTADD acc + integer shift-add product of the top n mantissa bits of b
// op(A) = A or A^T (A stored [K,M], the TN launcher); op(B) = B or B^T
// (B stored [N,K], the NT launcher).  Each output keeps ONE accumulator over
// k = 0..K-1 in order, like every reference tile shape, so results do not
// depend on the tiling; out-of-range operands are zero-padded (a zero MAC
// leaves acc unchanged).
//
// Design: CORDIC mode costs ~2n VALU lane-ops per MAC, so the kernel is
// VALU-bound by two orders of magnitude over LDS and HBM traffic.  A 64x64
// block tile (4x4 outputs per lane, 256 lanes = 4 wave64) staged through LDS
// with BK = 16 keeps 16 independent MAC chains per lane for latency hiding
// and reads only 2 ds_read_b128 per 16 MACs; the rotations of those MACs
// advance step-major, so independent FMA chains interleave in each wave's
// instruction stream.  FAST mode (1 FMA per MAC) runs on the matrix cores
// (gemm_mfma_fast_kernel, below) when it has enough 128x128 blocks and
// K >= 128; otherwise on VALU tiles of 8x8 or 16x8 per lane (8x8 split in
// 4x4 groups 64 apart, conflict-free LDS reads), the k loop unrolled by 2,
// bound by LDS bandwidth (128 B/clk/CU) as much as by the FMA rate.
// Launches with fewer than 1024 block tiles step down to 64x64, then 32x32
// (2x2 per lane; CORDIC and SHIFTADD below 2 blocks of 64x64 per CU) so
// every SIMD holds several waves.  The next K-tile is
// prefetched into registers while the current one is computed.
#include <hip/hip_runtime.h>
#include <atomic>
#include "rac_act.hpp"

namespace rac {

// CORDIC mode: rotations of kGroupRows tile rows (x TN columns) advance
// step-major (8 interleaved chains in the 4x4 register tile).
constexpr int kGroupRows = 2;
// Fewer block tiles than this (4 per CU) leave SIMDs with one wave or none;
// such launches step down to a smaller tile (64x64, then 32x32; the CORDIC
// and SHIFTADD 64x64 tile down to 2 blocks per CU).
constexpr long kMinTiles = 1024;

// Offset of a lane's i-th row (or column) inside the block tile, for the
// lane's 16-way index t.  Register tiles of 4k are split into k groups of 4
// spaced 64 apart, so a wave's float4 LDS reads of one group cover 256
// contiguous bytes (no bank conflicts for the 8x8 tile); 2 and 4 are
// contiguous.  Only the output a lane owns changes, never its arithmetic.
template <int TT>
__device__ __forceinline__ int lane_off(int t, int i) {
    if constexpr (TT % 4 == 0) return (i >> 2) * 64 + t * 4 + (i & 3);
    else return t * TT + i;
}

// FAST MACs are one FMA each: the k loop is unrolled by this so the next
// k-step's LDS reads issue under the current step's FMAs.
constexpr int kFastKUnroll = 2;

template <int MODE, int NITER, bool TA, bool TB, int TM, int TN>
struct GemmCfg {
    static constexpr int kThreads = 256;
    static constexpr int kBM = 16 * TM;
    static constexpr int kBN = 16 * TN;
    static constexpr int kBK = 16;
    static constexpr int kPad = 4;
    static constexpr int kALoads = kBM * kBK / kThreads;
    static constexpr int kBLoads = kBN * kBK / kThreads;
};

template <int MODE, int NITER, bool LIT = false>
__device__ __forceinline__ float mac(float a, float b, uint32_t bsign, float acc,
                                     int iters, float kinv) {
    if constexpr (MODE == kModeFast) {
        return __builtin_fmaf(a, b, acc);
    } else if constexpr (MODE == kModeCordic && LIT) {
        // the rotation as rac_kernels.hip:152-163 writes it, for inputs
        // outside the strength-reduced chain's range (cordic_needs_literal)
        const float x0 = as_f(as_u(a) ^ bsign);
        const float xr = cordic_rot_x_literal_rt(x0, NITER > 0 ? NITER : iters);
        return __builtin_fmaf(xr * kinv, __builtin_fabsf(b), acc);
    } else if constexpr (MODE == kModeCordic) {
        if constexpr (NITER > 0) {
            return mac_cordic<NITER>(a, b, bsign, acc);
        } else {
            const float x0 = as_f(as_u(a) ^ bsign);
            const float xr = cordic_rot_x_rt(x0, iters);
            return __builtin_fmaf(xr * kinv, __builtin_fabsf(b), acc);
        }
    } else {
        return acc + shiftadd_mul(a, b, iters);
    }
}

// Column tiles of row tile r in a causal score trapezoid (query rows
// row0 + r*BM .. row0 + r*BM + BM - 1, keys 0 .. N-1): those holding a key
// position not past the row tile's last query position.
__host__ __device__ __forceinline__ int trap_cols(int row0, int r, int BM, int BN, int N) {
    const long last = (long)row0 + (long)(r + 1) * BM - 1;
    const long c = last / BN + 1;
    const long ntn = (N + BN - 1) / BN;
    return (int)(c < ntn ? c : ntn);
}

template <int MODE, int NITER, bool TA, bool TB, int TM, int TN, bool FUSED, int SCHED>
__global__ __launch_bounds__(256) void gemm_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
    int M, int N, int K, float alpha, float beta, int iters, float kinv, long sa, long sb, long sc,
    GemmEpilogue ep, const int* k_causal, int exact_specials, int row0)
{
    using Cfg = GemmCfg<MODE, NITER, TA, TB, TM, TN>;
    constexpr int BM = Cfg::kBM, BN = Cfg::kBN, BK = Cfg::kBK, PAD = Cfg::kPad;
    // Tile schedule.  0: tile (blockIdx.y, blockIdx.x).  1 (causal attention
    // scores, square, BM == BN): only tiles on or below the diagonal, which
    // the softmax does not overwrite with -inf; workgroup (x, p) takes row p
    // col x for x <= p, else row nt-1-p col x-p-1, so every workgroup has one
    // tile and rows p and nt-1-p share a column of the grid (grid nt+1 x
    // ceil(nt/2)).  2 (causal P V): workgroup p computes row tiles p and
    // nt-1-p, whose K ranges (below) sum to a constant.  3 (causal attention
    // scores of query rows row0.. row0+M-1 against keys 0..N-1): only the
    // tiles on or below the diagonal, numbered row by row (row tile r has
    // trap_cols(r) of them), one workgroup each; consecutive workgroups go to
    // consecutive XCDs, so the trapezoid's work spreads over all of them (a
    // rectangular grid with the upper tiles skipped leaves the live ones on
    // a few XCDs).
    int tm = blockIdx.y, tn = blockIdx.x, tm2 = -1;
    if constexpr (SCHED == 3) {
        int l = blockIdx.x;
        tm = 0;
        for (;;) {
            const int c = trap_cols(row0, tm, BM, BN, N);
            if (l < c) break;
            l -= c;
            tm++;
        }
        tn = l;
    }
    if constexpr (SCHED == 1) {
        const int nt = (M + BM - 1) / BM, p = blockIdx.y, x = blockIdx.x;
        if (x > p) {
            tm = nt - 1 - p;
            tn = x - p - 1;
            if (tm == p) return;     // middle row of an odd tile count: covered by x <= p
        }
    } else if constexpr (SCHED == 2) {
        const int nt = (M + BM - 1) / BM, p = blockIdx.y;
        if (nt - 1 - p != p) tm2 = nt - 1 - p;
    }
    const long m0a = (long)tm * BM, m0b = tm2 < 0 ? -1L : (long)tm2 * BM, n0 = (long)tn * BN;
    A += (long)blockIdx.z * sa;
    B += (long)blockIdx.z * sb;
    C += (long)blockIdx.z * sc;
    __shared__ __attribute__((aligned(16))) float sA[BK][BM + PAD];
    __shared__ __attribute__((aligned(16))) float sB[BK][BN + PAD];
    // CORDIC mode: lit_pass[pass] is set when some A element of the output
    // tile's row panel lies outside the strength-reduced chain's range
    // (cordic_needs_literal); the tile is then recomputed on the literal
    // chain.  One flag per pass, so no flag is cleared while being read.
    __shared__ int lit_pass[2];

    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;
    if constexpr (MODE == kModeCordic) {
        if (tid == 0) lit_pass[0] = lit_pass[1] = 0;   // ordered before any set by the K loop's barriers
    }

    constexpr int kPasses = SCHED == 2 ? 2 : 1;
    for (int pass = 0; pass < kPasses; pass++) {
        const long m0 = pass ? m0b : m0a;
        if (m0 < 0) break;

        float acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = 0.0f;

        float ra[Cfg::kALoads], rb[Cfg::kBLoads];
        // Range of the A elements this lane staged, as |a| bit patterns: the
        // largest, and the smallest minus one (unsigned, so +-0 never counts).
        uint32_t a_hi = 0u, a_lo_m1 = 0xffffffffu;

        // Global -> register staging of one K-tile; element (m, k) of op(A) and
        // (k, n) of op(B), zero outside the matrix.  Index order is chosen so
        // consecutive lanes read consecutive addresses.
        auto load_tile = [&](int k0) {
#pragma unroll
            for (int r = 0; r < Cfg::kALoads; r++) {
                const int idx = tid + r * 256;
                int mm, kk;
                if constexpr (TA) { kk = idx / BM; mm = idx % BM; }
                else { mm = idx / BK; kk = idx % BK; }
                const long gm = m0 + mm, gk = (long)k0 + kk;
                float v = 0.0f;
                if (gm < M && gk < K) v = TA ? A[gk * M + gm] : A[gm * K + gk];
                ra[r] = v;
            }
#pragma unroll
            for (int r = 0; r < Cfg::kBLoads; r++) {
                const int idx = tid + r * 256;
                int nn, kk;
                if constexpr (TB) { nn = idx / BK; kk = idx % BK; }
                else { kk = idx / BN; nn = idx % BN; }
                const long gn = n0 + nn, gk = (long)k0 + kk;
                float v = 0.0f;
                if (gn < N && gk < K) v = TB ? B[gn * K + gk] : B[gk * N + gn];
                rb[r] = v;
            }
        };
        auto store_tile = [&]() {
#pragma unroll
            for (int r = 0; r < Cfg::kALoads; r++) {
                const int idx = tid + r * 256;
                int mm, kk;
                if constexpr (TA) { kk = idx / BM; mm = idx % BM; }
                else { mm = idx / BK; kk = idx % BK; }
                sA[kk][mm] = ra[r];
                if constexpr (MODE == kModeCordic) {
                    const uint32_t u = as_u(ra[r]) & 0x7fffffffu;
                    a_hi = max(a_hi, u);
                    a_lo_m1 = min(a_lo_m1, u - 1u);
                }
            }
#pragma unroll
            for (int r = 0; r < Cfg::kBLoads; r++) {
                const int idx = tid + r * 256;
                int nn, kk;
                if constexpr (TB) { nn = idx / BK; kk = idx % BK; }
                else { kk = idx / BN; nn = idx % BN; }
                sB[kk][nn] = rb[r];
            }
        };

        // Causal P V: row t of P is exactly 0 beyond column t, and with every v
        // finite (*k_causal == 1, checked on the device) fma(0, v, acc) == acc
        // (acc starts at +0 and can never become -0), so the K loop stops after
        // the tile's last row (query position row0 + m0 + BM - 1).
        int kend = K;
        if (k_causal && *k_causal == 1) kend = (int)min((long)K, (long)row0 + m0 + BM);
        load_tile(0);
        for (int k0 = 0; k0 < kend; k0 += BK) {
            __syncthreads();            // previous tile fully consumed
            store_tile();
            __syncthreads();
            if (k0 + BK < kend) load_tile(k0 + BK);   // prefetch overlaps the MACs
            // CORDIC steps are long VALU chains and stay rolled in the plain
            // 4x4 schedules; the 2x2 register tile (4 rotations per k-step,
            // too few independent chains to cover each step's LDS reads)
            // and the square causal attention schedules take two k-steps
            // per trip (measured: 1024^3 0.616 -> 0.542 ms, the attention
            // core with P kept 9.75 -> 9.36 ms; the 4096^3 NN launch 1%
            // slower, so it keeps one).  The accumulation order is unchanged.
            constexpr int KU = (MODE == kModeFast) ? kFastKUnroll : ((TM * TN <= 4 || SCHED == 1 || SCHED == 2) ? 2 : 1);
#pragma unroll 1
            for (int kb = 0; kb < BK; kb += KU)
#pragma unroll
            for (int ku = 0; ku < KU; ku++) {
                const int kk = kb + ku;
                float a[TM], b[TN];
                uint32_t bs[TN];
                if constexpr (TM % 4 == 0) {
#pragma unroll
                    for (int i = 0; i < TM; i += 4) {
                        const float4 v = *reinterpret_cast<const float4*>(&sA[kk][lane_off<TM>(ty, i)]);
                        a[i] = v.x; a[i + 1] = v.y; a[i + 2] = v.z; a[i + 3] = v.w;
                    }
                } else {
                    static_assert(TM == 2, "register tile");
                    const float2 v = *reinterpret_cast<const float2*>(&sA[kk][ty * TM]);
                    a[0] = v.x; a[1] = v.y;
                }
                if constexpr (TN % 4 == 0) {
#pragma unroll
                    for (int j = 0; j < TN; j += 4) {
                        const float4 v = *reinterpret_cast<const float4*>(&sB[kk][lane_off<TN>(tx, j)]);
                        b[j] = v.x; b[j + 1] = v.y; b[j + 2] = v.z; b[j + 3] = v.w;
                    }
                } else {
                    static_assert(TN == 2, "register tile");
                    const float2 v = *reinterpret_cast<const float2*>(&sB[kk][tx * TN]);
                    b[0] = v.x; b[1] = v.y;
                }
#pragma unroll
                for (int j = 0; j < TN; j++) bs[j] = as_u(b[j]) & 0x80000000u;
                if constexpr (MODE == kModeCordic && NITER > 0) {
                    // the rotations of kGroupRows x TN MACs advance step-major
                    // (independent chains interleave; same bits as mac<>)
                    constexpr int G = kGroupRows < TM ? kGroupRows : TM;
#pragma unroll
                    for (int i0 = 0; i0 < TM; i0 += G) {
                        float xr[G * TN];
#pragma unroll
                        for (int gi = 0; gi < G; gi++)
#pragma unroll
                            for (int j = 0; j < TN; j++) xr[gi * TN + j] = as_f(as_u(a[i0 + gi]) ^ bs[j]);
                        cordic_rot_x_vec<NITER, G * TN>(xr);
#pragma unroll
                        for (int gi = 0; gi < G; gi++)
#pragma unroll
                            for (int j = 0; j < TN; j++)
                                acc[i0 + gi][j] = __builtin_fmaf(xr[gi * TN + j] * cordic_kinv(NITER),
                                                                 __builtin_fabsf(b[j]), acc[i0 + gi][j]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int j = 0; j < TN; j++)
                            acc[i][j] = mac<MODE, NITER>(a[i], b[j], bs[j], acc[i][j], iters, kinv);
                }
            }
        }

        if constexpr (MODE == kModeCordic) {
            if (exact_specials && cordic_range_needs_literal(a_lo_m1, a_hi)) lit_pass[pass] = 1;
            __syncthreads();
            if (lit_pass[pass]) {
                // Rare: the tile's A panel holds subnormal, tiny (< 2^-105),
                // top-binade, infinite or NaN elements.  Recompute it straight
                // from global memory (zero outside the matrix, as the staged
                // tiles are): those elements' MACs on the literal chain, all
                // others on the strength-reduced one (the same bits there).
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++) acc[i][j] = 0.0f;
#pragma unroll 1
                for (int k = 0; k < kend; k++) {
                    float a[TM], b[TN];
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        const long gm = m0 + lane_off<TM>(ty, i);
                        a[i] = gm < M ? (TA ? A[(long)k * M + gm] : A[gm * K + k]) : 0.0f;
                    }
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        const long gn = n0 + lane_off<TN>(tx, j);
                        b[j] = gn < N ? (TB ? B[gn * K + k] : B[(long)k * N + gn]) : 0.0f;
                    }
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        if (cordic_needs_literal(a[i])) {
#pragma unroll
                            for (int j = 0; j < TN; j++)
                                acc[i][j] = mac<MODE, NITER, true>(a[i], b[j], as_u(b[j]) & 0x80000000u, acc[i][j],
                                                                   iters, NITER > 0 ? cordic_kinv(NITER > 0 ? NITER : 1)
                                                                                    : kinv);
                        } else {
#pragma unroll
                            for (int j = 0; j < TN; j++)
                                acc[i][j] = mac<MODE, NITER>(a[i], b[j], as_u(b[j]) & 0x80000000u, acc[i][j],
                                                             iters, kinv);
                        }
                    }
                }
            }
        }

#pragma unroll
        for (int i = 0; i < TM; i++) {
            const long gm = m0 + lane_off<TM>(ty, i);
            if (gm >= M) continue;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const long gn = n0 + lane_off<TN>(tx, j);
                if (gn >= N) continue;
                float* cp = C + gm * N + gn;
                // rac_kernels.hip:267-272
                float v = (beta != 0.0f) ? __builtin_fmaf(alpha, acc[i][j], beta * *cp)
                                         : alpha * acc[i][j];
                if constexpr (FUSED) {
                    // rac_torch.cu:770-775: + bias, then the activation in
                    // registers (the pre-activation is kept when asked for)
                    if (ep.bias) v = v + ep.bias[gn];
                    if (ep.pre) ep.pre[gm * N + gn] = v;
                    v = act_rt(v, ep.act, iters, ep.khinv);
                }
                *cp = v;
            }
        }
    }   // pass
}

// ── FAST mode on the matrix cores ───────────────────────────────────────
//
// v_mfma_f32_32x32x1_2b_f32 adds one product to each of its 2 x 32 x 32
// accumulators: D = A_i * B_j + C_ij with a single IEEE rounding, denormals
// kept — the same value as fmaf(a, b, acc) (checked on gfx950 over 8.4 M
// random, subnormal, special and exactly cancelling operands, 0 differences,
// where a separately rounded multiply and add differ in 37%).  Issued once
// per k in k order, it therefore gives every output the FAST MAC's
// accumulation chain bit for bit, at 2048 MACs per instruction for 3 LDS
// floats per lane and k, where the VALU form is bound by LDS bandwidth
// (4096^3: 1.06-1.15 ms against 1.48-1.53 ms on the 16x8 VALU tile).
//
// Block tile 2 WR x 128, BK = 32, staged global -> registers -> LDS with
// the next K-tile's loads in flight during the current one's MFMAs; 4
// waves in 2 x 2, each owning WR x 64 outputs (WR = 64 or 128) as 2 WR / 32
// instructions per k on independent accumulators (a dependent MFMA waits
// ~100 cycles for its predecessor, ~65 cycles of issue, so more chains per
// wave keep the matrix core busier).  For each 64-row group of the wave
// tile, lane l supplies A row l (lanes 0-31 feed the instruction's block 0,
// lanes 32-63 its block 1) and B column l % 32 of a 32-column half (both
// blocks read the same 32 columns), so block b covers rows 32 b .. 32 b + 31.
// Accumulator register r of lane l holds block r / 16, row
// ((r % 16) / 4) * 8 + (l / 32) * 4 + r % 4 of that block, column l % 32.
typedef float v32f __attribute__((ext_vector_type(32)));
constexpr int kMfBN = 128, kMfBK = 32, kMfMinK = 128;

// One operand's K-tile (32 k x ROWS rows) in LDS.  An operand stored with k
// contiguous in memory (A, or B^T of the NT layout) is kept as [row][k]
// rows of 36 floats, so a lane reads 4 consecutive k of its row in one
// ds_read_b128 (rows 144 B apart: 16 lanes cover all 64 banks); the other
// layout stays [k][row] (rows of ROWS + 4 floats) and is read one k at a time.
template <bool KC, int ROWS>
struct MfTile {
    static constexpr int kRows = KC ? ROWS : kMfBK;
    static constexpr int kCols = KC ? kMfBK + 4 : ROWS + 4;
    static constexpr int kVecs = ROWS * kMfBK / 4 / 256;      // float4 per lane
};

// Global -> registers: the 32 x ROWS tile at k0 (rows r0.. of an operand
// with `rows` rows, leading dimension ld) as float4 per lane, zero outside
// the matrix.  k-contiguous: 8 consecutive lanes read a row's 128
// contiguous bytes; otherwise ROWS / 4 consecutive lanes read one k's
// 4 ROWS contiguous bytes.  `vec`: 16-byte loads are aligned (base and ld
// multiples of 4 floats); otherwise every element is loaded on its own.
template <bool KC, int ROWS>
__device__ __forceinline__ void mf_load(const float* __restrict__ P, long ld, long rows, long K, long r0, int k0,
                                        bool vec, float4 (&v)[MfTile<KC, ROWS>::kVecs]) {
    constexpr int kPerK = ROWS / 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int r = 0; r < MfTile<KC, ROWS>::kVecs; r++) {
        const int idx = tid + r * 256;
        float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (KC) {
            const long gr = r0 + (idx >> 3), gk = (long)k0 + (idx & 7) * 4;
            const float* q = P + gr * ld + gk;
            if (vec && gr < rows && gk + 3 < K) {
                v[r] = *reinterpret_cast<const float4*>(q);
                continue;
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (gr < rows && gk + j < K) e[j] = q[j];
        } else {
            const long gk = (long)k0 + idx / kPerK, gr = r0 + (idx % kPerK) * 4;
            const float* q = P + gk * ld + gr;
            if (vec && gk < K && gr + 3 < rows) {
                v[r] = *reinterpret_cast<const float4*>(q);
                continue;
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (gk < K && gr + j < rows) e[j] = q[j];
        }
        v[r] = make_float4(e[0], e[1], e[2], e[3]);
    }
}

// S: the tile's LDS array (kRows x kCols floats, row-major)
template <bool KC, int ROWS>
__device__ __forceinline__ void mf_store(float* S, const float4 (&v)[MfTile<KC, ROWS>::kVecs]) {
    constexpr int kPerK = ROWS / 4, kC = MfTile<KC, ROWS>::kCols;
    const int tid = threadIdx.x;
#pragma unroll
    for (int r = 0; r < MfTile<KC, ROWS>::kVecs; r++) {
        const int idx = tid + r * 256;
        if constexpr (KC) *reinterpret_cast<float4*>(&S[(idx >> 3) * kC + (idx & 7) * 4]) = v[r];
        else *reinterpret_cast<float4*>(&S[(idx / kPerK) * kC + (idx % kPerK) * 4]) = v[r];
    }
}

// k = 4q .. 4q+3 of tile row `row`
template <bool KC, int ROWS>
__device__ __forceinline__ float4 mf_read4(const float* S, int row, int q) {
    constexpr int kC = MfTile<KC, ROWS>::kCols;
    if constexpr (KC) return *reinterpret_cast<const float4*>(&S[row * kC + 4 * q]);
    else return make_float4(S[4 * q * kC + row], S[(4 * q + 1) * kC + row], S[(4 * q + 2) * kC + row],
                            S[(4 * q + 3) * kC + row]);
}

// WR: rows of a wave's tile (64: 2 accumulator chains per wave, 128: 4);
// the block tile is 2 WR x 128.  TRAP: causal attention scores of query
// rows row0 .. row0 + M - 1 against keys 0 .. N - 1, only the tiles on or
// below the diagonal (trap_cols per row tile, numbered row by row along
// grid x, as gemm_kernel's schedule 3); the masked softmax overwrites the
// scores above the diagonal, so the others are never read.
template <bool TA, bool TB, bool FUSED, int WR, bool TRAP = false>
__global__ __launch_bounds__(256, WR == 128 ? 2 : 1) void gemm_mfma_fast_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
    int M, int N, int K, float alpha, float beta, int iters, long sa, long sb, long sc, GemmEpilogue ep,
    int vec_a, int vec_b, const int* k_causal, int row0)
{
    constexpr bool KA = !TA, KB = TB;     // operand stored with k contiguous
    constexpr int BM = 2 * WR, BN = kMfBN, WI = WR / 64;
    using TAt = MfTile<KA, BM>;
    using TBt = MfTile<KB, BN>;
    int tm = blockIdx.y, tn = blockIdx.x;
    if constexpr (TRAP) {
        int l = blockIdx.x;
        tm = 0;
        for (;;) {
            const int c = trap_cols(row0, tm, BM, BN, N);
            if (l < c) break;
            l -= c;
            tm++;
        }
        tn = l;
    }
    const long m0 = (long)tm * BM, n0 = (long)tn * BN;
    A += (long)blockIdx.z * sa;
    B += (long)blockIdx.z * sb;
    C += (long)blockIdx.z * sc;
    __shared__ __attribute__((aligned(16))) float sA[TAt::kRows][TAt::kCols];
    __shared__ __attribute__((aligned(16))) float sB[TBt::kRows][TBt::kCols];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = (wave >> 1) * WR, wc = (wave & 1) * 64;
    const long lda = TA ? M : K, ldb = TB ? K : N;

    v32f acc[WI][2];
#pragma unroll
    for (int i = 0; i < WI; i++)
#pragma unroll
        for (int r = 0; r < 32; r++) {
            acc[i][0][r] = 0.0f;
            acc[i][1][r] = 0.0f;
        }
    float4 va[TAt::kVecs], vb[TBt::kVecs];
    // Zero operands past K leave an accumulator unchanged: fma(0, 0, acc)
    // == acc because acc starts at +0 and never becomes -0.  Causal P V
    // (*k_causal == 1: every v finite) stops after the tile's last query
    // position, as gemm_kernel does.
    int kend = K;
    if (k_causal && *k_causal == 1) kend = (int)min((long)K, (long)row0 + m0 + BM);
    mf_load<KA, BM>(A, lda, M, K, m0, 0, vec_a, va);
    mf_load<KB, BN>(B, ldb, N, K, n0, 0, vec_b, vb);
    for (int k0 = 0; k0 < kend; k0 += kMfBK) {
        __syncthreads();
        mf_store<KA, BM>(&sA[0][0], va);
        mf_store<KB, BN>(&sB[0][0], vb);
        __syncthreads();
        if (k0 + kMfBK < kend) {
            mf_load<KA, BM>(A, lda, M, K, m0, k0 + kMfBK, vec_a, va);
            mf_load<KB, BN>(B, ldb, N, K, n0, k0 + kMfBK, vec_b, vb);
        }
#pragma unroll
        for (int q = 0; q < kMfBK / 4; q++) {
            float4 a[WI];
#pragma unroll
            for (int i = 0; i < WI; i++) a[i] = mf_read4<KA, BM>(&sA[0][0], wr + 64 * i + lane, q);
            const float4 b0 = mf_read4<KB, BN>(&sB[0][0], wc + (lane & 31), q);
            const float4 b1 = mf_read4<KB, BN>(&sB[0][0], wc + 32 + (lane & 31), q);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int i = 0; i < WI; i++) {
                    const float aj = j == 0 ? a[i].x : j == 1 ? a[i].y : j == 2 ? a[i].z : a[i].w;
                    const float b0j = j == 0 ? b0.x : j == 1 ? b0.y : j == 2 ? b0.z : b0.w;
                    const float b1j = j == 0 ? b1.x : j == 1 ? b1.y : j == 2 ? b1.z : b1.w;
                    acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x1f32(aj, b0j, acc[i][0], 0, 0, 0);
                    acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x1f32(aj, b1j, acc[i][1], 0, 0, 0);
                }
        }
    }

    const long col0 = n0 + wc + (lane & 31);
#pragma unroll
    for (int i = 0; i < WI; i++)
#pragma unroll
    for (int r = 0; r < 32; r++) {
        const long gm = m0 + wr + 64 * i + (r / 16) * 32 + ((r % 16) / 4) * 8 + (lane / 32) * 4 + (r % 4);
        if (gm >= M) continue;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const long gn = col0 + 32 * h;
            if (gn >= N) continue;
            float* cp = C + gm * N + gn;
            const float x = acc[i][h][r];
            // rac_kernels.hip:267-272
            float v = (beta != 0.0f) ? __builtin_fmaf(alpha, x, beta * *cp) : alpha * x;
            if constexpr (FUSED) {
                // rac_torch.cu:770-775
                if (ep.bias) v = v + ep.bias[gn];
                if (ep.pre) ep.pre[gm * N + gn] = v;
                v = act_rt(v, ep.act, iters, ep.khinv);
            }
            *cp = v;
        }
    }
}

// flag = 1 unless some x[i] is inf or NaN (flag must be 1 on entry; lanes
// only ever store 0, so concurrent stores agree).
__global__ __launch_bounds__(256) void all_finite_kernel(const float* __restrict__ x, long n,
                                                         int* __restrict__ flag) {
    const long stride = (long)gridDim.x * blockDim.x;
    bool ok = true;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        ok &= __builtin_isfinite(x[i]);
    if (!ok) *flag = 0;
}

__global__ void set_flag_kernel(int* flag, int v) { *flag = v; }

hipError_t all_finite_launch(const float* x, long n, int* flag, hipStream_t s) {
    hipLaunchKernelGGL(set_flag_kernel, dim3(1), dim3(1), 0, s, flag, 1);
    long blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(all_finite_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, n, flag);
    return hipGetLastError();
}

struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    int M, N, K;
    float alpha, beta;
    int iters;
    int batch;
    long sa, sb, sc;
    GemmEpilogue ep;
    bool fused;
    int sched;
    const int* k_causal;
    int exact_specials;
    int row0;
};

template <int MODE, int NITER, bool TA, bool TB, bool FUSED, int SCHED, int TM, int TN = TM>
static hipError_t launch_cfg(const GemmArgs& g, hipStream_t stream) {
    using Cfg = GemmCfg<MODE, NITER, TA, TB, TM, TN>;
    const float kinv = cordic_kinv(g.iters);
    const unsigned nt = (unsigned)((g.M + Cfg::kBM - 1) / Cfg::kBM);
    dim3 grid((unsigned)((g.N + Cfg::kBN - 1) / Cfg::kBN), nt, (unsigned)g.batch);
    if (g.sched == 1) grid = dim3(nt + 1, (nt + 1) / 2, (unsigned)g.batch);
    if (g.sched == 2) grid.y = (nt + 1) / 2;
    if (g.sched == 3) {
        long tiles = 0;
        for (unsigned r = 0; r < nt; r++) tiles += trap_cols(g.row0, (int)r, Cfg::kBM, Cfg::kBN, g.N);
        grid = dim3((unsigned)tiles, 1, (unsigned)g.batch);
    }
    hipLaunchKernelGGL((gemm_kernel<MODE, NITER, TA, TB, TM, TN, FUSED, SCHED>), grid, dim3(256), 0, stream,
                       g.A, g.B, g.C, g.M, g.N, g.K, g.alpha, g.beta, g.iters, kinv, g.sa, g.sb, g.sc,
                       g.ep, g.k_causal, g.exact_specials, g.row0);
    return hipGetLastError();
}

template <bool TA, bool TB, bool FUSED, int WR, bool TRAP = false>
static hipError_t launch_mfma_fast(const GemmArgs& g, hipStream_t stream) {
    constexpr int BM = 2 * WR;
    dim3 grid((unsigned)((g.N + kMfBN - 1) / kMfBN), (unsigned)((g.M + BM - 1) / BM), (unsigned)g.batch);
    if constexpr (TRAP) {
        long t = 0;
        for (int r = 0; r < (int)grid.y; r++) t += trap_cols(g.row0, r, BM, kMfBN, g.N);
        grid = dim3((unsigned)t, 1, (unsigned)g.batch);
    }
    // 16-byte loads need 16-byte aligned rows in every batch item
    auto aligned = [](const float* p, long ld, long stride) {
        return ((uintptr_t)p % 16 == 0) && ld % 4 == 0 && stride % 4 == 0;
    };
    const int vec_a = aligned(g.A, TA ? g.M : g.K, g.batch > 1 ? g.sa : 0);
    const int vec_b = aligned(g.B, TB ? g.K : g.N, g.batch > 1 ? g.sb : 0);
    hipLaunchKernelGGL((gemm_mfma_fast_kernel<TA, TB, FUSED, WR, TRAP>), grid, dim3(256), 0, stream, g.A, g.B, g.C,
                       g.M, g.N, g.K, g.alpha, g.beta, g.iters, g.sa, g.sb, g.sc, g.ep, vec_a, vec_b, g.k_causal,
                       g.row0);
    return hipGetLastError();
}

// Compute units of the current device (256 on MI355X), cached per device.
long device_cus() {
    static std::atomic<long> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256;
    }
    long v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        v = n;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Register tile: 8x8 per lane (128x128 block) for FAST (16x8 when that fills
// the CUs better), 4x4 (64x64) for the
// CORDIC and SHIFTADD MACs, stepping down while the launch would have fewer
// than kMinTiles blocks; the triangular and paired-row schedules keep the
// 64x64 tile they are written for.  The tile never changes a result: each
// output is one accumulator over k in order.
template <int MODE, int NITER, bool TA, bool TB, bool FUSED, int SCHED = 0>
static hipError_t launch_tiles(const GemmArgs& g, hipStream_t s) {
    constexpr int kBig = (MODE == kModeFast) ? 8 : 4;
    if constexpr (MODE == kModeFast && SCHED != 0) {
        // Causal attention products on the matrix cores under the rule of
        // the plain schedule below: the scores (1: square, row0 = 0; 3: a
        // chunk of query rows) over the tiles on or below the diagonal,
        // P V (2) as a plain launch whose row tiles stop at their causal
        // K limit (pairing row tiles for balance is not needed at MFMA
        // block counts).
        const long cus = device_cus();
        if (g.K >= kMfMinK) {
            if constexpr (SCHED == 2) {
                const long t = ((g.M + 127) / 128) * ((g.N + kMfBN - 1) / kMfBN) * (long)g.batch;
                if (4 * t >= cus && (double)g.M * g.N * g.batch >= 0.5 * (double)t * 128.0 * kMfBN)
                    return launch_mfma_fast<TA, TB, FUSED, 64>(g, s);
            } else {
                GemmArgs h = g;
                if constexpr (SCHED == 1) h.row0 = 0;
                long t = 0;
                for (int r = 0; r < (int)((g.M + 127) / 128); r++) t += trap_cols(h.row0, r, 128, kMfBN, g.N);
                if (g.M >= 64 && 4 * t * (long)g.batch >= cus) return launch_mfma_fast<TA, TB, FUSED, 64, true>(h, s);
            }
        }
    }
    if constexpr (SCHED == 2) {
        // Causal P V, row tiles p and nt-1-p per workgroup (equal K sums): on
        // 64x64 tiles while that gives 2 workgroups per CU, else on 32x32
        // while 4 per CU (the attention core's 512-row chunks: 4-9% faster
        // than unpaired), else unpaired (256-row chunks: no gain)
        const long cus = device_cus();
        const long pairs4 = (((g.M + 63) / 64 + 1) / 2) * ((g.N + 63) / 64) * (long)g.batch;
        if (pairs4 >= 2 * cus) return launch_cfg<MODE, NITER, TA, TB, FUSED, SCHED, 4>(g, s);
        const long pairs2 = (((g.M + 31) / 32 + 1) / 2) * ((g.N + 31) / 32) * (long)g.batch;
        if (pairs2 >= 4 * cus) return launch_cfg<MODE, NITER, TA, TB, FUSED, SCHED, 2>(g, s);
        GemmArgs h = g;
        h.sched = 0;
        return launch_tiles<MODE, NITER, TA, TB, FUSED, 0>(h, s);
    } else if constexpr (SCHED == 1) {
        return launch_cfg<MODE, NITER, TA, TB, FUSED, SCHED, 4>(g, s);
    } else {
        auto tiles = [&](long bm, long bn) {
            if constexpr (SCHED == 3) {      // the causal trapezoid's tiles only
                long t = 0;
                for (long r = 0; r < (g.M + bm - 1) / bm; r++) t += trap_cols(g.row0, (int)r, (int)bm, (int)bn, g.N);
                return t * (long)g.batch;
            }
            return ((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn) * (long)g.batch;
        };
        if constexpr (MODE == kModeFast && SCHED == 0) {
            // The matrix cores, once there are cus / 4 blocks of 128 x 128,
            // at least half of their outputs real and K >= 128.  An MFMA
            // block costs K x 128 cycles of its SIMDs whatever its fill:
            // measured against the VALU tiles (bit-identical), 64 blocks
            // (1024^2 x 1024, 32 x 256 x 128 x 2048) are 5-8% faster, 128
            // blocks (the attention P V chunks 32 x 512 x 128 x K, 512 x
            // 4096 x 4096 NT) 65-84% faster, while 32 blocks of a short M
            // (128 x 4096 x 4096) are 3x slower, and K = 37 (2050 x 2049)
            // 20 us against 16.
            // Wave tiles of 128 x 64 (4 accumulator chains per wave, 2
            // blocks of 256 x 128 per CU) beat 64 x 64 (2 chains, 3 blocks
            // of 128 x 128 per CU) by 5-7% when they fill a round of the CUs
            // and their rounds of resident blocks are fuller (4096^3,
            // 8192^3), and lose up to 19% when a partial last round remains
            // (2048 x 12288: 1.5 rounds against 2), so the fuller one is
            // taken, 64 x 64 on a tie.  The fused epilogue keeps 64 x 64
            // (with 4 chains it no longer fits the registers).
            const long cus = device_cus();
            auto fill = [&](long t, long per_cu) {
                const long slots = per_cu * cus, rounds = (t + slots - 1) / slots;
                return (double)t / (double)(rounds * slots);
            };
            const long t128 = tiles(128, kMfBN), t256 = tiles(256, kMfBN);
            const double used = (double)g.M * (double)g.N * (double)g.batch / ((double)t128 * kMfBN * 128.0);
            if (g.K >= kMfMinK && 4 * t128 >= cus && used >= 0.5) {
                if constexpr (!FUSED) {
                    if (t256 >= cus && fill(t256, 2) > fill(t128, 3)) return launch_mfma_fast<TA, TB, FUSED, 128>(g, s);
                }
                return launch_mfma_fast<TA, TB, FUSED, 64>(g, s);
            }
            // 16x8 per lane (256x128 blocks, 2 per CU at its register count)
            // reads 25% fewer LDS bytes per FMA than 8x8 (128x128, 3 per
            // CU); it is taken when it fills its rounds of resident blocks
            // at least as completely as 8x8 does
            if (t256 >= 2 * cus && fill(t256, 2) >= fill(t128, 3))
                return launch_cfg<MODE, NITER, TA, TB, FUSED, 0, 16, 8>(g, s);
        }
        if (tiles(16 * kBig, 16 * kBig) >= kMinTiles) return launch_cfg<MODE, NITER, TA, TB, FUSED, SCHED, kBig>(g, s);
        if constexpr (kBig == 4) {
            // CORDIC / SHIFTADD: two 64x64 blocks per CU (2 waves per SIMD,
            // 16 MAC chains each) still beat 32x32 blocks (measured, same
            // bits: 512-1023 blocks 5-6% faster, e.g. the attention core's
            // P V chunks 32 x 512 x 128 x K; at one block per CU 43% slower)
            if (tiles(64, 64) >= 2 * device_cus()) return launch_cfg<MODE, NITER, TA, TB, FUSED, SCHED, 4>(g, s);
        }
        if constexpr (kBig == 8) {
            if (tiles(64, 64) >= kMinTiles) return launch_cfg<MODE, NITER, TA, TB, FUSED, SCHED, 4>(g, s);
        }
        return launch_cfg<MODE, NITER, TA, TB, FUSED, SCHED, 2>(g, s);
    }
}

// The fused epilogue exists for the NT layout only (input @ weight^T, the
// linear layer), the triangular and trapezoidal schedules for NT only
// (causal Q K^T) and the paired-row schedule for NN only (causal P V);
// their callers never ask for another layout.
template <int MODE, int NITER>
static hipError_t launch_layout(int ta, int tb, const GemmArgs& g, hipStream_t s) {
    if (g.fused) return launch_tiles<MODE, NITER, false, true, true>(g, s);
    if (g.sched == 1) return launch_tiles<MODE, NITER, false, true, false, 1>(g, s);   // NT only
    if (g.sched == 2) return launch_tiles<MODE, NITER, false, false, false, 2>(g, s);  // NN only
    if (g.sched == 3) return launch_tiles<MODE, NITER, false, true, false, 3>(g, s);   // NT only
    if (!ta && !tb) return launch_tiles<MODE, NITER, false, false, false>(g, s);
    if (!ta && tb) return launch_tiles<MODE, NITER, false, true, false>(g, s);
    if (ta && !tb) return launch_tiles<MODE, NITER, true, false, false>(g, s);
    return launch_tiles<MODE, NITER, true, true, false>(g, s);
}

static hipError_t dispatch(int ta, int tb, int mode, const GemmArgs& g, hipStream_t s) {
    // few rows or columns (schedule 2, the causal P V, is then the plain
    // product with its causal K limit, which those kernels apply)
    if ((g.sched == 0 || g.sched == 2) && !ta && (g.M <= kSkinnyMaxRows || g.N <= kSkinnyMaxRows)) {
        const SkinnyArgs k{g.A, g.B, g.C, g.M, g.N, g.K, g.alpha, g.beta, g.iters, g.batch, g.sa, g.sb, g.sc,
                           g.ep, g.fused, tb != 0, g.k_causal, g.exact_specials, g.row0};
        return gemm_skinny_launch(k, mode, s);
    }
    if (mode == kModeFast) return launch_layout<kModeFast, 0>(ta, tb, g, s);
    if (mode == kModeShiftAdd) return launch_layout<kModeShiftAdd, 0>(ta, tb, g, s);
    switch (g.iters) {
        case 8: return launch_layout<kModeCordic, 8>(ta, tb, g, s);
        case 16: return launch_layout<kModeCordic, 16>(ta, tb, g, s);
        case 24: return launch_layout<kModeCordic, 24>(ta, tb, g, s);
        default: return launch_layout<kModeCordic, 0>(ta, tb, g, s);
    }
}

hipError_t gemm_launch(int ta, int tb, const float* A, const float* B, float* C,
                       int M, int N, int K, float alpha, float beta, int iters, int mode,
                       hipStream_t s, int batch, long sa, long sb, long sc, int sched,
                       const int* k_causal, bool exact_specials, int row0) {
    const GemmArgs g{A, B, C, M, N, K, alpha, beta, clamp_iters(iters), batch, sa, sb, sc,
                     GemmEpilogue(), false, sched, k_causal, exact_specials ? 1 : 0, row0};
    return dispatch(ta, tb, mode, g, s);
}

hipError_t gemm_fused_launch(const float* A, const float* W, float* C, int M, int N, int K,
                             const GemmEpilogue& ep, int iters, int mode, hipStream_t s) {
    const GemmArgs g{A, W, C, M, N, K, 1.0f, 0.0f, clamp_iters(iters), 1, 0, 0, 0, ep, true, 0, nullptr, 1, 0};
    return dispatch(0, 1, mode, g, s);
}

}  // namespace rac
