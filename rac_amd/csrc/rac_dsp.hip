// rac_dsp.hip — the RAC-DSP fixed-point CORDIC engine (the integer datapath
// that sim/rac_dsp_core.c:95-149 defines for the RTL) as batch kernels for
// gfx950, bit-exact with that model.
//
// Operands are 64-bit two's-complement integers: x, y in Q32.32, z in Q0.63
// fractions of pi.  One evaluation: quadrant fold (|z| >= pi/2 -> z + pi,
// x, y negated); for every op but vectoring a coarse stage of 10 circular
// micro-rotations whose direction word comes from a 1024-entry LUT indexed
// by the top bits of 2z (the "angle-index" stage: no decisions, only
// shift-adds); then 9 residual micro-rotations at shifts 8..16 (circular,
// hyperbolic for op 3, vectoring on sign(y) for op 2).  All arithmetic wraps
// modulo 2^64 (uint64_t here), as the hardware registers do.
//
// The ROMs (LUT, atan(2^-i) i < 17, atanh(2^-s) s = 8..16, plus the coarse
// stage's per-word angle derived from them) live in device memory per GPU,
// are copied into LDS by every workgroup (10.4 KB), and are
// either the library's generated contents (the rule of rtl/gen_coarse_lut.py,
// identical to the rtl/*.mem files) or what rac_load_all_roms read.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "rac_internal.hpp"

namespace rac {

template <int N>
__device__ __forceinline__ uint64_t asr64(uint64_t v) {
    return (uint64_t)((int64_t)v >> N);
}

// Every micro-rotation is written as an if / else on its direction: the two
// arms become exec-masked VALU blocks, so the choice costs scalar mask
// operations instead of v_cndmask selects (which issue at half rate, as do
// the 64-bit shifts and adds).  A 64-bit add is one v_lshl_add_u64, a
// subtraction two carry ops.

// Coarse step I: direction from bit I of the LUT word (z is handled by the
// per-word table).
template <int I>
__device__ __forceinline__ void dsp_coarse(uint64_t& x, uint64_t& y, uint32_t dv) {
    const uint64_t ys = asr64<I>(y), xs = asr64<I>(x);
    if ((dv >> I) & 1u) {
        x = x - ys;
        y = y + xs;
    } else {
        x = x + ys;
        y = y - xs;
    }
    if constexpr (I + 1 < kDspLutBits) dsp_coarse<I + 1>(x, y, dv);
}

// Residual step I (physical shift 8 + I); direction from the sign of z
// (sign of y for vectoring), constants from the ROMs in LDS.
template <int OP, int I>
__device__ __forceinline__ void dsp_residual(uint64_t& x, uint64_t& y, uint64_t& z, const int64_t* atan_rom,
                                             const int64_t* atanh_rom) {
    constexpr int PH = kDspResStart + I;
    const bool dpos = (OP == 2) ? ((int32_t)(y >> 32) < 0) : ((int32_t)(z >> 32) >= 0);
    const uint64_t xs = asr64<PH>(x), ys = asr64<PH>(y);
    const uint64_t c = (uint64_t)((OP == 3) ? atanh_rom[I] : atan_rom[PH]);
    if (dpos) {
        if constexpr (OP == 3) x = x + ys;
        else x = x - ys;
        y = y + xs;
        z = z - c;
    } else {
        if constexpr (OP == 3) x = x - ys;
        else x = x + ys;
        y = y - xs;
        z = z + c;
    }
    if constexpr (I + 1 < kDspRes) dsp_residual<OP, I + 1>(x, y, z, atan_rom, atanh_rom);
}

struct DspLds {
    uint16_t lut[kDspLut];
    int64_t coarse_z[kDspLut];
    int64_t atan_rom[kDspAtan];
    int64_t atanh_rom[kDspRes];
};

template <int OP>
__device__ __forceinline__ void dsp_eval(uint64_t& x, uint64_t& y, uint64_t& z, const DspLds& r) {
    if (((z >> 63) ^ (z >> 62)) & 1u) {      // |z| >= pi/2: rotate by pi first
        z ^= (uint64_t)1 << 63;
        x = (uint64_t)0 - x;
        y = (uint64_t)0 - y;
    }
    if constexpr (OP != 2) {
        // LUT index: top 10 bits of 2z, offset to unsigned
        const int idx = (int)(((int64_t)(z << 1) >> (64 - kDspLutBits)) + kDspLut / 2) & (kDspLut - 1);
        z = z - (uint64_t)r.coarse_z[idx];
        dsp_coarse<0>(x, y, r.lut[idx]);
    }
    dsp_residual<OP, 0>(x, y, z, r.atan_rom, r.atanh_rom);
}

// Stage the ROMs in LDS (every lane of the workgroup helps).
__device__ __forceinline__ void dsp_stage_roms(const DspRoms* __restrict__ g, DspLds& r) {
    for (int i = threadIdx.x; i < kDspLut; i += blockDim.x) {
        r.lut[i] = g->lut[i];
        r.coarse_z[i] = g->coarse_z[i];
    }
    for (int i = threadIdx.x; i < kDspAtan; i += blockDim.x) r.atan_rom[i] = g->atan_rom[i];
    for (int i = threadIdx.x; i < kDspRes; i += blockDim.x) r.atanh_rom[i] = g->atanh_rom[i];
    __syncthreads();
}

template <int OP>
__global__ __launch_bounds__(256) void dsp_eval_kernel(long n, const int64_t* __restrict__ xi,
                                                       const int64_t* __restrict__ yi,
                                                       const int64_t* __restrict__ zi, int64_t* __restrict__ xo,
                                                       int64_t* __restrict__ yo, int64_t* __restrict__ zo,
                                                       const DspRoms* __restrict__ roms) {
    __shared__ DspLds r;
    dsp_stage_roms(roms, r);
    const long stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        uint64_t x = (uint64_t)xi[i], y = yi ? (uint64_t)yi[i] : 0, z = (uint64_t)zi[i];
        dsp_eval<OP>(x, y, z, r);
        xo[i] = (int64_t)x;
        if (yo) yo[i] = (int64_t)y;
        if (zo) zo[i] = (int64_t)z;
    }
}

// Weight-stationary systolic product (sim/rac_systolic_ref.c:40-55):
// Y[k][c] = sum_r project(X[k][r], 0, W[r][c]).x.  A workgroup owns 64
// consecutive outputs (flattened k*N + c) and splits r over its 4 waves;
// the 4 partial sums are added through LDS.  The sum wraps modulo 2^64, so
// its order does not change the result.
constexpr int kSysOuts = 64;
constexpr int kSysSlices = 4;

__global__ __launch_bounds__(256) void dsp_systolic_kernel(int N, int K, const int64_t* __restrict__ W,
                                                           const int64_t* __restrict__ X,
                                                           int64_t* __restrict__ Y,
                                                           const DspRoms* __restrict__ roms) {
    __shared__ DspLds r;
    __shared__ uint64_t part[kSysSlices][kSysOuts];
    dsp_stage_roms(roms, r);
    const int lane = threadIdx.x % kSysOuts, slice = threadIdx.x / kSysOuts;
    const long o = (long)blockIdx.x * kSysOuts + lane;
    uint64_t sum = 0;
    if (o < (long)N * K) {
        const int k = (int)(o / N), c = (int)(o % N);
        for (int rr = slice; rr < N; rr += kSysSlices) {
            uint64_t x = (uint64_t)X[(long)k * N + rr], y = 0, z = (uint64_t)W[(long)rr * N + c];
            dsp_eval<0>(x, y, z, r);          // project: the circular rotation, x kept
            sum += x;
        }
    }
    part[slice][lane] = sum;
    __syncthreads();
    if (slice == 0 && o < (long)N * K) {
        uint64_t t = part[0][lane];
        for (int j = 1; j < kSysSlices; j++) t += part[j][lane];
        Y[o] = (int64_t)t;
    }
}

hipError_t dsp_eval_launch(int op, long n, const int64_t* x, const int64_t* y, const int64_t* z, int64_t* xo,
                           int64_t* yo, int64_t* zo, const DspRoms* roms, hipStream_t s) {
    long blocks = (n + 255) / 256;
    if (blocks > 256L * 32) blocks = 256L * 32;
    if (blocks < 1) blocks = 1;
    const dim3 g((unsigned)blocks), b(256);
    // op 2 vectoring, op 3 hyperbolic; every other op (0 rotate, 1 project,
    // ...) is the circular rotation (rac_dsp_core.c:102-103)
    if (op == 2)
        hipLaunchKernelGGL(dsp_eval_kernel<2>, g, b, 0, s, n, x, y, z, xo, yo, zo, roms);
    else if (op == 3)
        hipLaunchKernelGGL(dsp_eval_kernel<3>, g, b, 0, s, n, x, y, z, xo, yo, zo, roms);
    else
        hipLaunchKernelGGL(dsp_eval_kernel<0>, g, b, 0, s, n, x, y, z, xo, yo, zo, roms);
    return hipGetLastError();
}

hipError_t dsp_systolic_launch(int N, int K, const int64_t* W, const int64_t* X, int64_t* Y, const DspRoms* roms,
                               hipStream_t s) {
    const long outs = (long)N * K;
    hipLaunchKernelGGL(dsp_systolic_kernel, dim3((unsigned)((outs + kSysOuts - 1) / kSysOuts)),
                       dim3(kSysOuts * kSysSlices), 0, s, N, K, W, X, Y, roms);
    return hipGetLastError();
}

}  // namespace rac
