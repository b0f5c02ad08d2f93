// rac_q8.hip — Q8_0 weights (lib/c/rac_q8_0.h: blocks of 32 int8 with one
// fp16 scale, 34 bytes) and the decode GEMV out = act(W x + bias) on gfx950.
//
// The GEMV is HBM-bound: every weight byte is read once (34 bytes per 32
// weights, 3.8x less than fp32).  Results are bit-identical to the
// reference's AVX2 build (rac_q8_0.c:128-211): each block's 32 products
// combine in the order of its 8-lane vector tree, and the block terms of a
// row accumulate in block order as acc = fma(d_b, dot_b, acc).  That serial
// order is kept without serialising the memory stream:
//
//   * a workgroup owns 64 consecutive weight rows and walks K in chunks of
//     8 blocks (272 bytes per row, 16-byte aligned when K % 256 == 0);
//   * each chunk is fetched with 16-byte loads (64 x 272 contiguous-row
//     segments) into registers one chunk ahead, then written to LDS;
//   * all 256 lanes compute the 64 x 8 block dots (per input row) from LDS;
//   * one lane per (input row, weight row) then folds the chunk's 8 terms
//     into its accumulator in block order.
//
// Shapes the fast kernel does not cover (K % 256 != 0, unaligned buffers)
// take a generic kernel with the same arithmetic.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include "rac_internal.hpp"

namespace rac {

constexpr int kQ8Block = 32;
constexpr int kQ8Bytes = 34;
constexpr int kQ8Rows = 64;                    // weight rows per workgroup
constexpr int kQ8Chunk = 8;                    // blocks per chunk
constexpr int kQ8Seg = kQ8Chunk * kQ8Bytes;    // 272 bytes of one row per chunk
constexpr int kQ8Vec = kQ8Seg / 16;            // 17 16-byte vectors per segment
constexpr int kQ8Loads = (kQ8Rows * kQ8Vec + 255) / 256;   // per lane per chunk

// rac_fp16_to_fp32 (rac_q8_0.c:21-45) as bit operations.
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu, bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            // normalise: shift until bit 10 is set
            const int lz = __builtin_clz(mant) - 21;   // leading zeros within the 11-bit field
            mant = (mant << lz) & 0x3ffu;
            bits = (sign << 31) | ((uint32_t)(-14 - lz + 127) << 23) | (mant << 13);
        }
    } else if (ex == 31) {
        bits = (sign << 31) | (0xffu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((ex - 15 + 127) << 23) | (mant << 13);
    }
    return __uint_as_float(bits);
}

// rac_fp32_to_fp16 (rac_q8_0.c:47-64): truncating conversion.
__device__ __forceinline__ uint32_t float_to_half_bits(float f) {
    const uint32_t b = __float_as_uint(f);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int ex = (int)((b >> 23) & 0xffu) - 127 + 15;
    uint32_t mant = b & 0x7fffffu;
    if (ex <= 0) {
        if (ex < -10) return sign;
        mant = (mant | 0x800000u) >> (1 - ex);
        return sign | (mant >> 13);
    }
    if (ex >= 31) return sign | 0x7c00u | (mant ? 0x200u : 0u);
    return sign | ((uint32_t)ex << 10) | (mant >> 13);
}

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

// Fast path: K % 256 == 0, weights and inputs 16-byte aligned.  MG groups of
// 4 input rows (M <= 4 * MG); lane t accumulates outputs (m, j0 + t % 64)
// for m = t / 64 + 4 g.
template <int MG>
__global__ __launch_bounds__(256) void q8_gemv_kernel(const float* __restrict__ x,
                                                      const uint8_t* __restrict__ w,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ out, int M, int N, int K,
                                                      int act) {
    __shared__ __attribute__((aligned(16))) uint8_t sw[kQ8Rows * kQ8Seg];
    __shared__ __attribute__((aligned(16))) float sx[4 * MG][kQ8Chunk * kQ8Block];
    __shared__ float sdot[4 * MG][kQ8Rows][kQ8Chunk + 1];

    const int tid = threadIdx.x;
    const long j0 = (long)blockIdx.x * kQ8Rows;
    const int nrows = (int)min((long)kQ8Rows, (long)N - j0);
    const int nb = K / kQ8Block;
    const long rowB = (long)nb * kQ8Bytes;
    const int nchunks = nb / kQ8Chunk;

    uint4 rw[kQ8Loads];
    float4 rx[MG];
    auto fetch = [&](int c) {
#pragma unroll
        for (int i = 0; i < kQ8Loads; i++) {
            const int v = tid + i * 256;
            if (v < nrows * kQ8Vec) {
                const int r = v / kQ8Vec, o = v % kQ8Vec;
                rw[i] = *reinterpret_cast<const uint4*>(w + (j0 + r) * rowB + (long)c * kQ8Seg + o * 16);
            }
        }
        // inputs: 64 float4 per input row per chunk
#pragma unroll
        for (int g = 0; g < MG; g++) {
            const int m = tid / 64 + 4 * g;
            if (m < M)
                rx[g] = *reinterpret_cast<const float4*>(x + (long)m * K + (long)c * (kQ8Chunk * kQ8Block) +
                                                         (tid % 64) * 4);
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < kQ8Loads; i++) {
            const int v = tid + i * 256;
            if (v < nrows * kQ8Vec) {
                const int r = v / kQ8Vec, o = v % kQ8Vec;
                *reinterpret_cast<uint4*>(&sw[r * kQ8Seg + o * 16]) = rw[i];
            }
        }
#pragma unroll
        for (int g = 0; g < MG; g++) {
            const int m = tid / 64 + 4 * g;
            if (m < M) *reinterpret_cast<float4*>(&sx[m][(tid % 64) * 4]) = rx[g];
        }
    };

    float acc[MG];
#pragma unroll
    for (int g = 0; g < MG; g++) acc[g] = 0.0f;

    fetch(0);
    for (int c = 0; c < nchunks; c++) {
        __syncthreads();          // previous chunk's LDS fully consumed
        stash();
        __syncthreads();
        if (c + 1 < nchunks) fetch(c + 1);   // next chunk in flight during the math
        // block dots: lane t covers row r = t % 64, blocks t / 64 and t / 64 + 4
        const int r = tid % 64;
        if (r < nrows) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int k = tid / 64 + 4 * h;      // uniform across the wave
                // the block's 32 q bytes start at byte A = r*272 + k*34 + 2,
                // 4-aligned for odd k and 2 past a dword for even k: read
                // dwords and realign with one alignbit each
                const int A = r * kQ8Seg + k * kQ8Bytes + 2;
                const uint32_t* dw = reinterpret_cast<const uint32_t*>(&sw[A & ~3]);
                uint32_t word[8];
                if (k & 1) {
#pragma unroll
                    for (int i = 0; i < 8; i++) word[i] = dw[i];
                } else {
                    uint32_t d[9];
#pragma unroll
                    for (int i = 0; i < 9; i++) d[i] = dw[i];
#pragma unroll
                    for (int i = 0; i < 8; i++) word[i] = __builtin_amdgcn_alignbit(d[i + 1], d[i], 16);
                }
                float qf[kQ8Block];
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int b = 0; b < 4; b++) qf[4 * i + b] = (float)(int8_t)(word[i] >> (8 * b));
#pragma unroll
                for (int m = 0; m < 4 * MG; m++)
                    if (m < M) sdot[m][r][k] = q8_block_dot(qf, &sx[m][k * kQ8Block]);
            }
        }
        __syncthreads();
        // ordered fold of the chunk's 8 terms
        if (r < nrows) {
#pragma unroll
            for (int g = 0; g < MG; g++) {
                const int m = tid / 64 + 4 * g;
                if (m < M) {
#pragma unroll
                    for (int k = 0; k < kQ8Chunk; k++) {
                        const uint8_t* blk = &sw[r * kQ8Seg + k * kQ8Bytes];
                        const float d = half_bits_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
                        acc[g] = __builtin_fmaf(d, sdot[m][r][k], acc[g]);
                    }
                }
            }
        }
    }
    const int r = tid % 64;
    if (r < nrows) {
#pragma unroll
        for (int g = 0; g < MG; g++) {
            const int m = tid / 64 + 4 * g;
            if (m < M) out[(long)m * N + j0 + r] = q8_finish(acc[g], bias, j0 + r, act);
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

hipError_t q8_gemv_launch(const float* x, const uint8_t* w, const float* bias, float* out, int M, int N,
                          int K, int act, hipStream_t s) {
    const bool fast = (K % (kQ8Chunk * kQ8Block) == 0) && ((reinterpret_cast<uintptr_t>(w) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && M <= 16;
    if (fast) {
        const dim3 grid((unsigned)((N + kQ8Rows - 1) / kQ8Rows));
        const int mg = (M + 3) / 4;
        switch (mg) {
        case 1: hipLaunchKernelGGL((q8_gemv_kernel<1>), grid, dim3(256), 0, s, x, w, bias, out, M, N, K, act); break;
        case 2: hipLaunchKernelGGL((q8_gemv_kernel<2>), grid, dim3(256), 0, s, x, w, bias, out, M, N, K, act); break;
        case 3: hipLaunchKernelGGL((q8_gemv_kernel<3>), grid, dim3(256), 0, s, x, w, bias, out, M, N, K, act); break;
        default: hipLaunchKernelGGL((q8_gemv_kernel<4>), grid, dim3(256), 0, s, x, w, bias, out, M, N, K, act); break;
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
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kQ8Block; i++) {
        const float a = __builtin_fabsf(v[i]);
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float id = (d > 0.0f) ? 1.0f / d : 0.0f;
    uint8_t* o = dst + b * kQ8Bytes;
    const uint32_t h = float_to_half_bits(d);
    o[0] = (uint8_t)(h & 0xffu);
    o[1] = (uint8_t)(h >> 8);
#pragma unroll
    for (int i = 0; i < kQ8Block; i++) {
        const float t = __builtin_rintf(v[i] * id);
        // (int)lrintf(t) on the reference's x86-64 host: NaN and |t| >= 2^63
        // convert to LONG_MIN, whose low 32 bits are 0.  |t| exceeds 127 only
        // when id overflowed to inf (amax < 2^-121), so t is then +-inf or
        // NaN and q = 0; otherwise the clamp to [-127, 127] applies.
        const int q = (__builtin_fabsf(t) < 2147483648.0f) ? (int)__builtin_amdgcn_fmed3f(t, -127.0f, 127.0f) : 0;
        o[2 + i] = (uint8_t)(int8_t)q;
    }
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
