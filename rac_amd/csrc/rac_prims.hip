// rac_prims.hip — the remaining rac.h primitives (rac.h:101-250, 345-346) on
// gfx950: circular rotation, projection, polar/vectoring and the batch forms
// built from them.  Semantics follow the reference CPU library
// (rac_cpu.c:136-228, 275-288, 344-371): CORDIC where it uses CORDIC
// (rotation, vectoring), libm-style cosf/sinf where it uses them
// (projection, normalize, dot, coherence, DCT basis).
//
// These are not bandwidth-critical (scalars and small batches); one kernel,
// `prim_kernel`, evaluates any of them elementwise over a batch so every
// entry point is a single launch.
#include <hip/hip_runtime.h>
#include <math.h>
#include "rac_math.hpp"
#include "rac_internal.hpp"

namespace rac {

static __constant__ float g_atan24[24] = {
    kAtan[0], kAtan[1], kAtan[2], kAtan[3], kAtan[4], kAtan[5], kAtan[6], kAtan[7],
    kAtan[8], kAtan[9], kAtan[10], kAtan[11], kAtan[12], kAtan[13], kAtan[14], kAtan[15],
    kAtan[16], kAtan[17], kAtan[18], kAtan[19], kAtan[20], kAtan[21], kAtan[22], kAtan[23],
};
static __constant__ float g_khat25[25] = {
    kKhat[0], kKhat[1], kKhat[2], kKhat[3], kKhat[4], kKhat[5], kKhat[6], kKhat[7], kKhat[8],
    kKhat[9], kKhat[10], kKhat[11], kKhat[12], kKhat[13], kKhat[14], kKhat[15], kKhat[16],
    kKhat[17], kKhat[18], kKhat[19], kKhat[20], kKhat[21], kKhat[22], kKhat[23], kKhat[24],
};

// _cordic_rotate (rac_cpu.c:90-118) with a run-time iteration count;
// angles with |theta| >= 2^27 or +-inf return NaN (the reference's wrap
// loop does not terminate there).
__device__ void rotate_rt(float vx, float vy, float theta, int iters, float& ox, float& oy) {
    if (!(__builtin_fabsf(theta) < kWrapLimit)) {
        ox = oy = __builtin_nanf("");
        return;
    }
    while (theta > kPi) theta -= kTau;
    while (theta <= -kPi) theta += kTau;
    float x = vx, y = vy;
    if (theta > kPi * 0.5f) { x = -x; y = -y; theta -= kPi; }
    else if (theta < -kPi * 0.5f) { x = -x; y = -y; theta += kPi; }
    float angle = theta, scale = 1.0f;
    for (int i = 0; i < iters; i++) {
        const float d = (angle >= 0.0f) ? 1.0f : -1.0f;
        const float xn = x - d * y * scale;
        const float yn = y + d * x * scale;
        angle -= d * g_atan24[i];
        x = xn;
        y = yn;
        scale *= 0.5f;
    }
    ox = x;
    oy = y;
}

// rac_polar (rac_cpu.c:158-180): 16-step vectoring after a +-pi pre-rotation
// of left-half-plane vectors; mag = x * K_INV, angle = pre - z.
__device__ void polar16(float vx, float vy, float& mag, float& angle) {
    float pre = 0.0f;
    if (vx < 0.0f) {
        pre = (vy >= 0.0f) ? kPi : -kPi;
        vx = -vx;
        vy = -vy;
    }
    float x = vx, y = vy, z = 0.0f, scale = 1.0f;
    for (int i = 0; i < 16; i++) {
        const float d = (y < 0.0f) ? 1.0f : -1.0f;
        const float xn = x - d * y * scale;
        const float yn = y + d * x * scale;
        z += d * g_atan24[i];
        x = xn;
        y = yn;
        scale *= 0.5f;
    }
    mag = x * kKInv;
    angle = pre - z;
}

__device__ __forceinline__ float project(float vx, float vy, float theta) {   // rac_cpu.c:150-154
    return __builtin_fmaf(vx, cosf(theta), vy * sinf(theta));
}

__device__ __forceinline__ int clamp_prec(int iters) {   // rac_cpu.c:54-58
    return iters < 4 ? 4 : (iters > 24 ? 24 : iters);
}

// One primitive per element i.  a, b: float2 arrays (x, y interleaved) or
// scalars; th: angles; out: float2 (o2) or float (o1) results.
__global__ void prim_kernel(int op, long n, const float2* __restrict__ a, const float2* __restrict__ b,
                            const float* __restrict__ th, int iarg, float2* __restrict__ o2,
                            float* __restrict__ o1) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float x, y, m, ang, mb, ab;
    switch (op) {
    case kPrimRotate:        // rac_rotate: (v * K_INV) rotated, 16 steps
        rotate_rt(a[i].x * kKInv, a[i].y * kKInv, th[i], 16, x, y);
        o2[i] = make_float2(x, y);
        break;
    case kPrimRotateRaw:
        rotate_rt(a[i].x, a[i].y, th[i], 16, x, y);
        o2[i] = make_float2(x, y);
        break;
    case kPrimCompensate: {  // rac_cpu.c:145-148
        const float c = powf(kKInv, (float)iarg);
        o2[i] = make_float2(a[i].x * c, a[i].y * c);
        break;
    }
    case kPrimProject:
        o1[i] = project(a[i].x, a[i].y, th[i]);
        break;
    case kPrimPolar:
        polar16(a[i].x, a[i].y, m, ang);
        o2[i] = make_float2(m, ang);
        break;
    case kPrimNormalize:     // rac_cpu.c:188-192
        polar16(a[i].x, a[i].y, m, ang);
        o2[i] = make_float2(cosf(ang), sinf(ang));
        break;
    case kPrimDot:           // rac_cpu.c:196-201
        polar16(a[i].x, a[i].y, m, ang);
        polar16(b[i].x, b[i].y, mb, ab);
        o1[i] = m * mb * cosf(ang - ab);
        break;
    case kPrimCoherence:
        polar16(a[i].x, a[i].y, m, ang);
        polar16(b[i].x, b[i].y, mb, ab);
        o1[i] = cosf(ang - ab);
        break;
    case kPrimComplexMul:    // rac_cpu.c:212-217
        polar16(b[i].x, b[i].y, mb, ab);
        rotate_rt(a[i].x * kKInv, a[i].y * kKInv, ab, 16, x, y);
        o2[i] = make_float2(x * mb, y * mb);
        break;
    case kPrimRotateN: {     // rac_rotate_n (rac_cpu.c:275-280)
        const int it = clamp_prec(iarg);
        const float kinv = 1.0f / g_khat25[it];
        rotate_rt(a[i].x * kinv, a[i].y * kinv, th[i], it, x, y);
        o2[i] = make_float2(x, y);
        break;
    }
    case kPrimProjectN: {    // rac_project_n (rac_cpu.c:282-288)
        const int it = clamp_prec(iarg);
        rotate_rt(1.0f / g_khat25[it], 0.0f, th[i], it, x, y);
        o1[i] = __builtin_fmaf(a[i].x, x, a[i].y * y);
        break;
    }
    case kPrimInnerTerm:     // rac_inner's term: project(a, angle b) * |b|
        polar16(b[i].x, b[i].y, mb, ab);
        o1[i] = project(a[i].x, a[i].y, ab) * mb;
        break;
    default:
        break;
    }
}

// rac_outer (rac_cpu.c:362-371): C[i][j] = project(a[i], angle(b[j])) * |b[j]|.
__global__ void outer_kernel(const float2* __restrict__ a, const float2* __restrict__ b,
                             float* __restrict__ C, int m, int n) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)m * n) return;
    const int i = (int)(idx / n), j = (int)(idx % n);
    float mb, ab;
    polar16(b[j].x, b[j].y, mb, ab);
    C[idx] = project(a[i].x, a[i].y, ab) * mb;
}

// rac_dct (rac_cpu.c:219-228): X[k] = sum_i project((x[i], 0), theta_ik),
// theta = RAC_PI * (2i+1) * k / (2n), summed in order i = 0..n-1.
__global__ void dct_kernel(const float* __restrict__ x, float* __restrict__ X, int n) {
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= n) return;
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        const float theta = kPi * (float)(2 * i + 1) * (float)k / (float)(2 * n);
        sum += project(x[i], 0.0f, theta);
    }
    X[k] = sum;
}

// rac_inner (rac_cpu.c:351-360): one workgroup sums the n terms
// project(a[i], angle b[i]) * |b[i]| as lane-strided partial sums combined
// by a fixed tree (the reference's OpenMP reduction order is not fixed
// either; results agree to float rounding of the sum).
__global__ __launch_bounds__(256) void inner_kernel(const float2* __restrict__ a,
                                                    const float2* __restrict__ b, long n,
                                                    float* __restrict__ out) {
    __shared__ float red[4];
    float acc = 0.0f;
    for (long i = threadIdx.x; i < n; i += 256) {
        float mb, ab;
        polar16(b[i].x, b[i].y, mb, ab);
        acc += project(a[i].x, a[i].y, ab) * mb;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[0] = (red[0] + red[1]) + (red[2] + red[3]);
}

hipError_t prim_launch(int op, long n, const float2* a, const float2* b, const float* th, int iarg,
                       float2* o2, float* o1, hipStream_t s) {
    hipLaunchKernelGGL(prim_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, op, n, a, b, th,
                       iarg, o2, o1);
    return hipGetLastError();
}

hipError_t outer_launch(const float2* a, const float2* b, float* C, int m, int n, hipStream_t s) {
    const long total = (long)m * n;
    hipLaunchKernelGGL(outer_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a, b, C, m, n);
    return hipGetLastError();
}

hipError_t dct_launch(const float* x, float* X, int n, hipStream_t s) {
    hipLaunchKernelGGL(dct_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, X, n);
    return hipGetLastError();
}

hipError_t inner_launch(const float2* a, const float2* b, long n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(inner_kernel, dim3(1), dim3(256), 0, s, a, b, n, out);
    return hipGetLastError();
}

}  // namespace rac
