// rac_internal.hpp — launchers shared between the kernel files and the C-ABI
// shim (rac_capi.hip).  Every launcher validates nothing: the shim checks
// arguments before calling and returns the launch status.
#pragma once
#include <hip/hip_runtime.h>

namespace rac {

constexpr int kModeFast = 0;      // rac_kernels.hip:23
constexpr int kModeCordic = 1;
constexpr int kModeShiftAdd = 2;

inline int clamp_iters(int iters) {   // rac_kernels.hip:816-820
    return iters < 1 ? 1 : (iters > 24 ? 24 : iters);
}

// Host-side constants computed once (double precision, rounded once).
struct HostConsts {
    float exp_khinv[25];   // 1/K_h(n) of the first n Walther steps, n = 1..24
    float rsqrt_khinv;     // 1/K_h over the rsqrt's 16 steps
};
const HostConsts& host_consts();

hipError_t gemm_launch(int ta, int tb, const float* A, const float* B, float* C,
                       int M, int N, int K, float alpha, float beta, int iters, int mode,
                       hipStream_t s);

hipError_t softmax_launch(const float* x, float* y, long rows, long n, int iters,
                          hipStream_t s);
hipError_t rmsnorm_launch(const float* x, float* y, const float* gamma, float eps,
                          long rows, long d, hipStream_t s);
hipError_t layernorm_launch(const float* x, float* y, const float* gamma, const float* beta,
                            float eps, long rows, long d, hipStream_t s);

enum EltOp { kEltExp = 0, kEltSilu = 1, kEltSigmoid = 2, kEltTanh = 3, kEltGelu = 4, kEltRelu = 5 };
hipError_t eltwise_launch(int op, const float* x, float* y, long count, int iters,
                          hipStream_t s);

hipError_t rope_cache_launch(float* cos_out, float* sin_out, const float* inv_freq,
                             int max_seq, int half, hipStream_t s);
hipError_t rope_apply_launch(float* x, const float* cos_tab, const float* sin_tab,
                             int batch, int heads, int seq, int head_dim,
                             long sb, long sh, long st, hipStream_t s);
hipError_t rsqrt_launch(const float* x, float* y, long count, hipStream_t s);
hipError_t sincos_launch(const float* theta, float* s_out, float* c_out, long count,
                         hipStream_t s);

}  // namespace rac
