// rac_internal.hpp — launchers shared between the kernel files and the C-ABI
// shim (rac_capi.hip).  Every launcher validates nothing: the shim checks
// arguments before calling and returns the launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

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

// Fused epilogue of the linear layer: v = acc (+ bias[n]); pre[m, n] = v when
// pre != null; C = act(v) with the activation ids of rac_act.hpp; khinv is
// 1/K_h of the SiLU's CORDIC exp at the launch's iteration count.
struct GemmEpilogue {
    const float* bias = nullptr;
    float* pre = nullptr;
    int act = 0;
    float khinv = 0.0f;
};
// C[M,N] = act(A[M,K] W[N,K]^T + bias) in one launch.
hipError_t gemm_fused_launch(const float* A, const float* W, float* C, int M, int N, int K,
                             const GemmEpilogue& ep, int iters, int mode, hipStream_t s);
// d[i] = g[i] * act'(pre[i]) (rac_torch.cu:680-694).
hipError_t act_grad_launch(const float* g, const float* pre, float* d, long count, int act, int iters,
                           hipStream_t s);

// batch > 1: C_z = alpha op(A_z) op(B_z) + beta C_z for z < batch, with
// A_z = A + z*sa, B_z = B + z*sb, C_z = C + z*sc (element strides).
// sched 1 (square M == N): only output tiles on or below the diagonal are
// computed (causal attention scores; the tiles above are left unwritten).
// sched 2: each workgroup computes row tiles p and nt-1-p (balances the
// causal P V below).  sched 3 (NT): output rows are query positions
// row0 .. row0+M-1 and columns key positions; tiles wholly above the
// diagonal are skipped (left unwritten).  k_causal: device flag; when it
// holds 1, row tile m sums k only up to its last query position
// row0 + m*BM + BM - 1 (causal P V with a lower-triangular P and finite V).
// exact_specials (CORDIC mode): tiles whose A panel holds
// values outside the strength-reduced rotation chain's range are recomputed
// on the literal chain, so every input gives the reference's bits; false
// keeps the strength-reduced chain for every input (callers whose parity
// bar is a summation bound, where subnormal-rounding differences of tiny
// products are far below it).
// The same product for M <= 16 rows or N <= 16 columns, A row-major (not
// transposed): gemm_launch hands such launches (schedules 0 and 2) to the
// few-row / few-column kernels.
struct SkinnyArgs {
    const float* A;
    const float* B;
    float* C;
    int M, N, K;
    float alpha, beta;
    int iters;                 // clamped
    int batch;
    long sa, sb, sc;
    GemmEpilogue ep;
    bool fused;
    bool tb;
    const int* k_causal;
    int exact_specials;
    int row0;
};
hipError_t gemm_skinny_launch(const SkinnyArgs& g, int mode, hipStream_t s);
// Compute units of the current device (256 on MI355X), cached per device.
long device_cus();
constexpr int kSkinnyMaxRows = 16;      // and columns

hipError_t gemm_launch(int ta, int tb, const float* A, const float* B, float* C,
                       int M, int N, int K, float alpha, float beta, int iters, int mode,
                       hipStream_t s, int batch = 1, long sa = 0, long sb = 0, long sc = 0,
                       int sched = 0, const int* k_causal = nullptr, bool exact_specials = true,
                       int row0 = 0);
// *flag = 1 if every x[i] is finite, else 0 (stream-ordered).
hipError_t all_finite_launch(const float* x, long n, int* flag, hipStream_t s);

// Optional attention masking of each row r (query position t = row0 +
// r % seq, column j): causal -> x = -inf for j > t; then x += mask[t*ld + j]
// when mask != null (ld = mask_ld, or the row length when 0).  zero_guard:
// 1/sum replaced by 0 when sum is not > 0 (rac_cpu.c:687).  x and y may be
// the same buffer (in-place softmax).
struct SoftmaxMask {
    const float* mask = nullptr;
    int causal = 0;
    long seq = 0;
    int zero_guard = 0;
    long row0 = 0;
    long mask_ld = 0;
};
hipError_t softmax_launch(const float* x, float* y, long rows, long n, int iters,
                          hipStream_t s, const SoftmaxMask& mk = SoftmaxMask());
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
// Out of place: rows read at x (strides sb, sh, st), written at y (ob, oh, ot).
hipError_t rope_apply_out_launch(const float* x, float* y, const float* cos_tab, const float* sin_tab,
                                 int batch, int heads, int seq, int head_dim, long sb, long sh, long st,
                                 long ob, long oh, long ot, hipStream_t s);
hipError_t rsqrt_launch(const float* x, float* y, long count, hipStream_t s);

enum PrimOp {
    kPrimRotate = 0, kPrimRotateRaw = 1, kPrimCompensate = 2, kPrimProject = 3, kPrimPolar = 4,
    kPrimNormalize = 5, kPrimDot = 6, kPrimCoherence = 7, kPrimComplexMul = 8, kPrimRotateN = 9,
    kPrimProjectN = 10, kPrimInnerTerm = 11
};
hipError_t prim_launch(int op, long n, const float2* a, const float2* b, const float* th, int iarg,
                       float2* o2, float* o1, hipStream_t s);
hipError_t outer_launch(const float2* a, const float2* b, float* C, int m, int n, hipStream_t s);
hipError_t dct_launch(const float* x, float* X, int n, hipStream_t s);
hipError_t inner_launch(const float2* a, const float2* b, long n, float* out, hipStream_t s);
// Q8_0 (34-byte blocks of 32 int8 + fp16 scale): out[M,N] = act(x[M,K] W^T
// + bias), W [N, K/32] blocks; quantize / dequantize nblocks blocks.
hipError_t q8_gemv_launch(const float* x, const uint8_t* w, const float* bias, float* out, int M, int N,
                          int K, int act, hipStream_t s);
hipError_t q8_quantize_launch(const float* src, uint8_t* dst, long nblocks, hipStream_t s);
// One-row GEMVs of the decode step with rmsnorm(x) * gamma as input (the
// fast layout only: K % 256 == 0, 16-byte aligned weights; else
// hipErrorInvalidValue): plain (out = act(W h + bias)); Q|K|V (rows below
// split to q_out, the next kvw rows to the key cache and the kvw after to
// the value cache at *pos); gate / up pairs (2 n_ff interleaved rows,
// out[i] = silu(gate_i) * up_i).
hipError_t q8_rmsnorm_gemv_launch(const float* x, const float* gamma, float eps, const uint8_t* w,
                                  const float* bias, float* out, int N, int K, int act, hipStream_t s);
hipError_t q8_decode_qkv_launch(const float* x, const float* gamma, float eps, const uint8_t* w, float* q_out,
                                int split, float* kc, float* vc, int kvw, int dh, long t_cap, const int* pos,
                                int K, hipStream_t s);
hipError_t q8_decode_swiglu_launch(const float* x, const float* gamma, float eps, const uint8_t* w, float* out,
                                   int n_ff, int K, int iters, hipStream_t s);
// Decode step of a decoder layer (rac_decode.hip): the token's cache
// position is read from *pos in device memory.  Attention: one workgroup
// per query head over positions 0 .. *pos of a cache [n_kv_heads, t_cap,
// d_head]; d_head <= kDecodeMaxHead, positions < kDecodeMaxLen.
constexpr int kDecodeMaxHead = 256;
constexpr int kDecodeMaxLen = 8192;
hipError_t decode_attention_launch(const float* q, const float* kc, const float* vc, float* out, int n_heads,
                                   int n_kv_heads, int dh, long t_cap, const int* pos, float scale, int iters,
                                   hipStream_t s);
hipError_t kv_append_launch(const float* kv, float* kc, float* vc, int n_kv_heads, int dh, long t_cap,
                            const int* pos, hipStream_t s);
hipError_t position_advance_launch(int* pos, int by, hipStream_t s);
hipError_t swiglu_launch(const float* gu, float* out, long n, int iters, hipStream_t s);
hipError_t q8_dequantize_launch(const uint8_t* src, float* dst, long nblocks, hipStream_t s);
// Error channel of the C ABI (rac_last_error): set the message, return code.
int report(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int report_hip(hipError_t e, const char* what);     // RAC_ERR_DEVICE (-4) unless hipSuccess
bool is_device_ptr(const void* p);

// safetensors element conversion (dtype codes of safetensors_reader.h:37-49).
hipError_t st_convert_launch(int dtype, const void* src, long n, float* dst, hipStream_t s);
hipError_t st_quantize_launch(int dtype, const void* src, long nblocks, uint8_t* dst, hipStream_t s);

// RAC-DSP integer CORDIC engine (sim/rac_dsp_core.h geometry).
constexpr int kDspLutBits = 10;
constexpr int kDspLut = 1 << kDspLutBits;
constexpr int kDspRes = 9;
constexpr int kDspResStart = 8;
constexpr int kDspAtan = kDspResStart + kDspRes;
struct DspRoms {
    uint16_t lut[kDspLut];        // 10-bit direction words
    int64_t coarse_z[kDspLut];    // angle the coarse stage applies for each word:
                                  // wrapping sum of +-atan_rom[i] by its bits
    int64_t atan_rom[kDspAtan];   // atan(2^-i), Q0.63 fractions of pi
    int64_t atanh_rom[kDspRes];   // atanh(2^-(8+i)), same units
};
hipError_t dsp_eval_launch(int op, long n, const int64_t* x, const int64_t* y, const int64_t* z, int64_t* xo,
                           int64_t* yo, int64_t* zo, const DspRoms* roms, hipStream_t s);
hipError_t dsp_systolic_launch(int N, int K, const int64_t* W, const int64_t* X, int64_t* Y, const DspRoms* roms,
                               hipStream_t s);
hipError_t sincos_launch(const float* theta, float* s_out, float* c_out, long count,
                         hipStream_t s);

}  // namespace rac
