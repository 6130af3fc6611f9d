// K-split partials of the skinny W8A8 GEMM handed to the next kernel of a
// fused chain, which folds them while it reads its input instead of a fold
// launch of their own (one kernel boundary less per GEMM).
//
// The folded value of output (row, col) is the one the GEMM epilogue stores:
//   acc = sum over j < ksplit of part[j * m * n + row * n + col]  (int32,
//         exact in any order: |acc| <= 127 * 127 * K < 2^31 for K <= 131071)
//   s   = f32(*sa_dev * sb_vec[col])   (device activation scale, per-channel
//                                       weight scales)
//   y   = T(f32(acc * s))              (two f32 roundings, then one to T)
// With a residual `res` (T [m, n], a decode layer's residual stream), the
// folded value is T(f32(y) + f32(res[row, col])): the GEMM output as stored,
// then the residual add of a transformer block, rounded once more.
#pragma once

#include "ft_common.hpp"

namespace ft {

struct KFold {
    const int* part = nullptr;
    int ksplit = 0;  // 0: the GEMM was not split and stored y itself
    int n = 0;
    long long mn = 0;
    const float* sa_dev = nullptr;
    const float* sb_vec = nullptr;
    const void* res = nullptr;  // optional residual added after the epilogue
};

// Runs y[m, n] = A[m, k] . B[n, k]^T (int8; device activation scale *sa_dev,
// per-channel weight scales sb_vec; y_dtype FT_DT_F32 / BF16 / F16) as
// ft_qgemm_launch_ex does. When the dispatch splits K over workgroups, the
// int32 partials are left in the library's GEMM scratch, `f` describes them
// and the result is true: the caller's next launch on stream s must fold
// them (before any other GEMM reuses that scratch). Otherwise y is written
// and the result is false. qgemm.hip.
bool qgemm_deferred(const signed char* a, const signed char* b, const float* sa_dev,
                    const float* sb_vec, void* y, int y_dtype, int m, int n, int k,
                    hipStream_t s, KFold& f);

// The gate/up GEMM of swiglu_quant: y [m, 2 inter] = A . B^T as
// ft_qgemm_launch_ex writes it (B: inter gate rows, then inter up rows).
// Where the dispatch would run it unsplit on the skinny ring kernel, that
// kernel also takes each workgroup's max |silu(g) * u| over the stored
// values: part[0 .. nparts) (library scratch, valid until the next scratch
// user on stream s) and the result is 1. With q (codes [m, inter]) and
// scale_out given, and every workgroup resident at once, the kernel folds
// the maxima itself and writes swiglu_quant's codes and scale: result 2
// (y may then be null: not stored). Otherwise nothing is launched and the
// result is 0. qgemm.hip.
// The K-split partials `f` (ksplit >= 2) of a GEMM folded into y [m, n]
// (dtype FT_DT_*), plus f.res when non-null: one launch. qgemm.hip.
void kfold_store(const KFold& f, void* y, int dtype, int m, hipStream_t s);

int qgemm_swiglu_max(const signed char* a, const signed char* b, const float* sa_dev,
                     const float* sb_vec, void* y, int y_dtype, int m, int inter, int k,
                     hipStream_t s, float*& part, int& nparts, signed char* q = nullptr,
                     float* scale_out = nullptr);

// rmsnorm_quant (no residual) of a K-split GEMM's output still held as its
// partials: the row pass folds them and stores the rows into x_out (as the
// GEMM epilogue would), then the codes and the device scale; the same bits
// as the fold launch followed by rmsnorm_quant. dtype FT_DT_*. fused.hip.
void rmsnorm_quant_folded(int dtype, const KFold& fold, void* x_out, const float* w,
                          signed char* q, float* scale_out, int rows, int cols, float eps,
                          hipStream_t s);

// o_proj GEMM + rmsnorm_quant(y + residual) as ft_qgemm_rmsnorm_quant_launch,
// plus the residual stream h_out = T(y + residual) (the two roundings of a
// transformer block's residual add); y itself is stored only where the
// two-launch form needs it. fused.hip.
void qgemm_rmsnorm_quant_res(int dtype, const signed char* a_q, const float* sa_dev,
                             const signed char* w_q, const float* w_scales, void* y,
                             const void* residual,
                             const float* w, float eps, signed char* q, float* scale_out,
                             void* h_out, int rows, int n, int k, hipStream_t s);

// ft_qgemm_swiglu_quant_launch where h [rows, 2 inter] is scratch the
// caller does not read: the one-launch form (gate/up GEMM + SwiGLU maxima
// folded with grid_max + codes) skips storing it. fused.hip.
void qgemm_swiglu_quant_codes(int dtype, const signed char* a_q, const float* sa_dev,
                              const signed char* w_gu, const float* w_scales, void* h,
                              signed char* q, float* scale_out, int rows, int inter, int k,
                              hipStream_t s);

// y = T(f32(y) + f32(h)) over n elements (n % 4 == 0). fused.hip.
void residual_add(int dtype, void* y, const void* h, long long n, hipStream_t s);

__device__ __forceinline__ float kfold_sa(const KFold& f) { return *f.sa_dev; }

// composed scale of column col (one f32 rounding)
__device__ __forceinline__ float kfold_scale(const KFold& f, float sa, int col) {
    return sa * f.sb_vec[col];
}

// the stored value widened back to f32 (T = float: the f32 product itself)
template <typename T>
__device__ __forceinline__ float kfold_value(int acc, float s) {
    float v = (float)acc * s;
    asm("" : "+v"(v));  // rounded to f32 before the narrowing, never fused
    return (float)(T)v;
}

// the residual add of a folded value v (f32 of the stored T): T(v + r)
template <typename T>
__device__ __forceinline__ float kfold_add_res(float v, float r) {
    return (float)(T)(v + r);
}

// Fold widths: a kernel instantiated with FK = 4 or 8 loads all partials
// of an output in one batch of FK loads (ksplit <= FK; partial indices past
// ksplit are clamped and their values dropped by a select after the load,
// no branch between loads), so every load of a thread shares one memory
// round trip; FK = 1 loops over batches of 8 (any ksplit); FK = 0: no fold.
inline int kfold_width(int ksplit) { return ksplit <= 4 ? 4 : ksplit <= 8 ? 8 : 1; }

// int32 sum over the partials of output idx = row * n + col
template <int FK>
__device__ __forceinline__ int kfold_sum(const KFold& f, size_t idx) {
    constexpr int W = FK == 1 ? 8 : FK;
    int s = 0;
    for (int j0 = 0; j0 < (FK == 1 ? f.ksplit : 1); j0 += W) {
        int v[W];
#pragma unroll
        for (int u = 0; u < W; ++u)
            v[u] = f.part[(size_t)min(j0 + u, f.ksplit - 1) * f.mn + idx];
#pragma unroll
        for (int u = 0; u < W; ++u) s += j0 + u < f.ksplit ? v[u] : 0;
    }
    return s;
}

// four consecutive outputs idx .. idx + 3 (idx % 4 == 0, n % 4 == 0)
template <int FK>
__device__ __forceinline__ int4 kfold_sum4(const KFold& f, size_t idx) {
    constexpr int W = FK == 1 ? 8 : FK;
    int4 s = make_int4(0, 0, 0, 0);
    for (int j0 = 0; j0 < (FK == 1 ? f.ksplit : 1); j0 += W) {
        int4 v[W];
#pragma unroll
        for (int u = 0; u < W; ++u)
            v[u] = *reinterpret_cast<const int4*>(
                f.part + (size_t)min(j0 + u, f.ksplit - 1) * f.mn + idx);
#pragma unroll
        for (int u = 0; u < W; ++u) {
            const bool live = j0 + u < f.ksplit;
            s.x += live ? v[u].x : 0;
            s.y += live ? v[u].y : 0;
            s.z += live ? v[u].z : 0;
            s.w += live ? v[u].w : 0;
        }
    }
    return s;
}

}  // namespace ft
