// RMSNorm (+residual), RoPE (interleaved / NeoX, position offset) and
// SwiGLU for gfx950. All compute in float32 (RoPE angles in float64);
// storage f32 / bf16 / fp16.
//
// Reference semantics:
//   rmsnorm  rmsnorm.cu:110-130   y = (x+r) * (1/sqrt(sum((x+r)^2)/cols + eps)) * w
//   rope     rope.cu:96-143       angle = m * theta^(-2j/dim) in double,
//                                 rotation in double, rounded to f32
//   swiglu   activations.cu:501-511  y = g / (1 + exp(-g)) * u
#include "ft_common.hpp"

#include <cmath>

namespace ft {
namespace {

// ---------------------------------------------------------------------------
// RMSNorm: one workgroup per row. Each thread owns 4-element chunks
// c = tid, tid + NT, ... (vector path) and sums their squares in order;
// the wave butterfly and the cross-wave sum are fixed, so the result is
// deterministic for a given (cols, NT). The second pass re-reads the row
// (L2-resident: a row is at most a few tens of KB).
// ---------------------------------------------------------------------------
template <typename T, int NT, bool VEC>
__global__ __launch_bounds__(NT) void rmsnorm_kernel(
    const T* __restrict__ x, const T* __restrict__ r,
    const float* __restrict__ w, T* __restrict__ y, int cols, float eps) {
    __shared__ float red[NT / 64];
    const size_t base = (size_t)blockIdx.x * cols;
    const T* xr = x + base;
    const T* rr = r ? r + base : nullptr;
    T* yr = y + base;
    float acc = 0.0f;
    if (VEC) {
        const int chunks = cols >> 2;
        for (int c = threadIdx.x; c < chunks; c += NT) {
            float4 v = St<T>::ld4(xr + 4 * c);
            if (rr) {
                const float4 b = St<T>::ld4(rr + 4 * c);
                v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
            }
            acc = fmaf(v.x, v.x, acc);
            acc = fmaf(v.y, v.y, acc);
            acc = fmaf(v.z, v.z, acc);
            acc = fmaf(v.w, v.w, acc);
        }
    } else {
        for (int i = threadIdx.x; i < cols; i += NT) {
            const float v = St<T>::ld(xr + i) + (rr ? St<T>::ld(rr + i) : 0.0f);
            acc = fmaf(v, v, acc);
        }
    }
    const float total = block_sum<NT>(acc, red);
    const float inv = 1.0f / sqrtf(total / (float)cols + eps);
    if (VEC) {
        const int chunks = cols >> 2;
        for (int c = threadIdx.x; c < chunks; c += NT) {
            float4 v = St<T>::ld4(xr + 4 * c);
            if (rr) {
                const float4 b = St<T>::ld4(rr + 4 * c);
                v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
            }
            const float4 wv = *reinterpret_cast<const float4*>(w + 4 * c);
            St<T>::st4(yr + 4 * c,
                       make_float4(v.x * inv * wv.x, v.y * inv * wv.y,
                                   v.z * inv * wv.z, v.w * inv * wv.w));
        }
    } else {
        for (int i = threadIdx.x; i < cols; i += NT) {
            const float v = St<T>::ld(xr + i) + (rr ? St<T>::ld(rr + i) : 0.0f);
            St<T>::st(yr + i, v * inv * w[i]);
        }
    }
}

template <typename T>
bool aligned_for_vec(const void* p) {
    const size_t need = 4 * sizeof(T);
    return ((uintptr_t)p % need) == 0;
}

template <typename T>
void rmsnorm_run(const T* x, const float* w, const T* r, T* y, int rows,
                 int cols, float eps, hipStream_t s) {
    if (rows < 0 || cols <= 0)
        inval("rows must be >= 0 and cols must be > 0");
    if (rows == 0) return;
    if (!x || !w || !y) inval("rmsnorm: null operand");
    const bool vec = (cols % 4 == 0) && aligned_for_vec<T>(x) &&
                     aligned_for_vec<float>(w) && aligned_for_vec<T>(y) &&
                     (!r || aligned_for_vec<T>(r));
    constexpr int NT = 256;
    if (vec)
        rmsnorm_kernel<T, NT, true><<<rows, NT, 0, s>>>(x, r, w, y, cols, eps);
    else
        rmsnorm_kernel<T, NT, false><<<rows, NT, 0, s>>>(x, r, w, y, cols, eps);
    launch_check("rmsnorm kernel launch");
}

// ---------------------------------------------------------------------------
// RoPE: one thread per (row, pair). The angle is computed in float64
// (m * theta^(-2j/dim)), as are cos/sin and the rotation, then rounded to
// float32 once: at position 8192 an f32 angle would already be ~5e-4 rad
// off. Row r's position is base(r) + pos_offset, where base(r) is
// positions[r / rows_per_pos] when a device position table is given and
// r / rows_per_pos otherwise (rows_per_pos = 1 is the reference's
// "row r sits at r + pos_offset").
// ---------------------------------------------------------------------------
template <typename T, bool NEOX>
__global__ __launch_bounds__(256) void rope_kernel(
    const T* __restrict__ x, T* __restrict__ y, long long rows, int dim,
    double theta, int pos_offset, const int* __restrict__ positions,
    int rows_per_pos) {
    const int half = dim >> 1;
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= rows * half) return;
    const long long row = p / half;
    const int j = (int)(p - row * half);
    const long long pos_base = row / rows_per_pos;
    const long long m =
        (positions ? (long long)positions[pos_base] : pos_base) + pos_offset;
    const double angle = (double)m * pow(theta, -2.0 * j / dim);
    double sn, cs;
    sincos(angle, &sn, &cs);
    const long long i1 = row * dim + (NEOX ? j : 2 * j);
    const long long i2 = i1 + (NEOX ? half : 1);
    const float x1 = St<T>::ld(x + i1);
    const float x2 = St<T>::ld(x + i2);
    St<T>::st(y + i1, (float)(x1 * cs - x2 * sn));
    St<T>::st(y + i2, (float)(x1 * sn + x2 * cs));
}

template <typename T>
void rope_run(const T* x, T* y, long long rows, int dim, float theta,
              int pos_offset, const int* positions, int rows_per_pos,
              bool neox, hipStream_t s) {
    if (rows < 0 || dim <= 0) inval("seq must be >= 0 and dim must be > 0");
    if (dim % 2 != 0) inval("dim must be even (RoPE pairs elements)");
    if (pos_offset < 0) inval("pos_offset must be >= 0");
    if (rows_per_pos < 1) inval("rows_per_pos must be >= 1");
    if (rows == 0) return;
    if (!x || !y) inval("rope: null operand");
    const long long pairs = rows * (dim / 2);
    const unsigned grid = (unsigned)((pairs + 255) / 256);
    if (neox)
        rope_kernel<T, true><<<grid, 256, 0, s>>>(x, y, rows, dim, (double)theta,
                                                 pos_offset, positions,
                                                 rows_per_pos);
    else
        rope_kernel<T, false><<<grid, 256, 0, s>>>(x, y, rows, dim, (double)theta,
                                                  pos_offset, positions,
                                                  rows_per_pos);
    launch_check("rope kernel launch");
}

// ---------------------------------------------------------------------------
// SwiGLU: grid-stride over 4-element chunks (16 B of f32 / 8 B of halves per
// operand per thread), scalar path for misaligned views and the tail.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float swiglu_f(float g, float u) {
    return g / (1.0f + expf(-g)) * u;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void swiglu_kernel(
    const T* __restrict__ g, const T* __restrict__ u, T* __restrict__ y,
    long long n) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        const long long n4 = n >> 2;
        for (long long c = i; c < n4; c += stride) {
            const float4 a = St<T>::ld4(g + 4 * c);
            const float4 b = St<T>::ld4(u + 4 * c);
            St<T>::st4(y + 4 * c,
                       make_float4(swiglu_f(a.x, b.x), swiglu_f(a.y, b.y),
                                   swiglu_f(a.z, b.z), swiglu_f(a.w, b.w)));
        }
        for (long long t = (n4 << 2) + i; t < n; t += stride)
            St<T>::st(y + t, swiglu_f(St<T>::ld(g + t), St<T>::ld(u + t)));
    } else {
        for (long long t = i; t < n; t += stride)
            St<T>::st(y + t, swiglu_f(St<T>::ld(g + t), St<T>::ld(u + t)));
    }
}

template <typename T>
void swiglu_run(const T* g, const T* u, T* y, long long n, hipStream_t s) {
    if (n < 0) inval("n must be >= 0");
    if (n == 0) return;
    if (!g || !u || !y) inval("swiglu: null operand");
    const bool vec = aligned_for_vec<T>(g) && aligned_for_vec<T>(u) &&
                     aligned_for_vec<T>(y);
    const unsigned grid = grid_1d((n + 3) / 4, 256, dev_info().cu_count * 16);
    if (vec)
        swiglu_kernel<T, true><<<grid, 256, 0, s>>>(g, u, y, n);
    else
        swiglu_kernel<T, false><<<grid, 256, 0, s>>>(g, u, y, n);
    launch_check("swiglu kernel launch");
}

}  // namespace
}  // namespace ft

using ft::bf16;
using ft::f16;

extern "C" {

int ft_rmsnorm_launch(const float* x, const float* w, const float* r,
                      float* y, int rows, int cols, float eps,
                      uintptr_t stream) {
    return ft::guarded([&] {
        ft::rmsnorm_run<float>(x, w, r, y, rows, cols, eps, ft::as_stream(stream));
    });
}

int ft_rmsnorm_launch_bf16(const void* x, const float* w, const void* r,
                           void* y, int rows, int cols, float eps,
                           uintptr_t stream) {
    return ft::guarded([&] {
        ft::rmsnorm_run<bf16>((const bf16*)x, w, (const bf16*)r, (bf16*)y, rows,
                              cols, eps, ft::as_stream(stream));
    });
}

int ft_rmsnorm_launch_fp16(const void* x, const float* w, const void* r,
                           void* y, int rows, int cols, float eps,
                           uintptr_t stream) {
    return ft::guarded([&] {
        ft::rmsnorm_run<f16>((const f16*)x, w, (const f16*)r, (f16*)y, rows,
                             cols, eps, ft::as_stream(stream));
    });
}

int ft_rope_launch(const float* x, float* y, int seq, int dim, float theta,
                   int pos_offset, uintptr_t stream) {
    return ft::guarded([&] {
        ft::rope_run<float>(x, y, seq, dim, theta, pos_offset, nullptr, 1, false,
                            ft::as_stream(stream));
    });
}

int ft_rope_neox_launch(const float* x, float* y, int seq, int dim,
                        float theta, int pos_offset, uintptr_t stream) {
    return ft::guarded([&] {
        ft::rope_run<float>(x, y, seq, dim, theta, pos_offset, nullptr, 1, true,
                            ft::as_stream(stream));
    });
}

int ft_rope_launch_bf16(const void* x, void* y, int seq, int dim,
                        float theta, int pos_offset, uintptr_t stream) {
    return ft::guarded([&] {
        ft::rope_run<bf16>((const bf16*)x, (bf16*)y, seq, dim, theta, pos_offset,
                           nullptr, 1, false, ft::as_stream(stream));
    });
}

int ft_rope_neox_launch_bf16(const void* x, void* y, int seq, int dim,
                             float theta, int pos_offset, uintptr_t stream) {
    return ft::guarded([&] {
        ft::rope_run<bf16>((const bf16*)x, (bf16*)y, seq, dim, theta, pos_offset,
                           nullptr, 1, true, ft::as_stream(stream));
    });
}

int ft_rope_launch_fp16(const void* x, void* y, int seq, int dim,
                        float theta, int pos_offset, uintptr_t stream) {
    return ft::guarded([&] {
        ft::rope_run<f16>((const f16*)x, (f16*)y, seq, dim, theta, pos_offset,
                          nullptr, 1, false, ft::as_stream(stream));
    });
}

int ft_rope_neox_launch_fp16(const void* x, void* y, int seq, int dim,
                             float theta, int pos_offset, uintptr_t stream) {
    return ft::guarded([&] {
        ft::rope_run<f16>((const f16*)x, (f16*)y, seq, dim, theta, pos_offset,
                          nullptr, 1, true, ft::as_stream(stream));
    });
}

int ft_rope_launch_ex(const void* x, void* y, int dtype, long long rows,
                      int dim, float theta, int pos_offset,
                      const int* positions, int rows_per_pos, int neox,
                      uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
        switch (dtype) {
        case FT_DT_F32:
            ft::rope_run<float>((const float*)x, (float*)y, rows, dim, theta,
                                pos_offset, positions, rows_per_pos, neox != 0, s);
            break;
        case FT_DT_BF16:
            ft::rope_run<bf16>((const bf16*)x, (bf16*)y, rows, dim, theta,
                               pos_offset, positions, rows_per_pos, neox != 0, s);
            break;
        case FT_DT_F16:
            ft::rope_run<f16>((const f16*)x, (f16*)y, rows, dim, theta,
                              pos_offset, positions, rows_per_pos, neox != 0, s);
            break;
        default:
            ft::inval("rope: unknown dtype code");
        }
    });
}

int ft_swiglu_launch(const float* gate, const float* up, float* y,
                     long long n, uintptr_t stream) {
    return ft::guarded([&] {
        ft::swiglu_run<float>(gate, up, y, n, ft::as_stream(stream));
    });
}

int ft_swiglu_launch_bf16(const void* gate, const void* up, void* y,
                          long long n, uintptr_t stream) {
    return ft::guarded([&] {
        ft::swiglu_run<bf16>((const bf16*)gate, (const bf16*)up, (bf16*)y, n,
                             ft::as_stream(stream));
    });
}

int ft_swiglu_launch_fp16(const void* gate, const void* up, void* y,
                          long long n, uintptr_t stream) {
    return ft::guarded([&] {
        ft::swiglu_run<f16>((const f16*)gate, (const f16*)up, (f16*)y, n,
                            ft::as_stream(stream));
    });
}

}  // extern "C"
