// Symmetric per-tensor INT8 quantize for gfx950, device-resident scale.
//
// Arithmetic (reference quantize.cu:153-186, bit-exact):
//   absmax = max |x|                (order-independent: exact)
//   scale  = absmax > 0 ? absmax / 127 : 1      (IEEE f32 divide)
//   inv    = 1 / scale                           (IEEE f32 divide)
//   q      = clamp(rint(x * inv), -127, 127)     (round half to even)
//
// The reference reads the absmax back to the host between its two kernels
// (quantize.cu:55-67,195-215). Here the scale never leaves the device:
//   n <= kSmallN : one 1024-thread workgroup reduces, writes the scale and
//                  quantizes (x re-read from L2);
//   otherwise    : pass 1 writes one partial max per workgroup into library
//                  scratch; pass 2 has every workgroup fold those partials
//                  (identical result everywhere), quantize its share, and
//                  workgroup 0 store the scale.
// No memset, no atomics, no host sync: stream-ordered and capturable.
#include "ft_common.hpp"

namespace ft {
namespace {

constexpr long long kSmallN = 1 << 16;
constexpr int kPass1Blocks = 1024;

__device__ __forceinline__ float make_scale(float absmax) {
    return absmax > 0.0f ? absmax / 127.0f : 1.0f;
}

__device__ __forceinline__ signed char quant1(float x, float inv) {
    return (signed char)fmaxf(-127.0f, fminf(127.0f, rintf(x * inv)));
}

// Load 4 consecutive elements widened to float (exact for every type).
template <typename T>
__device__ __forceinline__ float4 ld4w(const T* p) { return St<T>::ld4(p); }

template <typename T, bool VEC>
__device__ __forceinline__ float local_absmax(const T* __restrict__ x,
                                              long long n, long long tid,
                                              long long stride) {
    float m = 0.0f;
    if (VEC) {
        const long long n4 = n >> 2;
        for (long long c = tid; c < n4; c += stride) {
            const float4 v = ld4w(x + 4 * c);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)),
                               fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        for (long long i = (n4 << 2) + tid; i < n; i += stride)
            m = fmaxf(m, fabsf(St<T>::ld(x + i)));
    } else {
        for (long long i = tid; i < n; i += stride)
            m = fmaxf(m, fabsf(St<T>::ld(x + i)));
    }
    return m;
}

template <typename T, bool VEC>
__device__ __forceinline__ void quantize_range(const T* __restrict__ x,
                                               signed char* __restrict__ q,
                                               long long n, float inv,
                                               long long tid,
                                               long long stride) {
    if (VEC) {
        const long long n4 = n >> 2;
        for (long long c = tid; c < n4; c += stride) {
            const float4 v = ld4w(x + 4 * c);
            char4 o;
            o.x = quant1(v.x, inv);
            o.y = quant1(v.y, inv);
            o.z = quant1(v.z, inv);
            o.w = quant1(v.w, inv);
            *reinterpret_cast<char4*>(q + 4 * c) = o;
        }
        for (long long i = (n4 << 2) + tid; i < n; i += stride)
            q[i] = quant1(St<T>::ld(x + i), inv);
    } else {
        for (long long i = tid; i < n; i += stride)
            q[i] = quant1(St<T>::ld(x + i), inv);
    }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(1024) void quantize_small_kernel(
    const T* __restrict__ x, signed char* __restrict__ q,
    float* __restrict__ scale_out, long long n) {
    __shared__ float red[16];
    const float m = block_max<1024>(
        local_absmax<T, VEC>(x, n, threadIdx.x, 1024), red);
    const float scale = make_scale(m);
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) *scale_out = scale;
    quantize_range<T, VEC>(x, q, n, inv, threadIdx.x, 1024);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void absmax_partial_kernel(
    const T* __restrict__ x, float* __restrict__ partial, long long n) {
    __shared__ float red[4];
    const long long tid = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long stride = (long long)gridDim.x * 256;
    const float m = block_max<256>(local_absmax<T, VEC>(x, n, tid, stride), red);
    if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void quantize_fold_kernel(
    const T* __restrict__ x, signed char* __restrict__ q,
    const float* __restrict__ partial, int nparts,
    float* __restrict__ scale_out, long long n) {
    __shared__ float red[4];
    float m = 0.0f;
    for (int i = threadIdx.x; i < nparts; i += 256) m = fmaxf(m, partial[i]);
    m = block_max<256>(m, red);
    const float scale = make_scale(m);
    const float inv = 1.0f / scale;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
    quantize_range<T, VEC>(x, q, n, inv, (long long)blockIdx.x * 256 + threadIdx.x,
                           (long long)gridDim.x * 256);
}

template <typename T>
void quantize_run(const T* x, signed char* q, float* scale_out, long long n,
                  hipStream_t s) {
    if (n < 0) inval("n must be >= 0");
    if (n == 0) return;
    if (!x || !q || !scale_out) inval("quantize: null operand");
    const bool vec = ((uintptr_t)x % (4 * sizeof(T)) == 0) &&
                     ((uintptr_t)q % 4 == 0);
    if (n <= kSmallN) {
        if (vec)
            quantize_small_kernel<T, true><<<1, 1024, 0, s>>>(x, q, scale_out, n);
        else
            quantize_small_kernel<T, false><<<1, 1024, 0, s>>>(x, q, scale_out, n);
        launch_check("quantize kernel launch");
        return;
    }
    float* partial =
        (float*)scratch(Scratch::QuantMax, kPass1Blocks * sizeof(float), s);
    const int g1 = (int)grid_1d((n + 3) / 4, 256, kPass1Blocks);
    const unsigned g2 = grid_1d((n + 3) / 4, 256, dev_info().cu_count * 8);
    if (vec) {
        absmax_partial_kernel<T, true><<<g1, 256, 0, s>>>(x, partial, n);
        launch_check("absmax kernel launch");
        quantize_fold_kernel<T, true><<<g2, 256, 0, s>>>(x, q, partial, g1,
                                                          scale_out, n);
    } else {
        absmax_partial_kernel<T, false><<<g1, 256, 0, s>>>(x, partial, n);
        launch_check("absmax kernel launch");
        quantize_fold_kernel<T, false><<<g2, 256, 0, s>>>(x, q, partial, g1,
                                                           scale_out, n);
    }
    launch_check("quantize kernel launch");
}

}  // namespace
}  // namespace ft

extern "C" {

int ft_quantize_int8_launch(const float* x, signed char* q, float* scale_out,
                            long long n, uintptr_t stream) {
    return ft::guarded([&] {
        ft::quantize_run<float>(x, q, scale_out, n, ft::as_stream(stream));
    });
}

int ft_quantize_int8_launch_ex(const void* x, int x_dtype, signed char* q,
                               float* scale_out, long long n,
                               uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
        switch (x_dtype) {
        case FT_DT_F32:
            ft::quantize_run<float>((const float*)x, q, scale_out, n, s);
            break;
        case FT_DT_BF16:
            ft::quantize_run<ft::bf16>((const ft::bf16*)x, q, scale_out, n, s);
            break;
        case FT_DT_F16:
            ft::quantize_run<ft::f16>((const ft::f16*)x, q, scale_out, n, s);
            break;
        default:
            ft::inval("quantize: unknown dtype code");
        }
    });
}

}  // extern "C"
