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
//
// Also here: dequantize (q * scale) and the fused dequantize-add-requantize
// qadd, with the same device-resident-scale structure.
#include "ft_common.hpp"

namespace ft {
namespace {

constexpr long long kSmallN = 1 << 16;
constexpr int kPass1Blocks = 1024;

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

template <typename T>
void quantize_from_partials(const T* x, signed char* q, const float* partial, int nparts,
                            float* scale_out, long long n, hipStream_t s) {
    if (n <= 0) return;
    if (!x || !q || !partial || !scale_out || nparts < 1) inval("quantize: null operand");
    const unsigned g2 = grid_1d((n + 3) / 4, 256, dev_info().cu_count * 8);
    if (((uintptr_t)x % (4 * sizeof(T)) == 0) && ((uintptr_t)q % 4 == 0))
        quantize_fold_kernel<T, true><<<g2, 256, 0, s>>>(x, q, partial, nparts, scale_out, n);
    else
        quantize_fold_kernel<T, false><<<g2, 256, 0, s>>>(x, q, partial, nparts, scale_out, n);
    launch_check("quantize kernel launch");
}

template <typename T>
void quantize_tensor(const T* x, signed char* q, float* scale_out, long long n,
                     hipStream_t s) {
    quantize_run<T>(x, q, scale_out, n, s);
}

template void quantize_from_partials<float>(const float*, signed char*, const float*, int,
                                            float*, long long, hipStream_t);
template void quantize_from_partials<bf16>(const bf16*, signed char*, const float*, int,
                                           float*, long long, hipStream_t);
template void quantize_from_partials<f16>(const f16*, signed char*, const float*, int,
                                          float*, long long, hipStream_t);
template void quantize_tensor<float>(const float*, signed char*, float*, long long,
                                     hipStream_t);
template void quantize_tensor<bf16>(const bf16*, signed char*, float*, long long,
                                    hipStream_t);
template void quantize_tensor<f16>(const f16*, signed char*, float*, long long, hipStream_t);

namespace {

// ---------------------------------------------------------------------------
// dequantize: x = (float)q * scale (reference quantize.cu:101-108), one
// rounding; 2-byte outputs are that f32 value rounded to nearest-even.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float dq1(signed char q, float sc) {
    float v = (float)q * sc;
    asm("" : "+v"(v));  // rounded to f32 before any narrowing (no mixed FMA)
    return v;
}

// 4 outputs, one 16-byte (f32) or 8-byte (bf16 / fp16) non-temporal store:
// the output is written once and not read back by this launch (a dequant
// stream of 2^28 codes at 8 workgroups per CU: 6.7 TB/s against 5.3 TB/s
// with plain stores; lanes store consecutive pieces, so every instruction
// writes whole lines)
template <typename T>
__device__ __forceinline__ void st4_nt(T* p, float4 v) {
    if constexpr (std::is_same<T, float>::value) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(f4{v.x, v.y, v.z, v.w}, reinterpret_cast<f4*>(p));
    } else {
        typedef T v4 __attribute__((ext_vector_type(4)));
        typedef int i2 __attribute__((ext_vector_type(2)));
        v4 u;
        u[0] = (T)v.x; u[1] = (T)v.y; u[2] = (T)v.z; u[3] = (T)v.w;
        __builtin_nontemporal_store(__builtin_bit_cast(i2, u), reinterpret_cast<i2*>(p));
    }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void dequantize_kernel(
    const signed char* __restrict__ q, T* __restrict__ x, float scale,
    const float* __restrict__ scale_dev, long long n) {
    const float sc = scale_dev ? *scale_dev : scale;
    const long long stride = (long long)gridDim.x * 256;
    const long long tid = (long long)blockIdx.x * 256 + threadIdx.x;
    long long done = 0;
    if (VEC) {
        const long long n4 = n >> 2;
        for (long long c = tid; c < n4; c += stride) {
            const char4 v = *reinterpret_cast<const char4*>(q + 4 * c);
            st4_nt(x + 4 * c, make_float4(dq1(v.x, sc), dq1(v.y, sc),
                                          dq1(v.z, sc), dq1(v.w, sc)));
        }
        done = n4 << 2;
    }
    for (long long i = done + tid; i < n; i += stride) St<T>::st(x + i, dq1(q[i], sc));
}

template <typename T>
void dequantize_run(const signed char* q, T* x, float scale, const float* scale_dev,
                    long long n, hipStream_t s) {
    if (n < 0) inval("n must be >= 0");
    if (n == 0) return;
    if (!q || !x) inval("dequantize: null operand");
    const unsigned grid = grid_1d((n + 3) / 4, 256, dev_info().cu_count * 8);
    if ((uintptr_t)q % 4 == 0 && (uintptr_t)x % (4 * sizeof(T)) == 0)
        dequantize_kernel<T, true><<<grid, 256, 0, s>>>(q, x, scale, scale_dev, n);
    else
        dequantize_kernel<T, false><<<grid, 256, 0, s>>>(q, x, scale, scale_dev, n);
    launch_check("dequantize kernel launch");
}

// ---------------------------------------------------------------------------
// qadd: y = requantize(fl(qa*sa) + fl(qb*sb)) with the sum's own per-tensor
// scale (reference quantize.cu:110-138,217-246): the dequantize -> add ->
// quantize_int8 chain in one pass per phase. Each product is rounded to f32
// on its own (the empty asm keeps the backend from contracting one product
// and the sum into an FMA), so the codes and scale equal
// quantize_int8(dequantize(qa, sa) + dequantize(qb, sb)) bit for bit.
// Same two-phase structure as quantize: one workgroup for small n, else
// per-workgroup maxima in scratch folded by every quantizing workgroup.
// ---------------------------------------------------------------------------
struct QaddSrc {
    const signed char* qa;
    const signed char* qb;
    float sa, sb;
    __device__ __forceinline__ float one(signed char a, signed char b) const {
        float pa = (float)a * sa;
        asm("" : "+v"(pa));
        float pb = (float)b * sb;
        asm("" : "+v"(pb));
        return pa + pb;
    }
    __device__ __forceinline__ float val(long long i) const { return one(qa[i], qb[i]); }
    // the 16 values of 16-byte chunk c (VEC paths: both inputs 16-byte aligned)
    __device__ __forceinline__ void chunk(long long c, float (&v)[16]) const {
        const int4 a4 = *reinterpret_cast<const int4*>(qa + 16 * c);
        const int4 b4 = *reinterpret_cast<const int4*>(qb + 16 * c);
        const signed char* a = reinterpret_cast<const signed char*>(&a4);
        const signed char* b = reinterpret_cast<const signed char*>(&b4);
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = one(a[j], b[j]);
    }
};

__device__ __forceinline__ QaddSrc qadd_src(const signed char* qa, const signed char* qb,
                                            float sa, float sb, const float* sa_dev,
                                            const float* sb_dev) {
    return QaddSrc{qa, qb, sa_dev ? *sa_dev : sa, sb_dev ? *sb_dev : sb};
}

// max |v| over the elements a thread owns: 16-byte chunks tid, tid + stride,
// ... (VEC), then single elements of the tail (or of everything)
template <bool VEC>
__device__ __forceinline__ float qadd_local_max(const QaddSrc& src, long long n,
                                                long long tid, long long stride) {
    float m = 0.0f;
    long long done = 0;
    if (VEC) {
        const long long nc = n >> 4;
        for (long long c = tid; c < nc; c += stride) {
            float v[16];
            src.chunk(c, v);
#pragma unroll
            for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(v[j]));
        }
        done = nc << 4;
    }
    for (long long i = done + tid; i < n; i += stride) m = fmaxf(m, fabsf(src.val(i)));
    return m;
}

template <bool VEC>
__device__ __forceinline__ void qadd_quant_range(const QaddSrc& src, signed char* qy,
                                                 long long n, float inv, long long tid,
                                                 long long stride) {
    long long done = 0;
    if (VEC) {
        const long long nc = n >> 4;
        for (long long c = tid; c < nc; c += stride) {
            float v[16];
            src.chunk(c, v);
            int4 o;
            signed char* ob = reinterpret_cast<signed char*>(&o);
#pragma unroll
            for (int j = 0; j < 16; ++j) ob[j] = quant1(v[j], inv);
            typedef int i4 __attribute__((ext_vector_type(4)));
            __builtin_nontemporal_store(i4{o.x, o.y, o.z, o.w}, reinterpret_cast<i4*>(qy + 16 * c));
        }
        done = nc << 4;
    }
    for (long long i = done + tid; i < n; i += stride) qy[i] = quant1(src.val(i), inv);
}

template <bool VEC>
__global__ __launch_bounds__(1024) void qadd_small_kernel(
    const signed char* __restrict__ qa, const signed char* __restrict__ qb, float sa,
    float sb, const float* __restrict__ sa_dev, const float* __restrict__ sb_dev,
    signed char* __restrict__ qy, float* __restrict__ scale_out, long long n) {
    __shared__ float red[16];
    const QaddSrc src = qadd_src(qa, qb, sa, sb, sa_dev, sb_dev);
    const float m = block_max<1024>(qadd_local_max<VEC>(src, n, threadIdx.x, 1024), red);
    const float scale = make_scale(m);
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) *scale_out = scale;
    qadd_quant_range<VEC>(src, qy, n, inv, threadIdx.x, 1024);
}

template <bool VEC>
__global__ __launch_bounds__(256) void qadd_absmax_kernel(
    const signed char* __restrict__ qa, const signed char* __restrict__ qb, float sa,
    float sb, const float* __restrict__ sa_dev, const float* __restrict__ sb_dev,
    float* __restrict__ partial, long long n) {
    __shared__ float red[4];
    const QaddSrc src = qadd_src(qa, qb, sa, sb, sa_dev, sb_dev);
    const float m = block_max<256>(
        qadd_local_max<VEC>(src, n, (long long)blockIdx.x * 256 + threadIdx.x,
                            (long long)gridDim.x * 256), red);
    if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

template <bool VEC>
__global__ __launch_bounds__(256) void qadd_fold_kernel(
    const signed char* __restrict__ qa, const signed char* __restrict__ qb, float sa,
    float sb, const float* __restrict__ sa_dev, const float* __restrict__ sb_dev,
    const float* __restrict__ partial, int nparts, signed char* __restrict__ qy,
    float* __restrict__ scale_out, long long n) {
    __shared__ float red[4];
    float m = 0.0f;
    for (int i = threadIdx.x; i < nparts; i += 256) m = fmaxf(m, partial[i]);
    m = block_max<256>(m, red);
    const float scale = make_scale(m);
    const float inv = 1.0f / scale;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
    const QaddSrc src = qadd_src(qa, qb, sa, sb, sa_dev, sb_dev);
    qadd_quant_range<VEC>(src, qy, n, inv, (long long)blockIdx.x * 256 + threadIdx.x,
                          (long long)gridDim.x * 256);
}

template <bool VEC>
void qadd_launch(const signed char* qa, const signed char* qb, float sa, float sb,
                 const float* sa_dev, const float* sb_dev, signed char* qy,
                 float* scale_out, long long n, hipStream_t s) {
    if (n <= kSmallN) {
        qadd_small_kernel<VEC><<<1, 1024, 0, s>>>(qa, qb, sa, sb, sa_dev, sb_dev, qy,
                                                  scale_out, n);
        launch_check("qadd kernel launch");
        return;
    }
    float* partial =
        (float*)scratch(Scratch::QuantMax, kPass1Blocks * sizeof(float), s);
    const long long units = VEC ? (n + 15) / 16 : n;
    const int g1 = (int)grid_1d(units, 256, kPass1Blocks);
    const unsigned g2 = grid_1d(units, 256, dev_info().cu_count * 8);
    qadd_absmax_kernel<VEC><<<g1, 256, 0, s>>>(qa, qb, sa, sb, sa_dev, sb_dev, partial, n);
    launch_check("qadd absmax kernel launch");
    qadd_fold_kernel<VEC><<<g2, 256, 0, s>>>(qa, qb, sa, sb, sa_dev, sb_dev, partial, g1,
                                             qy, scale_out, n);
    launch_check("qadd kernel launch");
}

void qadd_run(const signed char* qa, const signed char* qb, float sa, float sb,
              const float* sa_dev, const float* sb_dev, signed char* qy,
              float* scale_out, long long n, hipStream_t s) {
    if (n < 0) inval("n must be >= 0");
    if (n == 0) return;
    if (!qa || !qb || !qy || !scale_out) inval("qadd: null operand");
    const bool vec = ((uintptr_t)qa % 16 == 0) && ((uintptr_t)qb % 16 == 0) &&
                     ((uintptr_t)qy % 16 == 0);
    if (vec)
        qadd_launch<true>(qa, qb, sa, sb, sa_dev, sb_dev, qy, scale_out, n, s);
    else
        qadd_launch<false>(qa, qb, sa, sb, sa_dev, sb_dev, qy, scale_out, n, s);
}

}  // namespace
}  // namespace ft

extern "C" {

int ft_dequantize_int8_launch(const signed char* q, float* x, float scale,
                              long long n, uintptr_t stream) {
    return ft::guarded([&] {
        ft::dequantize_run<float>(q, x, scale, nullptr, n, ft::as_stream(stream));
    });
}

int ft_dequantize_int8_launch_ex(const signed char* q, float scale,
                                 const float* scale_dev, void* x, int x_dtype,
                                 long long n, uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
        switch (x_dtype) {
        case FT_DT_F32: ft::dequantize_run<float>(q, (float*)x, scale, scale_dev, n, s); break;
        case FT_DT_BF16: ft::dequantize_run<ft::bf16>(q, (ft::bf16*)x, scale, scale_dev, n, s); break;
        case FT_DT_F16: ft::dequantize_run<ft::f16>(q, (ft::f16*)x, scale, scale_dev, n, s); break;
        default: ft::inval("dequantize: unknown dtype code");
        }
    });
}

int ft_qadd_int8_launch(const signed char* qa, const signed char* qb, float sa,
                        float sb, signed char* qy, float* out_scale, long long n,
                        uintptr_t stream) {
    return ft::guarded([&] {
        ft::qadd_run(qa, qb, sa, sb, nullptr, nullptr, qy, out_scale, n,
                     ft::as_stream(stream));
    });
}

int ft_qadd_int8_launch_ex(const signed char* qa, const signed char* qb, float sa,
                           float sb, const float* sa_dev, const float* sb_dev,
                           signed char* qy, float* out_scale, long long n,
                           uintptr_t stream) {
    return ft::guarded([&] {
        ft::qadd_run(qa, qb, sa, sb, sa_dev, sb_dev, qy, out_scale, n,
                     ft::as_stream(stream));
    });
}

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
