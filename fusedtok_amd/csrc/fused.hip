// Fused decode-chain kernels for gfx950. The reference composes these steps
// from separate ops (rmsnorm -> quantize_int8, swiglu -> quantize_int8,
// rope -> kv_append_paged); each fused op here computes exactly what the
// unfused chain of this library computes on the same device, with fewer
// launches and no float intermediate in HBM:
//
//   rmsnorm_quant   y = RMSNorm(x [+ r]) * w in f32 -> per-tensor int8 codes
//                   + device scale (1 launch for up to 4 rows of up to
//                   4096 columns, else 2: per-row pass, fold+quantize)
//   swiglu_quant    y = silu(g) * u in f32 -> per-tensor int8 codes + device
//                   scale (2 launches); g / u may be strided row views (the
//                   halves of one gate|up GEMM output)
//   rope_kv_append  the QKV GEMM output row of each sequence -> RoPE(q) into
//                   q_out, RoPE(k) and v written into the paged cache at
//                   slot lens[b] (position lens[b] + pos_offset), one launch
//
// Arithmetic contracts:
//   RMSNorm sum of squares: thread t of 256 accumulates fmaf(v, v, acc) over
//   4-element chunks t, t + 256, ... in element order, then the wave
//   butterfly (xor 32, 16, ..., 1) and the sum of the 4 wave totals in
//   order; inv = 1 / sqrtf(total / cols + eps) (IEEE divide / sqrt);
//   y = (v * inv) * w. The standalone rmsnorm kernel uses the same order, so
//   rmsnorm_quant == quantize_int8(rmsnorm(x), f32 out) bit for bit.
//   Quantize: scale = max|y| / 127 (1 if 0), inv = 1 / scale,
//   q = clamp(rint(y * inv), -127, 127) (reference quantize.cu:169-186).
//   SwiGLU: g / (1 + expf(-g)) * u (reference activations.cu:68-72, 501-511).
//   RoPE: angle, cos/sin and rotation in float64 as the rope kernel.
#include "ft_common.hpp"
#include "kfold.hpp"

#include <cmath>

namespace ft {
namespace {

constexpr int kFNT = 256;

// ---------------------------------------------------------------------------
// rmsnorm_quant
// ---------------------------------------------------------------------------
struct RowStat {
    float absmax;
    float inv;
};

template <typename T>
__device__ __forceinline__ float4 rms_in4(const T* x, const T* r, size_t off) {
    float4 v = St<T>::ld4(x + off);
    if (r) {
        const float4 b = St<T>::ld4(r + off);
        v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
    }
    return v;
}

// x + r for kernels instantiated with (RES) and without a residual: the
// loads of a row are issued together, with no branch between them (a
// runtime residual test between loads made the compiler wait after each
// chunk, one memory round trip per chunk instead of one per row).
template <bool RES>
__device__ __forceinline__ float4 rms_add4(float4 xv, float4 rv) {
    if constexpr (RES)
        return make_float4(xv.x + rv.x, xv.y + rv.y, xv.z + rv.z, xv.w + rv.w);
    else
        return xv;
}

constexpr int kRowChunks = 4;  // 4-element chunks per thread held in registers

// The input rows of the row passes below. FK > 0: x is the output of a
// K-split GEMM, folded here from its partials (fold width FK, kfold.hpp);
// FRES: plus the fold's residual (fold.res, T), rounded again, as the
// GEMM's consumer in a decode layer adds its residual stream.
template <typename T, int FK, bool FRES>
struct RowIn {
    const T* x;
    const KFold& fold;
    float sa;
    // chunk c (4 elements at row offset base) as stored in T, widened to f32
    __device__ __forceinline__ float4 load4(size_t base, int c) const {
        if constexpr (FK > 0) {
            const int4 a = kfold_sum4<FK>(fold, base + 4 * c);
            float4 v = make_float4(kfold_value<T>(a.x, kfold_scale(fold, sa, 4 * c)),
                                   kfold_value<T>(a.y, kfold_scale(fold, sa, 4 * c + 1)),
                                   kfold_value<T>(a.z, kfold_scale(fold, sa, 4 * c + 2)),
                                   kfold_value<T>(a.w, kfold_scale(fold, sa, 4 * c + 3)));
            if constexpr (FRES) {
                const float4 r = St<T>::ld4(static_cast<const T*>(fold.res) + base + 4 * c);
                v = make_float4(kfold_add_res<T>(v.x, r.x), kfold_add_res<T>(v.y, r.y),
                                kfold_add_res<T>(v.z, r.z), kfold_add_res<T>(v.w, r.w));
            }
            return v;
        } else {
            return St<T>::ld4(x + base + 4 * c);
        }
    }
};

// T(v) stored to h (the residual stream x + r of a decode layer)
template <typename T>
__device__ __forceinline__ void st4_rounded(T* h, float4 v) {
    St<T>::st4(h, v);
}

// One workgroup per row: sum of squares -> inv, then the row's max |y| (the
// first pass of rmsnorm_quant's two-launch form). A row of up to 4096
// columns stays in registers between the two passes. FK > 0: the folded x
// is stored into x_out, as the GEMM would have stored it. HOUT (with RES):
// h_out receives T(x + r).
template <typename T, bool RES, int FK, bool FRES, bool HOUT>
__global__ __launch_bounds__(kFNT) void rmsq_rows(
    const T* __restrict__ x, const T* __restrict__ r, const float* __restrict__ w,
    RowStat* __restrict__ stat, int cols, float eps, KFold fold, T* __restrict__ x_out,
    T* __restrict__ h_out) {
    __shared__ float red[kFNT / 64];
    const size_t base = (size_t)blockIdx.x * cols;
    const int chunks = cols >> 2;
    constexpr bool FOLD = FK > 0;
    const RowIn<T, FK, FRES> in{x, fold, FOLD ? kfold_sa(fold) : 0.0f};
    float m = 0.0f;
    float inv;
    if (chunks <= kFNT * kRowChunks) {
        // the row, its residual and the weights in one round trip (indices
        // clamped to a real chunk; chunks past the row are not used below)
        float4 v[kRowChunks], rv[kRowChunks], wc[kRowChunks];
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
            const int c = min((int)threadIdx.x + j * kFNT, chunks - 1);
            v[j] = in.load4(base, c);
            if constexpr (RES) rv[j] = St<T>::ld4(r + base + 4 * c);
            wc[j] = *reinterpret_cast<const float4*>(w + 4 * c);
        }
        if constexpr (FOLD) {
#pragma unroll
            for (int j = 0; j < kRowChunks; ++j)
                if ((int)threadIdx.x + j * kFNT < chunks)
                    St<T>::st4(x_out + base + 4 * ((int)threadIdx.x + j * kFNT), v[j]);
        }
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) v[j] = rms_add4<RES>(v[j], rv[j]);
        if constexpr (HOUT) {
#pragma unroll
            for (int j = 0; j < kRowChunks; ++j)
                if ((int)threadIdx.x + j * kFNT < chunks)
                    st4_rounded(h_out + base + 4 * ((int)threadIdx.x + j * kFNT), v[j]);
        }
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
            if ((int)threadIdx.x + j * kFNT < chunks) {
                acc = fmaf(v[j].x, v[j].x, acc);
                acc = fmaf(v[j].y, v[j].y, acc);
                acc = fmaf(v[j].z, v[j].z, acc);
                acc = fmaf(v[j].w, v[j].w, acc);
            }
        }
        const float total = block_sum<kFNT>(acc, red);
        inv = 1.0f / sqrtf(total / (float)cols + eps);
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
            if ((int)threadIdx.x + j * kFNT < chunks) {
                m = fmaxf(m, fabsf(v[j].x * inv * wc[j].x));
                m = fmaxf(m, fabsf(v[j].y * inv * wc[j].y));
                m = fmaxf(m, fabsf(v[j].z * inv * wc[j].z));
                m = fmaxf(m, fabsf(v[j].w * inv * wc[j].w));
            }
        }
    } else {
        float acc = 0.0f;
        for (int c = threadIdx.x; c < chunks; c += kFNT) {
            float4 v = in.load4(base, c);
            if constexpr (FOLD) St<T>::st4(x_out + base + 4 * c, v);
            if constexpr (RES) v = rms_add4<true>(v, St<T>::ld4(r + base + 4 * c));
            if constexpr (HOUT) st4_rounded(h_out + base + 4 * c, v);
            acc = fmaf(v.x, v.x, acc);
            acc = fmaf(v.y, v.y, acc);
            acc = fmaf(v.z, v.z, acc);
            acc = fmaf(v.w, v.w, acc);
        }
        const float total = block_sum<kFNT>(acc, red);
        inv = 1.0f / sqrtf(total / (float)cols + eps);
        // second pass: the folded rows are read back from x_out (their
        // stored bits: the same values)
        const T* xs = FOLD ? x_out : x;
        for (int c = threadIdx.x; c < chunks; c += kFNT) {
            float4 v = St<T>::ld4(xs + base + 4 * c);
            if constexpr (RES) v = rms_add4<true>(v, St<T>::ld4(r + base + 4 * c));
            const float4 wv = *reinterpret_cast<const float4*>(w + 4 * c);
            m = fmaxf(m, fabsf(v.x * inv * wv.x));
            m = fmaxf(m, fabsf(v.y * inv * wv.y));
            m = fmaxf(m, fabsf(v.z * inv * wv.z));
            m = fmaxf(m, fabsf(v.w * inv * wv.w));
        }
    }
    m = block_max<kFNT>(m, red);
    if (threadIdx.x == 0) stat[blockIdx.x] = RowStat{m, inv};
}

// rmsnorm_quant in one launch: one workgroup per row of at most 4096
// columns, the register row pass of rmsq_rows, then the tensor's maximum
// through grid_max (every row's workgroup resident at once), then each
// workgroup quantizes its row from the same registers. The arithmetic is
// rmsq_rows' followed by rmsq_quant's, so codes and scale are the same bits
// as the two launches. x_out (FK > 0) may be null: the folded rows are then
// not stored.
template <typename T, bool RES, int FK, bool FRES, bool HOUT>
__global__ __launch_bounds__(kFNT) void rmsq_grid(
    const T* __restrict__ x, const T* __restrict__ r, const float* __restrict__ w,
    int cols, float eps, KFold fold, T* __restrict__ x_out, T* __restrict__ h_out,
    signed char* __restrict__ q, float* __restrict__ scale_out, GridMax gm) {
    __shared__ float red[kFNT / 64];
    const size_t base = (size_t)blockIdx.x * cols;
    const int chunks = cols >> 2;
    constexpr bool FOLD = FK > 0;
    const RowIn<T, FK, FRES> in{x, fold, FOLD ? kfold_sa(fold) : 0.0f};
    float4 v[kRowChunks], rv[kRowChunks], wc[kRowChunks];
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
        const int c = min((int)threadIdx.x + j * kFNT, chunks - 1);
        v[j] = in.load4(base, c);
        if constexpr (RES) rv[j] = St<T>::ld4(r + base + 4 * c);
        wc[j] = *reinterpret_cast<const float4*>(w + 4 * c);
    }
    if constexpr (FOLD) {
        if (x_out) {
#pragma unroll
            for (int j = 0; j < kRowChunks; ++j)
                if ((int)threadIdx.x + j * kFNT < chunks)
                    St<T>::st4(x_out + base + 4 * ((int)threadIdx.x + j * kFNT), v[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) v[j] = rms_add4<RES>(v[j], rv[j]);
    if constexpr (HOUT) {
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j)
            if ((int)threadIdx.x + j * kFNT < chunks)
                st4_rounded(h_out + base + 4 * ((int)threadIdx.x + j * kFNT), v[j]);
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
        if ((int)threadIdx.x + j * kFNT < chunks) {
            acc = fmaf(v[j].x, v[j].x, acc);
            acc = fmaf(v[j].y, v[j].y, acc);
            acc = fmaf(v[j].z, v[j].z, acc);
            acc = fmaf(v[j].w, v[j].w, acc);
        }
    }
    const float total = block_sum<kFNT>(acc, red);
    const float inv = 1.0f / sqrtf(total / (float)cols + eps);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
        if ((int)threadIdx.x + j * kFNT < chunks) {
            m = fmaxf(m, fabsf(v[j].x * inv * wc[j].x));
            m = fmaxf(m, fabsf(v[j].y * inv * wc[j].y));
            m = fmaxf(m, fabsf(v[j].z * inv * wc[j].z));
            m = fmaxf(m, fabsf(v[j].w * inv * wc[j].w));
        }
    }
    m = block_max<kFNT>(m, red);
    m = grid_max<kFNT>(gm, m, red);
    const float scale = make_scale(m);
    const float inv_s = 1.0f / scale;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
        const int c = (int)threadIdx.x + j * kFNT;
        if (c < chunks) {
            char4 o;
            o.x = quant1(v[j].x * inv * wc[j].x, inv_s);
            o.y = quant1(v[j].y * inv * wc[j].y, inv_s);
            o.z = quant1(v[j].z * inv * wc[j].z, inv_s);
            o.w = quant1(v[j].w * inv * wc[j].w, inv_s);
            *reinterpret_cast<char4*>(q + base + 4 * c) = o;
        }
    }
}

// Fold of the row maxima -> scale, then the codes. Each thread's first
// element (x, r, w and its row's inv) is loaded before the fold, so the fold's
// reads and the data reads share one round trip.
template <typename T, bool RES>
__global__ __launch_bounds__(kFNT) void rmsq_quant(
    const T* __restrict__ x, const T* __restrict__ r, const float* __restrict__ w,
    const RowStat* __restrict__ stat, signed char* __restrict__ q,
    float* __restrict__ scale_out, int rows, int cols) {
    __shared__ float red[kFNT / 64];
    const long long n4 = (long long)rows * cols / 4;
    const int cols4 = cols >> 2;
    const long long e0 = (long long)blockIdx.x * kFNT + threadIdx.x;
    // this thread's first element (clamped to a real one) with its row's
    // inv, loaded without branches so they share the fold's round trip
    const long long ec = e0 < n4 ? e0 : n4 - 1;
    const int row0 = (int)(ec / cols4);
    const int c0 = (int)(ec - (long long)row0 * cols4) * 4;
    float4 v0 = St<T>::ld4(x + (size_t)row0 * cols + c0);
    float4 rv0;
    if constexpr (RES) rv0 = St<T>::ld4(r + (size_t)row0 * cols + c0);
    const float4 w0 = *reinterpret_cast<const float4*>(w + c0);
    const float inv0 = stat[row0].inv;
    v0 = rms_add4<RES>(v0, rv0);
    float m = 0.0f;
    for (int i = threadIdx.x; i < rows; i += kFNT) m = fmaxf(m, stat[i].absmax);
    m = block_max<kFNT>(m, red);
    const float scale = make_scale(m);
    const float inv_s = 1.0f / scale;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
    if (e0 < n4) {
        char4 o;
        o.x = quant1(v0.x * inv0 * w0.x, inv_s);
        o.y = quant1(v0.y * inv0 * w0.y, inv_s);
        o.z = quant1(v0.z * inv0 * w0.z, inv_s);
        o.w = quant1(v0.w * inv0 * w0.w, inv_s);
        *reinterpret_cast<char4*>(q + 4 * e0) = o;
    }
    for (long long e = e0 + (long long)gridDim.x * kFNT; e < n4;
         e += (long long)gridDim.x * kFNT) {
        const int row = (int)(e / cols4);
        const int c = (int)(e - (long long)row * cols4) * 4;
        const float inv = stat[row].inv;
        const float4 v = rms_in4(x, r, (size_t)row * cols + c);
        const float4 wv = *reinterpret_cast<const float4*>(w + c);
        char4 o;
        o.x = quant1(v.x * inv * wv.x, inv_s);
        o.y = quant1(v.y * inv * wv.y, inv_s);
        o.z = quant1(v.z * inv * wv.z, inv_s);
        o.w = quant1(v.w * inv * wv.w, inv_s);
        *reinterpret_cast<char4*>(q + 4 * e) = o;
    }
}

// Small-M rmsnorm_quant in one launch: one workgroup of 256 * rows threads
// for up to 4 rows; lane g (256 threads) holds row g in registers, thread t
// chunks t, t + 256, t + 512, t + 768, so x (and r) are read once and the row
// pass, the tensor maximum and the codes come from the same registers. The
// arithmetic is the two-kernel path's: per row the same 256-thread chunk
// assignment, fmaf order, wave butterfly and in-order sum of the lane's 4
// wave totals; products (v * inv) * w; maxima are exact in any order. One CU
// keeps only ~64 cache-line misses in flight (~10 GB/s from HBM), so each
// further row adds ~0.75 us: past 4 rows the two kernels, which spread the
// rows over CUs, are faster.
constexpr int kRmsqRows = 1;    // rows per lane
constexpr int kRmsqMaxRows = 4 * kRmsqRows;
constexpr int kRmsqMaxCols = 4 * kFNT * kRowChunks;

template <typename T, bool RES>
__global__ __launch_bounds__(4 * kFNT) void rmsq_small(
    const T* __restrict__ x, const T* __restrict__ r, const float* __restrict__ w,
    signed char* __restrict__ q, float* __restrict__ scale_out, int rows, int cols,
    float eps) {
    __shared__ float red[kRmsqMaxRows][kFNT / 64];
    __shared__ float redm[4 * kFNT / 64];
    const int G = blockDim.x / kFNT;
    const int lane_g = threadIdx.x / kFNT;
    const int t = threadIdx.x % kFNT;
    const int wv = t >> 6;
    const int chunks = cols >> 2;

    float4 v[kRmsqRows][kRowChunks];
    float4 wc[kRowChunks];
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j)
        wc[j] = *reinterpret_cast<const float4*>(w + 4 * min(t + j * kFNT, chunks - 1));
    float4 rv[kRmsqRows][kRowChunks];
#pragma unroll
    for (int i = 0; i < kRmsqRows; ++i) {
        const int row = min(lane_g + i * G, rows - 1);
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
            const int c = min(t + j * kFNT, chunks - 1);  // clamped; unused past the row
            v[i][j] = St<T>::ld4(x + (size_t)row * cols + 4 * c);
            if constexpr (RES) rv[i][j] = St<T>::ld4(r + (size_t)row * cols + 4 * c);
        }
    }
#pragma unroll
    for (int i = 0; i < kRmsqRows; ++i)
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) v[i][j] = rms_add4<RES>(v[i][j], rv[i][j]);
#pragma unroll
    for (int i = 0; i < kRmsqRows; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
            if (t + j * kFNT < chunks) {
                acc = fmaf(v[i][j].x, v[i][j].x, acc);
                acc = fmaf(v[i][j].y, v[i][j].y, acc);
                acc = fmaf(v[i][j].z, v[i][j].z, acc);
                acc = fmaf(v[i][j].w, v[i][j].w, acc);
            }
        }
        acc = wave_sum(acc);
        if ((t & 63) == 0) red[lane_g + i * G][wv] = acc;
    }
    __syncthreads();
    float inv[kRmsqRows];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < kRmsqRows; ++i) {
        const int row = lane_g + i * G;
        inv[i] = 0.0f;
        if (row < rows) {
            float tot = 0.0f;
#pragma unroll
            for (int k = 0; k < kFNT / 64; ++k) tot += red[row][k];
            inv[i] = 1.0f / sqrtf(tot / (float)cols + eps);
#pragma unroll
            for (int j = 0; j < kRowChunks; ++j) {
                if (t + j * kFNT < chunks) {
                    m = fmaxf(m, fabsf(v[i][j].x * inv[i] * wc[j].x));
                    m = fmaxf(m, fabsf(v[i][j].y * inv[i] * wc[j].y));
                    m = fmaxf(m, fabsf(v[i][j].z * inv[i] * wc[j].z));
                    m = fmaxf(m, fabsf(v[i][j].w * inv[i] * wc[j].w));
                }
            }
        }
    }
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) redm[threadIdx.x >> 6] = m;
    __syncthreads();
    m = redm[0];
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k) m = fmaxf(m, redm[k]);
    const float scale = make_scale(m);
    const float inv_s = 1.0f / scale;
    if (threadIdx.x == 0) *scale_out = scale;
#pragma unroll
    for (int i = 0; i < kRmsqRows; ++i) {
        const int row = lane_g + i * G;
        if (row >= rows) continue;
#pragma unroll
        for (int j = 0; j < kRowChunks; ++j) {
            const int c = t + j * kFNT;
            if (c >= chunks) continue;
            char4 o;
            o.x = quant1(v[i][j].x * inv[i] * wc[j].x, inv_s);
            o.y = quant1(v[i][j].y * inv[i] * wc[j].y, inv_s);
            o.z = quant1(v[i][j].z * inv[i] * wc[j].z, inv_s);
            o.w = quant1(v[i][j].w * inv[i] * wc[j].w, inv_s);
            *reinterpret_cast<char4*>(q + (size_t)row * cols + 4 * c) = o;
        }
    }
}

template <typename T>
void rmsq_check(const T* x, const float* w, const T* r, const signed char* q,
                const float* scale_out, int rows, int cols) {
    if (rows < 0 || cols <= 0) inval("rows must be >= 0 and cols must be > 0");
    if (cols % 4 != 0) inval("rmsnorm_quant: cols must be a multiple of 4");
    if (rows == 0) return;
    if (!x || !w || !q || !scale_out) inval("rmsnorm_quant: null operand");
    const size_t a16 = 4 * sizeof(T);
    if ((uintptr_t)x % a16 || (r && (uintptr_t)r % a16) || (uintptr_t)w % 16 ||
        (uintptr_t)q % 4)
        inval("rmsnorm_quant: operands must be aligned to 4 elements");
}

// What a row pass takes and writes beyond rmsnorm_quant's own operands.
// fold.ksplit >= 2: x is a K-split GEMM's output still held as its partials
// (plus fold.res), folded by the row pass, which stores the rows into x_out
// (required by the two-launch form; the one-launch form skips the store
// when x_out is null). h_out (with a residual r): T(x + r), the residual
// stream of a decode layer.
template <typename T>
struct RmsqIo {
    KFold fold;
    T* x_out = nullptr;
    T* h_out = nullptr;
    bool store_x = true;  // false: the one-launch form need not store x_out
};

// Rows (workgroups) of the one-launch form. From 17 rows: below, the two
// launches measured as fast or faster (C2 chain, M = 8 / 16, same box:
// 15.74 / 16.35 us with two launches against 15.80 / 16.60 with one); at
// C4's 64 rows the two forms measured the same (layer 434.6-438.3 against
// 437.4-438.7 us): the kernel boundary a graph replay pays costs about the
// three dependent device-scope atomic round trips of grid_max.
constexpr int kRmsqGridMinRows = 17;
constexpr int kRmsqGridRows = 4096;

// instantiates the row kernel K<T, RES, FK, FRES, HOUT> for the run-time
// choices and calls launch(kernel pointer) with it
template <typename T, template <typename, bool, int, bool, bool> class K, typename L>
void rmsq_pick(bool res, int fk, bool fres, bool hout, L&& launch) {
    auto by_fk = [&](auto res_c, auto fres_c, auto hout_c) {
        constexpr bool R = decltype(res_c)::value, F = decltype(fres_c)::value,
                       H = decltype(hout_c)::value;
        if (fk == 0) launch(K<T, R, 0, false, H>{});
        else if (fk == 4) launch(K<T, R, 4, F, H>{});
        else if (fk == 8) launch(K<T, R, 8, F, H>{});
        else launch(K<T, R, 1, F, H>{});
    };
    using t_ = std::true_type;
    using f_ = std::false_type;
    if (res) {
        if (hout) by_fk(t_{}, f_{}, t_{});
        else by_fk(t_{}, f_{}, f_{});
    } else {
        if (fres) by_fk(f_{}, t_{}, f_{});
        else by_fk(f_{}, f_{}, f_{});
    }
}

// kernel tags: carry the template arguments to the launch lambdas
template <typename T, bool RES, int FK, bool FRES, bool HOUT>
struct RowsK {
    static constexpr auto fn = rmsq_rows<T, RES, FK, FRES, HOUT>;
};
template <typename T, bool RES, int FK, bool FRES, bool HOUT>
struct GridK {
    static constexpr auto fn = rmsq_grid<T, RES, FK, FRES, HOUT>;
};

// rmsnorm_quant of x (or of the folded partials) in one launch when every
// row's workgroup can be resident at once, else the row pass then the fold
// of the row maxima and the codes (two launches)
template <typename T>
void rmsq_rows_run(const T* x, const RmsqIo<T>& io, const float* w, const T* r,
                   signed char* q, float* scale_out, int rows, int cols, float eps,
                   hipStream_t s) {
    const bool fold = io.fold.ksplit > 1;
    const int fk = fold ? kfold_width(io.fold.ksplit) : 0;
    const bool fres = fold && io.fold.res;
    const bool hout = r && io.h_out;
    if (fres && r) inval("rmsnorm_quant: a fold residual and a norm residual together");
    if (cols <= 4 * kFNT * kRowChunks && rows >= kRmsqGridMinRows && rows <= kRmsqGridRows &&
        tune(Tune::RmsqSplit, 0) == 0) {
        const GridMax gm = gridmax_state(rows, s);
        bool done = false;
        rmsq_pick<T, GridK>(r != nullptr, fk, fres, hout, [&](auto k) {
            using Kt = decltype(k);
            if (!grid_resident((const void*)Kt::fn, rows, kFNT, GridUse::RmsNorm)) return;
            Kt::fn<<<(unsigned)rows, kFNT, 0, s>>>(x, r, w, cols, eps, io.fold,
                                                   io.store_x ? io.x_out : nullptr, io.h_out,
                                                   q, scale_out, gm);
            launch_check("rmsnorm_quant one-launch kernel launch");
            done = true;
        });
        if (done) return;
    }
    if (fold && !io.x_out) inval("rmsnorm_quant: the folded rows need a destination");
    RowStat* stat = (RowStat*)scratch(Scratch::QuantMax, (size_t)rows * sizeof(RowStat), s);
    rmsq_pick<T, RowsK>(r != nullptr, fk, fres, hout, [&](auto k) {
        decltype(k)::fn<<<(unsigned)rows, kFNT, 0, s>>>(x, r, w, stat, cols, eps, io.fold,
                                                        io.x_out, io.h_out);
    });
    launch_check("rmsnorm_quant row kernel launch");
    const T* xs = fold ? io.x_out : x;
    const long long n4 = (long long)rows * cols / 4;
    const unsigned grid = grid_1d(n4, kFNT, dev_info().cu_count * 4);
    if (r)
        rmsq_quant<T, true><<<grid, kFNT, 0, s>>>(xs, r, w, stat, q, scale_out, rows, cols);
    else
        rmsq_quant<T, false><<<grid, kFNT, 0, s>>>(xs, r, w, stat, q, scale_out, rows, cols);
    launch_check("rmsnorm_quant quantize kernel launch");
}

template <typename T>
void rmsnorm_quant_run(const T* x, const float* w, const T* r, signed char* q,
                       float* scale_out, int rows, int cols, float eps,
                       hipStream_t s, T* h_out = nullptr) {
    rmsq_check(x, w, r, q, scale_out, rows, cols);
    if (rows == 0) return;
    if (rows <= kRmsqMaxRows && cols <= kRmsqMaxCols && tune(Tune::RmsqSplit, 0) == 0 &&
        !(r && h_out)) {
        if (r)
            rmsq_small<T, true><<<1, (unsigned)(rows * kFNT), 0, s>>>(x, r, w, q, scale_out,
                                                                       rows, cols, eps);
        else
            rmsq_small<T, false><<<1, (unsigned)(rows * kFNT), 0, s>>>(x, r, w, q, scale_out,
                                                                        rows, cols, eps);
        launch_check("rmsnorm_quant small kernel launch");
        return;
    }
    RmsqIo<T> io;
    io.h_out = h_out;
    rmsq_rows_run<T>(x, io, w, r, q, scale_out, rows, cols, eps, s);
}


// o_proj-style GEMM (a_q codes with the device scale *sa_dev, w_q [n, k],
// per-channel w_scales) -> y [rows, n] in T, then rmsnorm_quant(y [+ r]).
// A K-split GEMM's partials are folded by the row pass, which stores y
// (when y_store; the one-launch form can skip it). h_out (with r): the
// residual stream T(y + r).
template <typename T>
void qgemm_rmsq_run(const signed char* a_q, const float* sa_dev, const signed char* w_q,
                    const float* w_scales, T* y, const T* r, const float* w, float eps,
                    signed char* q, float* scale_out, int rows, int n, int k, int dtype,
                    hipStream_t s, T* h_out = nullptr, bool y_store = true) {
    if (k < 1) inval("qgemm_rmsnorm_quant: k must be >= 1");
    rmsq_check(y, w, r, q, scale_out, rows, n);
    if (rows == 0) return;
    if (!a_q || !sa_dev || !w_q || !w_scales)
        inval("qgemm_rmsnorm_quant: null operand");
    RmsqIo<T> io;
    io.h_out = h_out;
    if (qgemm_deferred(a_q, w_q, sa_dev, w_scales, y, dtype, rows, n, k, s, io.fold)) {
        io.x_out = y;
        io.store_x = y_store;
        rmsq_rows_run<T>(nullptr, io, w, r, q, scale_out, rows, n, eps, s);
    } else {
        rmsnorm_quant_run<T>(y, w, r, q, scale_out, rows, n, eps, s, h_out);
    }
}

// ---------------------------------------------------------------------------
// swiglu_quant: element (row, c) of gate / up at row * ld + c
// ---------------------------------------------------------------------------
// VEC: cols and the row stride are multiples of 4 and g / u / q aligned to
// 4 elements: each thread takes 4 consecutive elements of a row per load
// (one 8-byte load per operand for half types), so a thread's few elements
// cost one round trip instead of one per element.
template <typename T, bool VEC>
__device__ __forceinline__ void swq_at(const T* g, const T* u, long long c, int cols,
                                       long long ld, float (&y)[4]) {
    if constexpr (VEC) {
        const int cols4 = cols >> 2;
        const long long row = c / cols4;
        const size_t off = (size_t)(row * ld + 4 * (c - row * cols4));
        const float4 gv = St<T>::ld4(g + off), uv = St<T>::ld4(u + off);
        y[0] = silu_mul(gv.x, uv.x);
        y[1] = silu_mul(gv.y, uv.y);
        y[2] = silu_mul(gv.z, uv.z);
        y[3] = silu_mul(gv.w, uv.w);
    } else {
        const long long row = c / cols;
        const size_t off = (size_t)(row * ld + (c - row * cols));
        y[0] = silu_mul(St<T>::ld(g + off), St<T>::ld(u + off));
    }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kFNT) void swq_absmax(
    const T* __restrict__ g, const T* __restrict__ u, float* __restrict__ part,
    int rows, int cols, long long ld) {
    __shared__ float red[kFNT / 64];
    constexpr int W = VEC ? 4 : 1;
    const long long n = (long long)rows * cols / W;
    float m = 0.0f;
    for (long long c = (long long)blockIdx.x * kFNT + threadIdx.x; c < n;
         c += (long long)gridDim.x * kFNT) {
        float y[4];
        swq_at<T, VEC>(g, u, c, cols, ld, y);
#pragma unroll
        for (int k = 0; k < W; ++k) m = fmaxf(m, fabsf(y[k]));
    }
    m = block_max<kFNT>(m, red);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// Fold of the partial maxima (4 loads per thread in flight), then the codes;
// each thread's first elements are loaded before the fold.
template <typename T, bool VEC>
__global__ __launch_bounds__(kFNT) void swq_quant(
    const T* __restrict__ g, const T* __restrict__ u, const float* __restrict__ part,
    int nparts, signed char* __restrict__ q, float* __restrict__ scale_out, int rows,
    int cols, long long ld) {
    __shared__ float red[kFNT / 64];
    constexpr int W = VEC ? 4 : 1;
    const long long n = (long long)rows * cols / W;
    const long long c0 = (long long)blockIdx.x * kFNT + threadIdx.x;
    float y0[4] = {0.f, 0.f, 0.f, 0.f};
    if (c0 < n) swq_at<T, VEC>(g, u, c0, cols, ld, y0);
    float m = 0.0f;
    for (int i0 = threadIdx.x; i0 < nparts; i0 += 4 * kFNT) {
        float pv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) pv[k] = i0 + k * kFNT < nparts ? part[i0 + k * kFNT] : 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) m = fmaxf(m, pv[k]);
    }
    m = block_max<kFNT>(m, red);
    const float scale = make_scale(m);
    const float inv_s = 1.0f / scale;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
    auto put = [&](long long c, const float (&y)[4]) {
        if constexpr (VEC) {
            char4 o;
            o.x = quant1(y[0], inv_s);
            o.y = quant1(y[1], inv_s);
            o.z = quant1(y[2], inv_s);
            o.w = quant1(y[3], inv_s);
            *reinterpret_cast<char4*>(q + 4 * c) = o;
        } else {
            q[c] = quant1(y[0], inv_s);
        }
    };
    if (c0 < n) put(c0, y0);
    for (long long c = c0 + (long long)gridDim.x * kFNT; c < n;
         c += (long long)gridDim.x * kFNT) {
        float y[4];
        swq_at<T, VEC>(g, u, c, cols, ld, y);
        put(c, y);
    }
}

constexpr int kSwqParts = 1024;

template <typename T>
void swiglu_quant_run(const T* g, const T* u, signed char* q, float* scale_out,
                      int rows, int cols, long long ld, hipStream_t s) {
    if (rows < 0 || cols < 0) inval("rows and cols must be >= 0");
    if (ld < cols) inval("swiglu_quant: row stride must be >= cols");
    if ((long long)rows * cols == 0) return;
    if (!g || !u || !q || !scale_out) inval("swiglu_quant: null operand");
    const size_t a4 = 4 * sizeof(T);
    const bool vec = cols % 4 == 0 && ld % 4 == 0 && (uintptr_t)g % a4 == 0 &&
                     (uintptr_t)u % a4 == 0 && (uintptr_t)q % 4 == 0;
    const long long n = (long long)rows * cols / (vec ? 4 : 1);
    float* part = (float*)scratch(Scratch::QuantMax, kSwqParts * sizeof(float), s);
    const unsigned g1 = grid_1d(n, kFNT, kSwqParts);
    const unsigned g2 = grid_1d(n, kFNT, dev_info().cu_count * 4);
    if (vec) {
        swq_absmax<T, true><<<g1, kFNT, 0, s>>>(g, u, part, rows, cols, ld);
        launch_check("swiglu_quant absmax kernel launch");
        swq_quant<T, true><<<g2, kFNT, 0, s>>>(g, u, part, (int)g1, q, scale_out, rows, cols,
                                               ld);
    } else {
        swq_absmax<T, false><<<g1, kFNT, 0, s>>>(g, u, part, rows, cols, ld);
        launch_check("swiglu_quant absmax kernel launch");
        swq_quant<T, false><<<g2, kFNT, 0, s>>>(g, u, part, (int)g1, q, scale_out, rows,
                                                cols, ld);
    }
    launch_check("swiglu_quant quantize kernel launch");
}

}  // namespace

void rmsnorm_quant_folded(int dtype, const KFold& fold, void* x_out, const float* w,
                          signed char* q, float* scale_out, int rows, int cols, float eps,
                          hipStream_t s) {
    if (fold.ksplit < 2 || fold.n != cols || fold.mn != (long long)rows * cols)
        inval("rmsnorm_quant_folded: partials do not match the rows");
#define FT_RQF(T)                                                                         \
    do {                                                                                  \
        rmsq_check<T>((const T*)x_out, w, nullptr, q, scale_out, rows, cols);             \
        RmsqIo<T> io;                                                                     \
        io.fold = fold;                                                                   \
        io.x_out = (T*)x_out;                                                             \
        if (rows > 0)                                                                     \
            rmsq_rows_run<T>(nullptr, io, w, nullptr, q, scale_out, rows, cols, eps, s);  \
    } while (0)
    switch (dtype) {
    case FT_DT_F32: FT_RQF(float); break;
    case FT_DT_BF16: FT_RQF(bf16); break;
    case FT_DT_F16: FT_RQF(f16); break;
    default: inval("rmsnorm_quant_folded: unknown dtype code");
    }
#undef FT_RQF
}

namespace {

// y = T(f32(y) + f32(h)) in place, 4 elements per thread
template <typename T>
__global__ __launch_bounds__(256) void residual_add_kernel(T* __restrict__ y,
                                                          const T* __restrict__ h,
                                                          long long n4) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const float4 a = St<T>::ld4(y + 4 * i), b = St<T>::ld4(h + 4 * i);
    St<T>::st4(y + 4 * i, make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w));
}

}  // namespace

void residual_add(int dtype, void* y, const void* h, long long n, hipStream_t s) {
    if (n <= 0) return;
    if (n % 4 != 0 || !y || !h) inval("residual_add: n must be a multiple of 4");
    const unsigned grid = grid_1d(n / 4, 256, 1 << 30);
    switch (dtype) {
    case FT_DT_F32:
        residual_add_kernel<float><<<grid, 256, 0, s>>>((float*)y, (const float*)h, n / 4);
        break;
    case FT_DT_BF16:
        residual_add_kernel<bf16><<<grid, 256, 0, s>>>((bf16*)y, (const bf16*)h, n / 4);
        break;
    case FT_DT_F16:
        residual_add_kernel<f16><<<grid, 256, 0, s>>>((f16*)y, (const f16*)h, n / 4);
        break;
    default: inval("residual_add: unknown dtype code");
    }
    launch_check("residual_add kernel launch");
}

void qgemm_rmsnorm_quant_res(int dtype, const signed char* a_q, const float* sa_dev,
                             const signed char* w_q, const float* w_scales, void* y,
                             const void* residual,
                             const float* w, float eps, signed char* q, float* scale_out,
                             void* h_out, int rows, int n, int k, hipStream_t s) {
#define FT_QRR(T)                                                                          \
    qgemm_rmsq_run<T>(a_q, sa_dev, w_q, w_scales, (T*)y, (const T*)residual, w, eps, q,   \
                      scale_out, rows, n, k, dtype, s, (T*)h_out, false)
    switch (dtype) {
    case FT_DT_F32: FT_QRR(float); break;
    case FT_DT_BF16: FT_QRR(bf16); break;
    case FT_DT_F16: FT_QRR(f16); break;
    default: inval("qgemm_rmsnorm_quant: unknown dtype code");
    }
#undef FT_QRR
}

namespace {

// gate/up GEMM (a_q codes with the device scale *sa_dev; w_gu [2 inter, k],
// gate rows then up rows, per-channel w_scales) -> h [rows, 2 inter] in T,
// then swiglu_quant(h[:, :inter], h[:, inter:]). Where the GEMM runs
// unsplit on the skinny ring kernel, its epilogue takes the SwiGLU maxima
// (the maximum is exact in any order): with every workgroup resident at
// once it also folds them and writes the codes (one launch; h is then
// stored only if store_h), else only the codes pass is left.
template <typename T>
void qgemm_swq_run(const signed char* a_q, const float* sa_dev, const signed char* w_gu,
                   const float* w_scales, T* h, signed char* q, float* scale_out, int rows,
                   int inter, int k, int dtype, hipStream_t s, bool store_h = true) {
    if (rows < 0 || inter < 1 || k < 0)
        inval("qgemm_swiglu_quant: rows and k must be >= 0, inter >= 1");
    if (rows == 0) return;
    if (!a_q || !sa_dev || !w_gu || !w_scales || !h || !q || !scale_out)
        inval("qgemm_swiglu_quant: null operand");
    const long long ld = 2LL * inter;
    float* part = nullptr;
    int nparts = 0;
    const int how = qgemm_swiglu_max(a_q, w_gu, sa_dev, w_scales, store_h ? h : nullptr, dtype,
                                     rows, inter, k, s, part, nparts, q, scale_out);
    if (how == 2) return;
    if (how == 0) {
        const int rc = ft_qgemm_launch_ex(a_q, w_gu, w_scales, 0.0f, 0.0f, sa_dev, h, dtype,
                                          rows, 2 * inter, k, (uintptr_t)s);
        if (rc != FT_OK) throw Error{rc, ft_last_error()};
        swiglu_quant_run<T>(h, h + inter, q, scale_out, rows, inter, ld, s);
        return;
    }
    const size_t a4 = 4 * sizeof(T);
    const bool vec = inter % 4 == 0 && (uintptr_t)h % a4 == 0 &&
                     (uintptr_t)(h + inter) % a4 == 0 && (uintptr_t)q % 4 == 0;
    const long long n = (long long)rows * inter / (vec ? 4 : 1);
    const unsigned grid = grid_1d(n, kFNT, dev_info().cu_count * 4);
    if (vec)
        swq_quant<T, true><<<grid, kFNT, 0, s>>>(h, h + inter, part, nparts, q, scale_out, rows,
                                                 inter, ld);
    else
        swq_quant<T, false><<<grid, kFNT, 0, s>>>(h, h + inter, part, nparts, q, scale_out,
                                                  rows, inter, ld);
    launch_check("swiglu_quant quantize kernel launch");
}

}  // namespace

void qgemm_swiglu_quant_codes(int dtype, const signed char* a_q, const float* sa_dev,
                              const signed char* w_gu, const float* w_scales, void* h,
                              signed char* q, float* scale_out, int rows, int inter, int k,
                              hipStream_t s) {
#define FT_QSW(T)                                                                       \
    qgemm_swq_run<T>(a_q, sa_dev, w_gu, w_scales, (T*)h, q, scale_out, rows, inter, k, \
                     dtype, s, false)
    switch (dtype) {
    case FT_DT_F32: FT_QSW(float); break;
    case FT_DT_BF16: FT_QSW(bf16); break;
    case FT_DT_F16: FT_QSW(f16); break;
    default: inval("qgemm_swiglu_quant: unknown dtype code");
    }
#undef FT_QSW
}

namespace {

// ---------------------------------------------------------------------------
// rope_kv_append_paged: one thread per (sequence b, head, pair j) of the
// Hq + Hkv rotated heads, plus one per (b, v head, pair) copied. The QKV row
// of sequence b is qkv[b * ld + (head * D ..)], heads ordered q | k | v.
// ---------------------------------------------------------------------------
template <typename T, bool NEOX, int FK>
__global__ __launch_bounds__(256) void rope_kv_kernel(
    const T* __restrict__ qkv, long long ld, KFold fold, T* __restrict__ qkv_out,
    const int* __restrict__ lens, int* __restrict__ lens_next, const int* __restrict__ table,
    T* __restrict__ q_out, T* __restrict__ k_pool, T* __restrict__ v_pool, int batch, int hq,
    int hkv, int dim, int page, int tbl_width, double theta, int pos_offset) {
    const int half = dim >> 1;
    const int heads = hq + 2 * hkv;
    const long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= (long long)batch * heads * half) return;
    const int b = (int)(p / ((long long)heads * half));
    const int rem = (int)(p - (long long)b * heads * half);
    const int h = rem / half, j = rem - (rem / half) * half;
    const int slot = lens[b];
    // the sequence's length after the append, for the attention that follows
    if (lens_next && rem == 0) lens_next[b] = slot + 1;
    const size_t row0 = (size_t)b * ld + (size_t)h * dim;
    const int i1 = NEOX ? j : 2 * j;
    const int i2 = NEOX ? j + half : 2 * j + 1;
    // the two inputs: the GEMM output as stored in T, read back or folded
    // from the K-split partials (and then also stored, as the GEMM would)
    constexpr bool FOLD = FK > 0;
    float x1, x2;
    if constexpr (FOLD) {
        const float sa = kfold_sa(fold);
        const int c1 = h * dim + i1, c2 = h * dim + i2;
        const int a1 = kfold_sum<FK>(fold, row0 + i1), a2 = kfold_sum<FK>(fold, row0 + i2);
        x1 = kfold_value<T>(a1, kfold_scale(fold, sa, c1));
        x2 = kfold_value<T>(a2, kfold_scale(fold, sa, c2));
        St<T>::st(qkv_out + row0 + i1, x1);
        St<T>::st(qkv_out + row0 + i2, x2);
    } else {
        x1 = St<T>::ld(qkv + row0 + i1);
        x2 = St<T>::ld(qkv + row0 + i2);
    }
    // destination row of a K / V head: skipped if the slot is outside the
    // table's capacity (the device lengths are trusted, never read back)
    auto cache_row = [&](T* pool, int kv) -> T* {
        if (slot < 0 || slot >= tbl_width * page) return nullptr;
        const int blk = table[(size_t)b * tbl_width + slot / page];
        return pool + (((size_t)blk * hkv + kv) * page + slot % page) * dim;
    };
    if (h >= hq + hkv) {  // v head: copy two elements
        T* dst = cache_row(v_pool, h - hq - hkv);
        if (dst) {
            if constexpr (FOLD) {
                St<T>::st(dst + i1, x1);
                St<T>::st(dst + i2, x2);
            } else {  // the stored bits, NaN payloads included
                dst[i1] = qkv[row0 + i1];
                dst[i2] = qkv[row0 + i2];
            }
        }
        return;
    }
    const long long m = (long long)slot + pos_offset;
    const double angle = (double)m * pow(theta, -2.0 * j / dim);
    double sn, cs;
    sincos(angle, &sn, &cs);
    const float y1 = (float)(x1 * cs - x2 * sn);
    const float y2 = (float)(x1 * sn + x2 * cs);
    T* dst = h < hq ? q_out + ((size_t)b * hq + h) * dim : cache_row(k_pool, h - hq);
    if (dst) {
        St<T>::st(dst + i1, y1);
        St<T>::st(dst + i2, y2);
    }
}

void rope_kv_check(long long ld, const int* lens, const int* table, const void* q_out,
                   const void* k_pool, const void* v_pool, int batch, int hq, int hkv, int dim,
                   int page, int tbl_width, int pos_offset) {
    if (batch < 0 || hq < 1 || hkv < 1 || dim < 2 || dim % 2 != 0)
        inval("rope_kv_append: batch >= 0, heads >= 1 and an even dim >= 2 are required");
    if (page < 1 || tbl_width < 0) inval("rope_kv_append: page >= 1, table width >= 0");
    if (ld < (long long)(hq + 2 * hkv) * dim) inval("rope_kv_append: qkv row stride too small");
    if (pos_offset < 0) inval("pos_offset must be >= 0");
    if ((long long)tbl_width * page > (1LL << 30)) inval("table capacity too large");
    if (batch > 0 && (!lens || !table || !q_out || !k_pool || !v_pool))
        inval("rope_kv_append: null operand");
    if ((long long)batch * (hq + 2 * hkv) * (dim / 2) > (1LL << 40))
        inval("rope_kv_append: problem too large");
}

// FOLD: the input row is the K-split GEMM's partials `fold` (ld = its n),
// folded in the kernel and also stored into qkv_out
template <typename T, bool FOLD>
void rope_kv_launch(const T* qkv, long long ld, const KFold& fold, T* qkv_out, const int* lens,
                    const int* table, T* q_out, T* k_pool, T* v_pool, int batch, int hq,
                    int hkv, int dim, int page, int tbl_width, float theta, int pos_offset,
                    bool neox, hipStream_t s, int* lens_next = nullptr) {
    if (batch == 0) return;
    const long long threads = (long long)batch * (hq + 2 * hkv) * (dim / 2);
    const unsigned grid = (unsigned)((threads + 255) / 256);
    const int fk = FOLD ? kfold_width(fold.ksplit) : 0;
#define FT_ROPE(NEOX_, FK_)                                                                \
    rope_kv_kernel<T, NEOX_, FK_><<<grid, 256, 0, s>>>(                                    \
        qkv, ld, fold, qkv_out, lens, lens_next, table, q_out, k_pool, v_pool, batch, hq, \
        hkv, dim, page, tbl_width, (double)theta, pos_offset)
    if (neox) {
        if (fk == 0) FT_ROPE(true, 0);
        else if (fk == 4) FT_ROPE(true, 4);
        else if (fk == 8) FT_ROPE(true, 8);
        else FT_ROPE(true, 1);
    } else {
        if (fk == 0) FT_ROPE(false, 0);
        else if (fk == 4) FT_ROPE(false, 4);
        else if (fk == 8) FT_ROPE(false, 8);
        else FT_ROPE(false, 1);
    }
#undef FT_ROPE
    launch_check("rope_kv_append kernel launch");
}

template <typename T>
void rope_kv_run(const T* qkv, long long ld, const int* lens, const int* table,
                 T* q_out, T* k_pool, T* v_pool, int batch, int hq, int hkv,
                 int dim, int page, int tbl_width, float theta, int pos_offset,
                 bool neox, hipStream_t s) {
    rope_kv_check(ld, lens, table, q_out, k_pool, v_pool, batch, hq, hkv, dim, page, tbl_width,
                  pos_offset);
    if (batch > 0 && !qkv) inval("rope_kv_append: null operand");
    rope_kv_launch<T, false>(qkv, ld, KFold{}, nullptr, lens, table, q_out, k_pool, v_pool,
                             batch, hq, hkv, dim, page, tbl_width, theta, pos_offset, neox, s);
}

// QKV GEMM (a_q [batch, k] codes with the device scale *sa_dev, w_q [n, k],
// per-channel w_scales) -> qkv [batch, n] in T, then rope_kv_run on it. A
// K-split GEMM's partials are folded by the RoPE kernel itself.
template <typename T>
void qgemm_rope_kv_run(const signed char* a_q, const float* sa_dev, const signed char* w_q,
                       const float* w_scales, T* qkv, const int* lens, const int* table,
                       T* q_out, T* k_pool, T* v_pool, int batch, int hq, int hkv, int dim,
                       int k, int page, int tbl_width, float theta, int pos_offset, bool neox,
                       int dtype, hipStream_t s, int* lens_next = nullptr) {
    const long long n = (long long)(hq + 2 * hkv) * dim;
    rope_kv_check(n, lens, table, q_out, k_pool, v_pool, batch, hq, hkv, dim, page, tbl_width,
                  pos_offset);
    if (n > (1LL << 30)) inval("qgemm_rope_kv_append: too many heads");
    if (k < 1) inval("qgemm_rope_kv_append: k must be >= 1");
    if (batch == 0) return;
    if (!a_q || !sa_dev || !w_q || !w_scales || !qkv)
        inval("qgemm_rope_kv_append: null operand");
    KFold fold;
    if (qgemm_deferred(a_q, w_q, sa_dev, w_scales, qkv, dtype, batch, (int)n, k, s,
                       fold))
        rope_kv_launch<T, true>(nullptr, n, fold, qkv, lens, table, q_out, k_pool, v_pool,
                                batch, hq, hkv, dim, page, tbl_width, theta, pos_offset, neox,
                                s, lens_next);
    else
        rope_kv_launch<T, false>(qkv, n, KFold{}, nullptr, lens, table, q_out, k_pool, v_pool,
                                 batch, hq, hkv, dim, page, tbl_width, theta, pos_offset, neox,
                                 s, lens_next);
}

}  // namespace

void qkv_rope_step(int dtype, const signed char* a_q, const float* sa_dev,
                   const signed char* w_q, const float* w_scales, int k, void* qkv,
                   const int* lens, int* lens_next, const int* table, void* q_out,
                   void* k_pool, void* v_pool, int batch, int hq, int hkv, int dim, int page,
                   int tbl_width, float theta, int pos_offset, bool neox, hipStream_t s) {
#define FT_QRK(T)                                                                           \
    qgemm_rope_kv_run<T>(a_q, sa_dev, w_q, w_scales, (T*)qkv, lens, table, (T*)q_out,       \
                         (T*)k_pool, (T*)v_pool, batch, hq, hkv, dim, k, page, tbl_width,    \
                         theta, pos_offset, neox, dtype, s, lens_next)
    switch (dtype) {
    case FT_DT_F32: FT_QRK(float); break;
    case FT_DT_BF16: FT_QRK(bf16); break;
    case FT_DT_F16: FT_QRK(f16); break;
    default: inval("qgemm_rope_kv_append: unknown dtype code");
    }
#undef FT_QRK
}

}  // namespace ft

extern "C" {

int ft_rmsnorm_quant_launch(const void* x, int x_dtype, const float* w,
                            const void* residual, signed char* q,
                            float* scale_out, int rows, int cols, float eps,
                            uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
        switch (x_dtype) {
        case FT_DT_F32:
            ft::rmsnorm_quant_run<float>((const float*)x, w, (const float*)residual, q,
                                         scale_out, rows, cols, eps, s);
            break;
        case FT_DT_BF16:
            ft::rmsnorm_quant_run<ft::bf16>((const ft::bf16*)x, w, (const ft::bf16*)residual,
                                            q, scale_out, rows, cols, eps, s);
            break;
        case FT_DT_F16:
            ft::rmsnorm_quant_run<ft::f16>((const ft::f16*)x, w, (const ft::f16*)residual,
                                           q, scale_out, rows, cols, eps, s);
            break;
        default:
            ft::inval("rmsnorm_quant: unknown dtype code");
        }
    });
}

int ft_swiglu_quant_launch(const void* gate, const void* up, int dtype,
                           signed char* q, float* scale_out, int rows, int cols,
                           long long ld, uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
        switch (dtype) {
        case FT_DT_F32:
            ft::swiglu_quant_run<float>((const float*)gate, (const float*)up, q, scale_out,
                                        rows, cols, ld, s);
            break;
        case FT_DT_BF16:
            ft::swiglu_quant_run<ft::bf16>((const ft::bf16*)gate, (const ft::bf16*)up, q,
                                           scale_out, rows, cols, ld, s);
            break;
        case FT_DT_F16:
            ft::swiglu_quant_run<ft::f16>((const ft::f16*)gate, (const ft::f16*)up, q,
                                          scale_out, rows, cols, ld, s);
            break;
        default:
            ft::inval("swiglu_quant: unknown dtype code");
        }
    });
}

int ft_rope_kv_append_paged_launch(const void* qkv, int dtype, long long ld,
                                   const int* lens, const int* table, void* q_out,
                                   void* k_pool, void* v_pool, int batch,
                                   int q_heads, int kv_heads, int dim, int page,
                                   int tbl_width, float theta, int pos_offset,
                                   int neox, uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
        switch (dtype) {
        case FT_DT_F32:
            ft::rope_kv_run<float>((const float*)qkv, ld, lens, table, (float*)q_out,
                                   (float*)k_pool, (float*)v_pool, batch, q_heads,
                                   kv_heads, dim, page, tbl_width, theta, pos_offset,
                                   neox != 0, s);
            break;
        case FT_DT_BF16:
            ft::rope_kv_run<ft::bf16>((const ft::bf16*)qkv, ld, lens, table,
                                      (ft::bf16*)q_out, (ft::bf16*)k_pool,
                                      (ft::bf16*)v_pool, batch, q_heads, kv_heads, dim,
                                      page, tbl_width, theta, pos_offset, neox != 0, s);
            break;
        case FT_DT_F16:
            ft::rope_kv_run<ft::f16>((const ft::f16*)qkv, ld, lens, table,
                                     (ft::f16*)q_out, (ft::f16*)k_pool,
                                     (ft::f16*)v_pool, batch, q_heads, kv_heads, dim,
                                     page, tbl_width, theta, pos_offset, neox != 0, s);
            break;
        default:
            ft::inval("rope_kv_append: unknown dtype code");
        }
    });
}

int ft_qgemm_rope_kv_append_paged_launch(const signed char* a_q, const float* sa_dev,
                                         const signed char* w_q, const float* w_scales,
                                         int k, int dtype, void* qkv, const int* lens,
                                         const int* table, void* q_out, void* k_pool,
                                         void* v_pool, int batch, int q_heads, int kv_heads,
                                         int dim, int page, int tbl_width, float theta,
                                         int pos_offset, int neox, uintptr_t stream) {
    return ft::guarded([&] {
        ft::qkv_rope_step(dtype, a_q, sa_dev, w_q, w_scales, k, qkv, lens, nullptr, table,
                          q_out, k_pool, v_pool, batch, q_heads, kv_heads, dim, page,
                          tbl_width, theta, pos_offset, neox != 0, ft::as_stream(stream));
    });
}

int ft_qgemm_rmsnorm_quant_launch(const signed char* a_q, const float* sa_dev,
                                  const signed char* w_q, const float* w_scales, int dtype,
                                  void* y, const void* residual, const float* w, float eps,
                                  signed char* q, float* scale_out, int rows, int n, int k,
                                  uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
#define FT_QRQ(T)                                                                          \
    ft::qgemm_rmsq_run<T>(a_q, sa_dev, w_q, w_scales, (T*)y, (const T*)residual, w, eps, q, \
                          scale_out, rows, n, k, dtype, s)
        switch (dtype) {
        case FT_DT_F32: FT_QRQ(float); break;
        case FT_DT_BF16: FT_QRQ(ft::bf16); break;
        case FT_DT_F16: FT_QRQ(ft::f16); break;
        default: ft::inval("qgemm_rmsnorm_quant: unknown dtype code");
        }
#undef FT_QRQ
    });
}

int ft_qgemm_swiglu_quant_launch(const signed char* a_q, const float* sa_dev,
                                 const signed char* w_gu, const float* w_scales, int dtype,
                                 void* h, signed char* q, float* scale_out, int rows, int inter,
                                 int k, uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
#define FT_QSQ(T) \
    ft::qgemm_swq_run<T>(a_q, sa_dev, w_gu, w_scales, (T*)h, q, scale_out, rows, inter, k, dtype, s)
        switch (dtype) {
        case FT_DT_F32: FT_QSQ(float); break;
        case FT_DT_BF16: FT_QSQ(ft::bf16); break;
        case FT_DT_F16: FT_QSQ(ft::f16); break;
        default: ft::inval("qgemm_swiglu_quant: unknown dtype code");
        }
#undef FT_QSQ
    });
}

}  // extern "C"
