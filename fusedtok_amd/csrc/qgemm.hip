// W8A8 GEMM for gfx950:  y[M,N] = float(int32(A_q[M,K] . B_q[N,K]^T)) * s_j
//
//   per-tensor   s_j = f32(sa * sb)        (reference qgemm.cu:612-629)
//   per-channel  s_j = f32(sa * sb[j])     (reference qgemm.cu:631-652)
//
// The int32 accumulation is exact in any order, the scale is composed with
// one f32 rounding and applied with one product, so the float32 output is
// bit-identical to the reference CPU path; bf16 / fp16 outputs are that f32
// value rounded to nearest-even.
//
// Kernels
//   qgemv_dot4     M == 1 (any M <= 8 when forced; decode GEMV, no MFMA):
//                  v_dot4_i32_i8 over 16-byte K pieces, several W rows in
//                  flight per wave, wave sums.
//   qgemm_dec_lds  2 <= M <= 16, K % 512 == 0, >= 320 column tiles: one
//                  wave per 16 columns over all of K; W and A rows DMA'd
//                  global->LDS in whole lines through a 2-stage ring, read
//                  back in the MFMA layout through an XOR swizzle.
//   qgemm_dec      2 <= M <= 16: 16 columns per workgroup over all of K, K
//                  split across the workgroup's waves, operands double-
//                  buffered in registers, partials folded in LDS.
//   qgemm_skinny_lds 16 < M <= 64, K % 256 == 0: the skinny tiling below with
//                  both operands DMA'd global->LDS in whole lines (256-byte
//                  K chunks, 2-stage ring, XOR-swizzled fragment reads).
//   qgemm_skinny   16 < M <= 64: W streamed once into the B operand of
//                  v_mfma_i32_16x16x64_i8, 64 columns per workgroup (A shared
//                  through L1), K split across workgroups when N alone cannot
//                  fill the chip; int32 partials folded by qgemm_ksum.
//   qgemm_big_w16  M, N >= 256, K % 128 == 0 (default): persistent 256x256
//                  tiles, 8 waves (two per SIMD, 64x128 each, on
//                  v_mfma_i32_16x16x64_i8), 128-byte K slabs DMA'd
//                  global->LDS into two stages.
//   qgemm_big_dma  M, N >= 256, K % 64 == 0: 256x256 tiles on
//                  v_mfma_i32_32x32x32_i8 fed by a 5-stage global->LDS DMA
//                  ring; LDS-staged, coalesced epilogue.
//   qgemm_big      M, N >= 256, other K: the same tiles, register-staged.
//   qgemm_tiled    64 < M (< 256 or N < 256): 128x128 tiles, 64-byte slabs
//                  double-buffered through LDS.
//   qgemm_scalar   any shape/alignment (K % 16 != 0, misaligned views).
//   K == 0         zero fill (a kernel, not a memset, so it captures cleanly).
#include "ft_common.hpp"
#include "kfold.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace ft {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef signed char i8;

enum OutKind { kOutF32 = 0, kOutBF16 = 1, kOutF16 = 2, kOutI32 = 3 };

typedef __attribute__((address_space(3))) void* lds_void_p;

// s_waitcnt with only the vector-memory count bounded (gfx9 encoding;
// expcnt and lgkmcnt fields at their maxima = no wait).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// 16-byte LDS read issued as inline asm, so that the compiler's tracking of
// global->LDS DMA does not put a vmcnt(0) before it; the value is valid
// only after an lgkmcnt wait that ties it (asm with the value as an in/out
// operand, so that its uses stay below the wait).
__device__ __forceinline__ i32x4 lds_read16(unsigned addr) {
    i32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

struct Epi {
    void* y;
    float sa;
    const float* sa_dev;  // device scale overrides sa when non-null
    float sb;
    const float* sb_vec;  // per-channel scales, null = per-tensor sb
};

__device__ __forceinline__ float epi_sa(const Epi& e) {
    return e.sa_dev ? *e.sa_dev : e.sa;
}

// Store of one output given the composed scale s = f32(sa * sb_j): two f32
// roundings (scale, then product), then one to the output type - never
// fused: the backend would otherwise fold the product and an f16 narrowing
// into one single-rounding mixed-precision FMA (v_fma_mixlo_f16), which can
// land on the other side of an f16 tie. The empty asm makes the rounded f32
// product opaque to it.
template <int OUT>
__device__ __forceinline__ void epi_store_scaled(const Epi& e, int n, int row, int col,
                                                 int acc, float s) {
    const size_t idx = (size_t)row * n + col;
    if constexpr (OUT == kOutI32) {
        static_cast<int*>(e.y)[idx] = acc;
    } else {
        float val = (float)acc * s;
        asm("" : "+v"(val));
        if constexpr (OUT == kOutF32) static_cast<float*>(e.y)[idx] = val;
        if constexpr (OUT == kOutBF16) static_cast<bf16*>(e.y)[idx] = (bf16)val;
        if constexpr (OUT == kOutF16) static_cast<f16*>(e.y)[idx] = (f16)val;
    }
}

// the value epi_store_scaled stores for (acc, s), widened back to f32
template <int OUT>
__device__ __forceinline__ float epi_stored(int acc, float s) {
    float val = (float)acc * s;
    asm("" : "+v"(val));
    if constexpr (OUT == kOutBF16) return (float)(bf16)val;
    if constexpr (OUT == kOutF16) return (float)(f16)val;
    return val;
}

template <int OUT>
__device__ __forceinline__ void epi_store(const Epi& e, float sa, int n,
                                          int row, int col, int acc) {
    float s = 0.0f;
    if constexpr (OUT != kOutI32) s = e.sb_vec ? sa * e.sb_vec[col] : sa * e.sb;
    epi_store_scaled<OUT>(e, n, row, col, acc, s);
}

// ---------------------------------------------------------------------------
// zero fill (K == 0): an empty dot product is 0 on every output type
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void zero_fill_kernel(unsigned char* p,
                                                        long long bytes) {
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < bytes; i += stride)
        p[i] = 0;
}

// ---------------------------------------------------------------------------
// scalar fallback
// ---------------------------------------------------------------------------
template <int OUT>
__global__ __launch_bounds__(256) void qgemm_scalar(const i8* __restrict__ a,
                                                    const i8* __restrict__ b,
                                                    Epi e, int m, int n, int k) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long long)m * n) return;
    const int row = (int)(idx / n), col = (int)(idx - (long long)row * n);
    const i8* ar = a + (size_t)row * k;
    const i8* br = b + (size_t)col * k;
    int acc = 0;
    for (int p = 0; p < k; ++p) acc += (int)ar[p] * (int)br[p];
    epi_store<OUT>(e, epi_sa(e), n, row, col, acc);
}

// ---------------------------------------------------------------------------
// decode GEMV (M <= 8, no MFMA): y[m][j] = sum_k A[m][k] * W[j][k] on
// v_dot4_i32_i8. A wave owns kGemvRows consecutive W rows at a time; its
// lanes span K in 16-byte pieces (lane l reads bytes 16 l + 1024 c of each
// row, so one load instruction covers 1 KB of a row contiguously). K is
// walked in passes of kGemvChunks KB: all weight and activation pieces of a
// pass are loaded before any is consumed, so a 4096-byte row costs one
// memory round trip. Every lane keeps the M x rows partial dot products,
// summed across the wave at the end (integer sums: exact in any order).
// ---------------------------------------------------------------------------
constexpr int kGemvRows = 4;
constexpr int kGemvChunks = 4;

template <int M_, int OUT>
__global__ __launch_bounds__(256) void qgemv_dot4(const i8* __restrict__ a,
                                                  const i8* __restrict__ b,
                                                  Epi e, int n, int k) {
    const int lane = threadIdx.x & 63;
    const int gwave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nwaves = gridDim.x * 4;
    const float sa = epi_sa(e);
    for (int j0 = gwave * kGemvRows; j0 < n; j0 += nwaves * kGemvRows) {
        int acc[kGemvRows][M_];
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
            for (int mm = 0; mm < M_; ++mm) acc[r][mm] = 0;
        for (int kp = 0; kp < k; kp += 1024 * kGemvChunks) {
            i32x4 w[kGemvChunks][kGemvRows], x[kGemvChunks][M_];
#pragma unroll
            for (int c = 0; c < kGemvChunks; ++c) {
                const int kk = kp + 1024 * c + 16 * lane;
                const bool kok = kk < k;  // k % 16 == 0: a piece is all in or out
                const i32x4 z = {0, 0, 0, 0};
#pragma unroll
                for (int r = 0; r < kGemvRows; ++r) {
                    const int row = min(j0 + r, n - 1);
                    // W is read once: non-temporal (1 KB of a row per
                    // instruction, whole lines; N=11008 K=4096: 10.6 vs
                    // 11.7 us with plain loads)
                    w[c][r] = kok ? __builtin_nontemporal_load(
                                        reinterpret_cast<const i32x4*>(b + (size_t)row * k + kk))
                                  : z;
                }
#pragma unroll
                for (int mm = 0; mm < M_; ++mm)
                    x[c][mm] = kok ? *reinterpret_cast<const i32x4*>(a + (size_t)mm * k + kk) : z;
            }
#pragma unroll
            for (int c = 0; c < kGemvChunks; ++c)
#pragma unroll
                for (int mm = 0; mm < M_; ++mm)
#pragma unroll
                    for (int r = 0; r < kGemvRows; ++r) {
                        int s = acc[r][mm];
                        s = __builtin_amdgcn_sdot4(w[c][r][0], x[c][mm][0], s, false);
                        s = __builtin_amdgcn_sdot4(w[c][r][1], x[c][mm][1], s, false);
                        s = __builtin_amdgcn_sdot4(w[c][r][2], x[c][mm][2], s, false);
                        s = __builtin_amdgcn_sdot4(w[c][r][3], x[c][mm][3], s, false);
                        acc[r][mm] = s;
                    }
        }
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
            for (int mm = 0; mm < M_; ++mm) {
                int v = acc[r][mm];
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
                acc[r][mm] = v;
            }
        // lane r * M_ + mm stores (r, mm)
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
            for (int mm = 0; mm < M_; ++mm)
                if (lane == r * M_ + mm && j0 + r < n)
                    epi_store<OUT>(e, sa, n, mm, j0 + r, acc[r][mm]);
    }
}

// ---------------------------------------------------------------------------
// RMSNorm -> per-tensor int8 quantize -> GEMV in one launch (one row,
// K <= 4096). Every workgroup normalises and quantises the row itself (8 KB
// of x from L2) with rmsnorm_quant's single-row arithmetic - thread t of 256
// takes 4-element chunks t, t + 256, ..; fmaf sum of squares; wave
// butterfly; the 4 wave totals in order; inv = 1 / sqrtf(total / K + eps);
// y = (v * inv) * w; scale = max|y| / 127; codes rint(y * (1 / scale)) -
// so its codes and scale are those of rmsnorm_quant bit for bit, and keeps
// the codes in LDS for the dot products. The wave's first weight rows are
// loaded before the normalisation, so the two overlap. Workgroup 0 also
// writes the codes and the scale. Each wave owns an even share of the rows
// (to within one); the dot products and the epilogue are qgemv_dot4's for
// M = 1 with sa = the computed scale.
// ---------------------------------------------------------------------------
template <typename T, bool RES, int OUT>
__global__ __launch_bounds__(256) void rmsq_gemv(
    const T* __restrict__ x, const T* __restrict__ res, const float* __restrict__ wn,
    float eps, const i8* __restrict__ b, Epi e, int n, int k, i8* __restrict__ q_out,
    float* __restrict__ scale_out) {
    static_assert(kGemvChunks * 1024 == 4096, "one pass covers K <= 4096");
    __shared__ __attribute__((aligned(16))) i8 xq[kGemvChunks * 1024];
    __shared__ float red[4], redm[4];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int gwave = blockIdx.x * 4 + wv;
    const int nwaves = gridDim.x * 4;
    // wave w owns rows [w n / nwaves, (w + 1) n / nwaves): every wave of the
    // grid gets the same number of rows to within one
    const int j_first = (int)((long long)gwave * n / nwaves);
    const int j_end = (int)((long long)(gwave + 1) * n / nwaves);
    const i32x4 z = {0, 0, 0, 0};

    i32x4 w[kGemvChunks][kGemvRows];
    // every load is issued, rows and K pieces clamped to real ones, so no
    // branch separates the loads and the compiler's wait counts stay exact;
    // a piece past K meets a zero activation piece below
    auto load_w = [&](int j0) {
#pragma unroll
        for (int c = 0; c < kGemvChunks; ++c) {
            const int kk = 1024 * c + 16 * lane;
#pragma unroll
            for (int r = 0; r < kGemvRows; ++r) {
                const int row = min(j0 + r, max(j_end - 1, 0));
                w[c][r] = __builtin_nontemporal_load(
                    reinterpret_cast<const i32x4*>(b + (size_t)row * k + min(kk, k - 16)));
            }
        }
    };
    // the row, its residual and the norm weights first, then this wave's
    // weight rows: loads complete in issue order, so the normalisation
    // below waits only for the row and runs while the weights stream in
    const int chunks = k >> 2;
    float4 v[4], rv[4], wc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = min(tid + 256 * j, chunks - 1);  // clamped: a real chunk
        v[j] = St<T>::ld4(x + 4 * c);
        if constexpr (RES) rv[j] = St<T>::ld4(res + 4 * c);
        wc[j] = *reinterpret_cast<const float4*>(wn + 4 * c);
    }
    // a wave past the last column tile loads clamped real rows it never uses
    __builtin_amdgcn_sched_barrier(0);
    load_w(j_first);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (RES) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j].x += rv[j].x; v[j].y += rv[j].y; v[j].z += rv[j].z; v[j].w += rv[j].w;
        }
    }

    // normalise and quantise the row (rmsnorm_quant's order)
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (tid + 256 * j < chunks) {
            acc = fmaf(v[j].x, v[j].x, acc);
            acc = fmaf(v[j].y, v[j].y, acc);
            acc = fmaf(v[j].z, v[j].z, acc);
            acc = fmaf(v[j].w, v[j].w, acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) red[wv] = acc;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)k + eps);
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (tid + 256 * j < chunks) {
            m = fmaxf(m, fabsf(v[j].x * inv * wc[j].x));
            m = fmaxf(m, fabsf(v[j].y * inv * wc[j].y));
            m = fmaxf(m, fabsf(v[j].z * inv * wc[j].z));
            m = fmaxf(m, fabsf(v[j].w * inv * wc[j].w));
        }
    }
    m = wave_max(m);
    if (lane == 0) redm[wv] = m;
    __syncthreads();
    m = redm[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) m = fmaxf(m, redm[i]);
    const float scale = make_scale(m);
    const float inv_s = 1.0f / scale;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = tid + 256 * j;
        if (c < chunks) {
            char4 o;
            o.x = quant1(v[j].x * inv * wc[j].x, inv_s);
            o.y = quant1(v[j].y * inv * wc[j].y, inv_s);
            o.z = quant1(v[j].z * inv * wc[j].z, inv_s);
            o.w = quant1(v[j].w * inv * wc[j].w, inv_s);
            *reinterpret_cast<char4*>(xq + 4 * c) = o;
            if (blockIdx.x == 0 && q_out) *reinterpret_cast<char4*>(q_out + 4 * c) = o;
        }
    }
    if (blockIdx.x == 0 && tid == 0 && scale_out) *scale_out = scale;
    __syncthreads();

    for (int j0 = j_first; j0 < j_end; j0 += kGemvRows) {
        if (j0 != j_first) load_w(j0);
        int accr[kGemvRows];
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r) accr[r] = 0;
#pragma unroll
        for (int c = 0; c < kGemvChunks; ++c) {
            const int kk = 1024 * c + 16 * lane;
            const i32x4 xv = kk < k ? *reinterpret_cast<const i32x4*>(xq + kk) : z;
#pragma unroll
            for (int r = 0; r < kGemvRows; ++r) {
                int sdot = accr[r];
                sdot = __builtin_amdgcn_sdot4(w[c][r][0], xv[0], sdot, false);
                sdot = __builtin_amdgcn_sdot4(w[c][r][1], xv[1], sdot, false);
                sdot = __builtin_amdgcn_sdot4(w[c][r][2], xv[2], sdot, false);
                sdot = __builtin_amdgcn_sdot4(w[c][r][3], xv[3], sdot, false);
                accr[r] = sdot;
            }
        }
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r) {
            int t = accr[r];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
            accr[r] = t;
        }
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r) {
            const int col = j0 + r;
            if (lane == r && col < j_end) {
                float s = 0.0f;
                if constexpr (OUT != kOutI32) s = e.sb_vec ? scale * e.sb_vec[col] : scale * e.sb;
                epi_store_scaled<OUT>(e, n, 0, col, accr[r], s);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// decode MFMA GEMM (M <= 16): a workgroup owns 16 output columns (W rows
// n0 .. n0 + 15) over the whole of K; its KW waves split K into 512-byte
// chunks taken round robin (wave w: chunks w, w + KW, ...), so each wave
// streams 16 rows x 512 B per chunk and no second launch is needed to fold
// a K split: the KW partial accumulators meet in LDS at the end (integer
// sums, exact in any order). Per 64-byte K step, lane (r, g) holds
// W[n0 + r][k + 16 g .. +15] (B operand of v_mfma_i32_16x16x64_i8) and
// A[r][k + 16 g .. +15] (A operand; rows past M read row M - 1 and only feed
// output rows that are never stored). Both operands are loaded straight to
// registers, double-buffered: chunk c + KW is in flight while chunk c is
// multiplied. Every load is unconditional (clamped address), so the
// compiler's vmcnt bookkeeping sees one fixed count per chunk; K pieces past
// the end are zeroed by a select on W.
// ---------------------------------------------------------------------------
constexpr int kDecChunk = 512;                // K bytes per chunk
constexpr int kDecSteps = kDecChunk / 64;     // MFMA K steps per chunk

template <int KW, int OUT>
__global__ __launch_bounds__(64 * KW) void qgemm_dec(
    const i8* __restrict__ a, const i8* __restrict__ b, Epi e, int m, int n,
    int k) {
    __shared__ i32x4 red[KW > 1 ? KW - 1 : 1][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const i8* brow = b + (size_t)min(n0 + r, n - 1) * k;
    const i8* arow = a + (size_t)min(r, m - 1) * k;
    const int chunks = (k + kDecChunk - 1) / kDecChunk;
    // K byte of step u's piece for this lane (lanes of one row group read
    // 64 contiguous bytes per step; wider per-lane runs measured no faster)
    auto piece = [&](int c, int u) { return c * kDecChunk + 64 * u + 16 * g; };

    i32x4 w0[kDecSteps], a0[kDecSteps], w1[kDecSteps], a1[kDecSteps];
    auto load = [&](int c, i32x4 (&wv)[kDecSteps], i32x4 (&av)[kDecSteps]) {
#pragma unroll
        for (int u = 0; u < kDecSteps; ++u) {
            // a piece past the end reads the row's last 16 bytes instead
            const int kb = min(piece(c, u), k - 16);
            wv[u] = *reinterpret_cast<const i32x4*>(brow + kb);
            av[u] = *reinterpret_cast<const i32x4*>(arow + kb);
        }
    };
    // the zeroing of pieces past K is applied here, next to the MFMA that
    // needs the value anyway (a select right after the load would make the
    // wave wait for each load in turn)
    auto mul = [&](int c, const i32x4 (&wv)[kDecSteps], const i32x4 (&av)[kDecSteps],
                   i32x4 acc) {
#pragma unroll
        for (int u = 0; u < kDecSteps; ++u) {
            const i32x4 wz = piece(c, u) < k ? wv[u] : i32x4{0, 0, 0, 0};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u], wz, acc, 0, 0, 0);
        }
        return acc;
    };

    // The loop body is one basic block: prefetches are issued whether or not
    // their chunk exists (clamped index), and a chunk past the end is
    // multiplied too, contributing zero (mul zeroes every W piece at or past
    // K). A load skipped or sunk on one path would make the compiler's wait
    // counts conservative, and the wave would wait for the prefetch it just
    // issued; sched_barrier keeps the scheduler from sinking a prefetch below
    // the multiplies it is meant to overlap.
    i32x4 acc = {0, 0, 0, 0};
    const int last = chunks - 1;
    load(min(wave, last), w0, a0);
    for (int c = wave; c < chunks; c += 2 * KW) {
        load(min(c + KW, last), w1, a1);
        __builtin_amdgcn_sched_barrier(0);
        acc = mul(c, w0, a0, acc);
        load(min(c + 2 * KW, last), w0, a0);
        __builtin_amdgcn_sched_barrier(0);
        acc = mul(c + KW, w1, a1, acc);
    }
    if (KW > 1) {
        if (wave > 0) red[wave - 1][lane] = acc;
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < KW - 1; ++w) {
            const i32x4 p = red[w][lane];
            acc[0] += p[0]; acc[1] += p[1]; acc[2] += p[2]; acc[3] += p[3];
        }
    }
    // lane (r, g) holds C[4 g + i][r] = (A row 4 g + i, W row n0 + r)
    const int col = n0 + r;
    if (col >= n) return;
    const float sa = epi_sa(e);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (4 * g + i < m) epi_store<OUT>(e, sa, n, 4 * g + i, col, acc[i]);
}

// ---------------------------------------------------------------------------
// decode MFMA GEMM through LDS (2 <= M <= 16, K % 512 == 0): one wave owns 16
// output columns over all of K, as qgemm_dec with KW = 1, but both operands
// arrive by global -> LDS DMA in whole 128-byte lines: one
// global_load_lds_dwordx4 covers 512 bytes of each of two rows (lanes 0-31
// the first, 32-63 the second), where the register path reads 64 bytes of
// each of 16 rows per instruction. An S-stage ring keeps S - 1 chunks of
// 16 W rows and 16 A rows x 512 bytes in flight.
//
// LDS layout of a stage: operand x (0 = A, 1 = W), row r, 16-byte slot s at
// x * 8192 + 512 r + 16 s holds K piece s ^ r of the chunk (lane l of a DMA
// reads piece (l & 31) ^ r, a permutation of each aligned group of 8 pieces,
// so every 8 lanes still cover one whole line). MFMA step u of lane (r, g)
// needs piece 4 u + g: slot (4 u + g) ^ r, and the 16 lanes of a ds_read_b128
// quarter (r = 0..15) hit 16 distinct 16-byte bank groups.
// ---------------------------------------------------------------------------
constexpr int kDwChunk = 512;
constexpr int kDwStage = 2 * 16 * kDwChunk;  // A and W, 16 rows each

template <int NSTAGE>
__device__ __forceinline__ void dw_wait_vm(int pending_chunks) {
    // 16 DMA instructions per chunk; waits until at most `pending_chunks`
    // chunks issued after the one needed are still in flight
    static_assert(NSTAGE >= 2 && NSTAGE <= 3, "stage count");
    switch (pending_chunks) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<16>(); break;
    default: wait_vmcnt<32>(); break;
    }
}

template <int NSTAGE, int CPOL, int OUT>
__global__ __launch_bounds__(64) void qgemm_dec_lds(
    const i8* __restrict__ a, const i8* __restrict__ b, Epi e, int m, int n, int k) {
    __shared__ __attribute__((aligned(16))) char lds[NSTAGE * kDwStage];
    const int lane = threadIdx.x;
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int chunks = k / kDwChunk;

    // DMA instruction i (0..7) of an operand: rows 2 i + (lane >> 5)
    const int hi = lane >> 5;
    const int sl = lane & 31;
    size_t aoff[8], boff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = 2 * i + hi;
        const int piece = sl ^ row;
        aoff[i] = (size_t)min(row, m - 1) * k + 16 * piece;
        boff[i] = (size_t)min(n0 + row, n - 1) * k + 16 * piece;
    }
    auto issue = [&](int c, int st) {
        char* dst = lds + st * kDwStage;
        const size_t kc = (size_t)c * kDwChunk;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_global_load_lds(b + boff[i] + kc,
                                             (lds_void_p)(dst + 16 * kDwChunk + 1024 * i), 16,
                                             0, CPOL);
            __builtin_amdgcn_global_load_lds(a + aoff[i] + kc, (lds_void_p)(dst + 1024 * i),
                                             16, 0, 0);
        }
    };

    const unsigned lds0 = lds_addr(lds);
    unsigned fo[kDecSteps];  // byte offset of step u's fragment in an operand
#pragma unroll
    for (int u = 0; u < kDecSteps; ++u) fo[u] = 512 * r + 16 * ((4 * u + g) ^ r);

#pragma unroll
    for (int j = 0; j < NSTAGE - 1; ++j)
        if (j < chunks) issue(j, j);

    i32x4 acc = {0, 0, 0, 0};
    int st = 0;
    for (int c = 0; c < chunks; ++c) {
        const int nxt = c + NSTAGE - 1;
        if (nxt < chunks) {
            issue(nxt, nxt % NSTAGE);
            dw_wait_vm<NSTAGE>(NSTAGE - 1);
        } else {
            dw_wait_vm<NSTAGE>(chunks - 1 - c);
        }
        const unsigned sa_ = lds0 + st * kDwStage;
        i32x4 fa[kDecSteps], fw[kDecSteps];
#pragma unroll
        for (int u = 0; u < kDecSteps; ++u) {
            fa[u] = lds_read16(sa_ + fo[u]);
            fw[u] = lds_read16(sa_ + 16 * kDwChunk + fo[u]);
        }
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fa[4]),
                       "+v"(fa[5]), "+v"(fa[6]), "+v"(fa[7]), "+v"(fw[0]), "+v"(fw[1]),
                       "+v"(fw[2]), "+v"(fw[3]), "+v"(fw[4]), "+v"(fw[5]), "+v"(fw[6]),
                       "+v"(fw[7]));
#pragma unroll
        for (int u = 0; u < kDecSteps; ++u)
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[u], fw[u], acc, 0, 0, 0);
        st = st + 1 == NSTAGE ? 0 : st + 1;
    }
    // lane (r, g) holds C[4 g + i][r] = (A row 4 g + i, W row n0 + r)
    const int col = n0 + r;
    if (col >= n) return;
    const float sa = epi_sa(e);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (4 * g + i < m) epi_store<OUT>(e, sa, n, 4 * g + i, col, acc[i]);
}

// ---------------------------------------------------------------------------
// skinny MFMA GEMM (M <= 16*MT <= 64): a workgroup covers 64 output columns,
// wave w the 16 columns of W rows [64 bx + 16 w, +16), over the workgroup's
// K range (K split across blockIdx.y when N alone cannot fill the chip).
// K is walked in 1 KB chunks. Per chunk, the A rows are copied into LDS
// once for the whole workgroup (global_load_lds_dwordx4: one instruction
// per 1 KB row, rows padded to kSkPitch bytes so the 16 rows of a fragment
// read fall in distinct banks), while each wave has all 16 of its W K-steps
// (lane (r, g): W[n0 + r][k + 16 g .. +15], the B operand of
// v_mfma_i32_16x16x64_i8) in flight. With a K split, int32 partials go to
// scratch and qgemm_ksum folds them (fixed order, exact) and applies the
// epilogue: a second launch instead of a device-scope fence per workgroup.
// ---------------------------------------------------------------------------
constexpr int kSkChunk = 1024;           // K bytes per chunk
constexpr int kSkSteps = kSkChunk / 64;  // MFMA K steps per chunk
constexpr int kSkPitch = kSkChunk + 16;  // LDS row pitch of staged A rows

template <int MT, int OUT>
__global__ __launch_bounds__(256) void qgemm_skinny(
    const i8* __restrict__ a, const i8* __restrict__ b, Epi e, int m, int n,
    int k, int ksplit, int* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) i8 sa_rows[16 * MT * kSkPitch];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int n0 = (blockIdx.x * 4 + wave) * 16;
    const bool live = n0 < n;  // this wave's column tile exists
    const int ks = blockIdx.y;
    const int chunks = (k + kSkChunk - 1) / kSkChunk;
    const int per = (chunks + ksplit - 1) / ksplit;
    const int c0 = ks * per, c1 = min(chunks, c0 + per);

    i32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = i32x4{0, 0, 0, 0};
    const i8* brow = b + (size_t)min(n0 + r, n - 1) * k + 16 * g;
    for (int c = c0; c < c1; ++c) {
        const int kc = c * kSkChunk;
        __syncthreads();  // every wave is done with the previous chunk's A
        // stage A rows [0, 16 MT) x [kc, kc + 1 KB): wave w copies rows w, w+4, ..
        // (rows past M repeat row M-1; K past the end reads zeros below)
        for (int row = wave; row < 16 * MT; row += 4) {
            const int src_row = min(row, m - 1);
            const int kk = min(kc + 16 * lane, k - 16);
            __builtin_amdgcn_global_load_lds(a + (size_t)src_row * k + kk,
                                             (lds_void_p)(sa_rows + row * kSkPitch), 16, 0, 0);
        }
        i32x4 bv[kSkSteps];
#pragma unroll
        for (int u = 0; u < kSkSteps; ++u) {
            const int kb = kc + 64 * u + 16 * g;
            const i32x4 z = {0, 0, 0, 0};
            bv[u] = (live && kb < k) ? *reinterpret_cast<const i32x4*>(brow + kc + 64 * u) : z;
        }
        __builtin_amdgcn_s_waitcnt(0);  // this wave's A copies (and W loads) landed
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kSkSteps; ++u) {
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                i32x4 av = *reinterpret_cast<const i32x4*>(
                    sa_rows + (16 * t + r) * kSkPitch + 64 * u + 16 * g);
                if (kc + 64 * u + 16 * g >= k) av = i32x4{0, 0, 0, 0};
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv[u], acc[t], 0, 0, 0);
            }
        }
    }
    if (!live) return;
    // C layout: lane (r, g) holds C[4g + i][r] = (A row 16t + 4g + i, W row n0 + r)
    const int col = n0 + r;
    if (col >= n) return;
    if (ksplit == 1) {
        const float sa = epi_sa(e);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * t + 4 * g + i;
                if (row < m) epi_store<OUT>(e, sa, n, row, col, acc[t][i]);
            }
    } else {
        int* mine = part + (size_t)ks * m * n;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * t + 4 * g + i;
                if (row < m) mine[(size_t)row * n + col] = acc[t][i];
            }
    }
}

// ---------------------------------------------------------------------------
// skinny MFMA GEMM through an LDS ring (M <= 16*MT <= 64, K % 256 == 0): the
// workgroup, waves and K split of qgemm_skinny, but both operands arrive by
// global -> LDS DMA in whole lines, 256-byte K chunks, NSTAGE chunks in the
// ring (NSTAGE - 1 in flight while one is multiplied). One DMA instruction
// covers 256 bytes of each of 4 rows (16 lanes per row); the A rows are
// copied once per workgroup (wave w: instructions w, w + 4, ..), each wave
// copies its own 16 W rows (non-temporal: read once).
//
// A stage holds A rows [0, 16 MT) then W rows [0, 64) (wave w's at 16 w),
// 256 bytes each; slot s of row r holds K piece s ^ (r & 15): lane l of a DMA
// reads piece (l & 15) ^ (r & 15), and the 16 lanes of a ds_read_b128
// quarter (rows 16 t + 0..15, piece 4 u + g) hit distinct bank groups.
// ---------------------------------------------------------------------------
constexpr int kSlChunk = 256;
constexpr int kSlSteps = kSlChunk / 64;

// one chunk of qgemm_skinny_lds: this wave's 4 W instructions (non-temporal)
// and its share of the 4 MT A instructions (instruction j = wave + NW i
// covers A rows 4 j .. 4 j + 3), into the stage at dst
template <int MT, int NW>
__device__ __forceinline__ void sl_issue(const i8* a, const i8* b, const size_t* aoff,
                                         const size_t* boff, char* dst, size_t kc, int wave) {
    constexpr int kArows = 16 * MT;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_global_load_lds(
            b + boff[i] + kc, (lds_void_p)(dst + (kArows + 16 * wave + 4 * i) * kSlChunk), 16,
            0, 2);
#pragma unroll
    for (int i = 0; i < 4 * MT / NW; ++i)
        __builtin_amdgcn_global_load_lds(a + aoff[i] + kc,
                                         (lds_void_p)(dst + 4 * (wave + NW * i) * kSlChunk), 16,
                                         0, 0);
}

// SWQ: the gate/up GEMM of a SwiGLU, n = 2 * inter (B holds the gate rows,
// then the up rows), inter % (8 * NW) == 0, ksplit == 1. The first NW / 2
// waves of workgroup x take gate columns 8 NW x + 16 w .., the other NW / 2
// the up columns inter + the same, so every gate output and its up partner
// are in one workgroup. After y is stored (skipped when e.y is null), the
// epilogue takes the workgroup's max |silu(g) * u| over the stored values.
// Without `sq` it goes to swq_part[x]: the partial maxima swiglu_quant
// folds, without its own pass over y. With `sq` (every workgroup resident
// at once) the tensor maximum is folded here (grid_max), and each
// workgroup writes the int8 codes of its SwiGLU outputs and workgroup 0 the
// scale, as swiglu_quant would: the whole gate/up -> SwiGLU -> quantize step
// in one launch.
struct SwqGrid {
    signed char* q = nullptr;  // [m, inter] codes, or null (partials only)
    float* scale = nullptr;
    GridMax gm{};
};
template <int MT, int NSTAGE, int NW, int OUT, bool SWQ>
__global__ __launch_bounds__(64 * NW) void qgemm_skinny_lds(
    const i8* __restrict__ a, const i8* __restrict__ b, Epi e, int m, int n,
    int k, int ksplit, int* __restrict__ part, int inter, float* __restrict__ swq_part,
    SwqGrid sq) {
    constexpr int kArows = 16 * MT;
    constexpr int kStage = (kArows + 16 * NW) * kSlChunk;
    constexpr int kAIns = kArows / 4 / NW;  // A DMA instructions per wave per chunk
    static_assert(NSTAGE == 2 || NSTAGE == 3, "stage count");
    static_assert(kAIns * NW * 4 == kArows, "A rows split evenly over the waves");
    static_assert(!SWQ || (16 * MT * (8 * NW + 1) + NW) * 4 <= NSTAGE * kStage,
                  "the SwiGLU exchange fits in the ring");
    __shared__ __attribute__((aligned(16))) char lds[NSTAGE * kStage];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    constexpr int kHalf = NW / 2;
    const int n0 = SWQ ? (wave < kHalf ? 0 : inter) + ((int)blockIdx.x * kHalf + wave % kHalf) * 16
                       : ((int)blockIdx.x * NW + wave) * 16;
    const bool live = n0 < n;
    const int ks = blockIdx.y;
    const int chunks = k / kSlChunk;
    const int per = (chunks + ksplit - 1) / ksplit;
    const int c0 = min(chunks, ks * per), c1 = min(chunks, c0 + per);

    // DMA lane roles: row (l >> 4) of the instruction's 4, piece (l & 15) ^ row
    const int drow = lane >> 4;
    size_t aoff[kAIns], boff[4];
#pragma unroll
    for (int i = 0; i < kAIns; ++i) {
        const int row = 4 * (wave + NW * i) + drow;  // A row staged by this lane
        aoff[i] = (size_t)min(row, m - 1) * k + 16 * ((lane & 15) ^ (row & 15));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * i + drow;  // of this wave's 16 W rows
        boff[i] = (size_t)min(n0 + row, n - 1) * k + 16 * ((lane & 15) ^ row);
    }
    constexpr int kIns = 4 + kAIns;  // DMA instructions per wave per chunk

    const unsigned lds0 = lds_addr(lds);
    unsigned fo[kSlSteps];  // offset of step u's fragment within a 16-row group
#pragma unroll
    for (int u = 0; u < kSlSteps; ++u) fo[u] = kSlChunk * r + 16 * ((4 * u + g) ^ r);

    i32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < NSTAGE - 1; ++j)
        if (c0 + j < c1)
            sl_issue<MT, NW>(a, b, aoff, boff, lds + j * kStage, (size_t)(c0 + j) * kSlChunk,
                             wave);
    int st = 0;
    for (int c = c0; c < c1; ++c) {
        // this wave's copies of chunk c landed (the later chunks may still fly)
        if (NSTAGE == 3 && c + 1 < c1)
            wait_vmcnt<kIns>();
        else
            wait_vmcnt<0>();
        // everyone's copies of chunk c landed; chunk c - 1 is free. A bare
        // barrier: __syncthreads() would add a release fence that drains the
        // chunk still in flight
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const int nxt = c + NSTAGE - 1;
        if (nxt < c1)
            sl_issue<MT, NW>(a, b, aoff, boff, lds + ((st + NSTAGE - 1) % NSTAGE) * kStage,
                         (size_t)nxt * kSlChunk, wave);
        const unsigned base = lds0 + st * kStage;
        i32x4 fw[kSlSteps], fa[MT][kSlSteps];
#pragma unroll
        for (int u = 0; u < kSlSteps; ++u)
            fw[u] = lds_read16(base + (kArows + 16 * wave) * kSlChunk + fo[u]);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int u = 0; u < kSlSteps; ++u)
                fa[t][u] = lds_read16(base + 16 * t * kSlChunk + fo[u]);
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fw[0]), "+v"(fw[1]), "+v"(fw[2]), "+v"(fw[3]));
#pragma unroll
        for (int t = 0; t < MT; ++t)
            asm volatile("" : "+v"(fa[t][0]), "+v"(fa[t][1]), "+v"(fa[t][2]), "+v"(fa[t][3]));
#pragma unroll
        for (int u = 0; u < kSlSteps; ++u)
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[t][u], fw[u], acc[t], 0, 0, 0);
        st = st + 1 == NSTAGE ? 0 : st + 1;
    }
    if constexpr (SWQ) {
        // every column is real (the grid covers inter exactly); rows past m
        // hold products of clamped A rows and are neither stored nor folded
        const int col = n0 + r;
        const float sa = epi_sa(e);
        const float sc = e.sb_vec ? sa * e.sb_vec[col] : sa * e.sb;
        float sv[MT][4];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * t + 4 * g + i;
                sv[t][i] = epi_stored<OUT>(acc[t][i], sc);
                if (row < m && e.y) epi_store_scaled<OUT>(e, n, row, col, acc[t][i], sc);
            }
        // the up values through LDS (the ring is free once every wave is
        // past its last chunk), then each gate lane folds its outputs
        constexpr int kXP = 16 * kHalf + 1;  // floats per row (bank spread)
        float* xch = reinterpret_cast<float*>(lds);
        float* red = xch + 16 * MT * kXP;
        const int cl = 16 * (wave % kHalf) + r;
        __syncthreads();
        if (wave >= kHalf) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) xch[(16 * t + 4 * g + i) * kXP + cl] = sv[t][i];
        }
        __syncthreads();
        float mx = 0.0f;
        if (wave < kHalf) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 16 * t + 4 * g + i;
                    // the SwiGLU output, kept for the codes below
                    sv[t][i] = silu_mul(sv[t][i], xch[row * kXP + cl]);
                    if (row < m) mx = fmaxf(mx, fabsf(sv[t][i]));
                }
        }
        mx = block_max<64 * NW>(mx, red);
        if (!sq.q) {
            if (threadIdx.x == 0) swq_part[blockIdx.x] = mx;
            return;
        }
        mx = grid_max<64 * NW>(sq.gm, mx, red);
        const float scale = make_scale(mx);
        const float inv_s = 1.0f / scale;
        if (blockIdx.x == 0 && threadIdx.x == 0) *sq.scale = scale;
        if (wave < kHalf) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 16 * t + 4 * g + i;
                    if (row < m) sq.q[(size_t)row * inter + col] = quant1(sv[t][i], inv_s);
                }
        }
        return;
    }
    const int col = n0 + r;
    const bool own = live && col < n;
    if (ksplit == 1) {
        if (!own) return;
        const float sa = epi_sa(e);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * t + 4 * g + i;
                if (row < m) epi_store<OUT>(e, sa, n, row, col, acc[t][i]);
            }
        return;
    }
    int* mine = part + (size_t)ks * m * n;
    if (own) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * t + 4 * g + i;
                if (row < m) mine[(size_t)row * n + col] = acc[t][i];
            }
    }
}

// K-split fold: out[row][col] = sum over ks of part[ks][row][col] (int32
// sums: exact in any order). Up to 8 partials are loaded at once, and the
// column scale with them, so a fold costs one memory round trip per 8
// partials instead of one per partial.
constexpr int kKsumBatch = 8;

// res (optional, OUT-typed [m, n]): the stored value plus res[idx], rounded
// again (a decode layer's residual add; kfold.hpp)
template <int OUT>
__global__ __launch_bounds__(256) void qgemm_ksum(const int* __restrict__ part,
                                                  Epi e, int m, int n, int ksplit,
                                                  const void* __restrict__ res) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long mn = (long long)m * n;
    if (idx >= mn) return;
    const int row = (int)(idx / n), col = (int)(idx - (long long)row * n);
    float sa = 0.0f, sb = 0.0f;
    if constexpr (OUT != kOutI32) {
        sa = epi_sa(e);
        sb = e.sb_vec ? e.sb_vec[col] : e.sb;
    }
    int s = 0;
    for (int j0 = 0; j0 < ksplit; j0 += kKsumBatch) {
        int v[kKsumBatch];
#pragma unroll
        for (int u = 0; u < kKsumBatch; ++u)
            v[u] = j0 + u < ksplit ? part[(size_t)(j0 + u) * mn + idx] : 0;
#pragma unroll
        for (int u = 0; u < kKsumBatch; ++u) s += v[u];
    }
    if constexpr (OUT == kOutBF16 || OUT == kOutF16 || OUT == kOutF32) {
        if (res) {
            using T = std::conditional_t<OUT == kOutBF16, bf16,
                                         std::conditional_t<OUT == kOutF16, f16, float>>;
            const float v = kfold_add_res<T>(epi_stored<OUT>(s, sa * sb),
                                             St<T>::ld(static_cast<const T*>(res) + idx));
            St<T>::st(static_cast<T*>(e.y) + idx, v);
            return;
        }
    }
    epi_store_scaled<OUT>(e, n, row, col, s, sa * sb);
}

// ---------------------------------------------------------------------------
// tiled (M > 64)
// ---------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN>
struct TileCfg {
    static constexpr int BK = 64;
    static constexpr int PITCH = BK + 16;          // bytes per LDS row
    static constexpr int NTHR = WM * WN * 64;
    static constexpr int MT = BM / WM / 32;        // 32x32 tiles per wave (M)
    static constexpr int NT = BN / WN / 32;        // 32x32 tiles per wave (N)
    static constexpr int ALOADS = BM * BK / 16 / NTHR;
    static constexpr int BLOADS = BN * BK / 16 / NTHR;
};

template <int BM, int BN, int WM, int WN, int OUT>
__global__ __launch_bounds__(WM * WN * 64) void qgemm_tiled(
    const i8* __restrict__ a, const i8* __restrict__ b, Epi e, int m, int n,
    int k) {
    using C = TileCfg<BM, BN, WM, WN>;
    constexpr int BK = C::BK, PITCH = C::PITCH, NTHR = C::NTHR;
    __shared__ __attribute__((aligned(16))) i8 lds_a[2][BM * PITCH];
    __shared__ __attribute__((aligned(16))) i8 lds_b[2][BN * PITCH];

    const int bm = blockIdx.y * BM, bn = blockIdx.x * BN;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave - (wave / WN) * WN;
    const int r32 = lane & 31, h = lane >> 5;

    i32x16 acc[C::MT][C::NT];
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int j = 0; j < C::NT; ++j)
#pragma unroll
            for (int t = 0; t < 16; ++t) acc[i][j][t] = 0;

    i32x4 ra[C::ALOADS], rb[C::BLOADS];
    auto gload = [&](int kt) {
        const int kb = kt * BK;
#pragma unroll
        for (int j = 0; j < C::ALOADS; ++j) {
            const int c = tid + j * NTHR;
            const int row = c >> 2, kc = (c & 3) * 16;
            const bool ok = (bm + row < m) && (kb + kc < k);
            const i32x4 z = {0, 0, 0, 0};
            ra[j] = ok ? *reinterpret_cast<const i32x4*>(a + (size_t)(bm + row) * k + kb + kc) : z;
        }
#pragma unroll
        for (int j = 0; j < C::BLOADS; ++j) {
            const int c = tid + j * NTHR;
            const int row = c >> 2, kc = (c & 3) * 16;
            const bool ok = (bn + row < n) && (kb + kc < k);
            const i32x4 z = {0, 0, 0, 0};
            rb[j] = ok ? *reinterpret_cast<const i32x4*>(b + (size_t)(bn + row) * k + kb + kc) : z;
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < C::ALOADS; ++j) {
            const int c = tid + j * NTHR;
            *reinterpret_cast<i32x4*>(&lds_a[buf][(c >> 2) * PITCH + (c & 3) * 16]) = ra[j];
        }
#pragma unroll
        for (int j = 0; j < C::BLOADS; ++j) {
            const int c = tid + j * NTHR;
            *reinterpret_cast<i32x4*>(&lds_b[buf][(c >> 2) * PITCH + (c & 3) * 16]) = rb[j];
        }
    };

    const int nk = (k + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            i32x4 fa[C::MT], fb[C::NT];
#pragma unroll
            for (int i = 0; i < C::MT; ++i)
                fa[i] = *reinterpret_cast<const i32x4*>(
                    &lds_a[cur][(wm * (BM / WM) + i * 32 + r32) * PITCH + ks * 32 + h * 16]);
#pragma unroll
            for (int j = 0; j < C::NT; ++j)
                fb[j] = *reinterpret_cast<const i32x4*>(
                    &lds_b[cur][(wn * (BN / WN) + j * 32 + r32) * PITCH + ks * 32 + h * 16]);
#pragma unroll
            for (int i = 0; i < C::MT; ++i)
#pragma unroll
                for (int j = 0; j < C::NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    // C layout 32x32: lane (r32, h), reg t -> row 8*(t/4) + 4h + t%4, col r32
    const float sa = epi_sa(e);
#pragma unroll
    for (int j = 0; j < C::NT; ++j) {
        const int col = bn + wn * (BN / WN) + j * 32 + r32;
        if (col >= n) continue;
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int row = bm + wm * (BM / WM) + i * 32 + 8 * (t >> 2) + 4 * h + (t & 3);
                if (row < m) epi_store<OUT>(e, sa, n, row, col, acc[i][j][t]);
            }
    }
}

// ---------------------------------------------------------------------------
// big (M >= 256, N >= 256): 256x256 workgroup tiles, K slabs of 64 bytes,
// 4 waves each owning a 128x128 sub-tile = 4x4 blocks of
// v_mfma_i32_32x32x32_i8 (256 int32 accumulators per lane, so one wave per
// SIMD). A and B slabs are staged global -> registers -> LDS, double
// buffered, one barrier per slab. LDS rows are 64 bytes = four 16-byte
// chunks; chunk c of row r is stored at position c ^ big_swz(r) with
// big_swz(r) = (r >> 2) & 3: the gfx950 LDS serves a ds_read_b128 16 lanes
// (256 bytes, all 64 banks) per cycle, and the 16 consecutive rows of such a
// group then hit 16 distinct 16-byte bank groups (rows r and r + 4k share the
// same 64-byte slot of the 256, so they need different chunk positions). Tiles are numbered XCD-aware: the
// tiles dispatched to one XCD are consecutive in a column-major walk of
// 4-row tile bands, so the ~32 tiles an XCD runs at a time cover a 4 x 8
// block of the output and share their A / B panels through its L2.
// ---------------------------------------------------------------------------
constexpr int kBigT = 256;    // tile edge (M and N)
constexpr int kBigK = 64;     // K bytes per slab
constexpr int kBigBand = 4;   // tile rows per band of the XCD-aware order

__device__ __forceinline__ int big_swz(int row) { return (row >> 2) & 3; }

__device__ __forceinline__ int big_lds_off(int row, int c) {
    return row * kBigK + ((c ^ big_swz(row)) << 4);
}

template <int OUT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void qgemm_big(const i8* __restrict__ a, const i8* __restrict__ b, Epi e,
               int m, int n, int k) {
    __shared__ __attribute__((aligned(16))) i8 lds_a[2][kBigT * kBigK];
    __shared__ __attribute__((aligned(16))) i8 lds_b[2][kBigT * kBigK];

    // ---- tile id: XCD-contiguous, then banded column-major ---------------
    const int tm = (m + kBigT - 1) / kBigT, tn = (n + kBigT - 1) / kBigT;
    const int ntiles = tm * tn;
    int pid = blockIdx.x;
    if (ntiles % 8 == 0) pid = (pid % 8) * (ntiles / 8) + pid / 8;
    const int band = pid / (kBigBand * tn);
    const int first_m = band * kBigBand;
    const int band_m = min(tm - first_m, kBigBand);
    const int in_band = pid - band * kBigBand * tn;
    const int tile_m = first_m + in_band % band_m;
    const int tile_n = in_band / band_m;
    const int bm = tile_m * kBigT, bn = tile_n * kBigT;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r32 = lane & 31, h = lane >> 5;

    // staging: 4 chunks of A and 4 of B per thread per slab; chunk q = tid +
    // 256 j lands at LDS position q (consecutive lanes, consecutive 16 B)
    i32x4 ga[4], gb[4];
    auto gload = [&](int kt) {
        const int kb = kt * kBigK;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int q = tid + 256 * j;
            const int row = q >> 2;
            const int c = (q & 3) ^ big_swz(row);
            const int kc = kb + 16 * c;
            const i32x4 z = {0, 0, 0, 0};
            ga[j] = (bm + row < m && kc < k)
                        ? *reinterpret_cast<const i32x4*>(a + (size_t)(bm + row) * k + kc) : z;
            gb[j] = (bn + row < n && kc < k)
                        ? *reinterpret_cast<const i32x4*>(b + (size_t)(bn + row) * k + kc) : z;
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int q = tid + 256 * j;
            *reinterpret_cast<i32x4*>(&lds_a[buf][q * 16]) = ga[j];
            *reinterpret_cast<i32x4*>(&lds_b[buf][q * 16]) = gb[j];
        }
    };

    i32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < 16; ++t) acc[i][j][t] = 0;

    const int nk = (k + kBigK - 1) / kBigK;
    gload(0);
    sstore(0);
    __syncthreads();
    if (nk > 1) gload(1);
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            i32x4 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                fa[i] = *reinterpret_cast<const i32x4*>(
                    &lds_a[cur][big_lds_off(wm * 128 + i * 32 + r32, 2 * s + h)]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                fb[j] = *reinterpret_cast<const i32x4*>(
                    &lds_b[cur][big_lds_off(wn * 128 + j * 32 + r32, 2 * s + h)]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
        if (kt + 2 < nk) gload(kt + 2);
    }

    // ---- epilogue: C layout 32x32, lane (r32, h), reg t -> row
    // 8*(t/4) + 4h + t%4, col r32
    const float sa = epi_sa(e);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = bn + wn * 128 + j * 32 + r32;
        if (col >= n) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int row = bm + wm * 128 + i * 32 + 8 * (t >> 2) + 4 * h + (t & 3);
                if (row < m) epi_store<OUT>(e, sa, n, row, col, acc[i][j][t]);
            }
    }
}

// ---------------------------------------------------------------------------
// big, DMA-fed (K % 64 == 0): the same tiles, order and LDS layout as
// qgemm_big, but
//  - slabs go global -> LDS directly (global_load_lds_dwordx4: lane i of a
//    wave's load lands at the wave's LDS base + 16 i), so no registers hold
//    them; a ring of kDmaStages 32 KB stages keeps kDmaStages - 1 slabs in
//    flight ahead of the MFMAs (the L2 / HBM latency under load spans
//    several slabs of MFMA work);
//  - operand fragments are read with inline-asm ds_read_b128 (invisible to
//    the compiler's LDS-DMA alias tracking, which would otherwise wait for
//    every in-flight slab before each read), interleaved with the MFMAs of
//    the previous fragment set; a slab is waited for with an explicit vmcnt
//    sized to the slabs issued after it, then a bare s_barrier;
//  - the accumulators hold C^T blocks (operands swapped), so each lane owns
//    4 consecutive output columns per register quad: 2-byte outputs are
//    staged through LDS per wave and leave as 16-byte row-contiguous stores,
//    4-byte outputs as 16-byte stores straight from registers.
// Rows past M / N load a clamped (real) row; they only feed outputs that
// are never stored.
// ---------------------------------------------------------------------------
constexpr int kDmaStages = 5;
constexpr int kSlabBytes = 2 * kBigT * kBigK;  // A + B slab, 32 KB
constexpr int kSlabLoads = 8;  // DMA instructions per thread per slab (4 A + 4 B)
constexpr int kEpiPitch = 272;  // LDS row pitch of the output staging (16-byte rows)



// Wait for every outstanding LDS read; the fragments are in/out operands, so
// nothing that uses them can be scheduled above the wait.
__device__ __forceinline__ void lds_wait(i32x4 (&f)[8]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]),
                   "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]));
}

// The scaled f32 value of one accumulator (two f32 roundings, unfused: see
// epi_store).
__device__ __forceinline__ float epi_val(int acc, float s) {
    float val = (float)acc * s;
    asm("" : "+v"(val));
    return val;
}

// Epilogue of the DMA-fed big kernels. acc[i][j] holds C^T: lane (r32, h),
// register t -> C[row = i*32 + r32][col = j*32 + 8(t/4) + 4h + t%4] of the
// wave's 128 x 128 sub-tile at (row0, col0), i.e. 4 consecutive columns per
// register quad. lds must hold 4 * 64 * kEpiPitch bytes no wave still reads.
template <int OUT>
__device__ __forceinline__ void big_epilogue(i32x16 (&acc)[4][4], i8* lds, const Epi& e,
                                             int m, int n, int row0, int col0,
                                             int lane, int wave, int r32, int h) {
    __syncthreads();  // every wave is done with the stages: LDS is reused
    const float sa = epi_sa(e);
    auto scales4 = [&](int col) {  // f32(sa * sb[col .. col+3]), clamped at n
        float4 s4;
        if (e.sb_vec) {
            s4.x = sa * e.sb_vec[min(col, n - 1)];
            s4.y = sa * e.sb_vec[min(col + 1, n - 1)];
            s4.z = sa * e.sb_vec[min(col + 2, n - 1)];
            s4.w = sa * e.sb_vec[min(col + 3, n - 1)];
        } else {
            const float s = sa * e.sb;
            s4 = make_float4(s, s, s, s);
        }
        return s4;
    };
    if constexpr (OUT == kOutBF16 || OUT == kOutF16) {
        typedef typename std::conditional<OUT == kOutBF16, bf16, f16>::type OT;
        typedef OT ot4 __attribute__((ext_vector_type(4)));
        i8* const stg = lds + wave * (64 * kEpiPitch);  // this wave's 64 rows
        float4 sc[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) sc[j][g] = scales4(col0 + j * 32 + 8 * g + 4 * h);
        OT* const y = static_cast<OT*>(e.y);
#pragma unroll
        for (int ih = 0; ih < 2; ++ih) {
#pragma unroll
            for (int i2 = 0; i2 < 2; ++i2) {
                const int i = 2 * ih + i2;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        ot4 v;
                        v[0] = (OT)epi_val(acc[i][j][4 * g + 0], sc[j][g].x);
                        v[1] = (OT)epi_val(acc[i][j][4 * g + 1], sc[j][g].y);
                        v[2] = (OT)epi_val(acc[i][j][4 * g + 2], sc[j][g].z);
                        v[3] = (OT)epi_val(acc[i][j][4 * g + 3], sc[j][g].w);
                        *reinterpret_cast<ot4*>(stg + (i2 * 32 + r32) * kEpiPitch +
                                                (j * 32 + 8 * g + 4 * h) * 2) = v;
                    }
            }
            // 64 rows x 256 bytes back out: 16 lanes per row, 16 bytes each
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const int lr = rr * 4 + (lane >> 4);
                const int row = row0 + ih * 64 + lr;
                const int cb = (lane & 15) * 8;  // first of 8 columns
                const i8* src = stg + lr * kEpiPitch + cb * 2;
                if (row >= m) continue;
                OT* dst = y + (size_t)row * n + col0 + cb;
                if ((n & 7) == 0) {
                    if (col0 + cb < n)
                        *reinterpret_cast<i32x4*>(dst) = *reinterpret_cast<const i32x4*>(src);
                } else {
#pragma unroll
                    for (int c = 0; c < 8; ++c)
                        if (col0 + cb + c < n) dst[c] = reinterpret_cast<const OT*>(src)[c];
                }
            }
        }
    } else {  // 4-byte outputs: 16-byte stores of 4 consecutive columns
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int col = col0 + j * 32 + 8 * g + 4 * h;
                float4 s4;
                if constexpr (OUT == kOutF32) s4 = scales4(col);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = row0 + i * 32 + r32;
                    if (row >= m || col >= n) continue;
                    i32x4 o;
                    if constexpr (OUT == kOutI32) {
                        o = i32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1],
                                  acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                    } else {
                        o = i32x4{__float_as_int(epi_val(acc[i][j][4 * g], s4.x)),
                                  __float_as_int(epi_val(acc[i][j][4 * g + 1], s4.y)),
                                  __float_as_int(epi_val(acc[i][j][4 * g + 2], s4.z)),
                                  __float_as_int(epi_val(acc[i][j][4 * g + 3], s4.w))};
                    }
                    int* dst = static_cast<int*>(e.y) + (size_t)row * n + col;
                    if ((n & 3) == 0) {
                        *reinterpret_cast<i32x4*>(dst) = o;
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            if (col + c < n) dst[c] = o[c];
                    }
                }
            }
    }
}

template <int OUT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void qgemm_big_dma(const i8* __restrict__ a, const i8* __restrict__ b, Epi e,
                   int m, int n, int k) {
    __shared__ __attribute__((aligned(16))) i8 lds[kDmaStages * kSlabBytes];

    const int tm = (m + kBigT - 1) / kBigT, tn = (n + kBigT - 1) / kBigT;
    const int ntiles = tm * tn;
    int pid = blockIdx.x;
    if (ntiles % 8 == 0) pid = (pid % 8) * (ntiles / 8) + pid / 8;
    const int band = pid / (kBigBand * tn);
    const int first_m = band * kBigBand;
    const int band_m = min(tm - first_m, kBigBand);
    const int in_band = pid - band * kBigBand * tn;
    const int bm = (first_m + in_band % band_m) * kBigT;
    const int bn = (in_band / band_m) * kBigT;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int r32 = lane & 31, h = lane >> 5;

    // this lane's sources: LDS chunk q = tid + 256 j holds tile row
    // q/4 = tid/4 + 64 j, logical chunk (q%4) ^ big_swz(row), which is
    // the same for all j. Addresses = wave-uniform tile base (scalar) + a
    // 32-bit per-lane offset (rows past the edge clamp to the last row).
    const int c16 = 16 * ((tid & 3) ^ big_swz(tid >> 2));
    unsigned aoff[4], boff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = (tid >> 2) + 64 * j;
        aoff[j] = (unsigned)(min(row, m - 1 - bm) * k + c16);
        boff[j] = (unsigned)(min(row, n - 1 - bn) * k + c16);
    }
    const i8* const abase = a + (size_t)bm * k;
    const i8* const bbase = b + (size_t)bn * k;
    auto stage_a = [&](int st) { return lds + st * kSlabBytes; };
    auto stage_b = [&](int st) { return lds + st * kSlabBytes + kBigT * kBigK; };
    auto issue = [&](int kt, int st) {
        const i8* ak = abase + (size_t)kt * kBigK;
        const i8* bk = bbase + (size_t)kt * kBigK;
        i8* la = stage_a(st);
        i8* lb = stage_b(st);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int dst = (256 * j + 64 * wave) * 16;  // this wave's 1 KB
            __builtin_amdgcn_global_load_lds(ak + aoff[j], (lds_void_p)(la + dst), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(bk + boff[j], (lds_void_p)(lb + dst), 16, 0, 0);
        }
    };

    i32x16 acc[4][4];  // acc[i][j] = C^T block (n block j, m block i)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < 16; ++t) acc[i][j][t] = 0;

    // Operand fragments of one 32-byte K step: f[0..3] A row blocks,
    // f[4..7] B column blocks; two sets (f0, f1) alternate. Row offsets of
    // this lane's fragment rows within a stage, chunk 0; chunk c of a row
    // sits at 16 * (c ^ big_swz(row)), i.e. XOR (c << 4) into the offset.
    unsigned arow_off[4], brow_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        arow_off[i] = (unsigned)big_lds_off(wm * 128 + i * 32 + r32, 0);
        brow_off[i] = (unsigned)big_lds_off(wn * 128 + i * 32 + r32, 0);
    }
    const unsigned lds0 = lds_addr(lds);
    // Fragment reads go out in the order their first use in the MFMA
    // sequence below needs them: A0, B0..B3, A1, A2, A3.
    auto frag_off = [&](int x, unsigned la, unsigned lb, unsigned cx) {
        constexpr int order[8] = {0, 4, 5, 6, 7, 1, 2, 3};
        const int fi = order[x];
        return fi < 4 ? la + (arow_off[fi] ^ cx) : lb + (brow_off[fi - 4] ^ cx);
    };
    auto read_frags = [&](int st, int sub, i32x4 (&f)[8]) {
        const unsigned la = lds0 + st * kSlabBytes, lb = la + kBigT * kBigK;
        const unsigned cx = (unsigned)((2 * sub + h) << 4);
        constexpr int order[8] = {0, 4, 5, 6, 7, 1, 2, 3};
#pragma unroll
        for (int x = 0; x < 8; ++x) f[order[x]] = lds_read16(frag_off(x, la, lb, cx));
    };
    // Wait until LDS reads leave at most N outstanding; the named fragments
    // are in/out operands, so nothing that uses them moves above the wait.
#define FT_LGKM_WAIT(N, ...)                                                    \
    do {                                                                       \
        __builtin_amdgcn_sched_barrier(0);                                     \
        asm volatile("s_waitcnt lgkmcnt(" #N ")" : __VA_ARGS__);               \
        __builtin_amdgcn_sched_barrier(0);                                     \
    } while (0)

    // 16 MFMAs on f while the next fragment set's 8 reads go out between
    // them (one after every odd MFMA); with a DMA tag, the 8 DMA
    // instructions of slab dma_kt into stage dma_st go out after the even
    // ones. (Issued in a burst right after the barrier, the four waves' 32
    // DMA instructions would queue at the CU's texture addresser with the
    // MFMA pipe idle until the last wave's had gone out.)
    // f was read in the previous call, in first-use order, and is waited for
    // piecewise: before MFMA q, floor(q/2) reads of this call are in flight
    // too, so "read r of f landed" is lgkmcnt(7 - r + floor(q/2)) (LDS
    // reads complete in order). The MFMA pipe never waits on the last
    // reads of f (A3 is first needed at q = 12).
    auto mfma_and_read = [&](i32x4 (&f)[8], int st, int sub, i32x4 (&nf)[8],
                             auto dma, int dma_kt, int dma_st) {
        const unsigned la = lds0 + st * kSlabBytes, lb = la + kBigT * kBigK;
        const unsigned cx = (unsigned)((2 * sub + h) << 4);
        const i8* ak = abase + (size_t)dma_kt * kBigK;
        const i8* bk = bbase + (size_t)dma_kt * kBigK;
        i8* da = stage_a(dma_st);
        i8* db = stage_b(dma_st);
        constexpr int order[8] = {0, 4, 5, 6, 7, 1, 2, 3};
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int i = q >> 2, j = q & 3;
            if (q == 0) FT_LGKM_WAIT(6, "+v"(f[0]), "+v"(f[4]));
            if (q == 1) FT_LGKM_WAIT(5, "+v"(f[5]));
            if (q == 2) FT_LGKM_WAIT(5, "+v"(f[6]));
            if (q == 3) FT_LGKM_WAIT(4, "+v"(f[7]));
            if (q == 4) FT_LGKM_WAIT(4, "+v"(f[1]));
            if (q == 8) FT_LGKM_WAIT(5, "+v"(f[2]));
            if (q == 12) FT_LGKM_WAIT(6, "+v"(f[3]));
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[4 + j], f[i], acc[i][j], 0, 0, 0);
            const int x = q >> 1;  // 0..7
            if (q & 1) {
                __builtin_amdgcn_sched_barrier(0);
                nf[order[x]] = lds_read16(frag_off(x, la, lb, cx));
                __builtin_amdgcn_sched_barrier(0);
            } else if constexpr (decltype(dma)::value) {
                // x = 2 jj: A rows 64 jj + ..; x = 2 jj + 1: B rows (the order
                // of issue(): A, B per jj)
                const int jj = x >> 1;
                const int dst = (256 * jj + 64 * wave) * 16;
                __builtin_amdgcn_sched_barrier(0);
                if (x & 1)
                    __builtin_amdgcn_global_load_lds(bk + boff[jj], (lds_void_p)(db + dst), 16, 0, 0);
                else
                    __builtin_amdgcn_global_load_lds(ak + aoff[jj], (lds_void_p)(da + dst), 16, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
#undef FT_LGKM_WAIT

    // Per slab kt (in stage st = kt % kDmaStages), with f0 = (kt, sub 0)
    // read:
    //   16 MFMAs on f0 while f1 = (kt, sub 1) is read;
    //   wait for slab kt+1's DMA, barrier;
    //   16 MFMAs on f1 while f0 = (kt+1, sub 0) is read and the stage of
    //   slab kt-1 is refilled with slab kt-1 + kDmaStages.
    // The barrier of slab kt certifies that every wave has consumed slab
    // kt-1 (its fragments fed MFMAs before the barrier, which needs them
    // landed), so that stage is free; and that slab kt+1's DMAs, waited for
    // by each wave before it, are visible to all. (After the last slab f0
    // reads a stale stage: in bounds, never used.)
    const int nk = k / kBigK;
    const int pre = min(kDmaStages, nk);
    for (int s = 0; s < pre; ++s) issue(s, s);
    // slab 0 landed: at most pre - 1 slabs issued after it still in flight
    switch (pre - 1) {
    case 4: wait_vmcnt<4 * kSlabLoads>(); break;
    case 3: wait_vmcnt<3 * kSlabLoads>(); break;
    case 2: wait_vmcnt<2 * kSlabLoads>(); break;
    case 1: wait_vmcnt<1 * kSlabLoads>(); break;
    default: wait_vmcnt<0>(); break;
    }
    __builtin_amdgcn_s_barrier();
    i32x4 f0[8], f1[8];
    read_frags(0, 0, f0);
    int st = 0;
    auto slab = [&](int kt, auto dma) {
        const int st_next = st + 1 == kDmaStages ? 0 : st + 1;
        const int st_prev = st == 0 ? kDmaStages - 1 : st - 1;
        mfma_and_read(f0, st, 1, f1, std::false_type{}, 0, 0);
        // slabs issued after kt+1: kt+2 .. min(nk - 1, kt + kDmaStages - 2)
        const int after = min(kDmaStages - 3, nk - 2 - kt);
        switch (after) {
        case 3: wait_vmcnt<3 * kSlabLoads>(); break;
        case 2: wait_vmcnt<2 * kSlabLoads>(); break;
        case 1: wait_vmcnt<1 * kSlabLoads>(); break;
        default: wait_vmcnt<0>(); break;
        }
        // bare barrier: __syncthreads() would add a release fence that
        // drains every in-flight DMA (the later slabs too)
        __builtin_amdgcn_s_barrier();
        mfma_and_read(f1, st_next, 0, f0, dma, kt - 1 + kDmaStages, st_prev);
        st = st_next;
    };
    // slab 0 has no previous stage to refill; slabs 1 .. nk - kDmaStages do
    int kt = 0;
    if (nk > 0) slab(kt++, std::false_type{});
    for (; kt - 1 + kDmaStages < nk; ++kt) slab(kt, std::true_type{});
    for (; kt < nk; ++kt) slab(kt, std::false_type{});
    // the last reads (stale, unused) still land in f0's registers: wait for
    // them before those registers can be given to anything else
    lds_wait(f0);

    big_epilogue<OUT>(acc, lds, e, m, n, bm + wm * 128, bn + wn * 128, lane, wave,
                      r32, h);
}

// ---------------------------------------------------------------------------
// big, DMA-fed, 128-byte slabs (K % 128 == 0; qgemm_big_w16): the tiles,
// order and operand layout of qgemm_big_dma, with each slab covering 128
// bytes of K, a whole cache line per row:
//  - a DMA instruction moves 8 rows x 128 B (8 full lines) instead of
//    16 rows x 64 B (16 half lines); streaming this kernel's operand traffic
//    alone (7.5 GB for 4096 x 8192 x 28672) runs at 18.5 TB/s L2 -> LDS this
//    way against 15.6 TB/s with 64-byte rows, at any ring depth;
//  - LDS rows are 128 B = eight 16-byte chunks, chunk c of row r at
//    position c ^ ((r >> 1) & 7): the 16 rows of a 16-lane ds_read_b128
//    group then hit 16 distinct 16-byte bank groups;
//  - two 64 KB stages: slab kt+1 lands while slab kt is multiplied; one
//    barrier per slab (four MFMA sub-steps of 32 bytes), placed before the
//    last sub-step so that sub-step's MFMAs overlap both the refill DMA of
//    the stage just consumed and the first fragment reads of slab kt+1;
//  - persistent: min(tiles, CUs) workgroups walk the tiles (XCD-aware
//    order kept: the grid is a multiple of 8), and the next tile's first two
//    slabs are in flight while the current tile's epilogue runs, out of a
//    separate LDS region (per-wave 16-row output staging and the tile's 256
//    column scales, fetched by DMA when the tile starts), so the epilogue
//    needs no barrier and the next tile no cold start.
// ---------------------------------------------------------------------------
constexpr int kK2 = 128;                     // K bytes per slab
constexpr int kSlab2 = 2 * kBigT * kK2;      // A + B, 64 KB
constexpr int kLoads2 = 16;                  // DMA instructions per thread per slab

// 8 waves per workgroup, two per SIMD: one wave's MFMAs issue while the
// other waits on a fragment read, a DMA issue slot or the slab barrier, and
// one wave's epilogue overlaps the other's MFMAs (4 waves of 128 x 128, one
// per SIMD, kept the matrix cores busy 60% of the cycles on 4096 x 8192 x
// 28672 against 70% with 8). Output staging is per wave, 16 rows x 64
// columns per pass (2-byte outputs), so the two stages, the staging and the
// scales fit in 147 KB.
constexpr int kW8Pitch = 144;                    // staging row pitch: 128 B + 16
constexpr int kW8Stg = 16 * kW8Pitch;            // per-wave staging, 16 rows
constexpr int kW8Spare = 2 * kSlab2;             // LDS offset of the staging
constexpr int kW8Scl = kW8Spare + 8 * kW8Stg;    // LDS offset of the 256 column scales
constexpr int kW8Lds = kW8Scl + 4 * kBigT;       // 150,528 bytes

// ---------------------------------------------------------------------------
// big, 8 waves, 16x16x64 MFMAs (qgemm_big_w16): 256 x 256 tiles in the
// XCD-aware order, 128-byte DMA slabs in two stages. Wave w = 4 g + v owns
// the 64 x 128 sub-tile at rows 128 g + 64 (v >> 1), columns 128 (v & 1),
// computed as 4 x 8 blocks of v_mfma_i32_16x16x64_i8 (128 accumulators per
// lane). The fragment bytes per MAC equal those of 32x32x32 blocks; what
// differs is the instruction: under the board power limit of random int8
// operands the 16x16x64 form sustains more operations per second (all CUs,
// operands cycling through 8 random register sets: 3.24 vs 2.91 POP/s).
// Lane (r16, q4) = (lane % 16, lane / 16) holds 16 bytes (chunk 4 s + q4 of
// 64-byte sub-step s) of row r16 of a 16-row block; the accumulator register
// t of block (i, j) is C[row 16 i + r16][col 16 j + 4 q4 + t].
// ---------------------------------------------------------------------------

// s_waitcnt lgkmcnt(n) for a compile-time n (after unrolling) in 6..11,
// tying the fragments x and y so that their uses stay below the wait.
__device__ __forceinline__ void lgkm_wait_xy(int n, i32x4& x, i32x4& y) {
    __builtin_amdgcn_sched_barrier(0);
    switch (n) {
    case 6: asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(x), "+v"(y)); break;
    case 7: asm volatile("s_waitcnt lgkmcnt(7)" : "+v"(x), "+v"(y)); break;
    case 8: asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(x), "+v"(y)); break;
    case 9: asm volatile("s_waitcnt lgkmcnt(9)" : "+v"(x), "+v"(y)); break;
    case 10: asm volatile("s_waitcnt lgkmcnt(10)" : "+v"(x), "+v"(y)); break;
    case 11: asm volatile("s_waitcnt lgkmcnt(11)" : "+v"(x), "+v"(y)); break;
    default: asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x), "+v"(y)); break;
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Read schedule of the 16x16x64 sub-step (32 MFMAs, q = 4 j + i multiplies
// B block j by A block i). The next sub-step's 12 fragments are read in
// their first-use order B0 A0 A1 A2 A3 B1 .. B7 (fragment index: A i = i,
// B j = 4 + j): read kW16Rd[q] goes out after MFMA q (-1: none), B j's once
// the current B j is dead. kW16Wait[q] is the lgkmcnt bound before MFMA q
// in a sub-step whose fragments are still landing (-1: no wait): the reads
// that MFMA q needs first have landed once at most (11 - their position)
// reads of the previous sub-step plus this sub-step's reads issued before
// MFMA q are outstanding (LDS reads return in order).
constexpr int kW16Rd[32] = {-1, -1, -1, 4, 0, 1, 2, 3, 5, -1, -1, -1, 6, -1, -1, -1,
                            7,  -1, -1, -1, 8, -1, -1, -1, 9, -1, -1, -1, 10, -1, -1, 11};
constexpr int kW16Wait[32] = {10, 9, 8, 7, 7, -1, -1, -1, 10, -1, -1, -1, 10, -1, -1, -1,
                              10, -1, -1, -1, 10, -1, -1, -1, 10, -1, -1, -1, 10, -1, -1, -1};

// Epilogue of qgemm_big_w16: the wave's 64 x 128 sub-tile at (row0, col0),
// acc[i][j] as above. scw: the sub-tile's 128 column scales in LDS, or null
// (read sb_vec from global). 2-byte outputs go through the wave's staging
// stg, 16 rows x 64 columns per pass, and leave as 128-byte row pieces (8
// lanes x 16 bytes); 4-byte outputs are stored from registers.
template <int OUT>
__device__ __forceinline__ void w16_epilogue(i32x4 (&acc)[4][8], i8* stg, const float* scw,
                                             const Epi& e, int m, int n, int row0,
                                             int col0, int lane, int r16, int q4) {
    const float sa = epi_sa(e);
    auto scales4 = [&](int jc) {  // f32(sa * sb[col0 + jc .. + 3]), clamped at n
        float4 s4;
        if (scw) {
            const float4 v = *reinterpret_cast<const float4*>(scw + jc);
            s4 = make_float4(sa * v.x, sa * v.y, sa * v.z, sa * v.w);
        } else if (e.sb_vec) {
            const int col = col0 + jc;
            s4.x = sa * e.sb_vec[min(col, n - 1)];
            s4.y = sa * e.sb_vec[min(col + 1, n - 1)];
            s4.z = sa * e.sb_vec[min(col + 2, n - 1)];
            s4.w = sa * e.sb_vec[min(col + 3, n - 1)];
        } else {
            const float sc = sa * e.sb;
            s4 = make_float4(sc, sc, sc, sc);
        }
        return s4;
    };
    if constexpr (OUT == kOutBF16 || OUT == kOutF16) {
        typedef typename std::conditional<OUT == kOutBF16, bf16, f16>::type OT;
        typedef OT ot4 __attribute__((ext_vector_type(4)));
        OT* const y = static_cast<OT*>(e.y);
        float4 sc[8];  // the lane's column scales, the same for every row block
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] = scales4(16 * j + 4 * q4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int jp = 0; jp < 2; ++jp) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int j = 4 * jp + jj;
                    const float4 s4 = sc[j];
                    ot4 v;
                    v[0] = (OT)epi_val(acc[i][j][0], s4.x);
                    v[1] = (OT)epi_val(acc[i][j][1], s4.y);
                    v[2] = (OT)epi_val(acc[i][j][2], s4.z);
                    v[3] = (OT)epi_val(acc[i][j][3], s4.w);
                    *reinterpret_cast<ot4*>(stg + r16 * kW8Pitch + (16 * jj + 4 * q4) * 2) = v;
                }
                // 16 rows x 128 bytes back out: 8 lanes per row, 16 bytes each.
                // Both pieces are read before the guarded stores, so the wave
                // waits once per pass rather than once per store.
                const int cb = (lane & 7) * 8;  // first of 8 columns
                const int col = col0 + jp * 64 + cb;
                i32x4 piece[2];
#pragma unroll
                for (int rr = 0; rr < 2; ++rr)
                    piece[rr] = *reinterpret_cast<const i32x4*>(
                        stg + (rr * 8 + (lane >> 3)) * kW8Pitch + cb * 2);
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    const int row = row0 + i * 16 + rr * 8 + (lane >> 3);
                    if (row >= m) continue;
                    OT* dst = y + (size_t)row * n + col;
                    if ((n & 7) == 0) {
                        // non-temporal: whole 128-byte lines, written once. All
                        // CUs reach their epilogues together, and the burst
                        // drains faster without cache allocation (C5a: 0.690
                        // against 0.732 ms with plain stores)
                        if (col < n)
                            __builtin_nontemporal_store(piece[rr], reinterpret_cast<i32x4*>(dst));
                    } else {
                        const OT* v = reinterpret_cast<const OT*>(&piece[rr]);
#pragma unroll
                        for (int c = 0; c < 8; ++c)
                            if (col + c < n) dst[c] = v[c];
                    }
                }
            }
        }
    } else {  // 4-byte outputs: 16-byte stores of 4 consecutive columns
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int col = col0 + 16 * j + 4 * q4;
            float4 s4;
            if constexpr (OUT == kOutF32) s4 = scales4(16 * j + 4 * q4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = row0 + i * 16 + r16;
                if (row >= m || col >= n) continue;
                i32x4 o;
                if constexpr (OUT == kOutI32) {
                    o = acc[i][j];
                } else {
                    o = i32x4{__float_as_int(epi_val(acc[i][j][0], s4.x)),
                              __float_as_int(epi_val(acc[i][j][1], s4.y)),
                              __float_as_int(epi_val(acc[i][j][2], s4.z)),
                              __float_as_int(epi_val(acc[i][j][3], s4.w))};
                }
                int* dst = static_cast<int*>(e.y) + (size_t)row * n + col;
                if ((n & 3) == 0) {
                    *reinterpret_cast<i32x4*>(dst) = o;
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (col + c < n) dst[c] = o[c];
                }
            }
        }
    }
}

template <int OUT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void qgemm_big_w16(const i8* __restrict__ a, const i8* __restrict__ b, Epi e,
                   int m, int n, int k, int scales_dma, int band) {
    __shared__ __attribute__((aligned(16))) i8 lds[kW8Lds];

    const int tm = (m + kBigT - 1) / kBigT, tn = (n + kBigT - 1) / kBigT;
    const int ntiles = tm * tn;
    // tile t -> (bm, bn): tile t runs on XCD t % 8 (the grid is a multiple
    // of 8), and the tiles one XCD holds at once form a block of `band` tile
    // rows, so they share A and B panels in that XCD's L2
    auto tile_origin = [&](int t, int& bm, int& bn) {
        int pid = t;
        if (ntiles % 8 == 0) pid = (pid % 8) * (ntiles / 8) + pid / 8;
        const int bi = pid / (band * tn);
        const int first_m = bi * band;
        const int band_m = min(tm - first_m, band);
        const int in_band = pid - bi * band * tn;
        bm = (first_m + in_band % band_m) * kBigT;
        bn = (in_band / band_m) * kBigT;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0..7
    const int wr = 128 * (wave >> 2) + 64 * ((wave & 3) >> 1);  // sub-tile row
    const int wc = 128 * (wave & 1);                            // sub-tile column
    const int r16 = lane & 15, q4 = lane >> 4;
    const int nk = k / kK2;

    // DMA: instruction j (0..3) of this wave fills
    // tile rows 64 j + 8 wave + lane / 8 of A and of B; the lane's LDS chunk
    // position lane % 8 holds logical chunk (lane % 8) ^ swz, swz = (row >> 1)
    // & 7. Rows past M / N read a clamped (real) row.
    const int c16 = 16 * ((lane & 7) ^ ((4 * wave + (lane >> 4)) & 7));
    unsigned aoff[4], boff[4];
    const i8* abase;
    const i8* bbase;
    auto set_tile = [&](int bm, int bn) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 64 * j + 8 * wave + (lane >> 3);
            aoff[j] = (unsigned)(min(row, m - 1 - bm) * k + c16);
            boff[j] = (unsigned)(min(row, n - 1 - bn) * k + c16);
        }
        abase = a + (size_t)bm * k;
        bbase = b + (size_t)bn * k;
    };
    auto dma1 = [&](int kt, int st, int x) {  // instruction x (0..7): A for even x
        const int j = x >> 1;
        i8* dst = lds + st * kSlab2 + (x & 1) * (kBigT * kK2) + (64 * j + 8 * wave) * kK2;
        if (x & 1)
            __builtin_amdgcn_global_load_lds(bbase + (size_t)kt * kK2 + boff[j],
                                             (lds_void_p)dst, 16, 0, 0);
        else
            __builtin_amdgcn_global_load_lds(abase + (size_t)kt * kK2 + aoff[j],
                                             (lds_void_p)dst, 16, 0, 0);
    };
    auto first_slabs = [&](int bm, int bn) {
        const int nsl = nk > 1 ? 2 : 1;
        for (int sl = 0; sl < nsl; ++sl) {
            const i8* ab = a + (size_t)bm * k + (size_t)sl * kK2;
            const i8* bb = b + (size_t)bn * k + (size_t)sl * kK2;
#pragma unroll
            for (int x = 0; x < 8; ++x) {
                const int j = x >> 1;
                const int row = 64 * j + 8 * wave + (lane >> 3);
                i8* dst = lds + sl * kSlab2 + (x & 1) * (kBigT * kK2) + (64 * j + 8 * wave) * kK2;
                const unsigned off = (x & 1) ? (unsigned)(min(row, n - 1 - bn) * k + c16)
                                             : (unsigned)(min(row, m - 1 - bm) * k + c16);
                __builtin_amdgcn_global_load_lds(((x & 1) ? bb : ab) + off, (lds_void_p)dst,
                                                 16, 0, 0);
            }
        }
    };

    // Fragment x (A block i: x = i; B block j: x = 4 + j) of sub-step s in
    // stage st: row R = (wr or wc) + 16 block + r16, chunk 4 s + q4 at offset
    // (R << 7) | 16 ((4 s + q4) ^ swz(R)). swz(R) = (r16 >> 1) & 7 for every
    // block (wr, wc and 16 block are multiples of 16), so the offset is a
    // per-sub-step base plus 2048 block.
    const unsigned lds0 = lds_addr(lds);
    unsigned abase_s[2], bbase_s[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const unsigned sw = 16u * ((4 * s + q4) ^ ((r16 >> 1) & 7));
        abase_s[s] = lds0 + (unsigned)((wr + r16) << 7) + sw;
        bbase_s[s] = lds0 + (unsigned)(kBigT * kK2) + (unsigned)((wc + r16) << 7) + sw;
    }
    auto frag_addr = [&](int st, int s, int x) {
        return (x < 4 ? abase_s[s] + 2048u * x : bbase_s[s] + 2048u * (x - 4)) +
               (unsigned)(st * kSlab2);
    };
    auto read_frags = [&](int st, int s, i32x4 (&f)[12]) {
        // first-use order: B0 A0 A1 A2 A3 B1 .. B7
        f[4] = lds_read16(frag_addr(st, s, 4));
#pragma unroll
        for (int x = 0; x < 4; ++x) f[x] = lds_read16(frag_addr(st, s, x));
#pragma unroll
        for (int x = 5; x < 12; ++x) f[x] = lds_read16(frag_addr(st, s, x));
    };
    auto frags_wait = [&](i32x4 (&f)[12]) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]),
                       "+v"(f[5]), "+v"(f[6]), "+v"(f[7]), "+v"(f[8]), "+v"(f[9]),
                       "+v"(f[10]), "+v"(f[11]));
    };

    i32x4 acc[4][8];  // acc[i][j] = C^T block (n block j, m block i)
    // 32 MFMAs on f (read in first-use order by the previous call), reading
    // the next sub-step (rst, rs) into nf on the kW16Rd schedule. With a DMA
    // tag, the 8 DMA instructions of slab dkt into stage dst go out after
    // MFMAs 1, 5, .., 29.
    auto step = [&](i32x4 (&f)[12], bool piecewise, int rst, int rs, i32x4 (&nf)[12],
                    auto dma, int dkt, int dst) {
#pragma unroll
        for (int q = 0; q < 32; ++q) {
            const int i = q & 3, j = q >> 2;
            if (piecewise && kW16Wait[q] >= 0) lgkm_wait_xy(kW16Wait[q], f[4 + j], f[i]);
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f[4 + j], f[i], acc[i][j], 0, 0, 0);
            if constexpr (decltype(dma)::value) {
                if ((q & 3) == 1) {
                    __builtin_amdgcn_sched_barrier(0);
                    dma1(dkt, dst, q >> 2);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (kW16Rd[q] >= 0) {
                __builtin_amdgcn_sched_barrier(0);
                nf[kW16Rd[q]] = lds_read16(frag_addr(rst, rs, kW16Rd[q]));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    int t = blockIdx.x;
    if (t < ntiles) {
        int bm0, bn0;
        tile_origin(t, bm0, bn0);
        first_slabs(bm0, bn0);
    }
    for (; t < ntiles; t += gridDim.x) {
        int bm, bn;
        tile_origin(t, bm, bn);
        set_tile(bm, bn);
        // slabs 0 and 1 of this tile are in flight (issued before the
        // previous tile's epilogue, or just above): wait for them and for
        // that epilogue's stores; after the barrier every wave's DMAs are
        // visible
        wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (scales_dma && wave == 0) {
            const int c = min(bn + 4 * lane, n - 4);
            __builtin_amdgcn_global_load_lds(e.sb_vec + c, (lds_void_p)(lds + kW8Scl), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

        // Per slab kt (stage st = kt & 1), with F0 = (kt, 0) read: sub-step 0
        // multiplies (kt, 0) while (kt, 1) is read; wait for (kt, 1) and slab
        // kt+1's DMA; barrier (every wave is past its reads of stage st; slab
        // kt+1 is visible); sub-step 1 multiplies (kt, 1) while (kt+1, 0) is
        // read from stage st ^ 1 and stage st is refilled with slab kt + 2.
        // After the last slab, F0 reads a stale stage: in bounds, unused.
        i32x4 f0[12], f1[12];
        read_frags(0, 0, f0);
        auto slab = [&](int kt, auto dma) {
            const int st = kt & 1;
            step(f0, true, st, 1, f1, std::false_type{}, 0, 0);
            frags_wait(f1);
            wait_vmcnt<0>();  // slab kt+1 (the only DMA in flight) and the scales
            __builtin_amdgcn_s_barrier();
            step(f1, false, st ^ 1, 0, f0, dma, kt + 2, st);
        };
        int kt = 0;
        for (; kt + 2 < nk; ++kt) slab(kt, std::true_type{});
        for (; kt < nk; ++kt) slab(kt, std::false_type{});
        frags_wait(f0);   // the last (unused) reads land before f0's registers are reused
        wait_vmcnt<0>();  // the scales of a one-slab tile
        __builtin_amdgcn_s_barrier();
        const int tn_ = t + gridDim.x;
        if (tn_ < ntiles) {
            int nbm, nbn;
            tile_origin(tn_, nbm, nbn);
            first_slabs(nbm, nbn);
        }
        w16_epilogue<OUT>(acc, lds + kW8Spare + wave * kW8Stg,
                          scales_dma ? reinterpret_cast<const float*>(lds + kW8Scl) + wc : nullptr,
                          e, m, n, bm + wr, bn + wc, lane, r16, q4);
    }
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------
// reference qgemm.cu:599-604 bounds m*n*k <= 2^38; this build instead bounds
// K so the int32 accumulator provably cannot wrap (|a*b| <= 128*128), which
// admits the large prefill shapes (4096 x 28672 x 8192).
void qgemm_check(int m, int n, int k) {
    if (m < 0 || n < 0 || k < 0) inval("m, n, k must be >= 0");
    if (k > 131071) inval("qgemm K too large for exact int32 accumulation (K <= 131071)");
}

size_t out_elem_bytes(int out) {
    return out == kOutBF16 || out == kOutF16 ? 2 : 4;
}

template <int OUT>
void qgemm_dispatch(const i8* a, const i8* b, const Epi& e, int m, int n, int k,
                    hipStream_t s, KFold* defer) {
    const bool aligned = (k % 16 == 0) && ((uintptr_t)a % 16 == 0) &&
                         ((uintptr_t)b % 16 == 0);
    // FT_QGEMM_KERNEL: 1 skinny, 2 tiled, 3 scalar, 4 big, 5 gemv, 6 decode
    const int force = tune(Tune::QgemmKernel, 0);
    if (!aligned || force == 3) {
        const long long total = (long long)m * n;
        qgemm_scalar<OUT><<<grid_1d(total, 256, 1 << 30), 256, 0, s>>>(a, b, e, m, n, k);
        launch_check("qgemm scalar kernel launch");
        return;
    }
    // decode shapes. Measured on MI355X (HIP-graph replays, weights cycled
    // past the 256 MB last-level cache): at M = 1 the dot4 GEMV streams W
    // fastest (1 KB contiguous per load instruction; N=28672 K=4096:
    // 24.1 us vs 28.3 us), from M = 2 the MFMA decode kernel wins (its dot
    // products cost 1/16 of the dot4 instructions; N=11008 K=4096 M=8:
    // 14.0 us vs 37.1 us).
    if ((m == 1 && force == 0) || force == 5) {
        if (m > 8) inval("gemv qgemm supports m <= 8");
        const long long waves = std::min<long long>((n + kGemvRows - 1) / kGemvRows,
                                                    (long long)dev_info().cu_count * 16);
        const unsigned grid = (unsigned)((waves + 3) / 4);
        switch (m) {
        case 1: qgemv_dot4<1, OUT><<<grid, 256, 0, s>>>(a, b, e, n, k); break;
        case 2: qgemv_dot4<2, OUT><<<grid, 256, 0, s>>>(a, b, e, n, k); break;
        case 3: qgemv_dot4<3, OUT><<<grid, 256, 0, s>>>(a, b, e, n, k); break;
        case 4: qgemv_dot4<4, OUT><<<grid, 256, 0, s>>>(a, b, e, n, k); break;
        case 5: qgemv_dot4<5, OUT><<<grid, 256, 0, s>>>(a, b, e, n, k); break;
        case 6: qgemv_dot4<6, OUT><<<grid, 256, 0, s>>>(a, b, e, n, k); break;
        case 7: qgemv_dot4<7, OUT><<<grid, 256, 0, s>>>(a, b, e, n, k); break;
        default: qgemv_dot4<8, OUT><<<grid, 256, 0, s>>>(a, b, e, n, k); break;
        }
        launch_check("qgemm gemv kernel launch");
        return;
    }
    if ((m <= 16 && force == 0) || force == 6) {
        if (m > 16) inval("decode qgemm supports m <= 16");
        const int tiles = (n + 15) / 16;
        const unsigned grid = (unsigned)tiles;
        // waves per 16-column tile: one long stream per wave when there are
        // enough tiles, else split K so that every CU still gets waves
        // (N=6144: 1 wave per tile 8.3 us vs 9.3 us; N=4096 K=14336: 2 waves
        // 13.4 us vs 18.9 us)
        int kw = tiles >= 320 ? 1 : tiles >= 128 ? 2 : 4;
        const int kw_forced = tune(Tune::QgemmDecKw, 0);
        if (kw_forced == 1 || kw_forced == 2 || kw_forced == 4) kw = kw_forced;
        // W and A through a 2-stage LDS ring in whole lines, W non-temporal
        // (C2 chain, M = 8 / 16: 21.1 / 23.3 us with register operands,
        // 16.5 / 17.4 us with the ring; 3 stages the same, 4 stages slower:
        // 64 KB per wave leaves 2 waves per CU; plain W loads 19.1 / 19.4 us)
        if (kw == 1 && k % kDwChunk == 0 && tune(Tune::QgemmDecRegs, 0) == 0) {
            qgemm_dec_lds<2, 2, OUT><<<grid, 64, 0, s>>>(a, b, e, m, n, k);
            launch_check("qgemm decode lds kernel launch");
            return;
        }
        if (kw == 1)
            qgemm_dec<1, OUT><<<grid, 64, 0, s>>>(a, b, e, m, n, k);
        else if (kw == 2)
            qgemm_dec<2, OUT><<<grid, 128, 0, s>>>(a, b, e, m, n, k);
        else
            qgemm_dec<4, OUT><<<grid, 256, 0, s>>>(a, b, e, m, n, k);
        launch_check("qgemm decode kernel launch");
        return;
    }
    if ((m <= 64 && force != 2 && force != 4) || force == 1) {
        if (m > 64) inval("skinny qgemm supports m <= 64");
        const int cus = dev_info().cu_count;
        const int mt = (m + 15) / 16;
        const bool ring = k % kSlChunk == 0 && tune(Tune::QgemmSkRegs, 0) == 0;
        // LDS ring: NW waves of 16 columns each; the ring holds the A rows
        // and the NW * 16 W rows of `stages` 256-byte K chunks
        // 3 ring stages (two chunks in flight; one workgroup per CU). 8 waves
        // (128 columns) when the column workgroups alone cover 3/4 of the CUs:
        // M = 64, graph replays, weights cycled past the last-level cache:
        // N=28672 K=4096 28.5 us against 30.2 with 4 waves and 2 stages;
        // N=4096 K=4096 9.9 vs 10.8; N=4096 K=14336 17.3 vs 19.6;
        // N=6144 K=4096 12.3 vs 13.9 (K split 2)
        const int stages = ring ? (tune(Tune::QgemmSkStages, 3) == 2 ? 2 : 3) : 2;
        const int wide = (n + 127) / 128;
        const int nw_pick = 4 * wide >= 3 * cus ? 8 : 4;
        const int nw = ring && mt >= 2 && tune(Tune::QgemmSkWaves, nw_pick) == 8 ? 8 : 4;
        const int lds_bytes = (16 * (mt <= 1 ? 1 : mt <= 2 ? 2 : 4) + 16 * nw) * kSlChunk * stages;
        const int per_cu = ring ? std::max(1, (160 << 10) / lds_bytes) : 2;
        const int col_wgs = (n + 16 * nw - 1) / (16 * nw);
        // K chunks the split divides: 256-byte ring chunks, 1 KB register chunks
        const int chunks = ring ? k / kSlChunk : (k + kSkChunk - 1) / kSkChunk;
        // no K split once the column workgroups alone fill 3/4 of the
        // resident slots (M=64, N=28672, K=4096: 38.9 us against 45.0 us
        // split in two, which also needs the fold launch); below that, as
        // many splits as fit in one round of resident workgroups (a partial
        // second round costs a whole extra round: N=6144, split 3 on 256
        // slots, 14.2 us against 12.3 with split 2)
        const int slots = per_cu * cus;
        int ksplit = 4 * col_wgs >= 3 * slots
                         ? 1
                         : std::max(1, std::min(slots / col_wgs, chunks));
        const int forced_split = tune(Tune::QgemmKsplit, 0);
        if (forced_split > 0) ksplit = std::min(forced_split, chunks);
        if (ksplit > 65535) ksplit = 65535;
        // the K split's int32 partials are folded by a second launch: a fold
        // by the last workgroup of each column tile (device-scope release /
        // acquire fences around a counter) measured 3-4x slower on every
        // split shape (N=6144 K=4096: 37.0 against 12.0 us)
        int* part = nullptr;
        if (ksplit > 1)
            part = (int*)scratch(Scratch::GemmPartials,
                                 (size_t)ksplit * m * n * sizeof(int), s);
        dim3 grid(col_wgs, ksplit);
        if (ring) {
#define FT_SK_LDS(MT, S, NW)                                                             \
    qgemm_skinny_lds<MT, S, NW, OUT, false><<<grid, 64 * NW, 0, s>>>(a, b, e, m, n, k, ksplit, \
                                                                     part, 0, nullptr,        \
                                                                     SwqGrid{})
            if (mt <= 1) {
                if (stages == 3) FT_SK_LDS(1, 3, 4); else FT_SK_LDS(1, 2, 4);
            } else if (mt <= 2) {
                if (nw == 8) { if (stages == 3) FT_SK_LDS(2, 3, 8); else FT_SK_LDS(2, 2, 8); }
                else { if (stages == 3) FT_SK_LDS(2, 3, 4); else FT_SK_LDS(2, 2, 4); }
            } else {
                if (nw == 8) { if (stages == 3) FT_SK_LDS(4, 3, 8); else FT_SK_LDS(4, 2, 8); }
                else { if (stages == 3) FT_SK_LDS(4, 3, 4); else FT_SK_LDS(4, 2, 4); }
            }
#undef FT_SK_LDS
        } else if (mt <= 1)
            qgemm_skinny<1, OUT><<<grid, 256, 0, s>>>(a, b, e, m, n, k, ksplit, part);
        else if (mt <= 2)
            qgemm_skinny<2, OUT><<<grid, 256, 0, s>>>(a, b, e, m, n, k, ksplit, part);
        else
            qgemm_skinny<4, OUT><<<grid, 256, 0, s>>>(a, b, e, m, n, k, ksplit, part);
        launch_check("qgemm skinny kernel launch");
        if (ksplit > 1 && defer) {  // the caller's next launch folds them
            defer->part = part;
            defer->ksplit = ksplit;
            defer->n = n;
            defer->mn = (long long)m * n;
            defer->sa_dev = e.sa_dev;
            defer->sb_vec = e.sb_vec;
            return;
        }
        if (ksplit > 1) {
            const long long mn = (long long)m * n;
            qgemm_ksum<OUT><<<grid_1d(mn, 256, 1 << 30), 256, 0, s>>>(part, e, m, n, ksplit,
                                                                      nullptr);
            launch_check("qgemm k-split fold launch");
        }
        return;
    }
    if ((m >= kBigT && n >= kBigT && force != 2) || force == 4) {
        const long long tiles = (long long)((m + kBigT - 1) / kBigT) * ((n + kBigT - 1) / kBigT);
        if (tiles > (1LL << 30)) inval("qgemm problem too large for one launch");
        // FT_QGEMM_BIG (tests): 1 the 64-byte-slab kernel, 2 the
        // register-staged one, on shapes that would take the default
        const int big = tune(Tune::QgemmBig, 0);
        if (k % kK2 == 0 && big == 0) {
            // persistent: a multiple of 8 workgroups (XCD-aware order), at
            // most one per CU. 8 waves by default: on C5a (4096 x 8192 x
            // 28672, random int8) the MFMA pipes are busy 70% of the cycles
            // against 60% with 4 waves (0.88 vs 0.93 ms); 16x16x64 MFMAs by
            // default: 0.807 vs 0.885 ms with 32x32x32 (same schedule; the
            // board power limit admits more 16x16x64 work per second)
            const long long cus = dev_info().cu_count;
            long long grid = std::min<long long>(tiles, cus);
            if (grid >= 8) grid -= grid % 8;
            const int band = std::max(1, tune(Tune::QgemmBand, kBigBand));
            const int scales_dma = e.sb_vec && (n % 4 == 0) &&
                                   ((uintptr_t)e.sb_vec % 16 == 0);
            qgemm_big_w16<OUT><<<(unsigned)grid, 512, 0, s>>>(a, b, e, m, n, k, scales_dma,
                                                              band);
        }
        else if (k % kBigK == 0 && big != 2)
            qgemm_big_dma<OUT><<<(unsigned)tiles, 256, 0, s>>>(a, b, e, m, n, k);
        else
            qgemm_big<OUT><<<(unsigned)tiles, 256, 0, s>>>(a, b, e, m, n, k);
        launch_check("qgemm big kernel launch");
        return;
    }
    constexpr int BM = 128, BN = 128;
    dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM);
    qgemm_tiled<BM, BN, 2, 2, OUT><<<grid, 256, 0, s>>>(a, b, e, m, n, k);
    launch_check("qgemm tiled kernel launch");
}

void qgemm_run(const i8* a, const i8* b, Epi e, int out, int m, int n, int k,
               hipStream_t s, KFold* defer = nullptr) {
    qgemm_check(m, n, k);
    if (m == 0 || n == 0) return;
    if (!e.y) inval("qgemm: null output");
    if (k == 0) {
        const long long bytes = (long long)m * n * out_elem_bytes(out);
        zero_fill_kernel<<<grid_1d(bytes, 256, 4096), 256, 0, s>>>((unsigned char*)e.y, bytes);
        launch_check("qgemm zero-fill kernel launch");
        return;
    }
    if (!a || !b) inval("qgemm: null operand");
    switch (out) {
    case kOutF32: qgemm_dispatch<kOutF32>(a, b, e, m, n, k, s, defer); break;
    case kOutBF16: qgemm_dispatch<kOutBF16>(a, b, e, m, n, k, s, defer); break;
    case kOutF16: qgemm_dispatch<kOutF16>(a, b, e, m, n, k, s, defer); break;
    case kOutI32: qgemm_dispatch<kOutI32>(a, b, e, m, n, k, s, defer); break;
    default: inval("qgemm: unknown output type");
    }
}

// The skinny ring kernel with the SwiGLU maxima in its epilogue, launched
// only where qgemm_dispatch takes qgemm_skinny_lds unsplit for the same
// shape (same waves, stages and column tiles), so y is the same bits.
// Returns 0 (not launched), 1 (the per-workgroup maxima are in part) or 2
// (q given and every workgroup resident: the codes and *scale_out written).
template <int OUT>
int swiglu_max_launch(const i8* a, const i8* b, const Epi& e, int m, int inter, int k,
                      hipStream_t s, float*& part, int& nparts, signed char* q,
                      float* scale_out) {
    const int n = 2 * inter;
    const bool aligned = (k % 16 == 0) && ((uintptr_t)a % 16 == 0) && ((uintptr_t)b % 16 == 0);
    if (!aligned || tune(Tune::QgemmKernel, 0) != 0 || m <= 16 || m > 64) return 0;
    if (k % kSlChunk != 0 || tune(Tune::QgemmSkRegs, 0) != 0) return 0;
    if (tune(Tune::QgemmSkStages, 3) == 2 || tune(Tune::QgemmKsplit, 0) != 0) return 0;
    const int cus = dev_info().cu_count;
    const int mt = (m + 15) / 16;  // 2 or 4
    const int wide = (n + 127) / 128;
    const int nw_pick = 4 * wide >= 3 * cus ? 8 : 4;
    const int nw = tune(Tune::QgemmSkWaves, nw_pick) == 8 ? 8 : 4;
    if (inter % (8 * nw) != 0) return 0;
    const int lds_bytes = (16 * (mt <= 2 ? 2 : 4) + 16 * nw) * kSlChunk * 3;
    const int slots = std::max(1, (160 << 10) / lds_bytes) * cus;
    const int col_wgs = inter / (8 * nw);
    if (4 * col_wgs < 3 * slots) return 0;  // the dispatch would split K
    part = (float*)scratch(Scratch::QuantMax, (size_t)col_wgs * sizeof(float), s);
    nparts = col_wgs;
    SwqGrid sq;
    if (q) sq = SwqGrid{q, scale_out, gridmax_state(col_wgs, s)};
    dim3 grid(col_wgs, 1);
    int launched = 0;
    auto go = [&](auto kernel, int threads) {
        if (sq.q && !grid_resident((const void*)kernel, col_wgs, threads, GridUse::SwiGLU)) sq = SwqGrid{};
        if (!sq.q && !e.y) return;  // the partials-only form needs y stored
        kernel<<<grid, threads, 0, s>>>(a, b, e, m, n, k, 1, nullptr, inter, part, sq);
        launch_check("qgemm swiglu-max kernel launch");
        launched = sq.q ? 2 : 1;
    };
    if (mt <= 2) {
        if (nw == 8) go(qgemm_skinny_lds<2, 3, 8, OUT, true>, 512);
        else go(qgemm_skinny_lds<2, 3, 4, OUT, true>, 256);
    } else {
        if (nw == 8) go(qgemm_skinny_lds<4, 3, 8, OUT, true>, 512);
        else go(qgemm_skinny_lds<4, 3, 4, OUT, true>, 256);
    }
    return launched;
}

}  // namespace

int qgemm_swiglu_max(const signed char* a, const signed char* b, const float* sa_dev,
                     const float* sb_vec, void* y, int y_dtype, int m, int inter, int k,
                     hipStream_t s, float*& part, int& nparts, signed char* q,
                     float* scale_out) {
    if (!sa_dev || !sb_vec) inval("qgemm: a device scale and per-channel scales are required");
    if (inter < 1 || (long long)m * 2 * inter > (1LL << 31) - 1) return 0;
    qgemm_check(m, 2 * inter, k);
    if (m == 0 || k == 0 || (!y && !q) || !a || !b) return 0;
    Epi e{y, 0.0f, sa_dev, 0.0f, sb_vec};
    switch (y_dtype) {
    case FT_DT_F32:
        return swiglu_max_launch<kOutF32>(a, b, e, m, inter, k, s, part, nparts, q, scale_out);
    case FT_DT_BF16:
        return swiglu_max_launch<kOutBF16>(a, b, e, m, inter, k, s, part, nparts, q, scale_out);
    case FT_DT_F16:
        return swiglu_max_launch<kOutF16>(a, b, e, m, inter, k, s, part, nparts, q, scale_out);
    default: inval("qgemm: unknown output dtype code");
    }
}

void kfold_store(const KFold& f, void* y, int dtype, int m, hipStream_t s) {
    if (f.ksplit < 2 || f.n < 1 || f.mn != (long long)m * f.n)
        inval("kfold_store: partials do not match the output");
    if (!y) inval("kfold_store: null output");
    Epi e{y, 0.0f, f.sa_dev, 0.0f, f.sb_vec};
    const unsigned grid = grid_1d(f.mn, 256, 1 << 30);
    switch (dtype) {
    case FT_DT_F32:
        qgemm_ksum<kOutF32><<<grid, 256, 0, s>>>(f.part, e, m, f.n, f.ksplit, f.res);
        break;
    case FT_DT_BF16:
        qgemm_ksum<kOutBF16><<<grid, 256, 0, s>>>(f.part, e, m, f.n, f.ksplit, f.res);
        break;
    case FT_DT_F16:
        qgemm_ksum<kOutF16><<<grid, 256, 0, s>>>(f.part, e, m, f.n, f.ksplit, f.res);
        break;
    default: inval("kfold_store: unknown dtype code");
    }
    launch_check("qgemm k-split fold launch");
}

bool qgemm_deferred(const signed char* a, const signed char* b, const float* sa_dev,
                    const float* sb_vec, void* y, int y_dtype, int m, int n, int k,
                    hipStream_t s, KFold& f) {
    if (!sa_dev || !sb_vec) inval("qgemm: a device scale and per-channel scales are required");
    int out;
    switch (y_dtype) {
    case FT_DT_F32: out = kOutF32; break;
    case FT_DT_BF16: out = kOutBF16; break;
    case FT_DT_F16: out = kOutF16; break;
    default: inval("qgemm: unknown output dtype code");
    }
    f = KFold{};
    Epi e{y, 0.0f, sa_dev, 0.0f, sb_vec};
    qgemm_run(a, b, e, out, m, n, k, s, &f);
    return f.ksplit > 1;
}

}  // namespace ft

extern "C" {

int ft_qgemm_launch(const signed char* aq, const signed char* bq, float* y,
                    int m, int n, int k, float sa, float sb,
                    uintptr_t stream) {
    return ft::guarded([&] {
        ft::Epi e{y, sa, nullptr, sb, nullptr};
        ft::qgemm_run(aq, bq, e, ft::kOutF32, m, n, k, ft::as_stream(stream));
    });
}

int ft_qgemm_perchannel_launch(const signed char* aq, const signed char* bq,
                               const float* sb_vec, float* y, int m, int n,
                               int k, float sa, uintptr_t stream) {
    return ft::guarded([&] {
        if (!sb_vec) ft::inval("per-channel scale vector is required");
        ft::Epi e{y, sa, nullptr, 0.0f, sb_vec};
        ft::qgemm_run(aq, bq, e, ft::kOutF32, m, n, k, ft::as_stream(stream));
    });
}

int ft_qgemm_launch_ex(const signed char* aq, const signed char* bq,
                       const float* sb_vec, float sb, float sa,
                       const float* sa_dev, void* y, int y_dtype, int m, int n,
                       int k, uintptr_t stream) {
    return ft::guarded([&] {
        int out;
        switch (y_dtype) {
        case FT_DT_F32: out = ft::kOutF32; break;
        case FT_DT_BF16: out = ft::kOutBF16; break;
        case FT_DT_F16: out = ft::kOutF16; break;
        default: ft::inval("qgemm: unknown output dtype code");
        }
        ft::Epi e{y, sa, sa_dev, sb, sb_vec};
        ft::qgemm_run(aq, bq, e, out, m, n, k, ft::as_stream(stream));
    });
}

int ft_rmsnorm_qgemm_launch(const void* x, int x_dtype, const float* w,
                            const void* residual, float eps, const signed char* bq,
                            const float* sb_vec, float sb, void* y, int y_dtype,
                            signed char* q, float* scale_out, int rows, int n, int k,
                            uintptr_t stream) {
    return ft::guarded([&] {
        int out;
        switch (y_dtype) {
        case FT_DT_F32: out = ft::kOutF32; break;
        case FT_DT_BF16: out = ft::kOutBF16; break;
        case FT_DT_F16: out = ft::kOutF16; break;
        default: ft::inval("rmsnorm_qgemm: unknown output dtype code");
        }
        if (rows < 0 || n < 0 || k <= 0)
            ft::inval("rmsnorm_qgemm: rows and n must be >= 0 and k > 0");
        // every shape check before the first launch: no partial writes on error
        ft::qgemm_check(rows, n, k);
        if (rows == 0) return;
        if (!x || !w || !q || !scale_out || (n > 0 && (!bq || !y)))
            ft::inval("rmsnorm_qgemm: null operand");
        hipStream_t s = ft::as_stream(stream);
        if (n == 0) {
            // no output columns: the codes and the scale are still produced
            const int rc = ft_rmsnorm_quant_launch(x, x_dtype, w, residual, q, scale_out, rows,
                                                   k, eps, stream);
            if (rc != FT_OK) throw ft::Error{rc, ft_last_error()};
            return;
        }
        const size_t esz = x_dtype == FT_DT_F32 ? 4 : 2;
        const bool fusable =
            rows == 1 && k <= ft::kGemvChunks * 1024 && k % 16 == 0 &&
            (uintptr_t)x % (4 * esz) == 0 && (!residual || (uintptr_t)residual % (4 * esz) == 0) &&
            (uintptr_t)w % 16 == 0 && (uintptr_t)bq % 16 == 0 && (uintptr_t)q % 4 == 0 &&
            ft::tune(ft::Tune::RmsqGemvSplit, 0) == 0;
        if (!fusable) {
            // the two-step chain: rmsnorm_quant, then the GEMM on its codes
            // with the device scale
            const int rc = ft_rmsnorm_quant_launch(x, x_dtype, w, residual, q, scale_out, rows,
                                                   k, eps, stream);
            if (rc != FT_OK) throw ft::Error{rc, ft_last_error()};
            ft::Epi e{y, 0.0f, scale_out, sb, sb_vec};
            ft::qgemm_run(q, bq, e, out, rows, n, k, s);
            return;
        }
        if (k % 4 != 0) ft::inval("rmsnorm_qgemm: k must be a multiple of 4");
        ft::Epi e{y, 0.0f, scale_out, sb, sb_vec};
        // three workgroups per CU with the rows split evenly over their
        // waves (C2, N = 11008: 3.58 rows per wave, 10.7 us per chain
        // against 11.0 us for 688 workgroups of 4-row waves, same box);
        // wider N: enough workgroups for one pass of kGemvRows rows per wave
        long long grid = 3LL * ft::dev_info().cu_count;
        if (grid * 4 * ft::kGemvRows < n) grid = (n + 4 * ft::kGemvRows - 1) / (4 * ft::kGemvRows);
        if (grid > 0x7fffffffLL) ft::inval("rmsnorm_qgemm problem too large for one launch");
#define FT_RQG(T, O)                                                                  \
    do {                                                                              \
        const unsigned g_ = (unsigned)grid;                                           \
        if (residual)                                                                 \
            ft::rmsq_gemv<T, true, O><<<g_, 256, 0, s>>>(                             \
                (const T*)x, (const T*)residual, w, eps, bq, e, n, k, q, scale_out);  \
        else                                                                          \
            ft::rmsq_gemv<T, false, O><<<g_, 256, 0, s>>>(                            \
                (const T*)x, nullptr, w, eps, bq, e, n, k, q, scale_out);             \
    } while (0)
#define FT_RQG_T(T)                                   \
    do {                                              \
        if (out == ft::kOutF32) FT_RQG(T, ft::kOutF32);   \
        else if (out == ft::kOutBF16) FT_RQG(T, ft::kOutBF16); \
        else FT_RQG(T, ft::kOutF16);                  \
    } while (0)
        switch (x_dtype) {
        case FT_DT_F32: FT_RQG_T(float); break;
        case FT_DT_BF16: FT_RQG_T(ft::bf16); break;
        case FT_DT_F16: FT_RQG_T(ft::f16); break;
        default: ft::inval("rmsnorm_qgemm: unknown x dtype code");
        }
#undef FT_RQG_T
#undef FT_RQG
        ft::launch_check("rmsnorm_qgemm kernel launch");
    });
}

int ft_qgemm_i32_launch(const signed char* aq, const signed char* bq, int* acc,
                        int m, int n, int k, uintptr_t stream) {
    return ft::guarded([&] {
        ft::Epi e{acc, 1.0f, nullptr, 1.0f, nullptr};
        ft::qgemm_run(aq, bq, e, ft::kOutI32, m, n, k, ft::as_stream(stream));
    });
}

}  // extern "C"
