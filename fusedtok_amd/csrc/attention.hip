// Flash-decoding attention (contiguous and paged KV) and KV append for
// gfx950.
//
//   out[b,h] = softmax(q[b,h] . K[b,h/G]^T / sqrt(D)) . V[b,h/G]
//
// Work decomposition (both cache layouts): a work unit is one
// (sequence b, kv head, token chunk of `chunk` rows). The grid is
// (Hkv * cmax, B) with cmax = ceil(span / chunk), span being the cache
// capacity (T, or table width * page). A unit whose chunk starts at or past
// lens[b] exits at once, so the work follows the REAL lengths rather than
// the capacity (the reference slices the capacity: attention.cu:1816-1821).
// Every live unit writes, for each of the G q heads of its kv group, the
// float32 partial (m = max score, l = sum exp(s - m), acc[D] = sum
// exp(s - m) v) into a library-owned workspace; a combine kernel folds a
// row's partials with the log-sum-exp rule and divides by l. len == 0 rows
// produce zeros (reference attention.cu:1349-1350).
//
// Two kernel families:
//   attn_decode_stream bf16/fp16 storage, D == 128, G <= 16: QK^T and PV on
//     + attn_combine_  the matrix cores (v_mfma_f32_16x16x32_{bf16,f16});
//       stream         every K/V byte is read once, straight into the MFMA
//                      operand layout with 16-byte loads, double-buffered;
//                      equal token segments per workgroup (stream split).
//   attn_chunk_generic any storage type, D % 4 == 0 <= 512, any G: VALU
//     + attn_combine   dot products, chunk scores staged in LDS; the grid
//                      covers the cache capacity in fixed chunks.
#include <climits>
#include "ft_common.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>

namespace ft {
namespace {

constexpr int kMaxDim = 512;
constexpr int kGenNT = 256;      // generic stage-1 workgroup
constexpr int kGenHeads = 8;     // q heads per generic pass
constexpr int kGenMaxChunk = 512;

// reference attention.cu:184-193
void attention_check(int batch, int hq, int hkv, long long t_seq, int dim) {
    if (batch < 0 || hq < 1 || hkv < 1 || t_seq < 0 || dim < 1)
        inval("attention shapes must satisfy batch>=0, heads>=1, rows>=0, dim>=1");
    if (hq % hkv != 0)
        inval("q heads must be a multiple of kv heads (contiguous GQA groups)");
    if (dim % 4 != 0 || dim > kMaxDim)
        inval("dim must be a multiple of 4 and at most 512");
}

inline int pow2_ceil(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

__device__ __forceinline__ int pow2_ceil_dev(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

constexpr float kLog2e = 1.4426950408889634f;

// Device-resident lengths are not read back by the host. A length outside
// [0, span] (span = the cache's row capacity) is clamped into it, so no
// value can make a kernel index past the cache or the block table.
__device__ __forceinline__ int clamp_len(const int* lens, int b, int span) {
    if (!lens) return span;
    return min(max(lens[b], 0), span);
}

// Chunk length: a power of two in [lo, hi] so that the capacity grid holds
// about `target` units.
int choose_chunk(int batch, int hkv, long long span, int lo, int hi,
                 long long target) {
    long long rows = (long long)batch * hkv * span;
    int c = lo;
    while (c < hi && rows / c > target) c <<= 1;
    return c;
}

struct RowMap {
    // contiguous: element offset (((b*hkv + kv) * t_rows) + t) * dim
    // paged:      element offset ((table[b*S + t/P] * hkv + kv) * P + t%P) * dim
    const int* table;
    int hkv, dim, rows_or_page, tbl_width, page_shift;  // page_shift >= 0 if P is 2^k
    __device__ __forceinline__ size_t operator()(int b, int kv, int t) const {
        if (!table)
            return (((size_t)b * hkv + kv) * rows_or_page + t) * dim;
        int pg, off;
        if (page_shift >= 0) {
            pg = t >> page_shift;
            off = t & (rows_or_page - 1);
        } else {
            pg = t / rows_or_page;
            off = t - pg * rows_or_page;
        }
        const int blk = table[(size_t)b * tbl_width + pg];
        return (((size_t)blk * hkv + kv) * rows_or_page + off) * dim;
    }
};

// ---------------------------------------------------------------------------
// generic stage 1
// ---------------------------------------------------------------------------
template <typename T, int CPL>
__global__ __launch_bounds__(kGenNT) void attn_chunk_generic(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int* __restrict__ lens, RowMap rm, float* __restrict__ ws_ml,
    float* __restrict__ ws_acc, int hq, int group, int span, int chunk,
    int cmax, float scale_log2) {
    __shared__ float sc[kGenHeads][kGenMaxChunk];
    __shared__ float ms[kGenHeads], ls[kGenHeads];
    __shared__ float4 red[kGenNT];

    const int per_b = rm.hkv * cmax;
    const int b = blockIdx.x / per_b;
    const int kv = (blockIdx.x - b * per_b) / cmax;
    const int c = blockIdx.x - b * per_b - kv * cmax;
    const int len = clamp_len(lens, b, span);
    const int t0 = c * chunk;
    if (t0 >= len) return;
    const int n = min(chunk, len - t0);
    const int dim = rm.dim;
    const int dc = dim >> 2;                     // 4-element chunks per row
    const int lpt = min(64, pow2_ceil_dev(dc));  // lanes per token (phase 1)
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int sub = lane / lpt, li = lane % lpt;
    const int tpw = 64 / lpt;

    for (int g0 = 0; g0 < group; g0 += kGenHeads) {
        const int gc = min(kGenHeads, group - g0);
        // ---- phase 1: scores s[g][t] = scale * q_g . k_t ------------------
        float4 qr[kGenHeads][CPL];
#pragma unroll
        for (int g = 0; g < kGenHeads; ++g)
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int ch = li + i * lpt;
                qr[g][i] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (g < gc && ch < dc)
                    qr[g][i] = St<T>::ld4(
                        q + ((size_t)b * hq + (size_t)kv * group + g0 + g) * dim +
                        4 * ch);
            }
        for (int t = wave * tpw + sub; t < n; t += 4 * tpw) {
            const T* kr = k + rm(b, kv, t0 + t);
            float part[kGenHeads];
#pragma unroll
            for (int g = 0; g < kGenHeads; ++g) part[g] = 0.0f;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int ch = li + i * lpt;
                if (ch < dc) {
                    const float4 kk = St<T>::ld4(kr + 4 * ch);
#pragma unroll
                    for (int g = 0; g < kGenHeads; ++g)
                        part[g] += qr[g][i].x * kk.x + qr[g][i].y * kk.y +
                                   qr[g][i].z * kk.z + qr[g][i].w * kk.w;
                }
            }
#pragma unroll
            for (int g = 0; g < kGenHeads; ++g)
                for (int o = lpt >> 1; o > 0; o >>= 1)
                    part[g] += __shfl_xor(part[g], o, 64);
            if (li == 0) {
#pragma unroll
                for (int g = 0; g < kGenHeads; ++g)
                    if (g < gc) sc[g][t] = part[g] * scale_log2;
            }
        }
        __syncthreads();
        // ---- phase 2: chunk softmax statistics -----------------------------
        for (int g = wave; g < gc; g += kGenNT / 64) {
            float m = -INFINITY;
            for (int t = lane; t < n; t += 64) m = fmaxf(m, sc[g][t]);
            m = wave_max(m);
            float l = 0.0f;
            for (int t = lane; t < n; t += 64) {
                const float p = exp2f(sc[g][t] - m);
                sc[g][t] = p;
                l += p;
            }
            l = wave_sum(l);
            if (lane == 0) {
                ms[g] = m;
                ls[g] = l;
            }
        }
        __syncthreads();
        // ---- phase 3: acc[g][d] = sum_t p[g][t] v[t][d] --------------------
        const int dcp = pow2_ceil_dev(dc);
        const int tg_n = kGenNT / dcp;
        const int my_dc = tid % dcp, my_tg = tid / dcp;
        float4 acc[kGenHeads];
#pragma unroll
        for (int g = 0; g < kGenHeads; ++g) acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (my_dc < dc) {
            for (int t = my_tg; t < n; t += tg_n) {
                const float4 vv = St<T>::ld4(v + rm(b, kv, t0 + t) + 4 * my_dc);
#pragma unroll
                for (int g = 0; g < kGenHeads; ++g) {
                    if (g < gc) {
                        const float p = sc[g][t];
                        acc[g].x += p * vv.x;
                        acc[g].y += p * vv.y;
                        acc[g].z += p * vv.z;
                        acc[g].w += p * vv.w;
                    }
                }
            }
        }
        const size_t slot0 = (((size_t)b * rm.hkv + kv) * cmax + c) * group + g0;
#pragma unroll
        for (int g = 0; g < kGenHeads; ++g) {
            if (g >= gc) break;
            red[tid] = acc[g];
            __syncthreads();
            if (my_tg == 0 && my_dc < dc) {
                float4 s = red[my_dc];
                for (int j = 1; j < tg_n; ++j) {
                    const float4 o = red[j * dcp + my_dc];
                    s.x += o.x; s.y += o.y; s.z += o.z; s.w += o.w;
                }
                *reinterpret_cast<float4*>(ws_acc + (slot0 + g) * dim + 4 * my_dc) = s;
            }
            __syncthreads();
        }
        if (tid < gc) {
            ws_ml[(slot0 + tid) * 2] = ms[tid];
            ws_ml[(slot0 + tid) * 2 + 1] = ls[tid];
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// MFMA decode kernel (bf16 / fp16 storage, D == 128, G <= 16)
//
// Work split ("stream" split-K). All (sequence b, kv head) token rows are
// laid end to end, b-major then kv: row (b, kv) owns the flat positions
// [Hkv*pref[b] + kv*len_b, + len_b) with pref the exclusive prefix of the
// lengths. The G workgroups of the grid each take one equal contiguous
// segment of that flat range (at least min_seg tokens), so every
// workgroup streams the same number of K/V bytes whatever the length mix,
// and the per-workgroup set-up is paid once per segment, not per chunk. A
// segment crossing row ends is processed as consecutive pieces, one per row
// it touches. A piece that is a whole row is normalised and stored here;
// any other piece writes its f32 (m, l, acc[D]) partial per head to slot
// (segment + row) - unique, since pieces are ordered in both indices - and
// attn_combine_stream folds a row's pieces after the kernel boundary.
// (Folding in the last-arriving workgroup instead needs a device-scope
// release/acquire per workgroup - an L2 writeback + invalidate on gfx950 -
// which costs far more than the second launch.)
//
// Inside a piece, the 4 waves walk 32-token steps st = wave, wave+4, ...
// with their own online-softmax state, merged in LDS at the piece end. With
// r = lane % 16 and g = lane / 16 (lane layout of v_mfma_f32_16x16x32:
// A[r][8g+i], B[8g+i][r], C[4g+i][r]):
//
//  scores   S^T[tok][head] = K[tok][:] . Q[head][:]  (4 MFMAs per 16 tokens)
//           A = K rows: lane loads K[tok r][32j+8g .. +7], one 16-byte load
//           B = Q^T   : lane holds Q[head r][32j+8g .. +7] (preloaded)
//           C         : lane gets S for tokens 4g+i (tile 0) and 16+4g+i
//                       (tile 1) of head r, i.e. tau(g,i) for i = 0..7 with
//                       tau(g,i) = i < 4 ? 4g+i : 16+4g+(i-4).
//  softmax  per lane for head r over its 8 tokens; the step max is folded
//           across the 4 lanes {r, r+16, r+32, r+48} (2 xor shuffles).
//  V^T      C' = V_tile . Sel_e, Sel_e[k][c] = (k == c + 16e), gives lane
//           (r,g) the values V[16h+4g+i][16n+r], n = 2j+e: the A operand of
//           the PV product below, in the same tau order. Selecting with 1.0
//           and adding zeros is exact, so the transpose is lossless.
//  PV       O^T[dim][head] += V^T[dim][tau] . P^T[tau][head]
//           A = V^T (above), B = P (the 8 probabilities the lane already
//           holds), C: lane holds O[head r][16n+4g+i]: every accumulator of a
//           lane belongs to head r, so the online rescale is per lane.
//           bf16 P is split into hi + lo parts (two MFMAs) so the weights
//           carry ~16 mantissa bits; fp16 P carries 11.
//
// Memory pipeline, per wave: K/V of two steps live in registers (buffers
// A, B); step st+4's 16 loads are issued before step st is computed. The
// block-table entries a step needs (one per lane per 16-token tile) are
// loaded two steps ahead of its K/V loads, so with the in-order load
// counter a K/V load never waits on a table entry issued after the K/V of
// the step being computed. Prefetches past the piece end are clamped to its
// last step (a real row), which keeps the load count per iteration fixed
// and the compiler's wait counts exact; tokens past the end are masked.
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mfma;
template <> struct Mfma<bf16> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    static constexpr bool kSplitP = true;
    __device__ __forceinline__ static f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<f16> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    static constexpr bool kSplitP = false;
    __device__ __forceinline__ static f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

constexpr int kMfmaDim = 128;
constexpr int kMfmaAccPitch = kMfmaDim + 4;  // LDS row pitch (bank spread)
constexpr int kStreamScanRows = 2048;        // sequences per launch (LDS prefix)
// Default minimum tokens per segment. Large decode batches are unaffected
// (C3's segments hold ~8.9k tokens); for a small one the floor trades
// per-segment set-up and combine work against idle CUs: 1 x 32 rows x 4096
// tokens (fp16, HIP-graph replays) takes 24.6 us at 1024 (128 segments),
// 20.0 us at 512, 21.3 us at 256.
constexpr int kStreamMinSeg = 512;

// Rows of equal length, each at least this long, take one segment per CU
// instead of two when the host launched the default two per CU (the
// launch's second half then returns at once). Measured on one box, two
// rounds each, one against two per CU: config 4's layer (64 rows of 8193
// tokens) 431.8-432.2 against 438.8-439.8 us, config 5b (8 x 8 rows of
// 131072) 646.1-646.5 against 659.9 us; config 3's ragged rows keep two
// per CU (0.390 against 0.401-0.403 ms per step with one).
constexpr int kStreamUniformLong = 4096;

// Row addressing modes of attn_decode_stream.
enum RowMode { kRowsContig = 0, kRowsPagedPow2 = 1, kRowsPagedDiv = 2 };

// Exclusive prefix of the clamped lengths into s_pref[0..batch] (wave 0;
// each lane takes a contiguous run of rows, then a wave scan of the runs),
// and their minimum and maximum into s_mm[0], s_mm[1].
__device__ __forceinline__ void scan_lengths(const int* __restrict__ lens,
                                             int batch, int span, int lane,
                                             long long* s_pref, int* s_mm) {
    const int per = (batch + 63) / 64;
    const int r0 = lane * per;
    long long local = 0;
    int lmin = INT_MAX, lmax = 0;
    for (int i = 0; i < per; ++i)
        if (r0 + i < batch) {
            const int l = clamp_len(lens, r0 + i, span);
            local += l;
            lmin = min(lmin, l);
            lmax = max(lmax, l);
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        lmin = min(lmin, __shfl_xor(lmin, o, 64));
        lmax = max(lmax, __shfl_xor(lmax, o, 64));
    }
    if (lane == 0) {
        s_mm[0] = lmin;
        s_mm[1] = lmax;
    }
    long long incl = local;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const long long y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    long long run = incl - local;
    for (int i = 0; i < per; ++i)
        if (r0 + i < batch) {
            s_pref[r0 + i] = run;
            run += clamp_len(lens, r0 + i, span);
        }
    if (lane == 63) s_pref[batch] = incl;
}

// A value every lane holds identically, moved to scalar registers (the
// compiler cannot prove that values read from LDS are wave-uniform).
__device__ __forceinline__ long long uniform64(long long x) {
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)x);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)((unsigned long long)x >> 32));
    return (long long)(((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ long long stream_seg_len(long long total, int nseg, int min_seg) {
    const long long s = (total + nseg - 1) / nseg;
    return s < min_seg ? (long long)min_seg : s;
}

// The fresh token of the appending decode: ap.k_new / ap.v_new [batch, hkv,
// D], written at position lens[b] of row (b, kv) in the pools ap.k_pool /
// ap.v_pool (the K / V the decode kernel reads, as writable pointers) when
// 0 <= lens[b] < span, and attended with the row's lens[b] cached tokens.
template <typename T>
struct AppendArgs {
    const T* k_new = nullptr;
    const T* v_new = nullptr;
    T* k_pool = nullptr;
    T* v_pool = nullptr;
};

// Element offset of row (b, kv)'s cache position t in a pool.
template <int MODE>
__device__ __forceinline__ size_t kv_row_offset(const int* table, int b, int kv, int t, int hkv,
                                                int rows_or_page, int page_shift,
                                                int tbl_width) {
    constexpr int D = kMfmaDim;
    if constexpr (MODE == kRowsContig) {
        return ((size_t)(b * hkv + kv) * rows_or_page + t) * D;
    } else {
        const int pg = MODE == kRowsPagedPow2 ? (t >> page_shift) : (t / rows_or_page);
        const int in_pg = MODE == kRowsPagedPow2 ? (t & (rows_or_page - 1)) : (t % rows_or_page);
        const int ent = table[(size_t)b * tbl_width + pg];
        return (((size_t)ent * hkv + kv) * rows_or_page + in_pg) * D;
    }
}

// NEW (the appending decode): every piece, whole rows included, leaves its
// partial for attn_combine_append, which folds the fresh token in.
template <typename T, int MODE, bool NEW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_decode_stream(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int* __restrict__ table, const int* __restrict__ lens,
    float* __restrict__ ws_ml, float* __restrict__ ws_acc,
    long long* __restrict__ pref_out, T* __restrict__ out, int batch, int hq, int hkv,
    int group, int rows_or_page, int page_shift, int tbl_width, int span, float scale_log2,
    int min_seg, int halve) {
    using M = Mfma<T>;
    using V8 = typename M::v8;
    constexpr int D = kMfmaDim;
    constexpr bool PAGED = MODE != kRowsContig;
    __shared__ float s_acc[4][16][kMfmaAccPitch];
    __shared__ float s_m[4][16], s_l[4][16];
    __shared__ long long s_pref[kStreamScanRows + 1];
    __shared__ int s_mm[2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform in a scalar register, so the step loops branch on scalars
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;

    if (wave == 0) scan_lengths(lens, batch, span, lane, s_pref, s_mm);
    __syncthreads();
    // segments: the grid, or half of it for long rows of equal length
    int nseg = (int)gridDim.x;
    if (halve && s_mm[0] == s_mm[1] && s_mm[0] >= kStreamUniformLong) nseg = (nseg + 1) >> 1;
    nseg = __builtin_amdgcn_readfirstlane(nseg);
    if (blockIdx.x == 0) {  // the combine kernel's copy of the prefix and the count
        for (int i = tid; i <= batch; i += 256) pref_out[i] = s_pref[i];
        if (tid == 0) pref_out[batch + 1] = nseg;
    }
    const long long total = uniform64(s_pref[batch]) * hkv;
    const long long S = stream_seg_len(total, nseg, min_seg);
    const long long seg_lo = (long long)blockIdx.x * S;
    if (seg_lo >= total) return;
    const long long seg_hi = min(seg_lo + S, total);

    // selection operands of the transposing MFMAs
    V8 sel0, sel1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        sel0[i] = (T)((8 * g + i == r) ? 1.0f : 0.0f);
        sel1[i] = (T)((8 * g + i == r + 16) ? 1.0f : 0.0f);
    }

    long long pos = seg_lo;
    while (pos < seg_hi) {
        // ---- locate the piece: row (b, kv), tokens [t0, t0 + n) ------------
        int lo = 0, hi = batch - 1;  // last sequence starting at or before pos
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (uniform64(s_pref[mid]) * hkv <= pos) lo = mid; else hi = mid - 1;
        }
        const int b = lo;
        const long long pb = uniform64(s_pref[b]);
        const long long base = pb * hkv;
        const int len = (int)(uniform64(s_pref[b + 1]) - pb);
        const int kv = (int)((pos - base) / len);
        const int t0 = (int)(pos - base - (long long)kv * len);
        const long long row_end = base + (long long)(kv + 1) * len;
        const long long piece_hi = min(seg_hi, row_end);
        const int n = (int)(piece_hi - pos);
        const bool whole = (t0 == 0 && n == len);
        const int row = b * hkv + kv;
        const int* trow = PAGED ? table + (size_t)b * tbl_width : nullptr;
        // B operand of the score MFMAs: Q[head r][32j + 8g .. +7]
        V8 qb[4];
        {
            const bool ok = r < group;
            const T* qrow = q + ((size_t)b * hq + (size_t)kv * group + (ok ? r : 0)) * D;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                V8 z = {};
                qb[j] = ok ? *reinterpret_cast<const V8*>(qrow + 32 * j + 8 * g) : z;
            }
        }

        f32x4 acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        float m_run = -INFINITY, l_run = 0.0f;

        // token (within the row) that lane row r of tile h of step st reads
        auto tok_of = [&](int st, int h) {
            return t0 + min((st << 5) + 16 * h + r, n - 1);
        };
        auto tbl_load = [&](int st, int (&e)[2]) {
            if constexpr (PAGED) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int t = tok_of(st, h);
                    e[h] = trow[MODE == kRowsPagedPow2 ? (t >> page_shift)
                                                        : (t / rows_or_page)];
                }
            }
        };
        // Load p (0..3) of tile h reads 4 whole rows, tile rows 4p ..
        // 4p + 3: lane l takes 16-byte chunk l % 16 of tile row 4p + l / 16,
        // whose table entry is held by lane 4p + l / 16. Whole 128-byte lines
        // per instruction, non-temporal: the pages are read once per launch
        // (a read of C3's pages in this pattern runs at 6.7 TB/s, against
        // 5.6 TB/s for half lines per instruction, non-temporal, and 5.1 TB/s
        // for plain loads either way).
        auto kv_load = [&](int st, const int (&e)[2], V8 (&kt)[2][4], V8 (&vt)[2][4]) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int rho = 4 * p + (lane >> 4);
                    const int t = t0 + min((st << 5) + 16 * h + rho, n - 1);
                    size_t off;
                    if constexpr (MODE == kRowsContig) {
                        off = ((size_t)row * rows_or_page + t) * D;
                    } else {
                        const int ent = __shfl(e[h], rho, 64);
                        const int in_pg = MODE == kRowsPagedPow2 ? (t & (rows_or_page - 1))
                                                                 : (t % rows_or_page);
                        off = (((size_t)ent * hkv + kv) * rows_or_page + in_pg) * D;
                    }
                    off += 8 * (lane & 15);
                    kt[h][p] = __builtin_nontemporal_load(reinterpret_cast<const V8*>(k + off));
                    vt[h][p] = __builtin_nontemporal_load(reinterpret_cast<const V8*>(v + off));
                }
            }
        };
        // Staging: the wave's 32 rows x 256 B of K (then V) in its own
        // s_acc slot (8448 B, written as s_acc only after the wave's last
        // step). Chunk c of row w sits at 16 (c ^ (w & 15)): the 16 lanes of
        // a write (one row) and of a fragment read (16 rows, one chunk) hit
        // 16 different 16-byte bank groups.
        char* const stg = reinterpret_cast<char*>(&s_acc[wave][0][0]);
        auto stage_write = [&](const V8 (&x)[2][4]) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int w = 16 * h + 4 * p + (lane >> 4);
                    *reinterpret_cast<V8*>(stg + w * 256 + 16 * ((lane & 15) ^ (w & 15))) = x[h][p];
                }
        };
        auto stage_read = [&](V8 (&f)[2][4]) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int w = 16 * h + r;
                    f[h][j] = *reinterpret_cast<const V8*>(stg + w * 256 + 16 * ((4 * j + g) ^ r));
                }
        };
        auto compute_step = [&](int st, const V8 (&kin)[2][4], const V8 (&vin)[2][4]) {
            const int tb = st << 5;
            // K through the staging, then V written behind K's fragment
            // reads, so V's load registers are free during the softmax. The
            // lanes exchange data through the staging: the hardware runs one
            // wave's LDS operations in issue order, and wave_lds_order()
            // keeps the compiler from moving a lane's LDS access across
            // the point where another lane's must have happened (the
            // previous step's V reads come before this step's K writes).
            V8 kt[2][4], vt[2][4];
            wave_lds_order();
            stage_write(kin);
            wave_lds_order();
            stage_read(kt);
            wave_lds_order();
            stage_write(vin);
            f32x4 s[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) s[h] = M::mma(kt[h][j], qb[j], s[h]);
            }
            float sv[8];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tok = tb + 16 * h + 4 * g + i;
                    sv[4 * h + i] = tok < n ? s[h][i] * scale_log2 : -INFINITY;
                }
            float mloc = sv[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) mloc = fmaxf(mloc, sv[i]);
            mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
            const float m_new = fmaxf(m_run, mloc);
            const float alpha = exp2f(m_run - m_new);
            m_run = m_new;
            float p[8];
            float psum = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                p[i] = exp2f(sv[i] - m_new);
                psum += p[i];
            }
            l_run = l_run * alpha + psum;
#pragma unroll
            for (int nn = 0; nn < 8; ++nn) acc[nn] *= alpha;
            V8 pb, pl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                pb[i] = (T)p[i];
                if (M::kSplitP) pl[i] = (T)(p[i] - (float)pb[i]);
            }
            wave_lds_order();
            stage_read(vt);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    const f32x4 a0 = M::mma(vt[0][j], e ? sel1 : sel0, z);
                    const f32x4 a1 = M::mma(vt[1][j], e ? sel1 : sel0, z);
                    V8 va;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        va[i] = (T)a0[i];
                        va[4 + i] = (T)a1[i];
                    }
                    acc[2 * j + e] = M::mma(va, pb, acc[2 * j + e]);
                    if (M::kSplitP) acc[2 * j + e] = M::mma(va, pl, acc[2 * j + e]);
                }
            }
        };

        // ---- stream the piece: two steps per iteration (buffers A, B) ------
        const int nsteps = (n + 31) >> 5;
        const int last = nsteps - 1;
        int st = wave;
        if (st < nsteps) {
            V8 ka[2][4], va_[2][4], kb[2][4], vb[2][4];
            int ea[2] = {0, 0}, eb[2] = {0, 0};
            tbl_load(st, ea);
            tbl_load(min(st + 4, last), eb);
            kv_load(st, ea, ka, va_);
            for (; st + 4 < nsteps; st += 8) {
                tbl_load(min(st + 8, last), ea);
                kv_load(st + 4, eb, kb, vb);
                // keep the prefetch ahead of the compute that follows it (the
                // scheduler would otherwise sink the loads below the waits)
                __builtin_amdgcn_sched_barrier(0);
                compute_step(st, ka, va_);
                tbl_load(min(st + 12, last), eb);
                kv_load(min(st + 8, last), ea, ka, va_);
                __builtin_amdgcn_sched_barrier(0);
                compute_step(st + 4, kb, vb);
            }
            if (st < nsteps) compute_step(st, ka, va_);
        }

        // ---- merge the 4 waves, then store the row or the piece's partial --
        l_run += __shfl_xor(l_run, 16, 64);
        l_run += __shfl_xor(l_run, 32, 64);
        if (lane < 16) {
            s_m[wave][lane] = m_run;
            s_l[wave][lane] = l_run;
        }
#pragma unroll
        for (int nn = 0; nn < 8; ++nn)
#pragma unroll
            for (int i = 0; i < 4; ++i) s_acc[wave][r][16 * nn + 4 * g + i] = acc[nn][i];
        __syncthreads();

        const int nvec = group * (D / 4);
        const size_t slot0 = ((size_t)blockIdx.x + row) * group;
        T* const orow = out + ((size_t)b * hq + (size_t)kv * group) * D;
        for (int idx = tid; idx < nvec; idx += 256) {
            const int hh = idx / (D / 4);
            const int d4 = idx - hh * (D / 4);
            float mx = -INFINITY;
#pragma unroll
            for (int w = 0; w < 4; ++w) mx = fmaxf(mx, s_m[w][hh]);
            float lsum = 0.0f;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float wt = exp2f(s_m[w][hh] - mx);
                lsum += s_l[w][hh] * wt;
                const float4 a = *reinterpret_cast<const float4*>(&s_acc[w][hh][4 * d4]);
                o.x += wt * a.x; o.y += wt * a.y; o.z += wt * a.z; o.w += wt * a.w;
            }
            if (whole && !NEW) {
                const float inv = 1.0f / lsum;
                St<T>::st4(orow + (size_t)hh * D + 4 * d4,
                           make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv));
            } else {
                *reinterpret_cast<float4*>(ws_acc + (slot0 + hh) * D + 4 * d4) = o;
                if (d4 == 0) {
                    ws_ml[(slot0 + hh) * 2] = mx;
                    ws_ml[(slot0 + hh) * 2 + 1] = lsum;
                }
            }
        }
        __syncthreads();  // LDS is reused by the next piece
        pos = piece_hi;
    }
}

// ---------------------------------------------------------------------------
// combine for attn_decode_stream, one wave per (b, q head). Row (b, kv)
// spans segments [s_lo, s_hi] of length S; its pieces' partials sit at
// slots s + row. A row inside one segment was stored by the decode kernel;
// a row of length 0 is zero-filled here (reference attention.cu:1349-1350).
// Lanes split into 2 groups of 32 (one float4 column of D = 128 each) that
// walk alternate pieces; the groups are summed with one xor shuffle.
// Returns the head's stored output (as T, widened to f32), columns
// 4 (lane & 31) .. + 3, in every lane.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float4 combine_head(const float* __restrict__ ws_ml,
                                               const float* __restrict__ ws_acc,
                                               const long long* __restrict__ pref,
                                               T* __restrict__ out, int bh, int batch, int hq,
                                               int hkv, int group, int min_seg, int lane,
                                               bool skip_empty = false) {
    constexpr int D = kMfmaDim;
    const int b = bh / hq;
    const int h = bh - b * hq;
    const int kv = h / group, gi = h - kv * group;
    T* o = out + (size_t)bh * D;
    const int len = (int)(pref[b + 1] - pref[b]);
    const int d4 = lane & 31;
    if (len == 0) {  // (skip_empty: written by the decode kernel)
        if (!skip_empty && lane < D / 4)
            St<T>::st4(o + 4 * lane, make_float4(0.f, 0.f, 0.f, 0.f));
        return make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // the decode kernel's segment count, after the prefix
    const long long S = stream_seg_len(pref[batch] * hkv, (int)pref[batch + 1], min_seg);
    const long long start = pref[b] * hkv + (long long)kv * len;
    const int s_lo = (int)(start / S), s_hi = (int)((start + len - 1) / S);
    // stored whole by the decode kernel: its stored values, read back here
    // (a maximum computed in the decode kernel's store phase slowed that
    // kernel's main loop: batch 64, context 8192, attention + quantize 357.4
    // against 348.1 us here)
    if (s_lo == s_hi) return St<T>::ld4(o + 4 * d4);
    const int row = b * hkv + kv;
    const int np = s_hi - s_lo + 1;
    auto slot = [&](int i) { return ((size_t)s_lo + i + row) * group + gi; };
    float mx = -INFINITY;
    for (int i = lane; i < np; i += 64) mx = fmaxf(mx, ws_ml[slot(i) * 2]);
    mx = wave_max(mx);
    float lsum = 0.0f;
    for (int i = lane; i < np; i += 64)
        lsum += ws_ml[slot(i) * 2 + 1] * exp2f(ws_ml[slot(i) * 2] - mx);
    lsum = wave_sum(lsum);
    const int grp = lane >> 5;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int i = grp; i < np; i += 2) {
        const size_t sl = slot(i);
        const float wt = exp2f(ws_ml[sl * 2] - mx);
        const float4 x = *reinterpret_cast<const float4*>(ws_acc + sl * D + 4 * d4);
        a.x += wt * x.x; a.y += wt * x.y; a.z += wt * x.z; a.w += wt * x.w;
    }
    a.x += __shfl_xor(a.x, 32, 64);
    a.y += __shfl_xor(a.y, 32, 64);
    a.z += __shfl_xor(a.z, 32, 64);
    a.w += __shfl_xor(a.w, 32, 64);
    const float inv = 1.0f / lsum;
    const float4 ov = make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
    if (grp == 0) St<T>::st4(o + 4 * d4, ov);
    return make_float4((float)(T)ov.x, (float)(T)ov.y, (float)(T)ov.z, (float)(T)ov.w);
}

// max |v| over a head's 128 stored values (lanes 0-31 hold them all, and
// lanes 32-63 the same again), in every lane
__device__ __forceinline__ float head_absmax(float4 v) {
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int o2 = 16; o2 > 0; o2 >>= 1) m = fmaxf(m, __shfl_xor(m, o2, 64));
    return m;
}

// AMAX: the max |stored output| of each head into amax[b * hq + h], which
// the per-tensor quantize of the output folds. skip_empty: rows of length 0
// were written by the decode kernel (its append form).
template <typename T, bool AMAX>
__global__ __launch_bounds__(64) void attn_combine_stream(
    const float* __restrict__ ws_ml, const float* __restrict__ ws_acc,
    const long long* __restrict__ pref, T* __restrict__ out, float* __restrict__ amax,
    int batch, int hq, int hkv, int group, int min_seg, int skip_empty) {
    const float4 v = combine_head<T>(ws_ml, ws_acc, pref, out, blockIdx.x, batch, hq, hkv,
                                     group, min_seg, threadIdx.x, skip_empty != 0);
    if constexpr (AMAX) {
        const float m = head_absmax(v);
        if (threadIdx.x == 0) amax[blockIdx.x] = m;
    }
}

// Combine of the appending decode (attention_append_run), one wave per
// (b, q head). Every piece of row (b, kv) was left as a partial (whole rows
// too); the fresh token - score q . k_new, value v_new - is folded in with
// them by the log-sum-exp rule, in float32, and the wave of the group's
// first q head writes k_new / v_new to position lens[b] of the pools (the
// decode kernel has finished reading them). A row with no cached token gets
// v_new alone (softmax weight 1: exactly v_new), or zeros when lens[b] has
// no room in the row or is negative (kv_append_paged then writes nothing).
template <typename T, int MODE>
__global__ __launch_bounds__(64) void attn_combine_append(
    const float* __restrict__ ws_ml, const float* __restrict__ ws_acc,
    const long long* __restrict__ pref, const int* __restrict__ lens, const T* __restrict__ q,
    AppendArgs<T> ap, const int* __restrict__ table, T* __restrict__ out, int batch, int hq,
    int hkv, int group, int min_seg, int span, int rows_or_page, int page_shift,
    int tbl_width, float scale_log2) {
    constexpr int D = kMfmaDim;
    const int bh = blockIdx.x, lane = threadIdx.x;
    const int b = bh / hq, h = bh - b * hq;
    const int kv = h / group, gi = h - kv * group;
    const int d4 = lane & 31;
    T* o = out + (size_t)bh * D;
    const int len = (int)(pref[b + 1] - pref[b]);
    const int raw = lens[b];
    const bool fresh = raw >= 0 && raw < span;  // then raw == len
    // the fresh token: lane d4 takes dims 4 d4 .. + 3 (lanes 32-63 again)
    float sv = -INFINITY;
    float4 vn = make_float4(0.f, 0.f, 0.f, 0.f);
    if (fresh) {
        const size_t nrow = ((size_t)b * hkv + kv) * D + 4 * d4;
        const float4 qq = St<T>::ld4(q + (size_t)bh * D + 4 * d4);
        const float4 kk = St<T>::ld4(ap.k_new + nrow);
        vn = St<T>::ld4(ap.v_new + nrow);
        float dot = qq.x * kk.x;
        dot = fmaf(qq.y, kk.y, dot);
        dot = fmaf(qq.z, kk.z, dot);
        dot = fmaf(qq.w, kk.w, dot);
#pragma unroll
        for (int o2 = 16; o2 > 0; o2 >>= 1) dot += __shfl_xor(dot, o2, 64);
        sv = dot * scale_log2;
        if (gi == 0 && lane < 32) {
            const size_t dst = kv_row_offset<MODE>(table, b, kv, raw, hkv, rows_or_page,
                                                   page_shift, tbl_width) + 4 * d4;
            St<T>::st4(ap.k_pool + dst, kk);
            St<T>::st4(ap.v_pool + dst, vn);
        }
    }
    int s_lo = 0, np = 0;
    if (len > 0) {
        const long long S = stream_seg_len(pref[batch] * hkv, (int)pref[batch + 1], min_seg);
        const long long start = pref[b] * hkv + (long long)kv * len;
        s_lo = (int)(start / S);
        np = (int)((start + len - 1) / S) - s_lo + 1;
    }
    const int row = b * hkv + kv;
    auto slot = [&](int i) { return ((size_t)s_lo + i + row) * group + gi; };
    float mx = sv;
    for (int i = lane; i < np; i += 64) mx = fmaxf(mx, ws_ml[slot(i) * 2]);
    mx = wave_max(mx);
    if (mx == -INFINITY) {  // no token at all
        if (lane < D / 4) St<T>::st4(o + 4 * lane, make_float4(0.f, 0.f, 0.f, 0.f));
        return;
    }
    float lsum = 0.0f;
    for (int i = lane; i < np; i += 64)
        lsum += ws_ml[slot(i) * 2 + 1] * exp2f(ws_ml[slot(i) * 2] - mx);
    lsum = wave_sum(lsum);
    const float pn = fresh ? exp2f(sv - mx) : 0.0f;
    lsum += pn;
    const int grp = lane >> 5;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int i = grp; i < np; i += 2) {
        const size_t sl = slot(i);
        const float wt = exp2f(ws_ml[sl * 2] - mx);
        const float4 x = *reinterpret_cast<const float4*>(ws_acc + sl * D + 4 * d4);
        a.x += wt * x.x; a.y += wt * x.y; a.z += wt * x.z; a.w += wt * x.w;
    }
    a.x += __shfl_xor(a.x, 32, 64);
    a.y += __shfl_xor(a.y, 32, 64);
    a.z += __shfl_xor(a.z, 32, 64);
    a.w += __shfl_xor(a.w, 32, 64);
    a.x += pn * vn.x; a.y += pn * vn.y; a.z += pn * vn.z; a.w += pn * vn.w;
    const float inv = 1.0f / lsum;
    if (grp == 0) St<T>::st4(o + 4 * d4, make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv));
}

// The combine and the per-tensor int8 quantize of the output in one launch:
// workgroups of kCqWaves waves, one (b, q head) per wave, every workgroup
// resident at once. The heads' maxima are folded with grid_max; then each
// wave writes its head's codes from the stored values it holds, and
// workgroup 0 the scale: quantize_int8's codes and scale (scale = max / 127,
// codes rint(v * (1 / scale)) clamped to +-127, quantize.cu:169-186).
// 16 waves per workgroup: config 4's 2048 heads take 128 workgroups, so
// 128 arrivals meet in grid_max (layer 432.5-432.9 us against 433.6-433.7
// with 8 waves and 437.0-437.2 with 4, same box).
constexpr int kCqWaves = 16;

template <typename T>
__global__ __launch_bounds__(64 * kCqWaves) void attn_combine_quant(
    const float* __restrict__ ws_ml, const float* __restrict__ ws_acc,
    const long long* __restrict__ pref, T* __restrict__ out, signed char* __restrict__ q,
    float* __restrict__ scale_out, int batch, int hq, int hkv, int group, int min_seg,
    GridMax gm) {
    __shared__ float red[kCqWaves];
    constexpr int D = kMfmaDim;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int bh = blockIdx.x * kCqWaves + wave;
    const bool live = bh < batch * hq;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live)
        v = combine_head<T>(ws_ml, ws_acc, pref, out, bh, batch, hq, hkv, group, min_seg, lane);
    float m = block_max<64 * kCqWaves>(live ? head_absmax(v) : 0.0f, red);
    m = grid_max<64 * kCqWaves>(gm, m, red);
    const float scale = make_scale(m);
    const float inv_s = 1.0f / scale;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
    if (live && lane < D / 4) {
        char4 c;
        c.x = quant1(v.x, inv_s);
        c.y = quant1(v.y, inv_s);
        c.z = quant1(v.z, inv_s);
        c.w = quant1(v.w, inv_s);
        *reinterpret_cast<char4*>(q + (size_t)bh * D + 4 * lane) = c;
    }
}

// ---------------------------------------------------------------------------
// combine: one wave per (b, q head). Folds the live chunks' partials (m in
// log2 units) with the log-sum-exp rule and divides by l. The wave's lanes
// are split into groups of L = min(64, pow2ceil(D/4)) lanes; each group
// walks every (64/L)-th chunk over the row's D/4 float4 columns, and the
// groups are summed with xor shuffles at the end (fixed order).
// skip_single: rows of exactly one chunk were already normalised and stored
// by the stage-1 kernel.
// ---------------------------------------------------------------------------
template <typename T, int CPL>
__global__ __launch_bounds__(64) void attn_combine(
    const float* __restrict__ ws_ml, const float* __restrict__ ws_acc,
    const int* __restrict__ lens, T* __restrict__ out, int hq, int hkv,
    int group, int dim, int span, int chunk, int cmax, int skip_single) {
    const int b = blockIdx.x / hq;
    const int h = blockIdx.x - b * hq;
    const int kv = h / group, gi = h - kv * group;
    const int lane = threadIdx.x;
    const int len = clamp_len(lens, b, span);
    const int nch = len > 0 ? (len + chunk - 1) / chunk : 0;
    const int dc = dim >> 2;
    T* o = out + ((size_t)b * hq + h) * dim;
    if (nch == 0) {
        for (int ch = lane; ch < dc; ch += 64)
            St<T>::st4(o + 4 * ch, make_float4(0.f, 0.f, 0.f, 0.f));
        return;
    }
    if (skip_single && nch == 1) return;
    const size_t s0 = ((size_t)b * hkv + kv) * cmax * group + gi;
    float mx = -INFINITY;
    for (int cc = lane; cc < nch; cc += 64)
        mx = fmaxf(mx, ws_ml[(s0 + (size_t)cc * group) * 2]);
    mx = wave_max(mx);
    float lsum = 0.0f;
    for (int cc = lane; cc < nch; cc += 64) {
        const size_t sl = s0 + (size_t)cc * group;
        lsum += ws_ml[sl * 2 + 1] * exp2f(ws_ml[sl * 2] - mx);
    }
    lsum = wave_sum(lsum);

    int L = 1;
    while (L < dc && L < 64) L <<= 1;
    const int groups = 64 / L;
    const int grp = lane / L, li = lane - grp * L;
    float4 a[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) a[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int cc = grp; cc < nch; cc += groups) {
        const size_t sl = s0 + (size_t)cc * group;
        const float wt = exp2f(ws_ml[sl * 2] - mx);
        const float* pa = ws_acc + sl * dim;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int d4 = li + i * L;
            if (d4 < dc) {
                const float4 x = *reinterpret_cast<const float4*>(pa + 4 * d4);
                a[i].x += wt * x.x; a[i].y += wt * x.y;
                a[i].z += wt * x.z; a[i].w += wt * x.w;
            }
        }
    }
    for (int off = L; off < 64; off <<= 1) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            a[i].x += __shfl_xor(a[i].x, off, 64);
            a[i].y += __shfl_xor(a[i].y, off, 64);
            a[i].z += __shfl_xor(a[i].z, off, 64);
            a[i].w += __shfl_xor(a[i].w, off, 64);
        }
    }
    if (grp != 0) return;
    const float inv = 1.0f / lsum;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int d4 = li + i * L;
        if (d4 < dc)
            St<T>::st4(o + 4 * d4, make_float4(a[i].x * inv, a[i].y * inv,
                                               a[i].z * inv, a[i].w * inv));
    }
}

template <typename T>
void launch_combine(const float* ws_ml, const float* ws_acc, const int* lens,
                    T* out, int batch, int hq, int hkv, int group, int dim,
                    int span, int chunk, int cmax, bool skip_single,
                    hipStream_t s) {
    const unsigned grid = (unsigned)((long long)batch * hq);
    if (dim / 4 <= 64)
        attn_combine<T, 1><<<grid, 64, 0, s>>>(ws_ml, ws_acc, lens, out, hq, hkv,
                                               group, dim, span, chunk, cmax,
                                               skip_single ? 1 : 0);
    else
        attn_combine<T, 2><<<grid, 64, 0, s>>>(ws_ml, ws_acc, lens, out, hq, hkv,
                                               group, dim, span, chunk, cmax,
                                               skip_single ? 1 : 0);
    launch_check("attention combine kernel launch");
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
template <typename T>
bool mfma_eligible(const T* q, const T* k, const T* v, int group, int dim) {
    if (std::is_same<T, float>::value) return false;
    if (dim != kMfmaDim || group > 16) return false;
    return ((uintptr_t)q % 16 == 0) && ((uintptr_t)k % 16 == 0) &&
           ((uintptr_t)v % 16 == 0);
}

// attn_decode_stream in the row mode of the layout (paged with a power-of-2
// page, paged with any page, contiguous).
// fresh: the appending decode's form (NEW).
template <typename T>
void launch_stream(bool paged, int page_shift, int nseg, hipStream_t s, const T* q,
                   const T* k, const T* v, const int* table, const int* lens, float* ws_ml,
                   float* ws_acc, long long* pref, T* out, int batch, int hq, int hkv,
                   int group, int rows_or_page, int tbl_width, int span, float scale_log2,
                   int min_seg, bool fresh, bool halve) {
    auto go = [&](auto kernel, const int* tbl, int shift, int width) {
        kernel<<<(unsigned)nseg, 256, 0, s>>>(q, k, v, tbl, lens, ws_ml, ws_acc, pref, out,
                                              batch, hq, hkv, group, rows_or_page, shift,
                                              width, span, scale_log2, min_seg, halve ? 1 : 0);
    };
    if (paged && page_shift >= 0) {
        if (fresh) go(attn_decode_stream<T, kRowsPagedPow2, true>, table, page_shift, tbl_width);
        else go(attn_decode_stream<T, kRowsPagedPow2, false>, table, page_shift, tbl_width);
    } else if (paged) {
        if (fresh) go(attn_decode_stream<T, kRowsPagedDiv, true>, table, -1, tbl_width);
        else go(attn_decode_stream<T, kRowsPagedDiv, false>, table, -1, tbl_width);
    } else {
        if (fresh) inval("attention: the append form is paged only");
        go(attn_decode_stream<T, kRowsContig, false>, nullptr, -1, 0);
    }
}

// Device workspace of one decode call (split partials and the length
// prefix): the library's per-device buffer, grown on demand, or a fixed
// region of `cap` bytes that the caller owns (the no-allocation entry
// point). A fixed region that is too small is an invalid argument, raised
// before anything is launched.
struct Workspace {
    void* fixed = nullptr;
    size_t cap = 0;
    // the contiguous decode's fallback (reference attention.cu:1514-1523,
    // where it runs the single-pass kernel instead): when the library's
    // buffer cannot be allocated (or grown under a capture), the partials go
    // to the static per-device array of FT_NOALLOC_WORKSPACE_BYTES; the paged
    // decode raises instead, as the reference's (attention.cu:1830-1844)
    void* (*fallback)() = nullptr;
    void* get(size_t bytes, hipStream_t s) const {
        if (!fixed) {
            try {
                return scratch(Scratch::AttnPartials, bytes, s);
            } catch (const Error& err) {
                if (!fallback || err.code != FT_EHIP || bytes > FT_NOALLOC_WORKSPACE_BYTES) throw;
                return fallback();
            }
        }
        if (bytes > cap)
            inval("attention: this call needs " + std::to_string(bytes) +
                  " bytes of split workspace; the static workspace holds " +
                  std::to_string(cap));
        return fixed;
    }
};

template <typename T>
// Returns 0, or 1 when the combine kernel wrote the per-head maxima into
// amax, or 2 when it also folded them and wrote the int8 codes of the
// output into qcodes and the scale into *qscale (quantize_int8's; the
// stream path with every combine workgroup resident at once).
int attention_run(const T* q, const T* k, const T* v, const int* table,
                   const int* lens, T* out, int batch, int hq, int hkv,
                   int rows_or_page, int tbl_width, int dim, bool paged,
                   hipStream_t s, const Workspace& wsp = Workspace{},
                   float* amax = nullptr, signed char* qcodes = nullptr,
                   float* qscale = nullptr, const AppendArgs<T>& ap = AppendArgs<T>{}) {
    long long span;
    if (paged) {
        span = (long long)tbl_width * rows_or_page;
        if (span > (1LL << 30)) inval("table capacity too large");
        attention_check(batch, hq, hkv, span, dim);
        if (rows_or_page < 1) inval("page size must be >= 1");
        if (tbl_width < 0) inval("table width must be >= 0");
        const int group = hq / hkv;
        if (!(group == 1 || group == 2 || group == 4 || group == 8 || group == 16))
            inval("paged decode supports GQA group sizes 1/2/4/8/16 "
                  "(use the contiguous op for other divisors)");
    } else {
        span = rows_or_page;
        attention_check(batch, hq, hkv, span, dim);
    }
    if (batch == 0) return 0;
    if (!q || !out || (span > 0 && (!k || !v)) || (paged && span > 0 && !table))
        inval("attention: null operand");
    const int group = hq / hkv;
    const bool fast = mfma_eligible(q, k, v, group, dim) && batch <= kStreamScanRows &&
                      tune(Tune::AttnForceGeneric, 0) == 0;
    int page_shift = -1;
    if (paged && (rows_or_page & (rows_or_page - 1)) == 0) {
        int sh = 0;
        while ((1 << sh) < rows_or_page) ++sh;
        page_shift = sh;
    }
    const float scale_log2 = (1.0f / sqrtf((float)dim)) * kLog2e;
    if constexpr (!std::is_same<T, float>::value) {
        if (fast && span > 0) {
            // stream split: G equal token segments, G = 2 workgroups per CU
            // (the kernel's register budget allows exactly two per CU); the
            // kernel takes one per CU for long rows of equal length unless
            // FT_ATTN_SEGS sets the count
            const int forced = tune(Tune::AttnSegs, 0);
            int nseg = forced > 0 ? forced : 2 * dev_info().cu_count;
            nseg = std::max(1, std::min(nseg, 1 << 20));
            const bool halve = forced <= 0;
            const int min_seg = std::max(32, tune(Tune::AttnMinSeg, kStreamMinSeg));
            const size_t nslots = ((size_t)nseg + (size_t)batch * hkv) * group;
            const size_t ml_floats = (nslots * 2 + 63) & ~(size_t)63;
            const size_t acc_floats = nslots * dim;
            char* ws = (char*)wsp.get(
                (ml_floats + acc_floats) * sizeof(float) + (batch + 2) * sizeof(long long), s);
            float* ws_ml = (float*)ws;
            float* ws_acc = ws_ml + ml_floats;
            long long* pref = (long long*)(ws_acc + acc_floats);
            if (ap.k_new && (amax || qcodes))
                inval("attention: the append form keeps no per-head maxima");
            launch_stream<T>(paged, page_shift, nseg, s, q, k, v, table, lens, ws_ml, ws_acc,
                             pref, out, batch, hq, hkv, group, rows_or_page, tbl_width,
                             (int)span, scale_log2, min_seg, ap.k_new != nullptr, halve);
            launch_check("attention decode kernel launch");
            if (ap.k_new) {
                const unsigned grid = (unsigned)((long long)batch * hq);
                if (page_shift >= 0)
                    attn_combine_append<T, kRowsPagedPow2><<<grid, 64, 0, s>>>(
                        ws_ml, ws_acc, pref, lens, q, ap, table, out, batch, hq, hkv, group,
                        min_seg, (int)span, rows_or_page, page_shift, tbl_width, scale_log2);
                else
                    attn_combine_append<T, kRowsPagedDiv><<<grid, 64, 0, s>>>(
                        ws_ml, ws_acc, pref, lens, q, ap, table, out, batch, hq, hkv, group,
                        min_seg, (int)span, rows_or_page, -1, tbl_width, scale_log2);
                launch_check("attention combine + append kernel launch");
                return 0;
            }
            if (qcodes) {
                const long long heads = (long long)batch * hq;
                const long long nwg = (heads + kCqWaves - 1) / kCqWaves;
                if (nwg <= (1 << 16)) {
                    const GridMax gm = gridmax_state((int)nwg, s);
                    if (grid_resident((const void*)attn_combine_quant<T>, (int)nwg,
                                      64 * kCqWaves, GridUse::AttnOut)) {
                        attn_combine_quant<T><<<(unsigned)nwg, 64 * kCqWaves, 0, s>>>(
                            ws_ml, ws_acc, pref, out, qcodes, qscale, batch, hq, hkv, group,
                            min_seg, gm);
                        launch_check("attention combine + quantize kernel launch");
                        return 2;
                    }
                }
            }
            if (amax)
                attn_combine_stream<T, true><<<(unsigned)((long long)batch * hq), 64, 0, s>>>(
                    ws_ml, ws_acc, pref, out, amax, batch, hq, hkv, group, min_seg, 0);
            else
                attn_combine_stream<T, false><<<(unsigned)((long long)batch * hq), 64, 0, s>>>(
                    ws_ml, ws_acc, pref, out, nullptr, batch, hq, hkv, group, min_seg, 0);
            launch_check("attention combine kernel launch");
            return amax ? 1 : 0;
        }
    }
    if (ap.k_new) inval("attention: the append form runs on the stream kernel only");
    const long long target = (long long)dev_info().cu_count * 16;
    int chunk = choose_chunk(batch, hkv, span, 64, kGenMaxChunk, target);
    const int forced = tune(Tune::AttnChunk, 0);
    if (forced > 0) chunk = std::min(forced, kGenMaxChunk);
    const int cmax = span > 0 ? (int)((span + chunk - 1) / chunk) : 1;
    const long long units = (long long)batch * hkv * cmax;
    if (units * 256 > (1LL << 31)) inval("attention problem too large for one launch");
    const size_t nslots = (size_t)units * group;
    const size_t ml_floats = (nslots * 2 + 63) & ~(size_t)63;
    float* ws = (float*)wsp.get((ml_floats + nslots * dim) * sizeof(float), s);
    float* ws_ml = ws;
    float* ws_acc = ws + ml_floats;
    RowMap rm;
    rm.table = paged ? table : nullptr;
    rm.hkv = hkv;
    rm.dim = dim;
    rm.rows_or_page = rows_or_page;
    rm.tbl_width = tbl_width;
    rm.page_shift = page_shift;
    if (span > 0) {
        if (dim / 4 <= 64)
            attn_chunk_generic<T, 1><<<(unsigned)units, kGenNT, 0, s>>>(
                q, k, v, lens, rm, ws_ml, ws_acc, hq, group, (int)span, chunk,
                cmax, scale_log2);
        else
            attn_chunk_generic<T, 2><<<(unsigned)units, kGenNT, 0, s>>>(
                q, k, v, lens, rm, ws_ml, ws_acc, hq, group, (int)span, chunk,
                cmax, scale_log2);
        launch_check("attention chunk kernel launch");
    }
    // (also the zero fill of every row when the cache holds no rows at all)
    launch_combine<T>(ws_ml, ws_acc, span > 0 ? lens : nullptr, out, batch, hq,
                      hkv, group, dim, (int)span, chunk, cmax, false, s);
    return 0;  // no per-head maxima on this path
}

// ---------------------------------------------------------------------------
// KV append: one thread per 4-element chunk of one head's row (reference
// attention.cu:1753-1782). Rows of the fresh token land at position lens[b].
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(
    const T* __restrict__ k_new, const T* __restrict__ v_new,
    const int* __restrict__ lens, RowMap rm, int capacity, int per_row,
    T* __restrict__ k_dst, T* __restrict__ v_dst) {
    const int b = blockIdx.x / per_row;
    const int dc = rm.dim >> 2;
    const int idx = (blockIdx.x - b * per_row) * 256 + threadIdx.x;
    if (idx >= rm.hkv * dc) return;
    const int h = idx / dc, ch = idx - h * dc;
    const int pos = lens[b];
    // device lengths are trusted by the API but never turned into an
    // out-of-range address: a position outside [0, capacity) writes nothing
    if (pos < 0 || pos >= capacity) return;
    const size_t dst = rm(b, h, pos) + 4 * ch;
    const size_t src = ((size_t)b * rm.hkv + h) * rm.dim + 4 * ch;
    if (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(k_dst + dst) = *reinterpret_cast<const float4*>(k_new + src);
        *reinterpret_cast<float4*>(v_dst + dst) = *reinterpret_cast<const float4*>(v_new + src);
    } else {
        *reinterpret_cast<uint2*>(k_dst + dst) = *reinterpret_cast<const uint2*>(k_new + src);
        *reinterpret_cast<uint2*>(v_dst + dst) = *reinterpret_cast<const uint2*>(v_new + src);
    }
}

template <typename T>
void kv_append_run(const T* k_new, const T* v_new, const int* table,
                   const int* lens, T* k_dst, T* v_dst, int batch, int hkv,
                   int dim, int rows_or_page, int tbl_width, bool paged,
                   hipStream_t s) {
    if (batch <= 0) return;  // nothing to append (reference attention.cu:1930-1931)
    if (dim % 4 != 0) inval("dim must be a multiple of 4");
    if (paged && rows_or_page < 1) inval("page size must be >= 1");
    if (hkv < 1 || dim < 1 || dim > kMaxDim) inval("kv heads >= 1 and 1 <= dim <= 512 required");
    if (rows_or_page < 0 || tbl_width < 0) inval("cache rows / table width must be >= 0");
    if (!k_new || !v_new || !lens || !k_dst || !v_dst || (paged && !table))
        inval("kv append: null operand");
    RowMap rm;
    rm.table = paged ? table : nullptr;
    rm.hkv = hkv;
    rm.dim = dim;
    rm.rows_or_page = rows_or_page;
    rm.tbl_width = tbl_width;
    rm.page_shift = -1;
    if (paged && (rows_or_page & (rows_or_page - 1)) == 0) {
        int sh = 0;
        while ((1 << sh) < rows_or_page) ++sh;
        rm.page_shift = sh;
    }
    const long long cap = paged ? (long long)tbl_width * rows_or_page
                                : (long long)rows_or_page;
    if (cap > (1LL << 30)) inval("cache capacity too large");
    if (cap == 0) return;  // no row can hold the token
    const int chunks = hkv * (dim / 4);
    const int per_row = (chunks + 255) / 256;
    if ((long long)batch * per_row > (1LL << 31) - 1) inval("kv append: batch too large");
    kv_append_kernel<T><<<(unsigned)(batch * per_row), 256, 0, s>>>(
        k_new, v_new, lens, rm, (int)cap, per_row, k_dst, v_dst);
    launch_check("kv append kernel launch");
}

__global__ __launch_bounds__(256) void lens_plus1_kernel(const int* __restrict__ lens,
                                                         int* __restrict__ out, int batch) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < batch) out[i] = lens[i] == INT_MAX ? INT_MAX : lens[i] + 1;
}

// kv_append_paged(k_pool, v_pool, table, k_new, v_new, lens) followed by
// attention_decode_paged(q, k_pool, v_pool, table, lens + 1), in one call.
// On the stream path (bf16 / fp16, D = 128) the decode
// kernel attends the lens[b] cached tokens (every piece leaves a partial)
// and attn_combine_append folds the fresh token from k_new / v_new into
// each row's log-sum-exp merge (float32) and writes it to the pools - one
// launch fewer. Elsewhere: the two ops, lens + 1 through library scratch.
template <typename T>
void attention_append_run(const T* q, T* k_pool, T* v_pool, const int* table, const T* k_new,
                          const T* v_new, const int* lens, T* out, int batch, int hq, int hkv,
                          int page, int tbl_width, int dim, hipStream_t s) {
    if (batch < 0) inval("batch must be >= 0");
    if (batch == 0) return;
    if (!lens || !k_new || !v_new) inval("attention append: null operand");
    const long long span = (long long)tbl_width * page;
    const int group = hkv > 0 ? hq / hkv : 0;
    const bool fast = !std::is_same<T, float>::value && hkv > 0 && hq % hkv == 0 &&
                      mfma_eligible(q, k_pool, v_pool, group, dim) &&
                      (uintptr_t)k_new % 16 == 0 && (uintptr_t)v_new % 16 == 0 &&
                      batch <= kStreamScanRows && tune(Tune::AttnForceGeneric, 0) == 0 &&
                      span > 0 && page >= 1 && tbl_width >= 0;
    if (fast) {
        AppendArgs<T> ap;
        ap.k_new = k_new;
        ap.v_new = v_new;
        ap.k_pool = k_pool;
        ap.v_pool = v_pool;
        attention_run<T>(q, k_pool, v_pool, table, lens, out, batch, hq, hkv, page, tbl_width,
                         dim, true, s, Workspace{}, nullptr, nullptr, nullptr, ap);
        return;
    }
    kv_append_run<T>(k_new, v_new, table, lens, k_pool, v_pool, batch, hkv, dim, page,
                     tbl_width, true, s);
    int* lens1 = (int*)scratch(Scratch::AttnLens, (size_t)batch * sizeof(int), s);
    lens_plus1_kernel<<<(unsigned)((batch + 255) / 256), 256, 0, s>>>(lens, lens1, batch);
    launch_check("lens + 1 kernel launch");
    attention_run<T>(q, k_pool, v_pool, table, lens1, out, batch, hq, hkv, page, tbl_width, dim,
                     true, s);
}

}  // namespace
}  // namespace ft

using ft::bf16;
using ft::f16;

namespace ft {
namespace {
// Paged decode followed by the per-tensor int8 quantize of its output. On
// the stream kernels' path the combine kernel also takes the max |stored
// output| of every (sequence, q head) (split rows from its fold, whole rows
// read back): where all its workgroups are resident at once it folds them
// (grid_max) and writes the codes and the scale itself, else it writes them
// out and the quantize is one launch over those B * Hq maxima; other paths
// quantize the output in full.
template <typename T>
void attention_paged_quant_run(const T* q, const T* k_pool, const T* v_pool, const int* table,
                               const int* lens, T* out, signed char* codes, float* scale_out,
                               int batch, int hq, int hkv, int page, int tbl_width, int dim,
                               hipStream_t s) {
    if (batch < 0 || hq < 1) inval("attention shapes must satisfy batch>=0, heads>=1, rows>=0, dim>=1");
    if (batch > 0 && (!codes || !scale_out)) inval("attention quantize: null operand");
    const long long rows = (long long)batch * hq;
    float* amax = rows > 0 ? (float*)scratch(Scratch::QuantMax, (size_t)rows * sizeof(float), s)
                           : nullptr;
    const int have = attention_run<T>(q, k_pool, v_pool, table, lens, out, batch, hq, hkv,
                                      page, tbl_width, dim, true, s, Workspace{}, amax, codes,
                                      scale_out);
    if (batch == 0 || have == 2) return;
    const long long n = rows * dim;
    if (have == 1)
        quantize_from_partials<T>(out, codes, amax, (int)rows, scale_out, n, s);
    else
        quantize_tensor<T>(out, codes, scale_out, n, s);
}
}  // namespace
}  // namespace ft

// ---------------------------------------------------------------------------
// Static workspace of the no-allocation entry point. Each GPU holds its own
// copy of this array for the life of the process. In host code `scratch` is
// only a host-side stand-in for the symbol, never a device address: the
// address of the current device's copy comes from hipGetSymbolAddress, once
// per device, and only that pointer is handed to kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[FT_NOALLOC_WORKSPACE_BYTES];

namespace {
constexpr int kMaxStaticDevices = 64;
std::mutex g_static_ws_mutex;
void* g_static_ws[kMaxStaticDevices];

// The current device's copy of `scratch`, looked up on the first call made
// with that device current.
void* static_workspace() {
    int dev = 0;
    ft::hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxStaticDevices)
        ft::inval("device id out of range for the static workspace");
    std::lock_guard<std::mutex> lock(g_static_ws_mutex);
    if (!g_static_ws[dev]) {
        void* p = nullptr;
        ft::hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                      "hipGetSymbolAddress(scratch)");
        g_static_ws[dev] = p;
    }
    return g_static_ws[dev];
}

// the contiguous decode's workspace: the library's buffer, or the static
// array when that cannot be allocated
ft::Workspace contiguous_workspace() {
    ft::Workspace w;
    w.fallback = &static_workspace;
    return w;
}
}  // namespace

extern "C" {

int ft_attention_decode_paged_quant_launch(const void* q, const void* k_pool,
                                           const void* v_pool, const int* table,
                                           const int* lens, void* out, int dtype,
                                           signed char* codes, float* scale_out, int batch,
                                           int q_heads, int kv_heads, int page,
                                           int tbl_width, int dim, uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
        switch (dtype) {
        case FT_DT_F32:
            ft::attention_paged_quant_run<float>((const float*)q, (const float*)k_pool,
                                                 (const float*)v_pool, table, lens, (float*)out,
                                                 codes, scale_out, batch, q_heads, kv_heads,
                                                 page, tbl_width, dim, s);
            break;
        case FT_DT_BF16:
            ft::attention_paged_quant_run<bf16>((const bf16*)q, (const bf16*)k_pool,
                                                (const bf16*)v_pool, table, lens, (bf16*)out,
                                                codes, scale_out, batch, q_heads, kv_heads,
                                                page, tbl_width, dim, s);
            break;
        case FT_DT_F16:
            ft::attention_paged_quant_run<f16>((const f16*)q, (const f16*)k_pool,
                                               (const f16*)v_pool, table, lens, (f16*)out,
                                               codes, scale_out, batch, q_heads, kv_heads,
                                               page, tbl_width, dim, s);
            break;
        default:
            ft::inval("attention quantize: unknown dtype code");
        }
    });
}

int ft_attention_decode_paged_append_launch(const void* q, void* k_pool, void* v_pool,
                                            const int* table, const void* k_new,
                                            const void* v_new, const int* lens, void* out,
                                            int dtype, int batch, int q_heads, int kv_heads,
                                            int page, int tbl_width, int dim,
                                            uintptr_t stream) {
    return ft::guarded([&] {
        hipStream_t s = ft::as_stream(stream);
        switch (dtype) {
        case FT_DT_F32:
            ft::attention_append_run<float>((const float*)q, (float*)k_pool, (float*)v_pool,
                                            table, (const float*)k_new, (const float*)v_new,
                                            lens, (float*)out, batch, q_heads, kv_heads, page,
                                            tbl_width, dim, s);
            break;
        case FT_DT_BF16:
            ft::attention_append_run<bf16>((const bf16*)q, (bf16*)k_pool, (bf16*)v_pool, table,
                                           (const bf16*)k_new, (const bf16*)v_new, lens,
                                           (bf16*)out, batch, q_heads, kv_heads, page,
                                           tbl_width, dim, s);
            break;
        case FT_DT_F16:
            ft::attention_append_run<f16>((const f16*)q, (f16*)k_pool, (f16*)v_pool, table,
                                          (const f16*)k_new, (const f16*)v_new, lens,
                                          (f16*)out, batch, q_heads, kv_heads, page, tbl_width,
                                          dim, s);
            break;
        default:
            ft::inval("attention append: unknown dtype code");
        }
    });
}

int ft_attention_decode_paged_launch_bf16_noalloc(const void* q, const void* k_pool,
                                                  const void* v_pool, const int* table,
                                                  const int* lens, void* out, int batch,
                                                  int q_heads, int kv_heads, int page,
                                                  int tbl_width, int dim,
                                                  uintptr_t stream) {
    return ft::guarded([&] {
        ft::Workspace wsp;
        wsp.fixed = static_workspace();
        wsp.cap = FT_NOALLOC_WORKSPACE_BYTES;
        ft::attention_run<bf16>((const bf16*)q, (const bf16*)k_pool, (const bf16*)v_pool,
                                table, lens, (bf16*)out, batch, q_heads, kv_heads, page,
                                tbl_width, dim, true, ft::as_stream(stream), wsp);
    });
}


int ft_attention_decode_launch(const float* q, const float* k, const float* v,
                               const int* lens, float* out, int batch,
                               int q_heads, int kv_heads, int cache_rows,
                               int dim, uintptr_t stream) {
    return ft::guarded([&] {
        ft::attention_run<float>(q, k, v, nullptr, lens, out, batch, q_heads,
                                 kv_heads, cache_rows, 0, dim, false,
                                 ft::as_stream(stream), contiguous_workspace());
    });
}

int ft_attention_decode_launch_bf16(const void* q, const void* k,
                                    const void* v, const int* lens, void* out,
                                    int batch, int q_heads, int kv_heads,
                                    int cache_rows, int dim, uintptr_t stream) {
    return ft::guarded([&] {
        ft::attention_run<bf16>((const bf16*)q, (const bf16*)k, (const bf16*)v,
                                nullptr, lens, (bf16*)out, batch, q_heads,
                                kv_heads, cache_rows, 0, dim, false,
                                ft::as_stream(stream), contiguous_workspace());
    });
}

int ft_attention_decode_launch_fp16(const void* q, const void* k,
                                    const void* v, const int* lens, void* out,
                                    int batch, int q_heads, int kv_heads,
                                    int cache_rows, int dim, uintptr_t stream) {
    return ft::guarded([&] {
        ft::attention_run<f16>((const f16*)q, (const f16*)k, (const f16*)v,
                               nullptr, lens, (f16*)out, batch, q_heads,
                               kv_heads, cache_rows, 0, dim, false,
                               ft::as_stream(stream), contiguous_workspace());
    });
}

int ft_attention_decode_paged_launch(const float* q, const float* k_pool,
                                     const float* v_pool, const int* table,
                                     const int* lens, float* out, int batch,
                                     int q_heads, int kv_heads, int page,
                                     int tbl_width, int dim, uintptr_t stream) {
    return ft::guarded([&] {
        ft::attention_run<float>(q, k_pool, v_pool, table, lens, out, batch,
                                 q_heads, kv_heads, page, tbl_width, dim, true,
                                 ft::as_stream(stream));
    });
}

int ft_attention_decode_paged_launch_bf16(const void* q, const void* k_pool,
                                          const void* v_pool, const int* table,
                                          const int* lens, void* out, int batch,
                                          int q_heads, int kv_heads, int page,
                                          int tbl_width, int dim,
                                          uintptr_t stream) {
    return ft::guarded([&] {
        ft::attention_run<bf16>((const bf16*)q, (const bf16*)k_pool,
                                (const bf16*)v_pool, table, lens, (bf16*)out,
                                batch, q_heads, kv_heads, page, tbl_width, dim,
                                true, ft::as_stream(stream));
    });
}

int ft_attention_decode_paged_launch_fp16(const void* q, const void* k_pool,
                                          const void* v_pool, const int* table,
                                          const int* lens, void* out, int batch,
                                          int q_heads, int kv_heads, int page,
                                          int tbl_width, int dim,
                                          uintptr_t stream) {
    return ft::guarded([&] {
        ft::attention_run<f16>((const f16*)q, (const f16*)k_pool,
                               (const f16*)v_pool, table, lens, (f16*)out,
                               batch, q_heads, kv_heads, page, tbl_width, dim,
                               true, ft::as_stream(stream));
    });
}

int ft_kv_append_paged_launch(const float* k_new, const float* v_new,
                              const int* table, const int* lens, float* k_pool,
                              float* v_pool, int batch, int hkv, int dim,
                              int page, int tbl_width, uintptr_t stream) {
    return ft::guarded([&] {
        ft::kv_append_run<float>(k_new, v_new, table, lens, k_pool, v_pool, batch,
                                 hkv, dim, page, tbl_width, true,
                                 ft::as_stream(stream));
    });
}

int ft_kv_append_paged_launch_bf16(const void* k_new, const void* v_new,
                                   const int* table, const int* lens,
                                   void* k_pool, void* v_pool, int batch,
                                   int hkv, int dim, int page, int tbl_width,
                                   uintptr_t stream) {
    return ft::guarded([&] {
        ft::kv_append_run<bf16>((const bf16*)k_new, (const bf16*)v_new, table,
                                lens, (bf16*)k_pool, (bf16*)v_pool, batch, hkv,
                                dim, page, tbl_width, true, ft::as_stream(stream));
    });
}

int ft_kv_append_paged_launch_fp16(const void* k_new, const void* v_new,
                                   const int* table, const int* lens,
                                   void* k_pool, void* v_pool, int batch,
                                   int hkv, int dim, int page, int tbl_width,
                                   uintptr_t stream) {
    return ft::guarded([&] {
        ft::kv_append_run<f16>((const f16*)k_new, (const f16*)v_new, table, lens,
                               (f16*)k_pool, (f16*)v_pool, batch, hkv, dim, page,
                               tbl_width, true, ft::as_stream(stream));
    });
}

int ft_kv_append_launch(const float* k_new, const float* v_new,
                        const int* lens, float* k_cache, float* v_cache,
                        int batch, int hkv, int dim, int t_rows,
                        uintptr_t stream) {
    return ft::guarded([&] {
        ft::kv_append_run<float>(k_new, v_new, nullptr, lens, k_cache, v_cache,
                                 batch, hkv, dim, t_rows, 0, false,
                                 ft::as_stream(stream));
    });
}

int ft_kv_append_launch_bf16(const void* k_new, const void* v_new,
                             const int* lens, void* k_cache, void* v_cache,
                             int batch, int hkv, int dim, int t_rows,
                             uintptr_t stream) {
    return ft::guarded([&] {
        ft::kv_append_run<bf16>((const bf16*)k_new, (const bf16*)v_new, nullptr,
                                lens, (bf16*)k_cache, (bf16*)v_cache, batch, hkv,
                                dim, t_rows, 0, false, ft::as_stream(stream));
    });
}

int ft_kv_append_launch_fp16(const void* k_new, const void* v_new,
                             const int* lens, void* k_cache, void* v_cache,
                             int batch, int hkv, int dim, int t_rows,
                             uintptr_t stream) {
    return ft::guarded([&] {
        ft::kv_append_run<f16>((const f16*)k_new, (const f16*)v_new, nullptr,
                               lens, (f16*)k_cache, (f16*)v_cache, batch, hkv,
                               dim, t_rows, 0, false, ft::as_stream(stream));
    });
}

}  // extern "C"
