// Post-logits sampling step for gfx950: argmax (greedy), nucleus sampling
// (sample_topp) and the fused decode step (repetition penalty ->
// temperature -> nucleus sampling), single row or one workgroup per row.
//
// Semantics (reference sampling.cu:103-120,466-516,1030-1081, topk.cu:5677,
// cuda_util.cuh:69-76): the value of token i is
//     v_i = l_i' * (1/T),  l_i' = (i penalised) ? (l_i > 0 ? l_i / pen : l_i * pen) : l_i
// tokens are ordered by (v desc, index asc), masses are exp(v - max); the
// nucleus is the shortest prefix of that order whose mass reaches p * total,
// and the token is where the prefix mass first reaches u * nucleus mass,
// u = splitmix_uniform(seed).
//
// Algorithm (one 1024-thread workgroup per row, or the row split across CUs
// by the sliced pipeline below when there are fewer rows than CUs; no sort
// of the vocabulary):
//   - masses are fixed point, q_i = rint(exp(v_i - max) * 2^40) in 64-bit
//     integers, so every sum is exact and order-free: the result is
//     deterministic per seed (no float atomics);
//   - one pass bins every token by its distance from the maximum in 1/64-nat
//     steps (2048 bins; the last takes everything from ~32 nats on, whose
//     mass is 0) with the bins' mass and count; bins are contiguous ranges
//     of the order, so a scan over them finds the bin where a prefix mass
//     crosses a threshold;
//   - the crossing bin's tokens are gathered into LDS (<= 4096); up to 1024
//     are resolved without sorting (an entry's prefix inside the bin is the
//     mass of the entries with a larger key), more are sorted by the exact
//     order key (value bits, then ~index) with a bitonic network and
//     scanned; a larger crossing bin (nearly flat logits) is resolved by
//     8-bit radix passes over the exact key, restricted to that bin;
//   - the nucleus cut and the draw are two such threshold queries, the
//     draw's threshold being u * (prefix mass through the cut).
// Compared with the reference CPU path (float sums in sorted order, host
// exp), the token is the same except when a threshold lands within float
// rounding of a prefix boundary - the limit the reference states for its
// own GPU path.
#include "ft_common.hpp"

#include <algorithm>
#include <cstdlib>

namespace ft {
namespace {

typedef unsigned long long u64;

constexpr int kSmpNT = 1024;
constexpr int kDistBins = 2048;
constexpr float kDistScale = 64.0f;       // bins per nat
constexpr int kGather = 4096;             // exact-sort capacity of one bin
constexpr int kMaxBitmapVocab = 1 << 19;  // penalty bitmap in LDS (64 KB)
constexpr float kFx = 1099511627776.0f;   // 2^40: fixed-point mass unit

__device__ __forceinline__ float splitmix_uniform(u64 seed) {
    u64 z = seed + 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return (float)((z >> 11) * (1.0 / 9007199254740992.0));
}

struct SampleRow {
    const float* x;
    int n;
    float inv_t;
    float pen;
    const unsigned* bits;  // penalised-token bitmap (LDS or global), or null
    int bit0;              // first token of bits[0] (a multiple of 32)
    // value of token i from its raw logit l
    __device__ __forceinline__ float val_of(int i, float l) const {
        if (bits && ((bits[(i - bit0) >> 5] >> (i & 31)) & 1u))
            l = l > 0.0f ? l / pen : l * pen;
        return l * inv_t + 0.0f;  // -0 -> +0: equal values order by index
    }
};

// Visit tokens [lo, hi) of a row (lo a multiple of 4) as f(i, v_i): 16-byte
// loads, U in flight per thread (the rows are read several times; one
// dependent 4-byte load per thread per step left each pass latency-bound).
// The order of the f calls is not fixed: every caller's result is
// independent of it (maxima, integer sums, candidates resolved by key).
template <int NT, int U = 4, typename F>
__device__ __forceinline__ void slice_scan(const SampleRow& row, int lo, int hi, F&& f) {
    const float* x = row.x;
    const int tid = threadIdx.x;
    int done = lo;
    if (((uintptr_t)(x + lo) & 15) == 0) {
        const int c0 = lo >> 2, n4 = hi >> 2;
        const float4* x4 = reinterpret_cast<const float4*>(x);
        // batches of U * NT vectors: a thread's U loads are issued together
        // (indices past the end clamped to the last vector and not used), so
        // each batch costs one memory round trip
        for (int base = c0; base < n4; base += U * NT) {
            float4 q[U];
#pragma unroll
            for (int u = 0; u < U; ++u) q[u] = x4[min(base + u * NT + tid, n4 - 1)];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = base + u * NT + tid;
                if (c < n4) {
                    const int i = 4 * c;
                    f(i, row.val_of(i, q[u].x));
                    f(i + 1, row.val_of(i + 1, q[u].y));
                    f(i + 2, row.val_of(i + 2, q[u].z));
                    f(i + 3, row.val_of(i + 3, q[u].w));
                }
            }
        }
        done = max(lo, 4 * n4);
    }
    for (int i = done + tid; i < hi; i += NT) f(i, row.val_of(i, x[i]));
}
template <int NT, typename F>
__device__ __forceinline__ void row_scan(const SampleRow& row, F&& f) {
    slice_scan<NT>(row, 0, row.n, f);
}

// order key: larger = earlier in the (value desc, index asc) order
__device__ __forceinline__ u64 order_key(float v, int i) {
    const unsigned b = __float_as_uint(v);
    const unsigned o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((u64)o << 32) | (unsigned)(~(unsigned)i);
}
__device__ __forceinline__ int key_index(u64 k) { return (int)~(unsigned)(k & 0xffffffffu); }
__device__ __forceinline__ float key_value(u64 k) {
    const unsigned o = (unsigned)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// q = trunc(exp(v - vmax) * 2^40): v_exp_f32 on (v - vmax) log2(e), then
// the product s < 2^41 split into 32-bit halves, each converted exactly
// (s - hi 2^32 is exact: s >= 2^32 has an exponent of at least 9)
__device__ __forceinline__ u64 mass_fx(float v, float vmax) {
    const float m = __builtin_amdgcn_exp2f((v - vmax) * 1.4426950408889634f);
    if (!(m > 0.0f)) return 0ULL;  // underflow or NaN
    const float s = m * kFx;
    const unsigned hi = (unsigned)(s * 2.3283064365386963e-10f);  // s / 2^32
    const unsigned lo = (unsigned)(s - (float)hi * 4294967296.0f);
    return ((u64)hi << 32) | lo;
}
// k >> s with s in [0, 64] (a shift by 64 gives 0)
__device__ __forceinline__ u64 shr64(u64 k, int s) { return s >= 64 ? 0ULL : k >> s; }
__device__ __forceinline__ int dist_bin(float v, float vmax) {
    const float d = (vmax - v) * kDistScale;  // >= 0; +inf for v = -inf
    return d < (float)(kDistBins - 1) ? (int)d : kDistBins - 1;
}

constexpr int kMaxSlices = 64;

struct SmpShared {
    u64 h_mass[kDistBins];
    int seg_off[kMaxSlices + 1];  // sliced path: gathered segment offsets
    u64 g_key[kGather];
    u64 g_q[kGather];
    u64 wsum[kSmpNT / 64];
    unsigned r_cnt[256];
    u64 r_key, r_mass, r_above;
    int r_bin, g_n, g_bin, g_cnt;
    float fred[kSmpNT / 64];
    unsigned bitmap[kMaxBitmapVocab / 32];
};

// inclusive scan of one value per thread over the workgroup
__device__ __forceinline__ u64 block_scan(u64 v, u64* wsum) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const u64 y = __shfl_up(v, o, 64);
        if (lane >= o) v += y;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    u64 off = 0;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    __syncthreads();
    return v + off;
}

template <bool MAX>
__device__ __forceinline__ u64 block_minmax(u64 v, u64* wsum) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const u64 y = __shfl_xor(v, o, 64);
        v = MAX ? (y > v ? y : v) : (y < v ? y : v);
    }
    if (lane == 0) wsum[wave] = v;
    __syncthreads();
    u64 r = wsum[0];
    for (int w = 1; w < kSmpNT / 64; ++w) r = MAX ? (wsum[w] > r ? wsum[w] : r) : (wsum[w] < r ? wsum[w] : r);
    __syncthreads();
    return r;
}

// Distance bin where the prefix mass crosses T (1 <= T <= total), into
// sh.r_bin, with the mass of the bins before it in sh.r_above: thread t owns
// bins 2t, 2t + 1 (exactly one thread matches; the defaults keep every
// later index in range regardless). Sets sh.r_key / sh.r_mass to defaults.
__device__ void find_bin(u64 T, SmpShared& sh) {
    const int tid = threadIdx.x;
    if (tid == 0) {
        sh.r_bin = 0;
        sh.r_above = 0;
        sh.r_key = 0;
        sh.r_mass = T;
    }
    const u64 m0 = sh.h_mass[2 * tid], m1 = sh.h_mass[2 * tid + 1];
    const u64 incl = block_scan(m0 + m1, sh.wsum);
    const u64 excl = incl - m0 - m1;
    if (excl < T && T <= incl) {
        const bool first = excl + m0 >= T;
        sh.r_bin = first ? 2 * tid : 2 * tid + 1;
        sh.r_above = first ? excl : excl + m0;
    }
    __syncthreads();
}

// Tokens gathered ahead by the sliced pipeline: every token of the bins a
// query can cross, in S segments of `cap` entries; segment sg holds
// sh.seg_off[sg + 1] - sh.seg_off[sg] of them (ok == 0: not gathered, scan
// the row).
struct Pregathered {
    const u64* key;
    const u64* q;
    int S, cap, ok;
};

// Smallest prefix of the order whose mass reaches T (1 <= T <= total):
// returns its last key in sh.r_key and the prefix mass in sh.r_mass.
__device__ void select_prefix(const SampleRow& row, float vmax, u64 T, SmpShared& sh,
                              const Pregathered& pre) {
    const int tid = threadIdx.x;
    find_bin(T, sh);
    const int bin = min(max(sh.r_bin, 0), kDistBins - 1);
    const u64 above = sh.r_above;
    // gather the bin and sort it exactly (reused when the previous query
    // sorted the same bin); a bin with more than kGather tokens goes to the
    // radix passes below
    if (sh.g_bin != bin) {
        if (tid == 0) sh.g_n = 0;
        __syncthreads();
        if (pre.ok) {
            // one flat pass over all segments: candidate j lies in the
            // segment whose offsets enclose it
            const int total = sh.seg_off[pre.S];
            for (int j = tid; j < total; j += kSmpNT) {
                int sg = 0;
                while (sh.seg_off[sg + 1] <= j) ++sg;
                const size_t at = (size_t)sg * pre.cap + (j - sh.seg_off[sg]);
                // the mass is loaded with the key, not after the bin test:
                // one memory round trip per query instead of two
                const u64 k = pre.key[at];
                const u64 q = pre.q[at];
                if (dist_bin(key_value(k), vmax) == bin) {
                    const int slot = atomicAdd(&sh.g_n, 1);
                    if (slot < kGather) {
                        sh.g_key[slot] = k;
                        sh.g_q[slot] = q;
                    }
                }
            }
        } else {
            row_scan<kSmpNT>(row, [&](int i, float v) {
                if (dist_bin(v, vmax) == bin) {
                    const int slot = atomicAdd(&sh.g_n, 1);
                    if (slot < kGather) {
                        sh.g_key[slot] = order_key(v, i);
                        sh.g_q[slot] = mass_fx(v, vmax);
                    }
                }
            });
        }
        __syncthreads();
        const int gcnt = sh.g_n;
        if (gcnt > kSmpNT && gcnt <= kGather) {  // a small bin needs no sort (below)
            int np2 = 1;
            while (np2 < gcnt) np2 <<= 1;
            for (int i = gcnt + tid; i < np2; i += kSmpNT) {
                sh.g_key[i] = 0;
                sh.g_q[i] = 0;
            }
            __syncthreads();
            // bitonic sort, descending by key
            for (int k = 2; k <= np2; k <<= 1)
                for (int j = k >> 1; j > 0; j >>= 1) {
                    for (int i = tid; i < np2; i += kSmpNT) {
                        const int ixj = i ^ j;
                        if (ixj > i) {
                            const u64 a = sh.g_key[i], b = sh.g_key[ixj];
                            const bool up = (i & k) == 0;
                            if (up ? a < b : a > b) {
                                sh.g_key[i] = b;
                                sh.g_key[ixj] = a;
                                const u64 t = sh.g_q[i];
                                sh.g_q[i] = sh.g_q[ixj];
                                sh.g_q[ixj] = t;
                            }
                        }
                    }
                    __syncthreads();
                }
        }
        if (tid == 0) {
            sh.g_cnt = gcnt;
            sh.g_bin = gcnt <= kGather ? bin : -2;
        }
        __syncthreads();
    }
    if (sh.g_bin == bin && sh.g_cnt <= kSmpNT) {
        // up to one entry per thread, unsorted. Keys are unique, so the mass
        // of the bin's order before entry i is the sum over the entries
        // with a larger key; the entry whose span (above + before, above +
        // before + q] holds T is the crossing one (every thread reads the
        // same entry at a time: LDS broadcasts, no barrier per step)
        // P adjacent threads share an entry (P = 1 .. 16, as many as the
        // bin's size allows), each summing over a 1/P share of the others,
        // four at a time; xor shuffles combine the shares.
        const int c = sh.g_cnt;
        const int P = c <= kSmpNT / 16 ? 16 : c <= kSmpNT / 8 ? 8 : c <= kSmpNT / 4 ? 4
                    : c <= kSmpNT / 2 ? 2 : 1;
        const int e = tid / P, part = tid - e * P;
        const u64 ki = e < c ? sh.g_key[e] : 0, qi = e < c ? sh.g_q[e] : 0;
        const int per = (c + P - 1) / P;
        const int j0 = part * per, j1 = min(c, j0 + per);
        u64 b0 = 0, b1 = 0, b2 = 0, b3 = 0;
        int j = j0;
        for (; j + 4 <= j1; j += 4) {
            const u64 k0 = sh.g_key[j], k1 = sh.g_key[j + 1], k2 = sh.g_key[j + 2],
                      k3 = sh.g_key[j + 3];
            const u64 q0 = sh.g_q[j], q1 = sh.g_q[j + 1], q2 = sh.g_q[j + 2], q3 = sh.g_q[j + 3];
            b0 += k0 > ki ? q0 : 0ULL;
            b1 += k1 > ki ? q1 : 0ULL;
            b2 += k2 > ki ? q2 : 0ULL;
            b3 += k3 > ki ? q3 : 0ULL;
        }
        for (; j < j1; ++j) b0 += sh.g_key[j] > ki ? sh.g_q[j] : 0ULL;
        u64 before = (b0 + b1) + (b2 + b3);
        for (int o = 1; o < P; o <<= 1) before += __shfl_xor(before, o, 64);
        const u64 lo_m = above + before;
        if (part == 0 && e < c && lo_m < T && T <= lo_m + qi) {
            sh.r_key = ki;
            sh.r_mass = lo_m + qi;
        }
        __syncthreads();
        return;
    }
    if (sh.g_bin == bin) {
        // scan the sorted bin: thread t owns entries 4t .. 4t + 3
        const int c = sh.g_cnt;
        u64 q[4], local = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * tid + e;
            q[e] = i < c ? sh.g_q[i] : 0;
            local += q[e];
        }
        const u64 incl = block_scan(local, sh.wsum) + above;
        u64 run = incl - local;
        if (run < T && T <= incl) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (run < T && T <= run + q[e]) {
                    sh.r_key = sh.g_key[4 * tid + e];
                    sh.r_mass = run + q[e];
                }
                run += q[e];
            }
        }
        __syncthreads();
        return;
    }
    // large bin: radix passes over the exact key, restricted to the bin
    u64 kmax = 0, kmin = ~0ULL;
    row_scan<kSmpNT>(row, [&](int i, float v) {
        if (dist_bin(v, vmax) == bin) {
            const u64 k = order_key(v, i);
            kmax = k > kmax ? k : kmax;
            kmin = k < kmin ? k : kmin;
        }
    });
    kmax = block_minmax<true>(kmax, sh.wsum);
    kmin = block_minmax<false>(kmin, sh.wsum);
    const int hb = 63 - __clzll(kmax ^ kmin);  // highest differing bit (cnt > 1: keys unique)
    int shift = hb >= 7 ? hb - 7 : 0;
    int width = hb - shift + 1;
    u64 prefix = shr64(kmax, hb + 1);          // bits above hb (shared by the whole bin)
    u64 above_r = above;
    u64* hm = sh.g_key;                        // 256 bins of mass
    u64* hk = sh.g_q;                          // 256 bins of max key
    unsigned* hc = sh.r_cnt;                   // 256 bins of count
    while (true) {
        for (int b = tid; b < 256; b += kSmpNT) {
            hm[b] = 0;
            hk[b] = 0;
            hc[b] = 0;
        }
        __syncthreads();
        row_scan<kSmpNT>(row, [&](int i, float v) {
            if (dist_bin(v, vmax) != bin) return;
            const u64 k = order_key(v, i);
            if (shr64(k, shift + width) != prefix) return;
            const int b = (int)((k >> shift) & ((1u << width) - 1u));
            atomicAdd(&hm[b], mass_fx(v, vmax));
            atomicAdd(&hc[b], 1u);
            atomicMax(&hk[b], k);
        });
        __syncthreads();
        // crossing digit from the top: thread t (< 256) owns digit 255 - t
        if (tid == 0) sh.r_bin = 0;
        {
            const int d = 255 - tid;
            const u64 m = tid < 256 ? hm[d] : 0;
            const u64 incl = block_scan(m, sh.wsum) + above_r;
            const u64 excl = incl - m;
            if (tid < 256 && excl < T && T <= incl) {
                sh.r_bin = d;
                sh.r_above = excl;
            }
            __syncthreads();
        }
        const int d = sh.r_bin & 255;
        above_r = sh.r_above;
        prefix = (prefix << width) | (u64)d;
        if (hc[d] == 1u || shift == 0) {
            if (tid == 0) {
                sh.r_key = shift == 0 ? prefix : hk[d];
                sh.r_mass = above_r + hm[d];
            }
            __syncthreads();
            // the gather buffers held the radix bins: never reuse them
            if (tid == 0) sh.g_bin = -2;
            __syncthreads();
            return;
        }
        width = shift >= 8 ? 8 : shift;
        shift -= width;
        __syncthreads();
    }
}

// One row per workgroup. ids/offs: penalised token ids of row r at
// ids[offs[r] .. offs[r + 1]) (offs null: ids[0 .. m_single)); seeds: one
// per row (null: seed0 for a single row).
__global__ __launch_bounds__(kSmpNT) void sample_topp_rows(
    const float* __restrict__ x, int n, float p, float inv_t, float pen,
    const long long* __restrict__ ids, const long long* __restrict__ offs, int m_single,
    const u64* __restrict__ seeds, u64 seed0, long long* __restrict__ out) {
    __shared__ SmpShared sh;
    const int r = blockIdx.x;
    const int tid = threadIdx.x;
    // the seed first: it may sit in host memory, and its round trip then
    // overlaps the passes below
    const u64 seed = seeds ? seeds[r] : seed0;
    SampleRow row{x + (size_t)r * n, n, inv_t, pen, nullptr, 0};
    const bool penal = ids != nullptr && pen != 1.0f;
    if (penal) {
        for (int w = tid; w < (n + 31) / 32; w += kSmpNT) sh.bitmap[w] = 0u;
        __syncthreads();
        const long long a = offs ? offs[r] : 0;
        const long long b = offs ? offs[r + 1] : m_single;
        for (long long j = a + tid; j < b; j += kSmpNT) {
            const long long id = ids[j];
            if (id >= 0 && id < n) atomicOr(&sh.bitmap[id >> 5], 1u << (id & 31));  // others dropped
        }
        __syncthreads();
        row.bits = sh.bitmap;
    }
    // row maximum
    float vmax = -INFINITY;
    row_scan<kSmpNT>(row, [&](int, float v) { vmax = fmaxf(vmax, v); });
    vmax = block_max<kSmpNT>(vmax, sh.fred);
    if (!(vmax > -INFINITY)) {
        // every value -inf (or NaN): the reference's float path never
        // reaches its cut and returns the last token of the order
        if (tid == 0) out[r] = n - 1;
        return;
    }
    // distance histogram (mass and count per bin)
    for (int b = tid; b < kDistBins; b += kSmpNT) sh.h_mass[b] = 0;
    if (tid == 0) sh.g_bin = -1;
    __syncthreads();
    row_scan<kSmpNT>(row, [&](int, float v) {
        const u64 q = mass_fx(v, vmax);
        if (q) atomicAdd(&sh.h_mass[dist_bin(v, vmax)], q);
    });
    __syncthreads();
    u64 total;
    {
        const u64 incl = block_scan(sh.h_mass[2 * tid] + sh.h_mass[2 * tid + 1], sh.wsum);
        if (tid == kSmpNT - 1) sh.r_mass = incl;
        __syncthreads();
        total = sh.r_mass;
        __syncthreads();
    }
    // nucleus cut: prefix mass >= p * total
    double tc = ceil((double)p * (double)total);
    u64 T = tc < 1.0 ? 1ULL : (u64)tc;
    if (T > total) T = total;
    const Pregathered none{nullptr, nullptr, 0, 0, 0};
    select_prefix(row, vmax, T, sh, none);
    const u64 nucleus = sh.r_mass;
    // draw: prefix mass >= u * nucleus mass
    const float u = splitmix_uniform(seed);
    double td = ceil((double)u * (double)nucleus);
    T = td < 1.0 ? 1ULL : (u64)td;
    if (T > nucleus) T = nucleus;
    select_prefix(row, vmax, T, sh, none);
    if (tid == 0) out[r] = key_index(sh.r_key);
}

// ---------------------------------------------------------------------------
// Sliced pipeline (fewer rows than CUs): each row is cut into S slices of
// slen tokens (a multiple of 32), so that S workgroups share a row's passes
// over the logits; the per-row steps run on one workgroup per row. Same
// arithmetic and order as sample_topp_rows (integer masses: every merge is
// exact), so the tokens are identical.
//   1 smp_slice_max    slice maxima; the slice's penalty bits to global;
//                      slice s clears its share of the row's histogram
//   2 smp_slice_hist   slice distance histograms from the row maximum, in
//                      LDS, then added into the row's histogram (integer
//                      atomics, so the sum does not depend on their order;
//                      writing S slice histograms for smp_plan to merge
//                      made the merge read S x 16 KB per row from one
//                      workgroup, ~15 us at 64 x 128k)
//   3 smp_plan         per row: total, the nucleus bin b1
//                      and the range [c_lo, c_hi] of bins the draw can
//                      cross (the nucleus mass lies in b1's prefix range and
//                      the draw threshold is monotone in it)
//   4 smp_gather       each slice collects the tokens of those bins (order
//                      key, mass) in LDS, one reservation per wave, and
//                      copies them to its own segment of the row's buffer
//                      (no atomics across workgroups: a shared counter per
//                      row kept this pass at 65 us on 64 x 128k rows)
//   5 smp_finish       the two threshold queries of sample_topp_rows on the
//                      merged histogram and the gathered tokens; a row whose
//                      candidates overflowed the buffer is resolved by full
//                      row scans, and a crossing bin beyond the exact sort's
//                      capacity by the radix passes, as in sample_topp_rows
// ---------------------------------------------------------------------------
constexpr int kSliceNT = 256;
constexpr int kMinSlice = 8192;    // tokens per slice at least
constexpr int kSliceCap = 1024;    // gathered candidates per slice
constexpr int kSliceLoads = 16;    // 16-byte loads in flight per thread: a
                                   // 16k-token slice in one round trip
// LDS bitmap words of one slice: the sliced path runs with S >= 2, so a
// slice holds at most ceil(n / 2) + 31 tokens, n <= kMaxBitmapVocab
constexpr int kSliceWords = (kMaxBitmapVocab / 2 + 32) / 32 + 1;

struct SmpPlan {
    u64 total;
    float vmax;
    int b1, c_lo, c_hi;
};

struct SliceArgs {
    const float* x;
    int n, S, slen, words;     // words: bitmap words per row
    float inv_t, pen;
    const long long* ids;      // null: no penalty
    const long long* offs;     // null: ids[0 .. m_single) for row 0
    int m_single;
    unsigned* bits;            // rows x words
    float* smax;               // rows x S
    u64* mhist;                // rows x kDistBins: the row's merged histogram
    SmpPlan* plan;             // rows
    int* gcnt;                 // rows x S
    u64* gkey;                 // rows x S x kSliceCap
    u64* gq;                   // rows x S x kSliceCap
    float p;
    const u64* seeds;
    u64 seed0;
    u64* seedv;                // rows: each row's seed, copied by smp_slice_max
    long long* out;
};

__device__ __forceinline__ SampleRow slice_row(const SliceArgs& a, int r) {
    SampleRow row{a.x + (size_t)r * a.n, a.n, a.inv_t, a.pen, nullptr, 0};
    if (a.ids) row.bits = a.bits + (size_t)r * a.words;
    return row;
}

// The row with the penalty bits of tokens [lo, hi) copied to LDS (a global
// bitmap word per token kept each pass waiting on dependent loads). Ends
// with a workgroup barrier in every case, so LDS set up before the call is
// visible to the whole workgroup after it.
__device__ __forceinline__ SampleRow slice_row_lds(const SliceArgs& a, int r, int lo, int hi,
                                                   unsigned* lbits) {
    SampleRow row{a.x + (size_t)r * a.n, a.n, a.inv_t, a.pen, nullptr, 0};
    if (a.ids) {
        const int w0 = lo >> 5, w1 = (hi + 31) >> 5;
        const unsigned* g = a.bits + (size_t)r * a.words;
        for (int w = w0 + (int)threadIdx.x; w < w1; w += kSliceNT) lbits[w - w0] = g[w];
        row.bits = lbits;
        row.bit0 = w0 * 32;
    }
    __syncthreads();
    return row;
}

__global__ __launch_bounds__(kSliceNT) void smp_slice_max(SliceArgs a) {
    __shared__ unsigned lbits[kSliceWords];
    __shared__ float red[kSliceNT / 64];
    const int r = blockIdx.x / a.S, s = blockIdx.x - r * a.S;
    const int lo = min(a.n, s * a.slen), hi = min(a.n, lo + a.slen);
    // The row's seed, copied to device memory for smp_plan and smp_finish:
    // the seeds (like the histories) may sit in host memory, and this read
    // overlaps the offsets' round trip here instead of adding one there.
    const bool seed_lane = s == 0 && threadIdx.x == 0;
    u64 seed = 0;
    if (seed_lane) seed = a.seeds ? a.seeds[r] : a.seed0;
    SampleRow row{a.x + (size_t)r * a.n, a.n, a.inv_t, a.pen, nullptr, 0};
    if (a.ids) {
        // this slice's words of the row's bitmap (slices own whole words)
        const int w0 = lo >> 5, w1 = (hi + 31) >> 5;
        for (int w = w0 + (int)threadIdx.x; w < w1; w += kSliceNT) lbits[w - w0] = 0u;
        __syncthreads();
        const long long ja = a.offs ? a.offs[r] : 0;
        const long long jb = a.offs ? a.offs[r + 1] : a.m_single;
        for (long long j = ja + threadIdx.x; j < jb; j += kSliceNT) {
            const long long id = a.ids[j];
            if (id >= lo && id < hi) atomicOr(&lbits[(id >> 5) - w0], 1u << (id & 31));
        }
        __syncthreads();
        for (int w = w0 + (int)threadIdx.x; w < w1; w += kSliceNT)
            a.bits[(size_t)r * a.words + w] = lbits[w - w0];
        row.bits = lbits;
        row.bit0 = w0 * 32;
    }
    // this slice's share of the row histogram smp_slice_hist adds into
    u64* mh = a.mhist + (size_t)r * kDistBins;
    for (int b = s * kDistBins / a.S + (int)threadIdx.x; b < (s + 1) * kDistBins / a.S;
         b += kSliceNT)
        mh[b] = 0;
    float vmax = -INFINITY;
    slice_scan<kSliceNT, kSliceLoads>(row, lo, hi, [&](int, float v) { vmax = fmaxf(vmax, v); });
    vmax = block_max<kSliceNT>(vmax, red);
    if (threadIdx.x == 0) a.smax[blockIdx.x] = vmax;
    if (seed_lane) a.seedv[r] = seed;
}

__device__ __forceinline__ float row_max_of(const SliceArgs& a, int r) {
    float vmax = -INFINITY;
    for (int s = 0; s < a.S; ++s) vmax = fmaxf(vmax, a.smax[r * a.S + s]);
    return vmax;
}

__global__ __launch_bounds__(kSliceNT) void smp_slice_hist(SliceArgs a) {
    __shared__ u64 hm[kDistBins];
    __shared__ unsigned lbits[kSliceWords];
    const int r = blockIdx.x / a.S, s = blockIdx.x - r * a.S;
    const float vmax = row_max_of(a, r);
    if (!(vmax > -INFINITY)) return;  // smp_plan settles the row
    const int lo = min(a.n, s * a.slen), hi = min(a.n, lo + a.slen);
    for (int b = threadIdx.x; b < kDistBins; b += kSliceNT) hm[b] = 0;
    const SampleRow row = slice_row_lds(a, r, lo, hi, lbits);  // (synchronises)
    slice_scan<kSliceNT, kSliceLoads>(row, lo, hi, [&](int, float v) {
        const u64 q = mass_fx(v, vmax);
        if (q) atomicAdd(&hm[dist_bin(v, vmax)], q);
    });
    __syncthreads();
    u64* mh = a.mhist + (size_t)r * kDistBins;
    for (int b = threadIdx.x; b < kDistBins; b += kSliceNT)
        if (hm[b]) atomicAdd(mh + b, hm[b]);
}

__global__ __launch_bounds__(kSmpNT) void smp_plan(SliceArgs a) {
    __shared__ SmpShared sh;
    const int r = blockIdx.x, tid = threadIdx.x;
    const u64 seed = a.seedv[r];
    const float vmax = row_max_of(a, r);
    if (!(vmax > -INFINITY)) {
        if (tid == 0) a.plan[r] = SmpPlan{0ULL, vmax, 0, 0, 0};
        return;
    }
    // one scan of the histogram serves the three bin queries below: thread
    // t owns bins 2t and 2t + 1, as in find_bin
    static_assert(kDistBins == 2 * kSmpNT, "two bins per thread");
    const u64* mh = a.mhist + (size_t)r * kDistBins;
    const u64 m0 = mh[2 * tid], m1 = mh[2 * tid + 1];
    sh.h_mass[2 * tid] = m0;
    sh.h_mass[2 * tid + 1] = m1;
    const u64 incl = block_scan(m0 + m1, sh.wsum);  // (its barriers order the stores)
    const u64 excl = incl - m0 - m1;
    if (tid == kSmpNT - 1) sh.r_mass = incl;
    __syncthreads();
    const u64 total = sh.r_mass;
    // find_bin's result from the scan above: with 1 <= T <= total exactly
    // one thread's pair holds the crossing; total == 0 (no token with mass,
    // e.g. a +inf logit) gives find_bin's defaults, bin 0 and nothing above
    auto cross = [&](u64 T) {
        if (total == 0) {  // uniform: every thread read the same total
            if (tid == 0) {
                sh.r_bin = 0;
                sh.r_above = 0;
            }
        } else if (excl < T && T <= incl) {
            const bool first = excl + m0 >= T;
            sh.r_bin = first ? 2 * tid : 2 * tid + 1;
            sh.r_above = first ? excl : excl + m0;
        }
        __syncthreads();
    };
    // the nucleus bin, as smp_finish will find it
    const double tc = ceil((double)a.p * (double)total);
    u64 T1 = tc < 1.0 ? 1ULL : (u64)tc;
    if (T1 > total) T1 = total;
    cross(T1);
    const int b1 = min(max(sh.r_bin, 0), kDistBins - 1);
    const u64 after_b1 = sh.r_above + sh.h_mass[b1];  // nucleus mass is in [T1, after_b1]
    __syncthreads();
    // the draw threshold for the extreme nucleus masses
    const float u = splitmix_uniform(seed);
    auto draw_t = [&](u64 nucleus) {
        const double td = ceil((double)u * (double)nucleus);
        u64 T = td < 1.0 ? 1ULL : (u64)td;
        return T > nucleus ? nucleus : T;
    };
    cross(draw_t(T1));
    const int c_lo = min(max(sh.r_bin, 0), kDistBins - 1);
    __syncthreads();
    cross(draw_t(after_b1));
    const int c_hi = min(max(sh.r_bin, 0), kDistBins - 1);
    __syncthreads();
    if (tid == 0) a.plan[r] = SmpPlan{total, vmax, b1, c_lo, c_hi};
}

__global__ __launch_bounds__(kSliceNT) void smp_gather(SliceArgs a) {
    __shared__ unsigned lbits[kSliceWords];
    __shared__ u64 lkey[kSliceCap], lq[kSliceCap];
    __shared__ int lcount;
    const int r = blockIdx.x / a.S, s = blockIdx.x - r * a.S;
    const SmpPlan pl = a.plan[r];
    if (!(pl.vmax > -INFINITY)) return;
    const int lo = min(a.n, s * a.slen), hi = min(a.n, lo + a.slen);
    const int lane = threadIdx.x & 63;
    if (threadIdx.x == 0) lcount = 0;
    const SampleRow row = slice_row_lds(a, r, lo, hi, lbits);  // (synchronises)
    slice_scan<kSliceNT, kSliceLoads>(row, lo, hi, [&](int i, float v) {
        const int b = dist_bin(v, pl.vmax);
        const bool cand = b == pl.b1 || (b >= pl.c_lo && b <= pl.c_hi);
        // one reservation per wave: the lowest candidate lane adds the
        // wave's count, the others take consecutive slots after it
        const u64 mask = __ballot(cand);
        if (cand) {
            const int leader = __ffsll((long long)mask) - 1;
            int base = 0;
            if (lane == leader) base = atomicAdd(&lcount, __popcll(mask));
            base = __shfl(base, leader, 64);
            const int slot = base + __popcll(mask & ((1ULL << lane) - 1ULL));
            if (slot < kSliceCap) {  // a larger count sends the row to row scans
                lkey[slot] = order_key(v, i);
                lq[slot] = mass_fx(v, pl.vmax);
            }
        }
    });
    __syncthreads();
    const int c = lcount;
    const size_t seg = (size_t)blockIdx.x * kSliceCap;
    for (int j = threadIdx.x; j < min(c, kSliceCap); j += kSliceNT) {
        a.gkey[seg + j] = lkey[j];
        a.gq[seg + j] = lq[j];
    }
    if (threadIdx.x == 0) a.gcnt[blockIdx.x] = c;
}

__global__ __launch_bounds__(kSmpNT) void smp_finish(SliceArgs a) {
    __shared__ SmpShared sh;
    const int r = blockIdx.x, tid = threadIdx.x;
    const u64 seed = a.seedv[r];
    const SmpPlan pl = a.plan[r];
    if (!(pl.vmax > -INFINITY)) {
        // every value -inf (or NaN): as sample_topp_rows
        if (tid == 0) a.out[r] = a.n - 1;
        return;
    }
    for (int b = tid; b < kDistBins; b += kSmpNT) sh.h_mass[b] = a.mhist[(size_t)r * kDistBins + b];
    if (tid == 0) sh.g_bin = -1;
    __syncthreads();
    const SampleRow row = slice_row(a, r);
    // the gathered segments of this row (any overflowed: full row scans)
    if (tid < 64) {
        const int c = tid < a.S ? a.gcnt[r * a.S + tid] : 0;
        const unsigned long long over = __ballot(c > kSliceCap);
        int incl = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o, 64);
            if (tid >= o) incl += y;
        }
        if (tid < a.S) sh.seg_off[tid + 1] = incl;
        if (tid == 0) {
            sh.seg_off[0] = 0;
            sh.g_cnt = over ? 0 : 1;
        }
    }
    __syncthreads();
    const Pregathered pre{a.gkey + (size_t)r * a.S * kSliceCap, a.gq + (size_t)r * a.S * kSliceCap,
                          a.S, kSliceCap, sh.g_cnt};
    __syncthreads();
    const u64 total = pl.total;
    const double tc = ceil((double)a.p * (double)total);
    u64 T = tc < 1.0 ? 1ULL : (u64)tc;
    if (T > total) T = total;
    select_prefix(row, pl.vmax, T, sh, pre);
    const u64 nucleus = sh.r_mass;
    const float u = splitmix_uniform(seed);
    const double td = ceil((double)u * (double)nucleus);
    T = td < 1.0 ? 1ULL : (u64)td;
    if (T > nucleus) T = nucleus;
    select_prefix(row, pl.vmax, T, sh, pre);
    if (tid == 0) a.out[r] = key_index(sh.r_key);
}

// argmax per row (earliest index on ties): a sequential scan with strict >
// keeps index 0 when x[0] is NaN and never picks a NaN elsewhere, so NaN
// counts as -inf except at index 0.
constexpr int kArgNT = 1024;

template <typename OUT>
__global__ __launch_bounds__(kArgNT) void argmax_rows(const float* __restrict__ x, int n,
                                                      OUT* __restrict__ out) {
    __shared__ float sv[kArgNT / 64];
    __shared__ int si[kArgNT / 64];
    const SampleRow row{x + (size_t)blockIdx.x * n, n, 1.0f, 1.0f, nullptr, 0};
    const int tid = threadIdx.x;
    float bv = -INFINITY;
    int bi = n;  // sentinel: no candidate
    row_scan<kArgNT>(row, [&](int i, float v) {
        if (v != v) v = -INFINITY;
        if (v > bv || (v == bv && i < bi)) {
            bv = v;
            bi = i;
        }
    });
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kArgNT / 64; ++w)
            if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) {
                bv = sv[w];
                bi = si[w];
            }
        const float x0 = row.x[0];
        out[blockIdx.x] = (OUT)((x0 != x0 || bi >= n) ? 0 : bi);
    }
}

// argmax with a row split across workgroups when there are fewer rows than
// CUs: workgroup (slice, row) reduces tokens [slice * slen, +slen) with the
// comparator of argmax_rows (value, then earliest index; NaN as -inf), and
// one wave per row folds the slice winners. The comparator is a total order
// on (value, -index), so any split gives argmax_rows' result; the index-0
// NaN rule is applied once, in the fold.
constexpr int kArgSliceNT = 256;
constexpr int kArgMaxSlices = 64;
constexpr int kArgMinSlice = 4096;  // tokens

__device__ __forceinline__ void arg_better(float& bv, int& bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}

__global__ __launch_bounds__(kArgSliceNT) void argmax_slices(const float* __restrict__ x, int n,
                                                             int slen, float* __restrict__ pv,
                                                             int* __restrict__ pi) {
    __shared__ float sv[kArgSliceNT / 64];
    __shared__ int si[kArgSliceNT / 64];
    const SampleRow row{x + (size_t)blockIdx.y * n, n, 1.0f, 1.0f, nullptr, 0};
    const int lo = blockIdx.x * slen;
    const int hi = min(n, lo + slen);
    const int tid = threadIdx.x;
    float bv = -INFINITY;
    int bi = n;
    slice_scan<kArgSliceNT>(row, lo, hi, [&](int i, float v) {
        if (v != v) v = -INFINITY;
        arg_better(bv, bi, v, i);
    });
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        arg_better(bv, bi, ov, oi);
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kArgSliceNT / 64; ++w) arg_better(bv, bi, sv[w], si[w]);
        pv[(size_t)blockIdx.y * gridDim.x + blockIdx.x] = bv;
        pi[(size_t)blockIdx.y * gridDim.x + blockIdx.x] = bi;
    }
}

template <typename OUT>
__global__ __launch_bounds__(64) void argmax_fold(const float* __restrict__ x, int n, int S,
                                                  const float* __restrict__ pv,
                                                  const int* __restrict__ pi,
                                                  OUT* __restrict__ out) {
    const int lane = threadIdx.x;
    const int r = blockIdx.x;
    float bv = -INFINITY;
    int bi = n;
    if (lane < S) {
        bv = pv[(size_t)r * S + lane];
        bi = pi[(size_t)r * S + lane];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        arg_better(bv, bi, ov, oi);
    }
    if (lane == 0) {
        const float x0 = x[(size_t)r * n];
        out[r] = (OUT)((x0 != x0 || bi >= n) ? 0 : bi);
    }
}

template <typename OUT>
void argmax_launch(const float* x, int rows, int n, OUT* out, hipStream_t s) {
    // slices of at least kArgMinSlice tokens, enough workgroups for ~4 per CU
    // (FT_ARG_SLICES forces a count, 1 = one workgroup per row)
    const int cus = dev_info().cu_count;
    int S = 1;
    if (rows < cus)
        S = std::min({(4 * cus + rows - 1) / rows, std::max(1, n / kArgMinSlice), kArgMaxSlices});
    const int forced = tune(Tune::ArgSlices, 0);
    if (forced > 0) S = std::min(forced, kArgMaxSlices);
    int slen = (n + S - 1) / S;
    slen = (slen + 3) & ~3;  // slices start on 4-token boundaries
    S = (n + slen - 1) / slen;
    if (S <= 1) {
        argmax_rows<OUT><<<(unsigned)rows, kArgNT, 0, s>>>(x, n, out);
        launch_check("argmax kernel launch");
        return;
    }
    const size_t pairs = (size_t)rows * S;
    char* buf = (char*)scratch(Scratch::Sampling, pairs * (sizeof(float) + sizeof(int)), s);
    float* pv = (float*)buf;
    int* pi = (int*)(buf + pairs * sizeof(float));
    argmax_slices<<<dim3((unsigned)S, (unsigned)rows), kArgSliceNT, 0, s>>>(x, n, slen, pv, pi);
    launch_check("argmax slice kernel launch");
    argmax_fold<OUT><<<(unsigned)rows, 64, 0, s>>>(x, n, S, pv, pi, out);
    launch_check("argmax fold kernel launch");
}

void sampling_check(int rows, int n, float p, float t) {
    if (rows < 0) inval("rows must be >= 0");
    if (n <= 0) inval("sample of empty logits");
    if (!(p > 0.0f && p <= 1.0f)) inval("p must be in (0, 1]");
    if (!(t > 0.0f)) inval("temperature must be > 0");
}

void topp_launch(const float* x, int rows, int n, float p, float t, float pen,
                 const long long* ids, const long long* offs, int m, const u64* seeds,
                 u64 seed0, long long* out, hipStream_t s) {
    sampling_check(rows, n, p, t);
    if (!(pen > 0.0f)) inval("penalty must be > 0");
    if (m < 0) inval("id count must be >= 0");
    const bool penal = pen != 1.0f && ((offs != nullptr) || m > 0);
    if (penal && n > kMaxBitmapVocab)
        inval("vocabulary too large for the penalty bitmap (n <= 524288)");
    if (rows == 0) return;
    if (!x || !out) inval("sampling: null operand");
    if (penal && !ids) inval("sampling: null token ids");
    const float inv_t = 1.0f / t;  // the reference's order (inv_t = 1.0f / t)
    // slices per row: enough workgroups for about two per CU, at least
    // kMinSlice tokens each; FT_SMP_SINGLE=1 keeps one workgroup per row
    const int cus = dev_info().cu_count;
    int S = 1;
    if (rows < cus && tune(Tune::SmpSingle, 0) == 0)
        S = std::min({(2 * cus + rows - 1) / rows, std::max(1, n / kMinSlice), kMaxSlices});
    // FT_SMP_SLICES forces the slice count (2 .. kMaxSlices, at most one
    // slice per 32 tokens)
    const int forced_s = tune(Tune::SmpSlices, 0);
    if (forced_s >= 2 && tune(Tune::SmpSingle, 0) == 0)
        S = std::min({forced_s, kMaxSlices, std::max(1, n / 32)});
    if (S <= 1) {
        sample_topp_rows<<<(unsigned)rows, kSmpNT, 0, s>>>(
            x, n, p, inv_t, pen, penal ? ids : nullptr, penal ? offs : nullptr, m, seeds, seed0,
            out);
        launch_check("sampling kernel launch");
        return;
    }
    int slen = (n + S - 1) / S;
    slen = (slen + 31) & ~31;  // whole bitmap words, 16-byte aligned starts
    S = (n + slen - 1) / slen;
    SliceArgs a{};
    a.x = x;
    a.n = n;
    a.S = S;
    a.slen = slen;
    a.words = (n + 31) / 32;
    a.inv_t = inv_t;
    a.pen = pen;
    a.ids = penal ? ids : nullptr;
    a.offs = penal ? offs : nullptr;
    a.m_single = m;
    a.p = p;
    a.seeds = seeds;
    a.seed0 = seed0;
    a.out = out;
    // scratch, 256-byte aligned pieces
    const size_t R = (size_t)rows;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) & ~(size_t)255;
        return at;
    };
    const size_t o_bits = take(R * a.words * 4), o_smax = take(R * S * 4),
                 o_mh = take(R * kDistBins * 8), o_plan = take(R * sizeof(SmpPlan)),
                 o_seed = take(R * 8),
                 o_gn = take(R * S * 4), o_gk = take(R * S * kSliceCap * 8),
                 o_gq = take(R * S * kSliceCap * 8);
    char* ws = (char*)scratch(Scratch::Sampling, off, s);
    a.bits = (unsigned*)(ws + o_bits);
    a.smax = (float*)(ws + o_smax);
    a.mhist = (u64*)(ws + o_mh);
    a.seedv = (u64*)(ws + o_seed);
    a.plan = (SmpPlan*)(ws + o_plan);
    a.gcnt = (int*)(ws + o_gn);
    a.gkey = (u64*)(ws + o_gk);
    a.gq = (u64*)(ws + o_gq);
    const unsigned grid = (unsigned)(rows * S);
    smp_slice_max<<<grid, kSliceNT, 0, s>>>(a);
    launch_check("sampling max kernel launch");
    smp_slice_hist<<<grid, kSliceNT, 0, s>>>(a);
    launch_check("sampling histogram kernel launch");
    smp_plan<<<(unsigned)rows, kSmpNT, 0, s>>>(a);
    launch_check("sampling plan kernel launch");
    smp_gather<<<grid, kSliceNT, 0, s>>>(a);
    launch_check("sampling gather kernel launch");
    smp_finish<<<(unsigned)rows, kSmpNT, 0, s>>>(a);
    launch_check("sampling kernel launch");
}

}  // namespace
}  // namespace ft

extern "C" {

int ft_argmax_launch(const float* x, int n, int* out, uintptr_t stream) {
    return ft::guarded([&] {
        if (n <= 0) ft::inval("argmax of empty vector");
        if (!x || !out) ft::inval("argmax: null operand");
        ft::argmax_launch<int>(x, 1, n, out, ft::as_stream(stream));
    });
}

int ft_argmax_batched_launch(const float* x, int rows, int n, long long* out,
                             uintptr_t stream) {
    return ft::guarded([&] {
        if (rows < 0) ft::inval("rows must be >= 0");
        if (n <= 0) ft::inval("argmax of empty vector");
        if (rows == 0) return;
        if (!x || !out) ft::inval("argmax: null operand");
        ft::argmax_launch<long long>(x, rows, n, out, ft::as_stream(stream));
    });
}

int ft_sample_topp_launch(const float* x, int n, float p, float t, unsigned long long seed,
                          long long* out, uintptr_t stream) {
    return ft::guarded([&] {
        ft::topp_launch(x, 1, n, p, t, 1.0f, nullptr, nullptr, 0, nullptr, seed, out,
                        ft::as_stream(stream));
    });
}

int ft_sample_topp_batched_launch(const float* x, int rows, int n, float p, float t,
                                  const unsigned long long* seeds, long long* out,
                                  uintptr_t stream) {
    return ft::guarded([&] {
        if (rows > 0 && !seeds) ft::inval("sampling: null seeds");
        ft::topp_launch(x, rows, n, p, t, 1.0f, nullptr, nullptr, 0, seeds, 0, out,
                        ft::as_stream(stream));
    });
}

int ft_decode_step_launch(const float* x, const long long* ids, int n, int m, float penalty,
                          float p, float t, unsigned long long seed, long long* out,
                          uintptr_t stream) {
    return ft::guarded([&] {
        ft::topp_launch(x, 1, n, p, t, penalty, ids, nullptr, m, nullptr, seed, out,
                        ft::as_stream(stream));
    });
}

int ft_decode_step_batched_launch(const float* x, int rows, int n, const long long* ids,
                                  const long long* offs, float penalty, float p, float t,
                                  const unsigned long long* seeds, long long* out,
                                  uintptr_t stream) {
    return ft::guarded([&] {
        if (rows > 0 && !seeds) ft::inval("sampling: null seeds");
        if (rows > 0 && !offs) ft::inval("sampling: null id offsets");
        ft::topp_launch(x, rows, n, p, t, penalty, ids, offs, 0, seeds, 0, out,
                        ft::as_stream(stream));
    });
}

}  // extern "C"
