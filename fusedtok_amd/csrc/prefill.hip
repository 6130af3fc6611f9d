// Prefill (fresh-sequence) attention for gfx950:
//
//   out[b, h, i] = softmax(q[b,h,i] . K[b,kv]^T / sqrt(D)) . V[b,kv],
//   kv = h / (Hq / Hkv), over key rows [0, i] (causal) or all S rows.
//   q, out: [B, Hq, S, D]; k, v: [B, Hkv, S, D]; D % 4 == 0, D <= 512.
//
// (reference attention.hpp:64-81 semantics, attention.cu:1591-1639 CPU
// path, attention.cu:1649-1739 launcher contract: no workspace, stream-
// ordered, capturable.)
//
// attn_prefill_mfma<T, D>: bf16 / fp16 storage, D in {64, 128}. A
// workgroup owns 128 query rows of one (b, q head), 32 per wave; 64-row K
// and V tiles stream through two LDS stages, both row-major.
// Everything is computed transposed, so every accumulator a lane holds
// belongs to one query row (r = lane % 16, g = lane / 16; operand layout
// of v_mfma_f32_16x16x32: A[r][8g+j], B[8g+j][r], C[4g+i][r]):
//
//   scores  S^T[kv][q] = K[kv][:] . Q[q][:]     A = K rows from LDS,
//           B = Q^T (the wave's Q in registers for the whole kernel);
//           lane (q, g) gets keys 4g + i of each 16-key block.
//   softmax online per query row: the 64 keys of a row sit in the 4 lanes
//           {q, q+16, q+32, q+48}: two lane swaps (v_permlane32/16_swap,
//           no LDS) for the tile maximum;
//           the rescale of the running output is a per-lane multiply.
//   PV      O^T[d][q] += V^T[d][kv] . P^T[kv][q]: B = P straight from the
//           score accumulators: for a 32-key step, lane (q, g) holds keys
//           {4g+i} of block 2ks and {16+4g+i} of block 2ks+1, so the k
//           slots are permuted (slot 8g+i <-> key 4g+i, slot 8g+4+i <->
//           key 16+4g+i). The V^T fragments come from the row-major V tile
//           through ds_read_b64_tr_b16, two per fragment: within each
//           16-lane group, destination lane i receives element i % 4 of
//           the 4-element pieces addressed by source lanes 4r + i / 4
//           (r = 0..3), so source lane s of group g addresses V row
//           (keys) 4g + s / 4 (+16 for the second read), columns 16 db +
//           4 (s % 4) .. + 3, and lane (d = i, g) gets keys 4g + r of d.
//   bf16:   P is split into hi + lo bf16 parts (two MFMAs), so the weights
//           carry ~16 mantissa bits; fp16 P carries 11.
//   sums    where P is one fp16 operand, the row sums are ones . P^T on the
//           same MFMA (the weights the PV product uses, 4 MFMAs per tile
//           instead of 32 adds per lane); the bf16 split loop adds in lanes.
//
// Causal work is uneven across query tiles: the grid runs the last (most
// keys) tiles of every head first.
//
// attn_prefill_generic<T>: f32 storage, and half storage with other D: one
// wave per query row, lanes across D in float4 chunks, online softmax over
// the keys (a parity path).
#include "ft_common.hpp"

#include <cstdlib>
#include <type_traits>

namespace ft {
namespace {

constexpr float kLog2eP = 1.4426950408889634f;
constexpr int kPQ = 128;                  // query rows per workgroup
constexpr int kPKV = 64;                  // key rows per tile
constexpr float kLazy = 8.0f;             // log2 of the largest unnormalised weight
// bf16 V elements from which V is converted to fp16 once per call
constexpr long long kPrepassMinElems = 1LL << 20;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct PMma;
template <> struct PMma<bf16> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    static constexpr bool kSplit = true;
    __device__ __forceinline__ static f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct PMma<f16> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    static constexpr bool kSplit = false;
    __device__ __forceinline__ static f32x4 mma(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <int D>
struct PCfg {
    static constexpr int kKPitch = D * 2 + 16;                 // bytes per K row
    static constexpr int kStage = 2 * kPKV * kKPitch;          // K tile, then V tile
    static constexpr int kKChunks = kPKV * D / 8 / 256;        // 16-byte chunks per thread
    static constexpr int kS = D / 32;                          // score k-steps
    static constexpr int kDB = D / 16;                         // output d blocks
};

// two floats -> one dword of two T values (round to nearest even)
template <typename T>
__device__ __forceinline__ int pack2(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef T t2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(int, __builtin_convertvector(f2{a, b}, t2));
}

// two bf16 (one dword) -> two fp16, exact for v = 0 and 2^-17 <= |v| < 2^16:
// fp16 keeps a bf16 value's 8 significant bits down to 2^-14 as a normal
// number and down to 2^-17 as a subnormal (step 2^-24); smaller values are
// rounded to that 2^-24 grid (an error of at most 2^-25)
__device__ __forceinline__ unsigned bf2_to_h2(unsigned w) {
    return (unsigned)pack2<f16>(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
}

// |bf16| bit patterns. A tile takes the fp16 PV product when its largest
// |v| (its scale) lies in [kF16Scale, kF16Hi): every value from 2^-17 up
// then converts exactly, and a smaller one is off by at most 2^-25 = 2^-17
// of the scale (bf16's own step is 2^-8 of a value), an absolute error of
// at most 2^-25 in the output, whose weights sum to 1. A tile whose values
// are all small (a scaled-down V) takes the bf16 split product, exact in
// V, so its outputs keep their relative precision. Inf and NaN are above
// kF16Hi.
constexpr unsigned kF16Scale = 0x3B80u;  // 2^-8
constexpr unsigned kF16Hi = 0x4780u;     // 2^16

// running maximum of the |v| bit patterns of two bf16 lanes
typedef unsigned short us2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void f16_range_acc(unsigned w, us2_t& mx) {
    mx = __builtin_elementwise_max(mx, __builtin_bit_cast(us2_t, w & 0x7fff7fffu));
}
// the workgroup's vote (every thread calls it): whether the tile whose
// pieces the threads' mx cover takes the fp16 product
__device__ __forceinline__ bool f16_tile_ok(us2_t mx) {
    const unsigned m = mx[0] > mx[1] ? mx[0] : mx[1];
    const int too_big = __syncthreads_or(m >= kF16Hi ? 1 : 0);
    const int has_scale = __syncthreads_or(m >= kF16Scale ? 1 : 0);
    return !too_big && has_scale;
}

// maximum over lanes l, l ^ 16, l ^ 32, l ^ 48 without LDS: with both
// operands x, v_permlane32_swap leaves x[l] and x[l ^ 32] in the two
// results of every lane (lanes < 32: (x[l], x[l + 32]); lanes >= 32:
// (x[l - 32], x[l])), v_permlane16_swap likewise x[l] and x[l ^ 16]
__device__ __forceinline__ float max4_rows(float x) {
    const unsigned u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const unsigned w = __float_as_uint(y);
    const auto c = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}

// V of bf16 inputs converted to fp16 once per call (one workgroup per
// 64-key tile of a (b, kv head) slab), with a flag per tile: 1 when the
// tile's largest |v| is in [2^-8, 2^16) (f16_tile_ok: the tile then takes
// the fp16 PV product). The attention kernel then stages those tiles
// as they are, instead of converting and voting in every one of the
// workgroups that read the tile (Hq / Hkv heads x S / 128 query tiles).
__global__ __launch_bounds__(256) void prefill_v_to_f16(const bf16* __restrict__ v,
                                                        f16* __restrict__ v16,
                                                        unsigned char* __restrict__ ok, int seq,
                                                        int dim, int nkt) {
    typedef unsigned short us2 __attribute__((ext_vector_type(2)));
    const int slab = blockIdx.x / nkt, kt = blockIdx.x - (blockIdx.x / nkt) * nkt;
    const size_t base = ((size_t)slab * seq + (size_t)kt * kPKV) * dim;
    const int rows = min(kPKV, seq - kt * kPKV);
    const int nchunk = rows * dim / 8;  // 16-byte chunks
    us2_t mx = {0, 0};
    for (int c = threadIdx.x; c < nchunk; c += 256) {
        i32x4_t x = *reinterpret_cast<const i32x4_t*>(v + base + 8 * (size_t)c);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            f16_range_acc((unsigned)x[w], mx);
            x[w] = (int)bf2_to_h2((unsigned)x[w]);
        }
        *reinterpret_cast<i32x4_t*>(v16 + base + 8 * (size_t)c) = x;
    }
    const bool fits = f16_tile_ok(mx);
    if (threadIdx.x == 0) ok[blockIdx.x] = fits ? 1 : 0;
}

// PRE (bf16 inputs): v16 / v_ok hold prefill_v_to_f16's output; the fp16 PV
// tiles are staged from v16 without conversion and chosen by v_ok instead of
// a workgroup vote (the same tiles, the same bits)
template <typename T, int D, bool PRE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_prefill_mfma(const T* __restrict__ q, const T* __restrict__ k,
                       const T* __restrict__ v, T* __restrict__ out, int batch,
                       int hq, int hkv, int seq, int causal, float scale_log2,
                       const f16* __restrict__ v16, const unsigned char* __restrict__ v_ok) {
    using M = PMma<T>;
    using V8 = typename M::v8;
    using C = PCfg<D>;
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    // bf16 inputs: P and V go through an fp16 PV product (P rounded to 11
    // significant bits) on every tile whose largest |v| is in [2^-8, 2^16)
    // (f16_tile_ok), bf16 hi + lo P otherwise
    constexpr bool kF16PV = std::is_same<T, bf16>::value;
    __shared__ __attribute__((aligned(16))) char smem[2 * C::kStage];

    const int nqt = (seq + kPQ - 1) / kPQ;
    const int nbh = batch * hq;
    const int qt = nqt - 1 - (int)(blockIdx.x / (unsigned)nbh);
    const int bh = (int)(blockIdx.x % (unsigned)nbh);
    const int b = bh / hq, h = bh - b * hq;
    const int kvh = h / (hq / hkv);
    const int q0 = qt * kPQ;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;

    const T* qh = q + ((size_t)b * hq + h) * seq * D;
    const T* kh = k + ((size_t)b * hkv + kvh) * seq * D;
    const T* vh = v + ((size_t)b * hkv + kvh) * seq * D;
    // the slab's fp16 copy (same element offsets) and tile flags
    const T* vh16 = PRE ? reinterpret_cast<const T*>(v16 + ((size_t)b * hkv + kvh) * seq * D)
                        : vh;
    const unsigned char* okh = PRE ? v_ok + ((size_t)b * hkv + kvh) * ((seq + kPKV - 1) / kPKV)
                                   : nullptr;

    // the wave's Q as B operands: row q0 + 32 wave + 16 qb + r16, elements
    // 32 s + 8 g .. +7 (rows past S read row S - 1; never stored)
    V8 qf[2][C::kS];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int row = min(q0 + 32 * wave + 16 * qb + r16, seq - 1);
#pragma unroll
        for (int s = 0; s < C::kS; ++s)
            qf[qb][s] = *reinterpret_cast<const V8*>(qh + (size_t)row * D + 32 * s + 8 * g);
    }

    const int nkv_all = (seq + kPKV - 1) / kPKV;
    const int nkt = causal ? min(nkv_all, min(q0 + kPQ - 1, seq - 1) / kPKV + 1) : nkv_all;

    // ---- staging: K and V rows as they are (V as fp16 on the fp16 PV path) -
    i32x4_t kreg[C::kKChunks], vreg[C::kKChunks];
    // from16: the tile's fp16 copy (PRE)
    auto load_tile = [&](int kt, bool from16) {
        const int kv0 = kt * kPKV;
        const T* vsrc = from16 ? vh16 : vh;
#pragma unroll
        for (int j = 0; j < C::kKChunks; ++j) {
            const int c = tid + 256 * j;
            const int row = min(kv0 + c / (D / 8), seq - 1);
            kreg[j] = *reinterpret_cast<const i32x4_t*>(kh + (size_t)row * D + 8 * (c % (D / 8)));
            vreg[j] = *reinterpret_cast<const i32x4_t*>(vsrc + (size_t)row * D + 8 * (c % (D / 8)));
        }
    };
    // f16v (bf16 inputs): V stored as fp16 for the fp16 PV product
    auto store_tile = [&](int st, bool f16v) {
        char* ks = smem + st * C::kStage;
        char* vs = ks + kPKV * C::kKPitch;
#pragma unroll
        for (int j = 0; j < C::kKChunks; ++j) {
            const int c = tid + 256 * j;
            const int off = (c / (D / 8)) * C::kKPitch + 16 * (c % (D / 8));
            *reinterpret_cast<i32x4_t*>(ks + off) = kreg[j];
            i32x4_t vv = vreg[j];
            if (kF16PV && !PRE && f16v) {
#pragma unroll
                for (int w = 0; w < 4; ++w) vv[w] = (int)bf2_to_h2((unsigned)vv[w]);
            }
            *reinterpret_cast<i32x4_t*>(vs + off) = vv;
        }
    };

    f32x4 o[C::kDB][2];
#pragma unroll
    for (int db = 0; db < C::kDB; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.f, 0.f};  // lane partial row sums (bf16 split loop)
    // row sums on the matrix core where P is one fp16 operand: ones . P^T
    // puts the sum of the tile's (fp16) weights of row q in every C slot of
    // lane (q, g); rescaled with the output
    f32x4 osum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const int wrow0 = q0 + 32 * wave;  // first query row of this wave
    const float lazy_raw = kLazy / scale_log2;

    // whether the V tile in vreg takes the fp16 product (f16_tile_ok, a
    // workgroup vote: every thread must call it)
    auto v_fits_f16 = [&]() {
        us2_t mx = {0, 0};
#pragma unroll
        for (int j = 0; j < C::kKChunks; ++j)
#pragma unroll
            for (int w = 0; w < 4; ++w) f16_range_acc((unsigned)vreg[j][w], mx);
        return f16_tile_ok(mx);
    };

    bool f16_first;
    if constexpr (PRE) {
        f16_first = okh[0] != 0;
        load_tile(0, f16_first);
    } else {
        load_tile(0, false);
        f16_first = kF16PV && v_fits_f16();
    }
    store_tile(0, f16_first);
    __syncthreads();
    // Tiles kt0 .. : the fp16 PV loop (F16) runs while each next tile votes
    // in range and hands over at the first one that does not (staged in
    // bf16); the bf16 loop then runs to the end. Two separate loops, so that
    // neither path's temporaries are live in the other.
    auto run = [&](auto f16_tag, int kt0) -> int {
        constexpr bool F16 = decltype(f16_tag)::value;
        constexpr bool kMmaSum = F16 || !M::kSplit;
        for (int kt = kt0; kt < nkt; ++kt) {
            // PRE: the next tile's flag picks its source before the load
            const bool pre_next = PRE && F16 && kt + 1 < nkt && okh[kt + 1] != 0;
            if (kt + 1 < nkt) load_tile(kt + 1, pre_next);
            const int kv0 = kt * kPKV;
            const bool active = !causal || kv0 <= wrow0 + 31;
            if (active) {
                const char* ks = smem + (kt & 1) * C::kStage;
                const char* vs = ks + kPKV * C::kKPitch;
                // V^T fragment (16 d rows from d0, keys 32 ks2 + slots): two
                // transposing reads, keys 4g + (0..3) and 16 + 4g + (0..3)
                auto vt_frag = [&](int d0, int ks2) {
                    typedef short v4s __attribute__((ext_vector_type(4)));
                    const char* p = vs + (32 * ks2 + 4 * g + (r16 >> 2)) * C::kKPitch +
                                    (d0 + 4 * (r16 & 3)) * 2;
                    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s*)(p));
                    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s*)(p + 16 * C::kKPitch));
                    typedef short v8s __attribute__((ext_vector_type(8)));
                    return v8s{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                };
                // Wave priorities: the matrix-core phases (scores, PV) issue
                // at the base level, the softmax chain and the staging +
                // barrier at level 1, so a SIMD's other wave, when it reaches
                // those, runs them ahead of this wave's MFMA stream (the MFMAs
                // then fill the gaps). Same-box A/B, S = 4096: bidirectional
                // 288-289 against 306-312 us, causal 160-163 against 175-176;
                // priority on the MFMA phases instead: 302 us.
                __builtin_amdgcn_s_setprio(0);
                // scores S^T for 4 key blocks x 2 query blocks: k-step outer,
                // so the 8 accumulator chains interleave on the matrix core
                // (each chain still sums its k-steps in order)
                f32x4 sc[4][2];
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    sc[kb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
                    sc[kb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int s = 0; s < C::kS; ++s) {
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb) {
                        const V8 kf = *reinterpret_cast<const V8*>(
                            ks + (16 * kb + r16) * C::kKPitch + (32 * s + 8 * g) * 2);
                        sc[kb][0] = M::mma(kf, qf[0][s], sc[kb][0]);
                        sc[kb][1] = M::mma(kf, qf[1][s], sc[kb][1]);
                    }
                }
                __builtin_amdgcn_s_setprio(1);
                // online softmax per query row, on raw scores (the 1/sqrt(D) *
                // log2(e) factor c > 0 commutes with max and folds into one FMA
                // per score: p = exp2(s c - m c)); masks only on the tiles that
                // cross this wave's diagonal or the sequence end
                const bool need_mask = (causal && kv0 + kPKV - 1 > wrow0) || kv0 + kPKV > seq;
                i32x4_t ph[2][2], pl[2][2];
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    float mt = -INFINITY;
                    if (need_mask) {
                        const int qrow = wrow0 + 16 * qb + r16;
#pragma unroll
                        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int key = kv0 + 16 * kb + 4 * g + i;
                                const bool valid = key < seq && (!causal || key <= qrow);
                                if (!valid) sc[kb][qb][i] = -INFINITY;
                            }
                    }
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                        for (int i = 0; i < 4; ++i) mt = fmaxf(mt, sc[kb][qb][i]);
                    mt = max4_rows(mt);
                    // lazy rescale: the running maximum moves only when the tile's
                    // exceeds it by more than kLazy / c (weights then stay
                    // <= 2^kLazy); a wave whose rows all keep theirs skips the
                    // output rescale
                    const bool upd = mt > m_run[qb] + lazy_raw;
                    const float m_new = upd ? mt : m_run[qb];
                    const float m_use = m_new == -INFINITY ? 0.f : m_new;
                    // v_exp_f32 directly: exp2f's expansion adds a denormal-range
                    // rescale per call; weights below 2^-126 of the row maximum
                    // flush to 0, which changes no sum at float precision
                    const float alpha = __builtin_amdgcn_exp2f((m_run[qb] - m_use) * scale_log2);
                    const float nmc = -m_use * scale_log2;
                    float p[4][4];
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            p[kb][i] = __builtin_amdgcn_exp2f(fmaf(sc[kb][qb][i], scale_log2, nmc));
                    if constexpr (!kMmaSum) {
                        float psum = 0.f;
#pragma unroll
                        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                            for (int i = 0; i < 4; ++i) psum += p[kb][i];
                        l_run[qb] = l_run[qb] * alpha + psum;
                    }
                    m_run[qb] = m_new;
                    if (__builtin_amdgcn_ballot_w64(upd)) {
#pragma unroll
                        for (int db = 0; db < C::kDB; ++db) o[db][qb] *= alpha;
                        osum[qb] *= alpha;
                        // l_run is nonzero only in the bf16 split loop, which
                        // rescales it above
                    }
                    // P^T fragments: dword w of step ks2 holds slots 8g + 2w, +1
#pragma unroll
                    for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
                        for (int w = 0; w < 4; ++w) {
                            const float p0 = p[2 * ks2 + (w >> 1)][2 * (w & 1)];
                            const float p1 = p[2 * ks2 + (w >> 1)][2 * (w & 1) + 1];
                            if constexpr (F16) {
                                ph[qb][ks2][w] = pack2<f16>(p0, p1);
                            } else if constexpr (M::kSplit) {
                                // hi: the top 16 bits (truncation, exact); lo: the
                                // exact remainder rounded to bf16; hi + lo carries
                                // ~16 significant bits of p
                                const unsigned u0 = __float_as_uint(p0), u1 = __float_as_uint(p1);
                                ph[qb][ks2][w] = (int)((u0 >> 16) | (u1 & 0xffff0000u));
                                const float r0 = p0 - __uint_as_float(u0 & 0xffff0000u);
                                const float r1 = p1 - __uint_as_float(u1 & 0xffff0000u);
                                pl[qb][ks2][w] = pack2<T>(r0, r1);
                            } else {
                                ph[qb][ks2][w] = pack2<T>(p0, p1);
                            }
                        }
                }
                __builtin_amdgcn_s_setprio(0);
                // O^T += V^T . P^T (and the row sums: ones . P^T)
                if constexpr (kMmaSum) {
                    const h8 ones = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f,
                                     (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f,
                                     (_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
                    for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
                        for (int qb = 0; qb < 2; ++qb)
                            osum[qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                ones, __builtin_bit_cast(h8, ph[qb][ks2]), osum[qb], 0, 0, 0);
                }
                if constexpr (F16) {
#pragma unroll
                    for (int db = 0; db < C::kDB; ++db)
#pragma unroll
                        for (int ks2 = 0; ks2 < 2; ++ks2) {
                            const h8 vf = __builtin_bit_cast(h8, vt_frag(16 * db, ks2));
#pragma unroll
                            for (int qb = 0; qb < 2; ++qb)
                                o[db][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    vf, __builtin_bit_cast(h8, ph[qb][ks2]), o[db][qb], 0, 0, 0);
                        }
                } else {
#pragma unroll
                    for (int db = 0; db < C::kDB; ++db)
#pragma unroll
                        for (int ks2 = 0; ks2 < 2; ++ks2) {
                            const V8 vf = __builtin_bit_cast(V8, vt_frag(16 * db, ks2));
#pragma unroll
                            for (int qb = 0; qb < 2; ++qb) {
                                o[db][qb] = M::mma(vf, __builtin_bit_cast(V8, ph[qb][ks2]), o[db][qb]);
                                if constexpr (M::kSplit)
                                    o[db][qb] = M::mma(vf, __builtin_bit_cast(V8, pl[qb][ks2]),
                                                       o[db][qb]);
                            }
                        }
                }
            }
            __builtin_amdgcn_s_setprio(1);
            if (kt + 1 < nkt) {
                const bool next_f16 = PRE ? pre_next : F16 && v_fits_f16();
                store_tile((kt + 1) & 1, next_f16);
                __syncthreads();
                if (F16 && !next_f16) return kt + 1;
            } else {
                __syncthreads();
            }
        }
        return nkt;
    };
    int kt_split = 0;
    if constexpr (kF16PV) {
        if (f16_first) kt_split = run(std::true_type{}, 0);
    }
    run(std::false_type{}, kt_split);

    // normalise and store: lane (q, g) holds d = 16 db + 4 g + i of row q
    T* oh = out + ((size_t)b * hq + h) * seq * D;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        float l = l_run[qb];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        l += osum[qb][0];
        const float inv = 1.0f / l;
        const int qrow = wrow0 + 16 * qb + r16;
        if (qrow >= seq) continue;
#pragma unroll
        for (int db = 0; db < C::kDB; ++db)
            St<T>::st4(oh + (size_t)qrow * D + 16 * db + 4 * g,
                       make_float4(o[db][qb][0] * inv, o[db][qb][1] * inv,
                                   o[db][qb][2] * inv, o[db][qb][3] * inv));
    }
}

// one wave per (b, q head, query row); lanes hold float4 chunks c = lane,
// lane + 64 of D
template <typename T>
__global__ __launch_bounds__(64) void attn_prefill_generic(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    T* __restrict__ out, int hq, int hkv, int seq, int dim, int causal, float scale) {
    const long long id = blockIdx.x;
    const int i = (int)(id % seq);
    const long long bh = id / seq;
    const int h = (int)(bh % hq);
    const long long b = bh / hq;
    const int kvh = h / (hq / hkv);
    const int lane = threadIdx.x;
    const int nc = dim / 4;
    const T* qr = q + ((size_t)bh * seq + i) * dim;
    const T* kh = k + ((size_t)b * hkv + kvh) * seq * dim;
    const T* vh = v + ((size_t)b * hkv + kvh) * seq * dim;
    const bool c0 = lane < nc, c1 = lane + 64 < nc;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 q0 = c0 ? St<T>::ld4(qr + 4 * lane) : z;
    const float4 q1 = c1 ? St<T>::ld4(qr + 4 * (lane + 64)) : z;
    float4 a0 = z, a1 = z;
    float m = -INFINITY, l = 0.f;
    const int lim = causal ? i + 1 : seq;
    for (int t = 0; t < lim; ++t) {
        const T* kr = kh + (size_t)t * dim;
        float d = 0.f;
        if (c0) {
            const float4 kk = St<T>::ld4(kr + 4 * lane);
            d = q0.x * kk.x + q0.y * kk.y + q0.z * kk.z + q0.w * kk.w;
        }
        if (c1) {
            const float4 kk = St<T>::ld4(kr + 4 * (lane + 64));
            d += q1.x * kk.x + q1.y * kk.y + q1.z * kk.z + q1.w * kk.w;
        }
        const float s = wave_sum(d) * scale;
        const float m_new = fmaxf(m, s);
        const float a = expf(m - m_new);
        const float p = expf(s - m_new);
        l = l * a + p;
        m = m_new;
        const T* vr = vh + (size_t)t * dim;
        if (c0) {
            const float4 vv = St<T>::ld4(vr + 4 * lane);
            a0 = make_float4(a0.x * a + p * vv.x, a0.y * a + p * vv.y,
                             a0.z * a + p * vv.z, a0.w * a + p * vv.w);
        }
        if (c1) {
            const float4 vv = St<T>::ld4(vr + 4 * (lane + 64));
            a1 = make_float4(a1.x * a + p * vv.x, a1.y * a + p * vv.y,
                             a1.z * a + p * vv.z, a1.w * a + p * vv.w);
        }
    }
    const float inv = 1.0f / l;
    T* orow = out + ((size_t)bh * seq + i) * dim;
    if (c0) St<T>::st4(orow + 4 * lane, make_float4(a0.x * inv, a0.y * inv, a0.z * inv, a0.w * inv));
    if (c1)
        St<T>::st4(orow + 4 * (lane + 64),
                   make_float4(a1.x * inv, a1.y * inv, a1.z * inv, a1.w * inv));
}

template <typename T>
void prefill_run(const T* q, const T* k, const T* v, T* out, int batch, int hq, int hkv,
                 int seq, int dim, bool causal, hipStream_t s) {
    if (batch < 0 || hq < 1 || hkv < 1 || seq < 0 || dim < 1)
        inval("attention shapes must satisfy batch>=0, heads>=1, rows>=0, dim>=1");
    if (hq % hkv != 0)
        inval("q heads must be a multiple of kv heads (contiguous GQA groups)");
    if (dim % 4 != 0 || dim > 512) inval("dim must be a multiple of 4 and at most 512");
    if (batch == 0 || seq == 0) return;  // nothing to compute
    if (!q || !k || !v || !out) inval("attention prefill: null operand");
    const float scale = 1.0f / sqrtf((float)dim);
    if constexpr (!std::is_same<T, float>::value) {
        const bool aligned = ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16 == 0;
        if ((dim == 64 || dim == 128) && aligned && !tune(Tune::PrefillForceGeneric, 0)) {
            const long long nqt = (seq + kPQ - 1) / kPQ;
            const long long grid = (long long)batch * hq * nqt;
            if (grid > 0x7fffffffLL) inval("attention prefill problem too large for one launch");
            const float sl2 = scale * kLog2eP;
            // bf16: V to fp16 once per call when the problem is large enough
            // for the extra launch to pay (FT_PREFILL_PREPASS: 0 in the kernel,
            // 2 always)
            const long long vel = (long long)batch * hkv * seq * dim;
            const int nkv = (seq + kPKV - 1) / kPKV;
            const int pp = tune(Tune::PrefillPrepass, 1);  // 0 never, 1 auto, 2 always
            const bool pre = std::is_same<T, bf16>::value &&
                             (pp == 2 || (pp == 1 && vel >= kPrepassMinElems));
            f16* v16 = nullptr;
            unsigned char* v_ok = nullptr;
            if (pre) {
                const size_t vbytes = ((size_t)vel * 2 + 255) & ~(size_t)255;
                char* ws = (char*)scratch(Scratch::PrefillV,
                                          vbytes + (size_t)batch * hkv * nkv, s);
                v16 = (f16*)ws;
                v_ok = (unsigned char*)(ws + vbytes);
                prefill_v_to_f16<<<(unsigned)((long long)batch * hkv * nkv), 256, 0, s>>>(
                    (const bf16*)v, v16, v_ok, seq, dim, nkv);
                launch_check("attention prefill V conversion launch");
            }
#define FT_PF(DD, PP)                                                                 \
    attn_prefill_mfma<T, DD, PP><<<(unsigned)grid, 256, 0, s>>>(                      \
        q, k, v, out, batch, hq, hkv, seq, causal ? 1 : 0, sl2, v16, v_ok)
            if (dim == 128) {
                if (pre) FT_PF(128, true); else FT_PF(128, false);
            } else {
                if (pre) FT_PF(64, true); else FT_PF(64, false);
            }
#undef FT_PF
            launch_check("attention prefill kernel launch");
            return;
        }
    }
    const long long grid = (long long)batch * hq * seq;
    if (grid > 0x7fffffffLL) inval("attention prefill problem too large for one launch");
    attn_prefill_generic<T><<<(unsigned)grid, 64, 0, s>>>(q, k, v, out, hq, hkv, seq, dim,
                                                          causal ? 1 : 0, scale);
    launch_check("attention prefill kernel launch");
}

}  // namespace
}  // namespace ft

extern "C" {

int ft_attention_prefill_launch(const float* q, const float* k, const float* v, float* out,
                                int batch, int q_heads, int kv_heads, int seq, int dim,
                                int causal, uintptr_t stream) {
    return ft::guarded([&] {
        ft::prefill_run<float>(q, k, v, out, batch, q_heads, kv_heads, seq, dim, causal != 0,
                               ft::as_stream(stream));
    });
}

int ft_attention_prefill_launch_bf16(const void* q, const void* k, const void* v, void* out,
                                     int batch, int q_heads, int kv_heads, int seq, int dim,
                                     int causal, uintptr_t stream) {
    return ft::guarded([&] {
        ft::prefill_run<ft::bf16>((const ft::bf16*)q, (const ft::bf16*)k, (const ft::bf16*)v,
                                  (ft::bf16*)out, batch, q_heads, kv_heads, seq, dim,
                                  causal != 0, ft::as_stream(stream));
    });
}

int ft_attention_prefill_launch_fp16(const void* q, const void* k, const void* v, void* out,
                                     int batch, int q_heads, int kv_heads, int seq, int dim,
                                     int causal, uintptr_t stream) {
    return ft::guarded([&] {
        ft::prefill_run<ft::f16>((const ft::f16*)q, (const ft::f16*)k, (const ft::f16*)v,
                                 (ft::f16*)out, batch, q_heads, kv_heads, seq, dim,
                                 causal != 0, ft::as_stream(stream));
    });
}

}  // extern "C"
