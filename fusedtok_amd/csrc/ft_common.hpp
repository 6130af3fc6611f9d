// Shared host/device plumbing for the gfx950 decode-path kernels.
//
// Host side: the status/error model of the C ABI (FT_OK / FT_EINVAL /
// FT_EHIP with a thread-local message), HIP error checks, cached device
// properties and the per-device scratch pool.
// Device side: storage-type traits (f32 / bf16 / fp16 widened to f32 at
// load, narrowed round-to-nearest-even at store) and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "../../include/fusedtok_amd.h"

namespace ft {

// ---------------------------------------------------------------------------
// host: error model
// ---------------------------------------------------------------------------

struct Error {
    int code;
    std::string msg;
};

[[noreturn]] inline void inval(const std::string& msg) {
    throw Error{FT_EINVAL, msg};
}

[[noreturn]] inline void hip_fail(const std::string& what, hipError_t e) {
    throw Error{FT_EHIP, what + ": " + hipGetErrorString(e)};
}

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) hip_fail(what, e);
}

// After a kernel launch: surface launch-configuration errors.
inline void launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) hip_fail(what, e);
}

void set_error(const std::string& msg);
void clear_error();

// Wrap a C-ABI body: exceptions never cross the ABI.
template <typename F>
int guarded(F&& body) {
    try {
        body();
        clear_error();
        return FT_OK;
    } catch (const Error& e) {
        set_error(e.msg);
        return e.code;
    } catch (const std::bad_alloc&) {
        set_error("host allocation failed");
        return FT_EHIP;
    } catch (const std::exception& e) {
        set_error(e.what());
        return FT_EHIP;
    } catch (...) {
        set_error("unknown error");
        return FT_EHIP;
    }
}

inline hipStream_t as_stream(uintptr_t s) {
    return reinterpret_cast<hipStream_t>(s);
}

// Device properties of the current device, cached per device id.
struct DevInfo {
    int id = 0;
    int cu_count = 256;
};
const DevInfo& dev_info();

// True if `s` is being captured into a HIP graph.
bool stream_capturing(hipStream_t s);

// Tuning and test switches. Each is read once per process, on first use,
// from the environment variable of the same name, and can be overridden at
// run time through ft_set_tuning() / ft_clear_tuning() (tests, sweeps). The
// defaults are the measured-fastest paths; no switch changes a result
// beyond the op's stated tolerance (the integer paths not at all).
enum class Tune : int {
    AttnForceGeneric = 0,  // FT_ATTN_FORCE_GENERIC: decode on the generic kernel
    AttnSegs,              // FT_ATTN_SEGS: stream-split segment count
    AttnMinSeg,            // FT_ATTN_MIN_SEG: minimum tokens per segment
    AttnChunk,             // FT_ATTN_CHUNK: generic kernel's chunk
    QgemmKernel,           // FT_QGEMM_KERNEL: force 1 skinny .. 6 decode
    QgemmDecKw,            // FT_QGEMM_DEC_KW: waves per decode column tile
    QgemmDecRegs,          // FT_QGEMM_DEC_REGS: register-operand decode kernel
    QgemmKsplit,           // FT_QGEMM_KSPLIT: skinny kernel K split
    QgemmSkRegs,           // FT_QGEMM_SK_REGS: register-operand skinny kernel
    QgemmSkWaves,          // FT_QGEMM_SK_WAVES: 4 or 8 waves (64 / 128 columns)
    QgemmSkStages,         // FT_QGEMM_SK_STAGES: LDS ring depth, 2 or 3
    QgemmBig,              // FT_QGEMM_BIG: 1 64-byte DMA slabs, 2 register-staged
    QgemmBand,             // FT_QGEMM_BAND: big-tile band height
    RmsqSplit,             // FT_RMSQ_SPLIT: rmsnorm_quant in two launches
    RmsqGemvSplit,         // FT_RMSQ_GEMV_SPLIT: rmsnorm_qgemm as two ops
    PrefillForceGeneric,   // FT_PREFILL_FORCE_GENERIC
    ArgSlices,             // FT_ARG_SLICES: argmax_batched slices per row
    SmpSingle,             // FT_SMP_SINGLE: sampling, one workgroup per row
    SmpSlices,             // FT_SMP_SLICES: sampling slices per row
    FailScratch,           // FT_FAIL_SCRATCH (test hook): every scratch request
                           // fails as an allocation failure would
    PrefillPrepass,        // FT_PREFILL_PREPASS: bf16 V to fp16 in a pre-pass
                           // (0 never: in the kernel; 1 large calls; 2 always)
    GridSync,              // FT_GRID_SYNC: bit mask of the per-tensor maxima not
                           // to fold inside one launch (grid_max), which then
                           // take their two-launch forms: 1 all, 2 SwiGLU,
                           // 4 attention output, 8 RMSNorm
    kCount
};
// The switch's value, or `dflt` when it is neither in the environment nor
// set through ft_set_tuning().
int tune(Tune which, int dflt);

// Per-device scratch buffers, one per purpose, grown on demand and kept for
// the process lifetime. Growth is refused during a stream capture (the
// caller must warm the shape up once outside the capture). Returned memory
// is uninitialised.
enum class Scratch : int {
    AttnPartials = 0,
    QuantMax = 1,
    GemmPartials = 2,
    Sampling = 3,
    PrefillV = 4,
    GridSync = 5,  // grid_max state (gridmax_state)
    AttnLens = 6,  // lens + 1 of the two-op form of the appending decode
    kCount = 7
};
void* scratch(Scratch which, size_t bytes, hipStream_t s);
// Same, but memory is zero when first allocated (or re-allocated); kernels
// that use it must leave it zero when they finish (e.g. arrival counters).
void* scratch_zeroed(Scratch which, size_t bytes, hipStream_t s);

// ---------------------------------------------------------------------------
// Grid-wide maximum inside one launch (grid_max below). The state is one
// 64-bit word (generation << 32 | arrivals) and one 32-bit slot per
// workgroup, zeroed when allocated; every launch leaves the arrivals at 0.
// Launches that use it are ordered on one stream: calls that overlap on one
// GPU race, as with the library's other scratch.
struct GridMax {
    unsigned long long* word;
    unsigned* slots;
};
// The state for up to `nwg` workgroups on the current device (grown outside
// a capture only, like scratch()). runtime.hip.
GridMax gridmax_state(int nwg, hipStream_t s);
// True when `nwg` workgroups of `kernel` (`threads` each, no dynamic LDS)
// can all be resident at once on the current device, and FT_GRID_SYNC does
// not turn off the in-launch maximum of this kind (GridUse). runtime.hip.
enum class GridUse : int { SwiGLU = 2, AttnOut = 4, RmsNorm = 8 };
bool grid_resident(const void* kernel, int nwg, int threads, GridUse use);

// Per-tensor int8 quantize of x[0, n) (T = float, bf16, f16) when its max |x|
// is already known as the max of nparts partial maxima (written by the
// producer of x): one launch, codes and *scale_out (device) as quantize_int8
// computes them. quantize.hip.
template <typename T>
void quantize_from_partials(const T* x, signed char* q, const float* partial, int nparts,
                            float* scale_out, long long n, hipStream_t s);
// The whole quantize_int8 (two launches above 64K elements). quantize.hip.
template <typename T>
void quantize_tensor(const T* x, signed char* q, float* scale_out, long long n,
                     hipStream_t s);

// QKV GEMM (K-split partials folded by the RoPE kernel) + RoPE + paged KV
// append, as ft_qgemm_rope_kv_append_paged_launch; lens_next (optional)
// receives lens[b] + 1 from the same kernel. fused.hip.
void qkv_rope_step(int dtype, const signed char* a_q, const float* sa_dev,
                   const signed char* w_q, const float* w_scales, int k, void* qkv,
                   const int* lens, int* lens_next, const int* table, void* q_out,
                   void* k_pool, void* v_pool, int batch, int hq, int hkv, int dim, int page,
                   int tbl_width, float theta, int pos_offset, bool neox, hipStream_t s);

// ---------------------------------------------------------------------------
// device: storage traits
// ---------------------------------------------------------------------------

using bf16 = __bf16;
using f16 = _Float16;

template <typename T> struct St;

template <> struct St<float> {
    __device__ __forceinline__ static float ld(const float* p) { return *p; }
    __device__ __forceinline__ static void st(float* p, float v) { *p = v; }
    __device__ __forceinline__ static float4 ld4(const float* p) {
        return *reinterpret_cast<const float4*>(p);
    }
    __device__ __forceinline__ static void st4(float* p, float4 v) {
        *reinterpret_cast<float4*>(p) = v;
    }
};

template <> struct St<bf16> {
    __device__ __forceinline__ static float ld(const bf16* p) {
        return (float)*p;
    }
    __device__ __forceinline__ static void st(bf16* p, float v) {
        *p = (bf16)v;
    }
    __device__ __forceinline__ static float4 ld4(const bf16* p) {
        typedef bf16 v4 __attribute__((ext_vector_type(4)));
        const v4 u = *reinterpret_cast<const v4*>(p);
        return make_float4((float)u[0], (float)u[1], (float)u[2],
                           (float)u[3]);
    }
    __device__ __forceinline__ static void st4(bf16* p, float4 v) {
        typedef bf16 v4 __attribute__((ext_vector_type(4)));
        v4 u;
        u[0] = (bf16)v.x; u[1] = (bf16)v.y; u[2] = (bf16)v.z; u[3] = (bf16)v.w;
        *reinterpret_cast<v4*>(p) = u;
    }
};

template <> struct St<f16> {
    __device__ __forceinline__ static float ld(const f16* p) {
        return (float)*p;
    }
    __device__ __forceinline__ static void st(f16* p, float v) {
        *p = (f16)v;
    }
    __device__ __forceinline__ static float4 ld4(const f16* p) {
        typedef f16 v4 __attribute__((ext_vector_type(4)));
        const v4 u = *reinterpret_cast<const v4*>(p);
        return make_float4((float)u[0], (float)u[1], (float)u[2],
                           (float)u[3]);
    }
    __device__ __forceinline__ static void st4(f16* p, float4 v) {
        typedef f16 v4 __attribute__((ext_vector_type(4)));
        v4 u;
        u[0] = (f16)v.x; u[1] = (f16)v.y; u[2] = (f16)v.z; u[3] = (f16)v.w;
        *reinterpret_cast<v4*>(p) = u;
    }
};

// ---------------------------------------------------------------------------
// device: wave64 reductions (butterfly over all 64 lanes)
// ---------------------------------------------------------------------------

// Per-tensor int8 quantisation (reference quantize.cu:169-186): scale =
// max|x| / 127 (1 when every value is 0); code = clamp(rint(x * inv), -127,
// 127) with inv = 1 / scale.
__device__ __forceinline__ float make_scale(float absmax) {
    return absmax > 0.0f ? absmax / 127.0f : 1.0f;
}

// max |v| of 4 values as they are stored in T (rounded to nearest-even):
// the quantity a later per-tensor quantize of the stored tensor folds
template <typename T>
__device__ __forceinline__ float stored_absmax4(float4 v) {
    return fmaxf(fmaxf(fabsf((float)(T)v.x), fabsf((float)(T)v.y)),
                 fmaxf(fabsf((float)(T)v.z), fabsf((float)(T)v.w)));
}

__device__ __forceinline__ signed char quant1(float x, float inv) {
    return (signed char)fmaxf(-127.0f, fminf(127.0f, rintf(x * inv)));
}

// SwiGLU of one element, silu(g) * u = g / (1 + e^-g) * u (reference
// activations.cu:68-72, 501-511). One definition for swiglu_quant and for
// the gate/up GEMM epilogue that takes its maximum, so both round alike.
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g / (1.0f + expf(-g)) * u;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Ordering point for data one wave's lanes exchange through LDS (a lane
// reads what another lane of the same wave wrote, or overwrites what
// another lane read). The hardware executes a wave's LDS instructions in
// issue order, so no barrier instruction is needed; the wavefront-scope
// release/acquire pair and the wave barrier tell the compiler that LDS
// accesses may not move across this point, which per-lane alias analysis
// alone would allow when it can prove one lane's addresses distinct. The
// fences name the local address space only: global loads (a kernel's
// prefetches) stay free to move across (decode attention, config 3: 1%
// faster than fences over every address space).
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Block-wide reductions for blockDim.x == NT (multiple of 64). `red` is
// LDS scratch of at least NT/64 floats. Every thread gets the result.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) t += red[i];
    __syncthreads();
    return t;
}

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) t = fmaxf(t, red[i]);
    __syncthreads();
    return t;
}

// Maximum over every workgroup of the launch of each workgroup's `m` (>= 0,
// the same in all NT threads of the workgroup), returned to every thread.
// All workgroups must be resident at once (grid_resident). Values cross
// workgroups only through device-scope atomics, which every XCD performs at
// one coherence point, so no release fence (an L2 writeback per workgroup,
// ~0.2 us each, serialised per XCD) is needed:
//   1. exchange m into this workgroup's slot and wait until it is performed;
//   2. arrive (add 1 to the word); the last arriver advances the generation
//      and clears the arrivals with one add, the others poll the word until
//      the generation moves (bounded: after kGridSpin polls, ~1 s, a
//      workgroup goes on with the slots as they are, so a misuse gives wrong
//      values and never a hang);
//   3. every slot now holds this launch's value: read them all.
constexpr unsigned kGridSpin = 1u << 20;

template <int NT>
__device__ __forceinline__ float grid_max(const GridMax& g, float m, float* red) {
    const unsigned nwg = gridDim.x * gridDim.y * gridDim.z;
    const unsigned wg = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_exchange(g.slots + wg, __float_as_uint(m),
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // the exchange has returned (so it was performed) before the arrival
        asm volatile("s_waitcnt vmcnt(0)" : : "v"(prev) : "memory");
        const unsigned long long old = __hip_atomic_fetch_add(
            g.word, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned gen = (unsigned)(old >> 32);
        if ((unsigned)old + 1u == nwg) {
            __hip_atomic_fetch_add(g.word, (1ull << 32) - nwg, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        } else {
            for (unsigned i = 0; i < kGridSpin; ++i) {
                const unsigned long long cur =
                    __hip_atomic_load(g.word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((unsigned)(cur >> 32) != gen) break;
                __builtin_amdgcn_s_sleep(8);
            }
        }
    }
    __syncthreads();
    float mx = 0.0f;
    for (unsigned i = threadIdx.x; i < nwg; i += NT)
        mx = fmaxf(mx, __uint_as_float(__hip_atomic_load(g.slots + i, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT)));
    return block_max<NT>(mx, red);
}

inline unsigned grid_1d(long long n, int per_block, int cap = 1 << 20) {
    long long g = (n + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

}  // namespace ft
