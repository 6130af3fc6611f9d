/*
 * fusedtok_amd.h - C ABI of the MI355X (gfx950) decode hot path.
 *
 * Every entry point here replaces one launcher of the reference kernel
 * library (fusedtok 2.5.0, include/fusedtok/cuda_launch.hpp); the
 * reference declaration each one stands in for is cited beside it, and the
 * argument order is the reference's.
 *
 * Contract (all entry points):
 *   - Pointers are device pointers owned by the caller (HIP allocations,
 *     e.g. torch tensors' data_ptr()). Nothing here takes ownership.
 *   - `stream` is a hipStream_t passed as an integer (0 = null stream).
 *     Launchers are asynchronous and stream-ordered; none synchronises
 *     the host (unlike the reference's quantize_int8_launch, which reads
 *     the absmax back mid-call: quantize.cu:195-215).
 *   - Return value: FT_OK, FT_EINVAL (bad shape/argument: the reference's
 *     std::invalid_argument -> Python ValueError) or FT_EHIP (HIP runtime
 *     failure: the reference's std::runtime_error -> Python RuntimeError).
 *     ft_last_error() returns the calling thread's last message.
 *   - Argument validation happens on the host before any HIP call, so the
 *     FT_EINVAL paths can be exercised without a GPU.
 *   - bf16/fp16 entry points take `void*` storage; every accumulator and
 *     softmax state stays float32 (reference: attention.cu:30-37).
 *   - Library-owned device scratch (attention split partials, quantize
 *     partial maxima) is allocated once per device on first use and kept
 *     for the process lifetime. Concurrent calls on different streams of
 *     one device share it and must be serialised by the caller (the same
 *     rule as the reference: cuda_launch.hpp:185-190). Warm a shape up
 *     once outside a HIP graph capture before capturing it.
 */
#ifndef FUSEDTOK_AMD_H
#define FUSEDTOK_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FT_OK = 0,
    FT_EINVAL = 1, /* invalid argument: ValueError */
    FT_EHIP = 2    /* HIP runtime failure: RuntimeError */
};

/* Output element types for the build's extra-dtype entry points. */
enum {
    FT_DT_F32 = 0,
    FT_DT_BF16 = 1,
    FT_DT_F16 = 2
};

/* Message of the last failing call on this thread ("" if none). */
const char* ft_last_error(void);

/* 1 if a usable HIP device is present. Replaces cuda_available()
 * (src/fusedtok.cu:34-37). */
int ft_device_available(void);

/* Library version string. */
const char* ft_version(void);

/* Device address of pinned host memory (hipHostMalloc, torch's          */
/* pin_memory=True), so that a launcher can read small host-staged      */
/* vectors in place instead of waiting on a copy; FT_EINVAL when the    */
/* runtime reports no device mapping. Build addition with no reference */
/* counterpart, for callers that stage per-call vectors (the samplers'  */
/* histories, offsets and seeds).                                       */
int ft_host_device_address(const void* host, void** dev);

/* Build addition (tests and measurement sweeps; no reference counterpart):
 * tuning switches. Each FT_* switch (FT_ATTN_SEGS, FT_QGEMM_KERNEL, ...) is
 * read from the environment once per process, on first use;
 * ft_set_tuning overrides its value for the rest of the process and
 * ft_clear_tuning restores the environment's value (or unset). An unknown
 * name is FT_EINVAL. No switch changes a result beyond the op's stated
 * tolerance (integer results not at all). */
int ft_set_tuning(const char* name, int value);
int ft_clear_tuning(const char* name);

/* ------------------------------------------------------------------ */
/* Attention, decode step, contiguous cache                            */
/* out[b,h] = softmax(q[b,h] . K[b,h/G]^T / sqrt(D)) . V[b,h/G]         */
/* q [B,Hq,D], k/v [B,Hkv,T,D], lens [B] or NULL, out [B,Hq,D].         */
/* Replaces attention_decode_launch{,_bf16,_fp16}                       */
/* (cuda_launch.hpp:336-359; attention.cu:1468-1585).                   */
/* ------------------------------------------------------------------ */
int ft_attention_decode_launch(const float* q, const float* k,
                               const float* v, const int* lens, float* out,
                               int batch, int q_heads, int kv_heads,
                               int cache_rows, int dim, uintptr_t stream);
int ft_attention_decode_launch_bf16(const void* q, const void* k,
                                    const void* v, const int* lens,
                                    void* out, int batch, int q_heads,
                                    int kv_heads, int cache_rows, int dim,
                                    uintptr_t stream);
int ft_attention_decode_launch_fp16(const void* q, const void* k,
                                    const void* v, const int* lens,
                                    void* out, int batch, int q_heads,
                                    int kv_heads, int cache_rows, int dim,
                                    uintptr_t stream);

/* ------------------------------------------------------------------ */
/* Attention, decode step, paged cache                                 */
/* pools [Nb,Hkv,P,D]; table [B,S] int32; token t of sequence b lives  */
/* at pool[table[b*S + t/P], kv, t%P, :]. GQA group in {1,2,4,8,16}.   */
/* Replaces attention_decode_paged_launch{,_bf16,_fp16}                */
/* (cuda_launch.hpp:397-416; attention.cu:1791-1915).                  */
/* ------------------------------------------------------------------ */
int ft_attention_decode_paged_launch(const float* q, const float* k_pool,
                                     const float* v_pool, const int* table,
                                     const int* lens, float* out, int batch,
                                     int q_heads, int kv_heads, int page,
                                     int tbl_width, int dim,
                                     uintptr_t stream);
int ft_attention_decode_paged_launch_bf16(const void* q, const void* k_pool,
                                          const void* v_pool,
                                          const int* table, const int* lens,
                                          void* out, int batch, int q_heads,
                                          int kv_heads, int page,
                                          int tbl_width, int dim,
                                          uintptr_t stream);
int ft_attention_decode_paged_launch_fp16(const void* q, const void* k_pool,
                                          const void* v_pool,
                                          const int* table, const int* lens,
                                          void* out, int batch, int q_heads,
                                          int kv_heads, int page,
                                          int tbl_width, int dim,
                                          uintptr_t stream);

/* No-allocation variant of ft_attention_decode_paged_launch_bf16. It   */
/* has no counterpart in the reference: it is for callers that cannot   */
/* allocate device memory (code under HIP graph capture, tight serving  */
/* loops, harnesses that forbid hipMalloc). Arguments and results are   */
/* those of ft_attention_decode_paged_launch_bf16, bit for bit; the     */
/* split partials live in a static per-device array of                  */
/* FT_NOALLOC_WORKSPACE_BYTES (16 MiB) instead of the library's growing */
/* buffer, and no hipMalloc, hipFree or other allocating routine is     */
/* called. A call whose partials do not fit returns FT_EINVAL before    */
/* anything is launched. With D = 128 and G = q_heads / kv_heads <= 16  */
/* the need is (2 * CUs + batch * kv_heads) * G * 520 + 8 * (batch + 2) */
/* bytes: 1.6 MB for batch 32 with 32 / 8 heads on 256 CUs; batch 512   */
/* at 32 / 8 heads still fits. Every call on one GPU shares that GPU's  */
/* array, which keeps the last call's contents: calls that overlap on   */
/* one GPU (unordered streams) race and must be serialised.             */
#define FT_NOALLOC_WORKSPACE_BYTES (16u << 20)
int ft_attention_decode_paged_launch_bf16_noalloc(const void* q, const void* k_pool,
                                                  const void* v_pool,
                                                  const int* table, const int* lens,
                                                  void* out, int batch, int q_heads,
                                                  int kv_heads, int page,
                                                  int tbl_width, int dim,
                                                  uintptr_t stream);

/* Build addition (decode step): ft_kv_append_paged_launch(k_new, v_new,
 * table, lens, k_pool, v_pool, ...) followed by
 * ft_attention_decode_paged_launch(q, k_pool, v_pool, table, lens + 1,
 * out, ...) in one call (reference: the two ops, attention.cu:1924-1966
 * then 1785-1900; lens is not modified). dtype FT_DT_F32 / BF16 / F16 for
 * q, the pools, k_new / v_new [batch, kv_heads, dim] and out. For bf16 /
 * fp16 with dim 128 the decode kernel attends the lens[b] cached
 * tokens, and its combine kernel folds the fresh token's
 * score and value into each row's log-sum-exp merge (in float32, so out
 * equals the two ops' within the attention tolerance, not bit for bit)
 * and writes the fresh K / V rows into the pools (equal bit for bit): one
 * launch fewer. Other shapes run the two ops. */
int ft_attention_decode_paged_append_launch(const void* q, void* k_pool, void* v_pool,
                                            const int* table, const void* k_new,
                                            const void* v_new, const int* lens, void* out,
                                            int dtype, int batch, int q_heads, int kv_heads,
                                            int page, int tbl_width, int dim,
                                            uintptr_t stream);

/* ------------------------------------------------------------------ */
/* KV append: one fresh token per sequence written at position lens[b] */
/* k_new/v_new [B,Hkv,D]. In place. Exact copies.                      */
/* Replaces kv_append_paged_launch{,_bf16,_fp16}                       */
/* (cuda_launch.hpp:426-441; attention.cu:1924-1966) and               */
/* kv_append_launch{,_bf16,_fp16} (cuda_launch.hpp:454-467;            */
/* attention.cu:1985-2035).                                            */
/* ------------------------------------------------------------------ */
int ft_kv_append_paged_launch(const float* k_new, const float* v_new,
                              const int* table, const int* lens,
                              float* k_pool, float* v_pool, int batch,
                              int hkv, int dim, int page, int tbl_width,
                              uintptr_t stream);
int ft_kv_append_paged_launch_bf16(const void* k_new, const void* v_new,
                                   const int* table, const int* lens,
                                   void* k_pool, void* v_pool, int batch,
                                   int hkv, int dim, int page, int tbl_width,
                                   uintptr_t stream);
int ft_kv_append_paged_launch_fp16(const void* k_new, const void* v_new,
                                   const int* table, const int* lens,
                                   void* k_pool, void* v_pool, int batch,
                                   int hkv, int dim, int page, int tbl_width,
                                   uintptr_t stream);
int ft_kv_append_launch(const float* k_new, const float* v_new,
                        const int* lens, float* k_cache, float* v_cache,
                        int batch, int hkv, int dim, int t_rows,
                        uintptr_t stream);
int ft_kv_append_launch_bf16(const void* k_new, const void* v_new,
                             const int* lens, void* k_cache, void* v_cache,
                             int batch, int hkv, int dim, int t_rows,
                             uintptr_t stream);
int ft_kv_append_launch_fp16(const void* k_new, const void* v_new,
                             const int* lens, void* k_cache, void* v_cache,
                             int batch, int hkv, int dim, int t_rows,
                             uintptr_t stream);

/* ------------------------------------------------------------------ */
/* Prefill (fresh-sequence) attention: q [B,Hq,S,D] attends over k / v  */
/* [B,Hkv,S,D]; causal != 0 masks query row i to key rows [0, i],      */
/* causal == 0 attends to all S rows; out [B,Hq,S,D] in q's dtype,     */
/* float32 softmax and accumulators. Same GQA grouping and D contract  */
/* as decode (D % 4 == 0, D <= 512). No workspace; capturable.         */
/* Replaces attention_prefill_launch{,_bf16,_fp16}                     */
/* (cuda_launch.hpp:362-378; attention.cu:1649-1739); causal is an int */
/* here (bool in the reference).                                       */
/* ------------------------------------------------------------------ */
int ft_attention_prefill_launch(const float* q, const float* k, const float* v,
                                float* out, int batch, int q_heads, int kv_heads,
                                int seq, int dim, int causal, uintptr_t stream);
int ft_attention_prefill_launch_bf16(const void* q, const void* k, const void* v,
                                     void* out, int batch, int q_heads, int kv_heads,
                                     int seq, int dim, int causal, uintptr_t stream);
int ft_attention_prefill_launch_fp16(const void* q, const void* k, const void* v,
                                     void* out, int batch, int q_heads, int kv_heads,
                                     int seq, int dim, int causal, uintptr_t stream);

/* ------------------------------------------------------------------ */
/* INT8 per-tensor symmetric quantize                                  */
/* scale = max|x|/127 (1.0 for all-zero input); inv = 1.0f/scale;      */
/* q = clamp(rint(x*inv), -127, 127). scale_out is a DEVICE float.     */
/* Replaces quantize_int8_launch (cuda_launch.hpp:191-192;             */
/* quantize.cu:195-215) without its host readback.                     */
/* ------------------------------------------------------------------ */
int ft_quantize_int8_launch(const float* x, signed char* q,
                            float* scale_out, long long n,
                            uintptr_t stream);
/* Build addition: the same quantize over bf16 / fp16 input (x_dtype is
 * FT_DT_*). Values are widened exactly to float before the same math. */
int ft_quantize_int8_launch_ex(const void* x, int x_dtype, signed char* q,
                               float* scale_out, long long n,
                               uintptr_t stream);

/* ------------------------------------------------------------------ */
/* INT8 dequantize: x[i] = (float)q[i] * scale (one f32 rounding).     */
/* Replaces dequantize_int8_launch (cuda_launch.hpp:194-195;           */
/* quantize.cu:101-108,188-193).                                       */
/* ------------------------------------------------------------------ */
int ft_dequantize_int8_launch(const signed char* q, float* x, float scale,
                              long long n, uintptr_t stream);
/* Build addition: scale_dev (a DEVICE float, e.g. a quantize scale_out)
 * overrides scale when non-NULL; x_dtype FT_DT_BF16 / FT_DT_F16 store the
 * f32 value rounded to nearest-even. */
int ft_dequantize_int8_launch_ex(const signed char* q, float scale,
                                 const float* scale_dev, void* x, int x_dtype,
                                 long long n, uintptr_t stream);

/* ------------------------------------------------------------------ */
/* Fused dequantize-add-requantize:                                    */
/*   v = f32(qa*sa) + f32(qb*sb) (each product rounded on its own);    */
/*   out_scale = max|v|/127 (1.0 if all zero), a DEVICE float;         */
/*   qy = clamp(rint(v * (1.0f/out_scale)), -127, 127).                */
/* Equals quantize_int8(dequantize(qa,sa) + dequantize(qb,sb)) bit for */
/* bit. Replaces qadd_int8_launch (cuda_launch.hpp:198-200;            */
/* quantize.cu:110-138,217-246) without its host readback.             */
/* ------------------------------------------------------------------ */
int ft_qadd_int8_launch(const signed char* qa, const signed char* qb, float sa,
                        float sb, signed char* qy, float* out_scale, long long n,
                        uintptr_t stream);
/* Build addition: DEVICE input scales (sa_dev / sb_dev override sa / sb
 * when non-NULL), e.g. the scale_out of an earlier quantize. */
int ft_qadd_int8_launch_ex(const signed char* qa, const signed char* qb, float sa,
                           float sb, const float* sa_dev, const float* sb_dev,
                           signed char* qy, float* out_scale, long long n,
                           uintptr_t stream);

/* ------------------------------------------------------------------ */
/* W8A8 GEMM: y[M,N] = float(int32(A_q[M,K] . B_q[N,K]^T)) * scale     */
/* Replaces qgemm_launch (cuda_launch.hpp:202-204; qgemm.cu:659-703)   */
/* and qgemm_perchannel_launch (cuda_launch.hpp:211-214;               */
/* qgemm.cu:706-746). Output float32.                                  */
/* ------------------------------------------------------------------ */
int ft_qgemm_launch(const signed char* aq, const signed char* bq, float* y,
                    int m, int n, int k, float sa, float sb,
                    uintptr_t stream);
int ft_qgemm_perchannel_launch(const signed char* aq, const signed char* bq,
                               const float* sb_vec, float* y, int m, int n,
                               int k, float sa, uintptr_t stream);
/* Build addition: per-channel GEMM with a bf16/fp16/f32 output. The f32
 * value is bit-identical to ft_qgemm_perchannel_launch's, then rounded to
 * nearest-even in the output type. sa_dev, when non-NULL, is a device
 * float read instead of `sa` (the device-resident scale written by
 * ft_quantize_int8_launch*). sb_vec == NULL means per-tensor: the scale
 * is f32(sa * sb). */
int ft_qgemm_launch_ex(const signed char* aq, const signed char* bq,
                       const float* sb_vec, float sb, float sa,
                       const float* sa_dev, void* y, int y_dtype, int m,
                       int n, int k, uintptr_t stream);
/* Build addition (test hook): the exact int32 accumulators
 * acc[M,N] = A_q . B_q^T, through the same kernels as the float paths. */
int ft_qgemm_i32_launch(const signed char* aq, const signed char* bq,
                        int* acc, int m, int n, int k, uintptr_t stream);

/* ------------------------------------------------------------------ */
/* RMSNorm (+ optional residual): y = (x+r) * rsqrt(mean((x+r)^2)+eps) * w */
/* x/r/y [rows, cols], w [cols] float32; r may be NULL.                */
/* Replaces rmsnorm_launch (cuda_launch.hpp:44-45; rmsnorm.cu:132-141)  */
/* and rmsnorm_launch_bf16 (cuda_launch.hpp:476-478; rmsnorm.cu:143-153)*/
/* ------------------------------------------------------------------ */
int ft_rmsnorm_launch(const float* x, const float* w, const float* r,
                      float* y, int rows, int cols, float eps,
                      uintptr_t stream);
int ft_rmsnorm_launch_bf16(const void* x, const float* w, const void* r,
                           void* y, int rows, int cols, float eps,
                           uintptr_t stream);
/* Build addition: fp16 storage. */
int ft_rmsnorm_launch_fp16(const void* x, const float* w, const void* r,
                           void* y, int rows, int cols, float eps,
                           uintptr_t stream);

/* ------------------------------------------------------------------ */
/* RoPE. x/y [seq, dim]; row r sits at position r + pos_offset;        */
/* pair j rotates by (r+pos_offset) * theta^(-2j/dim).                 */
/* Replaces rope_launch / rope_neox_launch (cuda_launch.hpp:56-59;     */
/* rope.cu:301-345) and their bf16 twins (cuda_launch.hpp:484-489).    */
/* ------------------------------------------------------------------ */
int ft_rope_launch(const float* x, float* y, int seq, int dim, float theta,
                   int pos_offset, uintptr_t stream);
int ft_rope_neox_launch(const float* x, float* y, int seq, int dim,
                        float theta, int pos_offset, uintptr_t stream);
int ft_rope_launch_bf16(const void* x, void* y, int seq, int dim,
                        float theta, int pos_offset, uintptr_t stream);
int ft_rope_neox_launch_bf16(const void* x, void* y, int seq, int dim,
                             float theta, int pos_offset, uintptr_t stream);
/* Build additions: fp16 storage. */
int ft_rope_launch_fp16(const void* x, void* y, int seq, int dim,
                        float theta, int pos_offset, uintptr_t stream);
int ft_rope_neox_launch_fp16(const void* x, void* y, int seq, int dim,
                             float theta, int pos_offset, uintptr_t stream);
/* Build addition: per-row positions. x/y [rows, dim] of dtype FT_DT_*;
 * row r sits at position base(r) + pos_offset with
 * base(r) = positions[r / rows_per_pos] (device int32) when positions is
 * non-NULL, else r / rows_per_pos. rows_per_pos = 1 with positions = NULL
 * is exactly ft_rope_launch. With q laid out [B, Hq, D] and rows_per_pos =
 * Hq, positions = per-sequence lengths rotates every head of sequence b at
 * its own decode position. */
int ft_rope_launch_ex(const void* x, void* y, int dtype, long long rows,
                      int dim, float theta, int pos_offset,
                      const int* positions, int rows_per_pos, int neox,
                      uintptr_t stream);

/* ------------------------------------------------------------------ */
/* SwiGLU: y = g / (1 + exp(-g)) * u                                   */
/* Replaces swiglu_launch (cuda_launch.hpp:40; activations.cu:513-516) */
/* and swiglu_launch_bf16 (cuda_launch.hpp:472-473;                    */
/* activations.cu:518-521).                                            */
/* ------------------------------------------------------------------ */
int ft_swiglu_launch(const float* gate, const float* up, float* y,
                     long long n, uintptr_t stream);
int ft_swiglu_launch_bf16(const void* gate, const void* up, void* y,
                          long long n, uintptr_t stream);
/* Build addition: fp16 storage. */
int ft_swiglu_launch_fp16(const void* gate, const void* up, void* y,
                          long long n, uintptr_t stream);

/* ------------------------------------------------------------------ */
/* Fused decode-chain steps. The reference has no fused layer op: a    */
/* decode layer calls rmsnorm_launch -> quantize_int8_launch,          */
/* swiglu_launch -> quantize_int8_launch and rope_launch ->            */
/* kv_append_paged_launch one after another (cuda_launch.hpp:40,       */
/* 44-45, 56-59, 191-192, 324-460). Each entry below is a build        */
/* addition that computes what that chain computes, without the float  */
/* intermediate in HBM. x_dtype / dtype are FT_DT_*.                   */
/* ------------------------------------------------------------------ */
/* RMSNorm (+ optional residual) then per-tensor int8 quantize of the
 * float32 result: q[rows, cols] int8 and *scale_out (DEVICE float) are
 * bit-identical to ft_rmsnorm_launch (float32 storage) followed by
 * ft_quantize_int8_launch. cols must be a multiple of 4 and x, residual
 * aligned to 4 elements, w to 16 bytes, q to 4 bytes. */
int ft_rmsnorm_quant_launch(const void* x, int x_dtype, const float* w,
                            const void* residual, signed char* q,
                            float* scale_out, int rows, int cols, float eps,
                            uintptr_t stream);
/* RMSNorm (+ optional residual) -> per-tensor int8 quantize -> W8A8
 * GEMM (BASELINE config 2's chain): q[rows, k] and *scale_out (DEVICE
 * float) as ft_rmsnorm_quant_launch writes them, and y[rows, n] (y_dtype
 * FT_DT_F32 / BF16 / F16) as ft_qgemm_launch_ex with sa_dev = scale_out
 * computes it from them (sb_vec per-channel, or per-tensor sb when NULL),
 * bit for bit. One row with k <= 4096 (k % 16 == 0, operands aligned as
 * for the two ops) runs as one launch; other shapes run the two ops. */
int ft_rmsnorm_qgemm_launch(const void* x, int x_dtype, const float* w,
                            const void* residual, float eps,
                            const signed char* bq, const float* sb_vec,
                            float sb, void* y, int y_dtype, signed char* q,
                            float* scale_out, int rows, int n, int k,
                            uintptr_t stream);
/* SwiGLU then per-tensor int8 quantize: gate / up element (r, c) at
 * r * ld + c (so the two halves of one [rows, 2*cols] gate|up GEMM
 * output are passed as base and base + cols with ld = 2*cols); q is the
 * dense [rows, cols] int8 result and *scale_out a DEVICE float. Equal to
 * ft_swiglu_launch (float32 storage) followed by ft_quantize_int8_launch. */
int ft_swiglu_quant_launch(const void* gate, const void* up, int dtype,
                           signed char* q, float* scale_out, int rows,
                           int cols, long long ld, uintptr_t stream);
/* RoPE of the decode token's q and k heads plus the paged KV append, in
 * one launch. qkv row b (element stride ld) holds q_heads, then kv_heads
 * k heads, then kv_heads v heads of `dim` elements. Sequence b's token
 * sits at position lens[b] + pos_offset: its q heads are rotated into
 * q_out [batch, q_heads, dim], its k heads rotated and its v heads copied
 * into slot lens[b] of the paged pools ([blocks, kv_heads, page, dim],
 * table [batch, tbl_width]), exactly as ft_rope_launch_ex with positions
 * = lens followed by ft_kv_append_paged_launch*. lens is NOT advanced; a
 * slot outside [0, tbl_width * page) is skipped. */
int ft_rope_kv_append_paged_launch(const void* qkv, int dtype, long long ld,
                                   const int* lens, const int* table,
                                   void* q_out, void* k_pool, void* v_pool,
                                   int batch, int q_heads, int kv_heads,
                                   int dim, int page, int tbl_width,
                                   float theta, int pos_offset, int neox,
                                   uintptr_t stream);
/* W8A8 GEMM then the decode token's RoPE + paged KV append: qkv =
 * ft_qgemm_launch_ex(a_q [batch, k], sa_dev, w_q [(q_heads + 2 kv_heads)
 * * dim, k], per-channel w_scales, y_dtype = dtype) and then
 * ft_rope_kv_append_paged_launch(qkv, dtype, ld = (q_heads + 2 kv_heads) *
 * dim, ...), bit for bit (qkv is written too). When the GEMM splits K over
 * workgroups, the RoPE kernel folds its partial sums itself (no fold
 * launch). */
int ft_qgemm_rope_kv_append_paged_launch(const signed char* a_q, const float* sa_dev,
                                         const signed char* w_q, const float* w_scales,
                                         int k, int dtype, void* qkv, const int* lens,
                                         const int* table, void* q_out, void* k_pool,
                                         void* v_pool, int batch, int q_heads, int kv_heads,
                                         int dim, int page, int tbl_width, float theta,
                                         int pos_offset, int neox, uintptr_t stream);
/* W8A8 GEMM then RMSNorm (+ optional residual) -> per-tensor int8
 * quantize: y [rows, n] = ft_qgemm_launch_ex(a_q, sa_dev, w_q [n, k],
 * per-channel w_scales, y_dtype = dtype), then ft_rmsnorm_quant_launch(y,
 * dtype, w, residual, q, scale_out, rows, n, eps), bit for bit. When the
 * GEMM splits K, the row pass folds its partial sums (and stores y). */
int ft_qgemm_rmsnorm_quant_launch(const signed char* a_q, const float* sa_dev,
                                  const signed char* w_q, const float* w_scales, int dtype,
                                  void* y, const void* residual, const float* w, float eps,
                                  signed char* q, float* scale_out, int rows, int n, int k,
                                  uintptr_t stream);
/* W8A8 gate/up GEMM then SwiGLU -> per-tensor int8 quantize: h [rows,
 * 2 inter] = ft_qgemm_launch_ex(a_q, sa_dev, w_gu [2 inter, k] (the inter
 * gate rows, then the inter up rows), per-channel w_scales, y_dtype =
 * dtype), then ft_swiglu_quant_launch(h, h + inter, dtype, q, scale_out,
 * rows, inter, 2 inter), bit for bit (q [rows, inter] int8, *scale_out a
 * DEVICE float). Where the GEMM runs unsplit on the skinny kernel (16 <
 * rows <= 64), each GEMM workgroup holds matching gate and up columns and
 * its epilogue takes the maximum |silu(g) * u| of the stored h, so the
 * SwiGLU's own maximum pass is not launched. */
int ft_qgemm_swiglu_quant_launch(const signed char* a_q, const float* sa_dev,
                                 const signed char* w_gu, const float* w_scales, int dtype,
                                 void* h, signed char* q, float* scale_out, int rows, int inter,
                                 int k, uintptr_t stream);
/* Paged decode attention then per-tensor int8 quantize of its output:
 * out [batch, q_heads, dim] as ft_attention_decode_paged_launch* writes it
 * (arguments as there; dtype FT_DT_*), and codes [batch, q_heads, dim]
 * int8 plus *scale_out (DEVICE float) bit-identical to quantizing that
 * stored out (ft_quantize_int8_launch for float32, its bf16 / fp16 form
 * otherwise) -- the decode layer's o_proj input. On the split-stream
 * attention path the combine kernel also writes the max |out| of each
 * (sequence, q head) and the quantize is one launch over those maxima. */
int ft_attention_decode_paged_quant_launch(const void* q, const void* k_pool,
                                           const void* v_pool, const int* table,
                                           const int* lens, void* out, int dtype,
                                           signed char* codes, float* scale_out,
                                           int batch, int q_heads, int kv_heads,
                                           int page, int tbl_width, int dim,
                                           uintptr_t stream);

/* ------------------------------------------------------------------ */
/* Decode layer (build addition). The reference has no layer op: a     */
/* decode layer calls the ops above one by one. This object runs one   */
/* Llama-shaped W8A8 decode layer as the fused chain                   */
/*   rmsnorm_quant(x, norm1) -> qgemm_rope_kv_append_paged (QKV)        */
/*   -> attention_decode_paged_quant over lens + 1 tokens               */
/*   -> qgemm_rmsnorm_quant (o_proj, residual x, norm2)                 */
/*   -> qgemm_swiglu_quant (gate/up) -> down GEMM -> y                  */
/* every step bit-identical to the unfused ops. Its activation buffers */
/* are allocated once at create (for max_batch rows); the weights are  */
/* borrowed and must outlive the layer. x, y [batch, hidden] and the   */
/* pools [blocks, kv_heads, page, head_dim] are of `dtype`; table      */
/* [batch, tbl_width] and lens [batch] are int32 (device; trusted).    */
/* The token of sequence b sits at position lens[b] + pos_offset and   */
/* is appended at slot lens[b]; lens is not advanced.                  */
/* ------------------------------------------------------------------ */
typedef struct ft_decode_layer ft_decode_layer;
typedef struct ft_decode_layer_desc {
    int hidden, q_heads, kv_heads, head_dim, inter;
    int page;       /* KV pool page size in tokens */
    int max_batch;  /* rows the activation buffers hold */
    int dtype;      /* FT_DT_F32 / BF16 / F16: activations and KV */
    float eps, theta;
    int neox, pos_offset;
    const float* norm1;        /* [hidden] */
    const float* norm2;        /* [hidden] */
    const signed char* w_qkv;  /* [(q_heads + 2 kv_heads) * head_dim, hidden] */
    const float* s_qkv;        /* per output channel */
    const signed char* w_o;    /* [hidden, q_heads * head_dim] */
    const float* s_o;
    const signed char* w_gu;   /* [2 * inter, hidden]: gate rows, then up rows */
    const float* s_gu;
    const signed char* w_down; /* [hidden, inter] */
    const float* s_down;
} ft_decode_layer_desc;
int ft_decode_layer_create(const ft_decode_layer_desc* desc, ft_decode_layer** out);
/* One forward on `stream`, with the device current at create. */
int ft_decode_layer_forward(ft_decode_layer* layer, const void* x, void* y, void* k_pool,
                            void* v_pool, const int* table, const int* lens, int batch,
                            int tbl_width, uintptr_t stream);
/* Runs one forward on `stream` (a warm-up that sizes the library's
 * scratch for the shape, with the same writes a replay makes), then
 * records the forward into a HIP graph kept by the layer (replacing an
 * earlier one). A replay reads the operands' CURRENT contents at the
 * captured addresses: write new inputs in place and replay. */
int ft_decode_layer_capture(ft_decode_layer* layer, const void* x, void* y, void* k_pool,
                            void* v_pool, const int* table, const int* lens, int batch,
                            int tbl_width, uintptr_t stream);
int ft_decode_layer_replay(ft_decode_layer* layer, uintptr_t stream);
/* FT_EINVAL (nothing freed) while a decode stack holds the layer. */
int ft_decode_layer_destroy(ft_decode_layer* layer);

/* Decode stack (build addition, no reference counterpart): n layers    */
/* chained x -> layer 0 -> layer 1 -> ... -> y, each layer's output the */
/* next one's input, with the same results as n ft_decode_layer_forward */
/* calls bit for bit. Where a layer's down GEMM splits K, its int32     */
/* partials are folded by the next layer's first RMSNorm row pass       */
/* instead of a fold launch of their own. The layers are borrowed (same */
/* device, dtype and hidden size; they must outlive the stack, and a    */
/* layer may appear more than once); table and lens are shared by all   */
/* layers, k_pools / v_pools are HOST arrays of n device pool pointers. */
/* The stack holds a reference on each layer: ft_decode_layer_destroy    */
/* refuses a layer until every stack using it has been destroyed.       */
/* The stack holds two [max_batch, hidden] buffers for the activations  */
/* between layers (max_batch = the smallest of its layers').            */
typedef struct ft_decode_stack ft_decode_stack;
int ft_decode_stack_create(ft_decode_layer* const* layers, int n_layers,
                           ft_decode_stack** out);
int ft_decode_stack_forward(ft_decode_stack* stack, const void* x, void* y,
                            void* const* k_pools, void* const* v_pools, const int* table,
                            const int* lens, int batch, int tbl_width, uintptr_t stream);
/* Warm-up forward, then the whole chain recorded into one HIP graph    */
/* (the layer capture contract above, for all n layers).                */
int ft_decode_stack_capture(ft_decode_stack* stack, const void* x, void* y,
                            void* const* k_pools, void* const* v_pools, const int* table,
                            const int* lens, int batch, int tbl_width, uintptr_t stream);
int ft_decode_stack_replay(ft_decode_stack* stack, uintptr_t stream);
int ft_decode_stack_destroy(ft_decode_stack* stack);

/* ------------------------------------------------------------------ */
/* Post-logits sampling                                                */
/* Greedy argmax: index of the first maximum of each row (a scan with  */
/* strict >: NaN never wins except at index 0). Replaces argmax_launch */
/* (cuda_launch.hpp:275) and argmax_batched_launch (:287-288).         */
/* ------------------------------------------------------------------ */
int ft_argmax_launch(const float* x, int n, int* out, uintptr_t stream);
int ft_argmax_batched_launch(const float* x, int rows, int n, long long* out,
                             uintptr_t stream);

/* Nucleus sampling of float32 logits: order tokens by (logit/T desc,   */
/* index asc), masses exp(v - max), nucleus = the shortest prefix whose */
/* mass reaches p * total, token = where the prefix mass first reaches  */
/* splitmix_uniform(seed) * nucleus mass (splitmix64 finalised to a     */
/* float in [0,1), reference cuda_util.cuh:69-76). Deterministic per    */
/* seed. p in (0,1], t > 0. The token is written to the DEVICE int64    */
/* *out without a host sync (the reference launchers return it after a  */
/* readback). Replaces sample_topp_launch (cuda_launch.hpp:73-74) and   */
/* sample_topp_batched_launch (:149-152); seeds: one DEVICE uint64 per  */
/* row.                                                                 */
int ft_sample_topp_launch(const float* x, int n, float p, float t,
                          unsigned long long seed, long long* out, uintptr_t stream);
int ft_sample_topp_batched_launch(const float* x, int rows, int n, float p, float t,
                                  const unsigned long long* seeds, long long* out,
                                  uintptr_t stream);

/* Fused decode step: CTRL repetition penalty over the DEVICE int64 ids  */
/* (each distinct id once, from the original logit: v > 0 ? v/penalty : */
/* v*penalty; ids outside [0, n) are dropped), then the temperature,    */
/* then nucleus sampling as above. penalty > 0 (1.0 disables); with a   */
/* penalty, n <= 524288. Batched: row r's ids are ids[offs[r] ..        */
/* offs[r+1]) (DEVICE int64 offsets, rows + 1 entries). Replaces        */
/* decode_step_launch (cuda_launch.hpp:138-141) and                     */
/* decode_step_batched_launch (:179-183), writing tokens to DEVICE      */
/* memory without a host sync. ids, offs and seeds may also be pinned  */
/* host memory at its device address (ft_host_device_address): the     */
/* kernels then read them in place, with no copy on the stream.         */
int ft_decode_step_launch(const float* x, const long long* ids, int n, int m,
                          float penalty, float p, float t, unsigned long long seed,
                          long long* out, uintptr_t stream);
int ft_decode_step_batched_launch(const float* x, int rows, int n, const long long* ids,
                                  const long long* offs, float penalty, float p, float t,
                                  const unsigned long long* seeds, long long* out,
                                  uintptr_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FUSEDTOK_AMD_H */
