// TEST INFRASTRUCTURE - NOT PART OF THE PRODUCT.
//
// CPU oracle for the decode hot path: a plain C++ restatement of the
// reference's single-threaded `*_cpu` functions (fusedtok 2.5.0), written
// from their documented semantics with the same loop order and float32
// arithmetic (no fast-math, no FMA contraction: built -ffp-contract=off).
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
// load it, and only as the checker / the timed CPU baseline. The product
// path (fusedtok_amd) never calls it.
//
// Each function cites the reference function it restates. Exported with a
// flat C ABI for ctypes: int status (0 ok, 1 invalid argument) and a
// thread-local message from or_last_error().
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_err;

struct Inval {
    std::string msg;
};

template <typename F>
int run(F&& f) {
    try {
        f();
        g_err.clear();
        return 0;
    } catch (const Inval& e) {
        g_err = e.msg;
        return 1;
    }
}

// reference attention.cu:184-193
void attention_check(int batch, int hq, int hkv, long long t_seq, int dim) {
    if (batch < 0 || hq < 1 || hkv < 1 || t_seq < 0 || dim < 1)
        throw Inval{"attention shapes must satisfy batch>=0, heads>=1, rows>=0, dim>=1"};
    if (hq % hkv != 0)
        throw Inval{"q heads must be a multiple of kv heads (contiguous GQA groups)"};
    if (dim % 4 != 0 || dim > 512)
        throw Inval{"dim must be a multiple of 4 and at most 512"};
}

}  // namespace

extern "C" {

const char* or_last_error(void) { return g_err.c_str(); }

// ---------------------------------------------------------------------------
// attention_decode_cpu (reference attention.cu:1318-1373): two-pass float32
// softmax per (b, h): scores = (q . k_t) * (1/sqrtf(D)), m = max, l = sum
// expf(s - m), out += (expf(s - m) / l) * v_t. len == 0 leaves a zero row.
// ---------------------------------------------------------------------------
int or_attention_decode(const float* q, const float* k, const float* v,
                        const int* lens, float* out, int batch, int hq,
                        int hkv, int t_seq, int dim) {
    return run([&] {
        attention_check(batch, hq, hkv, t_seq, dim);
        if (lens)
            for (int i = 0; i < batch; ++i)
                if (lens[i] < 0 || lens[i] > t_seq)
                    throw Inval{"lens entries must be within [0, cache rows]"};
        const int group = hq / hkv;
        const float scale = 1.0f / sqrtf((float)dim);
        std::memset(out, 0, sizeof(float) * (size_t)batch * hq * dim);
        std::vector<float> scores(t_seq > 0 ? t_seq : 1);
        for (int bi = 0; bi < batch; ++bi) {
            const int len = lens ? lens[bi] : t_seq;
            for (int h = 0; h < hq; ++h) {
                if (len == 0) continue;
                const int kv = h / group;
                const float* qp = q + ((size_t)bi * hq + h) * dim;
                const float* kp = k + (((size_t)bi * hkv + kv) * t_seq) * dim;
                const float* vp = v + (((size_t)bi * hkv + kv) * t_seq) * dim;
                float m = -INFINITY;
                for (int t = 0; t < len; ++t) {
                    float dot = 0.0f;
                    for (int d = 0; d < dim; ++d) dot += qp[d] * kp[(size_t)t * dim + d];
                    scores[t] = dot * scale;
                    m = fmaxf(m, scores[t]);
                }
                float l = 0.0f;
                for (int t = 0; t < len; ++t) l += expf(scores[t] - m);
                float* op = out + ((size_t)bi * hq + h) * dim;
                for (int t = 0; t < len; ++t) {
                    const float p = expf(scores[t] - m) / l;
                    for (int d = 0; d < dim; ++d) op[d] += p * vp[(size_t)t * dim + d];
                }
            }
        }
    });
}

// ---------------------------------------------------------------------------
// attention_prefill_cpu (reference attention.cu:1591-1639): per (b, h, row
// i), keys [0, i] (causal) or [0, S): the same two-pass float32 softmax as
// the decode step (scores = (q . k_t) * (1/sqrtf(D)), m, l = sum expf(s - m),
// out += (expf(s - m) / l) * v_t).
// ---------------------------------------------------------------------------
int or_attention_prefill(const float* q, const float* k, const float* v, float* out,
                         int batch, int hq, int hkv, int seq, int dim, int causal) {
    return run([&] {
        attention_check(batch, hq, hkv, seq, dim);
        const int group = hq / hkv;
        const float scale = 1.0f / sqrtf((float)dim);
        std::memset(out, 0, sizeof(float) * (size_t)batch * hq * seq * dim);
        std::vector<float> scores(seq > 0 ? seq : 1);
        for (int bi = 0; bi < batch; ++bi)
            for (int h = 0; h < hq; ++h) {
                const int kv = h / group;
                const float* qp = q + (((size_t)bi * hq + h) * seq) * dim;
                const float* kp = k + (((size_t)bi * hkv + kv) * seq) * dim;
                const float* vp = v + (((size_t)bi * hkv + kv) * seq) * dim;
                for (int i = 0; i < seq; ++i) {
                    const int lim = causal ? i + 1 : seq;
                    const float* qr = qp + (size_t)i * dim;
                    float m = -INFINITY;
                    for (int t = 0; t < lim; ++t) {
                        float dot = 0.0f;
                        for (int d = 0; d < dim; ++d) dot += qr[d] * kp[(size_t)t * dim + d];
                        scores[t] = dot * scale;
                        m = fmaxf(m, scores[t]);
                    }
                    float l = 0.0f;
                    for (int t = 0; t < lim; ++t) l += expf(scores[t] - m);
                    float* op = out + (((size_t)bi * hq + h) * seq + i) * dim;
                    for (int t = 0; t < lim; ++t) {
                        const float p = expf(scores[t] - m) / l;
                        for (int d = 0; d < dim; ++d) op[d] += p * vp[(size_t)t * dim + d];
                    }
                }
            }
    });
}

// ---------------------------------------------------------------------------
// attention_decode_paged_cpu (reference attention.cu:1382-1456): the same
// walk with row(t) = pool[table[b*S + t/P], kv, t%P, :]; validates lens and
// the table entries of the pages in use.
// ---------------------------------------------------------------------------
int or_attention_decode_paged(const float* q, const float* k_pool,
                              const float* v_pool, const int* table,
                              const int* lens, float* out, int batch, int hq,
                              int hkv, int page, int tbl_width, int num_blocks,
                              int dim) {
    return run([&] {
        attention_check(batch, hq, hkv, (long long)tbl_width * page, dim);
        if (page < 1) throw Inval{"page size must be >= 1"};
        const int span = tbl_width * page;
        if (lens)
            for (int i = 0; i < batch; ++i)
                if (lens[i] < 0 || lens[i] > span)
                    throw Inval{"lens entries must be within [0, table width * page]"};
        for (int bi = 0; bi < batch; ++bi) {
            const int used = lens ? lens[bi] : span;
            const int pages = (used + page - 1) / page;
            for (int s = 0; s < pages; ++s) {
                const int blk = table[(size_t)bi * tbl_width + s];
                if (blk < 0 || blk >= num_blocks)
                    throw Inval{"block table entries must be valid pool block ids"};
            }
        }
        const int group = hq / hkv;
        const float scale = 1.0f / sqrtf((float)dim);
        std::memset(out, 0, sizeof(float) * (size_t)batch * hq * dim);
        std::vector<float> scores(span > 0 ? span : 1);
        for (int bi = 0; bi < batch; ++bi) {
            const int len = lens ? lens[bi] : span;
            const int* rowT = table + (size_t)bi * tbl_width;
            for (int h = 0; h < hq; ++h) {
                if (len == 0) continue;
                const int kv = h / group;
                const float* qp = q + ((size_t)bi * hq + h) * dim;
                float m = -INFINITY;
                for (int t = 0; t < len; ++t) {
                    const size_t base = ((size_t)rowT[t / page] * hkv + kv) * page + (t % page);
                    const float* kp = k_pool + base * dim;
                    float dot = 0.0f;
                    for (int d = 0; d < dim; ++d) dot += qp[d] * kp[d];
                    scores[t] = dot * scale;
                    m = fmaxf(m, scores[t]);
                }
                float l = 0.0f;
                for (int t = 0; t < len; ++t) l += expf(scores[t] - m);
                float* op = out + ((size_t)bi * hq + h) * dim;
                for (int t = 0; t < len; ++t) {
                    const size_t base = ((size_t)rowT[t / page] * hkv + kv) * page + (t % page);
                    const float* vp = v_pool + base * dim;
                    const float p = expf(scores[t] - m) / l;
                    for (int d = 0; d < dim; ++d) op[d] += p * vp[d];
                }
            }
        }
    });
}

// ---------------------------------------------------------------------------
// kv_append_paged_cpu / kv_append_cpu (reference attention.cu:2037-2099):
// exact copies of each sequence's [Hkv, D] rows to position lens[b].
// `elem` is the element size in bytes (the copies are byte-exact, so the
// same routine serves f32 / bf16 / fp16 storage).
// ---------------------------------------------------------------------------
int or_kv_append_paged(const void* k_new, const void* v_new, const int* table,
                       const int* lens, void* k_pool, void* v_pool, int batch,
                       int hkv, int dim, int page, int tbl_width, int num_blocks,
                       int elem) {
    return run([&] {
        if (dim % 4 != 0) throw Inval{"dim must be a multiple of 4"};
        if (page < 1) throw Inval{"page size must be >= 1"};
        const size_t row = (size_t)dim * elem;
        for (int bi = 0; bi < batch; ++bi) {
            const int pos = lens[bi];
            if (pos < 0 || pos >= tbl_width * page)
                throw Inval{"lens entries must be within [0, table width * page)"};
            const int blk = table[(size_t)bi * tbl_width + pos / page];
            if (blk < 0 || blk >= num_blocks)
                throw Inval{"block table entries must be valid pool block ids"};
            const int off = pos % page;
            for (int h = 0; h < hkv; ++h) {
                const size_t dst = ((size_t)blk * hkv + h) * page + off;
                const size_t src = (size_t)bi * hkv + h;
                std::memcpy((char*)k_pool + dst * row, (const char*)k_new + src * row, row);
                std::memcpy((char*)v_pool + dst * row, (const char*)v_new + src * row, row);
            }
        }
    });
}

int or_kv_append(const void* k_new, const void* v_new, const int* lens,
                 void* k_cache, void* v_cache, int batch, int hkv, int dim,
                 int t_rows, int elem) {
    return run([&] {
        if (dim % 4 != 0) throw Inval{"dim must be a multiple of 4"};
        const size_t row = (size_t)dim * elem;
        for (int bi = 0; bi < batch; ++bi) {
            const int pos = lens[bi];
            if (pos < 0 || pos >= t_rows)
                throw Inval{"lens entries must be within [0, cache rows)"};
            for (int h = 0; h < hkv; ++h) {
                const size_t dst = ((size_t)bi * hkv + h) * t_rows + pos;
                const size_t src = (size_t)bi * hkv + h;
                std::memcpy((char*)k_cache + dst * row, (const char*)k_new + src * row, row);
                std::memcpy((char*)v_cache + dst * row, (const char*)v_new + src * row, row);
            }
        }
    });
}

// ---------------------------------------------------------------------------
// quantize_int8_cpu (reference quantize.cu:153-186): absmax, scale =
// absmax/127 (1.0 for all-zero input), inv = 1.0f/scale, q = clamp(rint(x *
// inv), -127, 127).
// ---------------------------------------------------------------------------
int or_quantize_int8(const float* x, long long n, signed char* q, float* scale_out) {
    return run([&] {
        float m = 0.0f;
        for (long long i = 0; i < n; ++i) m = std::fmax(m, std::fabs(x[i]));
        const float scale = m > 0.0f ? m / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        for (long long i = 0; i < n; ++i) {
            float v = std::rint(x[i] * inv);
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            q[i] = (signed char)v;
        }
        *scale_out = scale;
    });
}

// ---------------------------------------------------------------------------
// dequantize_int8_cpu (reference quantize.cu:188-193): x = (float)q * scale.
// ---------------------------------------------------------------------------
int or_dequantize_int8(const signed char* q, long long n, float scale, float* x) {
    return run([&] {
        for (long long i = 0; i < n; ++i) x[i] = (float)q[i] * scale;
    });
}

// ---------------------------------------------------------------------------
// qadd_int8 (reference quantize.cu:110-138,217-246; its only CPU statement is
// the explicit pipeline its test compares against, test_quantize.py:48-66):
// v = f32(qa*sa) + f32(qb*sb) (each product rounded, then the sum; no FMA
// contraction in this build of the oracle), then quantize_int8 of v.
// ---------------------------------------------------------------------------
int or_qadd_int8(const signed char* qa, const signed char* qb, long long n, float sa,
                 float sb, signed char* qy, float* scale_out) {
    std::vector<float> v((size_t)n);
    for (long long i = 0; i < n; ++i) {
        const float pa = (float)qa[i] * sa;
        const float pb = (float)qb[i] * sb;
        v[(size_t)i] = pa + pb;
    }
    return or_quantize_int8(v.data(), n, qy, scale_out);
}

// ---------------------------------------------------------------------------
// qgemm_cpu / qgemm_perchannel_cpu (reference qgemm.cu:612-652): exact int32
// dot products, then (float)acc * f32(sa*sb) or (float)acc * f32(sa*sb[j]).
// ---------------------------------------------------------------------------
static int qgemm_check(int m, int n, int k) {
    if (m < 0 || n < 0 || k < 0) throw Inval{"m, n, k must be >= 0"};
    return 0;
}

int or_qgemm_i32(const signed char* a, const signed char* b, int m, int n, int k,
                 int* acc_out) {
    return run([&] {
        qgemm_check(m, n, k);
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j) {
                int acc = 0;
                const signed char* ar = a + (size_t)i * k;
                const signed char* br = b + (size_t)j * k;
                for (int p = 0; p < k; ++p) acc += (int)ar[p] * (int)br[p];
                acc_out[(size_t)i * n + j] = acc;
            }
    });
}

int or_qgemm(const signed char* a, const signed char* b, int m, int n, int k,
             float sa, float sb, float* y) {
    return run([&] {
        qgemm_check(m, n, k);
        const float scale = sa * sb;
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j) {
                int acc = 0;
                const signed char* ar = a + (size_t)i * k;
                const signed char* br = b + (size_t)j * k;
                for (int p = 0; p < k; ++p) acc += (int)ar[p] * (int)br[p];
                y[(size_t)i * n + j] = (float)acc * scale;
            }
    });
}

int or_qgemm_perchannel(const signed char* a, const signed char* b,
                        const float* sb, int m, int n, int k, float sa, float* y) {
    return run([&] {
        qgemm_check(m, n, k);
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j) {
                int acc = 0;
                const signed char* ar = a + (size_t)i * k;
                const signed char* br = b + (size_t)j * k;
                for (int p = 0; p < k; ++p) acc += (int)ar[p] * (int)br[p];
                y[(size_t)i * n + j] = (float)acc * (sa * sb[j]);
            }
    });
}

// ---------------------------------------------------------------------------
// rmsnorm_cpu (reference rmsnorm.cu:110-130): sequential float32 sum of
// squares, inv = 1.0f / sqrt(acc/cols + eps), y = v * inv * w.
// ---------------------------------------------------------------------------
int or_rmsnorm(const float* x, const float* w, const float* residual, int rows,
               int cols, float eps, float* y) {
    return run([&] {
        if (rows < 0 || cols <= 0) throw Inval{"rows must be >= 0 and cols must be > 0"};
        for (int row = 0; row < rows; ++row) {
            const size_t base = (size_t)row * cols;
            float acc = 0.0f;
            for (int i = 0; i < cols; ++i) {
                const float v = x[base + i] + (residual ? residual[base + i] : 0.0f);
                acc += v * v;
            }
            const float inv_rms = 1.0f / std::sqrt(acc / cols + eps);
            for (int i = 0; i < cols; ++i) {
                const float v = x[base + i] + (residual ? residual[base + i] : 0.0f);
                y[base + i] = v * inv_rms * w[i];
            }
        }
    });
}

// ---------------------------------------------------------------------------
// RMSNorm in the summation order of this library's GPU kernels (the math of
// rmsnorm_cpu, reference rmsnorm.cu:110-130; only the rounding order
// differs): 256 threads, thread t accumulates fmaf(v, v, acc) over the
// 4-element chunks t, t + 256, ... in element order; each 64-lane wave adds
// lane l and lane l ^ o for o = 32, 16, ..., 1; the 4 wave totals are added
// in order. inv = 1 / sqrtf(total / cols + eps), y = (v * inv) * w.
// cols must be a multiple of 4.
// ---------------------------------------------------------------------------
static void rms_blocked_rows(const float* x, const float* w, const float* residual,
                             int rows, int cols, float eps, float* y) {
    constexpr int NT = 256;
    const int chunks = cols / 4;
    float lane[NT];
    for (int row = 0; row < rows; ++row) {
        const size_t base = (size_t)row * cols;
        auto val = [&](int i) {
            return x[base + i] + (residual ? residual[base + i] : 0.0f);
        };
        for (int t = 0; t < NT; ++t) {
            float acc = 0.0f;
            for (int c = t; c < chunks; c += NT)
                for (int e = 0; e < 4; ++e) {
                    const float v = val(4 * c + e);
                    acc = std::fma(v, v, acc);
                }
            lane[t] = acc;
        }
        float total = 0.0f;
        for (int wv = 0; wv < NT / 64; ++wv) {
            float* l = lane + 64 * wv;
            for (int o = 32; o > 0; o >>= 1) {
                float nxt[64];
                for (int i = 0; i < 64; ++i) nxt[i] = l[i] + l[i ^ o];
                for (int i = 0; i < 64; ++i) l[i] = nxt[i];
            }
            total += l[0];
        }
        const float inv = 1.0f / std::sqrt(total / (float)cols + eps);
        for (int i = 0; i < cols; ++i) y[base + i] = val(i) * inv * w[i];
    }
}

int or_rmsnorm_blocked(const float* x, const float* w, const float* residual, int rows,
                       int cols, float eps, float* y) {
    return run([&] {
        if (rows < 0 || cols <= 0) throw Inval{"rows must be >= 0 and cols must be > 0"};
        if (cols % 4 != 0) throw Inval{"cols must be a multiple of 4"};
        rms_blocked_rows(x, w, residual, rows, cols, eps, y);
    });
}

// rmsnorm_quant: or_rmsnorm_blocked then or_quantize_int8 over the whole
// (rows, cols) output (the reference chain rmsnorm -> quantize_int8).
int or_rmsnorm_quant(const float* x, const float* w, const float* residual, int rows,
                     int cols, float eps, signed char* q, float* scale_out) {
    int rc = 0;
    std::vector<float> y;
    rc = run([&] {
        if (rows < 0 || cols <= 0) throw Inval{"rows must be >= 0 and cols must be > 0"};
        if (cols % 4 != 0) throw Inval{"cols must be a multiple of 4"};
        y.resize((size_t)rows * cols);
        rms_blocked_rows(x, w, residual, rows, cols, eps, y.data());
    });
    if (rc != 0) return rc;
    return or_quantize_int8(y.data(), (long long)rows * cols, q, scale_out);
}

// swiglu_quant: swiglu_cpu on rows of a strided gate / up view (element
// (r, c) at r * ld + c), then quantize_int8 over the dense (rows, cols)
// result.
int or_swiglu_quant(const float* g, const float* u, int rows, int cols, long long ld,
                    signed char* q, float* scale_out) {
    int rc = 0;
    std::vector<float> y;
    rc = run([&] {
        if (rows < 0 || cols < 0) throw Inval{"rows and cols must be >= 0"};
        if (ld < cols) throw Inval{"row stride must be >= cols"};
        y.resize((size_t)rows * cols);
        for (int r = 0; r < rows; ++r)
            for (int c = 0; c < cols; ++c) {
                const float gv = g[(size_t)r * ld + c];
                y[(size_t)r * cols + c] = gv / (1.0f + std::exp(-gv)) * u[(size_t)r * ld + c];
            }
    });
    if (rc != 0) return rc;
    return or_quantize_int8(y.data(), (long long)rows * cols, q, scale_out);
}

// ---------------------------------------------------------------------------
// rope_cpu / rope_neox_cpu (reference rope.cu:96-143): angle = m *
// pow((double)theta, -2.0*j/dim) in double, cos/sin in double, the rotation
// in double, rounded to float. Row r sits at position r + pos_offset.
// ---------------------------------------------------------------------------
int or_rope(const float* x, int seq, int dim, float theta, int pos_offset,
            int neox, float* y) {
    return run([&] {
        if (seq < 0 || dim <= 0) throw Inval{"seq must be >= 0 and dim must be > 0"};
        if (dim % 2 != 0) throw Inval{"dim must be even (RoPE pairs elements)"};
        if (pos_offset < 0) throw Inval{"pos_offset must be >= 0"};
        for (int r = 0; r < seq; ++r) {
            const int m = r + pos_offset;
            for (int j = 0; j < dim / 2; ++j) {
                const double angle = m * std::pow((double)theta, -2.0 * j / dim);
                const double c = std::cos(angle), s = std::sin(angle);
                size_t i1, i2;
                if (neox) {
                    i1 = (size_t)r * dim + j;
                    i2 = i1 + dim / 2;
                } else {
                    i1 = (size_t)r * dim + 2 * j;
                    i2 = i1 + 1;
                }
                const float x1 = x[i1], x2 = x[i2];
                y[i1] = (float)(x1 * c - x2 * s);
                y[i2] = (float)(x1 * s + x2 * c);
            }
        }
    });
}

// ---------------------------------------------------------------------------
// swiglu_cpu (reference activations.cu:501-511): g / (1 + exp(-g)) * u.
// ---------------------------------------------------------------------------
int or_swiglu(const float* g, const float* u, long long n, float* y) {
    return run([&] {
        for (long long i = 0; i < n; ++i) {
            const float gv = g[i];
            y[i] = gv / (1.0f + std::exp(-gv)) * u[i];
        }
    });
}

// ---------------------------------------------------------------------------
// Post-logits sampling (reference sampling.cu, topk.cu, cuda_util.cuh).
// ---------------------------------------------------------------------------

// splitmix64 finalised to a float uniform in [0, 1) (reference
// cuda_util.cuh:69-76): the shared sampler RNG of the CPU and GPU paths.
float or_splitmix_uniform(unsigned long long seed) {
    unsigned long long z = seed + 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return (float)((z >> 11) * (1.0 / 9007199254740992.0));
}

// argmax_batched_cpu (reference sampling.cu:1065-1081): per row the first
// index of the maximum (a sequential scan with strict >).
int or_argmax_batched(const float* x, int rows, int n, long long* out) {
    return run([&] {
        if (rows < 0) throw Inval{"rows must be >= 0"};
        if (n <= 0) throw Inval{"argmax of empty vector"};
        for (int r = 0; r < rows; ++r) {
            const float* row = x + (size_t)r * n;
            long long best = 0;
            for (int i = 1; i < n; ++i)
                if (row[i] > row[best]) best = i;
            out[r] = best;
        }
    });
}

// repetition_penalty_cpu (reference sampling.cu:103-120): each distinct id
// once, from the original logit: v > 0 ? v / penalty : v * penalty.
int or_repetition_penalty(const float* logits, int n, const long long* ids, int m,
                          float penalty, float* y) {
    return run([&] {
        if (!(penalty > 0.0f)) throw Inval{"penalty must be > 0"};
        for (int j = 0; j < m; ++j)
            if (ids[j] < 0 || ids[j] >= n) throw Inval{"token id out of range"};
        std::memcpy(y, logits, sizeof(float) * (size_t)n);
        for (int j = 0; j < m; ++j) {
            const float v = logits[ids[j]];
            y[ids[j]] = v > 0.0f ? v / penalty : v * penalty;
        }
    });
}

// sample_topp_cpu (reference sampling.cu:466-516): order by (logit/T desc,
// index asc), float masses exp(v - max) summed in that order, nucleus = the
// shortest prefix with cum >= p * total, inverse-CDF draw at
// splitmix_uniform(seed) * nucleus mass.
static long long topp_row(const float* logits, int n, float p, float t,
                          unsigned long long seed) {
    if (n <= 0) throw Inval{"sample of empty logits"};
    if (!(p > 0.0f && p <= 1.0f)) throw Inval{"p must be in (0, 1]"};
    if (!(t > 0.0f)) throw Inval{"temperature must be > 0"};
    std::vector<unsigned int> order((size_t)n);
    for (int i = 0; i < n; ++i) order[(size_t)i] = (unsigned int)i;
    const float inv_t = 1.0f / t;
    std::sort(order.begin(), order.end(), [&](unsigned int a, unsigned int b) {
        const float va = logits[a] * inv_t, vb = logits[b] * inv_t;
        if (va != vb) return va > vb;
        return a < b;
    });
    const float row_max = logits[order[0]] * inv_t;
    auto mass_at = [&](size_t i) { return std::exp(logits[order[i]] * inv_t - row_max); };
    float total = 0.0f;
    for (size_t i = 0; i < (size_t)n; ++i) total += mass_at(i);
    float cum = 0.0f;
    size_t nucleus = 0;
    float nucleus_mass = 0.0f;
    for (size_t i = 0; i < (size_t)n; ++i) {
        cum += mass_at(i);
        nucleus = i + 1;
        if (cum >= p * total) {
            nucleus_mass = cum;
            break;
        }
    }
    const float u = or_splitmix_uniform(seed);
    const float target = u * nucleus_mass;
    cum = 0.0f;
    for (size_t i = 0; i < nucleus; ++i) {
        cum += mass_at(i);
        if (cum >= target) return (long long)order[i];
    }
    return (long long)order[nucleus - 1];
}

int or_sample_topp(const float* logits, int n, float p, float t, unsigned long long seed,
                   long long* out) {
    return run([&] { *out = topp_row(logits, n, p, t, seed); });
}

// decode_step / decode_step_batched CPU path (reference __init__.py:2410-2412,
// sampling.cu:1030-1062): repetition_penalty over the row's ids, then
// sample_topp with that row's seed.
int or_decode_step_batched(const float* logits, int rows, int n, const long long* ids,
                           const long long* offs, float penalty, float p, float t,
                           const unsigned long long* seeds, long long* out) {
    return run([&] {
        if (!(penalty > 0.0f)) throw Inval{"penalty must be > 0"};
        std::vector<float> row((size_t)n);
        for (int r = 0; r < rows; ++r) {
            const float* x = logits + (size_t)r * n;
            const long long a = offs ? offs[r] : 0, b = offs ? offs[r + 1] : 0;
            std::memcpy(row.data(), x, sizeof(float) * (size_t)n);
            for (long long j = a; j < b; ++j) {
                if (ids[j] < 0 || ids[j] >= n) throw Inval{"token id out of range"};
                const float v = x[ids[j]];
                row[(size_t)ids[j]] = v > 0.0f ? v / penalty : v * penalty;
            }
            out[r] = topp_row(row.data(), n, p, t, seeds[r]);
        }
    });
}

}  // extern "C"
