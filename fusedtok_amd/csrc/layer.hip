// Decode-layer object: one Llama-shaped W8A8 decode layer run as the fused
// chain of this library's ops, with its activation buffers allocated once at
// creation (so a forward allocates nothing once the library's scratch has
// grown to the shape) and a HIP-graph capture of the whole layer.
//
// Chain (T = the activation / KV storage type; every step bit-identical to
// the unfused ops it replaces):
//   rmsnorm_quant(x, norm1)                         -> q1, s1        1 launch
//   QKV GEMM + RoPE + paged KV append (K-split
//     partials folded by the RoPE kernel)           -> q_rot, pools  2
//   paged decode over lens + 1 tokens + quantize    -> qa, sa        3
//   o_proj GEMM + rmsnorm_quant(o + x, norm2),
//     residual stream r = T(o + x)                  -> q2, s2, r     2
//   gate/up GEMM + swiglu_quant(g[:, :inter],
//     g[:, inter:]) (SwiGLU maxima in the GEMM
//     epilogue on the skinny kernel)                -> g, q3, s3     2-3
//   down GEMM, then y = T(down + r)                 -> y             2
// (launch counts at config 4; the RMSNorm -> quantize steps take one launch
// where every row's workgroup is resident at once, grid_max). y is the
// Llama block output x + attn + mlp with the two residual adds rounded as a
// model's T tensors round them. The reference has no layer op: a decode
// layer there is these ops called one by one (cuda_launch.hpp:40-59,
// 185-216, 324-460), with the residual adds left to the caller.
#include "ft_common.hpp"
#include "kfold.hpp"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

struct ft_decode_layer {
    ft_decode_layer_desc d;
    int device = 0;
    size_t esz = 2;
    void* arena = nullptr;
    // activation buffers for max_batch rows
    signed char *q1 = nullptr, *qa = nullptr, *q2 = nullptr, *q3 = nullptr;
    void *qkv = nullptr, *qrot = nullptr, *att = nullptr, *o = nullptr, *h = nullptr;
    void* res = nullptr;  // residual stream T(o + x)
    int* lens_next = nullptr;
    float* scales = nullptr;  // s1, sa, s2, s3
    hipGraphExec_t graph = nullptr;
    // stacks holding this layer (once per appearance): its buffers stay
    // alive while any stack, or a graph a stack captured, may still use them
    std::atomic<int> stack_refs{0};
};

namespace ft {
namespace {

void rc_check(int rc) {
    if (rc != FT_OK) throw Error{rc, ft_last_error()};
}

size_t dtype_size(int dtype) {
    switch (dtype) {
    case FT_DT_F32: return 4;
    case FT_DT_BF16:
    case FT_DT_F16: return 2;
    default: inval("decode layer: unknown dtype code");
    }
}

void check_desc(const ft_decode_layer_desc& d) {
    if (d.hidden < 4 || d.hidden % 16 != 0)
        inval("decode layer: hidden must be a positive multiple of 16");
    if (d.q_heads < 1 || d.kv_heads < 1 || d.q_heads % d.kv_heads != 0)
        inval("decode layer: q_heads must be a positive multiple of kv_heads");
    const int g = d.q_heads / d.kv_heads;
    if (!(g == 1 || g == 2 || g == 4 || g == 8 || g == 16))
        inval("decode layer: the GQA group must be 1, 2, 4, 8 or 16");
    if (d.head_dim < 4 || d.head_dim % 4 != 0 || d.head_dim > 512)
        inval("decode layer: head_dim must be a multiple of 4 in [4, 512]");
    if ((d.q_heads * d.head_dim) % 16 != 0)
        inval("decode layer: q_heads * head_dim must be a multiple of 16");
    if (d.inter < 4 || d.inter % 16 != 0)
        inval("decode layer: inter must be a positive multiple of 16");
    if (d.page < 1) inval("decode layer: page must be >= 1");
    if (d.max_batch < 1) inval("decode layer: max_batch must be >= 1");
    if (d.pos_offset < 0) inval("decode layer: pos_offset must be >= 0");
    if (!d.norm1 || !d.norm2 || !d.w_qkv || !d.s_qkv || !d.w_o || !d.s_o || !d.w_gu ||
        !d.s_gu || !d.w_down || !d.s_down)
        inval("decode layer: null weight");
    (void)dtype_size(d.dtype);
}

struct Args {
    const void* x;
    void* y;
    void* k_pool;
    void* v_pool;
    const int* table;
    const int* lens;
    int batch;
    int tbl_width;
};

// Layer input handed over by the previous layer of a stack: its down
// GEMM's K-split partials (fold.ksplit > 1), folded by this layer's first
// RMSNorm row pass, which stores the rows into `store` (this layer's x).
struct HandIn {
    KFold fold;
    void* store = nullptr;
};

// in: a folded input (a.x unused), or null. defer: where this layer's down
// GEMM may leave its K-split partials for the next layer, with this layer's
// residual stream as the fold's residual (y not written when
// defer->ksplit > 1 on return), or null (y always written).
void forward(ft_decode_layer& L, const Args& a, hipStream_t s, const HandIn* in = nullptr,
             KFold* defer = nullptr) {
    const ft_decode_layer_desc& d = L.d;
    if (a.batch < 0 || a.batch > d.max_batch)
        inval("decode layer: batch must be in [0, max_batch]");
    if (a.tbl_width < 1) inval("decode layer: table width must be >= 1");
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev != L.device) inval("decode layer: called with another device current");
    if (a.batch == 0) return;
    const bool folded = in && in->fold.ksplit > 1;
    if ((!folded && !a.x) || (folded && !in->store) || !a.y || !a.k_pool || !a.v_pool ||
        !a.table || !a.lens)
        inval("decode layer: null operand");
    const void* x = folded ? in->store : a.x;  // this layer's input rows (and residual)
    const uintptr_t st = (uintptr_t)s;
    const int B = a.batch, hd = d.q_heads * d.head_dim;
    float* s1 = L.scales;
    float* sa = L.scales + 1;
    float* s2 = L.scales + 2;
    float* s3 = L.scales + 3;
    if (folded)
        rmsnorm_quant_folded(d.dtype, in->fold, in->store, d.norm1, L.q1, s1, B, d.hidden, d.eps,
                             s);
    else
        rc_check(ft_rmsnorm_quant_launch(a.x, d.dtype, d.norm1, nullptr, L.q1, s1, B, d.hidden,
                                         d.eps, st));
    qkv_rope_step(d.dtype, L.q1, s1, d.w_qkv, d.s_qkv, d.hidden, L.qkv, a.lens, L.lens_next,
                  a.table, L.qrot, a.k_pool, a.v_pool, B, d.q_heads, d.kv_heads, d.head_dim,
                  d.page, a.tbl_width, d.theta, d.pos_offset, d.neox != 0, s);
    rc_check(ft_attention_decode_paged_quant_launch(L.qrot, a.k_pool, a.v_pool, a.table,
                                                    L.lens_next, L.att, d.dtype, L.qa, sa, B,
                                                    d.q_heads, d.kv_heads, d.page,
                                                    a.tbl_width, d.head_dim, st));
    qgemm_rmsnorm_quant_res(d.dtype, L.qa, sa, d.w_o, d.s_o, L.o, x, d.norm2, d.eps, L.q2, s2,
                            L.res, B, d.hidden, hd, s);
    qgemm_swiglu_quant_codes(d.dtype, L.q2, s2, d.w_gu, d.s_gu, L.h, L.q3, s3, B, d.inter,
                             d.hidden, s);
    // down GEMM + the residual stream: folded with the K-split partials (by
    // the next layer's first row pass in a stack), else added in place
    KFold f;
    if (qgemm_deferred(L.q3, d.w_down, s3, d.s_down, a.y, d.dtype, B, d.hidden, d.inter, s, f)) {
        f.res = L.res;
        if (defer)
            *defer = f;
        else
            kfold_store(f, a.y, d.dtype, B, s);
    } else {
        if (defer) *defer = KFold{};
        residual_add(d.dtype, a.y, L.res, (long long)B * d.hidden, s);
    }
}

// ---- decode stack --------------------------------------------------------
void check_stack_layers(ft_decode_layer* const* layers, int n) {
    if (!layers || n < 1) inval("decode stack: needs at least one layer");
    for (int i = 0; i < n; ++i)
        if (!layers[i]) inval("decode stack: null layer");
    const ft_decode_layer_desc& d0 = layers[0]->d;
    for (int i = 1; i < n; ++i) {
        const ft_decode_layer& L = *layers[i];
        if (L.d.hidden != d0.hidden || L.d.dtype != d0.dtype || L.device != layers[0]->device)
            inval("decode stack: layers must share the device, dtype and hidden size");
    }
}

}  // namespace
}  // namespace ft

struct ft_decode_stack {
    std::vector<ft_decode_layer*> layers;  // borrowed
    int device = 0;
    int max_batch = 0;
    void* buf[2] = {nullptr, nullptr};     // activations between layers
    hipGraphExec_t graph = nullptr;
};

namespace ft {
namespace {

struct StackArgs {
    const void* x;
    void* y;
    void* const* k_pools;
    void* const* v_pools;
    const int* table;
    const int* lens;
    int batch;
    int tbl_width;
};

// x -> layer 0 -> .. -> y. Layer i < n - 1 writes (or, K split, leaves as
// partials for layer i + 1 to fold into) buffer i % 2, layer i + 1's input.
void stack_forward(ft_decode_stack& S, const StackArgs& a, hipStream_t s) {
    const int n = (int)S.layers.size();
    if (a.batch < 0 || a.batch > S.max_batch)
        inval("decode stack: batch must be in [0, max_batch]");
    if (!a.k_pools || !a.v_pools) inval("decode stack: null pool array");
    HandIn hand;
    const void* x = a.x;
    for (int i = 0; i < n; ++i) {
        const bool last = i == n - 1;
        void* y = last ? a.y : S.buf[i % 2];
        const Args la{x, y, a.k_pools[i], a.v_pools[i], a.table, a.lens, a.batch, a.tbl_width};
        KFold out;
        forward(*S.layers[i], la, s, hand.fold.ksplit > 1 ? &hand : nullptr,
                last ? nullptr : &out);
        if (!last) {
            hand.fold = out;  // ksplit 0: y was written and is the next input
            hand.store = y;
            x = y;
        }
    }
}

// Runs fwd(s) once on s (a warm-up that sizes the library's scratch for
// the shape: growth is refused under capture), then records fwd on a
// private stream into an instantiated HIP graph.
template <typename F>
hipGraphExec_t capture_graph(hipStream_t s, F&& fwd) {
    fwd(s);
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    hipStream_t cs = nullptr;
    hip_check(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking), "hipStreamCreate");
    hipGraph_t g = nullptr;
    hipGraphExec_t exec = nullptr;
    try {
        hip_check(hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal),
                  "hipStreamBeginCapture");
        try {
            fwd(cs);
        } catch (...) {
            hipGraph_t broken = nullptr;
            (void)hipStreamEndCapture(cs, &broken);
            if (broken) (void)hipGraphDestroy(broken);
            throw;
        }
        hip_check(hipStreamEndCapture(cs, &g), "hipStreamEndCapture");
        hip_check(hipGraphInstantiate(&exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    } catch (...) {
        if (g) (void)hipGraphDestroy(g);
        (void)hipStreamDestroy(cs);
        throw;
    }
    (void)hipGraphDestroy(g);
    (void)hipStreamDestroy(cs);
    return exec;
}

}  // namespace
}  // namespace ft

extern "C" {

int ft_decode_layer_create(const ft_decode_layer_desc* desc, ft_decode_layer** out) {
    return ft::guarded([&] {
        if (!desc || !out) ft::inval("decode layer: null argument");
        *out = nullptr;
        ft::check_desc(*desc);
        auto* L = new ft_decode_layer();
        L->d = *desc;
        L->esz = ft::dtype_size(desc->dtype);
        try {
            ft::hip_check(hipGetDevice(&L->device), "hipGetDevice");
            const size_t B = (size_t)desc->max_batch;
            const size_t hd = (size_t)desc->q_heads * desc->head_dim;
            const size_t nqkv = (size_t)(desc->q_heads + 2 * desc->kv_heads) * desc->head_dim;
            const size_t sizes[] = {
                B * desc->hidden,                // q1
                B * hd,                          // qa
                B * desc->hidden,                // q2
                B * desc->inter,                 // q3
                B * nqkv * L->esz,               // qkv
                B * hd * L->esz,                 // qrot
                B * hd * L->esz,                 // att
                B * desc->hidden * L->esz,       // o
                B * 2 * desc->inter * L->esz,    // h
                B * sizeof(int),                 // lens_next
                4 * sizeof(float),               // scales
                B * desc->hidden * L->esz,       // res
            };
            size_t off[12], total = 0;
            for (int i = 0; i < 12; ++i) {
                off[i] = total;
                total += (sizes[i] + 255) & ~(size_t)255;
            }
            hipError_t e = hipMalloc(&L->arena, total);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                L->arena = nullptr;
                ft::hip_fail("decode layer buffer allocation", e);
            }
            char* base = (char*)L->arena;
            L->q1 = (signed char*)(base + off[0]);
            L->qa = (signed char*)(base + off[1]);
            L->q2 = (signed char*)(base + off[2]);
            L->q3 = (signed char*)(base + off[3]);
            L->qkv = base + off[4];
            L->qrot = base + off[5];
            L->att = base + off[6];
            L->o = base + off[7];
            L->h = base + off[8];
            L->lens_next = (int*)(base + off[9]);
            L->scales = (float*)(base + off[10]);
            L->res = base + off[11];
        } catch (...) {
            delete L;
            throw;
        }
        *out = L;
    });
}

int ft_decode_layer_forward(ft_decode_layer* layer, const void* x, void* y, void* k_pool,
                            void* v_pool, const int* table, const int* lens, int batch,
                            int tbl_width, uintptr_t stream) {
    return ft::guarded([&] {
        if (!layer) ft::inval("decode layer: null layer");
        ft::forward(*layer, ft::Args{x, y, k_pool, v_pool, table, lens, batch, tbl_width},
                    ft::as_stream(stream));
    });
}

int ft_decode_layer_capture(ft_decode_layer* layer, const void* x, void* y, void* k_pool,
                            void* v_pool, const int* table, const int* lens, int batch,
                            int tbl_width, uintptr_t stream) {
    return ft::guarded([&] {
        if (!layer) ft::inval("decode layer: null layer");
        const ft::Args a{x, y, k_pool, v_pool, table, lens, batch, tbl_width};
        hipGraphExec_t exec = ft::capture_graph(
            ft::as_stream(stream), [&](hipStream_t cs) { ft::forward(*layer, a, cs); });
        if (layer->graph) (void)hipGraphExecDestroy(layer->graph);
        layer->graph = exec;
    });
}

int ft_decode_layer_replay(ft_decode_layer* layer, uintptr_t stream) {
    return ft::guarded([&] {
        if (!layer) ft::inval("decode layer: null layer");
        if (!layer->graph) ft::inval("decode layer: nothing captured");
        ft::hip_check(hipGraphLaunch(layer->graph, ft::as_stream(stream)), "hipGraphLaunch");
    });
}

int ft_decode_layer_destroy(ft_decode_layer* layer) {
    return ft::guarded([&] {
        if (!layer) return;
        if (layer->stack_refs.load() > 0)
            ft::inval("decode layer: still used by a decode stack (destroy the stack first)");
        if (layer->graph) (void)hipGraphExecDestroy(layer->graph);
        if (layer->arena) (void)hipFree(layer->arena);
        delete layer;
    });
}

int ft_decode_stack_create(ft_decode_layer* const* layers, int n_layers,
                           ft_decode_stack** out) {
    return ft::guarded([&] {
        if (!out) ft::inval("decode stack: null argument");
        *out = nullptr;
        ft::check_stack_layers(layers, n_layers);
        int dev = 0;
        ft::hip_check(hipGetDevice(&dev), "hipGetDevice");
        if (dev != layers[0]->device)
            ft::inval("decode stack: create it with the layers' device current");
        auto* S = new ft_decode_stack();
        S->layers.assign(layers, layers + n_layers);
        for (ft_decode_layer* L : S->layers) ++L->stack_refs;
        S->device = dev;
        S->max_batch = layers[0]->d.max_batch;
        for (int i = 1; i < n_layers; ++i)
            S->max_batch = std::min(S->max_batch, layers[i]->d.max_batch);
        const size_t bytes =
            (((size_t)S->max_batch * layers[0]->d.hidden * layers[0]->esz) + 255) & ~(size_t)255;
        if (n_layers > 1) {
            hipError_t e = hipMalloc(&S->buf[0], 2 * bytes);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                for (ft_decode_layer* L : S->layers) --L->stack_refs;
                delete S;
                ft::hip_fail("decode stack buffer allocation", e);
            }
            S->buf[1] = (char*)S->buf[0] + bytes;
        }
        *out = S;
    });
}

int ft_decode_stack_forward(ft_decode_stack* stack, const void* x, void* y,
                            void* const* k_pools, void* const* v_pools, const int* table,
                            const int* lens, int batch, int tbl_width, uintptr_t stream) {
    return ft::guarded([&] {
        if (!stack) ft::inval("decode stack: null stack");
        ft::stack_forward(*stack, ft::StackArgs{x, y, k_pools, v_pools, table, lens, batch,
                                                tbl_width},
                          ft::as_stream(stream));
    });
}

int ft_decode_stack_capture(ft_decode_stack* stack, const void* x, void* y,
                            void* const* k_pools, void* const* v_pools, const int* table,
                            const int* lens, int batch, int tbl_width, uintptr_t stream) {
    return ft::guarded([&] {
        if (!stack) ft::inval("decode stack: null stack");
        if (!k_pools || !v_pools) ft::inval("decode stack: null pool array");
        // the pool pointers are copied: the caller's arrays need not outlive
        // the call
        const std::vector<void*> kp(k_pools, k_pools + stack->layers.size());
        const std::vector<void*> vp(v_pools, v_pools + stack->layers.size());
        const ft::StackArgs a{x, y, kp.data(), vp.data(), table, lens, batch, tbl_width};
        hipGraphExec_t exec = ft::capture_graph(
            ft::as_stream(stream), [&](hipStream_t cs) { ft::stack_forward(*stack, a, cs); });
        if (stack->graph) (void)hipGraphExecDestroy(stack->graph);
        stack->graph = exec;
    });
}

int ft_decode_stack_replay(ft_decode_stack* stack, uintptr_t stream) {
    return ft::guarded([&] {
        if (!stack) ft::inval("decode stack: null stack");
        if (!stack->graph) ft::inval("decode stack: nothing captured");
        ft::hip_check(hipGraphLaunch(stack->graph, ft::as_stream(stream)), "hipGraphLaunch");
    });
}

int ft_decode_stack_destroy(ft_decode_stack* stack) {
    return ft::guarded([&] {
        if (!stack) return;
        if (stack->graph) (void)hipGraphExecDestroy(stack->graph);
        if (stack->buf[0]) (void)hipFree(stack->buf[0]);
        for (ft_decode_layer* L : stack->layers) --L->stack_refs;
        delete stack;
    });
}

}  // extern "C"
