// pybind11 module `_fusedtok`: the reference's `_launch` entry points
// (src/bindings.cpp:2171-2845, the zero-copy half) over this build's C ABI.
//
// Pointers travel as Python ints (torch `data_ptr()`), optional pointers as
// None, the stream as an int (`torch.cuda.current_stream().cuda_stream`).
// C-ABI status codes map to the reference's exception contract
// (bindings.cpp:14-16): FT_EINVAL -> ValueError, FT_EHIP -> RuntimeError.
// The host arithmetic lives entirely in the C library; nothing here
// computes.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <vector>

#include <cstdint>
#include <string>

#include "fusedtok_amd.h"

namespace py = pybind11;

namespace {

void check(int status) {
    if (status == FT_OK) return;
    const std::string msg = ft_last_error();
    if (status == FT_EINVAL) throw py::value_error(msg);
    throw std::runtime_error(msg);
}

uintptr_t opt_ptr(const py::object& o) {
    if (o.is_none()) return 0;
    return o.cast<uintptr_t>();
}

template <typename T>
T* P(uintptr_t p) {
    return reinterpret_cast<T*>(p);
}

}  // namespace

PYBIND11_MODULE(_fusedtok, m) {
    m.doc() = "gfx950 decode hot path (fusedtok-compatible launch entry points)";

    m.def("cuda_available", []() { return ft_device_available() != 0; },
          "True if a usable HIP device is present");
    m.def("version", []() { return std::string(ft_version()); });
    m.def("host_device_address",
          [](uintptr_t host) {
              void* dev = nullptr;
              return ft_host_device_address(reinterpret_cast<const void*>(host), &dev) == FT_OK
                         ? reinterpret_cast<uintptr_t>(dev)
                         : uintptr_t(0);
          },
          py::arg("host"),
          "device address of pinned host memory, or 0 when it has no device mapping");
    m.def("set_tuning",
          [](const std::string& name, int value) { check(ft_set_tuning(name.c_str(), value)); },
          py::arg("name"), py::arg("value"),
          "override a tuning / test switch (FT_* name) for this process");
    m.def("clear_tuning",
          [](const std::string& name) { check(ft_clear_tuning(name.c_str())); },
          py::arg("name"), "restore a switch to its environment value (or unset)");

    // ---- attention, contiguous ------------------------------------------
#define FT_ATT(NAME, FN, T)                                                    \
    m.def(NAME,                                                                \
          [](uintptr_t q, uintptr_t k, uintptr_t v, py::object lens,           \
             uintptr_t out, int batch, int hq, int hkv, int t_seq, int dim,    \
             uintptr_t stream) {                                               \
              check(FN(P<const T>(q), P<const T>(k), P<const T>(v),            \
                       P<const int>(opt_ptr(lens)), P<T>(out), batch, hq, hkv, \
                       t_seq, dim, stream));                                   \
          },                                                                   \
          py::arg("q"), py::arg("k"), py::arg("v"), py::arg("lens"),           \
          py::arg("out"), py::arg("batch"), py::arg("q_heads"),                \
          py::arg("kv_heads"), py::arg("cache_rows"), py::arg("dim"),          \
          py::arg("stream") = 0)
    FT_ATT("attention_decode_launch", ft_attention_decode_launch, float);
    FT_ATT("attention_decode_launch_bf16", ft_attention_decode_launch_bf16, void);
    FT_ATT("attention_decode_launch_fp16", ft_attention_decode_launch_fp16, void);
#undef FT_ATT

    // ---- attention, prefill -------------------------------------------------
#define FT_PRE(NAME, FN, T)                                                    \
    m.def(NAME,                                                                \
          [](uintptr_t q, uintptr_t k, uintptr_t v, uintptr_t out, int batch,  \
             int hq, int hkv, int seq, int dim, bool causal, uintptr_t stream) { \
              check(FN(P<const T>(q), P<const T>(k), P<const T>(v), P<T>(out), \
                       batch, hq, hkv, seq, dim, causal ? 1 : 0, stream));     \
          },                                                                   \
          py::arg("q"), py::arg("k"), py::arg("v"), py::arg("out"),            \
          py::arg("batch"), py::arg("q_heads"), py::arg("kv_heads"),           \
          py::arg("seq"), py::arg("dim"), py::arg("causal"),                   \
          py::arg("stream") = 0)
    FT_PRE("attention_prefill_launch", ft_attention_prefill_launch, float);
    FT_PRE("attention_prefill_launch_bf16", ft_attention_prefill_launch_bf16, void);
    FT_PRE("attention_prefill_launch_fp16", ft_attention_prefill_launch_fp16, void);
#undef FT_PRE

    // ---- attention, paged -----------------------------------------------
#define FT_ATTP(NAME, FN, T)                                                   \
    m.def(NAME,                                                                \
          [](uintptr_t q, uintptr_t kp, uintptr_t vp, uintptr_t table,         \
             py::object lens, uintptr_t out, int batch, int hq, int hkv,       \
             int page, int tbl_width, int dim, uintptr_t stream) {             \
              check(FN(P<const T>(q), P<const T>(kp), P<const T>(vp),          \
                       P<const int>(table), P<const int>(opt_ptr(lens)),       \
                       P<T>(out), batch, hq, hkv, page, tbl_width, dim,        \
                       stream));                                               \
          },                                                                   \
          py::arg("q"), py::arg("k_pool"), py::arg("v_pool"),                  \
          py::arg("table"), py::arg("lens"), py::arg("out"),                   \
          py::arg("batch"), py::arg("q_heads"), py::arg("kv_heads"),           \
          py::arg("page"), py::arg("tbl_width"), py::arg("dim"),               \
          py::arg("stream") = 0)
    FT_ATTP("attention_decode_paged_launch", ft_attention_decode_paged_launch, float);
    FT_ATTP("attention_decode_paged_launch_bf16",
            ft_attention_decode_paged_launch_bf16, void);
    FT_ATTP("attention_decode_paged_launch_fp16",
            ft_attention_decode_paged_launch_fp16, void);
#undef FT_ATTP
    m.def("attention_decode_paged_quant_launch",
          [](uintptr_t q, uintptr_t kp, uintptr_t vp, uintptr_t table, py::object lens,
             uintptr_t out, int dtype, uintptr_t codes, uintptr_t scale, int batch, int hq,
             int hkv, int page, int tbl_width, int dim, uintptr_t stream) {
              check(ft_attention_decode_paged_quant_launch(
                  P<const void>(q), P<const void>(kp), P<const void>(vp),
                  P<const int>(table), P<const int>(opt_ptr(lens)), P<void>(out), dtype,
                  P<signed char>(codes), P<float>(scale), batch, hq, hkv, page, tbl_width,
                  dim, stream));
          },
          py::arg("q"), py::arg("k_pool"), py::arg("v_pool"), py::arg("table"),
          py::arg("lens"), py::arg("out"), py::arg("dtype"), py::arg("codes"),
          py::arg("scale"), py::arg("batch"), py::arg("q_heads"), py::arg("kv_heads"),
          py::arg("page"), py::arg("tbl_width"), py::arg("dim"), py::arg("stream") = 0);

    m.def("attention_decode_paged_append_launch",
          [](uintptr_t q, uintptr_t kp, uintptr_t vp, uintptr_t table, uintptr_t kn,
             uintptr_t vn, uintptr_t lens, uintptr_t out, int dtype, int batch, int hq,
             int hkv, int page, int tbl_width, int dim, uintptr_t stream) {
              check(ft_attention_decode_paged_append_launch(
                  P<const void>(q), P<void>(kp), P<void>(vp), P<const int>(table),
                  P<const void>(kn), P<const void>(vn), P<const int>(lens), P<void>(out),
                  dtype, batch, hq, hkv, page, tbl_width, dim, stream));
          },
          py::arg("q"), py::arg("k_pool"), py::arg("v_pool"), py::arg("table"),
          py::arg("k_new"), py::arg("v_new"), py::arg("lens"), py::arg("out"),
          py::arg("dtype"), py::arg("batch"), py::arg("q_heads"), py::arg("kv_heads"),
          py::arg("page"), py::arg("tbl_width"), py::arg("dim"), py::arg("stream") = 0);

    // ---- kv append --------------------------------------------------------
#define FT_KVP(NAME, FN, T)                                                    \
    m.def(NAME,                                                                \
          [](uintptr_t kn, uintptr_t vn, uintptr_t table, uintptr_t lens,      \
             uintptr_t kp, uintptr_t vp, int batch, int hkv, int dim,          \
             int page, int tbl_width, uintptr_t stream) {                      \
              check(FN(P<const T>(kn), P<const T>(vn), P<const int>(table),    \
                       P<const int>(lens), P<T>(kp), P<T>(vp), batch, hkv,     \
                       dim, page, tbl_width, stream));                         \
          },                                                                   \
          py::arg("k_new"), py::arg("v_new"), py::arg("table"),                \
          py::arg("lens"), py::arg("k_pool"), py::arg("v_pool"),               \
          py::arg("batch"), py::arg("hkv"), py::arg("dim"), py::arg("page"),   \
          py::arg("tbl_width"), py::arg("stream") = 0)
    FT_KVP("kv_append_paged_launch", ft_kv_append_paged_launch, float);
    FT_KVP("kv_append_paged_launch_bf16", ft_kv_append_paged_launch_bf16, void);
    FT_KVP("kv_append_paged_launch_fp16", ft_kv_append_paged_launch_fp16, void);
#undef FT_KVP

#define FT_KV(NAME, FN, T)                                                     \
    m.def(NAME,                                                                \
          [](uintptr_t kn, uintptr_t vn, uintptr_t lens, uintptr_t kc,         \
             uintptr_t vc, int batch, int hkv, int dim, int t_rows,            \
             uintptr_t stream) {                                               \
              check(FN(P<const T>(kn), P<const T>(vn), P<const int>(lens),     \
                       P<T>(kc), P<T>(vc), batch, hkv, dim, t_rows, stream));  \
          },                                                                   \
          py::arg("k_new"), py::arg("v_new"), py::arg("lens"),                 \
          py::arg("k_cache"), py::arg("v_cache"), py::arg("batch"),            \
          py::arg("hkv"), py::arg("dim"), py::arg("t_rows"),                   \
          py::arg("stream") = 0)
    FT_KV("kv_append_launch", ft_kv_append_launch, float);
    FT_KV("kv_append_launch_bf16", ft_kv_append_launch_bf16, void);
    FT_KV("kv_append_launch_fp16", ft_kv_append_launch_fp16, void);
#undef FT_KV

    // ---- quantize -----------------------------------------------------------
    m.def("quantize_launch",
          [](uintptr_t x, uintptr_t q, uintptr_t scale, long long n,
             uintptr_t stream) {
              check(ft_quantize_int8_launch(P<const float>(x), P<signed char>(q),
                                            P<float>(scale), n, stream));
          },
          py::arg("x"), py::arg("q"), py::arg("scale"), py::arg("n"),
          py::arg("stream") = 0);
    m.def("quantize_launch_ex",
          [](uintptr_t x, int dtype, uintptr_t q, uintptr_t scale, long long n,
             uintptr_t stream) {
              check(ft_quantize_int8_launch_ex(P<const void>(x), dtype,
                                               P<signed char>(q), P<float>(scale),
                                               n, stream));
          },
          py::arg("x"), py::arg("dtype"), py::arg("q"), py::arg("scale"),
          py::arg("n"), py::arg("stream") = 0);
    m.def("dequantize_launch",
          [](uintptr_t q, uintptr_t x, float scale, long long n, uintptr_t stream) {
              check(ft_dequantize_int8_launch(P<const signed char>(q), P<float>(x),
                                              scale, n, stream));
          },
          py::arg("q"), py::arg("x"), py::arg("scale"), py::arg("n"),
          py::arg("stream") = 0);
    m.def("dequantize_launch_ex",
          [](uintptr_t q, float scale, py::object scale_dev, uintptr_t x, int dtype,
             long long n, uintptr_t stream) {
              check(ft_dequantize_int8_launch_ex(P<const signed char>(q), scale,
                                                 P<const float>(opt_ptr(scale_dev)),
                                                 P<void>(x), dtype, n, stream));
          },
          py::arg("q"), py::arg("scale"), py::arg("scale_dev"), py::arg("x"),
          py::arg("dtype"), py::arg("n"), py::arg("stream") = 0);
    m.def("qadd_launch",
          [](uintptr_t qa, uintptr_t qb, float sa, float sb, uintptr_t qy,
             uintptr_t out_scale, long long n, uintptr_t stream) {
              check(ft_qadd_int8_launch(P<const signed char>(qa), P<const signed char>(qb),
                                        sa, sb, P<signed char>(qy), P<float>(out_scale),
                                        n, stream));
          },
          py::arg("qa"), py::arg("qb"), py::arg("sa"), py::arg("sb"), py::arg("qy"),
          py::arg("out_scale"), py::arg("n"), py::arg("stream") = 0);
    m.def("qadd_launch_ex",
          [](uintptr_t qa, uintptr_t qb, float sa, float sb, py::object sa_dev,
             py::object sb_dev, uintptr_t qy, uintptr_t out_scale, long long n,
             uintptr_t stream) {
              check(ft_qadd_int8_launch_ex(
                  P<const signed char>(qa), P<const signed char>(qb), sa, sb,
                  P<const float>(opt_ptr(sa_dev)), P<const float>(opt_ptr(sb_dev)),
                  P<signed char>(qy), P<float>(out_scale), n, stream));
          },
          py::arg("qa"), py::arg("qb"), py::arg("sa"), py::arg("sb"),
          py::arg("sa_dev"), py::arg("sb_dev"), py::arg("qy"), py::arg("out_scale"),
          py::arg("n"), py::arg("stream") = 0);

    // ---- sampling -----------------------------------------------------------
    m.def("argmax_launch",
          [](uintptr_t x, int n, uintptr_t out, uintptr_t stream) {
              check(ft_argmax_launch(P<const float>(x), n, P<int>(out), stream));
          },
          py::arg("x"), py::arg("n"), py::arg("out"), py::arg("stream") = 0);
    m.def("argmax_batched_launch",
          [](uintptr_t x, int rows, int n, uintptr_t out, uintptr_t stream) {
              check(ft_argmax_batched_launch(P<const float>(x), rows, n, P<long long>(out),
                                             stream));
          },
          py::arg("x"), py::arg("rows"), py::arg("n"), py::arg("out"), py::arg("stream") = 0);
    m.def("sample_topp_launch",
          [](uintptr_t x, int n, float p, float t, unsigned long long seed, uintptr_t out,
             uintptr_t stream) {
              check(ft_sample_topp_launch(P<const float>(x), n, p, t, seed, P<long long>(out),
                                          stream));
          },
          py::arg("x"), py::arg("n"), py::arg("p"), py::arg("temperature"), py::arg("seed"),
          py::arg("out"), py::arg("stream") = 0);
    m.def("sample_topp_batched_launch",
          [](uintptr_t x, int rows, int n, float p, float t, uintptr_t seeds, uintptr_t out,
             uintptr_t stream) {
              check(ft_sample_topp_batched_launch(P<const float>(x), rows, n, p, t,
                                                  P<const unsigned long long>(seeds),
                                                  P<long long>(out), stream));
          },
          py::arg("x"), py::arg("rows"), py::arg("n"), py::arg("p"), py::arg("temperature"),
          py::arg("seeds"), py::arg("out"), py::arg("stream") = 0);
    m.def("decode_step_launch",
          [](uintptr_t x, py::object ids, int n, int m_, float penalty, float p, float t,
             unsigned long long seed, uintptr_t out, uintptr_t stream) {
              check(ft_decode_step_launch(P<const float>(x), P<const long long>(opt_ptr(ids)),
                                          n, m_, penalty, p, t, seed, P<long long>(out),
                                          stream));
          },
          py::arg("x"), py::arg("ids"), py::arg("n"), py::arg("m"), py::arg("penalty"),
          py::arg("p"), py::arg("temperature"), py::arg("seed"), py::arg("out"),
          py::arg("stream") = 0);
    m.def("decode_step_batched_launch",
          [](uintptr_t x, int rows, int n, py::object ids, uintptr_t offs, float penalty,
             float p, float t, uintptr_t seeds, uintptr_t out, uintptr_t stream) {
              check(ft_decode_step_batched_launch(
                  P<const float>(x), rows, n, P<const long long>(opt_ptr(ids)),
                  P<const long long>(offs), penalty, p, t, P<const unsigned long long>(seeds),
                  P<long long>(out), stream));
          },
          py::arg("x"), py::arg("rows"), py::arg("n"), py::arg("ids"), py::arg("offs"),
          py::arg("penalty"), py::arg("p"), py::arg("temperature"), py::arg("seeds"),
          py::arg("out"), py::arg("stream") = 0);

    // ---- qgemm --------------------------------------------------------------
    m.def("qgemm_launch",
          [](uintptr_t a, uintptr_t b, uintptr_t y, int mm, int n, int k,
             float sa, float sb, uintptr_t stream) {
              check(ft_qgemm_launch(P<const signed char>(a), P<const signed char>(b),
                                    P<float>(y), mm, n, k, sa, sb, stream));
          },
          py::arg("a"), py::arg("b"), py::arg("y"), py::arg("m"), py::arg("n"),
          py::arg("k"), py::arg("sa"), py::arg("sb"), py::arg("stream") = 0);
    m.def("qgemm_perchannel_launch",
          [](uintptr_t a, uintptr_t b, uintptr_t sb, uintptr_t y, int mm, int n,
             int k, float sa, uintptr_t stream) {
              check(ft_qgemm_perchannel_launch(
                  P<const signed char>(a), P<const signed char>(b),
                  P<const float>(sb), P<float>(y), mm, n, k, sa, stream));
          },
          py::arg("a"), py::arg("b"), py::arg("sb"), py::arg("y"), py::arg("m"),
          py::arg("n"), py::arg("k"), py::arg("sa"), py::arg("stream") = 0);
    m.def("qgemm_launch_ex",
          [](uintptr_t a, uintptr_t b, py::object sb_vec, float sb, float sa,
             py::object sa_dev, uintptr_t y, int y_dtype, int mm, int n, int k,
             uintptr_t stream) {
              check(ft_qgemm_launch_ex(
                  P<const signed char>(a), P<const signed char>(b),
                  P<const float>(opt_ptr(sb_vec)), sb, sa,
                  P<const float>(opt_ptr(sa_dev)), P<void>(y), y_dtype, mm, n, k,
                  stream));
          },
          py::arg("a"), py::arg("b"), py::arg("sb_vec"), py::arg("sb"),
          py::arg("sa"), py::arg("sa_dev"), py::arg("y"), py::arg("y_dtype"),
          py::arg("m"), py::arg("n"), py::arg("k"), py::arg("stream") = 0);
    m.def("qgemm_i32_launch",
          [](uintptr_t a, uintptr_t b, uintptr_t acc, int mm, int n, int k,
             uintptr_t stream) {
              check(ft_qgemm_i32_launch(P<const signed char>(a),
                                        P<const signed char>(b), P<int>(acc), mm,
                                        n, k, stream));
          },
          py::arg("a"), py::arg("b"), py::arg("acc"), py::arg("m"), py::arg("n"),
          py::arg("k"), py::arg("stream") = 0);

    // ---- rmsnorm --------------------------------------------------------------
    m.def("rmsnorm_launch",
          [](uintptr_t x, uintptr_t w, py::object r, uintptr_t y, int rows,
             int cols, float eps, uintptr_t stream) {
              check(ft_rmsnorm_launch(P<const float>(x), P<const float>(w),
                                      P<const float>(opt_ptr(r)), P<float>(y),
                                      rows, cols, eps, stream));
          },
          py::arg("x"), py::arg("weight"), py::arg("residual"), py::arg("out"),
          py::arg("rows"), py::arg("cols"), py::arg("eps"),
          py::arg("stream") = 0);
#define FT_RMS(NAME, FN)                                                       \
    m.def(NAME,                                                                \
          [](uintptr_t x, uintptr_t w, py::object r, uintptr_t y, int rows,    \
             int cols, float eps, uintptr_t stream) {                          \
              check(FN(P<const void>(x), P<const float>(w),                    \
                       P<const void>(opt_ptr(r)), P<void>(y), rows, cols, eps, \
                       stream));                                               \
          },                                                                   \
          py::arg("x"), py::arg("weight"), py::arg("residual"),                \
          py::arg("out"), py::arg("rows"), py::arg("cols"), py::arg("eps"),    \
          py::arg("stream") = 0)
    FT_RMS("rmsnorm_launch_bf16", ft_rmsnorm_launch_bf16);
    FT_RMS("rmsnorm_launch_fp16", ft_rmsnorm_launch_fp16);
#undef FT_RMS

    // ---- rope -----------------------------------------------------------------
    m.def("rope_launch",
          [](bool neox, uintptr_t x, uintptr_t y, int seq, int dim, float theta,
             int pos_offset, uintptr_t stream) {
              check(neox ? ft_rope_neox_launch(P<const float>(x), P<float>(y), seq,
                                               dim, theta, pos_offset, stream)
                         : ft_rope_launch(P<const float>(x), P<float>(y), seq, dim,
                                          theta, pos_offset, stream));
          },
          py::arg("neox"), py::arg("x"), py::arg("y"), py::arg("seq"),
          py::arg("dim"), py::arg("theta"), py::arg("pos_offset"),
          py::arg("stream") = 0);
#define FT_ROPE(NAME, FN)                                                      \
    m.def(NAME,                                                                \
          [](uintptr_t x, uintptr_t y, int seq, int dim, float theta,          \
             int pos_offset, uintptr_t stream) {                               \
              check(FN(P<const void>(x), P<void>(y), seq, dim, theta,          \
                       pos_offset, stream));                                   \
          },                                                                   \
          py::arg("x"), py::arg("y"), py::arg("seq"), py::arg("dim"),          \
          py::arg("theta"), py::arg("pos_offset"), py::arg("stream") = 0)
    FT_ROPE("rope_launch_bf16", ft_rope_launch_bf16);
    FT_ROPE("rope_neox_launch_bf16", ft_rope_neox_launch_bf16);
    FT_ROPE("rope_launch_fp16", ft_rope_launch_fp16);
    FT_ROPE("rope_neox_launch_fp16", ft_rope_neox_launch_fp16);
#undef FT_ROPE
    m.def("rope_launch_ex",
          [](uintptr_t x, uintptr_t y, int dtype, long long rows, int dim,
             float theta, int pos_offset, py::object positions, int rows_per_pos,
             bool neox, uintptr_t stream) {
              check(ft_rope_launch_ex(P<const void>(x), P<void>(y), dtype, rows, dim,
                                      theta, pos_offset,
                                      P<const int>(opt_ptr(positions)),
                                      rows_per_pos, neox ? 1 : 0, stream));
          },
          py::arg("x"), py::arg("y"), py::arg("dtype"), py::arg("rows"),
          py::arg("dim"), py::arg("theta"), py::arg("pos_offset"),
          py::arg("positions"), py::arg("rows_per_pos"), py::arg("neox"),
          py::arg("stream") = 0);

    // ---- swiglu -----------------------------------------------------------------
    m.def("swiglu_launch",
          [](uintptr_t g, uintptr_t u, uintptr_t y, long long n, uintptr_t stream) {
              check(ft_swiglu_launch(P<const float>(g), P<const float>(u), P<float>(y),
                                     n, stream));
          },
          py::arg("gate"), py::arg("up"), py::arg("out"), py::arg("n"),
          py::arg("stream") = 0);
    m.def("swiglu_launch_bf16",
          [](uintptr_t g, uintptr_t u, uintptr_t y, long long n, uintptr_t stream) {
              check(ft_swiglu_launch_bf16(P<const void>(g), P<const void>(u),
                                          P<void>(y), n, stream));
          },
          py::arg("gate"), py::arg("up"), py::arg("out"), py::arg("n"),
          py::arg("stream") = 0);
    m.def("swiglu_launch_fp16",
          [](uintptr_t g, uintptr_t u, uintptr_t y, long long n, uintptr_t stream) {
              check(ft_swiglu_launch_fp16(P<const void>(g), P<const void>(u),
                                          P<void>(y), n, stream));
          },
          py::arg("gate"), py::arg("up"), py::arg("out"), py::arg("n"),
          py::arg("stream") = 0);

    // ---- fused decode-chain steps ----------------------------------------------
    m.def("rmsnorm_quant_launch",
          [](uintptr_t x, int dtype, uintptr_t w, py::object r, uintptr_t q,
             uintptr_t scale, int rows, int cols, float eps, uintptr_t stream) {
              check(ft_rmsnorm_quant_launch(P<const void>(x), dtype, P<const float>(w),
                                            P<const void>(opt_ptr(r)),
                                            P<signed char>(q), P<float>(scale), rows,
                                            cols, eps, stream));
          },
          py::arg("x"), py::arg("dtype"), py::arg("weight"), py::arg("residual"),
          py::arg("q"), py::arg("scale"), py::arg("rows"), py::arg("cols"),
          py::arg("eps"), py::arg("stream") = 0);
    m.def("rmsnorm_qgemm_launch",
          [](uintptr_t x, int dtype, uintptr_t w, py::object r, float eps, uintptr_t bq,
             py::object sb_vec, float sb, uintptr_t y, int y_dtype, uintptr_t q,
             uintptr_t scale, int rows, int n, int k, uintptr_t stream) {
              check(ft_rmsnorm_qgemm_launch(P<const void>(x), dtype, P<const float>(w),
                                            P<const void>(opt_ptr(r)), eps,
                                            P<const signed char>(bq),
                                            P<const float>(opt_ptr(sb_vec)), sb, P<void>(y),
                                            y_dtype, P<signed char>(q), P<float>(scale),
                                            rows, n, k, stream));
          },
          py::arg("x"), py::arg("dtype"), py::arg("weight"), py::arg("residual"),
          py::arg("eps"), py::arg("b"), py::arg("sb_vec"), py::arg("sb"), py::arg("y"),
          py::arg("y_dtype"), py::arg("q"), py::arg("scale"), py::arg("rows"),
          py::arg("n"), py::arg("k"), py::arg("stream") = 0);
    m.def("swiglu_quant_launch",
          [](uintptr_t g, uintptr_t u, int dtype, uintptr_t q, uintptr_t scale,
             int rows, int cols, long long ld, uintptr_t stream) {
              check(ft_swiglu_quant_launch(P<const void>(g), P<const void>(u), dtype,
                                           P<signed char>(q), P<float>(scale), rows,
                                           cols, ld, stream));
          },
          py::arg("gate"), py::arg("up"), py::arg("dtype"), py::arg("q"),
          py::arg("scale"), py::arg("rows"), py::arg("cols"), py::arg("ld"),
          py::arg("stream") = 0);
    m.def("qgemm_rope_kv_append_paged_launch",
          [](uintptr_t a, uintptr_t sa, uintptr_t w, uintptr_t ws, int k, int dtype,
             uintptr_t qkv, uintptr_t lens, uintptr_t table, uintptr_t q_out, uintptr_t kp,
             uintptr_t vp, int batch, int hq, int hkv, int dim, int page, int tbl_width,
             float theta, int pos_offset, bool neox, uintptr_t stream) {
              check(ft_qgemm_rope_kv_append_paged_launch(
                  P<const signed char>(a), P<const float>(sa), P<const signed char>(w),
                  P<const float>(ws), k, dtype, P<void>(qkv), P<const int>(lens),
                  P<const int>(table), P<void>(q_out), P<void>(kp), P<void>(vp), batch, hq,
                  hkv, dim, page, tbl_width, theta, pos_offset, neox ? 1 : 0, stream));
          },
          py::arg("a_q"), py::arg("sa_dev"), py::arg("w_q"), py::arg("w_scales"),
          py::arg("k"), py::arg("dtype"), py::arg("qkv"), py::arg("lens"), py::arg("table"),
          py::arg("q_out"), py::arg("k_pool"), py::arg("v_pool"), py::arg("batch"),
          py::arg("q_heads"), py::arg("kv_heads"), py::arg("dim"), py::arg("page"),
          py::arg("tbl_width"), py::arg("theta"), py::arg("pos_offset"), py::arg("neox"),
          py::arg("stream") = 0);
    m.def("qgemm_rmsnorm_quant_launch",
          [](uintptr_t a, uintptr_t sa, uintptr_t w, uintptr_t ws, int dtype, uintptr_t y,
             py::object r, uintptr_t nw, float eps, uintptr_t q, uintptr_t scale, int rows,
             int n, int k, uintptr_t stream) {
              check(ft_qgemm_rmsnorm_quant_launch(
                  P<const signed char>(a), P<const float>(sa), P<const signed char>(w),
                  P<const float>(ws), dtype, P<void>(y), P<const void>(opt_ptr(r)),
                  P<const float>(nw), eps, P<signed char>(q), P<float>(scale), rows, n, k,
                  stream));
          },
          py::arg("a_q"), py::arg("sa_dev"), py::arg("w_q"), py::arg("w_scales"),
          py::arg("dtype"), py::arg("y"), py::arg("residual"), py::arg("weight"),
          py::arg("eps"), py::arg("q"), py::arg("scale"), py::arg("rows"), py::arg("n"),
          py::arg("k"), py::arg("stream") = 0);
    m.def("qgemm_swiglu_quant_launch",
          [](uintptr_t a, uintptr_t sa, uintptr_t w, uintptr_t ws, int dtype, uintptr_t h,
             uintptr_t q, uintptr_t scale, int rows, int inter, int k, uintptr_t stream) {
              check(ft_qgemm_swiglu_quant_launch(
                  P<const signed char>(a), P<const float>(sa), P<const signed char>(w),
                  P<const float>(ws), dtype, P<void>(h), P<signed char>(q), P<float>(scale),
                  rows, inter, k, stream));
          },
          py::arg("a_q"), py::arg("sa_dev"), py::arg("w_q"), py::arg("w_scales"),
          py::arg("dtype"), py::arg("h"), py::arg("q"), py::arg("scale"), py::arg("rows"),
          py::arg("inter"), py::arg("k"), py::arg("stream") = 0);
    // ---- decode layer object ---------------------------------------------
    m.def("decode_layer_create",
          [](int hidden, int hq, int hkv, int dim, int inter, int page, int max_batch, int dtype,
             float eps, float theta, bool neox, int pos_offset, uintptr_t n1, uintptr_t n2,
             uintptr_t wqkv, uintptr_t sqkv, uintptr_t wo, uintptr_t so, uintptr_t wgu,
             uintptr_t sgu, uintptr_t wd, uintptr_t sd) {
              ft_decode_layer_desc d{};
              d.hidden = hidden; d.q_heads = hq; d.kv_heads = hkv; d.head_dim = dim;
              d.inter = inter; d.page = page; d.max_batch = max_batch; d.dtype = dtype;
              d.eps = eps; d.theta = theta; d.neox = neox ? 1 : 0; d.pos_offset = pos_offset;
              d.norm1 = P<const float>(n1); d.norm2 = P<const float>(n2);
              d.w_qkv = P<const signed char>(wqkv); d.s_qkv = P<const float>(sqkv);
              d.w_o = P<const signed char>(wo); d.s_o = P<const float>(so);
              d.w_gu = P<const signed char>(wgu); d.s_gu = P<const float>(sgu);
              d.w_down = P<const signed char>(wd); d.s_down = P<const float>(sd);
              ft_decode_layer* L = nullptr;
              check(ft_decode_layer_create(&d, &L));
              return reinterpret_cast<uintptr_t>(L);
          },
          py::arg("hidden"), py::arg("q_heads"), py::arg("kv_heads"), py::arg("head_dim"),
          py::arg("inter"), py::arg("page"), py::arg("max_batch"), py::arg("dtype"),
          py::arg("eps"), py::arg("theta"), py::arg("neox"), py::arg("pos_offset"),
          py::arg("norm1"), py::arg("norm2"), py::arg("w_qkv"), py::arg("s_qkv"),
          py::arg("w_o"), py::arg("s_o"), py::arg("w_gu"), py::arg("s_gu"), py::arg("w_down"),
          py::arg("s_down"));
#define FT_LAYER_CALL(NAME, FN)                                                          \
    m.def(NAME,                                                                          \
          [](uintptr_t L, uintptr_t x, uintptr_t y, uintptr_t kp, uintptr_t vp,          \
             uintptr_t table, uintptr_t lens, int batch, int tbl_width, uintptr_t stream) { \
              check(FN(P<ft_decode_layer>(L), P<const void>(x), P<void>(y), P<void>(kp),   \
                       P<void>(vp), P<const int>(table), P<const int>(lens), batch,        \
                       tbl_width, stream));                                              \
          },                                                                             \
          py::arg("layer"), py::arg("x"), py::arg("y"), py::arg("k_pool"),               \
          py::arg("v_pool"), py::arg("table"), py::arg("lens"), py::arg("batch"),        \
          py::arg("tbl_width"), py::arg("stream") = 0)
    FT_LAYER_CALL("decode_layer_forward", ft_decode_layer_forward);
    FT_LAYER_CALL("decode_layer_capture", ft_decode_layer_capture);
#undef FT_LAYER_CALL
    m.def("decode_layer_replay",
          [](uintptr_t L, uintptr_t stream) {
              check(ft_decode_layer_replay(P<ft_decode_layer>(L), stream));
          },
          py::arg("layer"), py::arg("stream") = 0);
    m.def("decode_layer_destroy",
          [](uintptr_t L) { check(ft_decode_layer_destroy(P<ft_decode_layer>(L))); },
          py::arg("layer"));
    // ---- decode stack object ---------------------------------------------
    m.def("decode_stack_create",
          [](const std::vector<uintptr_t>& layers) {
              std::vector<ft_decode_layer*> ls;
              for (uintptr_t L : layers) ls.push_back(P<ft_decode_layer>(L));
              ft_decode_stack* S = nullptr;
              check(ft_decode_stack_create(ls.data(), (int)ls.size(), &S));
              return reinterpret_cast<uintptr_t>(S);
          },
          py::arg("layers"));
#define FT_STACK_CALL(NAME, FN)                                                           \
    m.def(NAME,                                                                           \
          [](uintptr_t S, uintptr_t x, uintptr_t y, const std::vector<uintptr_t>& kps,    \
             const std::vector<uintptr_t>& vps, uintptr_t table, uintptr_t lens, int batch, \
             int tbl_width, uintptr_t stream) {                                           \
              std::vector<void*> kp, vp;                                                  \
              for (uintptr_t a : kps) kp.push_back(P<void>(a));                           \
              for (uintptr_t a : vps) vp.push_back(P<void>(a));                           \
              check(FN(P<ft_decode_stack>(S), P<const void>(x), P<void>(y), kp.data(),     \
                       vp.data(), P<const int>(table), P<const int>(lens), batch,         \
                       tbl_width, stream));                                               \
          },                                                                              \
          py::arg("stack"), py::arg("x"), py::arg("y"), py::arg("k_pools"),               \
          py::arg("v_pools"), py::arg("table"), py::arg("lens"), py::arg("batch"),        \
          py::arg("tbl_width"), py::arg("stream") = 0)
    FT_STACK_CALL("decode_stack_forward", ft_decode_stack_forward);
    FT_STACK_CALL("decode_stack_capture", ft_decode_stack_capture);
#undef FT_STACK_CALL
    m.def("decode_stack_replay",
          [](uintptr_t S, uintptr_t stream) {
              check(ft_decode_stack_replay(P<ft_decode_stack>(S), stream));
          },
          py::arg("stack"), py::arg("stream") = 0);
    m.def("decode_stack_destroy",
          [](uintptr_t S) { check(ft_decode_stack_destroy(P<ft_decode_stack>(S))); },
          py::arg("stack"));
    m.def("rope_kv_append_paged_launch",
          [](uintptr_t qkv, int dtype, long long ld, uintptr_t lens, uintptr_t table,
             uintptr_t q_out, uintptr_t k_pool, uintptr_t v_pool, int batch,
             int q_heads, int kv_heads, int dim, int page, int tbl_width, float theta,
             int pos_offset, bool neox, uintptr_t stream) {
              check(ft_rope_kv_append_paged_launch(
                  P<const void>(qkv), dtype, ld, P<const int>(lens),
                  P<const int>(table), P<void>(q_out), P<void>(k_pool),
                  P<void>(v_pool), batch, q_heads, kv_heads, dim, page, tbl_width,
                  theta, pos_offset, neox ? 1 : 0, stream));
          },
          py::arg("qkv"), py::arg("dtype"), py::arg("ld"), py::arg("lens"),
          py::arg("table"), py::arg("q_out"), py::arg("k_pool"), py::arg("v_pool"),
          py::arg("batch"), py::arg("q_heads"), py::arg("kv_heads"), py::arg("dim"),
          py::arg("page"), py::arg("tbl_width"), py::arg("theta"),
          py::arg("pos_offset"), py::arg("neox"), py::arg("stream") = 0);
}
