// bindings.cpp -- the my_int4._C drop-in: the reference's 16 pybind11 ops
// (csrc/bindings.cpp:28-68) with the same names, argument names, argument
// meaning, output dtypes/shapes and TORCH_CHECK error behaviour.  Each op
// validates and allocates with torch on the input's device, takes torch's
// current HIP stream, and calls the C ABI of libwush_int4.so
// (include/wush_int4.h).  No computation happens here.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <vector>

#include "wush_int4.h"

namespace {

hipStream_t current_stream(const torch::Tensor& t) {
    return at::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

void check_status(int st, const char* op) {
    TORCH_CHECK(st == 0, "my_int4._C.", op, ": ", wush_error_string(st));
}

template <typename T>
T* ptr(const torch::Tensor& t) {
    return reinterpret_cast<T*>(t.data_ptr());
}

std::vector<int64_t> with_last(const torch::Tensor& t, int64_t last) {
    std::vector<int64_t> s = t.sizes().vec();
    s.back() = last;
    return s;
}

// quant_int4 (csrc/quant_int4.cu:109-134).  Also accepts fp16/fp32 input,
// which my_int4/rtn_int4.py:36 quantizes the same way.
std::vector<torch::Tensor> quant_int4(torch::Tensor x) {
    TORCH_CHECK(x.is_cuda() && x.is_contiguous(), "x must be contiguous CUDA tensor");
    const auto dt = x.scalar_type();
    TORCH_CHECK(dt == torch::kBFloat16 || dt == torch::kHalf || dt == torch::kFloat32,
                "x must be bf16 (fp16 and fp32 are also accepted)");
    TORCH_CHECK(x.dim() >= 1 && x.size(-1) % 32 == 0, "last dim must be multiple of 32");
    const at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    const int64_t n_groups = x.numel() / 32;
    auto q = torch::empty({x.numel() / 2}, torch::dtype(torch::kUInt8).device(x.device()));
    auto s = torch::empty({n_groups}, torch::dtype(torch::kBFloat16).device(x.device()));
    const int code = dt == torch::kBFloat16 ? WUSH_DTYPE_BF16 : (dt == torch::kHalf ? WUSH_DTYPE_F16 : WUSH_DTYPE_F32);
    check_status(wush_quant_int4(x.data_ptr(), code, ptr<uint8_t>(q), ptr<uint16_t>(s), n_groups,
                                 current_stream(x)),
                 "quant_int4");
    return {q.view(with_last(x, x.size(-1) / 2)), s.view(with_last(x, x.size(-1) / 32))};
}

// fused_transform_quant_int4 and its variants (csrc/fused_tq_int4.cu:87-118,
// fused_tq_smallm.cu:89-121, fused_tq_v3.cu:109-140, fused_tq_wmma.cu:131-162):
// one bit-exact implementation serves all four names.
std::vector<torch::Tensor> fused_tq_impl(torch::Tensor x, torch::Tensor t, bool need_rows) {
    TORCH_CHECK(x.is_cuda() && x.is_contiguous() && t.is_cuda() && t.is_contiguous(),
                "x/t must be contiguous CUDA tensors");
    TORCH_CHECK(x.scalar_type() == torch::kBFloat16 && t.scalar_type() == torch::kBFloat16,
                "x/t must be bf16");
    TORCH_CHECK(x.dim() >= 1, "x must have a last dimension");
    const int64_t K = x.size(-1);
    const int64_t C = K / 32;
    TORCH_CHECK(K % 32 == 0 && t.dim() == 3 && t.size(0) == C && t.size(1) == 32 && t.size(2) == 32,
                "T must be (K/32, 32, 32)");
    const int64_t rows = K ? x.numel() / K : 0;
    if (need_rows) TORCH_CHECK(rows >= 1, "rows must be >= 1");
    const at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    auto q = torch::empty({rows * C * 16}, torch::dtype(torch::kUInt8).device(x.device()));
    auto s = torch::empty({rows * C}, torch::dtype(torch::kBFloat16).device(x.device()));
    check_status(wush_fused_tq(ptr<uint16_t>(x), ptr<uint16_t>(t), ptr<uint8_t>(q), ptr<uint16_t>(s),
                               rows, K, current_stream(x)),
                 "fused_transform_quant_int4");
    return {q.view(with_last(x, K / 2)), s.view(with_last(x, C))};
}

std::vector<torch::Tensor> fused_transform_quant_int4(torch::Tensor x, torch::Tensor t) {
    return fused_tq_impl(x, t, false);
}
std::vector<torch::Tensor> fused_transform_quant_int4_smallm(torch::Tensor x, torch::Tensor t) {
    return fused_tq_impl(x, t, true);
}
std::vector<torch::Tensor> fused_transform_quant_int4_v3(torch::Tensor x, torch::Tensor t) {
    return fused_tq_impl(x, t, false);
}
std::vector<torch::Tensor> fused_transform_quant_int4_wmma(torch::Tensor x, torch::Tensor t) {
    return fused_tq_impl(x, t, false);
}

// Common checks of the packed GEMM operands (csrc/gemm_s4.cu:323-338).
void check_packed(const torch::Tensor& xq, const torch::Tensor& xs, const torch::Tensor& wq,
                  const torch::Tensor& ws) {
    TORCH_CHECK(xq.is_cuda() && wq.is_cuda(), "tensors must be CUDA");
    TORCH_CHECK(xq.scalar_type() == torch::kUInt8 && wq.scalar_type() == torch::kUInt8,
                "packed tensors must be uint8");
    TORCH_CHECK(xs.scalar_type() == torch::kBFloat16 && ws.scalar_type() == torch::kBFloat16,
                "scales must be bf16");
    TORCH_CHECK(xq.is_contiguous() && xs.is_contiguous() && wq.is_contiguous() && ws.is_contiguous(),
                "tensors must be contiguous");
    TORCH_CHECK(xs.is_cuda() && ws.is_cuda(), "tensors must be CUDA");
}

// Which kernel family computes a product with M activation rows.  Both give
// the same math (exact int32 group dots folded in fp32).  Measured on MI355X
// with the weights streamed from HBM: the dot8 streaming GEMV
// (wush_gemv_int4) is faster at M <= 4 on every shape and at every M <= 8 on
// the Llama-70B FFN weights (K=8192 N=57344 M=8: 51.8 vs 55.4 us); the
// K-split int8-MFMA streaming GEMM (wush_gemm_s4) is faster at 5 <= M <= 8
// when N <= 24576 (K=N=4096 M=8: 5.8 vs 7.2 us; K=N=8192 M=8: 11.9 vs
// 13.3 us; K=4096 N=24576 M=8: 14.3 vs 15.0 us).  Which shapes the GEMV
// takes at all (its LDS staging limit, and the K-split kernel's shapes) is
// the library's rule, which its build-time tuning macros change, so it is
// asked, not restated here.
bool gemv_preferred(int64_t M, int64_t N, int64_t K) {
    return wush_gemv_int4_supported(M, N, K) != 0 && (M <= 4 || N > 32768);
}

// Shared product launch: y (M, N) fp16 = group-scaled product.
torch::Tensor product_2d(const torch::Tensor& xq2, const torch::Tensor& xs2, const torch::Tensor& wq,
                         const torch::Tensor& ws, int64_t K, const char* op) {
    const int64_t M = xq2.size(0), N = wq.size(0);
    const at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(xq2.device());
    auto y = torch::empty({M, N}, torch::dtype(torch::kHalf).device(xq2.device()));
    if (gemv_preferred(M, N, K)) {
        check_status(wush_gemv_int4(ptr<uint8_t>(xq2), ptr<uint16_t>(xs2), ptr<uint8_t>(wq), ptr<uint16_t>(ws),
                                    ptr<uint16_t>(y), M, N, K, current_stream(xq2)),
                     op);
        return y;
    }
    const size_t wsb = wush_gemm_s4_workspace_bytes(M, N, K);
    torch::Tensor work;
    if (wsb) work = torch::empty({(int64_t)wsb}, torch::dtype(torch::kUInt8).device(xq2.device()));
    check_status(wush_gemm_s4(ptr<uint8_t>(xq2), ptr<uint16_t>(xs2), ptr<uint8_t>(wq), ptr<uint16_t>(ws),
                              ptr<uint16_t>(y), M, N, K, wsb ? work.data_ptr() : nullptr, wsb,
                              current_stream(xq2)),
                 op);
    return y;
}

// w4a4_gemm_s4 (csrc/gemm_s4.cu:320-379): y (M, N) fp16, K % 64 == 0.
torch::Tensor w4a4_gemm_s4(torch::Tensor xq, torch::Tensor xs, torch::Tensor wq, torch::Tensor ws) {
    check_packed(xq, xs, wq, ws);
    const int64_t K2 = xq.size(-1);
    const int64_t K = K2 * 2, G = K / 32;
    TORCH_CHECK(K % 64 == 0, "K must be multiple of 64");
    auto xq2 = xq.reshape({-1, K2});
    auto xs2 = xs.reshape({-1, G});
    TORCH_CHECK(wq.dim() == 2 && wq.size(1) == K2 && ws.size(-1) == G && ws.numel() == wq.size(0) * G,
                "K mismatch");
    TORCH_CHECK(xs2.size(0) == xq2.size(0), "K mismatch");
    return product_2d(xq2, xs2, wq, ws, K, "w4a4_gemm_s4");
}

// w4a4_gemm (csrc/gemm_int4.cu:89-130): y keeps xq's leading dims, (..., N).
torch::Tensor w4a4_gemm(torch::Tensor xq, torch::Tensor xs, torch::Tensor wq, torch::Tensor ws) {
    check_packed(xq, xs, wq, ws);
    TORCH_CHECK(wq.dim() == 2, "w must be 2D (N, K/2)");
    const int64_t K2 = xq.size(-1);
    const int64_t K = K2 * 2, G = K / 32;
    TORCH_CHECK(K % 32 == 0 && wq.size(1) == K2 && ws.size(-1) == G && xs.size(-1) == G,
                "K mismatch between x/w tensors");
    auto xq2 = xq.view({-1, K2});
    auto xs2 = xs.reshape({-1, G});
    auto y = product_2d(xq2, xs2, wq, ws, K, "w4a4_gemm");
    return y.view(with_last(xq, wq.size(0)));
}

// w4a4_gemm_v1 (csrc/gemm_wmma.cu:128-172): y (M, N).
torch::Tensor w4a4_gemm_v1(torch::Tensor xq, torch::Tensor xs, torch::Tensor wq, torch::Tensor ws) {
    check_packed(xq, xs, wq, ws);
    const int64_t K2 = xq.size(-1);
    const int64_t K = K2 * 2, G = K / 32;
    TORCH_CHECK(K % 32 == 0 && wq.dim() == 2 && wq.size(1) == K2 && ws.size(-1) == G, "K mismatch");
    return product_2d(xq.reshape({-1, K2}), xs.reshape({-1, G}), wq, ws, K, "w4a4_gemm_v1");
}

// w4a4_gemm_v2 (csrc/gemm_wmma2.cu:141-181): y (M, N), K % 64 == 0.
torch::Tensor w4a4_gemm_v2(torch::Tensor xq, torch::Tensor xs, torch::Tensor wq, torch::Tensor ws) {
    check_packed(xq, xs, wq, ws);
    const int64_t K2 = xq.size(-1);
    const int64_t K = K2 * 2, G = K / 32;
    TORCH_CHECK(K % 64 == 0, "K must be multiple of 64");
    TORCH_CHECK(wq.dim() == 2 && wq.size(1) == K2 && ws.size(-1) == G, "K mismatch");
    return product_2d(xq.reshape({-1, K2}), xs.reshape({-1, G}), wq, ws, K, "w4a4_gemm_v2");
}

// w4a4_gemv (csrc/gemv_int4.cu:191-223): single row, y (N,) fp16.
torch::Tensor w4a4_gemv(torch::Tensor xq, torch::Tensor xs, torch::Tensor wq, torch::Tensor ws) {
    check_packed(xq, xs, wq, ws);
    TORCH_CHECK(xq.dim() <= 2 && xq.numel() == xq.size(-1), "gemv expects a single row");
    const int64_t K2 = xq.size(-1);
    const int64_t K = K2 * 2, G = K / 32;
    TORCH_CHECK(K % 32 == 0 && wq.dim() == 2 && wq.size(1) == K2 && ws.size(-1) == G && xs.numel() == G,
                "K mismatch");
    auto y = product_2d(xq.reshape({1, K2}), xs.reshape({1, G}), wq, ws, K, "w4a4_gemv");
    return y.view({wq.size(0)});
}

// w4a4_gemv_multi (csrc/gemv_int4.cu:145-189): 1 <= M <= 8, y (M, N) fp16.
torch::Tensor w4a4_gemv_multi(torch::Tensor xq, torch::Tensor xs, torch::Tensor wq, torch::Tensor ws) {
    check_packed(xq, xs, wq, ws);
    const int64_t K2 = xq.size(-1);
    const int64_t K = K2 * 2, G = K / 32;
    auto xq2 = xq.reshape({-1, K2});
    auto xs2 = xs.reshape({-1, G});
    const int64_t M = xq2.size(0);
    TORCH_CHECK(M >= 1 && M <= 8, "gemv_multi expects 1<=M<=8");
    TORCH_CHECK(K % 32 == 0 && wq.dim() == 2 && wq.size(1) == K2 && ws.size(-1) == G && xs2.size(0) == M,
                "K mismatch");
    return product_2d(xq2, xs2, wq, ws, K, "w4a4_gemv_multi");
}

// s4_atom_selftest (csrc/gemm_s4.cu:74-82): c (8, 8) int32 = a (8, 32) @ b (32, 8).
torch::Tensor s4_atom_selftest(torch::Tensor a, torch::Tensor b) {
    TORCH_CHECK(a.is_cuda() && b.is_cuda() && a.is_contiguous() && b.is_contiguous(),
                "a/b must be contiguous CUDA tensors");
    TORCH_CHECK(a.scalar_type() == torch::kInt8 && b.scalar_type() == torch::kInt8, "a/b must be int8");
    TORCH_CHECK(a.numel() == 256 && b.numel() == 256, "a must be (8, 32) and b (32, 8)");
    const at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(a.device());
    auto c = torch::zeros({8, 8}, torch::dtype(torch::kInt32).device(a.device()));
    check_status(wush_mfma_selftest(ptr<int8_t>(a), ptr<int8_t>(b), ptr<int32_t>(c), current_stream(a)),
                 "s4_atom_selftest");
    return c;
}

// quant_int4_tensor_scale (csrc/fast_path.cu:42-59): flat (numel/2) codes,
// inverse scale (float)(1.0 / scale) computed in double like the reference.
torch::Tensor quant_int4_tensor_scale(torch::Tensor x, double scale) {
    TORCH_CHECK(x.is_cuda() && x.is_contiguous() && x.scalar_type() == torch::kBFloat16,
                "x must be contiguous CUDA bf16");
    TORCH_CHECK(x.numel() % 32 == 0, "numel must be multiple of 32");
    const at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    auto q = torch::empty({x.numel() / 2}, torch::dtype(torch::kUInt8).device(x.device()));
    const float inv = (float)(1.0 / scale);
    check_status(wush_quant_int4_tensor_scale(ptr<uint16_t>(x), ptr<uint8_t>(q), x.numel(), inv, nullptr,
                                              current_stream(x)),
                 "quant_int4_tensor_scale");
    return q;
}

// quant_int4_tensor_scale_dev (csrc/fast_path.cu:92-109).
torch::Tensor quant_int4_tensor_scale_dev(torch::Tensor x, torch::Tensor inv_scale) {
    TORCH_CHECK(x.is_cuda() && x.is_contiguous() && x.scalar_type() == torch::kBFloat16,
                "x must be contiguous CUDA bf16");
    TORCH_CHECK(x.numel() % 32 == 0, "numel must be multiple of 32");
    TORCH_CHECK(inv_scale.is_cuda() && inv_scale.scalar_type() == torch::kFloat32 &&
                    inv_scale.is_contiguous() && inv_scale.numel() == 1,
                "inv_scale must be 1-elem contiguous fp32 CUDA tensor");
    const at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(x.device());
    auto q = torch::empty({x.numel() / 2}, torch::dtype(torch::kUInt8).device(x.device()));
    check_status(wush_quant_int4_tensor_scale(ptr<uint16_t>(x), ptr<uint8_t>(q), x.numel(), 0.0f,
                                              ptr<float>(inv_scale), current_stream(x)),
                 "quant_int4_tensor_scale_dev");
    return q;
}

// w4a4_gemm_cutlass / _dev (csrc/gemm_cutlass_int4.cu:132-188): K from wq,
// xq 1-D or 2-D, y (M, N) fp16 = alpha * xq @ wq^T.
torch::Tensor gemm_tensor_scale_impl(torch::Tensor xq, torch::Tensor wq, double alpha,
                                     const torch::Tensor* alpha_dev, const char* op) {
    TORCH_CHECK(xq.is_cuda() && wq.is_cuda(), "tensors must be CUDA");
    TORCH_CHECK(xq.scalar_type() == torch::kUInt8 && wq.scalar_type() == torch::kUInt8,
                "packed tensors must be uint8");
    TORCH_CHECK(xq.is_contiguous() && wq.is_contiguous(), "tensors must be contiguous");
    TORCH_CHECK(wq.dim() == 2, "w must be 2D (N, K/2)");
    const int64_t K2 = wq.size(1);
    TORCH_CHECK(K2 > 0, "K must be positive");
    const int64_t M = xq.numel() / K2;
    TORCH_CHECK(M * K2 == xq.numel(), "xq numel must equal M*K/2 (K from wq)");
    TORCH_CHECK((2 * K2) % 32 == 0, "K must be a multiple of 32");
    TORCH_CHECK(2 * K2 <= WUSH_TENSOR_SCALE_MAX_K, "K must be <= ", WUSH_TENSOR_SCALE_MAX_K,
                " (the per-tensor GEMM's int32 accumulator holds 256 * sum(qx * qw))");
    const int64_t N = wq.size(0);
    const at::hip::OptionalHIPGuardMasqueradingAsCUDA guard(xq.device());
    auto y = torch::empty({M, N}, torch::dtype(torch::kHalf).device(xq.device()));
    check_status(wush_gemm_s4_tensor_scale(ptr<uint8_t>(xq), ptr<uint8_t>(wq), ptr<uint16_t>(y), M, N,
                                           2 * K2, (float)alpha,
                                           alpha_dev ? ptr<float>(*alpha_dev) : nullptr, current_stream(xq)),
                 op);
    return y;
}

torch::Tensor w4a4_gemm_cutlass(torch::Tensor xq, torch::Tensor wq, double alpha) {
    return gemm_tensor_scale_impl(xq, wq, alpha, nullptr, "w4a4_gemm_cutlass");
}

torch::Tensor w4a4_gemm_cutlass_dev(torch::Tensor xq, torch::Tensor wq, torch::Tensor alpha) {
    TORCH_CHECK(alpha.is_cuda() && alpha.scalar_type() == torch::kFloat32 && alpha.is_contiguous() &&
                    alpha.numel() == 1,
                "alpha must be 1-elem contiguous fp32 CUDA tensor");
    return gemm_tensor_scale_impl(xq, wq, 0.0, &alpha, "w4a4_gemm_cutlass_dev");
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "my_int4._C on MI355X: HIP/gfx950 kernels behind the reference op signatures";
    // One-time per-device set-up (launch attributes, occupancy tables) at
    // import, so that no op run inside a HIP graph capture has to do it.
    // Without a GPU this reports hipErrorNoDevice; the ops then report errors
    // themselves when called.
    m.attr("setup_status") = wush_init();
    m.def("quant_int4_tensor_scale", &quant_int4_tensor_scale, "Per-tensor INT4 quantize",
          py::arg("x"), py::arg("scale"));
    m.def("quant_int4_tensor_scale_dev", &quant_int4_tensor_scale_dev,
          "Per-tensor INT4 quantize, inv_scale from a 1-elem fp32 device tensor", py::arg("x"),
          py::arg("inv_scale"));
    m.def("quant_int4", &quant_int4, "INT4 sigma-clip group quantize (G=32, bf16 scale)", py::arg("x"));
    m.def("w4a4_gemm", &w4a4_gemm, "W4A4 group-scaled matmul (y keeps xq's leading dims)", py::arg("xq"),
          py::arg("xs"), py::arg("wq"), py::arg("ws"));
    m.def("w4a4_gemm_v1", &w4a4_gemm_v1, "W4A4 group-scaled matmul", py::arg("xq"), py::arg("xs"),
          py::arg("wq"), py::arg("ws"));
    m.def("w4a4_gemm_cutlass", &w4a4_gemm_cutlass, "W4A4 per-tensor matmul on int8 MFMA", py::arg("xq"),
          py::arg("wq"), py::arg("alpha"));
    m.def("w4a4_gemm_cutlass_dev", &w4a4_gemm_cutlass_dev,
          "W4A4 per-tensor matmul, alpha from a 1-elem fp32 device tensor", py::arg("xq"), py::arg("wq"),
          py::arg("alpha"));
    m.def("w4a4_gemm_s4", &w4a4_gemm_s4,
          "W4A4 group-scaled matmul: int8 MFMA with exact int32 group dots below prefill sizes, fp16 MFMA on "
          "code*scale operands for prefill (M >= 256)",
          py::arg("xq"),
          py::arg("xs"), py::arg("wq"), py::arg("ws"));
    m.def("s4_atom_selftest", &s4_atom_selftest, "verify the int8 MFMA fragment layout");
    m.def("w4a4_gemv", &w4a4_gemv, "W4A4 INT4 gemv (M=1 decode path)", py::arg("xq"), py::arg("xs"),
          py::arg("wq"), py::arg("ws"));
    m.def("w4a4_gemv_multi", &w4a4_gemv_multi, "W4A4 INT4 gemv, 1<=M<=8 (batched decode)", py::arg("xq"),
          py::arg("xs"), py::arg("wq"), py::arg("ws"));
    m.def("fused_transform_quant_int4_v3", &fused_transform_quant_int4_v3,
          "Fused WUSH transform + INT4 quantize (bit-exact)", py::arg("x"), py::arg("t"));
    m.def("fused_transform_quant_int4_smallm", &fused_transform_quant_int4_smallm,
          "Fused WUSH transform + INT4 quantize (bit-exact)", py::arg("x"), py::arg("t"));
    m.def("fused_transform_quant_int4", &fused_transform_quant_int4,
          "Fused WUSH transform + INT4 quantize (bit-exact)", py::arg("x"), py::arg("t"));
    m.def("w4a4_gemm_v2", &w4a4_gemm_v2, "W4A4 group-scaled matmul (K % 64 == 0)", py::arg("xq"),
          py::arg("xs"), py::arg("wq"), py::arg("ws"));
    m.def("fused_transform_quant_int4_wmma", &fused_transform_quant_int4_wmma,
          "Fused WUSH transform + INT4 quantize (bit-exact)", py::arg("x"), py::arg("t"));
    m.def("abi_version", &wush_abi_version, "C ABI version of libwush_int4.so");
}
