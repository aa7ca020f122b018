// pybind11 module `cmpext3` (built as cmp_ext_amd/_cmpext3*.so): the Python
// surface of the MI355X GEMM library.  It mirrors the GEMM part of the
// reference bindings (src/main.cpp:155-357, :1594-1602) and adds the three
// dtype-specific matmul entry points.  Tensor checks and output allocation
// happen here; every product goes through the C ABI (cmpext3_gemm_prepare, then
// cmpext3_gemm_run with the workspace the plan asks for), which launches the
// hand-written gfx950 kernels on PyTorch's current stream.
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <climits>
#include <string>
#include <vector>

#include "../../include/cmpext3_gemm.h"

namespace {

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kHalf: return CMPEXT3_F16;
    case at::kBFloat16: return CMPEXT3_BF16;
    case at::kFloat: return CMPEXT3_F32;
    default: return -1;
  }
}

void* current_stream(const torch::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

void check_status(int st, const char* op) {
  TORCH_CHECK(st == CMPEXT3_OK, "cmpext3.", op, ": ", cmpext3_status_string(st));
}

int64_t checked_int(int64_t v, const char* what) {
  TORCH_CHECK(v <= INT_MAX, what, " = ", v, " exceeds the supported range (2^31 - 1)");
  return v;
}

// The prepared call each operator ran last on this thread (cmpext3.last_plan()).
thread_local cmpext3_gemm_call g_last_call;
thread_local bool g_has_last_call = false;

// Runs a prepared call on PyTorch's current stream of `like`'s device with the
// workspace its plan asks for (from PyTorch's caching allocator), so the
// kernel is chosen once per operator call.
void run_prepared(const cmpext3_gemm_call& call, const torch::Tensor& like, const char* op) {
  const int64_t need = cmpext3_gemm_call_workspace_size(&call);
  check_status(need < 0 ? (int)need : CMPEXT3_OK, op);
  torch::Tensor ws;
  if (need > 0) ws = torch::empty({need}, like.options().dtype(torch::kUInt8));
  check_status(cmpext3_gemm_run(&call, ws.defined() ? ws.data_ptr() : nullptr, need, current_stream(like)), op);
  g_last_call = call;
  g_has_last_call = true;
}

// Prepares C = A * op(B) (+ bias) for this call's exact pointers, pitches and
// strides (the bindings provide whatever workspace the plan wants) and runs it.
void gemm(int code, int layout, const torch::Tensor& a, int64_t lda, int64_t stride_a, const torch::Tensor& b,
          int64_t ldb, int64_t stride_b, torch::Tensor& c, int64_t ldc, int64_t stride_c, const void* bias,
          int flags, int64_t M, int64_t N, int64_t K, int64_t batch, const char* op) {
  cmpext3_gemm_call call;
  check_status(cmpext3_gemm_prepare(&call, code, layout, a.data_ptr(), lda, stride_a, b.data_ptr(), ldb, stride_b,
                                    c.data_ptr(), ldc, stride_c, bias, flags, (int)M, (int)N, (int)K, (int)batch,
                                    INT64_MAX),
               op);
  run_prepared(call, a, op);
}

// A 2-D operand usable as row-major with unit inner stride: returns the row
// pitch, or -1 if a copy is needed.
// Row pitches the kernels can address from a tile's base with 32-bit byte offsets (256 rows
// of 4-byte elements); a view with a larger pitch is copied instead.
constexpr int64_t kMaxPitch = INT_MAX / (256 * 4);

int64_t row_pitch(const torch::Tensor& t) {
  const int64_t rows = t.size(0), cols = t.size(1);
  if (cols > 1 && t.stride(1) != 1) return -1;
  if (rows <= 1) return std::max<int64_t>(cols, 1);
  if (t.stride(0) < std::max<int64_t>(cols, 1) || t.stride(0) > kMaxPitch) return -1;
  return t.stride(0);
}

// A 3-D operand [batch, rows, cols] whose matrices are row-major with unit inner stride:
// sets the row pitch and the batch stride (>= 0; batch entries may overlap, as in an
// expanded view, since operands are only read) and returns true; false if a copy is needed.
bool batch_rows(const torch::Tensor& t, int64_t& ld, int64_t& stride) {
  const int64_t rows = t.size(1), cols = t.size(2);
  if (cols > 1 && t.stride(2) != 1) return false;
  ld = rows <= 1 ? std::max<int64_t>(cols, 1) : t.stride(1);
  if (ld < std::max<int64_t>(cols, 1) || ld > kMaxPitch || t.stride(0) < 0) return false;
  stride = t.stride(0);
  return true;
}

// C = A[M,K] * B[K,N].  B may also be a transposed view of a row-major
// [N,K] tensor (e.g. W.t()), which is consumed in place with the NK layout.
torch::Tensor matmul_impl(const torch::Tensor& a_in, const torch::Tensor& b_in, at::ScalarType want,
                          const char* op) {
  TORCH_CHECK(a_in.dim() == 2 && b_in.dim() == 2, "cmpext3.", op, ": expected 2-D tensors, got ",
              a_in.dim(), "-D and ", b_in.dim(), "-D");
  TORCH_CHECK(a_in.scalar_type() == want && b_in.scalar_type() == want, "cmpext3.", op, ": expected ",
              c10::toString(want), " tensors, got ", a_in.scalar_type(), " and ", b_in.scalar_type());
  TORCH_CHECK(a_in.size(1) == b_in.size(0), "cmpext3.", op, ": shape mismatch ", a_in.sizes(), " x ",
              b_in.sizes());
  TORCH_CHECK(a_in.is_cuda() && b_in.is_cuda(), "cmpext3.", op, ": tensors must be on a GPU");
  TORCH_CHECK(a_in.device() == b_in.device(), "cmpext3.", op, ": device mismatch");
  const int64_t M = checked_int(a_in.size(0), "M"), K = checked_int(a_in.size(1), "K"),
                N = checked_int(b_in.size(1), "N");
  c10::DeviceGuard guard(a_in.device());
  torch::Tensor a = a_in;
  int64_t lda = row_pitch(a);
  if (lda < 0) {
    a = a.contiguous();
    lda = std::max<int64_t>(K, 1);
  }
  torch::Tensor b = b_in;
  int layout = CMPEXT3_B_KN;
  int64_t ldb = row_pitch(b);
  if (ldb < 0) {
    const torch::Tensor bt = b.t();  // [N, K]
    const int64_t pt = row_pitch(bt);
    if (pt >= 0) {
      layout = CMPEXT3_B_NK;
      ldb = pt;
    } else {
      b = b.contiguous();
      ldb = std::max<int64_t>(N, 1);
    }
  }
  torch::Tensor c = torch::empty({M, N}, a.options());
  gemm(dtype_code(want), layout, a, lda, 0, b, ldb, 0, c, std::max<int64_t>(N, 1), 0, nullptr, 0, M, N, K, 1, op);
  return c;
}

torch::Tensor fp16_matmul(const torch::Tensor& a, const torch::Tensor& b) {
  return matmul_impl(a, b, at::kHalf, "fp16_matmul");
}
torch::Tensor bf16_matmul(const torch::Tensor& a, const torch::Tensor& b) {
  return matmul_impl(a, b, at::kBFloat16, "bf16_matmul");
}
torch::Tensor fp32_matmul(const torch::Tensor& a, const torch::Tensor& b) {
  return matmul_impl(a, b, at::kFloat, "fp32_matmul");
}

// linear(input[..., K], weight[N, K], bias[N]) -> [..., N]
// Reference: custom_linear_forward, src/main.cpp:155-256.  The weight is read
// in place ([N,K] layout) instead of being transposed into a copy (:182), and
// the bias is added in the GEMM epilogue instead of a second kernel (:229-246).
torch::Tensor linear(torch::Tensor input, const torch::Tensor& weight, c10::optional<torch::Tensor> bias) {
  TORCH_CHECK(input.dim() >= 2, "Input dim >= 2");
  TORCH_CHECK(weight.dim() == 2, "Weight dim == 2");
  TORCH_CHECK(input.device() == weight.device(), "Device mismatch");
  TORCH_CHECK(input.scalar_type() == weight.scalar_type(), "Dtype mismatch");
  const int code = dtype_code(input.scalar_type());
  TORCH_CHECK(code >= 0, "Unsupported dtype");
  const int64_t N = weight.size(0), K = weight.size(1);
  TORCH_CHECK(input.size(-1) == K, "Input shape mismatch with Weight");
  TORCH_CHECK(input.is_cuda(), "cmpext3.linear: tensors must be on a GPU");
  c10::DeviceGuard guard(input.device());
  int64_t M = 1;
  for (int64_t d = 0; d + 1 < input.dim(); ++d) M *= input.size(d);
  checked_int(M, "M");
  checked_int(N, "N");
  checked_int(K, "K");
  // x as [M, K]: a 2-D input with rows of unit stride is read in place (its row pitch as
  // lda); any other non-contiguous input is copied
  torch::Tensor x = input;
  int64_t lda = input.dim() == 2 ? row_pitch(input) : -1;
  if (lda < 0) {
    x = input.contiguous().view({M, K});
    lda = std::max<int64_t>(K, 1);
  }
  // the weight read in place: [N, K] rows (B given as [N, K]), or a transposed view of a
  // [K, N] tensor (B given as [K, N]); otherwise copied
  torch::Tensor w = weight;
  int layout = CMPEXT3_B_NK;
  int64_t ldb = row_pitch(weight);
  if (ldb < 0) {
    const torch::Tensor wt = weight.t();  // [K, N]
    ldb = row_pitch(wt);
    if (ldb >= 0) {
      layout = CMPEXT3_B_KN;
      w = wt;
    } else {
      w = weight.contiguous();
      ldb = std::max<int64_t>(K, 1);
    }
  }
  const void* bias_ptr = nullptr;
  torch::Tensor bias_c;
  if (bias.has_value() && bias->defined()) {
    bias_c = *bias;
    TORCH_CHECK(bias_c.device() == input.device(), "Bias device mismatch");
    TORCH_CHECK(bias_c.scalar_type() == input.scalar_type(), "Bias dtype mismatch");
    TORCH_CHECK(bias_c.dim() == 1, "Bias must be 1D");
    TORCH_CHECK(bias_c.size(0) == N, "Bias size mismatch");
    bias_c = bias_c.contiguous();
    bias_ptr = bias_c.data_ptr();
  }
  std::vector<int64_t> out_shape(input.sizes().begin(), input.sizes().end() - 1);
  out_shape.push_back(N);
  torch::Tensor out = torch::empty(out_shape, input.options());
  gemm(code, layout, x, lda, 0, w, ldb, 0, out, std::max<int64_t>(N, 1), 0, bias_ptr, 0, M, N, K, 1, "linear");
  return out;
}

// bmm(input[B, M, K], mat2[B, K, N]) -> [B, M, N]
// Reference: custom_bmm_forward, src/main.cpp:273-357, which launches one
// GEMM per batch entry from a host loop (:313-351); here it is one launch.
torch::Tensor bmm(torch::Tensor input, torch::Tensor mat2) {
  TORCH_CHECK(input.dim() == 3, "Input must be 3D (B, M, K)");
  TORCH_CHECK(mat2.dim() == 3, "Mat2 must be 3D (B, K, N)");
  TORCH_CHECK(input.device() == mat2.device(), "Device mismatch");
  TORCH_CHECK(input.dtype() == mat2.dtype(), "Dtype mismatch");
  const int code = dtype_code(input.scalar_type());
  TORCH_CHECK(code >= 0, "Unsupported dtype for custom bmm");
  const int64_t Bn = input.size(0), M = input.size(1), K = input.size(2);
  const int64_t N = mat2.size(2);
  TORCH_CHECK(Bn == mat2.size(0), "Batch size mismatch");
  TORCH_CHECK(K == mat2.size(1), "Contracting dimension (K) mismatch");
  TORCH_CHECK(input.is_cuda(), "cmpext3.bmm: tensors must be on a GPU");
  checked_int(Bn, "batch");
  checked_int(M, "M");
  checked_int(N, "N");
  checked_int(K, "K");
  c10::DeviceGuard guard(input.device());
  // Operands read in place where their matrices have rows of unit stride: input as
  // [M, K] rows (its row pitch and batch stride), mat2 as [K, N] rows or as a transposed
  // view of [N, K] rows (B given as [N, K], e.g. the keys of Q K^T); otherwise copied.
  int64_t lda = 0, stride_a = 0;
  if (!batch_rows(input, lda, stride_a)) {
    input = input.contiguous();
    lda = std::max<int64_t>(K, 1);
    stride_a = M * K;
  }
  int layout = CMPEXT3_B_KN;
  int64_t ldb = 0, stride_b = 0;
  if (!batch_rows(mat2, ldb, stride_b)) {
    if (batch_rows(mat2.transpose(1, 2), ldb, stride_b)) {
      layout = CMPEXT3_B_NK;
    } else {
      mat2 = mat2.contiguous();
      ldb = std::max<int64_t>(N, 1);
      stride_b = K * N;
    }
  }
  torch::Tensor out = torch::empty({Bn, M, N}, input.options());
  gemm(code, layout, input, lda, Bn > 1 ? stride_a : 0, mat2, ldb, Bn > 1 ? stride_b : 0, out,
       std::max<int64_t>(N, 1), M * N, nullptr, 0, M, N, K, Bn, "bmm");
  return out;
}

// stride / padding / dilation as the reference parses them (src/main.cpp:140-148):
// an int means the same value for H and W, otherwise a sequence of ints.
std::vector<int64_t> expand_param(const py::object& v) {
  if (py::isinstance<py::int_>(v)) {
    const int64_t x = v.cast<int64_t>();
    return {x, x};
  }
  std::vector<int64_t> r = v.cast<std::vector<int64_t>>();
  TORCH_CHECK(!r.empty(), "cmpext3.conv2d: stride, padding and dilation need at least one value");
  return r;
}

// conv2d(input[B, C_in, H, W], weight[C_out, C_in, 1, 1], bias[C_out]) -> [B, C_out, H, W]
// Reference: custom_conv2d_forward, src/main.cpp:363-424 (checks :372-388, the
// 1x1 branch :402-424).  The reference runs that branch as permute to NHWC +
// linear on a contiguous copy + permute back into a second copy; here every
// image is one GEMM out_b = W * in_b on the NCHW data as it lies, with the
// bias added per output channel in the epilogue, all images in one launch.
// A channels-last input is read in place (B given as [H*W, C_in] per image), as the
// reference's permute to NHWC makes it contiguous at no cost there (:407); the output is
// NCHW-contiguous either way, as the reference's (:423).
// The reference's general direct-convolution kernels (launch_conv2d_*, :458-488)
// are not part of this library: any other kernel size, stride, padding or
// dilation raises.
torch::Tensor conv2d(torch::Tensor input, torch::Tensor weight, c10::optional<torch::Tensor> bias,
                     const py::object& stride, const py::object& padding, const py::object& dilation,
                     int64_t groups) {
  TORCH_CHECK(input.dim() == 4, "Input must be 4D (NCHW)");
  TORCH_CHECK(weight.dim() == 4, "Weight must be 4D (O I/G kH kW)");
  TORCH_CHECK(input.device() == weight.device(), "Device mismatch");
  TORCH_CHECK(groups == 1, "Currently only groups=1 is supported in this custom op");
  TORCH_CHECK(input.size(1) == weight.size(1), "Input channels mismatch weight channels");
  const std::vector<int64_t> s = expand_param(stride), pd = expand_param(padding), dl = expand_param(dilation);
  const int64_t s_h = s[0], s_w = s.size() > 1 ? s[1] : s[0];
  const int64_t p_h = pd[0], p_w = pd.size() > 1 ? pd[1] : pd[0];
  const int64_t d_h = dl[0], d_w = dl.size() > 1 ? dl[1] : dl[0];
  const int64_t kH = weight.size(2), kW = weight.size(3);
  TORCH_CHECK(kH == 1 && kW == 1 && s_h == 1 && s_w == 1 && p_h == 0 && p_w == 0 && d_h == 1 && d_w == 1,
              "cmpext3.conv2d: only the 1x1 kernel with stride 1, padding 0 and dilation 1 is provided "
              "(it runs on the GEMM path); got kernel ", kH, "x", kW, ", stride (", s_h, ", ", s_w,
              "), padding (", p_h, ", ", p_w, "), dilation (", d_h, ", ", d_w, ")");
  TORCH_CHECK(input.scalar_type() == weight.scalar_type(), "Dtype mismatch");
  const int code = dtype_code(input.scalar_type());
  TORCH_CHECK(code >= 0, "Unsupported dtype for custom_conv2d");
  TORCH_CHECK(input.is_cuda(), "cmpext3.conv2d: tensors must be on a GPU");
  const int64_t Bn = input.size(0), Cin = input.size(1), H = input.size(2), W = input.size(3);
  const int64_t Cout = weight.size(0);
  checked_int(Bn, "batch");
  checked_int(Cin, "C_in");
  checked_int(Cout, "C_out");
  const int64_t hw = checked_int(H * W, "H*W");
  c10::DeviceGuard guard(input.device());
  // A channels-last (NHWC) input is read as it lies: image b is then [H*W, C_in], B given as
  // [N, K]; any other layout is made NCHW-contiguous.
  const bool nhwc = !input.is_contiguous() && input.is_contiguous(at::MemoryFormat::ChannelsLast);
  if (!nhwc) input = input.contiguous();
  weight = weight.contiguous();
  const void* bias_ptr = nullptr;
  torch::Tensor bias_c;
  if (bias.has_value() && bias->defined()) {
    bias_c = *bias;
    TORCH_CHECK(bias_c.device() == input.device(), "Bias device mismatch");
    TORCH_CHECK(bias_c.scalar_type() == input.scalar_type(), "Bias dtype mismatch");
    TORCH_CHECK(bias_c.dim() == 1, "Bias must be 1D");
    TORCH_CHECK(bias_c.size(0) == Cout, "Bias size mismatch");
    bias_c = bias_c.contiguous();
    bias_ptr = bias_c.data_ptr();
  }
  torch::Tensor out = torch::empty({Bn, Cout, H, W}, input.options());
  // the GEMMs of cmpext3_conv2d_1x1: out_b[C_out, HW] = W[C_out, C_in] * in_b[C_in, HW] for
  // every image b, the weight shared (stride 0), the bias per output row; from an NHWC
  // input, out_b = W * (in_b[HW, C_in])^T
  if (nhwc)
    gemm(code, CMPEXT3_B_NK, weight, std::max<int64_t>(Cin, 1), 0, input, std::max<int64_t>(Cin, 1), hw * Cin,
         out, std::max<int64_t>(hw, 1), Cout * hw, bias_ptr, CMPEXT3_BIAS_PER_ROW, Cout, hw, Cin, Bn, "conv2d");
  else
    gemm(code, CMPEXT3_B_KN, weight, std::max<int64_t>(Cin, 1), 0, input, std::max<int64_t>(hw, 1), Cin * hw,
         out, std::max<int64_t>(hw, 1), Cout * hw, bias_ptr, CMPEXT3_BIAS_PER_ROW, Cout, hw, Cin, Bn, "conv2d");
  return out;
}

std::string plan(const std::string& dtype, int64_t M, int64_t N, int64_t K, const std::string& layout,
                 int64_t batch, bool has_bias) {
  int code = dtype == "f16" || dtype == "fp16" ? CMPEXT3_F16
             : dtype == "bf16"                  ? CMPEXT3_BF16
             : dtype == "f32" || dtype == "fp32" ? CMPEXT3_F32
                                                : -1;
  const int lay = layout == "NK" ? CMPEXT3_B_NK : CMPEXT3_B_KN;
  const int64_t ldb = lay == CMPEXT3_B_KN ? N : K;
  char buf[640];
  // packed operands at 16-byte aligned addresses, and the workspace the plan asks for
  // (what the bindings provide); cmpext3.last_plan() reports what a call actually ran
  const int st = cmpext3_gemm_plan(code, lay, (int)M, (int)N, (int)K, std::max<int64_t>(K, 1),
                                   std::max<int64_t>(ldb, 1), std::max<int64_t>(N, 1), 16, has_bias ? 1 : 0,
                                   (int)batch, INT64_MAX, buf, sizeof buf);
  TORCH_CHECK(st >= 0, "cmpext3.plan: ", cmpext3_status_string(st));
  return std::string(buf);
}

std::string last_plan() {
  TORCH_CHECK(g_has_last_call, "cmpext3.last_plan: no operator has run on this thread yet");
  char buf[640];
  const int st = cmpext3_gemm_call_describe(&g_last_call, buf, sizeof buf);
  TORCH_CHECK(st >= 0, "cmpext3.last_plan: ", cmpext3_status_string(st));
  return std::string(buf);
}

}  // namespace

PYBIND11_MODULE(_cmpext3, m) {
  m.doc() = "cmpext3 dense GEMM operators for AMD Instinct MI355X (gfx950)";
  m.def("fp16_matmul", &fp16_matmul, "C = A @ B for fp16 (fp32 accumulate)", py::arg("a"), py::arg("b"));
  m.def("bf16_matmul", &bf16_matmul, "C = A @ B for bf16 (fp32 accumulate)", py::arg("a"), py::arg("b"));
  m.def("fp32_matmul", &fp32_matmul, "C = A @ B for fp32", py::arg("a"), py::arg("b"));
  m.def("linear", &linear, "Custom linear layer implementation", py::arg("input"), py::arg("weight"),
        py::arg("bias") = py::none());
  m.def("bmm", &bmm, "Custom Batch Matrix Multiplication", py::arg("input"), py::arg("mat2"));
  m.def("conv2d", &conv2d, "Custom conv2d layer (1x1, stride 1, padding 0: runs as a GEMM)", py::arg("input"),
        py::arg("weight"), py::arg("bias") = py::none(), py::arg("stride") = 1, py::arg("padding") = 0,
        py::arg("dilation") = 1, py::arg("groups") = 1);
  m.def("plan", &plan, "Describe the kernel chosen for a GEMM shape", py::arg("dtype"), py::arg("M"),
        py::arg("N"), py::arg("K"), py::arg("layout") = "KN", py::arg("batch") = 1,
        py::arg("has_bias") = false);
  m.def("last_plan", &last_plan,
        "Describe the kernel(s) the last operator call on this thread ran (its actual pointers, pitches and "
        "workspace)");
  m.def("version", []() { return std::string(cmpext3_version()); });
}
