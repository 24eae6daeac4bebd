// custom_cuda_kernals_amd._native: the validating binding layer between the
// Python API and the C ABI of libcustom_kernels_amd.so.
//
// It restates the observable behaviour of the reference's Rust/PyO3 module
// `custom_cuda._native` (src/lib.rs:11-29, src/kernels/*.rs) in C++:
//   * the same function names and positional arguments, returning None;
//   * the same per-tensor checks in the same order (device type "cuda" ->
//     contiguity -> dtype tag), read through the same Python attributes
//     (device.type, is_contiguous(), str(dtype), data_ptr(), device.index,
//     shape) - src/kernels/tensor.rs:38-121;
//   * the same error mapping: validation failures raise ValueError,
//     a non-zero launcher status raises RuntimeError
//     (src/kernels/error.rs:9-36);
//   * launches on torch.cuda.current_stream(device_index).cuda_stream
//     (src/kernels/rmsnorm_residual.rs:87-94); no synchronisation. The
//     tensors' device is made current for the launch and restored after it
//     (a device guard, as torch's own ops use).
// A torch.Tensor is read through its at::Tensor (device, contiguity, dtype,
// data pointer, shape: no Python calls, about 0.2 us per tensor against 0.8
// through the attributes); any other object goes through the Python
// attributes the reference reads. Both give the same checks in the same
// order with the same messages. The current stream comes from c10's HIP
// stream registry, which torch.cuda.current_stream reads too. The kernels are
// reached through the C ABI only.
#include <torch/csrc/autograd/python_variable.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <atomic>
#include <cstdint>
#include <optional>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/custom_kernels_amd.h"

namespace py = pybind11;

namespace {

enum Tag : int32_t { F32 = 0, F16 = 1, BF16 = 2, F8E4M3 = 3, F8E5M2 = 4 };

const char* tag_debug(int32_t t) {
  switch (t) {
    case F32: return "F32";
    case F16: return "F16";
    case BF16: return "BF16";
    case F8E4M3: return "F8E4M3";
    case F8E5M2: return "F8E5M2";
    default: return "?";
  }
}

const char* tag_to_dtype_str(int32_t t) {
  switch (t) {
    case F32: return "torch.float32";
    case F16: return "torch.float16";
    case BF16: return "torch.bfloat16";
    case F8E4M3: return "torch.float8_e4m3fn";
    default: return "torch.float8_e5m2";
  }
}

std::optional<int32_t> tag_from_dtype_str(const std::string& s) {
  if (s == "torch.float32") return F32;
  if (s == "torch.float16") return F16;
  if (s == "torch.bfloat16") return BF16;
  if (s == "torch.float8_e4m3fn") return F8E4M3;
  if (s == "torch.float8_e5m2") return F8E5M2;
  return std::nullopt;
}

std::string shape_str(const std::vector<int64_t>& v) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < v.size(); ++i) o << (i ? ", " : "") << v[i];
  o << "]";
  return o.str();
}

[[noreturn]] void value_error(const std::string& msg) { throw py::value_error(msg); }
[[noreturn]] void shape_mismatch(const std::string& msg) { value_error("shape mismatch: " + msg); }
[[noreturn]] void unsupported_dtype(const std::string& what) {
  value_error("unsupported dtype '" + what + "'; expected float32, float16, or bfloat16");
}

struct RawView {
  uintptr_t ptr;
  int64_t device_index;
  std::vector<int64_t> shape;
  std::string dtype_str;
  int32_t tag = -1;  // the dtype tag when dtype_str is one of the five tagged dtypes
};

struct View {
  uintptr_t ptr;
  int32_t dtype;
  int64_t device_index;
  std::vector<int64_t> shape;
};

// Python objects looked up once per process (the GIL is held in every bound
// function). They are never released: destroying them after the interpreter
// has shut down would be unsafe.
struct PyCache {
  py::object dtypes[5];  // torch.float32 .. torch.float8_e5m2, indexed by tag
};

const PyCache& py_cache() {
  static PyCache* c = [] {
    auto* p = new PyCache;
    py::module_ torch = py::module_::import("torch");
    const char* names[5] = {"float32", "float16", "bfloat16", "float8_e4m3fn", "float8_e5m2"};
    for (int i = 0; i < 5; ++i) p->dtypes[i] = torch.attr(names[i]);
    return p;
  }();
  return *c;
}

// The tag of a tagged scalar type, -1 otherwise.
int32_t tag_of(c10::ScalarType t) {
  switch (t) {
    case c10::ScalarType::Float: return F32;
    case c10::ScalarType::Half: return F16;
    case c10::ScalarType::BFloat16: return BF16;
    case c10::ScalarType::Float8_e4m3fn: return F8E4M3;
    case c10::ScalarType::Float8_e5m2: return F8E5M2;
    default: return -1;
  }
}

RawView validate_and_extract(const char* name, const py::handle& obj) {
  if (THPVariable_Check(obj.ptr())) {
    const at::Tensor& t = THPVariable_Unpack(obj.ptr());
    const c10::Device dev = t.device();
    if (dev.type() != c10::DeviceType::CUDA) {
      value_error(std::string("argument '") + name + "' must be a CUDA tensor, got device type '" +
                  c10::DeviceTypeName(dev.type(), /*lower_case=*/true) + "'");
    }
    if (!t.is_contiguous()) value_error(std::string("argument '") + name + "' must be contiguous");
    RawView v;
    v.tag = tag_of(t.scalar_type());
    if (v.tag >= 0) {
      v.dtype_str = tag_to_dtype_str(v.tag);
    } else if (t.scalar_type() == c10::ScalarType::Int) {
      v.dtype_str = "torch.int32";
    } else if (t.scalar_type() == c10::ScalarType::Long) {
      v.dtype_str = "torch.int64";
    } else {
      v.dtype_str = py::str(obj.attr("dtype"));
    }
    v.ptr = reinterpret_cast<uintptr_t>(t.data_ptr());
    v.device_index = dev.index();
    const c10::IntArrayRef sizes = t.sizes();
    v.shape.assign(sizes.begin(), sizes.end());
    return v;
  }
  py::object device = obj.attr("device");
  const std::string device_type = py::str(device.attr("type"));
  if (device_type != "cuda") {
    value_error(std::string("argument '") + name + "' must be a CUDA tensor, got device type '" +
                device_type + "'");
  }
  if (!obj.attr("is_contiguous")().cast<bool>()) {
    value_error(std::string("argument '") + name + "' must be contiguous");
  }
  RawView v;
  py::object dtype = obj.attr("dtype");
  const PyCache& cache = py_cache();
  for (int i = 0; i < 5 && v.dtype_str.empty(); ++i) {
    if (dtype.is(cache.dtypes[i])) v.dtype_str = tag_to_dtype_str(i);
  }
  if (v.dtype_str.empty()) v.dtype_str = py::str(dtype);
  v.ptr = obj.attr("data_ptr")().cast<uintptr_t>();
  v.device_index = device.attr("index").cast<int64_t>();
  py::object shape = obj.attr("shape");
  if (PyTuple_Check(shape.ptr())) {  // torch.Size is a tuple
    const Py_ssize_t n = PyTuple_GET_SIZE(shape.ptr());
    v.shape.reserve((size_t)n);
    for (Py_ssize_t i = 0; i < n; ++i) v.shape.push_back(py::handle(PyTuple_GET_ITEM(shape.ptr(), i)).cast<int64_t>());
  } else {
    for (py::handle d : shape) v.shape.push_back(d.cast<int64_t>());
  }
  return v;
}

View validate_tensor(const char* name, const py::handle& obj) {
  RawView r = validate_and_extract(name, obj);
  if (r.tag >= 0) return View{r.ptr, r.tag, r.device_index, std::move(r.shape)};
  auto tag = tag_from_dtype_str(r.dtype_str);
  if (!tag) unsupported_dtype(r.dtype_str);
  return View{r.ptr, *tag, r.device_index, std::move(r.shape)};
}

View validate_int32_tensor(const char* name, const py::handle& obj) {
  RawView r = validate_and_extract(name, obj);
  if (r.dtype_str != "torch.int32") {
    unsupported_dtype(std::string(name) + " must be int32, got " + r.dtype_str);
  }
  return View{r.ptr, -1, r.device_index, std::move(r.shape)};
}

void check_dtype_matches(const char* name, const View& v, const View& expected, const char* ref) {
  if (v.dtype != expected.dtype) {
    value_error(std::string("dtype mismatch: '") + name + "' is " + tag_debug(v.dtype) +
                " but expected " + tag_debug(expected.dtype) + " (must match '" + ref + "')");
  }
}

// The stream handed to the most recent launcher (test hook: tells a test
// which stream a call launched on, whether or not the runtime let that
// stream overlap others).
std::atomic<uintptr_t> last_launch_stream{0};

// One launch's context: the tensors' device is the current HIP device until
// the launcher returns (as in torch's own ops, so the launchers' per-device
// state, such as the one-pass grid's occupancy and the no-allocation array,
// is that device's; the caller's current device is restored afterwards), and
// st is torch.cuda.current_stream(device_index).cuda_stream, the current HIP
// stream of that device in c10's registry.
struct Launch {
  c10::hip::HIPGuard guard;
  void* st;
  explicit Launch(int64_t device_index)
      : guard(static_cast<c10::DeviceIndex>(device_index)),
        st(c10::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(device_index)).stream()) {
    last_launch_stream.store(reinterpret_cast<uintptr_t>(st), std::memory_order_relaxed);
  }
};

void check_launch(const char* launcher, int32_t err) {
  if (err != 0) {
    throw std::runtime_error(std::string("HIP error: ") + launcher + " failed, hipError_t = " +
                             std::to_string(err));
  }
}

int64_t product(const std::vector<int64_t>& v, size_t begin, size_t end) {
  int64_t p = 1;
  for (size_t i = begin; i < end; ++i) p *= v[i];
  return p;
}

int32_t parse_fp8_format(const std::string& f) {
  if (f == "e4m3") return F8E4M3;
  if (f == "e5m2") return F8E5M2;
  value_error("fp8_format must be 'e4m3' or 'e5m2', got \"" + f + "\"");
}

void require_f32(const char* what, const View& v) {
  if (v.dtype != F32) {
    unsupported_dtype(std::string(what) + " must be float32, got " + tag_debug(v.dtype));
  }
}

void require_fp8_out(const View& v, int32_t fmt, const std::string& fmt_str, const char* name) {
  if (v.dtype != fmt) {
    unsupported_dtype(std::string(name) + " dtype " + tag_debug(v.dtype) +
                      " does not match requested fp8_format \"" + fmt_str + "\"");
  }
}

// ---- reference functions (src/lib.rs:13-15,26-27) -------------------------

// src/kernels/rmsnorm_residual.rs:46-115
void rmsnorm_residual_fwd(py::handle x, py::handle residual, py::handle weight, py::handle y,
                          py::handle residual_out, double eps) {
  View xv = validate_tensor("x", x);
  View rv = validate_tensor("residual", residual);
  View wv = validate_tensor("weight", weight);
  View yv = validate_tensor("y", y);
  View rov = validate_tensor("residual_out", residual_out);
  check_dtype_matches("residual", rv, xv, "x");
  check_dtype_matches("weight", wv, xv, "x");
  check_dtype_matches("y", yv, xv, "x");
  check_dtype_matches("residual_out", rov, xv, "x");
  if (rv.shape != xv.shape || yv.shape != xv.shape || rov.shape != xv.shape) {
    shape_mismatch("x/residual/y/residual_out must share the same shape; got x=" + shape_str(xv.shape) +
                   ", residual=" + shape_str(rv.shape) + ", y=" + shape_str(yv.shape) +
                   ", residual_out=" + shape_str(rov.shape));
  }
  if (xv.shape.empty()) shape_mismatch("x must have at least 1 dimension");
  const int64_t cols = xv.shape.back();
  if (wv.shape != std::vector<int64_t>{cols}) {
    shape_mismatch("weight shape " + shape_str(wv.shape) + " must be [" + std::to_string(cols) +
                   "] (x's last dimension)");
  }
  const int64_t rows = product(xv.shape, 0, xv.shape.size() - 1);
  const Launch launch(xv.device_index);
  void* st = launch.st;
  check_launch("launch_rmsnorm_residual_fwd",
               launch_rmsnorm_residual_fwd((const void*)xv.ptr, (const void*)rv.ptr, (const void*)wv.ptr,
                                           (void*)yv.ptr, (void*)rov.ptr, rows, cols, (float)eps,
                                           xv.dtype, st));
}

// src/kernels/swiglu.rs:31-79
void swiglu_fwd(py::handle gate, py::handle up, py::handle y) {
  View gv = validate_tensor("gate", gate);
  View uv = validate_tensor("up", up);
  View yv = validate_tensor("y", y);
  check_dtype_matches("up", uv, gv, "x");
  check_dtype_matches("y", yv, gv, "x");
  if (uv.shape != gv.shape || yv.shape != gv.shape) {
    shape_mismatch("gate/up/y must share the same shape; got gate=" + shape_str(gv.shape) +
                   ", up=" + shape_str(uv.shape) + ", y=" + shape_str(yv.shape));
  }
  const int64_t n = product(gv.shape, 0, gv.shape.size());
  const Launch launch(gv.device_index);
  void* st = launch.st;
  check_launch("launch_swiglu_fwd", launch_swiglu_fwd((const void*)gv.ptr, (const void*)uv.ptr,
                                                      (void*)yv.ptr, n, gv.dtype, st));
}

// src/kernels/rope.rs:42-153
void rope_fwd(py::handle q, py::handle k, py::handle cos, py::handle sin, py::handle q_out,
              py::handle k_out) {
  View qv = validate_tensor("q", q);
  View kv = validate_tensor("k", k);
  View cv = validate_tensor("cos", cos);
  View sv = validate_tensor("sin", sin);
  View qov = validate_tensor("q_out", q_out);
  View kov = validate_tensor("k_out", k_out);
  check_dtype_matches("k", kv, qv, "x");
  check_dtype_matches("q_out", qov, qv, "x");
  check_dtype_matches("k_out", kov, kv, "x");
  if (cv.dtype != F32) {
    unsupported_dtype(std::string("cos must be float32 (RoPE tables are always fp32), got ") + tag_debug(cv.dtype));
  }
  if (sv.dtype != F32) {
    unsupported_dtype(std::string("sin must be float32 (RoPE tables are always fp32), got ") + tag_debug(sv.dtype));
  }
  if (qv.shape.size() != 4) {
    shape_mismatch("q must be 4-D [batch, seq_len, n_q_heads, head_dim], got " + shape_str(qv.shape));
  }
  if (kv.shape.size() != 4) {
    shape_mismatch("k must be 4-D [batch, seq_len, n_kv_heads, head_dim], got " + shape_str(kv.shape));
  }
  if (qov.shape != qv.shape) shape_mismatch("q_out must match q's shape");
  if (kov.shape != kv.shape) shape_mismatch("k_out must match k's shape");
  const int64_t batch = qv.shape[0], seq_len = qv.shape[1], n_q_heads = qv.shape[2], head_dim = qv.shape[3];
  const int64_t n_kv_heads = kv.shape[2];
  if (kv.shape[0] != batch || kv.shape[1] != seq_len || kv.shape[3] != head_dim) {
    shape_mismatch("q and k must share batch/seq_len/head_dim; got q=" + shape_str(qv.shape) +
                   ", k=" + shape_str(kv.shape));
  }
  if (head_dim % 2 != 0) shape_mismatch("head_dim must be even, got " + std::to_string(head_dim));
  const int64_t half = head_dim / 2;
  const std::vector<int64_t> table{seq_len, half};
  if (cv.shape != table || sv.shape != table) {
    shape_mismatch("cos/sin must have shape [" + std::to_string(seq_len) + ", " + std::to_string(half) +
                   "]; got cos=" + shape_str(cv.shape) + ", sin=" + shape_str(sv.shape));
  }
  const Launch launch(qv.device_index);
  void* st = launch.st;
  check_launch("launch_rope_fwd",
               launch_rope_fwd((const void*)qv.ptr, (const void*)kv.ptr, (const void*)cv.ptr,
                               (const void*)sv.ptr, (void*)qov.ptr, (void*)kov.ptr, batch, seq_len,
                               n_q_heads, n_kv_heads, head_dim, qv.dtype, st));
}

// Shared checks of the FP8 bindings (src/kernels/fp8_quant.rs:71-99).
void check_fp8_common(const View& xv, const View& qv, int32_t fmt, const std::string& fmt_str) {
  require_fp8_out(qv, fmt, fmt_str, "x_fp8");
}

void check_2d_and_codes(const View& xv, const View& qv) {
  if (xv.shape.size() != 2) shape_mismatch("x must be 2-D [M, N]; got " + shape_str(xv.shape));
  const int64_t m = xv.shape[0], n = xv.shape[1];
  if (qv.shape != std::vector<int64_t>{m, n}) {
    shape_mismatch("x_fp8 shape " + shape_str(qv.shape) + " must be [" + std::to_string(m) + ", " +
                   std::to_string(n) + "]");
  }
}

// src/kernels/fp8_quant.rs:61-131
void fp8_quant_block_fwd(py::handle x, py::handle x_fp8, py::handle scale, const std::string& fmt_str) {
  const int32_t fmt = parse_fp8_format(fmt_str);
  View xv = validate_tensor("x", x);
  View qv = validate_tensor("x_fp8", x_fp8);
  View sv = validate_tensor("scale", scale);
  check_fp8_common(xv, qv, fmt, fmt_str);
  require_f32("scale", sv);
  check_2d_and_codes(xv, qv);
  const int64_t m = xv.shape[0], n = xv.shape[1];
  const int64_t nrb = (m + 127) / 128, ncb = (n + 127) / 128;
  if (sv.shape != std::vector<int64_t>{nrb, ncb}) {
    shape_mismatch("scale shape " + shape_str(sv.shape) + " must be [" + std::to_string(nrb) + ", " +
                   std::to_string(ncb) + "] (ceil(M/128), ceil(N/128))");
  }
  const Launch launch(xv.device_index);
  void* st = launch.st;
  check_launch("launch_fp8_quant_block_fwd",
               launch_fp8_quant_block_fwd((const void*)xv.ptr, (uint8_t*)qv.ptr, (float*)sv.ptr, m, n,
                                          xv.dtype, fmt, st));
}

// src/kernels/fp8_quant.rs:138-210
void fp8_quant_tensor_fwd(py::handle x, py::handle x_fp8, py::handle scale, py::handle amax_scratch,
                          const std::string& fmt_str) {
  const int32_t fmt = parse_fp8_format(fmt_str);
  View xv = validate_tensor("x", x);
  View qv = validate_tensor("x_fp8", x_fp8);
  View sv = validate_tensor("scale", scale);
  // None (an addition) skips the caller-visible amax word; the Python API
  // passes it, having no use for that word.
  std::optional<View> av;
  if (!amax_scratch.is_none()) av = validate_int32_tensor("amax_scratch", amax_scratch);
  check_fp8_common(xv, qv, fmt, fmt_str);
  require_f32("scale", sv);
  check_2d_and_codes(xv, qv);
  if (av && product(av->shape, 0, av->shape.size()) != 1) {
    shape_mismatch("amax_scratch must have exactly 1 element; got shape " + shape_str(av->shape));
  }
  const int64_t m = xv.shape[0], n = xv.shape[1];
  const Launch launch(xv.device_index);
  void* st = launch.st;
  check_launch("launch_fp8_quant_tensor_fwd",
               launch_fp8_quant_tensor_fwd((const void*)xv.ptr, (uint8_t*)qv.ptr, (float*)sv.ptr,
                                           av ? (int32_t*)av->ptr : nullptr, m, n, xv.dtype, fmt, st));
}

// ---- additive functions ----------------------------------------------------

void fp8_quant_token_fwd(py::handle x, py::handle x_fp8, py::handle scale, const std::string& fmt_str) {
  const int32_t fmt = parse_fp8_format(fmt_str);
  View xv = validate_tensor("x", x);
  View qv = validate_tensor("x_fp8", x_fp8);
  View sv = validate_tensor("scale", scale);
  check_fp8_common(xv, qv, fmt, fmt_str);
  require_f32("scale", sv);
  check_2d_and_codes(xv, qv);
  const int64_t m = xv.shape[0], n = xv.shape[1];
  if (sv.shape != std::vector<int64_t>{m}) {
    shape_mismatch("scale shape " + shape_str(sv.shape) + " must be [" + std::to_string(m) + "] (one per row)");
  }
  const Launch launch(xv.device_index);
  void* st = launch.st;
  check_launch("launch_fp8_quant_token_fwd",
               launch_fp8_quant_token_fwd((const void*)xv.ptr, (uint8_t*)qv.ptr, (float*)sv.ptr, m, n,
                                          xv.dtype, fmt, st));
}

// The float32 one-element tensor that receives a static scale (the scale
// tensor the Python API returns), or nullptr for None.
float* static_scale_out(py::handle scale_out) {
  if (scale_out.is_none()) return nullptr;
  View sv = validate_tensor("scale", scale_out);
  require_f32("scale", sv);
  if (product(sv.shape, 0, sv.shape.size()) != 1) {
    shape_mismatch("a static scale is returned in a one-element tensor; got shape " + shape_str(sv.shape));
  }
  return (float*)sv.ptr;
}

void fp8_quant_static_fwd(py::handle x, py::handle x_fp8, double scale, const std::string& fmt_str,
                          py::handle scale_out) {
  const int32_t fmt = parse_fp8_format(fmt_str);
  View xv = validate_tensor("x", x);
  View qv = validate_tensor("x_fp8", x_fp8);
  check_fp8_common(xv, qv, fmt, fmt_str);
  check_2d_and_codes(xv, qv);
  float* so = static_scale_out(scale_out);
  const int64_t m = xv.shape[0], n = xv.shape[1];
  const Launch launch(xv.device_index);
  void* st = launch.st;
  check_launch("launch_fp8_quant_static_fwd",
               launch_fp8_quant_static_fwd((const void*)xv.ptr, (uint8_t*)qv.ptr, (float)scale, so, m, n,
                                           xv.dtype, fmt, st));
}

// Scale argument of the fused FP8 bindings: a float32 [rows] tensor for
// dynamic per-token scales, or (static_scale given) None or a one-element
// float32 tensor that receives the static scale.
float* fused_scale_arg(py::handle scale, const std::optional<double>& static_scale, int64_t rows) {
  if (static_scale) return static_scale_out(scale);
  if (scale.is_none()) value_error("scale must be a float32 tensor of shape [rows] when static_scale is None");
  View sv = validate_tensor("scale", scale);
  require_f32("scale", sv);
  if (sv.shape != std::vector<int64_t>{rows}) {
    shape_mismatch("scale shape " + shape_str(sv.shape) + " must be [" + std::to_string(rows) + "] (one per row)");
  }
  return (float*)sv.ptr;
}

void rmsnorm_residual_fp8_fwd(py::handle x, py::handle residual, py::handle weight, py::handle y_fp8,
                              py::handle scale, py::handle residual_out, double eps,
                              const std::string& fmt_str, std::optional<double> static_scale) {
  const int32_t fmt = parse_fp8_format(fmt_str);
  View xv = validate_tensor("x", x);
  View rv = validate_tensor("residual", residual);
  View wv = validate_tensor("weight", weight);
  View qv = validate_tensor("y_fp8", y_fp8);
  View rov = validate_tensor("residual_out", residual_out);
  check_dtype_matches("residual", rv, xv, "x");
  check_dtype_matches("weight", wv, xv, "x");
  check_dtype_matches("residual_out", rov, xv, "x");
  require_fp8_out(qv, fmt, fmt_str, "y_fp8");
  if (rv.shape != xv.shape || qv.shape != xv.shape || rov.shape != xv.shape) {
    shape_mismatch("x/residual/y_fp8/residual_out must share the same shape; got x=" + shape_str(xv.shape) +
                   ", residual=" + shape_str(rv.shape) + ", y_fp8=" + shape_str(qv.shape) +
                   ", residual_out=" + shape_str(rov.shape));
  }
  if (xv.shape.empty()) shape_mismatch("x must have at least 1 dimension");
  const int64_t cols = xv.shape.back();
  if (wv.shape != std::vector<int64_t>{cols}) {
    shape_mismatch("weight shape " + shape_str(wv.shape) + " must be [" + std::to_string(cols) +
                   "] (x's last dimension)");
  }
  const int64_t rows = product(xv.shape, 0, xv.shape.size() - 1);
  float* sp = fused_scale_arg(scale, static_scale, rows);
  const Launch launch(xv.device_index);
  void* st = launch.st;
  check_launch("launch_rmsnorm_residual_fp8_fwd",
               launch_rmsnorm_residual_fp8_fwd(
                   (const void*)xv.ptr, (const void*)rv.ptr, (const void*)wv.ptr, (uint8_t*)qv.ptr, sp,
                   (void*)rov.ptr, rows, cols, (float)eps, static_scale ? (float)*static_scale : 0.0f,
                   static_scale ? CCK_SCALE_STATIC : CCK_SCALE_TOKEN, xv.dtype, fmt, st));
}

void swiglu_fp8_fwd(py::handle gate, py::handle up, py::handle y_fp8, py::handle scale,
                    const std::string& fmt_str, std::optional<double> static_scale) {
  const int32_t fmt = parse_fp8_format(fmt_str);
  View gv = validate_tensor("gate", gate);
  View uv = validate_tensor("up", up);
  View qv = validate_tensor("y_fp8", y_fp8);
  check_dtype_matches("up", uv, gv, "gate");
  require_fp8_out(qv, fmt, fmt_str, "y_fp8");
  if (uv.shape != gv.shape || qv.shape != gv.shape) {
    shape_mismatch("gate/up/y_fp8 must share the same shape; got gate=" + shape_str(gv.shape) +
                   ", up=" + shape_str(uv.shape) + ", y_fp8=" + shape_str(qv.shape));
  }
  if (gv.shape.empty()) shape_mismatch("gate must have at least 1 dimension");
  const int64_t cols = gv.shape.back();
  const int64_t rows = product(gv.shape, 0, gv.shape.size() - 1);
  float* sp = fused_scale_arg(scale, static_scale, rows);
  const Launch launch(gv.device_index);
  void* st = launch.st;
  check_launch("launch_swiglu_fp8_fwd",
               launch_swiglu_fp8_fwd((const void*)gv.ptr, (const void*)uv.ptr, (uint8_t*)qv.ptr, sp, rows,
                                     cols, static_scale ? (float)*static_scale : 0.0f,
                                     static_scale ? CCK_SCALE_STATIC : CCK_SCALE_TOKEN, gv.dtype, fmt,
                                     st));
}

// ---- MoE dispatch (src/kernels/token_permute.rs, src/kernels/moe_router.rs) --

View validate_int64_tensor(const char* name, const py::handle& obj) {
  RawView r = validate_and_extract(name, obj);
  if (r.dtype_str != "torch.int64") {
    unsupported_dtype(std::string(name) + " must be int64, got " + r.dtype_str);
  }
  return View{r.ptr, -1, r.device_index, std::move(r.shape)};
}

// src/kernels/token_permute.rs:45-106. Calls the bounds-checked launcher (the
// binding knows the source row count).
void token_gather_fwd(py::handle src, py::handle indices, py::handle dst) {
  View sv = validate_tensor("src", src);
  View iv = validate_int64_tensor("indices", indices);
  View dv = validate_tensor("dst", dst);
  check_dtype_matches("dst", dv, sv, "x");
  if (sv.shape.size() != 2 || dv.shape.size() != 2) {
    shape_mismatch("src and dst must be 2-D; got src=" + shape_str(sv.shape) + ", dst=" + shape_str(dv.shape));
  }
  const int64_t hidden = sv.shape[1];
  if (dv.shape[1] != hidden) {
    shape_mismatch("dst's hidden dim (" + std::to_string(dv.shape[1]) + ") must match src's (" +
                   std::to_string(hidden) + ")");
  }
  if (iv.shape.size() != 1 || iv.shape[0] != dv.shape[0]) {
    shape_mismatch("indices shape " + shape_str(iv.shape) + " must be [" + std::to_string(dv.shape[0]) +
                   "] (dst's row count)");
  }
  const Launch launch(sv.device_index);
  void* st = launch.st;
  check_launch("launch_token_gather_fwd",
               launch_token_gather_checked_fwd((const void*)sv.ptr, (const int64_t*)iv.ptr, (void*)dv.ptr,
                                               sv.shape[0], dv.shape[0], hidden, sv.dtype, st));
}

// src/kernels/token_permute.rs:115-201.
void token_combine_fwd(py::handle expert_output, py::handle unpermute_index, py::handle weights,
                       py::handle combined) {
  View ev = validate_tensor("expert_output", expert_output);
  View iv = validate_int64_tensor("unpermute_index", unpermute_index);
  View wv = validate_tensor("weights", weights);
  View cv = validate_tensor("combined", combined);
  check_dtype_matches("combined", cv, ev, "x");
  require_f32("weights", wv);
  if (ev.shape.size() != 2 || cv.shape.size() != 2) {
    shape_mismatch("expert_output and combined must be 2-D; got expert_output=" + shape_str(ev.shape) +
                   ", combined=" + shape_str(cv.shape));
  }
  const int64_t hidden = ev.shape[1];
  if (cv.shape[1] != hidden) {
    shape_mismatch("combined's hidden dim (" + std::to_string(cv.shape[1]) + ") must match expert_output's (" +
                   std::to_string(hidden) + ")");
  }
  if (iv.shape.size() != 2 || wv.shape.size() != 2) {
    shape_mismatch("unpermute_index and weights must be 2-D [T, k]; got unpermute_index=" + shape_str(iv.shape) +
                   ", weights=" + shape_str(wv.shape));
  }
  const int64_t n_tokens = iv.shape[0], k = iv.shape[1];
  if (wv.shape != std::vector<int64_t>{n_tokens, k}) {
    shape_mismatch("weights shape " + shape_str(wv.shape) + " must match unpermute_index's [" +
                   std::to_string(n_tokens) + ", " + std::to_string(k) + "]");
  }
  if (cv.shape[0] != n_tokens) {
    shape_mismatch("combined's row count (" + std::to_string(cv.shape[0]) + ") must match unpermute_index's [" +
                   std::to_string(n_tokens) + ", ...]");
  }
  const Launch launch(ev.device_index);
  void* st = launch.st;
  check_launch("launch_token_combine_fwd",
               launch_token_combine_checked_fwd((const void*)ev.ptr, (const int64_t*)iv.ptr, (const float*)wv.ptr,
                                                (void*)cv.ptr, ev.shape[0], n_tokens, k, hidden, ev.dtype, st));
}

// src/kernels/moe_router.rs:36-116.
// Additive (baselines/token_permute.py:55-70 as one kernel).
void moe_permutation_fwd(py::handle topk_indices, py::handle permute_index, py::handle unpermute_index,
                         int64_t num_experts) {
  View tv = validate_int64_tensor("topk_indices", topk_indices);
  View pv = validate_int64_tensor("permute_index", permute_index);
  View uv = validate_int64_tensor("unpermute_index", unpermute_index);
  if (tv.shape.size() != 2) {
    shape_mismatch("topk_indices must be 2-D [num_tokens, k], got " + shape_str(tv.shape));
  }
  const int64_t n_tokens = tv.shape[0], k = tv.shape[1];
  if (pv.shape != std::vector<int64_t>{n_tokens * k}) {
    shape_mismatch("permute_index shape " + shape_str(pv.shape) + " must be [" + std::to_string(n_tokens * k) + "]");
  }
  if (uv.shape != tv.shape) {
    shape_mismatch("unpermute_index shape " + shape_str(uv.shape) + " must match topk_indices' " +
                   shape_str(tv.shape));
  }
  if (num_experts < 1 || num_experts > 256) {
    shape_mismatch("num_experts (" + std::to_string(num_experts) + ") must be in [1, 256]");
  }
  const Launch launch(tv.device_index);
  void* st = launch.st;
  check_launch("launch_moe_permutation_fwd",
               launch_moe_permutation_fwd((const int64_t*)tv.ptr, (int64_t*)pv.ptr, (int64_t*)uv.ptr, n_tokens, k,
                                          num_experts, st));
}

void moe_router_fwd(py::handle logits, py::handle topk_weights, py::handle topk_indices, bool renormalize) {
  View lv = validate_tensor("logits", logits);
  View wv = validate_tensor("topk_weights", topk_weights);
  View iv = validate_int64_tensor("topk_indices", topk_indices);
  require_f32("topk_weights", wv);
  if (lv.shape.size() != 2) {
    shape_mismatch("logits must be 2-D [num_tokens, num_experts], got " + shape_str(lv.shape));
  }
  const int64_t n_tokens = lv.shape[0], n_experts = lv.shape[1];
  if (wv.shape.size() != 2 || wv.shape[0] != n_tokens) {
    shape_mismatch("topk_weights shape " + shape_str(wv.shape) + " must be [" + std::to_string(n_tokens) + ", k]");
  }
  const int64_t k = wv.shape[1];
  if (iv.shape != std::vector<int64_t>{n_tokens, k}) {
    shape_mismatch("topk_indices shape " + shape_str(iv.shape) + " must match topk_weights' [" +
                   std::to_string(n_tokens) + ", " + std::to_string(k) + "]");
  }
  if (k > n_experts) {
    throw std::runtime_error("k (" + std::to_string(k) + ") must be <= num_experts (" + std::to_string(n_experts) +
                             ")");
  }
  if (n_experts > 256) {
    shape_mismatch("num_experts (" + std::to_string(n_experts) +
                   ") exceeds this kernel's supported maximum of 256");
  }
  const Launch launch(lv.device_index);
  void* st = launch.st;
  check_launch("launch_moe_router_fwd",
               launch_moe_router_fwd((const void*)lv.ptr, (float*)wv.ptr, (int64_t*)iv.ptr, n_tokens, n_experts, k,
                                     lv.dtype, renormalize ? 1 : 0, st));
}

}  // namespace

PYBIND11_MODULE(_native, m) {
  m.doc() = "Validating binding over the libcustom_kernels_amd C ABI (gfx950).";
  m.def("rmsnorm_residual_fwd", &rmsnorm_residual_fwd, py::arg("x"), py::arg("residual"), py::arg("weight"),
        py::arg("y"), py::arg("residual_out"), py::arg("eps"));
  m.def("swiglu_fwd", &swiglu_fwd, py::arg("gate"), py::arg("up"), py::arg("y"));
  m.def("rope_fwd", &rope_fwd, py::arg("q"), py::arg("k"), py::arg("cos"), py::arg("sin"), py::arg("q_out"),
        py::arg("k_out"));
  m.def("fp8_quant_block_fwd", &fp8_quant_block_fwd, py::arg("x"), py::arg("x_fp8"), py::arg("scale"),
        py::arg("fp8_format"));
  m.def("fp8_quant_tensor_fwd", &fp8_quant_tensor_fwd, py::arg("x"), py::arg("x_fp8"), py::arg("scale"),
        py::arg("amax_scratch"), py::arg("fp8_format"));
  m.def("fp8_quant_token_fwd", &fp8_quant_token_fwd, py::arg("x"), py::arg("x_fp8"), py::arg("scale"),
        py::arg("fp8_format"));
  m.def("fp8_quant_static_fwd", &fp8_quant_static_fwd, py::arg("x"), py::arg("x_fp8"), py::arg("scale"),
        py::arg("fp8_format"), py::arg("scale_out") = py::none());
  m.def("rmsnorm_residual_fp8_fwd", &rmsnorm_residual_fp8_fwd, py::arg("x"), py::arg("residual"),
        py::arg("weight"), py::arg("y_fp8"), py::arg("scale"), py::arg("residual_out"), py::arg("eps"),
        py::arg("fp8_format"), py::arg("static_scale") = py::none());
  m.def("token_gather_fwd", &token_gather_fwd, py::arg("src"), py::arg("indices"), py::arg("dst"));
  m.def("token_combine_fwd", &token_combine_fwd, py::arg("expert_output"), py::arg("unpermute_index"),
        py::arg("weights"), py::arg("combined"));
  m.def("moe_permutation_fwd", &moe_permutation_fwd, py::arg("topk_indices"), py::arg("permute_index"),
        py::arg("unpermute_index"), py::arg("num_experts"));
  m.def("moe_router_fwd", &moe_router_fwd, py::arg("logits"), py::arg("topk_weights"), py::arg("topk_indices"),
        py::arg("renormalize"));
  m.def("_last_launch_stream", [] { return last_launch_stream.load(std::memory_order_relaxed); },
        "Test hook: the hipStream_t (as an int) the most recent call launched on.");
  m.def("swiglu_fp8_fwd", &swiglu_fp8_fwd, py::arg("gate"), py::arg("up"), py::arg("y_fp8"), py::arg("scale"),
        py::arg("fp8_format"), py::arg("static_scale") = py::none());
}
