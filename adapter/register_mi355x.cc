// onnx-light kernels backed by the MI355X library (include/onnxl_amd.h).
//
// This translation unit is compiled inside the onnx-light tree (it includes
// the runtime's headers) and linked with onnx-light-amd/libonnxl_amd.so and
// the HIP runtime (amdhip64).  Call RegisterMi355xKernelFunctions() once,
// after the built-in kernels are registered (onnx_kernels::
// RegisterKernelFunctions) and before any session resolves its kernels: the
// registries are not synchronised (core/runtime/kernels/
// kernel_dispatch_table.h:134-137).  Unchanged models and RuntimeSessions then
// run the operators below on the GPU.
//
// What it does:
//  - one KernelBase subclass per operator of the quantized-matmul path
//    (MatMulInteger, QLinearMatMul, DequantizeLinear, MatMul, QuantizeLinear,
//    DynamicQuantizeLinear, ConvInteger, QLinearConv, Cast, DequantizePacked,
//    GroupedMatMul, com.microsoft:MatMulNBits on ORT-packed weights, and
//    ai.rt:Dequantize on AWQ / GPTQ / BitBLAS / bitsandbytes / QQQ /
//    GPTQModel FP8 / VPTQ encoded weights), and for the fused nodes the GPU
//    patterns produce
//    (ai.rt.amd:DequantizeLinearMatMul,
//    ai.rt.amd:DequantizePackedMatMul, ai.rt.amd:DequantizeEncodedMatMul on
//    an encoded weight, ai.rt.amd:DequantizeLinearGroupedMatMul on quantized
//    MoE experts),
//    registered with RegisterKernelFn(..., Device::kCPU, overwrite = true),
//    the plain key the built-ins use (examples/register_custom_kernel/
//    main.cc:105-114): a kGPU key would need RuntimeContextOptions.device =
//    kGPU0, and then every other operator of the graph would fail to resolve;
//  - the reference's contract for outputs: host tensors, complete when Run
//    returns.  Host-descriptor calls stage their inputs to HBM, compute and
//    copy the output back before returning;
//  - constant inputs (weights, scales, zero points) are moved to HBM once per
//    session through the kernel-preparation hooks (HasPreparations /
//    DeclarePreparations, core/runtime/kernels/kernel_context.h:238-249), the
//    way the built-in Gemm packs its constant B (km/kernel_gemm.cc:378-405).
//    A constant INT4 / UINT4 weight of the fused node is also tiled there by
//    onnxl_amd_prepare_weight;
//  - inputs the library does not take (dtypes, ranks, formats it reports as
//    ONNXL_AMD_UNSUPPORTED) run on the built-in kernel that was registered
//    for the operator before this one; library errors become the reference's
//    exception types (std::invalid_argument / std::runtime_error).
#include "onnx_core/runtime/kernels/cast_helper.h"
#include "onnx_core/runtime/kernels/kernel_context.h"
#include "onnx_core/runtime/kernels/kernel_dispatch_table.h"
#include "onnx_core/runtime/kernels/node_helpers.h"
#include "onnx_core/runtime/memory/simple_tensor.h"
#include "onnx_core/runtime/quantization.h"
#include "onnx_core/runtime/runtime_context.h"
#include "onnx_core/symbolic/sym_tensor.h"
#include "onnx_proto/onnx.h"

#include <hip/hip_runtime.h>

#include "onnxl_amd.h"

#include <cctype>
#include <charconv>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <system_error>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

namespace rt = ONNX_LIGHT_NAMESPACE::core::runtime;
namespace sym = ONNX_LIGHT_NAMESPACE::core::symbolic;
using ONNX_LIGHT_NAMESPACE::NodeProto;

namespace mi355x {

// ONNX TensorProto data types used below.
constexpr int32_t kFloat = 1, kUint8 = 2, kInt8 = 3, kInt32 = 6, kFloat16 = 10, kDouble = 11, kBfloat16 = 16,
                  kUint4 = 21, kInt4 = 22;
constexpr const char *kFusedDomain = "ai.rt.amd";

// Library status -> the reference's exception types.
void Check(int rc) {
  if (rc == ONNXL_AMD_OK) return;
  if (rc == ONNXL_AMD_INVALID_ARGUMENT) throw std::invalid_argument(onnxl_amd_last_error());
  throw std::runtime_error(onnxl_amd_last_error());
}

void CheckHip(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string("mi355x: ") + what + ": " + hipGetErrorString(e));
}

onnxl_amd_tensor Absent() {
  onnxl_amd_tensor d{};
  d.rank = -1;
  return d;
}

// Host tensor -> C-ABI descriptor.  The library never writes an input.
onnxl_amd_tensor Describe(const rt::Tensor *t) {
  if (t == nullptr || t->data_type == 0) return Absent();  // absent optional input
  if (t->shape.size() > ONNXL_AMD_MAX_RANK)
    throw std::invalid_argument("mi355x: tensor rank above " + std::to_string(ONNXL_AMD_MAX_RANK));
  onnxl_amd_tensor d{};
  d.data_type = t->data_type;
  d.rank = static_cast<int32_t>(t->shape.size());
  for (int i = 0; i < d.rank; ++i) d.dims[i] = t->shape[i];
  d.data = const_cast<uint8_t *>(t->bytes());
  d.size_bytes = static_cast<int64_t>(t->size_bytes());
  d.location = ONNXL_AMD_HOST;
  d.layout = ONNXL_AMD_LAYOUT_ONNX;
  return d;
}

onnxl_amd_tensor DescribeOutput(rt::Tensor &t) {
  onnxl_amd_tensor d = Describe(&t);
  d.data = t.mutable_bytes();
  return d;
}

rt::Shape ShapeOf(const int64_t *dims, int32_t rank) {
  return rt::Shape(std::vector<int64_t>(dims, dims + rank));
}

int64_t Count(const rt::Shape &s) {
  int64_t n = 1;
  for (size_t i = 0; i < s.size(); ++i) n *= s[i];
  return n;
}

// HBM copy of a session constant, owned by the kernel that prepared it.
struct DeviceTensor {
  onnxl_amd_tensor desc{};
  void *ptr = nullptr;
  DeviceTensor() = default;
  DeviceTensor(const DeviceTensor &) = delete;
  DeviceTensor &operator=(const DeviceTensor &) = delete;
  ~DeviceTensor() {
    if (ptr != nullptr) (void)hipFree(ptr);
  }
  void Allocate(int64_t bytes) {
    CheckHip(hipMalloc(&ptr, static_cast<size_t>(bytes > 0 ? bytes : 16)), "hipMalloc");
  }
};

std::shared_ptr<DeviceTensor> UploadToHbm(const rt::Tensor &t) {
  auto d = std::make_shared<DeviceTensor>();
  d->desc = Describe(&t);
  d->Allocate(d->desc.size_bytes);
  if (d->desc.size_bytes > 0)
    CheckHip(hipMemcpy(d->ptr, t.bytes(), t.size_bytes(), hipMemcpyHostToDevice), "hipMemcpy");
  d->desc.data = d->ptr;
  d->desc.location = ONNXL_AMD_DEVICE;
  return d;
}

// A device buffer reused across runs (the fused node's activations and
// output); grows only when a larger shape arrives.
struct Staging {
  void *ptr = nullptr;
  size_t bytes = 0;
  ~Staging() {
    if (ptr != nullptr) (void)hipFree(ptr);
  }
  void *Reserve(size_t n) {
    if (n > bytes) {
      if (ptr != nullptr) CheckHip(hipFree(ptr), "hipFree");
      ptr = nullptr;
      CheckHip(hipMalloc(&ptr, n > 0 ? n : 16), "hipMalloc");
      bytes = n;
    }
    return ptr;
  }
};

// ---------------------------------------------------------------------------
// Common base: constant inputs moved to HBM at preparation time, and the
// built-in kernel of the same operator for the inputs the library does not
// take.
class Mi355xKernel : public rt::KernelBase {
public:
  Mi355xKernel(const rt::KernelContext &kc, std::unique_ptr<rt::KernelBase> builtin)
      : rt::KernelBase(kc), builtin_(std::move(builtin)) {}

  bool HasPreparations(const std::unordered_set<std::string> &immutable_inputs) const override {
    for (int i : ConstantInputs())
      if (i < node_->input_size() && !node_->input(i).empty() &&
          immutable_inputs.count(node_->input(i)) != 0)
        return true;
    return builtin_ != nullptr && builtin_->HasPreparations(immutable_inputs);
  }

  void DeclarePreparations(const std::unordered_set<std::string> &immutable_inputs,
                           std::vector<rt::KernelPreparation> &preparations) override {
    for (int i : ConstantInputs()) {
      if (i >= node_->input_size() || node_->input(i).empty() || immutable_inputs.count(node_->input(i)) == 0)
        continue;
      const std::string source = node_->input(i);
      rt::KernelPreparation p;
      p.info.source_inputs = {source};
      p.info.representation = Representation(i);
      p.info.output_slots = {source + ":" + p.info.representation};
      // The prepared copy lives in HBM: no host memory beyond the source.
      p.estimate_memory = [source](const rt::RuntimeContext &ctx) {
        return rt::KernelPreparationMemory{ctx.Get(source).size_bytes(), 0, 0};
      };
      p.execute = [this, i, source](rt::RuntimeContext &ctx) {
        auto d = Prepare(i, ctx.Get(source));
        std::lock_guard<std::mutex> lock(mu_);
        prepared_[i] = std::move(d);  // published only once complete
      };
      preparations.push_back(std::move(p));
    }
    // The built-in kernel keeps its own preparations for the inputs it runs.
    if (builtin_ != nullptr) builtin_->DeclarePreparations(immutable_inputs, preparations);
  }

protected:
  // Node inputs that are worth keeping in HBM when they are constants.
  virtual std::vector<int> ConstantInputs() const { return {}; }
  virtual std::string Representation(int /*index*/) const { return "mi355x:hbm-copy-v1"; }
  virtual std::shared_ptr<DeviceTensor> Prepare(int /*index*/, const rt::Tensor &t) { return UploadToHbm(t); }

  // Descriptor of input `i` for this run: its HBM copy when prepared, else the
  // host tensor, else absent.
  onnxl_amd_tensor In(int i, rt::RuntimeContext &ctx) const {
    auto it = prepared_.find(i);
    if (it != prepared_.end()) return it->second->desc;
    if (i >= node_->input_size() || node_->input(i).empty()) return Absent();
    return Describe(rt::GetOptionalInput(*node_, i, ctx));
  }
  bool Prepared(int i) const { return prepared_.count(i) != 0; }

  // Runs the built-in kernel (after the library reported UNSUPPORTED).
  void RunBuiltin(rt::RuntimeContext &ctx, const char *why) {
    if (builtin_ == nullptr)
      throw std::runtime_error(std::string("mi355x: ") + node_->op_type() + ": " + why +
                               " and no built-in kernel is registered");
    builtin_->Run(ctx);
  }

  // Library call with the built-in kernel as the fallback for UNSUPPORTED.
  // Returns true when the library computed the output.
  bool Call(int rc, rt::RuntimeContext &ctx) {
    if (rc == ONNXL_AMD_UNSUPPORTED) {
      RunBuiltin(ctx, onnxl_amd_last_error());
      return false;
    }
    Check(rc);
    return true;
  }

  std::unique_ptr<rt::KernelBase> builtin_;
  std::map<int, std::shared_ptr<DeviceTensor>> prepared_;
  std::mutex mu_;
};

// MatMul output shape as the reference computes it (km/matmul_shape_utils.h).
rt::Shape MatMulShape(const onnxl_amd_tensor &a, const onnxl_amd_tensor &b) {
  int64_t dims[ONNXL_AMD_MAX_RANK];
  int32_t rank = 0;
  Check(onnxl_amd_matmul_shape(a.dims, a.rank, b.dims, b.rank, dims, &rank));
  return ShapeOf(dims, rank);
}

// ---------------------------------------------------------------------------
// MatMulInteger (km/kernel_matmul_integer.cc): A, B, optional zero points.
class Mi355xMatMulInteger : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:MatMulInteger";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 2);
    rt::RequireOutputCount(node, 1);
    const onnxl_amd_tensor a = In(0, ctx), b = In(1, ctx), za = In(2, ctx), zb = In(3, ctx);
    const rt::Shape shape = MatMulShape(a, b);
    rt::Tensor y = ctx.MakeOutputTensor(0, kInt32, shape, static_cast<size_t>(Count(shape)) * 4);
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_matmul_integer(&a, &b, &za, &zb, &dy, nullptr), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1, 2, 3}; }
};

// QLinearMatMul (kq/kernel_qlinearmatmul.cc:269-296): 8 inputs.
class Mi355xQLinearMatMul : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:QLinearMatMul";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireInputCount(node, 8);
    rt::RequireOutputCount(node, 1);
    onnxl_amd_tensor in[8];
    for (int i = 0; i < 8; ++i) in[i] = In(i, ctx);
    const rt::Shape shape = MatMulShape(in[0], in[3]);
    rt::Tensor y = ctx.MakeOutputTensor(0, in[7].data_type, shape, static_cast<size_t>(Count(shape)));
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_qlinear_matmul(&in[0], &in[1], &in[2], &in[3], &in[4], &in[5], &in[6], &in[7], &dy, nullptr),
             ctx))
      rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1, 2, 3, 4, 5, 6, 7}; }
};

// Bytes of `count` elements of `dtype`, 4-bit types packed two per byte.
size_t ByteSize(int32_t dtype, int64_t count) { return rt::PackedByteSize(dtype, count); }

// DequantizeLinear (kq/kernel_dequantizelinear.cc:695-712): axis defaults to
// 1; y takes x_scale's dtype.
class Mi355xDequantizeLinear : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:DequantizeLinear";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 2);
    rt::RequireOutputCount(node, 1);
    const onnxl_amd_tensor x = In(0, ctx), s = In(1, ctx), z = In(2, ctx);
    const int64_t axis = rt::GetAttributeIntOrDefault(node, "axis", 1);
    const rt::Shape shape = ShapeOf(x.dims, x.rank);
    rt::Tensor y = ctx.MakeOutputTensor(0, s.data_type, shape, ByteSize(s.data_type, Count(shape)));
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_dequantize_linear(&x, &s, &z, axis, &dy, nullptr), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {0, 1, 2}; }
};

// QuantizeLinear (kq/kernel_quantizelinear.cc:917-941): y's dtype is the zero
// point's, else output_dtype, else UINT8.
class Mi355xQuantizeLinear : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:QuantizeLinear";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 2);
    rt::RequireOutputCount(node, 1);
    const onnxl_amd_tensor x = In(0, ctx), s = In(1, ctx), z = In(2, ctx);
    const int64_t axis = rt::GetAttributeIntOrDefault(node, "axis", 1);  // may be negative
    const int64_t odt = rt::GetAttributeIntOrDefault(node, "output_dtype", 0);
    const int32_t yt = z.rank >= 0 ? z.data_type : (odt != 0 ? static_cast<int32_t>(odt) : kUint8);
    const rt::Shape shape = ShapeOf(x.dims, x.rank);
    rt::Tensor y = ctx.MakeOutputTensor(0, yt, shape, ByteSize(yt, Count(shape)));
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_quantize_linear(&x, &s, &z, axis, static_cast<int32_t>(odt), &dy, nullptr), ctx))
      rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1, 2}; }
};

// DynamicQuantizeLinear (kq/kernel_dynamicquantizelinear.cc): three outputs.
// The library reports non-finite x as y_scale = NaN; the outputs are host
// tensors, complete on return, so the adapter raises the reference's error.
class Mi355xDynamicQuantizeLinear : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:DynamicQuantizeLinear";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireInputCount(node, 1);
    rt::RequireOutputCount(node, 3);
    const onnxl_amd_tensor x = In(0, ctx);
    const rt::Shape shape = ShapeOf(x.dims, x.rank);
    rt::Tensor y = ctx.MakeOutputTensor(0, kUint8, shape, static_cast<size_t>(Count(shape)));
    rt::Tensor s = ctx.MakeOutputTensor(1, kFloat, rt::Shape{}, sizeof(float));
    rt::Tensor z = ctx.MakeOutputTensor(2, kUint8, rt::Shape{}, 1);
    onnxl_amd_tensor dy = DescribeOutput(y), ds = DescribeOutput(s), dz = DescribeOutput(z);
    if (!Call(onnxl_amd_dynamic_quantize_linear(&x, &dy, &ds, &dz, nullptr), ctx)) return;
    float scale;
    std::memcpy(&scale, s.bytes(), sizeof(float));
    if (std::isnan(scale)) throw std::invalid_argument("kernel::DynamicQuantizeLinear: x elements must be finite.");
    rt::SetOutput(node, 0, std::move(y), ctx);
    rt::SetOutput(node, 1, std::move(s), ctx);
    rt::SetOutput(node, 2, std::move(z), ctx);
  }
};

// MatMul (km/kernel_matmul.cc): FLOAT16 / BFLOAT16 on the GPU, every other
// dtype on the built-in kernel.
class Mi355xMatMul : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:MatMul";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireInputCount(node, 2);
    rt::RequireOutputCount(node, 1);
    const onnxl_amd_tensor a = In(0, ctx), b = In(1, ctx);
    if ((a.data_type != kFloat16 && a.data_type != kBfloat16) || b.data_type != a.data_type) {
      RunBuiltin(ctx, "dtype other than FLOAT16 / BFLOAT16");
      return;
    }
    const rt::Shape shape = MatMulShape(a, b);
    rt::Tensor y = ctx.MakeOutputTensor(0, a.data_type, shape, static_cast<size_t>(Count(shape)) * 2);
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_matmul(&a, &b, &dy, nullptr), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1}; }
};

// Cast (ext/kernels/kernels/tensor/kernel_cast.cc:360-370): FLOAT ->
// FLOAT16 / BFLOAT16 on the GPU (the Cast between DequantizeLinear and a
// 16-bit MatMul), every other pair on the built-in kernel.
class Mi355xCast : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:Cast";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireInputCount(node, 1);
    rt::RequireOutputCount(node, 1);
    const onnxl_amd_tensor x = In(0, ctx);
    const int32_t to = static_cast<int32_t>(rt::GetAttributeIntOrDefault(node, "to", 0));
    if (x.data_type != kFloat || (to != kFloat16 && to != kBfloat16) ||
        rt::GetAttributeIntOrDefault(node, "saturate", 1) != 1) {
      RunBuiltin(ctx, "cast other than FLOAT -> FLOAT16 / BFLOAT16");
      return;
    }
    const rt::Shape shape = ShapeOf(x.dims, x.rank);
    rt::Tensor y = ctx.MakeOutputTensor(0, to, shape, static_cast<size_t>(Count(shape)) * 2);
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_cast(&x, to, &dy, nullptr), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
  }
};

// Convolution attributes as ConvInteger::Run / QLinearConv::Run read them
// (nn/kernel_conv_integer.cc:306-330, kq/kernel_qlinearconv.cc:352-375).
// Returns false when the node has more spatial dims than the library takes.
bool ConvAttrs(const NodeProto &node, onnxl_amd_conv_attrs &a) {
  a = onnxl_amd_conv_attrs{};
  const std::vector<int64_t> ks = rt::GetAttributeIntsOrDefault(node, "kernel_shape", {});
  const std::vector<int64_t> st = rt::GetAttributeIntsOrDefault(node, "strides", {});
  const std::vector<int64_t> pd = rt::GetAttributeIntsOrDefault(node, "pads", {});
  const std::vector<int64_t> dl = rt::GetAttributeIntsOrDefault(node, "dilations", {});
  if (ks.size() > ONNXL_AMD_MAX_CONV_SPATIAL || st.size() > ONNXL_AMD_MAX_CONV_SPATIAL ||
      pd.size() > 2 * ONNXL_AMD_MAX_CONV_SPATIAL || dl.size() > ONNXL_AMD_MAX_CONV_SPATIAL)
    return false;
  a.n_kernel_shape = static_cast<int32_t>(ks.size());
  a.n_strides = static_cast<int32_t>(st.size());
  a.n_pads = static_cast<int32_t>(pd.size());
  a.n_dilations = static_cast<int32_t>(dl.size());
  for (size_t i = 0; i < ks.size(); ++i) a.kernel_shape[i] = ks[i];
  for (size_t i = 0; i < st.size(); ++i) a.strides[i] = st[i];
  for (size_t i = 0; i < pd.size(); ++i) a.pads[i] = pd[i];
  for (size_t i = 0; i < dl.size(); ++i) a.dilations[i] = dl[i];
  a.group = rt::GetAttributeIntOrDefault(node, "group", 1);
  const std::string ap = rt::GetAttributeStringOrDefault(node, "auto_pad", "NOTSET");
  a.auto_pad = ap == "SAME_UPPER"   ? ONNXL_AMD_AUTO_PAD_SAME_UPPER
               : ap == "SAME_LOWER" ? ONNXL_AMD_AUTO_PAD_SAME_LOWER
               : ap == "VALID"      ? ONNXL_AMD_AUTO_PAD_VALID
                                    : ONNXL_AMD_AUTO_PAD_NOTSET;  // as AutoPadFromString
  return true;
}

rt::Shape ConvShape(const onnxl_amd_tensor &x, const onnxl_amd_tensor &w, const onnxl_amd_conv_attrs &a) {
  int64_t dims[ONNXL_AMD_MAX_RANK];
  int32_t rank = 0;
  Check(onnxl_amd_conv_shape(x.dims, x.rank, w.dims, w.rank, &a, dims, &rank));
  return ShapeOf(dims, rank);
}

// ConvInteger (nn/kernel_conv_integer.cc:306-330).
class Mi355xConvInteger : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:ConvInteger";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 2);
    rt::RequireOutputCount(node, 1);
    onnxl_amd_conv_attrs attrs;
    if (!ConvAttrs(node, attrs)) {
      RunBuiltin(ctx, "more than 3 spatial dims");
      return;
    }
    const onnxl_amd_tensor x = In(0, ctx), w = In(1, ctx), zx = In(2, ctx), zw = In(3, ctx);
    if (x.rank < 3 || x.rank > 2 + ONNXL_AMD_MAX_CONV_SPATIAL) {
      RunBuiltin(ctx, "input rank outside 3..5");
      return;
    }
    const rt::Shape shape = ConvShape(x, w, attrs);
    rt::Tensor y = ctx.MakeOutputTensor(0, kInt32, shape, static_cast<size_t>(Count(shape)) * 4);
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_conv_integer(&x, &w, &zx, &zw, &attrs, &dy, nullptr), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1, 3}; }
};

// QLinearConv (kq/kernel_qlinearconv.cc:352-375): 8 inputs and an optional
// INT32 bias; y takes y_zero_point's dtype.
class Mi355xQLinearConv : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:QLinearConv";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 8);
    rt::RequireOutputCount(node, 1);
    onnxl_amd_conv_attrs attrs;
    if (!ConvAttrs(node, attrs)) {
      RunBuiltin(ctx, "more than 3 spatial dims");
      return;
    }
    onnxl_amd_tensor in[9];
    for (int i = 0; i < 9; ++i) in[i] = In(i, ctx);
    if (in[0].rank < 3 || in[0].rank > 2 + ONNXL_AMD_MAX_CONV_SPATIAL) {
      RunBuiltin(ctx, "input rank outside 3..5");
      return;
    }
    const rt::Shape shape = ConvShape(in[0], in[3], attrs);
    rt::Tensor y = ctx.MakeOutputTensor(0, in[7].data_type, shape, static_cast<size_t>(Count(shape)));
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_qlinear_conv(&in[0], &in[1], &in[2], &in[3], &in[4], &in[5], &in[6], &in[7], &in[8], &attrs,
                                    &dy, nullptr),
             ctx))
      rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1, 2, 3, 4, 5, 6, 7, 8}; }
};

// DequantizePacked (kq/kernel_dequantize_packed.cc:13-26): format, shape and
// output_dtype attributes; the GGUF formats the GPU decodes, the others on
// the built-in kernel.
class Mi355xDequantizePacked : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:DequantizePacked";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireInputCount(node, 1);
    rt::RequireOutputCount(node, 1);
    const std::string format = rt::GetRequiredAttributeString(node, "format");
    const std::vector<int64_t> dims = rt::GetAttributeIntsOrDefault(node, "shape", {});
    const int64_t odt = rt::GetAttributeIntOrDefault(node, "output_dtype", kFloat);
    const onnxl_amd_tensor x = In(0, ctx);
    if (dims.empty() || dims.size() > ONNXL_AMD_MAX_RANK) {
      RunBuiltin(ctx, "shape attribute the library does not take");
      return;
    }
    const rt::Shape shape(dims);
    rt::Tensor y = ctx.MakeOutputTensor(0, static_cast<int32_t>(odt), shape,
                                        ByteSize(static_cast<int32_t>(odt), Count(shape)));
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_dequantize_packed(&x, format.c_str(), dims.data(), static_cast<int32_t>(dims.size()), odt, &dy,
                                         nullptr),
             ctx))
      rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {0}; }
};

// GroupedMatMul (math/kernel_grouped_matmul.cc:105-114): input [M, K],
// weights [G, K, N] (or [G, N, K] with transB), group_indices [M, S],
// optional bias [G, N] -> [M, S, N].  FLOAT16 / BFLOAT16 on the GPU, FLOAT and
// DOUBLE on the built-in kernel.  Host indices are range-checked by the
// library before any work, with the reference's message.
class Mi355xGroupedMatMul : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.onnx:GroupedMatMul";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 3);
    rt::RequireOutputCount(node, 1);
    const onnxl_amd_tensor x = In(0, ctx), w = In(1, ctx), idx = In(2, ctx), b = In(3, ctx);
    const int64_t transB = rt::GetAttributeIntOrDefault(node, "transB", 0);
    if (x.data_type != kFloat16 && x.data_type != kBfloat16) {
      RunBuiltin(ctx, "dtype other than FLOAT16 / BFLOAT16");
      return;
    }
    if (x.rank != 2 || w.rank != 3 || idx.rank != 2) {  // the library raises the reference's error
      onnxl_amd_tensor none{};
      Check(onnxl_amd_grouped_matmul(&x, &w, &idx, &b, transB, &none, nullptr));
    }
    const rt::Shape shape{x.dims[0], idx.dims[1], w.dims[transB != 0 ? 1 : 2]};
    rt::Tensor y = ctx.MakeOutputTensor(0, x.data_type, shape, static_cast<size_t>(Count(shape)) * 2);
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(onnxl_amd_grouped_matmul(&x, &w, &idx, &b, transB, &dy, nullptr), ctx))
      rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1, 3}; }
};

// com.microsoft:MatMulNBits (the ORT operator whose inputs
// ExportMatMulNBitsInputs writes, onnx_core/runtime/quantization.h:492-532):
// A [..., K] FLOAT16, B UINT8 [N, groups, blob], scales FLOAT16 [N, groups],
// optional packed zero points; attributes K, N, bits, block_size.  The
// weight is prepared once (onnxl_amd_prepare_matmul_nbits) into the fused
// kernels' operands when B, scales and zero points are session constants,
// else before each run; then one fused DequantizeLinear -> MatMul call.
class Mi355xMatMulNBits : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:com.microsoft:MatMulNBits";
  using Mi355xKernel::Mi355xKernel;

  bool HasPreparations(const std::unordered_set<std::string> &immutable_inputs) const override {
    return Constants(immutable_inputs);
  }
  void DeclarePreparations(const std::unordered_set<std::string> &immutable_inputs,
                           std::vector<rt::KernelPreparation> &preparations) override {
    if (!Constants(immutable_inputs)) return;
    rt::KernelPreparation p;
    for (int i = 1; i < 4 && i < node_->input_size(); ++i)
      if (!node_->input(i).empty()) p.info.source_inputs.push_back(node_->input(i));
    p.info.representation = "mi355x:matmul-nbits-prepared-v1";
    p.info.output_slots = {node_->input(1) + ":" + p.info.representation};
    const std::vector<std::string> sources = p.info.source_inputs;
    p.estimate_memory = [sources](const rt::RuntimeContext &ctx) {
      size_t bytes = 0;
      for (const auto &s : sources) bytes += ctx.Get(s).size_bytes();
      return rt::KernelPreparationMemory{bytes, 0, 0};  // the prepared operands live in HBM
    };
    p.execute = [this](rt::RuntimeContext &ctx) {
      auto w = PrepareWeight(ctx);
      std::lock_guard<std::mutex> lock(mu_);
      weight_ = std::move(w);
    };
    preparations.push_back(std::move(p));
  }

  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 3);
    rt::RequireOutputCount(node, 1);
    for (int i = 4; i < node.input_size(); ++i)
      if (!node.input(i).empty()) throw std::invalid_argument("mi355x: MatMulNBits g_idx and bias inputs are not supported.");
    const onnxl_amd_tensor a = In(0, ctx);
    std::shared_ptr<Prepared> w = weight_ ? weight_ : PrepareWeight(ctx);  // non-constant weights: every run
    const rt::Shape shape = MatMulShape(a, w->weight.desc);
    rt::Tensor y = ctx.MakeOutputTensor(0, kFloat16, shape, static_cast<size_t>(Count(shape)) * 2);
    onnxl_amd_tensor dy = DescribeOutput(y);
    const onnxl_amd_tensor z = w->has_zp ? w->zero_point.desc : Absent();
    Check(onnxl_amd_dequantize_linear_matmul(&a, &w->weight.desc, &w->scale.desc, &z, /*axis=*/0, /*cast_to=*/0, &dy,
                                             nullptr));
    rt::SetOutput(node, 0, std::move(y), ctx);
  }

private:
  struct Prepared {
    DeviceTensor weight, scale, zero_point;
    bool has_zp = false;
  };

  bool Constants(const std::unordered_set<std::string> &immutable_inputs) const {
    for (int i = 1; i < 4 && i < node_->input_size(); ++i)
      if (!node_->input(i).empty() && immutable_inputs.count(node_->input(i)) == 0) return false;
    return node_->input_size() >= 3;
  }

  std::shared_ptr<Prepared> PrepareWeight(rt::RuntimeContext &ctx) const {
    const NodeProto &node = *node_;
    const int64_t K = rt::GetRequiredAttributeInt(node, "K"), N = rt::GetRequiredAttributeInt(node, "N");
    const int64_t bits = rt::GetRequiredAttributeInt(node, "bits");
    const int64_t block = rt::GetRequiredAttributeInt(node, "block_size");
    const onnxl_amd_tensor B = In(1, ctx), s = In(2, ctx), zp = In(3, ctx);
    auto w = std::make_shared<Prepared>();
    w->has_zp = zp.rank >= 0;
    int64_t wb = 0, sb = 0, zb = 0;
    Check(onnxl_amd_prepare_matmul_nbits_size(K, N, bits, block, w->has_zp ? 1 : 0, &wb, &sb, &zb));
    w->weight.Allocate(wb);
    w->scale.Allocate(sb);
    w->zero_point.Allocate(zb);
    for (auto *d : {&w->weight, &w->scale, &w->zero_point}) {
      d->desc = onnxl_amd_tensor{};
      d->desc.data = d->ptr;
      d->desc.location = ONNXL_AMD_DEVICE;
    }
    w->weight.desc.size_bytes = wb;
    w->scale.desc.size_bytes = sb;
    w->zero_point.desc.size_bytes = zb;
    Check(onnxl_amd_prepare_matmul_nbits(&B, &s, &zp, K, N, bits, block, &w->weight.desc, &w->scale.desc,
                                         &w->zero_point.desc, nullptr));
    Check(onnxl_amd_synchronize(nullptr));
    return w;
  }

  std::shared_ptr<Prepared> weight_;
};

// AWQ and GPTQ weights carried as encoded values (EncodedValueProto with the
// struct types "onnx_light.awq_weights.v1" / "onnx_light.gptq_weights.v1").
// The native tensors come from the reference's own exporters
// (ExportAwqWeights / ExportGptqWeights, onnx_core/runtime/quantization.h:632,
// :727), which validate the encoding and its schema; the library then takes
// them as host descriptors.
struct Checkpoint {
  bool awq = false, bitblas = false;
  std::string kind;  // AWQ variant, GPTQ format or BitBLAS originating method
  int64_t K = 0, N = 0, bits = 0, group = 0;
  int32_t symmetric = 0;  // BitBLAS
  std::unordered_map<std::string, rt::Tensor> tensors;
  onnxl_amd_tensor T(const char *name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? Absent() : Describe(&it->second);
  }
  onnxl_amd_tensor Zeros() const { return T(kind == "llm-awq" ? "scaled_zeros" : "qzeros"); }
  // The dense decode y [N, K] through the encoding's entry point.
  int Decode(onnxl_amd_tensor *y) const {
    const onnxl_amd_tensor qw = T("qweight"), sc = T("scales"), gi = T("g_idx"), qz = Zeros();
    if (bitblas)
      return onnxl_amd_dequantize_bitblas(kind.c_str(), &qw, &sc, &qz, K, N, bits, group, symmetric, y, nullptr);
    return awq ? onnxl_amd_dequantize_awq(kind.c_str(), &qw, &qz, &sc, K, N, bits, group, y, nullptr)
               : onnxl_amd_dequantize_gptq(kind.c_str(), &qw, &qz, &sc, &gi, K, N, bits, group, y, nullptr);
  }
  int PreparedSizes(int64_t *wb, int64_t *sb, int64_t *zb) const {
    const onnxl_amd_tensor qw = T("qweight"), sc = T("scales");
    if (bitblas) return onnxl_amd_prepare_bitblas_size(kind.c_str(), K, N, bits, group, symmetric, wb, sb, zb);
    return awq ? onnxl_amd_prepare_awq_size(kind.c_str(), K, N, bits, group, sc.data_type, wb, sb, zb)
               : onnxl_amd_prepare_gptq_size(kind.c_str(), K, N, bits, group, qw.data_type, sc.data_type, wb, sb, zb);
  }
  int Prepare(onnxl_amd_tensor *w, onnxl_amd_tensor *s, onnxl_amd_tensor *z) const {
    const onnxl_amd_tensor qw = T("qweight"), sc = T("scales"), gi = T("g_idx"), qz = Zeros();
    if (bitblas)
      return onnxl_amd_prepare_bitblas(kind.c_str(), &qw, &sc, &qz, K, N, bits, group, symmetric, w, s, z, nullptr);
    return awq ? onnxl_amd_prepare_awq(kind.c_str(), &qw, &qz, &sc, K, N, bits, group, w, s, z, nullptr)
               : onnxl_amd_prepare_gptq(kind.c_str(), &qw, &qz, &sc, &gi, K, N, bits, group, w, s, z, nullptr);
  }
};

// False when the encoded value is none of AWQ, GPTQ and BitBLAS.
template <typename Catalogue>
bool ExportCheckpoint(const rt::RuntimeValue &value, const Catalogue &catalogue, Checkpoint &out) {
  if (value.kind != rt::RuntimeValue::Kind::kEncoded || value.Encoded().has_parameter_ref() ||
      !value.Encoded().has_struct_type())
    return false;
  const auto &enc = value.Encoded();
  const std::string type = catalogue.Resolve(enc.struct_type()).name().value();
  if (type == "onnx_light.awq_weights.v1") {
    rt::AwqWeights w = rt::ExportAwqWeights(enc, size_t{1} << 30, catalogue);
    out.awq = true;
    out.kind = w.variant;
    out.K = w.in_features, out.N = w.out_features, out.bits = w.bits, out.group = w.group_size;
    out.tensors = std::move(w.tensors);
    return true;
  }
  if (type == "onnx_light.gptq_weights.v1") {
    rt::GptqWeights w = rt::ExportGptqWeights(enc, size_t{1} << 30, catalogue);
    out.kind = w.format;
    out.K = w.in_features, out.N = w.out_features, out.bits = w.bits, out.group = w.group_size;
    out.tensors = std::move(w.tensors);
    return true;
  }
  if (type == "onnx_light.bitblas_weights.v1") {  // layout and revision checked by the exporter
    rt::BitblasWeights w = rt::ExportBitblasWeights(enc, size_t{1} << 30, catalogue);
    out.bitblas = true;
    out.kind = w.method;
    out.K = w.in_features, out.N = w.out_features, out.bits = w.bits, out.group = w.group_size;
    out.symmetric = w.symmetric ? 1 : 0;
    out.tensors = std::move(w.tensors);
    return true;
  }
  return false;
}

// bitsandbytes weights carried as encoded values (struct type
// "onnx_light.bitsandbytes_weights.v1").  The native tensors come from the
// reference's exporter (ExportBitsAndBytesWeights, quantization.h:811), which
// validates the encoding, its schema and the JSON quant state; the state's
// numbers are the schema's constant fields (format, out_features,
// in_features, block_size, nested_block_size: bitsandbytes.cc:275-289) and
// the nested offset is read from the JSON the exporter has checked.
struct BnbCheckpoint {
  int32_t format = 0;
  int64_t rows = 0, cols = 0, block = 0, nested = 0;
  float offset = 0.f;
  std::unordered_map<std::string, rt::Tensor> tensors;
  onnxl_amd_tensor T(const char *name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? Absent() : Describe(&it->second);
  }
  onnxl_amd_tensor Absmax() const { return T(format == 2 ? "weight_scb" : "weight_absmax"); }
};

// The number after "nested_offset": in a checked JSON state.
float NestedOffset(const rt::Tensor &json) {
  const std::string text(reinterpret_cast<const char *>(json.bytes()), json.size_bytes());
  size_t at = text.find("\"nested_offset\"");
  if (at == std::string::npos) throw std::invalid_argument("mi355x: bitsandbytes state without nested_offset");
  at = text.find(':', at) + 1;
  while (at < text.size() && std::isspace(static_cast<unsigned char>(text[at]))) ++at;
  size_t end = at;
  while (end < text.size() && text[end] != ',' && text[end] != '}' &&
         !std::isspace(static_cast<unsigned char>(text[end])))
    ++end;
  double value = 0;
  const auto parsed = std::from_chars(text.data() + at, text.data() + end, value);
  if (parsed.ec != std::errc{}) throw std::invalid_argument("mi355x: bitsandbytes invalid nested offset");
  return static_cast<float>(value);
}

// False when the encoded value is not a bitsandbytes weight.
template <typename Catalogue>
bool ExportBitsAndBytes(const rt::RuntimeValue &value, const Catalogue &catalogue, BnbCheckpoint &out) {
  if (value.kind != rt::RuntimeValue::Kind::kEncoded || value.Encoded().has_parameter_ref() ||
      !value.Encoded().has_struct_type())
    return false;
  const auto &enc = value.Encoded();
  const auto &type = catalogue.Resolve(enc.struct_type());
  if (type.name().value() != "onnx_light.bitsandbytes_weights.v1") return false;
  rt::BitsAndBytesWeights w = rt::ExportBitsAndBytesWeights(enc, size_t{1} << 30, catalogue);
  auto number = [&](int i) { return type.structure().field(i).constant().int64_data(0); };
  out.format = static_cast<int32_t>(number(0));
  out.rows = number(1);
  out.cols = number(2);
  out.block = number(3);
  out.nested = number(4);
  out.tensors = std::move(w.tensors);
  if (out.nested) out.offset = NestedOffset(out.tensors.at("weight_quant_state"));
  return true;
}

// VPTQ weights carried as encoded values (struct type
// "onnx_light.vptq_weights.v1"): the constructor metadata and native tensors
// from the reference's exporter (ExportVptqWeights, quantization.h:901),
// which validates the encoding and its canonical schema.
struct VptqCheckpoint {
  onnxl_amd_vptq_config config{};
  int32_t dtype = 0;
  std::unordered_map<std::string, rt::Tensor> tensors;
  int Decode(onnxl_amd_tensor *y) const {
    auto t = [&](const char *name) {
      auto it = tensors.find(name);
      return it == tensors.end() ? Absent() : Describe(&it->second);
    };
    const onnxl_amd_tensor ix = t("indices"), c = t("centroids.weight"), rc = t("res_centroids.weight");
    const onnxl_amd_tensor oc = t("outlier_centroids.weight"), oi = t("outlier_indices");
    const onnxl_amd_tensor sc = t("weight_scale"), bi = t("weight_bias"), pm = t("perm");
    return onnxl_amd_dequantize_vptq(&config, &ix, &c, &rc, &oc, &oi, &sc, &bi, &pm, y, nullptr);
  }
};

// False when the encoded value is not a VPTQ weight.
template <typename Catalogue>
bool ExportVptq(const rt::RuntimeValue &value, const Catalogue &catalogue, VptqCheckpoint &out) {
  if (value.kind != rt::RuntimeValue::Kind::kEncoded || value.Encoded().has_parameter_ref() ||
      !value.Encoded().has_struct_type())
    return false;
  const auto &enc = value.Encoded();
  if (catalogue.Resolve(enc.struct_type()).name().value() != "onnx_light.vptq_weights.v1") return false;
  rt::VptqWeights w = rt::ExportVptqWeights(enc, size_t{1} << 30, catalogue);
  onnxl_amd_vptq_config &c = out.config;
  c.in_features = w.in_features;
  c.out_features = w.out_features;
  c.bits = w.bits;
  for (int i = 0; i < 2; ++i) {
    c.vector_lens[i] = w.vector_lens[i];
    c.num_centroids[i] = w.num_centroids[i];
    c.num_res_centroids[i] = w.num_res_centroids[i];
  }
  c.npercent = w.npercent;
  c.group_size = w.group_size;
  c.group_num = w.group_num;
  c.enable_norm = w.enable_norm ? 1 : 0;
  c.norm_dim = static_cast<int32_t>(w.norm_dim);
  c.enable_perm = w.enable_perm ? 1 : 0;
  out.tensors = std::move(w.tensors);
  return true;
}

// GPTQModel FP8 weights carried as encoded values (struct type
// "onnx_light.gptqmodel_fp8_weights.v1"): the FP8 codes and inverse scales
// from the reference's exporter (ExportGptqModelFp8Weights,
// quantization.h:607), which validates the encoding, its schema and the
// inverse-scale semantics.
struct GptqFp8Checkpoint {
  int64_t k = 0, n = 0;
  std::string method;
  std::vector<int64_t> block;
  std::unordered_map<std::string, rt::Tensor> tensors;
  int Decode(onnxl_amd_tensor *y) const {
    const onnxl_amd_tensor w = Describe(&tensors.at("weight")), s = Describe(&tensors.at("weight_scale_inv"));
    return onnxl_amd_dequantize_gptqmodel_fp8(k, n, method.c_str(), block.empty() ? nullptr : block.data(),
                                              static_cast<int32_t>(block.size()), &w, &s, y, nullptr);
  }
};

// False when the encoded value is not a GPTQModel FP8 weight.
template <typename Catalogue>
bool ExportGptqFp8(const rt::RuntimeValue &value, const Catalogue &catalogue, GptqFp8Checkpoint &out) {
  if (value.kind != rt::RuntimeValue::Kind::kEncoded || value.Encoded().has_parameter_ref() ||
      !value.Encoded().has_struct_type())
    return false;
  const auto &enc = value.Encoded();
  if (catalogue.Resolve(enc.struct_type()).name().value() != "onnx_light.gptqmodel_fp8_weights.v1") return false;
  rt::GptqModelFp8Weights w = rt::ExportGptqModelFp8Weights(enc, size_t{1} << 30, catalogue);
  out.k = w.in_features;
  out.n = w.out_features;
  out.method = w.weight_scale_method;
  out.block.assign(w.weight_block_size.begin(), w.weight_block_size.end());
  out.tensors = std::move(w.tensors);
  return true;
}

// QQQ weights carried as encoded values (struct type
// "onnx_light.qqq_weights.v1").  The native tensors (B, s_channel, s_group)
// and numbers come from the reference's exporter (ExportQqqWeights,
// quantization.h:697), which validates the encoding and its schema.
struct QqqCheckpoint {
  int64_t k = 0, n = 0, group = -1, bits = 4;
  std::unordered_map<std::string, rt::Tensor> tensors;
  onnxl_amd_tensor T(const char *name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? Absent() : Describe(&it->second);
  }
};

// False when the encoded value is not a QQQ weight.
template <typename Catalogue>
bool ExportQqq(const rt::RuntimeValue &value, const Catalogue &catalogue, QqqCheckpoint &out) {
  if (value.kind != rt::RuntimeValue::Kind::kEncoded || value.Encoded().has_parameter_ref() ||
      !value.Encoded().has_struct_type())
    return false;
  const auto &enc = value.Encoded();
  if (catalogue.Resolve(enc.struct_type()).name().value() != "onnx_light.qqq_weights.v1") return false;
  rt::QqqWeights w = rt::ExportQqqWeights(enc, size_t{1} << 30, catalogue);
  out.k = w.in_features;
  out.n = w.out_features;
  out.group = w.group_size;
  out.bits = static_cast<int64_t>(w.bits);
  out.tensors = std::move(w.tensors);
  return true;
}

// EXL3 weights carried as encoded values (struct type
// "onnx_light.exl3_weights.v1"): the trellis, suh, svh and codebook marker
// from the reference's exporter (ExportExl3Weights, quantization.h:851),
// which validates the encoding, its schema and the upstream revision.
struct Exl3Checkpoint {
  std::unordered_map<std::string, rt::Tensor> tensors;
  int64_t k = 0, n = 0;
  onnxl_amd_tensor T(const char *name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? Absent() : Describe(&it->second);
  }
  int Decode(onnxl_amd_tensor *y) const {
    const onnxl_amd_tensor t = T("trellis"), u = T("suh"), v = T("svh"), m1 = T("mcg"), m2 = T("mul1");
    return onnxl_amd_dequantize_exl3(&t, &u, &v, &m1, &m2, y, nullptr);
  }
};

// False when the encoded value is not an EXL3 weight.
template <typename Catalogue>
bool ExportExl3(const rt::RuntimeValue &value, const Catalogue &catalogue, Exl3Checkpoint &out) {
  if (value.kind != rt::RuntimeValue::Kind::kEncoded || value.Encoded().has_parameter_ref() ||
      !value.Encoded().has_struct_type())
    return false;
  const auto &enc = value.Encoded();
  if (catalogue.Resolve(enc.struct_type()).name().value() != "onnx_light.exl3_weights.v1") return false;
  rt::Exl3Weights w = rt::ExportExl3Weights(enc, size_t{1} << 30, catalogue);
  out.tensors = std::move(w.tensors);
  const rt::Tensor &trellis = out.tensors.at("trellis");
  out.k = trellis.shape[0] * 16;
  out.n = trellis.shape[1] * 16;
  return true;
}

// MX and NVFP4 weights carried as encoded values (struct types
// "onnx_light.mxfp4_weights.v1", "onnx_light.mxfp6_e2m3_weights.v1",
// "onnx_light.mxfp8_weights.v1", "onnx_light.nvfp4_weights.v1"): the native
// tensors from the reference's exporters (ExportMxfp4Weights /
// ExportMxfp6E2m3Weights / ExportMxfp8Weights / ExportNvfp4Weights,
// quantization.h:943-1012), which validate the encoding and its schema.
struct MxCheckpoint {
  std::string format;
  rt::Tensor weight, scale;
  float global = 0.f;
  int64_t rows = 0, cols = 0;
  int Decode(onnxl_amd_tensor *y) const {
    const onnxl_amd_tensor w = Describe(&weight), s = Describe(&scale);
    return onnxl_amd_dequantize_mx_weights(format.c_str(), &w, &s, global, y, nullptr);
  }
};

// False when the encoded value is not an MX / NVFP4 weight.
template <typename Catalogue>
bool ExportMx(const rt::RuntimeValue &value, const Catalogue &catalogue, MxCheckpoint &out) {
  if (value.kind != rt::RuntimeValue::Kind::kEncoded || value.Encoded().has_parameter_ref() ||
      !value.Encoded().has_struct_type())
    return false;
  const auto &enc = value.Encoded();
  const std::string type = catalogue.Resolve(enc.struct_type()).name().value();
  if (type == "onnx_light.mxfp4_weights.v1") {
    rt::Mxfp4Weights w = rt::ExportMxfp4Weights(enc, catalogue);
    out.format = "mxfp4", out.weight = std::move(w.weight_packed), out.scale = std::move(w.weight_scale);
    out.cols = out.weight.shape[1] * 2;
  } else if (type == "onnx_light.mxfp6_e2m3_weights.v1") {
    rt::Mxfp6E2m3Weights w = rt::ExportMxfp6E2m3Weights(enc, catalogue);
    out.format = "mxfp6_e2m3", out.weight = std::move(w.weight_packed), out.scale = std::move(w.weight_scale);
    out.cols = out.weight.shape[1] / 3 * 4;
  } else if (type == "onnx_light.mxfp8_weights.v1") {
    rt::Mxfp8Weights w = rt::ExportMxfp8Weights(enc, catalogue);
    out.format = "mxfp8", out.weight = std::move(w.weight), out.scale = std::move(w.weight_scale);
    out.cols = out.weight.shape[1];
  } else if (type == "onnx_light.nvfp4_weights.v1") {
    rt::Nvfp4Weights w = rt::ExportNvfp4Weights(enc, catalogue);
    out.format = "nvfp4", out.weight = std::move(w.weight_packed), out.scale = std::move(w.weight_scale);
    out.global = w.weight_global_scale;
    out.cols = out.weight.shape[1] * 2;
  } else {
    return false;
  }
  out.rows = out.weight.shape[0];
  return true;
}

// ai.rt:Dequantize(Q; dtype) (onnx_extensions/kernels/kernels/quantization/
// kernel_dequantize.cc:18-43): AWQ, GPTQ, BitBLAS, bitsandbytes, QQQ,
// GPTQModel FP8 and VPTQ encodings decode on the GPU to [out_features,
// in_features] of dtype (onnxl_amd_dequantize_awq / _gptq / _bitblas /
// _bitsandbytes / _qqq / _gptqmodel_fp8 / _vptq), the MX / NVFP4 weights to
// their [rows, cols] (onnxl_amd_dequantize_mx_weights) and EXL3 weights to
// their [k, n] (onnxl_amd_dequantize_exl3); every other
// encoding, and values that reference shared parameters, run on the built-in
// kernel.
class Mi355xDequantize : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.rt:Dequantize";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireInputCount(node, 1);
    rt::RequireOutputCount(node, 1);
    const int64_t dtype = rt::GetRequiredAttributeInt(node, "dtype");
    if (dtype != kFloat && dtype != kDouble && dtype != kFloat16 && dtype != kBfloat16)
      throw std::invalid_argument("Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16.");
    const auto value = ctx.values().find(node.input(0));
    BnbCheckpoint b;
    if (value != ctx.values().end() && ExportBitsAndBytes(value->second, ctx.struct_type_catalogue(), b)) {
      const rt::Shape shape{b.rows, b.cols};
      rt::Tensor y = ctx.MakeOutputTensor(0, static_cast<int32_t>(dtype), shape,
                                          ByteSize(static_cast<int32_t>(dtype), Count(shape)));
      onnxl_amd_tensor dy = DescribeOutput(y);
      const onnxl_amd_tensor w = b.T("weight"), am = b.Absmax(), qm = b.T("weight_quant_map");
      const onnxl_amd_tensor na = b.T("weight_nested_absmax"), nm = b.T("weight_nested_quant_map");
      if (Call(onnxl_amd_dequantize_bitsandbytes(b.format, b.rows, b.cols, b.block, b.nested, b.offset, &w, &am, &qm,
                                                 &na, &nm, &dy, nullptr),
               ctx))
        rt::SetOutput(node, 0, std::move(y), ctx);
      return;
    }
    VptqCheckpoint v;
    if (value != ctx.values().end() && ExportVptq(value->second, ctx.struct_type_catalogue(), v)) {
      const rt::Shape shape{v.config.out_features, v.config.in_features};
      rt::Tensor y = ctx.MakeOutputTensor(0, static_cast<int32_t>(dtype), shape,
                                          ByteSize(static_cast<int32_t>(dtype), Count(shape)));
      onnxl_amd_tensor dy = DescribeOutput(y);
      if (Call(v.Decode(&dy), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
      return;
    }
    GptqFp8Checkpoint f;
    if (value != ctx.values().end() && ExportGptqFp8(value->second, ctx.struct_type_catalogue(), f)) {
      const rt::Shape shape{f.n, f.k};
      rt::Tensor y = ctx.MakeOutputTensor(0, static_cast<int32_t>(dtype), shape,
                                          ByteSize(static_cast<int32_t>(dtype), Count(shape)));
      onnxl_amd_tensor dy = DescribeOutput(y);
      if (Call(f.Decode(&dy), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
      return;
    }
    Exl3Checkpoint x3;
    if (value != ctx.values().end() && ExportExl3(value->second, ctx.struct_type_catalogue(), x3)) {
      const rt::Shape shape{x3.k, x3.n};
      rt::Tensor y = ctx.MakeOutputTensor(0, static_cast<int32_t>(dtype), shape,
                                          ByteSize(static_cast<int32_t>(dtype), Count(shape)));
      onnxl_amd_tensor dy = DescribeOutput(y);
      if (Call(x3.Decode(&dy), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
      return;
    }
    MxCheckpoint mx;
    if (value != ctx.values().end() && ExportMx(value->second, ctx.struct_type_catalogue(), mx)) {
      const rt::Shape shape{mx.rows, mx.cols};
      rt::Tensor y = ctx.MakeOutputTensor(0, static_cast<int32_t>(dtype), shape,
                                          ByteSize(static_cast<int32_t>(dtype), Count(shape)));
      onnxl_amd_tensor dy = DescribeOutput(y);
      if (Call(mx.Decode(&dy), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
      return;
    }
    QqqCheckpoint q;
    if (value != ctx.values().end() && ExportQqq(value->second, ctx.struct_type_catalogue(), q)) {
      const rt::Shape shape{q.n, q.k};
      rt::Tensor y = ctx.MakeOutputTensor(0, static_cast<int32_t>(dtype), shape,
                                          ByteSize(static_cast<int32_t>(dtype), Count(shape)));
      onnxl_amd_tensor dy = DescribeOutput(y);
      const onnxl_amd_tensor qb = q.T("B"), qc = q.T("s_channel"), qg = q.T("s_group");
      if (Call(onnxl_amd_dequantize_qqq(q.k, q.n, q.group, q.bits, &qb, &qc, &qg, &dy, nullptr), ctx))
        rt::SetOutput(node, 0, std::move(y), ctx);
      return;
    }
    Checkpoint c;
    if (value == ctx.values().end() || !ExportCheckpoint(value->second, ctx.struct_type_catalogue(), c)) {
      RunBuiltin(ctx, "encoding other than AWQ / GPTQ / BitBLAS / bitsandbytes / QQQ / GPTQModel FP8 / VPTQ / MX / EXL3");
      return;
    }
    const rt::Shape shape{c.N, c.K};
    rt::Tensor y = ctx.MakeOutputTensor(0, static_cast<int32_t>(dtype), shape,
                                        ByteSize(static_cast<int32_t>(dtype), Count(shape)));
    onnxl_amd_tensor dy = DescribeOutput(y);
    if (Call(c.Decode(&dy), ctx)) rt::SetOutput(node, 0, std::move(y), ctx);
  }
};

// ---------------------------------------------------------------------------
// Fused nodes.  They exist only in graphs rewritten by the GPU patterns, so
// there is no built-in kernel: the adapter computes their chain itself when
// the fused kernel does not take an input.

// ai.rt.amd:DequantizeLinearMatMul(A, x, x_scale[, x_zero_point]; axis,
// cast_to) = MatMul(A, [Cast(to=cast_to)](DequantizeLinear(x, x_scale,
// x_zero_point, axis))).  A constant INT4 / UINT4 weight is tiled once at
// preparation.  When x, x_scale and x_zero_point are all prepared, each run
// stages A into a reused device buffer and calls the no-allocation entry
// point, so a steady serving loop performs no device allocation at all; when
// that entry point's fixed scratch is too small it calls the allocating one.
class Mi355xDequantizeLinearMatMul : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.rt.amd:DequantizeLinearMatMul";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 3);
    rt::RequireOutputCount(node, 1);
    const int64_t axis = rt::GetAttributeIntOrDefault(node, "axis", 1);
    const int32_t cast_to = static_cast<int32_t>(rt::GetAttributeIntOrDefault(node, "cast_to", 0));
    onnxl_amd_tensor a = In(0, ctx), x = In(1, ctx), s = In(2, ctx), z = In(3, ctx);
    // logical weight shape [K, N] (a prepared weight's dims are the logical ones)
    const rt::Shape shape = MatMulShape(a, x);
    const size_t y_bytes = static_cast<size_t>(Count(shape)) * 2;
    rt::Tensor y = ctx.MakeOutputTensor(0, a.data_type, shape, y_bytes);
    onnxl_amd_tensor dy = DescribeOutput(y);
    const bool constants_on_device = Prepared(1) && Prepared(2) && (z.rank < 0 || Prepared(3));
    if (constants_on_device) {
      // device-resident call: stage A, compute, copy Y back
      const size_t a_bytes = static_cast<size_t>(a.size_bytes);
      void *da = a_stage_.Reserve(a_bytes);
      void *dyp = y_stage_.Reserve(y_bytes);
      if (a_bytes > 0) CheckHip(hipMemcpy(da, a.data, a_bytes, hipMemcpyHostToDevice), "hipMemcpy");
      onnxl_amd_tensor ad = a, yd = dy;
      ad.data = da;
      ad.location = ONNXL_AMD_DEVICE;
      yd.data = dyp;
      yd.location = ONNXL_AMD_DEVICE;
      int rc = onnxl_amd_dequantize_linear_matmul_noalloc(&ad, &x, &s, &z, axis, cast_to, &yd, nullptr);
      if (rc == ONNXL_AMD_UNSUPPORTED)  // beyond the fixed scratch: the allocating entry point
        rc = onnxl_amd_dequantize_linear_matmul(&ad, &x, &s, &z, axis, cast_to, &yd, nullptr);
      if (rc == ONNXL_AMD_UNSUPPORTED) {
        RunChain(ctx, a, x, s, z, axis, cast_to, y);
      } else {
        Check(rc);
        Check(onnxl_amd_synchronize(nullptr));
        if (y_bytes > 0) CheckHip(hipMemcpy(y.mutable_bytes(), dyp, y_bytes, hipMemcpyDeviceToHost), "hipMemcpy");
      }
    } else {
      const int rc = onnxl_amd_dequantize_linear_matmul(&a, &x, &s, &z, axis, cast_to, &dy, nullptr);
      if (rc == ONNXL_AMD_UNSUPPORTED) RunChain(ctx, a, x, s, z, axis, cast_to, y);
      else Check(rc);
    }
    rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1, 2, 3}; }
  std::string Representation(int index) const override {
    return index == 1 ? "mi355x:tiled-int4-or-hbm-copy-v1" : "mi355x:hbm-copy-v1";
  }
  std::shared_ptr<DeviceTensor> Prepare(int index, const rt::Tensor &t) override {
    if (index != 1 || (t.data_type != kInt4 && t.data_type != kUint4) || t.shape.size() != 2) return UploadToHbm(t);
    // Tiled 4-bit weight: each 16-column tile's K range contiguous.
    auto host = Describe(&t);
    int64_t bytes = 0;
    Check(onnxl_amd_prepare_weight_size(&host, &bytes));
    auto d = std::make_shared<DeviceTensor>();
    d->Allocate(bytes);
    d->desc = onnxl_amd_tensor{};
    d->desc.data = d->ptr;
    d->desc.size_bytes = bytes;
    d->desc.location = ONNXL_AMD_DEVICE;
    Check(onnxl_amd_prepare_weight(&host, &d->desc, nullptr));
    Check(onnxl_amd_synchronize(nullptr));
    return d;
  }

private:
  // The unfused chain on the GPU for inputs the fused kernel does not take:
  // DequantizeLinear into x_scale's dtype, the optional Cast, then MatMul.
  void RunChain(rt::RuntimeContext &ctx, const onnxl_amd_tensor &a, const onnxl_amd_tensor &x,
                const onnxl_amd_tensor &s, const onnxl_amd_tensor &z, int64_t axis, int32_t cast_to, rt::Tensor &y) {
    if (x.layout != ONNXL_AMD_LAYOUT_ONNX)
      throw std::runtime_error("mi355x: DequantizeLinearMatMul: prepared weight outside the fused kernel's range");
    const rt::Shape wshape = ShapeOf(x.dims, x.rank);
    const int64_t n = Count(wshape);
    rt::Tensor w = ctx.MakeTemporaryTensor(s.data_type, wshape, ByteSize(s.data_type, n));
    onnxl_amd_tensor dw = DescribeOutput(w);
    Check(onnxl_amd_dequantize_linear(&x, &s, &z, axis, &dw, nullptr));
    onnxl_amd_tensor b = dw;
    rt::Tensor wc;
    if (cast_to != 0) {
      wc = ctx.MakeTemporaryTensor(cast_to, wshape, static_cast<size_t>(n) * 2);
      onnxl_amd_tensor dwc = DescribeOutput(wc);
      Check(onnxl_amd_cast(&dw, cast_to, &dwc, nullptr));
      b = dwc;
    }
    onnxl_amd_tensor dy = DescribeOutput(y);
    Check(onnxl_amd_matmul(&a, &b, &dy, nullptr));
  }

  Staging a_stage_, y_stage_;
};

// ai.rt.amd:DequantizeLinearGroupedMatMul(input, x, x_scale, x_zero_point | "",
// group_indices[, bias]; axis, cast_to, transB) = GroupedMatMul(input,
// [Cast(to=cast_to)](DequantizeLinear(x, x_scale, x_zero_point, axis)),
// group_indices, bias, transB): quantized MoE experts.  The constant experts,
// scales, zero points and bias are kept in HBM; one fused call per run (fp8
// experts on the matrix cores, the others dequantized on the device into the
// 16-bit grouped GEMM).
class Mi355xDequantizeLinearGroupedMatMul : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.rt.amd:DequantizeLinearGroupedMatMul";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireMinInputCount(node, 5);
    rt::RequireOutputCount(node, 1);
    const int64_t axis = rt::GetAttributeIntOrDefault(node, "axis", 1);
    const int32_t cast_to = static_cast<int32_t>(rt::GetAttributeIntOrDefault(node, "cast_to", 0));
    const int64_t transB = rt::GetAttributeIntOrDefault(node, "transB", 0);
    const onnxl_amd_tensor a = In(0, ctx), x = In(1, ctx), s = In(2, ctx), z = In(3, ctx), idx = In(4, ctx),
                           b = In(5, ctx);
    if (a.rank != 2 || x.rank != 3 || idx.rank != 2) {  // the library raises the reference's error
      onnxl_amd_tensor none{};
      Check(onnxl_amd_dequantize_linear_grouped_matmul(&a, &x, &s, &z, axis, cast_to, &idx, &b, transB, &none,
                                                       nullptr));
    }
    const rt::Shape shape{a.dims[0], idx.dims[1], x.dims[transB != 0 ? 1 : 2]};
    rt::Tensor y = ctx.MakeOutputTensor(0, a.data_type, shape, static_cast<size_t>(Count(shape)) * 2);
    onnxl_amd_tensor dy = DescribeOutput(y);
    const int rc = onnxl_amd_dequantize_linear_grouped_matmul(&a, &x, &s, &z, axis, cast_to, &idx, &b, transB, &dy,
                                                              nullptr);
    if (rc == ONNXL_AMD_UNSUPPORTED) RunChain(ctx, a, x, s, z, axis, cast_to, idx, b, transB, y);
    else Check(rc);
    rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1, 2, 3, 5}; }

private:
  // The unfused chain through the library: DequantizeLinear into x_scale's
  // dtype, the optional Cast, then GroupedMatMul.
  void RunChain(rt::RuntimeContext &ctx, const onnxl_amd_tensor &a, const onnxl_amd_tensor &x,
                const onnxl_amd_tensor &s, const onnxl_amd_tensor &z, int64_t axis, int32_t cast_to,
                const onnxl_amd_tensor &idx, const onnxl_amd_tensor &b, int64_t transB, rt::Tensor &y) {
    const rt::Shape wshape = ShapeOf(x.dims, x.rank);
    const int64_t n = Count(wshape);
    rt::Tensor w = ctx.MakeTemporaryTensor(s.data_type, wshape, ByteSize(s.data_type, n));
    onnxl_amd_tensor dw = DescribeOutput(w);
    Check(onnxl_amd_dequantize_linear(&x, &s, &z, axis, &dw, nullptr));
    onnxl_amd_tensor wt = dw;
    rt::Tensor wc;
    if (cast_to != 0) {
      wc = ctx.MakeTemporaryTensor(cast_to, wshape, static_cast<size_t>(n) * 2);
      onnxl_amd_tensor dwc = DescribeOutput(wc);
      Check(onnxl_amd_cast(&dw, cast_to, &dwc, nullptr));
      wt = dwc;
    }
    onnxl_amd_tensor dy = DescribeOutput(y);
    Check(onnxl_amd_grouped_matmul(&a, &wt, &idx, &b, transB, &dy, nullptr));
  }
};

// ai.rt.amd:DequantizePackedMatMul(A, x; format, shape = [N, K]) =
// MatMul(A, Transpose(DequantizePacked(x, format, shape, FLOAT16))), the
// chain onnx_core/runtime/dequantize_packed.cc:334-372 -> km/kernel_matmul.cc.
// Every GGUF profile and M runs in the one entry point: the fused decode
// GEMVs (q4_0, q8_0, q2_k-q6_k, iq4_xs at M <= 8), else the weight decoded to
// FLOAT16 [N, K] on the device and multiplied by the MFMA GEMM reading its
// rows, with no transpose written and nothing staged on the host.
class Mi355xDequantizePackedMatMul : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.rt.amd:DequantizePackedMatMul";
  using Mi355xKernel::Mi355xKernel;
  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireInputCount(node, 2);
    rt::RequireOutputCount(node, 1);
    const std::string format = rt::GetRequiredAttributeString(node, "format");
    const std::vector<int64_t> nk = rt::GetAttributeIntsOrDefault(node, "shape", {});
    if (nk.size() != 2) throw std::invalid_argument("DequantizePackedMatMul: shape must be [N, K].");
    const onnxl_amd_tensor a = In(0, ctx), x = In(1, ctx);
    onnxl_amd_tensor wt{};  // logical [K, N] operand for the output shape
    wt.rank = 2;
    wt.dims[0] = nk[1];
    wt.dims[1] = nk[0];
    const rt::Shape shape = MatMulShape(a, wt);
    rt::Tensor y = ctx.MakeOutputTensor(0, kFloat16, shape, static_cast<size_t>(Count(shape)) * 2);
    onnxl_amd_tensor dy = DescribeOutput(y);
    // every format and M runs on the device (decode GEMV, or the decoded
    // weight through the MFMA GEMM): nothing comes back to the host here
    Check(onnxl_amd_dequantize_packed_matmul(&a, &x, format.c_str(), nk.data(), 2, &dy, nullptr));
    rt::SetOutput(node, 0, std::move(y), ctx);
  }

protected:
  std::vector<int> ConstantInputs() const override { return {1}; }
};

// ai.rt.amd:DequantizeEncodedMatMul(A, Q) = MatMul(A, Transpose(Dequantize(Q,
// dtype = A's dtype))) for an encoded weight Q of logical shape [N, K] (the
// node the DequantizeEncodedMatMulGpu pattern writes): an AWQ, GPTQ, BitBLAS
// or QQQ weight is prepared once (onnxl_amd_prepare_awq / _gptq / _bitblas /
// _qqq) into the fused DequantizeLinear -> MatMul operands when Q is a
// session constant, else before each run; then one fused call.  What the preparation does not take
// (AWQ gemv_fast / llm-awq, GPTQ act-order group maps and partial groups)
// decodes to a dense weight on the GPU, and any other encoding through the
// reference's DequantizeTensor; the dense weight is transposed once and the
// MatMul runs on the GPU.
class Mi355xDequantizeEncodedMatMul : public Mi355xKernel {
public:
  static constexpr const char *name = "onnxl_amd:CPU:ai.rt.amd:DequantizeEncodedMatMul";
  using Mi355xKernel::Mi355xKernel;

  bool HasPreparations(const std::unordered_set<std::string> &immutable_inputs) const override {
    return node_->input_size() >= 2 && immutable_inputs.count(node_->input(1)) != 0;
  }
  void DeclarePreparations(const std::unordered_set<std::string> &immutable_inputs,
                           std::vector<rt::KernelPreparation> &preparations) override {
    if (!HasPreparations(immutable_inputs)) return;
    rt::KernelPreparation p;
    p.info.source_inputs = {node_->input(1)};
    p.info.representation = "mi355x:encoded-weight-prepared-v1";
    p.info.output_slots = {node_->input(1) + ":" + p.info.representation};
    p.estimate_memory = [](const rt::RuntimeContext &) { return rt::KernelPreparationMemory{0, 0, 0}; };
    p.execute = [this](rt::RuntimeContext &ctx) {
      auto w = PrepareWeight(ctx);
      std::lock_guard<std::mutex> lock(mu_);
      weight_ = std::move(w);
    };
    preparations.push_back(std::move(p));
  }

  void Run(rt::RuntimeContext &ctx) override {
    const NodeProto &node = *node_;
    rt::RequireInputCount(node, 2);
    rt::RequireOutputCount(node, 1);
    const onnxl_amd_tensor a = In(0, ctx);
    std::shared_ptr<Prepared> w = weight_ ? weight_ : PrepareWeight(ctx);
    if (w->bnb) {  // the bitsandbytes codes and resolved scales in HBM, one fused call
      rt::Shape shape(a.dims, a.dims + a.rank);
      if (shape.empty() || shape.back() != w->cols)
        throw std::invalid_argument("mi355x: DequantizeEncodedMatMul: A's last dimension must be in_features.");
      shape.back() = w->rows;
      rt::Tensor y = ctx.MakeOutputTensor(0, a.data_type, shape, static_cast<size_t>(Count(shape)) * 2);
      onnxl_amd_tensor dy = DescribeOutput(y);
      Check(onnxl_amd_bitsandbytes_matmul(&a, w->format, w->rows, w->cols, w->block, &w->weight.desc,
                                          &w->scale.desc, &dy, nullptr));
      rt::SetOutput(node, 0, std::move(y), ctx);
      return;
    }
    if (!w->fused) {  // the decoded weight [K, N] in HBM, MatMul on the GPU
      const rt::Shape shape = MatMulShape(a, w->dense_t.desc);
      rt::Tensor y = ctx.MakeOutputTensor(0, a.data_type, shape, static_cast<size_t>(Count(shape)) * 2);
      onnxl_amd_tensor dy = DescribeOutput(y);
      Check(onnxl_amd_matmul(&a, &w->dense_t.desc, &dy, nullptr));
      rt::SetOutput(node, 0, std::move(y), ctx);
      return;
    }
    const rt::Shape shape = MatMulShape(a, w->weight.desc);
    rt::Tensor y = ctx.MakeOutputTensor(0, a.data_type, shape, static_cast<size_t>(Count(shape)) * 2);
    onnxl_amd_tensor dy = DescribeOutput(y);
    const int32_t cast_to = w->scale.desc.data_type == kFloat ? a.data_type : 0;
    const int64_t axis = w->scale.desc.rank == 1 ? 1 : 0;  // per-column (QQQ) or blocked along K
    Check(onnxl_amd_dequantize_linear_matmul(&a, &w->weight.desc, &w->scale.desc, &w->zero_point.desc, axis,
                                             cast_to, &dy, nullptr));
    rt::SetOutput(node, 0, std::move(y), ctx);
  }

private:
  struct Prepared {
    bool fused = false;
    DeviceTensor weight, scale, zero_point;  // fused operands (bitsandbytes: codes and resolved scales)
    DeviceTensor dense_t;                    // the decoded weight, transposed to [K, N]
    bool bnb = false;
    int32_t format = 0;
    int64_t rows = 0, cols = 0, block = 0;
  };

  // A bitsandbytes weight: its codes uploaded once, the reference's checks
  // and the nonfinite-reconstruction check in A's dtype once, the block scales
  // resolved once (onnxl_amd_prepare_bitsandbytes).
  std::shared_ptr<Prepared> PrepareBitsAndBytes(rt::RuntimeContext &ctx, const BnbCheckpoint &b) const {
    const onnxl_amd_tensor a = In(0, ctx);
    auto w = std::make_shared<Prepared>();
    w->bnb = true;
    w->format = b.format;
    w->rows = b.rows;
    w->cols = b.cols;
    w->block = b.block;
    const onnxl_amd_tensor codes = b.T("weight"), am = b.Absmax(), qm = b.T("weight_quant_map");
    const onnxl_amd_tensor na = b.T("weight_nested_absmax"), nm = b.T("weight_nested_quant_map");
    w->weight.Allocate(codes.size_bytes);
    if (codes.size_bytes > 0)
      CheckHip(hipMemcpy(w->weight.ptr, codes.data, static_cast<size_t>(codes.size_bytes), hipMemcpyHostToDevice),
               "hipMemcpy");
    w->weight.desc = codes;
    w->weight.desc.data = w->weight.ptr;
    w->weight.desc.location = ONNXL_AMD_DEVICE;
    int64_t sb = 0;
    Check(onnxl_amd_prepare_bitsandbytes_size(b.format, b.rows, b.cols, b.block, &sb));
    w->scale.Allocate(sb);
    w->scale.desc = onnxl_amd_tensor{};
    w->scale.desc.data = w->scale.ptr;
    w->scale.desc.location = ONNXL_AMD_DEVICE;
    w->scale.desc.size_bytes = sb;
    Check(onnxl_amd_prepare_bitsandbytes(b.format, b.rows, b.cols, b.block, b.nested, b.offset, &w->weight.desc, &am,
                                         &qm, &na, &nm, a.data_type, &w->scale.desc, nullptr));
    Check(onnxl_amd_synchronize(nullptr));
    return w;
  }

  // FLOAT16 scales widened to FLOAT (exactly), once per weight: with BFLOAT16
  // activations the fused node then runs DequantizeLinear in FLOAT and casts
  // each weight to BFLOAT16, which is the reference's one rounding of the
  // FLOAT value (Dequantize with dtype = BFLOAT16); a FLOAT16 DequantizeLinear
  // output could not feed a BFLOAT16 MatMul.
  static void WidenScales(DeviceTensor &scale) {
    const size_t count = static_cast<size_t>(scale.desc.size_bytes / 2);
    std::vector<uint16_t> h(count);
    std::vector<float> f(count);
    CheckHip(hipMemcpy(h.data(), scale.ptr, count * 2, hipMemcpyDeviceToHost), "hipMemcpy");
    for (size_t i = 0; i < count; ++i) f[i] = rt::Float16BitsToFloat(h[i]);
    void *wide = nullptr;
    CheckHip(hipMalloc(&wide, count * 4 > 0 ? count * 4 : 16), "hipMalloc");
    CheckHip(hipMemcpy(wide, f.data(), count * 4, hipMemcpyHostToDevice), "hipMemcpy");
    CheckHip(hipFree(scale.ptr), "hipFree");
    scale.ptr = wide;
    scale.desc.data = wide;
    scale.desc.data_type = kFloat;
    scale.desc.size_bytes = static_cast<int64_t>(count * 4);
  }

  // A QQQ weight: the reference's checks in A's dtype once, then the fused
  // operands (tiled INT4 codes with 16 x channel scales, or INT8 integers with
  // the channel scales) for onnxl_amd_dequantize_linear_matmul; null when
  // the library has no such operand for it (UNSUPPORTED).
  std::shared_ptr<Prepared> PrepareQqq(rt::RuntimeContext &ctx, const QqqCheckpoint &q) const {
    const onnxl_amd_tensor a = In(0, ctx);
    int64_t wb = 0, sb = 0;
    Check(onnxl_amd_prepare_qqq_size(q.k, q.n, q.group, q.bits, &wb, &sb));
    auto w = std::make_shared<Prepared>();
    w->weight.Allocate(wb);
    w->scale.Allocate(sb);
    DeviceTensor *outs[2] = {&w->weight, &w->scale};
    const int64_t sizes[2] = {wb, sb};
    for (int i = 0; i < 2; ++i) {
      outs[i]->desc = onnxl_amd_tensor{};
      outs[i]->desc.data = outs[i]->ptr;
      outs[i]->desc.location = ONNXL_AMD_DEVICE;
      outs[i]->desc.size_bytes = sizes[i];
    }
    w->zero_point.desc = Absent();
    const onnxl_amd_tensor qb = q.T("B"), qc = q.T("s_channel"), qg = q.T("s_group");
    const int rc = onnxl_amd_prepare_qqq(q.k, q.n, q.group, q.bits, &qb, &qc, &qg, a.data_type, &w->weight.desc,
                                         &w->scale.desc, nullptr);
    if (rc == ONNXL_AMD_UNSUPPORTED) return nullptr;
    Check(rc);
    Check(onnxl_amd_synchronize(nullptr));
    w->fused = true;
    return w;
  }

  std::shared_ptr<Prepared> PrepareWeight(rt::RuntimeContext &ctx) const {
    const auto value = ctx.values().find(node_->input(1));
    if (value == ctx.values().end() || value->second.kind != rt::RuntimeValue::Kind::kEncoded)
      throw std::invalid_argument("Dequantize requires an EncodedValueProto input.");
    BnbCheckpoint b;
    if (ExportBitsAndBytes(value->second, ctx.struct_type_catalogue(), b)) return PrepareBitsAndBytes(ctx, b);
    QqqCheckpoint q;
    if (ExportQqq(value->second, ctx.struct_type_catalogue(), q)) {
      auto w = PrepareQqq(ctx, q);
      return w ? w : DenseOther(ctx, value->second);
    }
    VptqCheckpoint v;
    if (ExportVptq(value->second, ctx.struct_type_catalogue(), v)) {  // codebook lookups: dense
      auto w = std::make_shared<Prepared>();
      DenseFromDevice(In(0, ctx), v.config.out_features, v.config.in_features,
                      [&](onnxl_amd_tensor *y) { return v.Decode(y); }, *w);
      return w;
    }
    GptqFp8Checkpoint f;
    if (ExportGptqFp8(value->second, ctx.struct_type_catalogue(), f)) {  // a division per weight: dense
      auto w = std::make_shared<Prepared>();
      DenseFromDevice(In(0, ctx), f.n, f.k, [&](onnxl_amd_tensor *y) { return f.Decode(y); }, *w);
      return w;
    }
    Exl3Checkpoint x3;
    if (ExportExl3(value->second, ctx.struct_type_catalogue(), x3)) {  // [k, n] = [N, K]: dense
      auto w = std::make_shared<Prepared>();
      DenseFromDevice(In(0, ctx), x3.k, x3.n, [&](onnxl_amd_tensor *y) { return x3.Decode(y); }, *w);
      return w;
    }
    MxCheckpoint mx;
    if (ExportMx(value->second, ctx.struct_type_catalogue(), mx)) {  // [rows, cols] = [N, K]: dense
      auto w = std::make_shared<Prepared>();
      DenseFromDevice(In(0, ctx), mx.rows, mx.cols, [&](onnxl_amd_tensor *y) { return mx.Decode(y); }, *w);
      return w;
    }
    Checkpoint c;
    if (!ExportCheckpoint(value->second, ctx.struct_type_catalogue(), c)) return DenseOther(ctx, value->second);
    auto w = std::make_shared<Prepared>();
    int64_t wb = 0, sb = 0, zb = 0;
    Check(c.PreparedSizes(&wb, &sb, &zb));
    w->weight.Allocate(wb);
    w->scale.Allocate(sb);
    w->zero_point.Allocate(zb);
    const int64_t sizes[3] = {wb, sb, zb};
    DeviceTensor *outs[3] = {&w->weight, &w->scale, &w->zero_point};
    for (int i = 0; i < 3; ++i) {
      outs[i]->desc = onnxl_amd_tensor{};
      outs[i]->desc.data = outs[i]->ptr;
      outs[i]->desc.location = ONNXL_AMD_DEVICE;
      outs[i]->desc.size_bytes = sizes[i];
    }
    const int rc = c.Prepare(&w->weight.desc, &w->scale.desc, &w->zero_point.desc);
    if (rc != ONNXL_AMD_UNSUPPORTED) {
      Check(rc);
      Check(onnxl_amd_synchronize(nullptr));
      w->fused = true;
      if (In(0, ctx).data_type == kBfloat16 && w->scale.desc.data_type == kFloat16) WidenScales(w->scale);
      return w;
    }
    DenseFromDevice(In(0, ctx), c.N, c.K, [&](onnxl_amd_tensor *y) { return c.Decode(y); }, *w);
    return w;
  }

  // A weight [N, K] decoded on the GPU in the activations' dtype by `decode`
  // into device memory and transposed to [K, N] there; once per weight, with
  // no host copy.
  template <typename Decode>
  static void DenseFromDevice(const onnxl_amd_tensor &a, int64_t N, int64_t K, Decode &&decode, Prepared &w) {
    const int64_t bytes = N * K * 2;
    DeviceTensor nk;  // the decoded [N, K], freed once transposed
    nk.Allocate(bytes);
    nk.desc.data_type = a.data_type;
    nk.desc.rank = 2;
    nk.desc.dims[0] = N;
    nk.desc.dims[1] = K;
    nk.desc.data = nk.ptr;
    nk.desc.size_bytes = bytes;
    nk.desc.location = ONNXL_AMD_DEVICE;
    Check(decode(&nk.desc));
    TransposeOnDevice(nk.desc, w);
  }

  // w.dense_t = the [K, N] transpose of the device tensor nk [N, K], on the
  // GPU (onnxl_amd_transpose_2d), complete on return.
  static void TransposeOnDevice(const onnxl_amd_tensor &nk, Prepared &w) {
    w.dense_t.Allocate(nk.size_bytes);
    w.dense_t.desc = nk;
    w.dense_t.desc.dims[0] = nk.dims[1];
    w.dense_t.desc.dims[1] = nk.dims[0];
    w.dense_t.desc.data = w.dense_t.ptr;
    Check(onnxl_amd_transpose_2d(&nk, &w.dense_t.desc, nullptr));
    Check(onnxl_amd_synchronize(nullptr));
  }

  // Any other encoding: the reference's decode in A's dtype (materializing a
  // shared-parameter reference first, as kernel_dequantize.cc:28-36 does),
  // transposed to [K, N] and uploaded once.
  std::shared_ptr<Prepared> DenseOther(rt::RuntimeContext &ctx, const rt::RuntimeValue &value) const {
    const onnxl_amd_tensor a = In(0, ctx);
    const auto &catalogue = ctx.struct_type_catalogue();
    const rt::Tensor nk = value.Encoded().has_parameter_ref()
                              ? rt::DequantizeTensor(rt::MaterializeQuantizedValue(value, catalogue), {}, nullptr,
                                                     a.data_type)
                              : rt::DequantizeTensor(value.Encoded(), catalogue, nullptr, a.data_type);
    if (nk.shape.size() != 2 || nk.data_type != a.data_type)
      throw std::invalid_argument("mi355x: DequantizeEncodedMatMul takes a 2-D encoded weight.");
    auto w = std::make_shared<Prepared>();
    const auto up = UploadToHbm(nk);  // [N, K], transposed on the GPU
    TransposeOnDevice(up->desc, *w);
    return w;
  }

  std::shared_ptr<Prepared> weight_;
};

// ---------------------------------------------------------------------------
// Registration.

rt::NodeKernelFn BuiltinFactory(const std::string &key) {
  const auto &table = rt::KernelDispatchTable();
  const auto it = table.find(key);
  return it == table.end() ? rt::NodeKernelFn{} : it->second;
}

template <typename K> void Register(const char *domain, const char *op_type) {
  const std::string key = std::string(*domain ? domain : "ai.onnx") + ":" + op_type;
  rt::NodeKernelFn builtin = BuiltinFactory(key);  // captured before the override
  rt::RegisterKernelFn(
      domain, op_type, sym::Device::kCPU,
      [builtin](const NodeProto &node, rt::RuntimeContext &ctx,
                const rt::KernelContext &kc) -> std::unique_ptr<rt::KernelBase> {
        std::unique_ptr<rt::KernelBase> fallback = builtin ? builtin(node, ctx, kc) : nullptr;
        auto k = std::make_unique<K>(kc, std::move(fallback));
        k->set_node(node);
        return k;
      },
      /*overwrite=*/true);
}

std::once_flag g_registered;

}  // namespace mi355x

// Registers the MI355X kernels over the built-in CPU kernels of the same
// operators (and the two fused nodes).  Call once, after the built-ins are
// registered; later calls do nothing.  Returns the library version string.
const char *RegisterMi355xKernelFunctions(int device_ordinal = 0) {
  using namespace mi355x;
  std::call_once(g_registered, [device_ordinal] {
    Check(onnxl_amd_init(device_ordinal));
    Register<Mi355xMatMulInteger>("", "MatMulInteger");
    Register<Mi355xQLinearMatMul>("", "QLinearMatMul");
    Register<Mi355xDequantizeLinear>("", "DequantizeLinear");
    Register<Mi355xQuantizeLinear>("", "QuantizeLinear");
    Register<Mi355xDynamicQuantizeLinear>("", "DynamicQuantizeLinear");
    Register<Mi355xMatMul>("", "MatMul");
    Register<Mi355xCast>("", "Cast");
    Register<Mi355xConvInteger>("", "ConvInteger");
    Register<Mi355xQLinearConv>("", "QLinearConv");
    Register<Mi355xDequantizePacked>("", "DequantizePacked");
    Register<Mi355xGroupedMatMul>("", "GroupedMatMul");
    Register<Mi355xMatMulNBits>("com.microsoft", "MatMulNBits");
    Register<Mi355xDequantizeLinearMatMul>(kFusedDomain, "DequantizeLinearMatMul");
    Register<Mi355xDequantizePackedMatMul>(kFusedDomain, "DequantizePackedMatMul");
    Register<Mi355xDequantize>("ai.rt", "Dequantize");
    Register<Mi355xDequantizeEncodedMatMul>(kFusedDomain, "DequantizeEncodedMatMul");
    Register<Mi355xDequantizeLinearGroupedMatMul>(kFusedDomain, "DequantizeLinearGroupedMatMul");
  });
  return onnxl_amd_version();
}

// Releases the library's device buffers; call after every session has ended.
void ShutdownMi355xKernelFunctions() { mi355x::Check(onnxl_amd_shutdown()); }
