// Host-side helpers shared by the C ABI: status/exception mapping, dtype
// table, tensor-descriptor accessors, HIP error checks and the per-device
// workspace.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/onnxl_amd.h"

namespace onnxl_amd {

// ONNX TensorProto.DataType codes used on this path.
enum DType : int32_t {
  kFloat = 1, kUint8 = 2, kInt8 = 3, kUint16 = 4, kInt16 = 5, kInt32 = 6, kInt64 = 7,
  kFloat16 = 10, kDouble = 11, kBfloat16 = 16, kFloat8E4M3FN = 17, kFloat8E4M3FNUZ = 18, kFloat8E5M2 = 19,
  kFloat8E5M2FNUZ = 20, kUint4 = 21, kInt4 = 22, kFloat4E2M1 = 23, kFloat8E8M0 = 24, kUint2 = 25, kInt2 = 26,
  kFloat6E2M3 = 27, kFloat6E3M2 = 28
};

// Validation failure, mapped to ONNXL_AMD_INVALID_ARGUMENT (the reference
// throws std::invalid_argument prefixed "[onnx-light] ").
struct InvalidArgument : std::runtime_error {
  explicit InvalidArgument(const std::string &m) : std::runtime_error("[onnx-light] " + m) {}
};
// Valid for the reference, not implemented on this GPU path.
struct Unsupported : std::runtime_error {
  explicit Unsupported(const std::string &m) : std::runtime_error("[onnx-light-amd] " + m) {}
};
struct DeviceError : std::runtime_error {
  explicit DeviceError(const std::string &m) : std::runtime_error("[onnx-light-amd] " + m) {}
};
struct NotInitialized : std::runtime_error {
  NotInitialized() : std::runtime_error("[onnx-light-amd] onnxl_amd_init has not been called") {}
};

template <typename... Args> std::string Cat(const Args &...args) {
  std::ostringstream os;
  (os << ... << args);
  return os.str();
}

#define OLA_ENFORCE(cond, ...)                                                                  \
  do {                                                                                          \
    if (!(cond)) throw ::onnxl_amd::InvalidArgument(::onnxl_amd::Cat(__VA_ARGS__));             \
  } while (0)

#define OLA_HIP(expr)                                                                           \
  do {                                                                                          \
    hipError_t e_ = (expr);                                                                     \
    if (e_ != hipSuccess)                                                                       \
      throw ::onnxl_amd::DeviceError(::onnxl_amd::Cat(#expr, " failed: ", hipGetErrorString(e_))); \
  } while (0)

using Shape = std::vector<int64_t>;

// Absent optional input: NULL or rank -1 (the reference's empty Tensor{}).
inline bool Absent(const onnxl_amd_tensor *t) { return t == nullptr || t->rank < 0; }

inline Shape ShapeOf(const onnxl_amd_tensor &t) {
  return Shape(t.dims, t.dims + (t.rank > 0 ? t.rank : 0));
}

inline int64_t NumElements(const Shape &s) {
  int64_t n = 1;
  for (int64_t d : s) n *= d;
  return n;
}
inline int64_t NumElements(const onnxl_amd_tensor &t) { return NumElements(ShapeOf(t)); }

// Bytes per element; 4-bit types return 0 (use PackedBytes).
inline int64_t ElementSize(int32_t dt) {
  switch (dt) {
  case kUint8: case kInt8: case kFloat8E4M3FN: case kFloat8E4M3FNUZ: case kFloat8E5M2: case kFloat8E5M2FNUZ:
  case kFloat8E8M0:
    return 1;
  case kUint16: case kInt16: case kFloat16: case kBfloat16: return 2;
  case kFloat: case kInt32: return 4;
  case kInt64: case kDouble: return 8;
  default: return 0;
  }
}
inline bool IsFourBit(int32_t dt) { return dt == kInt4 || dt == kUint4; }
// Bits per element of the packed sub-byte types (0 for byte-sized ones).
inline int SubByteBits(int32_t dt) {
  switch (dt) {
  case kInt4: case kUint4: case kFloat4E2M1: return 4;
  case kInt2: case kUint2: return 2;
  case kFloat6E2M3: case kFloat6E3M2: return 6;
  default: return 0;
  }
}
// Payload bytes of n elements (sub-byte types: ceil(n * bits / 8),
// core/runtime/memory/simple_tensor.h:949).
inline int64_t PackedBytes(int32_t dt, int64_t n) {
  const int bits = SubByteBits(dt);
  return bits ? (n * bits + 7) / 8 : n * ElementSize(dt);
}

inline const char *DTypeName(int32_t dt) {
  switch (dt) {
  case kFloat: return "FLOAT"; case kUint8: return "UINT8"; case kInt8: return "INT8";
  case kUint16: return "UINT16"; case kInt16: return "INT16"; case kInt32: return "INT32";
  case kFloat16: return "FLOAT16"; case kBfloat16: return "BFLOAT16";
  case kFloat8E4M3FN: return "FLOAT8E4M3FN"; case kUint4: return "UINT4"; case kInt4: return "INT4";
  default: return "?";
  }
}

// ---------------------------------------------------------------------------
// MatMul shape rules, km/matmul_shape_utils.h:24-106.

struct MatMulPlan {
  int64_t M = 0, K = 0, N = 0;
  Shape out_shape;   // as the reference reports it (promoted dims dropped)
  Shape out_prefix;  // broadcast batch dims
  Shape a_bstride;   // element stride of A per out_prefix dim (0 = broadcast)
  Shape b_bstride;
  int64_t batch = 1; // product of out_prefix
  int64_t a_mats = 1, b_mats = 1; // distinct A / B matrices
};

// Throws InvalidArgument with the kernel's own message suffixes.
MatMulPlan MakeMatMulPlan(const Shape &a, const Shape &b, const char *kname, const char *rank0_msg,
                          const char *inner_msg, const char *bcast_msg);

// ---------------------------------------------------------------------------
// Per-device state: the workspace every launcher borrows from.

class Workspace {
public:
  // Returns device memory of at least `bytes`, 256-byte aligned.  Growing it
  // allocates a larger buffer and retires the old one without freeing it:
  // launches already queued, and HIP graphs captured earlier, keep valid
  // pointers.  Retired buffers are freed by Release().
  void *Get(size_t bytes);
  // Zero-initialised counters that kernels leave at zero when they finish
  // (grown the same way).
  unsigned *Counters(size_t count);
  void Release();

private:
  void *ptr_ = nullptr;
  size_t cap_ = 0;
  unsigned *counters_ = nullptr;
  size_t counters_cap_ = 0;
  std::vector<void *> retired_;
};

struct DeviceContext {
  int device = -1;
  Workspace ws;
  int num_cus = 0;
};

DeviceContext &Ctx();  // throws NotInitialized when onnxl_amd_init was not called
bool Initialized();

// Bump allocator over the workspace for the scratch pieces of one call.
class Scratch {
public:
  explicit Scratch(size_t total) : base_(static_cast<char *>(Ctx().ws.Get(total))), cap_(total) {}
  void *Take(size_t bytes) {
    const size_t at = (off_ + 255) & ~size_t(255);
    if (at + bytes > cap_) throw DeviceError("internal: scratch overflow");
    off_ = at + bytes;
    return base_ + at;
  }
  static size_t Round(size_t b) { return (b + 255) & ~size_t(255); }

private:
  char *base_;
  size_t cap_;
  size_t off_ = 0;
};

}  // namespace onnxl_amd
