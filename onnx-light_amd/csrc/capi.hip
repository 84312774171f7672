// C ABI of the gfx950 quantized-matmul kernels (include/onnxl_amd.h).
//
// Host side of every entry point: the reference kernel's validation (same
// checks, order and message text, cited per function), staging of host
// payloads, the zero-point / scale arithmetic that the reference does on the
// host, and the kernel launch.  No computation falls back to the CPU: a shape
// or dtype without a GPU kernel returns ONNXL_AMD_UNSUPPORTED.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <limits>
#include <memory>
#include <mutex>

#include "checkpoint_layout.hpp"
#include "common.hpp"
#include "kernels.hpp"

// Scratch of onnxl_amd_dequantize_linear_matmul_noalloc: a fixed array that
// every GPU the library runs on holds for the life of the process (each GPU
// its own copy, at its own address).  The first 64 KiB hold the split-K
// counters of the int4 GEMV (zeroed once per device at set-up; every GEMV
// launch returns the counters it used to zero), the rest holds partial sums
// or a dequantised weight.  Host code never passes `scratch` itself to a
// kernel: it is a host-side stand-in; the device address comes from
// hipGetSymbolAddress (onnxl_amd::NoAllocScratch).
static __device__ __align__(256) unsigned char scratch[8u << 20];

namespace onnxl_amd {

// ---------------------------------------------------------------------------
// Library state.

namespace {
DeviceContext g_ctx;
std::atomic<bool> g_init{false};
std::mutex g_mu;  // serialises entry points: one workspace per device
thread_local std::string g_last_error;

constexpr size_t kNoAllocBytes = sizeof(scratch);
constexpr size_t kNoAllocCounterBytes = size_t(64) << 10;
constexpr size_t kNoAllocDataBytes = kNoAllocBytes - kNoAllocCounterBytes;
constexpr int kMaxDevices = 64;
void *g_noalloc_ptr[kMaxDevices] = {};  // device address of `scratch` per device (under g_mu)

__global__ __launch_bounds__(256) void ZeroWordsKernel(unsigned *p, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Once per device, with that device current: looks up the device address of
// `scratch` and clears its counters (with a fill kernel, then waits).
void SetUpNoAllocScratch(int device) {
  OLA_ENFORCE(device >= 0 && device < kMaxDevices, "onnxl_amd_init: device ", device, " above ", kMaxDevices - 1);
  if (g_noalloc_ptr[device] != nullptr) return;
  void *ptr = nullptr;
  OLA_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  OLA_ENFORCE(ptr != nullptr, "onnxl_amd_init: no device address for the no-allocation scratch");
  const size_t words = kNoAllocCounterBytes / sizeof(unsigned);
  hipLaunchKernelGGL(ZeroWordsKernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, nullptr,
                     static_cast<unsigned *>(ptr), words);
  OLA_HIP(hipGetLastError());
  OLA_HIP(hipDeviceSynchronize());
  g_noalloc_ptr[device] = ptr;
}
}  // namespace

bool Initialized() { return g_init.load(); }

DeviceContext &Ctx() {
  if (!g_init.load()) throw NotInitialized();
  return g_ctx;
}

namespace {
// The current device's address of `scratch` (set up by onnxl_amd_init).
void *NoAllocScratch() {
  const int dev = Ctx().device;
  void *ptr = dev >= 0 && dev < kMaxDevices ? g_noalloc_ptr[dev] : nullptr;
  if (ptr == nullptr) throw DeviceError("internal: the no-allocation scratch was not set up for this device");
  return ptr;
}
}  // namespace

void *Workspace::Get(size_t bytes) {
  if (bytes <= cap_ && ptr_ != nullptr) return ptr_;
  size_t want = std::max<size_t>(bytes, size_t(1) << 20);
  want = std::max(want, cap_ * 2);
  void *fresh = nullptr;
  OLA_HIP(hipMalloc(&fresh, want));
  if (ptr_ != nullptr) retired_.push_back(ptr_);
  ptr_ = fresh;
  cap_ = want;
  return ptr_;
}

unsigned *Workspace::Counters(size_t count) {
  if (count <= counters_cap_ && counters_ != nullptr) return counters_;
  size_t want = std::max<size_t>(count, 4096);
  want = std::max(want, counters_cap_ * 2);
  unsigned *fresh = nullptr;
  OLA_HIP(hipMalloc(&fresh, want * sizeof(unsigned)));
  const hipError_t err = hipMemset(fresh, 0, want * sizeof(unsigned));
  if (err != hipSuccess) {
    (void)hipFree(fresh);
    OLA_HIP(err);
  }
  if (counters_ != nullptr) retired_.push_back(counters_);
  counters_ = fresh;
  counters_cap_ = want;
  return counters_;
}

void Workspace::Release() {
  if (ptr_) (void)hipFree(ptr_);
  if (counters_) (void)hipFree(counters_);
  for (void *q : retired_) (void)hipFree(q);
  retired_.clear();
  ptr_ = nullptr;
  counters_ = nullptr;
  cap_ = counters_cap_ = 0;
}

// ---------------------------------------------------------------------------
// MatMul shape rules, km/matmul_shape_utils.h:24-106.

MatMulPlan MakeMatMulPlan(const Shape &a, const Shape &b, const char *kname, const char *rank0_msg,
                          const char *inner_msg, const char *bcast_msg) {
  OLA_ENFORCE(!a.empty() && !b.empty(), kname, rank0_msg);
  const Shape a2 = a.size() == 1 ? Shape{1, a[0]} : a;
  const Shape b2 = b.size() == 1 ? Shape{b[0], 1} : b;
  MatMulPlan p;
  p.M = a2[a2.size() - 2];
  p.K = a2[a2.size() - 1];
  p.N = b2[b2.size() - 1];
  OLA_ENFORCE(p.K == b2[b2.size() - 2], kname, inner_msg);
  const size_t ap = a2.size() - 2, bp = b2.size() - 2;
  const size_t rank = std::max(ap, bp);
  Shape as(a2.size()), bs(b2.size());
  as.back() = 1;
  for (size_t i = a2.size() - 1; i-- > 0;) as[i] = as[i + 1] * a2[i + 1];
  bs.back() = 1;
  for (size_t i = b2.size() - 1; i-- > 0;) bs[i] = bs[i + 1] * b2[i + 1];
  for (size_t i = 0; i < rank; ++i) {
    const bool ha = i + ap >= rank, hb = i + bp >= rank;
    const int64_t da = ha ? a2[i - (rank - ap)] : 1;
    const int64_t db = hb ? b2[i - (rank - bp)] : 1;
    int64_t d;
    if (da == db || da == 1) {
      d = db;
    } else if (db == 1) {
      d = da;
    } else {
      throw InvalidArgument(Cat(kname, bcast_msg));
    }
    p.out_prefix.push_back(d);
    p.a_bstride.push_back(ha && da != 1 ? as[i - (rank - ap)] : 0);
    p.b_bstride.push_back(hb && db != 1 ? bs[i - (rank - bp)] : 0);
    p.batch *= d;
  }
  for (size_t i = 0; i < ap; ++i) p.a_mats *= a2[i];
  for (size_t i = 0; i < bp; ++i) p.b_mats *= b2[i];
  p.out_shape = p.out_prefix;
  if (a.size() != 1) p.out_shape.push_back(p.M);
  if (b.size() != 1) p.out_shape.push_back(p.N);
  return p;
}

namespace {

BatchMap ToBatchMap(const MatMulPlan &p) {
  BatchMap m;
  // Leading broadcast dims that are 1 everywhere carry no offset; drop dims
  // of size 1 to fit kMaxBatchRank.
  for (size_t i = 0; i < p.out_prefix.size(); ++i) {
    if (p.out_prefix[i] == 1) continue;
    if (m.rank == kMaxBatchRank) throw Unsupported("MatMul batch rank above 6 (non-unit dims)");
    m.dims[m.rank] = p.out_prefix[i];
    m.a_stride[m.rank] = p.a_bstride[i];
    m.b_stride[m.rank] = p.b_bstride[i];
    ++m.rank;
  }
  return m;
}

// ---------------------------------------------------------------------------
// Descriptor helpers.

void CheckDescriptor(const onnxl_amd_tensor *t, const char *what, bool allow_tiled = false) {
  if (t == nullptr) return;
  OLA_ENFORCE(t->rank <= ONNXL_AMD_MAX_RANK, what, ": rank above ", ONNXL_AMD_MAX_RANK);
  if (t->rank < 0) return;
  for (int i = 0; i < t->rank; ++i) OLA_ENFORCE(t->dims[i] >= 0, what, ": negative dimension");
  OLA_ENFORCE(t->location == ONNXL_AMD_DEVICE || t->location == ONNXL_AMD_HOST, what,
              ": unknown location");
  const bool tiled = t->layout == ONNXL_AMD_LAYOUT_TILED_INT4;
  OLA_ENFORCE(t->layout == ONNXL_AMD_LAYOUT_ONNX || (allow_tiled && tiled), what, ": layout ", t->layout,
              " is not accepted here");
  if (tiled)
    OLA_ENFORCE(IsFourBit(t->data_type) && t->rank == 2, what,
                ": the tiled layout holds 2-D INT4 / UINT4 weights only");
  const int64_t need = tiled ? TiledInt4Bytes(t->dims[0], t->dims[1])
                             : PackedBytes(t->data_type, NumElements(*t));
  OLA_ENFORCE(t->size_bytes >= need, what, ": payload of ", t->size_bytes,
              " bytes is smaller than its shape needs (", need, ")");
  OLA_ENFORCE(need == 0 || t->data != nullptr, what, ": null payload");
}

// Copies `bytes` of element data from a descriptor (host or device) to host.
void ReadBytes(const onnxl_amd_tensor &t, int64_t offset, void *dst, size_t bytes) {
  const char *src = static_cast<const char *>(t.data) + offset;
  if (t.location == ONNXL_AMD_HOST) {
    std::memcpy(dst, src, bytes);
  } else {
    OLA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  }
}

// One call's device view of its tensors: host payloads staged into scratch.
class Staging {
public:
  Staging(hipStream_t s, size_t extra_scratch, std::initializer_list<const onnxl_amd_tensor *> in,
          std::initializer_list<onnxl_amd_tensor *> out)
      : stream_(s) {
    size_t total = Scratch::Round(extra_scratch) + 256;
    for (auto *t : in)
      if (t && t->rank >= 0 && t->location == ONNXL_AMD_HOST) total += Scratch::Round(t->size_bytes) + 256;
    for (auto *t : out)
      if (t && t->location == ONNXL_AMD_HOST) total += Scratch::Round(t->size_bytes) + 256;
    scratch_ = std::make_unique<Scratch>(total);
    extra_ = extra_scratch ? scratch_->Take(extra_scratch) : nullptr;
    for (auto *t : in) {
      if (t && t->rank >= 0 && t->location == ONNXL_AMD_HOST && t->size_bytes > 0) {
        void *d = scratch_->Take(t->size_bytes);
        OLA_HIP(hipMemcpyAsync(d, t->data, t->size_bytes, hipMemcpyHostToDevice, s));
        dev_.push_back({t, d});
      }
    }
    for (auto *t : out) {
      if (t && t->location == ONNXL_AMD_HOST && t->size_bytes > 0) {
        void *d = scratch_->Take(t->size_bytes);
        dev_.push_back({t, d});
        outs_.push_back({t, d});
      }
    }
  }
  const void *In(const onnxl_amd_tensor *t) const {
    if (t == nullptr || t->rank < 0) return nullptr;
    for (auto &e : dev_)
      if (e.first == t) return e.second;
    return t->data;
  }
  void *Out(onnxl_amd_tensor *t) const { return const_cast<void *>(In(t)); }
  void *Extra() const { return extra_; }
  // Copies host outputs back and waits when any payload was on the host.
  void Finish() {
    for (auto &e : outs_)
      OLA_HIP(hipMemcpyAsync(e.first->data, e.second, e.first->size_bytes, hipMemcpyDeviceToHost,
                             stream_));
    if (!dev_.empty()) OLA_HIP(hipStreamSynchronize(stream_));
    OLA_HIP(hipGetLastError());
  }

private:
  hipStream_t stream_;
  std::unique_ptr<Scratch> scratch_;
  void *extra_ = nullptr;
  std::vector<std::pair<const onnxl_amd_tensor *, void *>> dev_;
  std::vector<std::pair<onnxl_amd_tensor *, void *>> outs_;
};

bool IsInt8OrUint8(int32_t dt) { return dt == kInt8 || dt == kUint8; }

// Pinned staging for ReadLeadingBytes: 8 slots of 8 bytes, allocated on first
// use and freed by onnxl_amd_shutdown.  Every entry point runs under g_mu, so
// one buffer serves all threads.
uint8_t *g_pinned = nullptr;

// The first bytes[i] (<= 8) bytes of each descriptor ts[i] (null: skipped)
// into host[i]: host payloads directly, device ones by copies on `stream`
// into pinned memory with one synchronisation of that stream for all of them
// (not one blocking copy each, which also waits for the whole device).  A
// payload shorter than bytes[i] (an empty scalar the caller's checks reject
// next) is not read: host[i] stays zero.  Caller holds g_mu.
void ReadLeadingBytes(hipStream_t stream, int n, const onnxl_amd_tensor *const *ts, const size_t *bytes,
                      uint8_t (*host)[8]) {
  bool any_device = false;
  auto readable = [&](int i) { return ts[i] && ts[i]->data && (size_t)ts[i]->size_bytes >= bytes[i]; };
  for (int i = 0; i < n; ++i) {
    std::memset(host[i], 0, 8);
    if (!readable(i)) continue;
    if (ts[i]->location == ONNXL_AMD_HOST) {
      std::memcpy(host[i], ts[i]->data, bytes[i]);
      continue;
    }
    if (!g_pinned) OLA_HIP(hipHostMalloc(reinterpret_cast<void **>(&g_pinned), 64, hipHostMallocDefault));
    OLA_HIP(hipMemcpyAsync(g_pinned + 8 * i, ts[i]->data, bytes[i], hipMemcpyDeviceToHost, stream));
    any_device = true;
  }
  if (!any_device) return;
  OLA_HIP(hipStreamSynchronize(stream));
  for (int i = 0; i < n; ++i)
    if (readable(i) && ts[i]->location != ONNXL_AMD_HOST) std::memcpy(host[i], g_pinned + 8 * i, bytes[i]);
}

// Whether `stream` is being captured into a HIP graph: it cannot be
// synchronised then, so device-resident scalars are left for the kernels to
// read.
bool Capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st == hipStreamCaptureStatusActive;
}

bool OnDevice(const onnxl_amd_tensor *t) { return t && t->data && t->location != ONNXL_AMD_HOST; }

// The convolutions read their scalars on the host (they shape the padding
// and select the kernel): under graph capture those must be host-resident.
void RejectCapturedDeviceScalars(hipStream_t stream, std::initializer_list<const onnxl_amd_tensor *> ts,
                                 const char *op) {
  bool dev = false;
  for (auto *t : ts) dev = dev || OnDevice(t);
  if (dev && Capturing(stream))
    throw Unsupported(Cat(op, ": device-resident scalar zero points and scales cannot be read while the stream is "
                              "captured into a graph; pass them as host scalars."));
}

// An INT8 / UINT8 element's value from its byte.
int32_t ByteInt(const onnxl_amd_tensor &t, uint8_t b) {
  return t.data_type == kInt8 ? (int32_t)(int8_t)b : (int32_t)b;
}

// Two optional scalar zero points (null: absent, 0) read together.
void ReadTwoZeroPoints(hipStream_t stream, const onnxl_amd_tensor *z0, const onnxl_amd_tensor *z1, int32_t &v0,
                       int32_t &v1) {
  const onnxl_amd_tensor *ts[2] = {z0, z1};
  const size_t one[2] = {1, 1};
  uint8_t host[2][8] = {};
  ReadLeadingBytes(stream, 2, ts, one, host);
  v0 = z0 ? ByteInt(*z0, host[0][0]) : 0;
  v1 = z1 ? ByteInt(*z1, host[1][0]) : 0;
}

float HalfBitsToFloat(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  uint32_t f;
  if (exp == 0x1f) {
    f = sign | 0x7f800000u | (man << 13);
  } else if (exp == 0) {
    float v = std::ldexp((float)man, -24);
    return sign ? -v : v;
  } else {
    f = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  std::memcpy(&out, &f, 4);
  return out;
}

// ---------------------------------------------------------------------------
// MatMulInteger, km/kernel_matmul_integer.cc.

constexpr const char *kMmiName = "kernel::MatMulInteger";

// ZeroPointCount, km/kernel_matmul_integer.cc:40-57.
int64_t ZeroPointCount(const onnxl_amd_tensor *t, int32_t expected_dtype, int64_t expected_size,
                       const char *name) {
  if (Absent(t) || (t->rank == 0 && t->size_bytes == 0)) return 1;
  OLA_ENFORCE(t->data_type == expected_dtype, kMmiName, ": '", name,
              "' dtype must match its data input.");
  OLA_ENFORCE(t->rank <= 1, kMmiName, ": '", name, "' must be a scalar or a 1-D tensor.");
  const int64_t numel = NumElements(*t);
  OLA_ENFORCE(numel == 1 || numel == expected_size, kMmiName, ": '", name,
              "' must be a scalar, a one-element 1-D tensor, or a 1-D tensor whose size matches "
              "the corresponding matrix dimension.");
  return numel;
}

int MatMulInteger(const onnxl_amd_tensor *a, const onnxl_amd_tensor *b,
                  const onnxl_amd_tensor *a_zp, const onnxl_amd_tensor *b_zp,
                  onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(a && b && y, kMmiName, ": A, B and the output are required.");
  CheckDescriptor(a, "A");
  CheckDescriptor(b, "B");
  CheckDescriptor(a_zp, "a_zero_point");
  CheckDescriptor(b_zp, "b_zero_point");
  CheckDescriptor(y, "Y");
  // ComputeMatMulInteger, :178-208
  OLA_ENFORCE(IsInt8OrUint8(a->data_type), kMmiName, ": A must be INT8 or UINT8.");
  OLA_ENFORCE(IsInt8OrUint8(b->data_type), kMmiName, ": B must be INT8 or UINT8.");
  OLA_ENFORCE(y->data_type == kInt32, kMmiName, ": output dtype must be INT32.");
  const MatMulPlan plan = MakeMatMulPlan(
      ShapeOf(*a), ShapeOf(*b), kMmiName, ": rank-0 inputs are not accepted.",
      ": incompatible inner dimensions.", ": inputs are not broadcast-compatible on batch dimensions.");
  OLA_ENFORCE(ShapeOf(*y) == plan.out_shape, kMmiName, ": preallocated output has invalid shape.");
  OLA_ENFORCE(y->size_bytes == NumElements(plan.out_shape) * 4, kMmiName,
              ": preallocated output buffer size does not match its shape.");
  const int64_t a_count = ZeroPointCount(a_zp, a->data_type, plan.M, "a_zero_point");
  const int64_t b_count = ZeroPointCount(b_zp, b->data_type, plan.N, "b_zero_point");

  IGemmParams p{};
  p.M = plan.M;
  p.N = plan.N;
  p.K = plan.K;
  p.batch = plan.batch;
  p.bm = ToBatchMap(plan);
  p.a_u8 = a->data_type == kUint8;
  p.b_u8 = b->data_type == kUint8;
  const int32_t ca = p.a_u8 ? 128 : 0, cb = p.b_u8 ? 128 : 0;
  const bool a_present = !(Absent(a_zp) || (a_zp->rank == 0 && a_zp->size_bytes == 0));
  const bool b_present = !(Absent(b_zp) || (b_zp->rank == 0 && b_zp->size_bytes == 0));
  // The reference indexes per-row values only when more than one is given
  // (a_per_row = a_size > 1, :118-119).
  const bool a_vec = a_present && a_count > 1;
  const bool b_vec = b_present && b_count > 1;
  // Single zero points: read on the host, or under graph capture (no
  // synchronisation possible) left on the device for the kernels to read.
  const onnxl_amd_tensor *za_t = (a_present && !a_vec && a_count == 1) ? a_zp : nullptr;
  const onnxl_amd_tensor *zb_t = (b_present && !b_vec && b_count == 1) ? b_zp : nullptr;
  const bool in_place = Capturing(stream);
  const bool dev_za = in_place && OnDevice(za_t), dev_zb = in_place && OnDevice(zb_t);
  int32_t za = 0, zb = 0;
  ReadTwoZeroPoints(stream, dev_za ? nullptr : za_t, dev_zb ? nullptr : zb_t, za, zb);
  p.alpha_scalar = ca - za;
  p.beta_scalar = cb - zb;
  p.need_cb = a_vec || p.alpha_scalar != 0 || dev_za;
  p.need_ra = b_vec || p.beta_scalar != 0 || dev_zb;
  if (dev_za) p.dev.za = static_cast<const uint8_t *>(za_t->data);
  if (dev_zb) p.dev.zb = static_cast<const uint8_t *>(zb_t->data);
  p.epilogue = kEpiInt32;

  Staging st(stream, 0, {a, b, a_vec ? a_zp : nullptr, b_vec ? b_zp : nullptr}, {y});
  p.A = static_cast<const int8_t *>(st.In(a));
  p.B = static_cast<const int8_t *>(st.In(b));
  p.a_zp = a_vec ? static_cast<const uint8_t *>(st.In(a_zp)) : nullptr;
  p.b_zp = b_vec ? static_cast<const uint8_t *>(st.In(b_zp)) : nullptr;
  p.Y = st.Out(y);
  LaunchIGemm(p, stream);
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// QLinearMatMul, kq/kernel_qlinearmatmul.cc.

constexpr const char *kQlmName = "kernel::QLinearMatMul";

// QLinearMatMul's six scalars at once: the reference's checks in its order
// (:35-51), then one ReadLeadingBytes for all of them.
struct QlmScalars {
  int32_t za, zb, zy;
  float as, bs, ys;
};

// With `in_place`, device-resident ones are not read (their host slots stay
// 0): the kernels read them (QDevScalars).
QlmScalars QReadScalars(const onnxl_amd_tensor *a_zp, const onnxl_amd_tensor *b_zp, const onnxl_amd_tensor *y_zp,
                        const onnxl_amd_tensor *a_s, const onnxl_amd_tensor *b_s, const onnxl_amd_tensor *y_s,
                        hipStream_t stream, bool in_place) {
  const onnxl_amd_tensor *ts[6] = {a_zp, b_zp, y_zp, a_s, b_s, y_s};
  const char *names[6] = {"a_zero_point", "b_zero_point", "y_zero_point", "a_scale", "b_scale", "y_scale"};
  for (int i = 0; i < 6; ++i) {
    OLA_ENFORCE(NumElements(*ts[i]) == 1, kQlmName, ": '", names[i], "' must be a scalar.");
    if (i >= 3 && ts[i]->data_type != kFloat && ts[i]->data_type != kFloat16)
      throw InvalidArgument(Cat(kQlmName, ": '", names[i],
                                "' must be a FLOAT or FLOAT16 scalar for the reference kernel."));
  }
  const size_t bytes[6] = {1, 1, 1, ts[3]->data_type == kFloat ? 4u : 2u, ts[4]->data_type == kFloat ? 4u : 2u,
                           ts[5]->data_type == kFloat ? 4u : 2u};
  uint8_t host[6][8] = {};
  const onnxl_amd_tensor *read[6];
  for (int i = 0; i < 6; ++i) read[i] = in_place && OnDevice(ts[i]) ? nullptr : ts[i];
  ReadLeadingBytes(stream, 6, read, bytes, host);
  QlmScalars r{};
  int32_t *zs[3] = {&r.za, &r.zb, &r.zy};
  for (int i = 0; i < 3; ++i) *zs[i] = ByteInt(*ts[i], host[i][0]);
  float *fs[3] = {&r.as, &r.bs, &r.ys};
  for (int i = 3; i < 6; ++i) {
    if (ts[i]->data_type == kFloat) {
      std::memcpy(fs[i - 3], host[i], 4);
    } else {
      uint16_t h;
      std::memcpy(&h, host[i], 2);
      *fs[i - 3] = HalfBitsToFloat(h);
    }
  }
  return r;
}

int QLinearMatMul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *a_scale,
                  const onnxl_amd_tensor *a_zp, const onnxl_amd_tensor *b,
                  const onnxl_amd_tensor *b_scale, const onnxl_amd_tensor *b_zp,
                  const onnxl_amd_tensor *y_scale, const onnxl_amd_tensor *y_zp,
                  onnxl_amd_tensor *y, hipStream_t stream) {
  const onnxl_amd_tensor *req[] = {a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp, y};
  for (auto *t : req) OLA_ENFORCE(!Absent(t), kQlmName, ": all 8 inputs and the output are required.");
  const char *names[] = {"a", "a_scale", "a_zero_point", "b", "b_scale", "b_zero_point", "y_scale",
                         "y_zero_point", "y"};
  for (int i = 0; i < 9; ++i) CheckDescriptor(req[i], names[i]);
  // :225-227 (allocating overload), then :246-264
  OLA_ENFORCE(IsInt8OrUint8(a->data_type), kQlmName, ": a must be INT8 or UINT8.");
  OLA_ENFORCE(IsInt8OrUint8(b->data_type), kQlmName, ": b must be INT8 or UINT8.");
  OLA_ENFORCE(IsInt8OrUint8(y_zp->data_type), kQlmName, ": y_zero_point must be INT8 or UINT8.");
  OLA_ENFORCE(a_zp->data_type == a->data_type, kQlmName, ": a_zero_point dtype must match a.");
  OLA_ENFORCE(b_zp->data_type == b->data_type, kQlmName, ": b_zero_point dtype must match b.");
  OLA_ENFORCE(y->data_type == y_zp->data_type, kQlmName, ": output dtype must match y_zero_point.");
  const MatMulPlan plan = MakeMatMulPlan(
      ShapeOf(*a), ShapeOf(*b), kQlmName, ": rank-0 inputs are not accepted.",
      ": incompatible inner dimensions.", ": inputs are not broadcast-compatible on batch dimensions.");
  OLA_ENFORCE(ShapeOf(*y) == plan.out_shape, kQlmName, ": preallocated output has invalid shape.");
  OLA_ENFORCE(y->size_bytes >= NumElements(plan.out_shape), kQlmName,
              ": preallocated output buffer size does not match its shape.");
  // Under graph capture the device-resident scalars are read by the kernels
  // (no synchronisation); a zero y_scale among them is then not reported.
  const bool in_place = Capturing(stream);
  const QlmScalars sc = QReadScalars(a_zp, b_zp, y_zp, a_scale, b_scale, y_scale, stream, in_place);
  const int32_t za = sc.za, zb = sc.zb, zy = sc.zy;
  const float as = sc.as, bs = sc.bs, ys = sc.ys;
  const bool dev_za = in_place && OnDevice(a_zp), dev_zb = in_place && OnDevice(b_zp);
  const bool dev_zy = in_place && OnDevice(y_zp);
  const bool dev_scale = in_place && (OnDevice(a_scale) || OnDevice(b_scale) || OnDevice(y_scale));
  OLA_ENFORCE(dev_scale || ys != 0.0f, kQlmName, ": y_scale must be non-zero.");

  // The reference accumulates in int64 (:187-191); the MFMA path is exact
  // while |sum| < 2^31, guaranteed by K * max|a-za| * max|b-zb| < 2^31 (an
  // unread zero point counts with its dtype's widest span, 255).
  auto span = [](int32_t dt, int32_t z, bool unread) -> int64_t {
    if (unread) return 255;
    const int64_t lo = dt == kInt8 ? -128 : 0, hi = dt == kInt8 ? 127 : 255;
    return std::max<int64_t>(std::llabs(lo - z), std::llabs(hi - z));
  };
  const double bound =
      (double)plan.K * (double)span(a->data_type, za, dev_za) * (double)span(b->data_type, zb, dev_zb);
  const bool exact32 = bound < 2147483648.0;  // else the int64-accumulating kernel

  IGemmParams p{};
  p.M = plan.M;
  p.N = plan.N;
  p.K = plan.K;
  p.batch = plan.batch;
  p.bm = ToBatchMap(plan);
  p.a_u8 = a->data_type == kUint8;
  p.b_u8 = b->data_type == kUint8;
  p.alpha_scalar = (p.a_u8 ? 128 : 0) - za;
  p.beta_scalar = (p.b_u8 ? 128 : 0) - zb;
  p.need_cb = p.alpha_scalar != 0;
  p.need_ra = p.beta_scalar != 0;
  // combined scale in fp32, left to right (:156)
  const float ab = as * bs;
  p.cs = ab / ys;
  p.zy = (float)zy;
  p.y_signed = y->data_type == kInt8;
  p.qmin = p.y_signed ? -128.0f : 0.0f;
  p.qmax = p.y_signed ? 127.0f : 255.0f;
  p.epilogue = kEpiQuant8;
  if (dev_za) p.dev.za = static_cast<const uint8_t *>(a_zp->data);
  if (dev_zb) p.dev.zb = static_cast<const uint8_t *>(b_zp->data);
  if (dev_zy) p.dev.zy = static_cast<const uint8_t *>(y_zp->data);
  if (dev_scale) {  // the quotient on the device, host-resident scales as values
    p.dev.scales = 1;
    p.dev.as = OnDevice(a_scale) ? a_scale->data : nullptr;
    p.dev.bs = OnDevice(b_scale) ? b_scale->data : nullptr;
    p.dev.ys = OnDevice(y_scale) ? y_scale->data : nullptr;
    p.dev.as_f16 = a_scale->data_type == kFloat16;
    p.dev.bs_f16 = b_scale->data_type == kFloat16;
    p.dev.ys_f16 = y_scale->data_type == kFloat16;
    p.dev.as_h = as;
    p.dev.bs_h = bs;
    p.dev.ys_h = ys;
  }
  if (dev_za || dev_zb) p.need_ra = p.need_cb = 1;

  Staging st(stream, 0, {a, b}, {y});
  p.A = static_cast<const int8_t *>(st.In(a));
  p.B = static_cast<const int8_t *>(st.In(b));
  p.Y = st.Out(y);
  if (exact32) LaunchIGemm(p, stream);
  else LaunchQlmExact(p, za, zb, stream);
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// DequantizeLinear, kq/kernel_dequantizelinear.cc.

constexpr const char *kDqSupportedMsg =
    "kernel::DequantizeLinear: only UINT8, INT8, UINT16, INT16, INT32, FLOAT8E4M3FN, "
    "FLOAT8E4M3FNUZ, FLOAT8E5M2, FLOAT8E5M2FNUZ, INT4, UINT4, INT2, UINT2 and FLOAT4E2M1 inputs "
    "are supported.";

bool IsSupportedScaleDType(int32_t dt) { return dt == kFloat || dt == kFloat16; }

bool DqGpuDtype(int32_t dt) {
  switch (dt) {
  case kUint8: case kInt8: case kUint16: case kInt16: case kInt32: case kFloat8E4M3FN: case kFloat8E4M3FNUZ:
  case kFloat8E5M2: case kFloat8E5M2FNUZ: case kInt4: case kUint4: case kFloat4E2M1: case kUint2: case kInt2:
  case kFloat6E2M3: case kFloat6E3M2:
    return true;
  default:
    return false;
  }
}

void CheckDqDtype(int32_t dt) {
  if (!DqGpuDtype(dt)) throw InvalidArgument(Cat("unsupported data type ", dt, ", ", kDqSupportedMsg));
}

void CheckDqOutput(const onnxl_amd_tensor &x, const onnxl_amd_tensor &y) {
  OLA_ENFORCE(ShapeOf(y) == ShapeOf(x),
              "kernel::DequantizeLinear preallocated output shape must match x shape.");
  OLA_ENFORCE(y.size_bytes == NumElements(x) * ElementSize(y.data_type),
              "kernel::DequantizeLinear preallocated output buffer has unexpected size in bytes.");
}

int DequantizeLinear(const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale,
                     const onnxl_amd_tensor *x_zp, int64_t axis, onnxl_amd_tensor *y,
                     hipStream_t stream) {
  OLA_ENFORCE(!Absent(x) && !Absent(x_scale) && y, "kernel::DequantizeLinear: x, x_scale and the "
              "output are required.");
  CheckDescriptor(x, "x");
  CheckDescriptor(x_scale, "x_scale");
  CheckDescriptor(x_zp, "x_zero_point");
  CheckDescriptor(y, "y");
  const bool has_zp = !Absent(x_zp);
  DequantParams p{};
  p.n = NumElements(*x);
  p.x_dtype = x->data_type;
  if (NumElements(*x_scale) == 1) {
    // per-tensor, :349-410 (no zero point) and :426-502
    OLA_ENFORCE(IsSupportedScaleDType(x_scale->data_type),
                "kernel::DequantizeLinear: x_scale must be FLOAT or FLOAT16.");
    if (has_zp) {
      OLA_ENFORCE(NumElements(*x_zp) == 1,
                  "kernel::DequantizeLinear: x_zero_point must be a scalar (per-tensor dequantization).");
      OLA_ENFORCE(x->data_type == x_zp->data_type,
                  "kernel::DequantizeLinear: x_zero_point data_type must match x.");
      OLA_ENFORCE(y->data_type == x_scale->data_type,
                  "kernel::DequantizeLinear: output dtype must match x_scale.");
    } else {
      OLA_ENFORCE(y->data_type == x_scale->data_type,
                  "kernel::DequantizeLinear: output (no x_zero_point) dtype must match x_scale.");
    }
    CheckDqOutput(*x, *y);
    CheckDqDtype(x->data_type);
    p.mode = 0;
  } else {
    // per-axis / blocked, :522-651 (with zero point) and :670-693 (without)
    if (!has_zp)
      OLA_ENFORCE(axis >= 0 && axis < x->rank, "kernel::DequantizeLinear: axis out of range.");
    OLA_ENFORCE(IsSupportedScaleDType(x_scale->data_type),
                "kernel::DequantizeLinear: x_scale must be FLOAT or FLOAT16.");
    if (has_zp)
      OLA_ENFORCE(x->data_type == x_zp->data_type,
                  "kernel::DequantizeLinear: x_zero_point data_type must match x.");
    OLA_ENFORCE(y->data_type == x_scale->data_type,
                "kernel::DequantizeLinear: output dtype must match x_scale.");
    CheckDqOutput(*x, *y);
    OLA_ENFORCE(axis >= 0 && axis < x->rank, "kernel::DequantizeLinear: axis out of range.");
    if (has_zp)
      OLA_ENFORCE(ShapeOf(*x_scale) == ShapeOf(*x_zp),
                  "kernel::DequantizeLinear: x_scale and x_zero_point must have the same shape.");
    const Shape xs = ShapeOf(*x), ss = ShapeOf(*x_scale);
    p.inner = 1;
    for (int d = (int)axis + 1; d < x->rank; ++d) p.inner *= xs[d];
    p.axis_len = xs[axis];
    if (ss.size() == xs.size()) {
      for (size_t d = 0; d < xs.size(); ++d) {
        const int64_t s_dim = ss[d];
        OLA_ENFORCE(s_dim > 0 && xs[d] % s_dim == 0,
                    "kernel::DequantizeLinear: blocked x_scale dimension must divide the matching x "
                    "dimension.");
        OLA_ENFORCE((int64_t)d == axis || s_dim == xs[d],
                    "kernel::DequantizeLinear: blocked x_scale may only differ from x along the "
                    "quantization axis.");
      }
      p.mode = 2;
      p.s_axis = ss[axis];
      p.block = xs[axis] / ss[axis];
    } else {
      OLA_ENFORCE(NumElements(*x_scale) == xs[axis],
                  "kernel::DequantizeLinear: x_scale element count must equal axis dimension.");
      p.mode = 1;
    }
    CheckDqDtype(x->data_type);
  }
  p.scale_f16 = x_scale->data_type == kFloat16;
  Staging st(stream, 0, {x, x_scale, has_zp ? x_zp : nullptr}, {y});
  p.x = st.In(x);
  p.scale = st.In(x_scale);
  p.zp = has_zp ? st.In(x_zp) : nullptr;
  p.y = st.Out(y);
  LaunchDequantize(p, stream);
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// QuantizeLinear, kq/kernel_quantizelinear.cc.  Dispatch as Run (:917-941):
// a zero point fixes the output dtype; otherwise output_dtype does; otherwise
// the output is UINT8 and the scale must be a scalar.

// Output types with a zero point: every type of :543-648 and :700-822 (all
// of DequantizeLinear's inputs but INT32 and FLOAT8E8M0).
bool QlGpuOutput(int32_t dt) {
  return dt == kUint8 || dt == kInt8 || dt == kUint16 || dt == kInt16 || dt == kInt4 || dt == kUint4 ||
         dt == kFloat8E4M3FN || dt == kFloat8E4M3FNUZ || dt == kFloat8E5M2 || dt == kFloat8E5M2FNUZ ||
         dt == kFloat4E2M1 || dt == kUint2 || dt == kInt2 || dt == kFloat6E2M3 || dt == kFloat6E3M2;
}

int QuantizeLinear(const onnxl_amd_tensor *x, const onnxl_amd_tensor *y_scale, const onnxl_amd_tensor *y_zp,
                   int64_t axis, int32_t output_dtype, onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(!Absent(x) && !Absent(y_scale) && y,
              "kernel::QuantizeLinear: x, y_scale and the output are required.");
  CheckDescriptor(x, "x");
  CheckDescriptor(y_scale, "y_scale");
  CheckDescriptor(y_zp, "y_zero_point");
  CheckDescriptor(y, "y");
  // FloatValues (:33-55)
  OLA_ENFORCE(x->data_type == kFloat || x->data_type == kFloat16,
              "kernel::QuantizeLinear: x must be FLOAT or FLOAT16.");
  OLA_ENFORCE(y_scale->data_type == kFloat || y_scale->data_type == kFloat16,
              "kernel::QuantizeLinear: y_scale must be FLOAT or FLOAT16.");
  const bool has_zp = !Absent(y_zp);
  if (axis < 0) axis += x->rank;  // :928-930
  const bool scalar = NumElements(*y_scale) == 1;
  int32_t yt = kUint8;
  if (has_zp) {
    OLA_ENFORCE(y->data_type == y_zp->data_type,
                "kernel::QuantizeLinear: output data_type must match y_zero_point.");
    yt = y_zp->data_type;
    if (scalar)
      OLA_ENFORCE(NumElements(*y_zp) == 1,
                  "kernel::QuantizeLinear: y_zero_point must be a scalar (per-tensor quantization).");
  } else if (output_dtype != 0) {
    OLA_ENFORCE(y->data_type == output_dtype, "kernel::QuantizeLinear: output data_type must match output_dtype.");
    yt = output_dtype;
  } else {
    OLA_ENFORCE(scalar, "kernel::QuantizeLinear: y_scale must be a scalar (per-tensor quantization).");
    OLA_ENFORCE(y->data_type == kUint8,
                "kernel::QuantizeLinear: without y_zero_point and output_dtype the output is UINT8.");
  }
  const int64_t n = NumElements(*x);
  OLA_ENFORCE(ShapeOf(*y) == ShapeOf(*x), "kernel::QuantizeLinear preallocated output shape must match x shape.");
  QuantParams p{};
  p.n = n;
  p.mode = 0;
  if (!scalar) {
    OLA_ENFORCE(axis >= 0 && axis < x->rank, "kernel::QuantizeLinear: axis out of range.");
    if (has_zp)
      OLA_ENFORCE(ShapeOf(*y_scale) == ShapeOf(*y_zp),
                  "kernel::QuantizeLinear: y_scale and y_zero_point must have the same shape.");
    const Shape xs = ShapeOf(*x), ss = ShapeOf(*y_scale);
    p.inner = 1;
    for (int d = (int)axis + 1; d < x->rank; ++d) p.inner *= xs[d];
    p.axis_len = xs[axis];
    if (ss.size() == xs.size()) {  // blocked (:684-693)
      for (size_t d = 0; d < xs.size(); ++d) {
        const int64_t s_dim = ss[d];
        OLA_ENFORCE(s_dim > 0 && xs[d] % s_dim == 0,
                    "kernel::QuantizeLinear: blocked y_scale dimension must divide the matching x dimension.");
        OLA_ENFORCE((int64_t)d == axis || s_dim == xs[d],
                    "kernel::QuantizeLinear: blocked y_scale may only differ from x along the quantization axis.");
      }
      p.mode = 2;
      p.s_axis = ss[axis];
      p.block = xs[axis] / ss[axis];
    } else {  // per-axis (:694-698)
      OLA_ENFORCE(NumElements(*y_scale) == xs[axis],
                  "kernel::QuantizeLinear: y_scale element count must equal axis dimension.");
      p.mode = 1;
    }
  }
  // Output types: the no-zero-point overloads take 8- and 16-bit integers
  // (:485-532 adds FLOAT4E2M1 and FLOAT6 per tensor; :891-915 per axis and
  // blocked); with a zero point every type of :543-648 and :700-822.
  const bool no_zp_ok = yt == kUint8 || yt == kInt8 || yt == kUint16 || yt == kInt16 ||
                        (scalar && (yt == kFloat4E2M1 || yt == kFloat6E2M3 || yt == kFloat6E3M2));
  if (has_zp ? !QlGpuOutput(yt) : !no_zp_ok)
    throw InvalidArgument(Cat("unsupported data type ", yt, ", kernel::QuantizeLinear: unsupported output dtype."));
  OLA_ENFORCE(y->size_bytes == PackedBytes(yt, n),
              "kernel::QuantizeLinear preallocated output buffer has unexpected size in bytes.");
  p.x_f16 = x->data_type == kFloat16;
  p.scale_f16 = y_scale->data_type == kFloat16;
  p.y_dtype = yt;
  Staging st(stream, 0, {x, y_scale, has_zp ? y_zp : nullptr}, {y});
  p.x = st.In(x);
  p.scale = st.In(y_scale);
  p.zp = has_zp ? st.In(y_zp) : nullptr;
  p.y = st.Out(y);
  p.vec = reinterpret_cast<uintptr_t>(p.x) % 16 == 0 && reinterpret_cast<uintptr_t>(p.y) % 16 == 0;
  LaunchQuantize(p, stream);
  st.Finish();
  return ONNXL_AMD_OK;
}

// DynamicQuantizeLinear, kq/kernel_dynamicquantizelinear.cc:57-121.
int DynamicQuantizeLinear(const onnxl_amd_tensor *x, onnxl_amd_tensor *y, onnxl_amd_tensor *y_scale,
                          onnxl_amd_tensor *y_zp, hipStream_t stream) {
  OLA_ENFORCE(!Absent(x) && y && y_scale && y_zp,
              "kernel::DynamicQuantizeLinear: x, y, y_scale and y_zero_point are required.");
  CheckDescriptor(x, "x");
  CheckDescriptor(y, "y");
  CheckDescriptor(y_scale, "y_scale");
  CheckDescriptor(y_zp, "y_zero_point");
  OLA_ENFORCE(x->data_type == kFloat, "kernel::DynamicQuantizeLinear: x must be FLOAT.");
  OLA_ENFORCE(y->data_type == kUint8, "kernel::DynamicQuantizeLinear: y must be UINT8.");
  OLA_ENFORCE(ShapeOf(*y) == ShapeOf(*x), "kernel::DynamicQuantizeLinear: y shape must match x shape.");
  const int64_t n = NumElements(*x);
  OLA_ENFORCE(y->size_bytes == n, "kernel::DynamicQuantizeLinear: y buffer has unexpected size.");
  OLA_ENFORCE(y_scale->data_type == kFloat, "kernel::DynamicQuantizeLinear: y_scale must be FLOAT.");
  OLA_ENFORCE(y_scale->rank == 0 && y_scale->size_bytes == 4,
              "kernel::DynamicQuantizeLinear: y_scale must be a scalar FLOAT.");
  OLA_ENFORCE(y_zp->data_type == kUint8, "kernel::DynamicQuantizeLinear: y_zero_point must be UINT8.");
  OLA_ENFORCE(y_zp->rank == 0 && y_zp->size_bytes == 1,
              "kernel::DynamicQuantizeLinear: y_zero_point must be a scalar UINT8.");
  OLA_ENFORCE(n > 0, "kernel::DynamicQuantizeLinear: x must be non-empty.");
  Staging st(stream, DynQuantScratchBytes(n), {x}, {y, y_scale, y_zp});
  LaunchDynamicQuantize(static_cast<const float *>(st.In(x)), n, static_cast<uint8_t *>(st.Out(y)),
                        static_cast<float *>(st.Out(y_scale)), static_cast<uint8_t *>(st.Out(y_zp)), st.Extra(),
                        stream);
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// ConvInteger (nn/kernel_conv_integer.cc) and QLinearConv
// (kq/kernel_qlinearconv.cc).

constexpr const char *kCiName = "kernel::ConvInteger";
constexpr const char *kQcName = "kernel::QLinearConv";

struct ConvResolved {
  Shape k, s, d, pads, out;
};

// ResolveAttributes + ComputeOutputSpatial (kernel_conv_integer.cc:24-54,
// :107-141; kernel_qlinearconv.cc:53-119).  The rank checks run first so a
// malformed x cannot index past its shape.
ConvResolved ResolveConv(const Shape &xs, const Shape &ws, const onnxl_amd_conv_attrs *a, const char *name) {
  OLA_ENFORCE(a != nullptr, name, ": attributes are required.");
  OLA_ENFORCE(xs.size() >= 3, name, ": x must have rank >= 3.");
  OLA_ENFORCE(ws.size() == xs.size(), name, ": w rank must match x rank.");
  OLA_ENFORCE(a->n_kernel_shape >= 0 && a->n_kernel_shape <= ONNXL_AMD_MAX_CONV_SPATIAL && a->n_strides >= 0 &&
                  a->n_strides <= ONNXL_AMD_MAX_CONV_SPATIAL && a->n_dilations >= 0 &&
                  a->n_dilations <= ONNXL_AMD_MAX_CONV_SPATIAL && a->n_pads >= 0 &&
                  a->n_pads <= 2 * ONNXL_AMD_MAX_CONV_SPATIAL,
              name, ": attribute counts out of range.");
  const size_t sr = xs.size() - 2;
  ConvResolved r;
  r.k = a->n_kernel_shape ? Shape(a->kernel_shape, a->kernel_shape + a->n_kernel_shape)
                          : Shape(ws.begin() + 2, ws.end());
  OLA_ENFORCE(r.k.size() == sr, name, ": 'kernel_shape' size must match input spatial rank.");
  r.s = a->n_strides ? Shape(a->strides, a->strides + a->n_strides) : Shape(sr, 1);
  OLA_ENFORCE(r.s.size() == sr, name, ": 'strides' size must match input spatial rank.");
  r.d = a->n_dilations ? Shape(a->dilations, a->dilations + a->n_dilations) : Shape(sr, 1);
  OLA_ENFORCE(r.d.size() == sr, name, ": 'dilations' size must match input spatial rank.");
  if (a->auto_pad == ONNXL_AMD_AUTO_PAD_NOTSET) {
    r.pads = a->n_pads ? Shape(a->pads, a->pads + a->n_pads) : Shape(2 * sr, 0);
    OLA_ENFORCE(r.pads.size() == 2 * sr, name, ": 'pads' size must be 2 * spatial rank.");
  } else {
    OLA_ENFORCE(a->auto_pad == ONNXL_AMD_AUTO_PAD_SAME_UPPER || a->auto_pad == ONNXL_AMD_AUTO_PAD_SAME_LOWER ||
                    a->auto_pad == ONNXL_AMD_AUTO_PAD_VALID,
                name, ": 'auto_pad' must be NOTSET/SAME_UPPER/SAME_LOWER/VALID.");
    r.pads.assign(2 * sr, 0);
  }
  r.out.assign(sr, 0);
  for (size_t i = 0; i < sr; ++i) {
    const int64_t in = xs[i + 2], st = r.s[i];
    OLA_ENFORCE(st > 0 && r.d[i] > 0 && r.k[i] > 0, name, ": strides, dilations and kernel_shape must be positive.");
    const int64_t eff_k = (r.k[i] - 1) * r.d[i] + 1;
    if (a->auto_pad == ONNXL_AMD_AUTO_PAD_VALID) {
      r.out[i] = (in - eff_k) / st + 1;
    } else if (a->auto_pad == ONNXL_AMD_AUTO_PAD_NOTSET) {
      r.out[i] = (in + r.pads[i] + r.pads[i + sr] - eff_k) / st + 1;
    } else {
      const int64_t out = (in + st - 1) / st;
      const int64_t need = std::max<int64_t>(0, (out - 1) * st + eff_k - in);
      if (a->auto_pad == ONNXL_AMD_AUTO_PAD_SAME_UPPER) {
        r.pads[i] = need / 2;
        r.pads[i + sr] = need - need / 2;
      } else {
        r.pads[i + sr] = need / 2;
        r.pads[i] = need - need / 2;
      }
      r.out[i] = out;
    }
  }
  return r;
}

// x / w validation shared by both kernels (kernel_conv_integer.cc:74-88,
// kernel_qlinearconv.cc:178-192).
void CheckConvOperands(const onnxl_amd_tensor &x, const onnxl_amd_tensor &w, int64_t group, const char *name) {
  OLA_ENFORCE(IsInt8OrUint8(x.data_type), name, ": x must be INT8 or UINT8.");
  OLA_ENFORCE(IsInt8OrUint8(w.data_type), name, ": w must be INT8 or UINT8.");
  OLA_ENFORCE(group >= 1, name, ": 'group' must be >= 1.");
  OLA_ENFORCE(x.dims[1] == w.dims[1] * group, name, ": x.shape[1] must equal w.shape[1] * group.");
  OLA_ENFORCE(w.dims[0] % group == 0, name, ": w.shape[0] must be divisible by group.");
}

Shape ConvOutShape(const onnxl_amd_tensor &x, const onnxl_amd_tensor &w, const ConvResolved &r) {
  Shape out = {x.dims[0], w.dims[0]};
  out.insert(out.end(), r.out.begin(), r.out.end());
  return out;
}

// Geometry for the kernels; the GPU kernels take up to 3 spatial dims and
// the kernel_shape the weights actually have (the reference indexes w with
// the kernel_shape attribute).
ConvGeom MakeConvGeom(const onnxl_amd_tensor &x, const onnxl_amd_tensor &w, const ConvResolved &r, int64_t group,
                      const char *name) {
  const size_t sr = r.k.size();
  if (sr > 3) throw Unsupported(Cat(name, ": more than 3 spatial dimensions has no GPU kernel"));
  for (size_t i = 0; i < sr; ++i)
    if (r.k[i] != w.dims[i + 2]) throw Unsupported(Cat(name, ": kernel_shape differs from w's shape"));
  ConvGeom g{};
  g.N = x.dims[0];
  g.C = x.dims[1];
  g.G = group;
  g.cpg = w.dims[1];
  g.M = w.dims[0];
  g.Mg = g.M / group;
  for (int i = 0; i < 3; ++i) {
    g.in[i] = g.out[i] = 1;
    g.k[i] = 1;
    g.s[i] = g.d[i] = 1;
    g.pb[i] = 0;
  }
  for (size_t i = 0; i < sr; ++i) {
    const size_t j = 3 - sr + i;
    g.in[j] = x.dims[2 + i];
    g.out[j] = r.out[i];
    g.k[j] = (int)r.k[i];
    g.s[j] = r.s[i];
    g.d[j] = r.d[i];
    g.pb[j] = r.pads[i];
  }
  g.in_size = g.in[0] * g.in[1] * g.in[2];
  g.P = g.out[0] * g.out[1] * g.out[2];
  g.ks = (int64_t)g.k[0] * g.k[1] * g.k[2];
  g.Kc = g.cpg * g.ks;
  return g;
}

bool PresentOptional(const onnxl_amd_tensor *t) { return !(Absent(t) || (t->rank == 0 && t->size_bytes == 0)); }

// The GEMM over im2col columns: A = W as [G, Mg, Kc] (broadcast over the
// batch), B = Col [N, G, Kc, P], Y = [N, G, Mg, P] int32 sums.  a_zp: Mg
// per-row weight zero points on device (group 1 only), or nullptr with the
// scalar w_zp.
IGemmParams ConvGemmParams(const ConvGeom &g, const uint8_t *w, int w_u8, const uint8_t *a_zp, int32_t w_zp,
                           const uint8_t *col, int x_u8, int32_t x_zp, void *y) {
  IGemmParams p{};
  p.A = reinterpret_cast<const int8_t *>(w);
  p.B = reinterpret_cast<const int8_t *>(col);
  p.Y = y;
  p.M = g.Mg;
  p.N = g.P;
  p.K = g.Kc;
  p.batch = g.N * g.G;
  p.bm.rank = 2;
  p.bm.dims[0] = g.N;
  p.bm.dims[1] = g.G;
  p.bm.a_stride[0] = 0;
  p.bm.a_stride[1] = g.Mg * g.Kc;
  p.bm.b_stride[0] = g.G * g.Kc * g.P;
  p.bm.b_stride[1] = g.Kc * g.P;
  p.a_u8 = w_u8;
  p.b_u8 = x_u8;
  p.a_zp = a_zp;
  p.b_zp = nullptr;
  p.alpha_scalar = (w_u8 ? 128 : 0) - (a_zp ? 0 : w_zp);
  p.beta_scalar = (x_u8 ? 128 : 0) - x_zp;
  p.need_cb = a_zp != nullptr || p.alpha_scalar != 0;
  p.need_ra = p.beta_scalar != 0;
  p.epilogue = kEpiInt32;
  return p;
}

void LaunchConvGemm(const ConvGeom &g, const uint8_t *w, int w_u8, const uint8_t *a_zp, int32_t w_zp,
                    const uint8_t *col, int x_u8, int32_t x_zp, int32_t *y, hipStream_t stream) {
  LaunchIGemm(ConvGemmParams(g, w, w_u8, a_zp, w_zp, col, x_u8, x_zp, y), stream);
}

// The implicit GEMM (no im2col matrix in HBM) for group-1 2-D convolutions
// with C % 128 == 0 (ConvImplicitEligible) and a 16-byte aligned output.  Its
// scratch holds the zero-point-padded NHWC input, then the tap-major weight.
bool ConvImplicit(const ConvGeom &g, const onnxl_amd_tensor &y) {
  return ConvImplicitEligible(g) &&
         (y.location == ONNXL_AMD_HOST || reinterpret_cast<uintptr_t>(y.data) % 16 == 0);
}

size_t ConvImplicitScratch(const ConvGeom &g) {
  return Scratch::Round(ConvImplicitInputBytes(g)) + (size_t)(g.M * g.Kc);
}

// Launches the two operand passes into `scratch` and returns the GEMM over
// them: A = the tap-major weight [M, Kc], B = one padded image per batch entry.
IGemmParams ConvImplicitGemm(const ConvGeom &g, const uint8_t *x, int x_u8, int32_t x_zp, const uint8_t *w,
                             int w_u8, const uint8_t *a_zp, int32_t w_zp, void *y, void *scratch,
                             hipStream_t stream) {
  uint8_t *xh = static_cast<uint8_t *>(scratch);
  uint8_t *wr = xh + Scratch::Round(ConvImplicitInputBytes(g));
  LaunchConvImplicitOperands(g, x, (uint8_t)x_zp, w, xh, wr, stream);
  IGemmParams p = ConvGemmParams(g, wr, w_u8, a_zp, w_zp, xh, x_u8, x_zp, y);
  p.implicit_conv = 1;
  p.cv = ConvImplicitDesc(g);
  p.bm.b_stride[0] = p.cv.image_bytes;  // group 1: one padded image per batch entry
  p.bm.b_stride[1] = 0;
  return p;
}

int ConvInteger(const onnxl_amd_tensor *x, const onnxl_amd_tensor *w, const onnxl_amd_tensor *x_zp,
                const onnxl_amd_tensor *w_zp, const onnxl_amd_conv_attrs *attrs, onnxl_amd_tensor *y,
                hipStream_t stream) {
  OLA_ENFORCE(!Absent(x) && !Absent(w) && y, kCiName, ": x, w and the output are required.");
  CheckDescriptor(x, "x");
  CheckDescriptor(w, "w");
  CheckDescriptor(x_zp, "x_zero_point");
  CheckDescriptor(w_zp, "w_zero_point");
  CheckDescriptor(y, "y");
  const ConvResolved r = ResolveConv(ShapeOf(*x), ShapeOf(*w), attrs, kCiName);
  CheckConvOperands(*x, *w, attrs->group, kCiName);  // ValidateInputs, :74-88
  const int64_t M = w->dims[0];
  const bool xz_present = PresentOptional(x_zp), wz_present = PresentOptional(w_zp);
  if (xz_present) {  // :88-96
    OLA_ENFORCE(x_zp->data_type == x->data_type, kCiName, ": x_zero_point dtype must match x.");
    OLA_ENFORCE(NumElements(*x_zp) == 1, kCiName, ": x_zero_point must be a scalar.");
  }
  if (wz_present) {  // :97-106
    OLA_ENFORCE(w_zp->data_type == w->data_type, kCiName, ": w_zero_point dtype must match w.");
    const int64_t numel = NumElements(*w_zp);
    OLA_ENFORCE(numel == 1 || numel == M, kCiName, ": w_zero_point must be a scalar or 1-D of length M.");
  }
  const Shape out_shape = ConvOutShape(*x, *w, r);  // :184-201
  OLA_ENFORCE(y->data_type == kInt32, kCiName, " preallocated output must be INT32.");
  OLA_ENFORCE(ShapeOf(*y) == out_shape, kCiName, " preallocated output shape mismatch.");
  OLA_ENFORCE(y->size_bytes == NumElements(out_shape) * 4, kCiName,
              " preallocated output buffer has unexpected size.");
  const ConvGeom g = MakeConvGeom(*x, *w, r, attrs->group, kCiName);
  // :240-246: per-channel only for a 1-D zero point of length M
  const bool w_per_channel = wz_present && w_zp->rank == 1 && w_zp->dims[0] == M;
  int32_t xz = 0, wz = 0;
  RejectCapturedDeviceScalars(stream, {xz_present ? x_zp : nullptr, wz_present && !w_per_channel ? w_zp : nullptr},
                              kCiName);
  ReadTwoZeroPoints(stream, xz_present ? x_zp : nullptr, wz_present && !w_per_channel ? w_zp : nullptr, xz, wz);
  const bool gemm = (g.G == 1 || !w_per_channel) && g.Kc > 0;
  const bool implicit = gemm && ConvImplicit(g, *y);
  const size_t col_bytes = implicit ? ConvImplicitScratch(g) : (gemm ? ConvColBytes(g) : 0);
  Staging st(stream, col_bytes, {x, w, w_per_channel ? w_zp : nullptr}, {y});
  const uint8_t *xd = static_cast<const uint8_t *>(st.In(x));
  const uint8_t *wd = static_cast<const uint8_t *>(st.In(w));
  const uint8_t *wzd = w_per_channel ? static_cast<const uint8_t *>(st.In(w_zp)) : nullptr;
  int32_t *yd = static_cast<int32_t *>(st.Out(y));
  if (g.N * g.M * g.P > 0) {
    if (implicit) {
      LaunchIGemm(ConvImplicitGemm(g, xd, x->data_type == kUint8, xz, wd, w->data_type == kUint8, wzd, wz, yd,
                                   st.Extra(), stream),
                  stream);
    } else if (gemm) {
      const uint8_t *col = xd;
      if (!ConvColIsInput(g)) {
        col = static_cast<uint8_t *>(st.Extra());
        LaunchImToCol(g, xd, (uint8_t)xz, static_cast<uint8_t *>(st.Extra()), stream);
      }
      LaunchConvGemm(g, wd, w->data_type == kUint8, wzd, wz, col, x->data_type == kUint8, xz, yd, stream);
    } else {
      LaunchDirectConv(g, xd, x->data_type == kUint8, (uint8_t)xz, wd, w->data_type == kUint8, wzd, wz, nullptr,
                       yd, stream);
    }
  }
  st.Finish();
  return ONNXL_AMD_OK;
}

int QLinearConv(const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale, const onnxl_amd_tensor *x_zp,
                const onnxl_amd_tensor *w, const onnxl_amd_tensor *w_scale, const onnxl_amd_tensor *w_zp,
                const onnxl_amd_tensor *y_scale, const onnxl_amd_tensor *y_zp, const onnxl_amd_tensor *bias,
                const onnxl_amd_conv_attrs *attrs, onnxl_amd_tensor *y, hipStream_t stream) {
  const onnxl_amd_tensor *req[] = {x, x_scale, x_zp, w, w_scale, w_zp, y_scale, y_zp, y};
  for (auto *t : req) OLA_ENFORCE(!Absent(t), kQcName, ": the 8 inputs and the output are required.");
  const char *names[] = {"x", "x_scale", "x_zero_point", "w", "w_scale", "w_zero_point", "y_scale",
                         "y_zero_point", "y"};
  for (int i = 0; i < 9; ++i) CheckDescriptor(req[i], names[i]);
  CheckDescriptor(bias, "B");
  const ConvResolved r = ResolveConv(ShapeOf(*x), ShapeOf(*w), attrs, kQcName);  // :178-180
  OLA_ENFORCE(IsInt8OrUint8(x->data_type), kQcName, ": x must be INT8 or UINT8.");
  OLA_ENFORCE(IsInt8OrUint8(w->data_type), kQcName, ": w must be INT8 or UINT8.");
  OLA_ENFORCE(IsInt8OrUint8(y_zp->data_type), kQcName, ": y_zero_point must be INT8 or UINT8.");
  CheckConvOperands(*x, *w, attrs->group, kQcName);
  const Shape out_shape = ConvOutShape(*x, *w, r);  // :194-199
  OLA_ENFORCE(y->data_type == y_zp->data_type, kQcName, ": output dtype must match y_zero_point.");
  OLA_ENFORCE(ShapeOf(*y) == out_shape, kQcName, ": preallocated output shape mismatch.");
  OLA_ENFORCE(y->size_bytes == NumElements(out_shape), kQcName, ": preallocated output buffer has unexpected size.");
  // :200-211 (ReadScalarInt :38-45, ReadFloatElem :47-51): the checks in
  // the reference's order, then the four scalars read together
  OLA_ENFORCE(NumElements(*x_zp) == 1, kQcName, ": 'x_zero_point' must be a scalar.");
  OLA_ENFORCE(NumElements(*y_zp) == 1, kQcName, ": 'y_zero_point' must be a scalar.");
  OLA_ENFORCE(x_zp->data_type == x->data_type, kQcName, ": x_zero_point dtype must match x.");
  OLA_ENFORCE(w_zp->data_type == w->data_type, kQcName, ": w_zero_point dtype must match w.");
  OLA_ENFORCE(x_scale->data_type == kFloat, kQcName, ": scale must be FLOAT for the reference kernel.");
  OLA_ENFORCE(y_scale->data_type == kFloat, kQcName, ": scale must be FLOAT for the reference kernel.");
  // a scalar w_zero_point rides in the same batch (one synchronisation);
  // per-channel ones are read by the kernels
  const bool w_zp_scalar = !(NumElements(*w_zp) == w->dims[0] && w->dims[0] > 1);
  const onnxl_amd_tensor *sts[5] = {x_zp, y_zp, x_scale, y_scale, w_zp_scalar ? w_zp : nullptr};
  const size_t sbytes[5] = {1, 1, 4, 4, 1};
  uint8_t shost[5][8] = {};
  RejectCapturedDeviceScalars(stream, {sts[0], sts[1], sts[2], sts[3], sts[4]}, kQcName);
  ReadLeadingBytes(stream, 5, sts, sbytes, shost);
  const int32_t xz = ByteInt(*x_zp, shost[0][0]), yz = ByteInt(*y_zp, shost[1][0]);
  float xs, ys;
  std::memcpy(&xs, shost[2], 4);
  std::memcpy(&ys, shost[3], 4);
  OLA_ENFORCE(ys != 0.0f, kQcName, ": y_scale must be non-zero.");
  OLA_ENFORCE(NumElements(*x_scale) == 1 && NumElements(*y_scale) == 1, kQcName,
              ": 'x_scale' and 'y_scale' must be scalar.");
  const int64_t M = w->dims[0];
  const int64_t ws_n = NumElements(*w_scale), wz_n = NumElements(*w_zp);  // :213-227
  OLA_ENFORCE(ws_n == 1 || ws_n == M, kQcName, ": 'w_scale' must be scalar or length-M.");
  OLA_ENFORCE(wz_n == 1 || wz_n == M, kQcName, ": 'w_zero_point' must be scalar or length-M.");
  OLA_ENFORCE(w_scale->data_type == kFloat, kQcName, ": scale must be FLOAT for the reference kernel.");
  const bool has_bias = PresentOptional(bias);  // :229-238
  if (has_bias) {
    OLA_ENFORCE(bias->data_type == kInt32, kQcName, ": B must be INT32.");
    OLA_ENFORCE(NumElements(*bias) == M, kQcName, ": B must be 1-D with length M.");
  }
  const ConvGeom g = MakeConvGeom(*x, *w, r, attrs->group, kQcName);
  const bool w_per_channel = wz_n == M && M > 1;
  const int32_t wz = w_per_channel ? 0 : ByteInt(*w_zp, shost[4][0]);
  // The reference accumulates in int64 (:306-330).  The GEMM's int32 sums are
  // exact while Kc * max|x - x_zp| * max|w - w_zp| < 2^31; the bias is added
  // in int64 afterwards.  Otherwise, and for grouped convolutions with
  // per-channel weight zero points, the direct kernel sums in int64.
  auto span = [](int32_t dt, int32_t z) -> int64_t {
    const int64_t lo = dt == kInt8 ? -128 : 0, hi = dt == kInt8 ? 127 : 255;
    return std::max<int64_t>(std::llabs(lo - z), std::llabs(hi - z));
  };
  const int64_t w_span = w_per_channel ? 255 : span(w->data_type, wz);
  const bool exact32 = (double)g.Kc * (double)span(x->data_type, xz) * (double)w_span < 2147483648.0;
  const bool gemm = exact32 && (g.G == 1 || !w_per_channel) && g.Kc > 0;
  const bool implicit = gemm && ConvImplicit(g, *y);  // the GEMM epilogue requantizes
  const size_t col_bytes = implicit ? ConvImplicitScratch(g) : (gemm ? ConvColBytes(g) : 0);
  const size_t acc_off = Scratch::Round(col_bytes);
  const size_t acc_bytes = gemm && !implicit ? (size_t)(g.N * g.M * g.P) * 4 : 0;
  Staging st(stream, acc_off + acc_bytes, {x, w, w_scale, w_per_channel ? w_zp : nullptr, has_bias ? bias : nullptr},
             {y});
  const uint8_t *xd = static_cast<const uint8_t *>(st.In(x));
  const uint8_t *wd = static_cast<const uint8_t *>(st.In(w));
  const uint8_t *wzd = w_per_channel ? static_cast<const uint8_t *>(st.In(w_zp)) : nullptr;
  ConvQuant q{};
  q.x_scale = xs;
  q.y_scale = ys;
  q.w_scale = static_cast<const float *>(st.In(w_scale));
  q.w_scale_per_channel = ws_n == M && M > 1;
  q.bias = has_bias ? static_cast<const int32_t *>(st.In(bias)) : nullptr;
  const bool y_signed = y->data_type == kInt8;
  q.zy = (float)yz;
  q.qmin = y_signed ? -128.f : 0.f;
  q.qmax = y_signed ? 127.f : 255.f;
  uint8_t *yd = static_cast<uint8_t *>(st.Out(y));
  if (g.N * g.M * g.P > 0) {
    if (gemm) {
      const uint8_t *col = xd;
      int32_t *acc = reinterpret_cast<int32_t *>(static_cast<char *>(st.Extra()) + acc_off);
      if (!implicit && !ConvColIsInput(g)) {
        col = static_cast<uint8_t *>(st.Extra());
        LaunchImToCol(g, xd, (uint8_t)xz, static_cast<uint8_t *>(st.Extra()), stream);
      }
      // group 1 on the pipelined kernel: the GEMM epilogue requantizes each
      // output channel's row itself; otherwise int32 sums, then the pass
      IGemmParams p = implicit ? ConvImplicitGemm(g, xd, x->data_type == kUint8, xz, wd, w->data_type == kUint8, wzd,
                                                  wz, yd, st.Extra(), stream)
                               : ConvGemmParams(g, wd, w->data_type == kUint8, wzd, wz, col, x->data_type == kUint8,
                                                xz, yd);
      p.epilogue = kEpiQuant8Row;
      p.zy = q.zy;
      p.qmin = q.qmin;
      p.qmax = q.qmax;
      p.y_signed = y_signed;
      p.row_wscale = q.w_scale;
      p.row_wscale_per = q.w_scale_per_channel;
      p.row_xs = q.x_scale;
      p.row_ys = q.y_scale;
      p.row_bias = q.bias;
      if (implicit || (g.G == 1 && IGemmFastEligible(p))) {
        LaunchIGemm(p, stream);
      } else {
        LaunchConvGemm(g, wd, w->data_type == kUint8, wzd, wz, col, x->data_type == kUint8, xz, acc, stream);
        LaunchConvRequant(g, acc, q, yd, stream);
      }
    } else {
      LaunchDirectConv(g, xd, x->data_type == kUint8, (uint8_t)xz, wd, w->data_type == kUint8, wzd, wz, &q, yd,
                       stream);
    }
  }
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// DequantizePacked, onnx_core/runtime/dequantize_packed.cc:296-372.

struct PackedProfile {
  const char *format;
  int64_t block_size, block_bytes;
  int ggml_type;
};

// The reference's 27 fixed wire profiles (ggml block sizes and bytes,
// dequantize_packed.cc:27-36), all decoded on the GPU.
constexpr PackedProfile kPackedProfiles[] = {
    {"gguf:q4_0", 32, 18, 2},      {"gguf:q4_1", 32, 20, 3},      {"gguf:q5_0", 32, 22, 6},
    {"gguf:q5_1", 32, 24, 7},      {"gguf:q8_0", 32, 34, 8},      {"gguf:q8_1", 32, 36, 9},
    {"gguf:q2_k", 256, 84, 10},    {"gguf:q3_k", 256, 110, 11},   {"gguf:q4_k", 256, 144, 12},
    {"gguf:q5_k", 256, 176, 13},   {"gguf:q6_k", 256, 210, 14},   {"gguf:q8_k", 256, 292, 15},
    {"gguf:iq2_xxs", 256, 66, 16}, {"gguf:iq2_xs", 256, 74, 17},  {"gguf:iq3_xxs", 256, 98, 18},
    {"gguf:iq1_s", 256, 50, 19},   {"gguf:iq4_nl", 32, 18, 20},   {"gguf:iq3_s", 256, 110, 21},
    {"gguf:iq2_s", 256, 82, 22},   {"gguf:iq4_xs", 256, 136, 23}, {"gguf:iq1_m", 256, 56, 29},
    {"gguf:tq1_0", 256, 54, 34},   {"gguf:tq2_0", 256, 66, 35},   {"gguf:mxfp4", 32, 17, 39},
    {"gguf:nvfp4", 64, 36, 40},    {"gguf:q1_0", 128, 18, 41},    {"gguf:q2_0", 64, 18, 42}};

int DequantizePacked(const onnxl_amd_tensor *x, const char *format, const int64_t *shape, int32_t rank,
                     int64_t output_dtype, onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(format != nullptr && x && y && (rank == 0 || shape) && rank >= 0 && rank <= ONNXL_AMD_MAX_RANK,
              "DequantizePacked: invalid arguments.");
  CheckDescriptor(x, "x");
  CheckDescriptor(y, "y");
  const PackedProfile *prof = nullptr;  // PackedQuantizationLayout, :296-302
  for (const auto &pp : kPackedProfiles)
    if (std::strcmp(pp.format, format) == 0) prof = &pp;
  if (!prof) throw InvalidArgument(Cat("DequantizePacked: unsupported format '", format, "'."));
  // ValidatePackedQuantizationShape, :304-332
  OLA_ENFORCE(output_dtype == kFloat || output_dtype == kFloat16 || output_dtype == kBfloat16 ||
                  output_dtype == kDouble,
              "DequantizePacked: output_dtype must be FLOAT, FLOAT16, BFLOAT16 or DOUBLE.");
  OLA_ENFORCE(rank >= 1, "DequantizePacked: shape must have rank at least one.");
  bool empty = false;
  for (int i = 0; i < rank; ++i) {
    OLA_ENFORCE(shape[i] >= 0, "DequantizePacked: dimensions must be nonnegative.");
    empty |= shape[i] == 0;
  }
  OLA_ENFORCE(shape[rank - 1] % prof->block_size == 0,
              "DequantizePacked: last dimension must contain complete blocks.");
  int64_t count = 1;
  for (int i = 0; i < rank && !empty; ++i) {
    OLA_ENFORCE(shape[i] == 0 || count <= INT64_MAX / shape[i], "DequantizePacked: dimension exceeds size_t.");
    count *= shape[i];
  }
  if (empty) count = 0;
  const int64_t expected = count / prof->block_size * prof->block_bytes;
  // DequantizePackedTensor, :337-343
  OLA_ENFORCE(x->data_type == kUint8 && x->rank == 1, "DequantizePacked: x must be a one-dimensional UINT8 tensor.");
  OLA_ENFORCE(x->dims[0] == expected && x->size_bytes == expected,
              "DequantizePacked: packed input length must match exactly.");
  OLA_ENFORCE(y->data_type == output_dtype, "DequantizePacked: preallocated output dtype must be output_dtype.");
  OLA_ENFORCE(ShapeOf(*y) == Shape(shape, shape + rank), "DequantizePacked: preallocated output shape mismatch.");
  OLA_ENFORCE(y->size_bytes == count * ElementSize((int32_t)output_dtype),
              "DequantizePacked: preallocated output buffer has unexpected size.");
  if (!PackedFormatOnGpu(prof->ggml_type))
    throw Unsupported(Cat("DequantizePacked: format ", format, " has no GPU kernel"));
  Staging st(stream, 0, {x}, {y});
  LaunchDequantizePacked(prof->ggml_type, static_cast<const uint8_t *>(st.In(x)), count / prof->block_size,
                         (int)output_dtype, st.Out(y), stream);
  st.Finish();
  return ONNXL_AMD_OK;
}

// Fused DequantizePacked(format, shape [N, K], FLOAT16) -> MatMul with the
// weight transposed: y = a @ W^T.  No single reference kernel: it computes
// the chain dequantize_packed.cc:334-372 -> km/kernel_matmul.cc:181-223 that a
// DequantizePacked -> Transpose -> MatMul subgraph runs node by node.
//  - decode GEMVs (1 <= M <= 8) fused for q4_0, q8_0, q2_k, q3_k, q4_k, q5_k,
//    q6_k and iq4_xs;
//  - every other format, M or alignment: the weight decoded to FLOAT16 [N, K]
//    in the workspace (the chain's rounding), then the 16-bit MFMA GEMM
//    reading its rows as the B operand (no transpose is written).
int DequantizePackedMatMul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x, const char *format,
                           const int64_t *shape, int32_t rank, onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(a && x && y && format && shape && rank == 2, "DequantizePackedMatMul: invalid arguments.");
  CheckDescriptor(a, "a");
  CheckDescriptor(x, "x");
  CheckDescriptor(y, "y");
  const int64_t N = shape[0], K = shape[1];
  OLA_ENFORCE(N >= 0 && K >= 0, "DequantizePacked: dimensions must be nonnegative.");
  OLA_ENFORCE(a->data_type == kFloat16 && a->rank == 2 && a->dims[1] == K,
              "DequantizePackedMatMul: a must be FLOAT16 [M, K].");
  const int64_t M = a->dims[0];
  OLA_ENFORCE(y->data_type == kFloat16 && ShapeOf(*y) == Shape({M, N}) && y->size_bytes == M * N * 2,
              "DequantizePackedMatMul: y must be FLOAT16 [M, N].");
  const PackedProfile *prof = nullptr;
  for (const auto &pp : kPackedProfiles)
    if (std::strcmp(pp.format, format) == 0) prof = &pp;
  if (!prof) throw InvalidArgument(Cat("DequantizePacked: unsupported format '", format, "'."));
  const int64_t bv = prof->block_size, bb = prof->block_bytes;
  OLA_ENFORCE(K % bv == 0, "DequantizePacked: last dimension must contain complete blocks.");
  OLA_ENFORCE(x->data_type == kUint8 && x->rank == 1, "DequantizePacked: x must be a one-dimensional UINT8 tensor.");
  OLA_ENFORCE(x->dims[0] == N * (K / bv) * bb && x->size_bytes == x->dims[0],
              "DequantizePacked: packed input length must match exactly.");
  if (M == 0 || N == 0) return ONNXL_AMD_OK;  // empty [M, N] result, nothing to launch
  const int t = prof->ggml_type;
  const bool q40 = t == 2, q80 = t == 8;
  const int k_align = GemvKAlignment(t);  // the 256-value formats with a fused GEMV
  // the fused GEMVs take these when the operands are aligned (host payloads
  // are staged into aligned scratch)
  const bool gemv_format = (q40 || q80 || k_align > 0) && M <= 8 && K > 0;
  auto aligned = [](const onnxl_amd_tensor *t, int b) {
    return t->location == ONNXL_AMD_HOST || reinterpret_cast<uintptr_t>(t->data) % b == 0;
  };
  const bool try_gemv = gemv_format && (q40 || q80 ? K % 64 == 0 : true) && aligned(a, 16) &&
                        aligned(x, q40 || q80 ? 4 : k_align);
  const int64_t w_bytes = try_gemv ? 0 : N * K * 2;
  Staging st(stream, (size_t)w_bytes, {a, x}, {y});
  const void *ad = st.In(a), *xd = st.In(x);
  uint16_t *yd = static_cast<uint16_t *>(st.Out(y));
  if (try_gemv) {
    if (k_align > 0)
      LaunchGemvK(t, static_cast<const uint16_t *>(ad), static_cast<const uint8_t *>(xd), M, N, K, yd, stream);
    else
      (q80 ? LaunchGemvQ80 : LaunchGemvQ40)(static_cast<const uint16_t *>(ad), static_cast<const uint8_t *>(xd), M,
                                           N, K, yd, stream);
  } else {
    uint16_t *w = static_cast<uint16_t *>(st.Extra());
    LaunchDequantizePacked(t, static_cast<const uint8_t *>(xd), N * (K / bv), kFloat16, w, stream);
    HMatMulParams h{};
    h.A = static_cast<const uint16_t *>(ad);
    h.B = w;
    h.Y = yd;
    h.M = M;
    h.N = N;
    h.K = K;
    h.batch = 1;
    h.bf16 = 0;
    LaunchHMatMulBT(h, stream);
  }
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// Cast FLOAT -> FLOAT16 / BFLOAT16.

int Cast(const onnxl_amd_tensor *x, int32_t to, onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(!Absent(x) && y, "kernel::Cast: input and output are required.");
  CheckDescriptor(x, "x");
  CheckDescriptor(y, "y");
  if (x->data_type != kFloat || (to != kFloat16 && to != kBfloat16))
    throw Unsupported("Cast: only FLOAT -> FLOAT16 / BFLOAT16 runs on the GPU path");
  OLA_ENFORCE(y->data_type == to, "kernel::Cast: output dtype must match 'to'.");
  OLA_ENFORCE(ShapeOf(*y) == ShapeOf(*x), "kernel::Cast: output shape must match input shape.");
  OLA_ENFORCE(y->size_bytes == NumElements(*x) * 2, "kernel::Cast: output size does not match.");
  Staging st(stream, 0, {x}, {y});
  LaunchCastF32(static_cast<const float *>(st.In(x)), st.Out(y), NumElements(*x), to == kBfloat16,
                stream);
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// Transpose of a 2-D tensor (perm [1, 0]), tensor/kernel_transpose.cc:98-111
// (the preallocated output's checks with the reference's messages).

int Transpose2d(const onnxl_amd_tensor *x, onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(!Absent(x) && y, "kernel::Transpose: input and output are required.");
  CheckDescriptor(x, "x");
  CheckDescriptor(y, "y");
  if (x->rank != 2) throw Unsupported("Transpose: the GPU path transposes 2-D tensors (perm [1, 0]).");
  const int64_t width = PackedBytes(x->data_type, 1);
  if (PackedBytes(x->data_type, 2) != 2 * width || !(width == 1 || width == 2 || width == 4 || width == 8))
    throw Unsupported("Transpose: the GPU path takes 1, 2, 4 or 8-byte elements.");
  OLA_ENFORCE(y->data_type == x->data_type, "kernel::Transpose: preallocated output dtype must match input dtype.");
  OLA_ENFORCE(y->rank == 2 && y->dims[0] == x->dims[1] && y->dims[1] == x->dims[0],
              "kernel::Transpose: preallocated output shape mismatch.");
  OLA_ENFORCE(y->size_bytes >= NumElements(*x) * width && y->data != nullptr,
              "kernel::Transpose: preallocated output buffer is too small.");
  if ((x->dims[0] + 63) / 64 > 65535 || (x->dims[1] + 63) / 64 > (int64_t(1) << 31) - 1)
    throw Unsupported("Transpose: more than 65535 row blocks of 64.");
  Ctx();
  Staging st(stream, 0, {x}, {y});
  LaunchTranspose2d(st.In(x), st.Out(y), x->dims[0], x->dims[1], (int)width, stream);
  OLA_HIP(hipGetLastError());
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// MatMul FLOAT16 / BFLOAT16, km/kernel_matmul.cc:225-253.

constexpr const char *kMmName = "kernel::MatMul";

int MatMul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *b, onnxl_amd_tensor *y,
           hipStream_t stream) {
  OLA_ENFORCE(!Absent(a) && !Absent(b) && y, kMmName, ": A, B and the output are required.");
  CheckDescriptor(a, "A");
  CheckDescriptor(b, "B");
  CheckDescriptor(y, "Y");
  OLA_ENFORCE(a->data_type == b->data_type, kMmName, " inputs must share the same dtype.");
  if (a->data_type != kFloat16 && a->data_type != kBfloat16)
    throw Unsupported("MatMul: only FLOAT16 / BFLOAT16 run on the GPU path");
  OLA_ENFORCE(y->data_type == a->data_type, kMmName,
              " preallocated output must have the same dtype as input A.");
  const MatMulPlan plan = MakeMatMulPlan(ShapeOf(*a), ShapeOf(*b), kMmName,
                                         " does not accept rank-0 inputs.",
                                         " got incompatible inner dimensions.",
                                         " inputs are not broadcast-compatible on batch dimensions.");
  OLA_ENFORCE(ShapeOf(*y) == plan.out_shape, kMmName, " preallocated output has an invalid shape.");
  OLA_ENFORCE(y->size_bytes == NumElements(plan.out_shape) * 2, kMmName,
              " preallocated output buffer size does not match its shape.");
  HMatMulParams p{};
  p.M = plan.M;
  p.N = plan.N;
  p.K = plan.K;
  p.batch = plan.batch;
  p.bm = ToBatchMap(plan);
  p.bf16 = a->data_type == kBfloat16;
  Staging st(stream, 0, {a, b}, {y});
  p.A = static_cast<const uint16_t *>(st.In(a));
  p.B = static_cast<const uint16_t *>(st.In(b));
  p.Y = static_cast<uint16_t *>(st.Out(y));
  LaunchHMatMul(p, stream);
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// Fused DequantizeLinear -> [Cast] -> MatMul.

constexpr const char *kDqmName = "DequantizeLinearMatMul";

// Validation of the fused node (the DequantizeLinear, Cast and MatMul nodes'
// own checks) and its launch parameters; payload pointers are left unset.
DqMatMulParams PlanDqMatMul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x,
                            const onnxl_amd_tensor *x_scale, const onnxl_amd_tensor *x_zp, int64_t axis,
                            int32_t cast_to, onnxl_amd_tensor *y) {
  OLA_ENFORCE(!Absent(a) && !Absent(x) && !Absent(x_scale) && y, kDqmName,
              ": A, x, x_scale and the output are required.");
  CheckDescriptor(a, "A");
  CheckDescriptor(x, "x", /*allow_tiled=*/true);
  CheckDescriptor(x_scale, "x_scale");
  CheckDescriptor(x_zp, "x_zero_point");
  CheckDescriptor(y, "Y");
  const bool has_zp = !Absent(x_zp);
  // The DequantizeLinear node's own checks (kq/kernel_dequantizelinear.cc:522-565).
  OLA_ENFORCE(IsSupportedScaleDType(x_scale->data_type),
              "kernel::DequantizeLinear: x_scale must be FLOAT or FLOAT16.");
  if (has_zp)
    OLA_ENFORCE(x->data_type == x_zp->data_type,
                "kernel::DequantizeLinear: x_zero_point data_type must match x.");
  OLA_ENFORCE(x->rank == 2, kDqmName, ": the quantized weight must be 2-D [K, N].");
  const Shape xs = ShapeOf(*x), ss = ShapeOf(*x_scale);
  const int64_t K = xs[0], N = xs[1];
  DqMatMulParams p{};
  const int64_t scount = NumElements(*x_scale);
  if (scount == 1) {
    if (has_zp)
      OLA_ENFORCE(NumElements(*x_zp) == 1,
                  "kernel::DequantizeLinear: x_zero_point must be a scalar (per-tensor dequantization).");
    p.mode = 0;
  } else {
    OLA_ENFORCE(axis >= 0 && axis < 2, "kernel::DequantizeLinear: axis out of range.");
    if (has_zp)
      OLA_ENFORCE(ShapeOf(*x_scale) == ShapeOf(*x_zp),
                  "kernel::DequantizeLinear: x_scale and x_zero_point must have the same shape.");
    if (ss.size() == 2) {
      for (size_t d = 0; d < 2; ++d) {
        OLA_ENFORCE(ss[d] > 0 && xs[d] % ss[d] == 0,
                    "kernel::DequantizeLinear: blocked x_scale dimension must divide the matching x "
                    "dimension.");
        OLA_ENFORCE((int64_t)d == axis || ss[d] == xs[d],
                    "kernel::DequantizeLinear: blocked x_scale may only differ from x along the "
                    "quantization axis.");
      }
      if (axis != 0) throw Unsupported(Cat(kDqmName, ": scales blocked along N"));
      p.mode = 2;
      p.block = K / ss[0];
    } else {
      OLA_ENFORCE(scount == xs[axis],
                  "kernel::DequantizeLinear: x_scale element count must equal axis dimension.");
      if (axis != 1) throw Unsupported(Cat(kDqmName, ": 1-D per-row (axis 0) scales"));
      p.mode = 1;
    }
  }
  switch (x->data_type) {
  case kInt4: case kUint4: case kInt8: case kUint8: case kFloat8E4M3FN: break;
  default: throw Unsupported(Cat(kDqmName, ": weight dtype ", x->data_type, " has no GPU kernel"));
  }
  // Rounding chain of the unfused graph: DequantizeLinear output = x_scale
  // dtype; optional Cast; then MatMul requires both operands to share A's dtype.
  const int32_t dq_out = x_scale->data_type;
  const int32_t w_dtype = cast_to ? cast_to : dq_out;
  OLA_ENFORCE(a->data_type == kFloat16 || a->data_type == kBfloat16, kDqmName,
              ": A must be FLOAT16 or BFLOAT16.");
  OLA_ENFORCE(w_dtype == a->data_type, kMmName, " inputs must share the same dtype.");
  if (cast_to)
    OLA_ENFORCE(dq_out == kFloat, kDqmName, ": the Cast step must convert a FLOAT DequantizeLinear output.");
  OLA_ENFORCE(y->data_type == a->data_type, kMmName,
              " preallocated output must have the same dtype as input A.");
  const MatMulPlan plan = MakeMatMulPlan(ShapeOf(*a), xs, kMmName, " does not accept rank-0 inputs.",
                                         " got incompatible inner dimensions.",
                                         " inputs are not broadcast-compatible on batch dimensions.");
  OLA_ENFORCE(ShapeOf(*y) == plan.out_shape, kMmName, " preallocated output has an invalid shape.");
  OLA_ENFORCE(y->size_bytes == NumElements(plan.out_shape) * 2, kMmName,
              " preallocated output buffer size does not match its shape.");
  p.M = plan.M * plan.batch;  // A batches are contiguous rows; W is shared
  p.N = N;
  p.K = K;
  p.w_dtype = x->data_type;
  p.scale_f16 = x_scale->data_type == kFloat16;
  p.a_bf16 = a->data_type == kBfloat16;
  p.deq_round_f16 = dq_out == kFloat16;
  p.cast_round = cast_to == kBfloat16 ? 16 : (cast_to == kFloat16 ? 10 : 0);
  p.w_tiled = x->layout == ONNXL_AMD_LAYOUT_TILED_INT4;
  return p;
}

int DqMatMul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale,
             const onnxl_amd_tensor *x_zp, int64_t axis, int32_t cast_to, onnxl_amd_tensor *y,
             hipStream_t stream) {
  DqMatMulParams p = PlanDqMatMul(a, x, x_scale, x_zp, axis, cast_to, y);
  const bool has_zp = !Absent(x_zp);
  const size_t scratch_bytes = DqMatMulScratchBytes(p);
  Staging st(stream, scratch_bytes, {a, x, x_scale, has_zp ? x_zp : nullptr}, {y});
  p.A = st.In(a);
  p.W = static_cast<const uint8_t *>(st.In(x));
  p.scale = st.In(x_scale);
  p.zp = has_zp ? static_cast<const uint8_t *>(st.In(x_zp)) : nullptr;
  p.Y = st.Out(y);
  const size_t nc = DqMatMulCounters(p);
  unsigned *counters = nc ? Ctx().ws.Counters(nc) : nullptr;
  if (!LaunchDqMatMul(p, st.Extra(), scratch_bytes, counters, nc, stream))
    throw Unsupported(Cat(kDqmName, ": no GPU kernel for this shape / dtype combination"));
  st.Finish();
  return ONNXL_AMD_OK;
}

// The same node with no allocation: every payload on the device, scratch and
// counters taken from the device's fixed array (NoAllocScratch).
int DqMatMulNoAlloc(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale,
                    const onnxl_amd_tensor *x_zp, int64_t axis, int32_t cast_to, onnxl_amd_tensor *y,
                    hipStream_t stream) {
  DqMatMulParams p = PlanDqMatMul(a, x, x_scale, x_zp, axis, cast_to, y);
  const bool has_zp = !Absent(x_zp);
  for (const onnxl_amd_tensor *t : {a, x, x_scale, has_zp ? x_zp : nullptr, (const onnxl_amd_tensor *)y})
    OLA_ENFORCE(t == nullptr || t->location == ONNXL_AMD_DEVICE, kDqmName,
                ": the no-allocation entry point takes device payloads only (no host staging).");
  char *base = static_cast<char *>(NoAllocScratch());
  p.A = a->data;
  p.W = static_cast<const uint8_t *>(x->data);
  p.scale = x_scale->data;
  p.zp = has_zp ? static_cast<const uint8_t *>(x_zp->data) : nullptr;
  p.Y = y->data;
  const size_t need = DqMatMulScratchBytes(p), nc = DqMatMulCounters(p);
  if (need > kNoAllocDataBytes || nc * sizeof(unsigned) > kNoAllocCounterBytes)
    throw Unsupported(Cat(kDqmName, ": this call needs ", need, " bytes of scratch and ", nc,
                          " counters; the no-allocation entry point holds ", kNoAllocDataBytes, " bytes and ",
                          kNoAllocCounterBytes / sizeof(unsigned), " counters (use the allocating entry point)"));
  if (!LaunchDqMatMul(p, base + kNoAllocCounterBytes, kNoAllocDataBytes, reinterpret_cast<unsigned *>(base),
                      kNoAllocCounterBytes / sizeof(unsigned), stream))
    throw Unsupported(Cat(kDqmName, ": no GPU kernel for this shape / dtype combination"));
  OLA_HIP(hipGetLastError());
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// GroupedMatMul.  Validation and messages of GroupedMatMul::operator()
// (math/kernel_grouped_matmul.cc:50-90).

constexpr const char *kGmmName = "kernel::GroupedMatMul";
constexpr int64_t kGmmMaxGroups = 4096;  // routing counters in LDS

// The GroupedMatMul node's checks (:48-88) for weights of shape w_shape and
// dtype w_dtype (the weights tensor itself, or the dequantized experts of the
// fused node), then this build's limits.  Fills the shape fields of p.
// `weights` (null for the fused node) joins the payload checks in the
// reference's order.
void PlanGrouped(const onnxl_amd_tensor *input, const Shape &w_shape, int32_t w_dtype,
                 const onnxl_amd_tensor *weights, const onnxl_amd_tensor *group_indices,
                 const onnxl_amd_tensor *bias, int64_t transB, const onnxl_amd_tensor *y, GroupedParams &p) {
  const bool tb = transB != 0;
  OLA_ENFORCE(input->rank == 2 && w_shape.size() == 3 && group_indices->rank == 2, kGmmName,
              " expects input rank 2, weights rank 3, and indices rank 2.");
  const int64_t M = input->dims[0], K = input->dims[1], G = w_shape[0];
  const int64_t N = w_shape[tb ? 1 : 2], S = group_indices->dims[1];
  OLA_ENFORCE(K == w_shape[tb ? 2 : 1] && M == group_indices->dims[0], kGmmName,
              " incompatible input dimensions.");
  const int32_t dt = input->data_type;
  OLA_ENFORCE(dt == kFloat || dt == kDouble || dt == kFloat16 || dt == kBfloat16, kGmmName,
              " expects floating-point inputs.");
  OLA_ENFORCE(w_dtype == dt, kGmmName, " weights must match the input dtype.");
  OLA_ENFORCE(group_indices->data_type == kInt32 || group_indices->data_type == kInt64, kGmmName,
              " indices must be INT32 or INT64.");
  for (const onnxl_amd_tensor *t : {input, weights, group_indices})
    OLA_ENFORCE(!t || t->size_bytes == PackedBytes(t->data_type, NumElements(*t)), kGmmName,
                " tensor payload does not match its shape.");
  const bool has_bias = !Absent(bias);
  if (has_bias) {
    OLA_ENFORCE(bias->data_type == dt && bias->rank == 2 && bias->dims[0] == G && bias->dims[1] == N, kGmmName,
                " bias must have shape [G,N] and match the input dtype.");
    OLA_ENFORCE(bias->size_bytes == PackedBytes(dt, G * N), kGmmName, " tensor payload does not match its shape.");
  }
  const int64_t P = M * S;
  if (group_indices->location == ONNXL_AMD_HOST) {
    // host indices: the reference's range check before any work
    const bool i64 = group_indices->data_type == kInt64;
    for (int64_t i = 0; i < P; ++i) {
      const int64_t g = i64 ? static_cast<const int64_t *>(group_indices->data)[i]
                            : static_cast<const int32_t *>(group_indices->data)[i];
      OLA_ENFORCE(g >= 0 && g < G, kGmmName, " group index must be in [0,G).");
    }
  }
  OLA_ENFORCE(y->data_type == dt && y->rank == 3 && y->dims[0] == M && y->dims[1] == S && y->dims[2] == N, kGmmName,
              ": the output must be [M, S, N] of the input dtype.");
  OLA_ENFORCE(y->size_bytes == PackedBytes(dt, P * N), kGmmName, ": output buffer size does not match its shape.");
  if (dt != kFloat16 && dt != kBfloat16) throw Unsupported("GroupedMatMul: only FLOAT16 / BFLOAT16 run on the GPU path");
  if (G > kGmmMaxGroups) throw Unsupported(Cat("GroupedMatMul: more than ", kGmmMaxGroups, " groups"));
  OLA_ENFORCE(P < (int64_t(1) << 31) - 1, kGmmName, ": more than 2^31 (token, selection) pairs");
  p.M = M;
  p.K = K;
  p.N = N;
  p.G = G;
  p.S = S;
  p.idx64 = group_indices->data_type == kInt64;
  p.transB = tb;
  p.bf16 = dt == kBfloat16;
  p.nbn = (N + 127) / 128;
}

// Routing workspace of a grouped launch: row and tile offsets (G + 1 each)
// and the routed pairs (M * S), as int32.
size_t GroupedRouteBytes(const GroupedParams &p) { return (size_t)(2 * (p.G + 1) + p.M * p.S) * sizeof(int32_t); }

void SetGroupedRoute(GroupedParams &p, void *ws) {
  int32_t *w32 = static_cast<int32_t *>(ws);
  p.row_off = w32;
  p.tile_off = w32 + (p.G + 1);
  p.rows = w32 + 2 * (p.G + 1);
}

int GroupedMatMul(const onnxl_amd_tensor *input, const onnxl_amd_tensor *weights,
                  const onnxl_amd_tensor *group_indices, const onnxl_amd_tensor *bias, int64_t transB,
                  onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(!Absent(input) && !Absent(weights) && !Absent(group_indices) && y, kGmmName,
              ": input, weights, group_indices and the output are required.");
  CheckDescriptor(input, "input");
  CheckDescriptor(weights, "weights");
  CheckDescriptor(group_indices, "group_indices");
  CheckDescriptor(bias, "bias");
  CheckDescriptor(y, "output");
  GroupedParams p{};
  PlanGrouped(input, ShapeOf(*weights), weights->data_type, weights, group_indices, bias, transB, y, p);
  if (p.M * p.S == 0 || p.N == 0) return ONNXL_AMD_OK;
  Ctx();
  const bool has_bias = !Absent(bias);
  Staging st(stream, GroupedRouteBytes(p), {input, weights, group_indices, has_bias ? bias : nullptr}, {y});
  p.A = st.In(input);
  p.W = st.In(weights);
  p.idx = st.In(group_indices);
  p.bias = has_bias ? st.In(bias) : nullptr;
  p.Y = st.Out(y);
  SetGroupedRoute(p, st.Extra());
  LaunchGroupedMatMul(p, stream);
  OLA_HIP(hipGetLastError());
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// Fused DequantizeLinear -> [Cast] -> GroupedMatMul: quantized MoE experts.

constexpr const char *kDqgName = "DequantizeLinearGroupedMatMul";

int DqGroupedMatMul(const onnxl_amd_tensor *input, const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale,
                    const onnxl_amd_tensor *x_zp, int64_t axis, int32_t cast_to,
                    const onnxl_amd_tensor *group_indices, const onnxl_amd_tensor *bias, int64_t transB,
                    onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(!Absent(input) && !Absent(x) && !Absent(x_scale) && !Absent(group_indices) && y, kDqgName,
              ": input, x, x_scale, group_indices and the output are required.");
  CheckDescriptor(input, "input");
  CheckDescriptor(x, "x");
  CheckDescriptor(x_scale, "x_scale");
  CheckDescriptor(x_zp, "x_zero_point");
  CheckDescriptor(group_indices, "group_indices");
  CheckDescriptor(bias, "bias");
  CheckDescriptor(y, "output");
  const bool has_zp = !Absent(x_zp);
  // The DequantizeLinear node's checks (kq/kernel_dequantizelinear.cc:522-565),
  // as onnxl_amd_dequantize_linear makes them.
  DqGroupedParams q{};
  OLA_ENFORCE(IsSupportedScaleDType(x_scale->data_type),
              "kernel::DequantizeLinear: x_scale must be FLOAT or FLOAT16.");
  if (has_zp)
    OLA_ENFORCE(x->data_type == x_zp->data_type, "kernel::DequantizeLinear: x_zero_point data_type must match x.");
  OLA_ENFORCE(x->rank == 3, kDqgName, ": the quantized experts must be 3-D.");
  const Shape xs = ShapeOf(*x), ss = ShapeOf(*x_scale);
  OLA_ENFORCE(x->size_bytes == PackedBytes(x->data_type, NumElements(*x)), kDqgName,
              ": x payload does not match its shape.");
  if (NumElements(*x_scale) == 1) {
    if (has_zp)
      OLA_ENFORCE(NumElements(*x_zp) == 1,
                  "kernel::DequantizeLinear: x_zero_point must be a scalar (per-tensor dequantization).");
    q.scale_kind = 0;
  } else {
    OLA_ENFORCE(axis >= 0 && axis < x->rank, "kernel::DequantizeLinear: axis out of range.");
    if (has_zp)
      OLA_ENFORCE(ShapeOf(*x_scale) == ShapeOf(*x_zp),
                  "kernel::DequantizeLinear: x_scale and x_zero_point must have the same shape.");
    q.inner = 1;
    for (int d = (int)axis + 1; d < x->rank; ++d) q.inner *= xs[d];
    q.axis_dim = xs[axis];
    if (ss.size() == xs.size()) {
      for (size_t d = 0; d < xs.size(); ++d) {
        OLA_ENFORCE(ss[d] > 0 && xs[d] % ss[d] == 0,
                    "kernel::DequantizeLinear: blocked x_scale dimension must divide the matching x dimension.");
        OLA_ENFORCE((int64_t)d == axis || ss[d] == xs[d],
                    "kernel::DequantizeLinear: blocked x_scale may only differ from x along the quantization axis.");
      }
      q.scale_kind = 2;
      q.block = xs[axis] / ss[axis];
    } else {
      OLA_ENFORCE(NumElements(*x_scale) == xs[axis],
                  "kernel::DequantizeLinear: x_scale element count must equal axis dimension.");
      q.scale_kind = 1;
    }
  }
  switch (x->data_type) {
  case kInt4: case kUint4: case kInt8: case kUint8: case kFloat8E4M3FN: break;
  default: throw Unsupported(Cat(kDqgName, ": weight dtype ", x->data_type, " has no GPU kernel"));
  }
  // the Cast node, then GroupedMatMul on the weights' final dtype
  const int32_t dq_out = x_scale->data_type;
  if (cast_to) {
    OLA_ENFORCE(dq_out == kFloat, kDqgName, ": the Cast step must convert a FLOAT DequantizeLinear output.");
    OLA_ENFORCE(cast_to == kFloat16 || cast_to == kBfloat16, kDqgName, ": Cast to FLOAT16 or BFLOAT16 only.");
  }
  PlanGrouped(input, xs, cast_to ? cast_to : dq_out, nullptr, group_indices, bias, transB, y, q.g);
  q.x_dtype = x->data_type;
  q.scale_f16 = x_scale->data_type == kFloat16;
  q.deq_round_f16 = dq_out == kFloat16;
  q.cast_round = cast_to == kBfloat16 ? 16 : (cast_to == kFloat16 ? 10 : 0);
  // fp8 experts on the core: FLOAT scales constant along K within a group
  // (per tensor, per expert [G], per column [N] or [G, 1, N]), the Cast to
  // BFLOAT16, no zero point, weights [G, K, N]
  if (x->data_type == kFloat8E4M3FN && dq_out == kFloat && cast_to == kBfloat16 && !has_zp && !transB) {
    const int64_t N = xs[2];
    if (q.scale_kind == 0) {
      q.fused = 1;
    } else if (q.scale_kind == 1 && axis == 0) {
      q.fused = 1, q.scale_grp_stride = 1;
    } else if (q.scale_kind == 1 && axis == 2) {
      q.fused = 1, q.scale_per_col = 1;
    } else if (q.scale_kind == 2 && axis == 1 && ss[1] == 1) {
      q.fused = 1, q.scale_per_col = 1, q.scale_grp_stride = N;
    }
  }
  const GroupedParams &g = q.g;
  if (g.M * g.S == 0 || g.N == 0) return ONNXL_AMD_OK;
  Ctx();
  // the fused check needs the device addresses: staged host payloads sit in
  // 256-byte aligned scratch, so judge on an aligned stand-in for those
  auto addr = [](const onnxl_amd_tensor *t) -> const void * {
    return t->location == ONNXL_AMD_HOST ? reinterpret_cast<const void *>(uintptr_t(256)) : t->data;
  };
  q.g.A = addr(input);
  q.X = static_cast<const uint8_t *>(addr(x));
  q.g.Y = const_cast<void *>(addr(y));
  q.g.bias = Absent(bias) ? nullptr : addr(bias);
  const bool fused = DqGroupedFusedEligible(q);
  const size_t route = Scratch::Round(GroupedRouteBytes(g));
  const size_t w16 = fused ? 0 : (size_t)(g.G * g.K * g.N) * 2;
  const bool has_bias = !Absent(bias);
  Staging st(stream, route + w16, {input, x, x_scale, has_zp ? x_zp : nullptr, group_indices,
                                   has_bias ? bias : nullptr}, {y});
  q.g.A = st.In(input);
  q.X = static_cast<const uint8_t *>(st.In(x));
  q.scale = st.In(x_scale);
  q.zp = has_zp ? static_cast<const uint8_t *>(st.In(x_zp)) : nullptr;
  q.g.idx = st.In(group_indices);
  q.g.bias = has_bias ? st.In(bias) : nullptr;
  q.g.Y = st.Out(y);
  SetGroupedRoute(q.g, st.Extra());
  q.w16 = fused ? nullptr : reinterpret_cast<uint16_t *>(static_cast<char *>(st.Extra()) + route);
  if (!fused) q.fused = 0;
  LaunchDqGroupedMatMul(q, stream);
  OLA_HIP(hipGetLastError());
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// ORT MatMulNBits preparation.  The format's own checks
// (onnx_core/runtime/quantization.cc:117-124 dimensions, :940-970 storage
// sizes, :1826-1860 padding bits and finite scales), then the limits of the
// fused kernels this prepares for.

struct NbitsLayout {
  int64_t groups, blob, zcol;
  int64_t weight_bytes, scale_bytes, zp_bytes;  // prepared sizes
};

NbitsLayout PlanNbits(int64_t K, int64_t N, int64_t bits, int64_t block, bool has_zp) {
  OLA_ENFORCE(K > 0 && N > 0, "ORT MatMulNBits requires positive K and N dimensions.");
  OLA_ENFORCE(block >= 16 && block <= 0xffffffffLL && (block & (block - 1)) == 0,
              "ORT MatMulNBits block_size must be a power of two in [16, UINT32_MAX].");
  OLA_ENFORCE(bits == 2 || bits == 4 || bits == 8, "Expected an ORT MatMulNBits quantization format.");
  if (K % block != 0)
    throw Unsupported(Cat("MatMulNBits: K = ", K, " is not a multiple of block_size ", block,
                          " (a partial last block has no fused kernel)"));
  NbitsLayout l{};
  l.groups = K / block;
  l.blob = block * bits / 8;
  l.zcol = (l.groups * bits + 7) / 8;
  l.weight_bytes = bits <= 4 ? TiledInt4Bytes(K, N) : K * N;  // 2-bit codes as 4-bit ones
  l.scale_bytes = l.groups * N * 2;
  l.zp_bytes = !has_zp ? 0 : (bits == 8 ? l.groups * N : (l.groups * N + 1) / 2);
  return l;
}

int PrepareMatMulNbits(const onnxl_amd_tensor *B, const onnxl_amd_tensor *scales, const onnxl_amd_tensor *zero_points,
                       int64_t K, int64_t N, int64_t bits, int64_t block, onnxl_amd_tensor *weight,
                       onnxl_amd_tensor *scale, onnxl_amd_tensor *zero_point, hipStream_t stream) {
  OLA_ENFORCE(!Absent(B) && !Absent(scales) && weight && scale, "prepare_matmul_nbits: B, scales, weight and scale are required.");
  CheckDescriptor(B, "B");
  CheckDescriptor(scales, "scales");
  CheckDescriptor(zero_points, "zero_points");
  const bool has_zp = !Absent(zero_points);
  const NbitsLayout l = PlanNbits(K, N, bits, block, has_zp);
  OLA_ENFORCE(B->data_type == kUint8 && B->rank == 3 && B->dims[0] == N && B->dims[1] == l.groups &&
                  B->dims[2] == l.blob,
              "prepare_matmul_nbits: B must be UINT8 [N, groups, block_size * bits / 8].");
  if (scales->data_type != kFloat16)
    throw Unsupported("MatMulNBits: only FLOAT16 scales (FLOAT16 weights) have a fused kernel");
  OLA_ENFORCE(scales->rank == 2 && scales->dims[0] == N && scales->dims[1] == l.groups,
              "prepare_matmul_nbits: scales must be [N, groups].");
  if (has_zp) {
    if (zero_points->data_type != kUint8)
      throw Unsupported("MatMulNBits: floating-point zero points have no fused kernel");
    OLA_ENFORCE(zero_points->rank == 2 && zero_points->dims[0] == N && zero_points->dims[1] == l.zcol,
                "Invalid ORT MatMulNBits zero-point dtype.");
  }
  // the format's value checks, on a host copy (one-time preparation)
  {
    std::vector<uint16_t> sc((size_t)(N * l.groups));
    ReadBytes(*scales, 0, sc.data(), sc.size() * 2);
    for (uint16_t h : sc) OLA_ENFORCE((h & 0x7c00u) != 0x7c00u, "Nonfinite ORT MatMulNBits scale.");
    if (has_zp) {
      const int64_t per = 8 / bits;
      if (l.groups % per != 0) {
        std::vector<uint8_t> zb((size_t)(N * l.zcol));
        ReadBytes(*zero_points, 0, zb.data(), zb.size());
        for (int64_t n = 0; n < N; ++n)
          OLA_ENFORCE((zb[(size_t)((n + 1) * l.zcol - 1)] >> ((l.groups % per) * bits)) == 0,
                      "Nonzero ORT MatMulNBits zero-point padding.");
      }
    }
  }
  const bool four = bits <= 4;  // 2-bit codes are prepared as 4-bit ones
  auto out_ok = [](onnxl_amd_tensor *t, int64_t need, const char *what) {
    OLA_ENFORCE(t->location == ONNXL_AMD_DEVICE, "prepare_matmul_nbits: ", what, " must be device memory.");
    OLA_ENFORCE(t->size_bytes >= need, "prepare_matmul_nbits: ", what, " holds ", t->size_bytes, " bytes, needs ", need);
    OLA_ENFORCE(need == 0 || (t->data != nullptr && reinterpret_cast<uintptr_t>(t->data) % 16 == 0),
                "prepare_matmul_nbits: ", what, " must be a 16-byte aligned device buffer.");
  };
  out_ok(weight, l.weight_bytes, "weight");
  out_ok(scale, l.scale_bytes, "scale");
  if (has_zp) {
    OLA_ENFORCE(zero_point, "prepare_matmul_nbits: zero_point is required with zero_points.");
    out_ok(zero_point, l.zp_bytes, "zero_point");
  }
  Ctx();
  Staging st(stream, 0, {B, scales, has_zp ? zero_points : nullptr}, {});
  NbitsPrepParams p{};
  p.B = static_cast<const uint8_t *>(st.In(B));
  p.scales = static_cast<const uint16_t *>(st.In(scales));
  p.zp = has_zp ? static_cast<const uint8_t *>(st.In(zero_points)) : nullptr;
  p.K = K;
  p.N = N;
  p.block = block;
  p.bits = bits;
  p.weight = weight->data;
  p.scale_out = scale->data;
  p.zp_out = has_zp ? zero_point->data : nullptr;
  LaunchPrepareNbits(p, stream);
  OLA_HIP(hipGetLastError());
  st.Finish();
  auto set = [](onnxl_amd_tensor *t, int32_t dt, int64_t d0, int64_t d1, int32_t layout) {
    t->data_type = dt;
    t->rank = 2;
    for (int i = 0; i < ONNXL_AMD_MAX_RANK; ++i) t->dims[i] = i == 0 ? d0 : (i == 1 ? d1 : 0);
    t->layout = layout;
  };
  set(weight, four ? (has_zp ? kUint4 : kInt4) : (has_zp ? kUint8 : kInt8), K, N,
      four ? ONNXL_AMD_LAYOUT_TILED_INT4 : ONNXL_AMD_LAYOUT_ONNX);
  set(scale, kFloat16, l.groups, N, ONNXL_AMD_LAYOUT_ONNX);
  if (has_zp) set(zero_point, four ? kUint4 : kUint8, l.groups, N, ONNXL_AMD_LAYOUT_ONNX);
  else if (zero_point) zero_point->rank = -1;
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// AWQ and GPTQ checkpoint weights (onnx_core/runtime/awq.cc:47-246,
// onnx_core/runtime/gptq.cc:49-253): the formats' geometry and value checks
// with the reference's messages, then either preparation into the fused
// DequantizeLinear -> MatMul operands or a dense decode to [N, K].  Value
// checks run on host copies (one-time work per weight).

struct CkptPlan {
  CkptLayout L{};                 // qweight / qzeros pointers set per use
  const char *fmt = "AWQ";        // message prefix
  int32_t word_type = kInt32, zeros_type = kInt32, scale_type = kFloat16;
  const char *zeros_name = "qzeros";
  Shape qweight_shape, qzeros_shape, scales_shape;
  bool trivial_groups = true;     // GPTQ: g_idx[k] == k / group (set after reading g_idx)
};

// awq.cc:64-118 (Geometry), in the reference's order of checks.
CkptPlan PlanAwq(const char *variant, int64_t K, int64_t N, int64_t bits, int64_t group, int32_t scale_type) {
  const std::string v = variant ? variant : "";
  OLA_ENFORCE(K > 0 && N > 0 && (bits == 4 || (bits == 8 && v == "gemm")),
              "AWQ requires positive dimensions, supported bits and group_axis=1.");
  OLA_ENFORCE(v == "gemm" || v == "gemv" || v == "gemv_fast" || v == "llm-awq", "AWQ unsupported variant.");
  OLA_ENFORCE(group == -1 || group > 0, "AWQ unsupported group size.");
  const int64_t eff = group == -1 ? K : group;
  OLA_ENFORCE(K % eff == 0, "AWQ requires complete groups.");
  CkptPlan p;
  CkptLayout &L = p.L;
  L.K = K, L.N = N, L.bits = (int)bits, L.group = eff, L.groups = K / eff, L.width = 4;
  p.scale_type = scale_type;
  if (v == "gemm") {
    OLA_ENFORCE(N % (32 / bits) == 0 && (scale_type == kFloat16 || scale_type == kBfloat16),
                "AWQ GEMM requires complete INT32 words and FP16/BF16 scales.");
    L.kind = kAwqGemm;
    p.qweight_shape = {K, N / (32 / bits)};
    p.qzeros_shape = {L.groups, N / (32 / bits)};
    p.scales_shape = {L.groups, N};
    return p;
  }
  OLA_ENFORCE(eff >= 128 || eff == 16 || eff == 32 || eff == 64, "AWQ invalid effective group size.");
  OLA_ENFORCE(scale_type == kFloat16, "AWQ GEMV requires FLOAT16 parameters.");
  const int64_t multiplier = eff >= 128 ? 1 : 128 / eff;
  const int64_t words = L.groups / 8 + (L.groups % 8 != 0);
  L.padded = (words / multiplier + (words % multiplier != 0)) * multiplier * 8;
  if (v == "gemv") {
    OLA_ENFORCE(K % 8 == 0, "AWQ GEMV requires K divisible by eight.");
    L.kind = kAwqGemv;
    p.qweight_shape = {N, K / 8};
    p.qzeros_shape = {N, L.padded / 8};
    p.scales_shape = {N, L.padded};
  } else {
    OLA_ENFORCE(K % 64 == 0 && N % 4 == 0, "AWQ GEMV_FAST requires K divisible by 64 and N by four.");
    L.kind = kAwqFast;
    L.width = 2;
    p.word_type = kInt16;
    p.zeros_type = kFloat16;
    p.zeros_name = v == "llm-awq" ? "scaled_zeros" : "qzeros";
    p.qweight_shape = {N / 4, K};
    p.qzeros_shape = {L.padded, N};
    p.scales_shape = {L.padded, N};
  }
  return p;
}

// gptq.cc:67-123 (Geometry), in the reference's order of checks; the word
// dtype is qweight's.
CkptPlan PlanGptq(const char *format, int64_t K, int64_t N, int64_t bits, int64_t group, int32_t word_type,
                  int32_t scale_type) {
  const std::string f = format ? format : "";
  OLA_ENFORCE(f == "gptq" || f == "gptq_v2" || f == "gptq_p", "GPTQ unsupported format.");
  OLA_ENFORCE(K > 0 && N > 0 && bits >= 2 && bits <= 8, "GPTQ invalid dimensions, bits or group axis.");
  OLA_ENFORCE(group == -1 || group > 0, "GPTQ invalid group size.");
  OLA_ENFORCE(word_type == kInt8 || word_type == kInt16 || word_type == kInt32 || word_type == kInt64,
              "GPTQ unsupported packed word dtype.");
  const int width = (int)ElementSize(word_type);
  OLA_ENFORCE(f != "gptq_p" || width == 4, "GPTQ planar checkpoint format requires INT32 words.");
  OLA_ENFORCE(f == "gptq_p" || bits == 2 || bits == 3 || bits == 4 || bits == 8,
              "GPTQ five-, six- and seven-bit codes require the gptq_p format.");
  const bool planar = bits == 5 || bits == 6 || bits == 7 || (f == "gptq_p" && bits == 3);
  if (bits == 3 || planar)
    OLA_ENFORCE(width == 4 && K % 32 == 0 && N % 32 == 0,
                "GPTQ three-bit and planar layouts require INT32 and 32-code blocks.");
  OLA_ENFORCE(scale_type == kFloat16 || scale_type == kBfloat16 || scale_type == kFloat,
              "GPTQ unsupported scales dtype.");
  CkptPlan p;
  p.fmt = "GPTQ";
  CkptLayout &L = p.L;
  L.kind = kGptq, L.K = K, L.N = N, L.bits = (int)bits, L.width = width, L.planar = planar;
  L.zero_add = f == "gptq" ? 1 : 0;
  L.group = group == -1 ? K : group;
  L.groups = (K + L.group - 1) / L.group;
  const int64_t wb = 8 * width;
  L.zero_columns = (N * bits + wb - 1) / wb;
  p.word_type = p.zeros_type = word_type;
  p.scale_type = scale_type;
  p.qweight_shape = {(K * bits + wb - 1) / wb, N};
  p.qzeros_shape = {L.groups, L.zero_columns};
  p.scales_shape = {L.groups, N};
  return p;
}

void CheckCkptTensor(const CkptPlan &p, const onnxl_amd_tensor *t, int32_t type, const Shape &shape,
                     const char *name) {
  OLA_ENFORCE(!Absent(t) && t->data_type == type && ShapeOf(*t) == shape &&
                  t->size_bytes >= NumElements(shape) * ElementSize(type) && t->data != nullptr,
              p.fmt, " invalid tensor type, shape or byte extent: ", name, ".");
  CheckDescriptor(t, name);
  OLA_ENFORCE(reinterpret_cast<uintptr_t>(t->data) % ElementSize(type) == 0, p.fmt, ": ", name,
              " must be aligned to its ", ElementSize(type), "-byte elements.");
}

float Bf16BitsToFloat(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Host copies of a checkpoint's parameters, then the formats' value checks.
struct CkptHost {
  std::vector<float> scales, zero_terms;  // decoded; zero_terms: AWQ gemv_fast / llm-awq
  std::vector<uint8_t> qzeros, qweight;   // raw words (qweight read only when a scan needs it)
  std::vector<int32_t> g_idx;             // GPTQ
};

std::vector<float> ReadFloats(const onnxl_amd_tensor &t) {
  const int64_t n = NumElements(t);
  std::vector<float> out((size_t)n);
  if (t.data_type == kFloat) {
    ReadBytes(t, 0, out.data(), (size_t)n * 4);
    return out;
  }
  std::vector<uint16_t> h((size_t)n);
  ReadBytes(t, 0, h.data(), (size_t)n * 2);
  for (int64_t i = 0; i < n; ++i) out[i] = t.data_type == kFloat16 ? HalfBitsToFloat(h[i]) : Bf16BitsToFloat(h[i]);
  return out;
}

// The value of weight (k, n) of group g as the kernels compute it.
float CkptValue(const CkptLayout &L, const CkptHost &h, int64_t g, int64_t k, int64_t n) {
  const int64_t si = CkptScaleIndex(L, g, n);
  const double code = (double)CkptCode(L, k, n);
  if (L.kind == kAwqFast) {
    const float product = (float)(code * (double)h.scales[si]);  // exact in double, one rounding
    volatile float sum = product + h.zero_terms[si];
    return sum;
  }
  return (float)((code - (double)CkptZero(L, g, n)) * (double)h.scales[si]);
}

// Throws `msg` when some value reaches `limit` in magnitude (or is not
// finite).  A (group, column) pair whose bound max|code - zero| * |scale|
// (+ |zero term|) stays below the limit needs no scan; the others are
// scanned exactly over their rows, reading qweight on first need.
void CheckCkptMagnitudes(const CkptPlan &p, const onnxl_amd_tensor *qweight, CkptHost &h, double limit,
                         const std::string &msg) {
  CkptLayout L = p.L;
  L.qzeros = h.qzeros.data();
  const double maxq = (double)((1u << L.bits) - 1);
  for (int64_t g = 0; g < L.groups; ++g)
    for (int64_t n = 0; n < L.N; ++n) {
      const int64_t si = CkptScaleIndex(L, g, n);
      double bound;
      if (L.kind == kAwqFast) {
        bound = maxq * std::fabs((double)h.scales[si]) + std::fabs((double)h.zero_terms[si]);
      } else {
        const double z = (double)CkptZero(L, g, n);
        bound = std::max(z, maxq - z) * std::fabs((double)h.scales[si]);
      }
      if (bound < limit * 0.999) continue;
      if (h.qweight.empty()) {
        h.qweight.resize((size_t)(NumElements(*qweight) * ElementSize(qweight->data_type)));
        ReadBytes(*qweight, 0, h.qweight.data(), h.qweight.size());
      }
      L.qweight = h.qweight.data();
      for (int64_t k = 0; k < L.K; ++k) {
        const int64_t gk = h.g_idx.empty() ? k / L.group : (int64_t)h.g_idx[(size_t)k];
        if (gk != g) continue;
        const float v = CkptValue(L, h, g, k, n);
        OLA_ENFORCE(std::isfinite(v) && std::fabs((double)v) < limit, msg);
      }
    }
}

constexpr double kFloatOverflow = 3.4028235677973366e38 * (1.0 + 1.0 / (1 << 25));  // FLT_MAX + half an ulp

// awq.cc:156-183 and :232-245 (CheckParameter, CheckReconstruction).
CkptHost CheckAwqValues(CkptPlan &p, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                        const onnxl_amd_tensor *scales) {
  CkptHost h;
  CkptLayout &L = p.L;
  if (L.kind == kAwqFast) {
    h.zero_terms = ReadFloats(*qzeros);
    for (float z : h.zero_terms) OLA_ENFORCE(std::isfinite(z), "AWQ nonfinite parameter.");
  } else {
    h.qzeros.resize((size_t)(NumElements(*qzeros) * 4));
    ReadBytes(*qzeros, 0, h.qzeros.data(), h.qzeros.size());
  }
  h.scales = ReadFloats(*scales);
  for (size_t i = 0; i < h.scales.size(); ++i) {
    OLA_ENFORCE(std::isfinite(h.scales[i]), "AWQ nonfinite parameter.");
    const int64_t g = L.kind == kAwqGemv ? (int64_t)i % L.padded : (int64_t)i / L.N;
    OLA_ENFORCE(g >= L.groups || h.scales[i] > 0, "AWQ nonpositive used scale.");
  }
  if (p.scale_type != kFloat16)  // finite FP16 parameters cannot overflow FLOAT with these codes
    CheckCkptMagnitudes(p, qweight, h, kFloatOverflow, "AWQ FLOAT reconstruction overflow.");
  return h;
}

// gptq.cc:230-253 (CheckData).
CkptHost CheckGptqValues(CkptPlan &p, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                         const onnxl_amd_tensor *scales, const onnxl_amd_tensor *g_idx) {
  CkptHost h;
  CkptLayout &L = p.L;
  h.g_idx.resize((size_t)L.K);
  ReadBytes(*g_idx, 0, h.g_idx.data(), h.g_idx.size() * 4);
  for (int64_t k = 0; k < L.K; ++k) {
    OLA_ENFORCE(h.g_idx[k] >= 0 && h.g_idx[k] < L.groups, "GPTQ invalid group map index.");
    if (h.g_idx[k] != k / L.group) p.trivial_groups = false;
  }
  h.qzeros.resize((size_t)(NumElements(*qzeros) * L.width));
  ReadBytes(*qzeros, 0, h.qzeros.data(), h.qzeros.size());
  h.scales = ReadFloats(*scales);
  CkptLayout Lz = L;
  Lz.qzeros = h.qzeros.data();
  const uint32_t maxq = (1u << L.bits) - 1;
  for (size_t i = 0; i < h.scales.size(); ++i) {
    OLA_ENFORCE(std::isfinite(h.scales[i]) && h.scales[i] > 0, "GPTQ nonfinite or nonpositive scale.");
    if (L.zero_add)
      OLA_ENFORCE(GptqField(Lz, Lz.qzeros, (int64_t)i % L.N, (int64_t)i / L.N, true) != maxq,
                  "GPTQ v1 all-ones zero field has ambiguous upstream conversion semantics.");
  }
  if (p.scale_type != kFloat16)
    CheckCkptMagnitudes(p, qweight, h, kFloatOverflow, "GPTQ FLOAT reconstruction overflow.");
  return h;
}

struct CkptSizes {
  int64_t weight, scale, zp;
};

CkptSizes CkptPreparedSizes(const CkptPlan &p) {
  const CkptLayout &L = p.L;
  const bool four = L.bits <= 4;
  return {four ? TiledInt4Bytes(L.K, L.N) : L.K * L.N, L.groups * L.N * (p.scale_type == kFloat16 ? 2 : 4),
          four ? (L.groups * L.N + 1) / 2 : L.groups * L.N};
}

// Writes the fused kernels' operands (see LaunchCkptPrepare) and sets the
// output descriptors: weight UINT4 tiled (bits <= 4) or UINT8 [K, N], zero
// point UINT4 / UINT8 [groups, N], scale FLOAT16 [groups, N] for FLOAT16
// scales, else FLOAT (BFLOAT16 widened exactly).
int PrepareCkpt(const char *what, CkptPlan &p, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                const onnxl_amd_tensor *scales, onnxl_amd_tensor *weight, onnxl_amd_tensor *scale,
                onnxl_amd_tensor *zero_point, hipStream_t stream) {
  OLA_ENFORCE(weight && scale && zero_point, what, ": weight, scale and zero_point are required.");
  const CkptSizes sz = CkptPreparedSizes(p);
  auto out_ok = [&](onnxl_amd_tensor *t, int64_t need, const char *name) {
    OLA_ENFORCE(t->location == ONNXL_AMD_DEVICE, what, ": ", name, " must be device memory.");
    OLA_ENFORCE(t->size_bytes >= need, what, ": ", name, " holds ", t->size_bytes, " bytes, needs ", need);
    OLA_ENFORCE(need == 0 || (t->data != nullptr && reinterpret_cast<uintptr_t>(t->data) % 16 == 0), what, ": ",
                name, " must be a 16-byte aligned device buffer.");
  };
  out_ok(weight, sz.weight, "weight");
  out_ok(scale, sz.scale, "scale");
  out_ok(zero_point, sz.zp, "zero_point");
  Ctx();
  Staging st(stream, 0, {qweight, qzeros, scales}, {});
  CkptLayout L = p.L;
  L.qweight = static_cast<const uint8_t *>(st.In(qweight));
  L.qzeros = static_cast<const uint8_t *>(st.In(qzeros));
  LaunchCkptPrepare(L, st.In(scales), p.scale_type, weight->data, scale->data, zero_point->data, stream);
  OLA_HIP(hipGetLastError());
  st.Finish();
  const bool four = L.bits <= 4;
  auto set = [](onnxl_amd_tensor *t, int32_t dt, int64_t d0, int64_t d1, int32_t layout) {
    t->data_type = dt;
    t->rank = 2;
    for (int i = 0; i < ONNXL_AMD_MAX_RANK; ++i) t->dims[i] = i == 0 ? d0 : (i == 1 ? d1 : 0);
    t->layout = layout;
  };
  set(weight, four ? kUint4 : kUint8, L.K, L.N, four ? ONNXL_AMD_LAYOUT_TILED_INT4 : ONNXL_AMD_LAYOUT_ONNX);
  set(scale, p.scale_type == kFloat16 ? kFloat16 : kFloat, L.groups, L.N, ONNXL_AMD_LAYOUT_ONNX);
  set(zero_point, four ? kUint4 : kUint8, L.groups, L.N, ONNXL_AMD_LAYOUT_ONNX);
  return ONNXL_AMD_OK;
}

// The dense decode: y [N, K] of y's dtype, then the reference's output
// checks (quantization.cc:184-200, WriteFloat).
int DecodeCkpt(CkptPlan &p, CkptHost &h, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
               const onnxl_amd_tensor *scales, const onnxl_amd_tensor *g_idx, onnxl_amd_tensor *y,
               hipStream_t stream) {
  const CkptLayout &L0 = p.L;
  OLA_ENFORCE(y != nullptr, p.fmt, ": y is required.");
  CheckDescriptor(y, "y");
  const int32_t odt = y->data_type;
  OLA_ENFORCE(odt == kFloat || odt == kDouble || odt == kFloat16 || odt == kBfloat16,
              "Quantization requires FLOAT, DOUBLE, FLOAT16 or BFLOAT16.");
  OLA_ENFORCE(y->rank == 2 && y->dims[0] == L0.N && y->dims[1] == L0.K, p.fmt, ": y must be [N, K] = [", L0.N,
              ", ", L0.K, "].");
  if (odt == kFloat16 || odt == kBfloat16) {
    // the largest magnitude that rounds to a finite value, plus the tie that rounds away
    const double limit = odt == kFloat16 ? 65520.0 : std::ldexp(1.99609375, 127);
    CheckCkptMagnitudes(p, qweight, h, limit, "Dequantization output dtype overflow.");
  }
  Ctx();
  Staging st(stream, 0, {qweight, qzeros, scales, g_idx}, {y});
  CkptLayout L = L0;
  L.qweight = static_cast<const uint8_t *>(st.In(qweight));
  L.qzeros = static_cast<const uint8_t *>(st.In(qzeros));
  LaunchCkptDecode(L, st.In(scales), p.scale_type,
                   L.kind == kAwqFast ? static_cast<const uint16_t *>(st.In(qzeros)) : nullptr,
                   g_idx && p.trivial_groups == false ? static_cast<const int32_t *>(st.In(g_idx)) : nullptr, odt,
                   st.Out(y), stream);
  OLA_HIP(hipGetLastError());
  st.Finish();
  return ONNXL_AMD_OK;
}

void CheckAwqTensors(const CkptPlan &p, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                     const onnxl_amd_tensor *scales) {
  CheckCkptTensor(p, qweight, p.word_type, p.qweight_shape, "qweight");
  CheckCkptTensor(p, qzeros, p.zeros_type, p.qzeros_shape, p.zeros_name);
  CheckCkptTensor(p, scales, p.scale_type, p.scales_shape, "scales");
}

CkptPlan AwqFromTensors(const char *variant, const onnxl_amd_tensor *scales, int64_t K, int64_t N, int64_t bits,
                        int64_t group) {
  OLA_ENFORCE(!Absent(scales), "AWQ missing scales.");
  return PlanAwq(variant, K, N, bits, group, scales->data_type);
}

CkptPlan GptqFromTensors(const char *format, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                         const onnxl_amd_tensor *scales, const onnxl_amd_tensor *g_idx, int64_t K, int64_t N,
                         int64_t bits, int64_t group) {
  OLA_ENFORCE(!Absent(scales), "GPTQ missing scales.");
  OLA_ENFORCE(!Absent(qweight), "GPTQ missing tensor qweight.");
  CkptPlan p = PlanGptq(format, K, N, bits, group, qweight->data_type, scales->data_type);
  CheckCkptTensor(p, qweight, p.word_type, p.qweight_shape, "qweight");
  CheckCkptTensor(p, qzeros, p.zeros_type, p.qzeros_shape, "qzeros");
  CheckCkptTensor(p, scales, p.scale_type, p.scales_shape, "scales");
  CheckCkptTensor(p, g_idx, kInt32, {K}, "g_idx");
  return p;
}

int PrepareAwq(const char *variant, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
               const onnxl_amd_tensor *scales, int64_t K, int64_t N, int64_t bits, int64_t group,
               onnxl_amd_tensor *weight, onnxl_amd_tensor *scale, onnxl_amd_tensor *zero_point, hipStream_t stream) {
  CkptPlan p = AwqFromTensors(variant, scales, K, N, bits, group);
  CheckAwqTensors(p, qweight, qzeros, scales);
  CheckAwqValues(p, qweight, qzeros, scales);
  if (p.L.kind == kAwqFast)
    throw Unsupported("AWQ gemv_fast / llm-awq: float zero terms have no fused DequantizeLinear kernel "
                      "(onnxl_amd_dequantize_awq decodes them)");
  return PrepareCkpt("prepare_awq", p, qweight, qzeros, scales, weight, scale, zero_point, stream);
}

int PrepareGptq(const char *format, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                const onnxl_amd_tensor *scales, const onnxl_amd_tensor *g_idx, int64_t K, int64_t N, int64_t bits,
                int64_t group, onnxl_amd_tensor *weight, onnxl_amd_tensor *scale, onnxl_amd_tensor *zero_point,
                hipStream_t stream) {
  CkptPlan p = GptqFromTensors(format, qweight, qzeros, scales, g_idx, K, N, bits, group);
  CheckGptqValues(p, qweight, qzeros, scales, g_idx);
  if (K % p.L.group != 0)
    throw Unsupported(Cat("GPTQ: K = ", K, " is not a multiple of group_size ", group,
                          " (a partial last group has no fused kernel)"));
  if (!p.trivial_groups)
    throw Unsupported("GPTQ: a group map other than g_idx[k] = k / group_size (act-order) has no fused kernel "
                      "(onnxl_amd_dequantize_gptq decodes it)");
  return PrepareCkpt("prepare_gptq", p, qweight, qzeros, scales, weight, scale, zero_point, stream);
}

// ---------------------------------------------------------------------------
// BitBLAS row-packed weights (onnx_core/runtime/bitblas.cc): the geometry of
// Geometry (:38-84) in the reference's order, CheckTensor (:101-106),
// CheckScales (:228-237), then the GPTQ affine values the reference
// reconstructs through (Affine, :251-290; gptq.cc:222-228): code (k, n) the
// k-th `bits`-bit field of row n of qweight (XOR the midpoint for codes from
// symmetric GPTQ, whose zero is the midpoint), zero (g, n) the n-th field of
// qzeros row g, scale (g, n) = scales[n, g].

CkptPlan PlanBitblas(const char *method, int64_t K, int64_t N, int64_t bits, int64_t group, int32_t symmetric,
                     int32_t scale_type) {
  const std::string m = method ? method : "";
  OLA_ENFORCE(m == "gptq" || m == "awq", "BitBLAS requires an explicit GPTQ/AWQ originating method.");
  OLA_ENFORCE(K > 0 && N > 0 && K % 32 == 0 && N % (m == "gptq" ? 32 : 16) == 0,
              "BitBLAS row-packed checkpoint requires aligned, unpadded dimensions.");
  OLA_ENFORCE(bits >= 2 && bits <= 8 && (m == "awq" || bits == 2 || bits == 4 || bits == 8),
              "BitBLAS unsupported bit width for the originating method.");
  OLA_ENFORCE(group == -1 || group == K || group == 32 || group == 64 || group == 128,
              "BitBLAS unsupported group size.");
  const int64_t eff = group == -1 ? K : group;
  OLA_ENFORCE(K % eff == 0, "BitBLAS incomplete group.");
  constexpr int64_t kLimit = int64_t(1) << 30;
  OLA_ENFORCE(K <= kLimit / 4 / N, "BitBLAS logical FLOAT weights exceed max_bytes.");
  OLA_ENFORCE(scale_type == kFloat16, "BitBLAS row-packed checkpoint reader requires FP16 scales.");
  CkptPlan p;
  p.fmt = "BitBLAS";
  CkptLayout &L = p.L;
  L.kind = kBitblas, L.K = K, L.N = N, L.bits = (int)bits, L.width = 1;
  L.group = eff, L.groups = K / eff, L.padded = L.groups;
  L.signed_codes = m == "gptq" && symmetric != 0;
  p.word_type = p.zeros_type = kInt8;
  p.scale_type = kFloat16;
  p.qweight_shape = {N, K / 8 * bits};
  p.scales_shape = {N, L.groups};
  p.qzeros_shape = L.signed_codes ? Shape{0} : Shape{L.groups, N / 8 * bits};
  const int64_t zb = L.signed_codes ? 0 : L.groups * (N / 8 * bits);
  OLA_ENFORCE(N * (K / 8 * bits) + 2 * N * L.groups + zb <= kLimit, "BitBLAS checkpoint exceeds max_bytes.");
  return p;
}

CkptPlan BitblasFromTensors(const char *method, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *scales,
                            const onnxl_amd_tensor *qzeros, int64_t K, int64_t N, int64_t bits, int64_t group,
                            int32_t symmetric) {
  OLA_ENFORCE(!Absent(scales), "BitBLAS missing scales.");
  CkptPlan p = PlanBitblas(method, K, N, bits, group, symmetric, scales->data_type);
  auto check = [&](const onnxl_amd_tensor *t, int32_t type, const Shape &shape, const char *name) {
    const int64_t bytes = NumElements(shape) * ElementSize(type);
    const bool empty_ok = bytes == 0 && Absent(t);
    OLA_ENFORCE(empty_ok || (!Absent(t) && t->data_type == type && ShapeOf(*t) == shape && t->size_bytes == bytes &&
                             (bytes == 0 || t->data != nullptr)),
                "BitBLAS invalid tensor type, shape or extent: ", name, ".");
    if (!Absent(t)) CheckDescriptor(t, name);
  };
  check(qweight, kInt8, p.qweight_shape, "qweight");
  check(scales, kFloat16, p.scales_shape, "scales");
  check(qzeros, kInt8, p.qzeros_shape, "qzeros");
  return p;
}

// CheckScales: every FP16 scale finite and positive (the stored [N, groups]
// order); the zero fields read for the output-range scan.
CkptHost CheckBitblasValues(CkptPlan &p, const onnxl_amd_tensor *qzeros, const onnxl_amd_tensor *scales) {
  CkptHost h;
  h.scales = ReadFloats(*scales);
  for (float v : h.scales) OLA_ENFORCE(std::isfinite(v) && v > 0.f, "BitBLAS nonfinite or nonpositive scale.");
  if (!p.L.signed_codes) {
    h.qzeros.resize((size_t)NumElements(*qzeros));
    ReadBytes(*qzeros, 0, h.qzeros.data(), h.qzeros.size());
  }
  return h;
}

// ---------------------------------------------------------------------------
// bitsandbytes weights (onnx_core/runtime/bitsandbytes.cc): the geometry and
// tensor checks of Geometry / CheckTensor (:222-258, :317-321) on the parsed
// state, CheckParameters (:348-379), the reconstruction (:502-539) and the
// prepared fused MatMul.

struct BnbState {
  int32_t format;
  int64_t rows, cols, block, nested_block, count, blocks;
  float offset;
};

// `bytes` of a descriptor's payload to host, ordered on `stream`.
void ReadOnStream(hipStream_t stream, const onnxl_amd_tensor &t, void *dst, size_t bytes) {
  if (bytes == 0) return;
  if (t.location == ONNXL_AMD_HOST) {
    std::memcpy(dst, t.data, bytes);
    return;
  }
  OLA_HIP(hipMemcpyAsync(dst, t.data, bytes, hipMemcpyDeviceToHost, stream));
  OLA_HIP(hipStreamSynchronize(stream));
}

void BnbTensor(const onnxl_amd_tensor *t, const char *name, int32_t dtype, int64_t elements, int64_t bytes) {
  OLA_ENFORCE(!Absent(t) && t->data_type == dtype && NumElements(*t) == elements && t->size_bytes == bytes &&
                  t->data != nullptr,
              "bitsandbytes invalid tensor type, shape or byte extent: ", name, ".");
  CheckDescriptor(t, name);
}

BnbState BnbGeometry(int32_t format, int64_t rows, int64_t cols, int64_t block, int64_t nested_block, float offset,
                     const onnxl_amd_tensor *weight, const onnxl_amd_tensor *absmax,
                     const onnxl_amd_tensor *quant_map, const onnxl_amd_tensor *nested_absmax,
                     const onnxl_amd_tensor *nested_quant_map) {
  BnbState g{format, rows, cols, block, nested_block, 0, 0, offset};
  OLA_ENFORCE(rows > 0 && cols > 0 && rows <= (int64_t(1) << 40) / cols,
              "bitsandbytes invalid dimensions or max_bytes.");
  g.count = rows * cols;
  if (format == 2) {
    OLA_ENFORCE(block == 0 && nested_block == 0, "bitsandbytes invalid INT8 metadata.");
    g.blocks = rows;
    BnbTensor(weight, "weight", kInt8, g.count, g.count);
    BnbTensor(absmax, "weight_scb", kFloat, rows, rows * 4);
    return g;
  }
  const bool pow2 = block >= 32 && block <= 4096 && (block & (block - 1)) == 0;
  OLA_ENFORCE((format == 0 || format == 1) && pow2 && (nested_block == 0 || nested_block == 256),
              "bitsandbytes unsupported four-bit state.");
  g.blocks = (g.count + block - 1) / block;
  BnbTensor(weight, "weight", kUint8, (g.count + 1) / 2, (g.count + 1) / 2);
  if (nested_block)
    BnbTensor(absmax, "weight_absmax", kUint8, g.blocks, g.blocks);
  else
    BnbTensor(absmax, "weight_absmax", kFloat, g.blocks, g.blocks * 4);
  BnbTensor(quant_map, "weight_quant_map", kFloat, 16, 64);
  if (nested_block) {
    const int64_t nb = (g.blocks + 255) / 256;
    BnbTensor(nested_absmax, "weight_nested_absmax", kFloat, nb, nb * 4);
    BnbTensor(nested_quant_map, "weight_nested_quant_map", kFloat, 256, 1024);
    OLA_ENFORCE(std::isfinite(offset) && offset >= 0.f, "bitsandbytes invalid nested offset.");
  }
  return g;
}

// The format's 16 code values (nf4 as float, fp4 over 12), native index order.
float BnbTableValue(int32_t format, int j) {
  static const double nf4[16] = {-1, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                                 -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0,
                                 0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
                                 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
                                 0.7229568362236023, 1};
  static const float fp4[16] = {0.f, 1.f / 192, 2.f / 3, 1.f,  1.f / 3,  0.5f,  1.f / 6,  0.25f,
                                0.f, -1.f / 192, -2.f / 3, -1.f, -1.f / 3, -0.5f, -1.f / 6, -0.25f};
  return format == 0 ? (float)nf4[j] : fp4[j];
}

// Device work of one bitsandbytes call: its staged inputs, the resolved
// scales (in `scales`, or in the call's scratch) and the flag word.
struct BnbRun {
  BnbParams p{};
  std::unique_ptr<Staging> st;
  onnxl_amd_tensor flag_desc{};

  BnbRun(hipStream_t stream, const BnbState &g, size_t extra, const onnxl_amd_tensor *weight,
         const onnxl_amd_tensor *absmax, const onnxl_amd_tensor *nested_absmax,
         const onnxl_amd_tensor *nested_quant_map, onnxl_amd_tensor *y, float *scales) {
    const size_t sc_bytes = scales ? 0 : Scratch::Round((size_t)g.blocks * 4);
    st.reset(new Staging(stream, sc_bytes + 256 + extra, {weight, absmax, nested_absmax, nested_quant_map}, {y}));
    char *x = static_cast<char *>(st->Extra());
    p.scales = scales ? scales : reinterpret_cast<float *>(x);
    p.flag = reinterpret_cast<unsigned *>(x + sc_bytes);
    p.format = g.format;
    p.rows = g.rows;
    p.cols = g.cols;
    p.block_shift = g.format == 2 ? 0 : __builtin_ctzll((unsigned long long)g.block);
    p.nested = g.nested_block != 0;
    p.offset = g.offset;
    p.blocks = g.blocks;
    p.codes = static_cast<const uint8_t *>(st->In(weight));
    p.absmax = st->In(absmax);
    p.nested_absmax = static_cast<const float *>(st->In(nested_absmax));
    p.nested_map = static_cast<const float *>(st->In(nested_quant_map));
    hipLaunchKernelGGL(ZeroWordsKernel, dim3(1), dim3(256), 0, stream, p.flag, (size_t)1);
    flag_desc.data_type = kInt32;
    flag_desc.rank = 1;
    flag_desc.dims[0] = 1;
    flag_desc.data = p.flag;
    flag_desc.size_bytes = 4;
    flag_desc.location = ONNXL_AMD_DEVICE;
  }
  void *ExtraAfterFlag() const { return reinterpret_cast<char *>(p.flag) + 256; }
  unsigned Flag(hipStream_t stream) {
    unsigned v = 0;
    ReadOnStream(stream, flag_desc, &v, 4);
    return v;
  }
};

// CheckParameters in the reference's order: the FLOAT maxima (absmax, or the
// int8 row maxima) on the device, the quant map (finite, then canonical, entry
// by entry), the nested tables, then every nested scale (the device flags).
void BnbCheck(hipStream_t stream, const BnbState &g, BnbRun &run, const onnxl_amd_tensor *quant_map,
              const onnxl_amd_tensor *nested_absmax, const onnxl_amd_tensor *nested_quant_map) {
  LaunchBnbScales(run.p, stream);
  const unsigned flag = run.Flag(stream);
  constexpr const char *kBadTable = "bitsandbytes nonfinite table or invalid absmax.";
  OLA_ENFORCE(!(flag & kBnbBadAbsmax), kBadTable);
  if (g.format != 2) {
    float qm[16];
    ReadOnStream(stream, *quant_map, qm, 64);
    for (int j = 0; j < 16; ++j) OLA_ENFORCE(std::isfinite(qm[j]), kBadTable);
    if (g.nested_block) {
      std::vector<float> na((size_t)NumElements(*nested_absmax)), nm(256);
      ReadOnStream(stream, *nested_absmax, na.data(), na.size() * 4);
      ReadOnStream(stream, *nested_quant_map, nm.data(), 1024);
      for (float v : na) OLA_ENFORCE(std::isfinite(v) && v >= 0.f, kBadTable);
      for (float v : nm) OLA_ENFORCE(std::isfinite(v), kBadTable);
    }
    for (int j = 0; j < 16; ++j)
      OLA_ENFORCE(qm[j] == BnbTableValue(g.format, j), "bitsandbytes noncanonical NF4/FP4 table.");
  }
  OLA_ENFORCE(!(flag & kBnbBadScale), "bitsandbytes nonfinite reconstruction.");
}

int DequantizeBnb(int32_t format, int64_t rows, int64_t cols, int64_t block, int64_t nested_block, float offset,
                  const onnxl_amd_tensor *weight, const onnxl_amd_tensor *absmax, const onnxl_amd_tensor *quant_map,
                  const onnxl_amd_tensor *nested_absmax, const onnxl_amd_tensor *nested_quant_map,
                  onnxl_amd_tensor *y, hipStream_t stream) {
  const BnbState g =
      BnbGeometry(format, rows, cols, block, nested_block, offset, weight, absmax, quant_map, nested_absmax,
                  nested_quant_map);
  OLA_ENFORCE(y && (y->data_type == kFloat || y->data_type == kFloat16 || y->data_type == kBfloat16),
              "bitsandbytes unsupported reconstruction_dtype.");
  CheckDescriptor(y, "y");
  OLA_ENFORCE(y->rank == 2 && y->dims[0] == rows && y->dims[1] == cols &&
                  y->size_bytes == g.count * (y->data_type == kFloat ? 4 : 2),
              "bitsandbytes: y must be [rows, cols] of reconstruction_dtype.");
  BnbRun run(stream, g, 0, weight, absmax, nested_absmax, nested_quant_map, y, nullptr);
  BnbCheck(stream, g, run, quant_map, nested_absmax, nested_quant_map);
  LaunchBnbDecode(run.p, y->data_type, run.st->Out(y), stream);
  OLA_ENFORCE(!(run.Flag(stream) & kBnbBadValue), "bitsandbytes nonfinite reconstruction.");
  run.st->Finish();
  return ONNXL_AMD_OK;
}

int PrepareBnb(int32_t format, int64_t rows, int64_t cols, int64_t block, int64_t nested_block, float offset,
               const onnxl_amd_tensor *weight, const onnxl_amd_tensor *absmax, const onnxl_amd_tensor *quant_map,
               const onnxl_amd_tensor *nested_absmax, const onnxl_amd_tensor *nested_quant_map,
               int32_t reconstruction_dtype, onnxl_amd_tensor *scales, hipStream_t stream) {
  const BnbState g =
      BnbGeometry(format, rows, cols, block, nested_block, offset, weight, absmax, quant_map, nested_absmax,
                  nested_quant_map);
  OLA_ENFORCE(reconstruction_dtype == kFloat || reconstruction_dtype == kFloat16 ||
                  reconstruction_dtype == kBfloat16,
              "bitsandbytes unsupported reconstruction_dtype.");
  OLA_ENFORCE(scales && scales->location == ONNXL_AMD_DEVICE && scales->data != nullptr &&
                  scales->size_bytes >= g.blocks * 4,
              "prepare_bitsandbytes: scales must be a device buffer of ", g.blocks * 4, " bytes.");
  BnbRun run(stream, g, 0, weight, absmax, nested_absmax, nested_quant_map, nullptr,
             static_cast<float *>(scales->data));
  BnbCheck(stream, g, run, quant_map, nested_absmax, nested_quant_map);
  // every value of the weight reconstructed in the dtype, nothing written
  BnbParams check = run.p;
  LaunchBnbDecode(check, reconstruction_dtype, nullptr, stream);
  OLA_ENFORCE(!(run.Flag(stream) & kBnbBadValue), "bitsandbytes nonfinite reconstruction.");
  scales->data_type = kFloat;
  scales->rank = 1;
  scales->dims[0] = g.blocks;
  run.st->Finish();
  return ONNXL_AMD_OK;
}

int64_t BnbBlocks(int32_t format, int64_t rows, int64_t cols, int64_t block) {
  if (format == 2) return rows;
  return block > 0 ? (rows * cols + block - 1) / block : 0;
}

int BnbMatMul(const onnxl_amd_tensor *a, int32_t format, int64_t rows, int64_t cols, int64_t block,
              const onnxl_amd_tensor *weight, const onnxl_amd_tensor *scales, onnxl_amd_tensor *y,
              hipStream_t stream) {
  constexpr const char *kName = "bitsandbytes_matmul";
  OLA_ENFORCE(!Absent(a) && y, kName, ": a and y are required.");
  CheckDescriptor(a, "a");
  CheckDescriptor(y, "y");
  OLA_ENFORCE(a->data_type == kFloat16 || a->data_type == kBfloat16, kName, ": a must be FLOAT16 or BFLOAT16.");
  OLA_ENFORCE(a->rank >= 1 && a->dims[a->rank - 1] == cols, kName, ": the last dimension of a must be cols.");
  OLA_ENFORCE(format >= 0 && format <= 2 && rows > 0 && cols > 0 &&
                  (format == 2 ? block == 0
                               : block >= 32 && block <= 4096 && (block & (block - 1)) == 0),
              kName, ": unsupported format or block.");
  const int64_t count = rows * cols, blocks = BnbBlocks(format, rows, cols, block);
  OLA_ENFORCE(!Absent(weight) && weight->size_bytes == (format == 2 ? count : (count + 1) / 2) &&
                  (weight->data_type == (format == 2 ? kInt8 : kUint8)),
              kName, ": weight does not match the format and shape.");
  OLA_ENFORCE(!Absent(scales) && scales->data_type == kFloat && scales->size_bytes >= blocks * 4, kName,
              ": scales must be the FLOAT scales onnxl_amd_prepare_bitsandbytes wrote.");
  CheckDescriptor(weight, "weight");
  CheckDescriptor(scales, "scales");
  const int64_t M = NumElements(*a) / cols;
  OLA_ENFORCE(y->data_type == a->data_type && y->rank == a->rank && y->dims[y->rank - 1] == rows &&
                  NumElements(*y) == M * rows && y->size_bytes == M * rows * 2,
              kName, ": y must be a's leading dims x rows, a's dtype.");
  if (M == 0) return ONNXL_AMD_OK;
  const bool fp16 = a->data_type == kFloat16;
  auto aligned = [](const onnxl_amd_tensor *t) {
    return t->location == ONNXL_AMD_HOST || reinterpret_cast<uintptr_t>(t->data) % 16 == 0;
  };
  const bool gemv = fp16 && (format == 0 || format == 1) && M <= 4 && cols % 32 == 0 && cols % block == 0 &&
                    aligned(a) && aligned(weight) && count / 2 < (int64_t(1) << 40);
  const size_t w_bytes = gemv ? 0 : (size_t)count * 2;
  Staging st(stream, w_bytes + 256, {a, weight, scales}, {y});
  const uint16_t *ad = static_cast<const uint16_t *>(st.In(a));
  const uint8_t *codes = static_cast<const uint8_t *>(st.In(weight));
  const float *sc = static_cast<const float *>(st.In(scales));
  uint16_t *yd = static_cast<uint16_t *>(st.Out(y));
  if (gemv) {
    LaunchBnbGemv(format, ad, codes, sc, M, rows, cols, block, yd, stream);
  } else {
    // the weight decoded to [rows, cols] in a's dtype, then Y = A W^T
    BnbParams p{};
    p.format = format;
    p.rows = rows;
    p.cols = cols;
    p.block_shift = format == 2 ? 0 : __builtin_ctzll((unsigned long long)block);
    p.blocks = blocks;
    p.codes = codes;
    p.scales = const_cast<float *>(sc);
    char *x = static_cast<char *>(st.Extra());
    p.flag = reinterpret_cast<unsigned *>(x + w_bytes);  // values were checked by the preparation
    uint16_t *w = reinterpret_cast<uint16_t *>(x);
    LaunchBnbDecode(p, a->data_type, w, stream);
    HMatMulParams h{};
    h.A = ad;
    h.B = w;
    h.Y = yd;
    h.M = M;
    h.N = rows;
    h.K = cols;
    h.batch = 1;
    h.bf16 = fp16 ? 0 : 1;
    LaunchHMatMulBT(h, stream);
  }
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// GPTQModel FP8 weights (onnx_core/runtime/gptqmodel_fp8.cc): Geometry
// (:58-101) in the reference's order with DecodeValues' 1 << 30 byte limit,
// the tensor check of ImportGptqModelFp8Weights (:246-254), CheckData
// (:164-173) and the reconstruction (:160-162) on the device, WriteFloat's
// output check.

bool QqqDtype(int32_t dt);

// ---------------------------------------------------------------------------
// MX and NVFP4 weights (onnx_core/runtime/quantization.cc): the checks of
// ImportMxfp4Weights (:2193-2212), ImportMxfp8Weights (:2214-2229),
// ImportMxfp6E2m3Weights (:2279-2298) and ImportNvfp4Weights (:2099-2118)
// in their order (matrix, packed columns, Geometry, the two tensors), then
// the Validate*Reconstruction walks (:1350-1359, :1477-1486, :1608-1613,
// :1714-1720) on the device with the first failing group and element
// raised as the reference words it, then WriteFloat's output range.

int DequantizeMx(const char *format_name, const onnxl_amd_tensor *weight, const onnxl_amd_tensor *scale,
                 float global, onnxl_amd_tensor *y, hipStream_t stream) {
  const std::string f = format_name ? format_name : "";
  int fmt;
  if (f == "mxfp4") fmt = kMxFp4;
  else if (f == "mxfp6_e2m3") fmt = kMxFp6E2M3;
  else if (f == "mxfp8") fmt = kMxFp8;
  else if (f == "nvfp4") fmt = kMxNvfp4;
  else throw Unsupported(Cat("MX weights: unknown format '", f, "' (mxfp4, mxfp6_e2m3, mxfp8 or nvfp4)."));
  // the reference's names for the format in its messages
  const char *tag = fmt == kMxFp4 ? "MXFP4 WEIGHT" : (fmt == kMxNvfp4 ? "NVFP4 WEIGHT"
                                                     : (fmt == kMxFp8 ? "MXFP8" : "MXFP6 E2M3"));
  const int group = fmt == kMxNvfp4 ? 16 : 32;
  constexpr int64_t kMax = std::numeric_limits<int64_t>::max();
  OLA_ENFORCE(!Absent(weight) && weight->rank == 2, tag,
              fmt == kMxFp8 ? " weights must be a matrix." : " packed weights must be a matrix.");
  const int64_t rows = weight->dims[0], wcols = weight->dims[1];
  int64_t cols;
  if (fmt == kMxFp8) {
    cols = wcols;
  } else if (fmt == kMxFp6E2M3) {
    OLA_ENFORCE(wcols > 0 && wcols % 3 == 0 && wcols / 3 <= kMax / 4, "Invalid MXFP6 E2M3 packed columns.");
    cols = wcols / 3 * 4;
  } else {
    OLA_ENFORCE(wcols > 0 && wcols <= kMax / 2, tag, " packed columns overflow.");
    cols = wcols * 2;
  }
  // Geometry
  OLA_ENFORCE(rows > 0 && cols > 0 && cols % group == 0, tag, " requires positive [rows,cols] with cols divisible by ",
              group, ".");
  OLA_ENFORCE(rows <= kMax / cols, tag, " element count exceeds INT64.");
  const int64_t count = rows * cols;
  const int64_t code_bytes = fmt == kMxFp8 ? count : (fmt == kMxFp6E2M3 ? count / 4 * 3 : count / 2);
  const int64_t scale_bytes = count / group;
  // ValidateMxfp4Tensor / ValidateNvfp4Tensor / ValidateMxTensor
  const std::string bad = fmt == kMxFp4 || fmt == kMxNvfp4 ? Cat("Invalid ", tag, " tensor type, shape or storage.")
                                                          : std::string("Invalid MX tensor type, shape or storage.");
  const int32_t code_type = fmt == kMxFp8 ? kFloat8E4M3FN : kUint8;
  OLA_ENFORCE(weight->data_type == code_type && weight->size_bytes == code_bytes && weight->data != nullptr, bad);
  const int32_t scale_type = fmt == kMxNvfp4 ? kFloat8E4M3FN : kUint8;
  OLA_ENFORCE(!Absent(scale) && scale->data_type == scale_type && scale->rank == 2 && scale->dims[0] == rows &&
                  scale->dims[1] == cols / group && scale->size_bytes == scale_bytes && scale->data != nullptr,
              bad);
  CheckDescriptor(weight, "weight");
  CheckDescriptor(scale, "weight_scale");
  OLA_ENFORCE(y != nullptr && QqqDtype(y->data_type), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16.");
  CheckDescriptor(y, "y");
  const int64_t width = y->data_type == kDouble ? 8 : (y->data_type == kFloat ? 4 : 2);
  OLA_ENFORCE(y->rank == 2 && y->dims[0] == rows && y->dims[1] == cols && y->size_bytes == count * width &&
                  y->data != nullptr,
              "MX weights: y must be [rows, cols] of its dtype.");
  Ctx();
  Staging st(stream, 256, {weight, scale}, {y});
  MxParams p{};
  p.count = count;
  p.codes = static_cast<const uint8_t *>(st.In(weight));
  p.scales = static_cast<const uint8_t *>(st.In(scale));
  p.global = global;
  void *out = st.Out(y);
  p.aligned = (reinterpret_cast<uintptr_t>(p.codes) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0) ? 1 : 0;
  p.first = static_cast<uint64_t *>(st.Extra());
  p.flag = reinterpret_cast<unsigned *>(p.first + 1);
  hipLaunchKernelGGL(ZeroWordsKernel, dim3(1), dim3(256), 0, stream, reinterpret_cast<unsigned *>(p.first), (size_t)3);
  LaunchMxDecode(p, fmt, y->data_type, out, stream);
  OLA_HIP(hipGetLastError());
  onnxl_amd_tensor fd{};
  fd.data_type = kInt32, fd.rank = 1, fd.dims[0] = 3, fd.data = p.first, fd.size_bytes = 12;
  fd.location = ONNXL_AMD_DEVICE;
  uint32_t words[3] = {};
  ReadOnStream(stream, fd, words, 12);
  const uint64_t first = (uint64_t)words[0] | ((uint64_t)words[1] << 32);
  if (first != 0) {
    const uint64_t key = ~first;
    const int64_t g = (int64_t)(key / 128);
    const int step = (int)(key % 128), e = (step - 3) / 2;
    const bool code = step >= 3 && (step - 3) % 2 == 0;
    switch (fmt) {
    case kMxFp4:  // Mxfp4Scale :1458-1461, Mxfp4Reconstruct :1463-1470
      OLA_ENFORCE(step != 0, "MXFP4 WEIGHT E8M0 scale is NaN in group ", g, ".");
      OLA_ENFORCE(false, "MXFP4 WEIGHT reconstruction overflow or nonfinite value in group ", g, ", element ", e, ".");
      break;
    case kMxNvfp4:  // Nvfp4EffectiveScale :1322-1333, Nvfp4Reconstruct :1335-1342
      OLA_ENFORCE(step != 0, "NVFP4 WEIGHT scales must be positive and finite in group ", g, ".");
      OLA_ENFORCE(step != 1, "NVFP4 WEIGHT effective scale overflow or nonfinite value in group ", g, ".");
      OLA_ENFORCE(step != 2, "NVFP4 WEIGHT effective scale rounds to zero in group ", g, ".");
      OLA_ENFORCE(false, "NVFP4 WEIGHT reconstruction overflow or nonfinite value in group ", g, ", element ", e, ".");
      break;
    case kMxFp8:  // Mxfp8Scale :1591-1595, Mxfp8Reconstruct :1597-1600, RoundFloat :41-45
      OLA_ENFORCE(step != 0, "MXFP8 E8M0 scale must not be NaN.");
      OLA_ENFORCE(!code, "MXFP8 E4M3FN weight must not be NaN.");
      OLA_ENFORCE(false, "FLOAT reconstruction overflow or nonfinite value.");
      break;
    default:  // Mxfp6E2m3Scale :1700-1703, RoundFloat :41-45
      OLA_ENFORCE(step != 0, "MXFP6 E2M3 E8M0 scale byte 255 is invalid.");
      OLA_ENFORCE(false, "FLOAT reconstruction overflow or nonfinite value.");
    }
  }
  OLA_ENFORCE(!(words[2] & kMxBadOutput), "Dequantization output dtype overflow.");
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// EXL3 weights (onnx_core/runtime/exl3.cc): Validate (:136-165) in the
// reference's order with its 1 << 30 byte limit (Geometry :45-69, CheckTensor
// :111-115, CheckScales :117-124 on the host, CheckMarker :126-134), then the
// reconstruction (:309-357) on the device and WriteFloat's range check.

int DequantizeExl3(const onnxl_amd_tensor *trellis, const onnxl_amd_tensor *suh, const onnxl_amd_tensor *svh,
                   const onnxl_amd_tensor *mcg, const onnxl_amd_tensor *mul1, onnxl_amd_tensor *y,
                   hipStream_t stream) {
  constexpr int64_t kLimit = int64_t(1) << 30, kMax = std::numeric_limits<int64_t>::max();
  OLA_ENFORCE(!Absent(trellis), "EXL3 missing tensor trellis.");
  OLA_ENFORCE(trellis->rank == 3 && trellis->dims[0] > 0 && trellis->dims[1] > 0 && trellis->dims[0] <= kMax / 16 &&
                  trellis->dims[1] <= kMax / 16 && trellis->dims[2] % 16 == 0,
              "EXL3 invalid trellis dimensions.");
  const int book = !Absent(mcg) ? 1 : (!Absent(mul1) ? 2 : 0);
  const int64_t k = trellis->dims[0] * 16, n = trellis->dims[1] * 16, rate = trellis->dims[2] / 16;
  // Geometry
  OLA_ENFORCE(k % 128 == 0 && n % 128 == 0, "EXL3 dimensions must be positive multiples of 128.");
  OLA_ENFORCE(rate >= 1 && rate <= 8, "EXL3 unsupported trellis rate.");
  OLA_ENFORCE(k <= kLimit / 4 / n, "EXL3 logical FLOAT weights exceed max_bytes.");
  const int64_t count = k * n, packed = count / 8 * rate, scales = 2 * k + 2 * n;
  OLA_ENFORCE(packed <= kLimit && scales <= kLimit - packed && (book == 0 || kLimit - packed - scales >= 4),
              "EXL3 checkpoint exceeds max_bytes.");
  OLA_ENFORCE(!(book == 1 && !Absent(mul1)), "EXL3 unexpected side tensors or conflicting codebooks.");
  OLA_ENFORCE(trellis->data_type == kInt16 && trellis->size_bytes == packed && trellis->data != nullptr,
              "EXL3 invalid tensor type, shape or byte extent.");
  CheckDescriptor(trellis, "trellis");
  // suh then svh: each tensor's check, then its values finite
  const onnxl_amd_tensor *side[2] = {suh, svh};
  const char *side_name[2] = {"suh", "svh"};
  const int64_t side_count[2] = {k, n};
  for (int i = 0; i < 2; ++i) {
    const onnxl_amd_tensor *t = side[i];
    OLA_ENFORCE(!Absent(t), "EXL3 missing tensor ", side_name[i], ".");
    OLA_ENFORCE(t->data_type == kFloat16 && t->rank == 1 && t->dims[0] == side_count[i] &&
                    t->size_bytes == side_count[i] * 2 && t->data != nullptr,
                "EXL3 invalid tensor type, shape or byte extent.");
    CheckDescriptor(t, side_name[i]);
    std::vector<uint16_t> h((size_t)side_count[i]);
    if (t->location != ONNXL_AMD_HOST) Ctx();
    ReadOnStream(stream, *t, h.data(), h.size() * 2);
    for (uint16_t b : h) OLA_ENFORCE((b & 0x7c00u) != 0x7c00u, "EXL3 nonfinite scale.");
  }
  if (book) {
    const onnxl_amd_tensor *m = book == 1 ? mcg : mul1;
    OLA_ENFORCE(m->data_type == kInt32 && m->rank == 0 && m->size_bytes == 4 && m->data != nullptr,
                "EXL3 invalid tensor type, shape or byte extent.");
    CheckDescriptor(m, book == 1 ? "mcg" : "mul1");
    uint32_t marker = 0;
    if (m->location != ONNXL_AMD_HOST) Ctx();
    ReadOnStream(stream, *m, &marker, 4);
    OLA_ENFORCE(marker == (book == 1 ? 0xcbac1fedu : 0x83dcd12du), "EXL3 invalid codebook marker.");
  }
  OLA_ENFORCE(y != nullptr && QqqDtype(y->data_type), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16.");
  CheckDescriptor(y, "y");
  const int64_t width = y->data_type == kDouble ? 8 : (y->data_type == kFloat ? 4 : 2);
  OLA_ENFORCE(y->rank == 2 && y->dims[0] == k && y->dims[1] == n && y->size_bytes == count * width &&
                  y->data != nullptr,
              "EXL3: y must be [k, n] of its dtype.");
  Ctx();
  Staging st(stream, 256, {trellis, suh, svh}, {y});
  Exl3Params p{};
  p.k = k, p.n = n, p.bits = (int)rate, p.book = book;
  p.trellis = static_cast<const uint16_t *>(st.In(trellis));
  p.suh = static_cast<const uint16_t *>(st.In(suh));
  p.svh = static_cast<const uint16_t *>(st.In(svh));
  p.flag = static_cast<unsigned *>(st.Extra());
  OLA_ENFORCE(reinterpret_cast<uintptr_t>(p.trellis) % 2 == 0 && reinterpret_cast<uintptr_t>(p.suh) % 2 == 0 &&
                  reinterpret_cast<uintptr_t>(p.svh) % 2 == 0,
              "EXL3: trellis, suh and svh must be 2-byte aligned.");
  void *out = st.Out(y);
  OLA_ENFORCE(reinterpret_cast<uintptr_t>(out) % width == 0, "EXL3: y must be aligned to its element size.");
  hipLaunchKernelGGL(ZeroWordsKernel, dim3(1), dim3(256), 0, stream, p.flag, (size_t)1);
  LaunchExl3Decode(p, y->data_type, out, stream);
  OLA_HIP(hipGetLastError());
  onnxl_amd_tensor fd{};
  fd.data_type = kInt32, fd.rank = 1, fd.dims[0] = 1, fd.data = p.flag, fd.size_bytes = 4;
  fd.location = ONNXL_AMD_DEVICE;
  unsigned flag = 0;
  ReadOnStream(stream, fd, &flag, 4);
  OLA_ENFORCE(!(flag & kExl3BadValue), "EXL3 nonfinite reconstruction.");
  OLA_ENFORCE(!(flag & kExl3BadOutput), "Dequantization output dtype overflow.");
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// VPTQ weights (onnx_core/runtime/vptq.cc): Layout (:52-129) in the
// reference's order with DecodeValues' 1 << 30 byte limit, the tensor checks
// of ImportVptqWeights (:359-367), CheckData (:203-240: the indices on the
// device, the outlier indices and the permutation on the host), the
// reconstruction on the device and WriteFloat's checks.

int64_t VptqPositive(int64_t v) {
  OLA_ENFORCE(v > 0, "VPTQ invalid positive dimension.");
  return v;
}

int DequantizeVptq(const onnxl_amd_vptq_config *cfg, const onnxl_amd_tensor *indices,
                   const onnxl_amd_tensor *centroids, const onnxl_amd_tensor *res_centroids,
                   const onnxl_amd_tensor *outlier_centroids, const onnxl_amd_tensor *outlier_indices,
                   const onnxl_amd_tensor *weight_scale, const onnxl_amd_tensor *weight_bias,
                   const onnxl_amd_tensor *perm, onnxl_amd_tensor *y, hipStream_t stream) {
  OLA_ENFORCE(cfg != nullptr, "VPTQ: config is required.");
  const onnxl_amd_vptq_config &w = *cfg;
  OLA_ENFORCE(!Absent(centroids), "VPTQ missing centroids.weight.");
  constexpr int64_t kLimit = int64_t(1) << 30;
  VptqParams p{};
  p.k = VptqPositive(w.in_features);
  p.n = VptqPositive(w.out_features);
  OLA_ENFORCE(p.k <= kLimit / 4 / p.n, "VPTQ FLOAT output exceeds max_bytes.");
  OLA_ENFORCE(!w.enable_perm || p.k <= int64_t(std::numeric_limits<int32_t>::max()) + 1,
              "VPTQ permutation exceeds INT32 channel range.");
  OLA_ENFORCE(w.bits >= 1 && w.bits <= 8 && w.vector_lens[1] > 0 && w.num_centroids[1] > 1 &&
                  w.num_res_centroids[1] != 1 && w.num_res_centroids[0] <= 1,
              "VPTQ unsupported codebook or outlier residual configuration.");
  const int32_t dtype = centroids->data_type;
  OLA_ENFORCE(dtype == kFloat || dtype == kFloat16 || dtype == kBfloat16, "VPTQ unsupported codebook dtype.");
  OLA_ENFORCE(std::isfinite(w.npercent) && w.npercent >= 0 && w.npercent < 100 && (w.norm_dim == 0 || w.norm_dim == 1),
              "VPTQ invalid constructor metadata.");
  const bool outlier = w.npercent > 0 && w.vector_lens[0] > 0 && w.num_centroids[0] > 1;
  OLA_ENFORCE(w.npercent == 0 || outlier, "VPTQ unusable outlier codebook.");
  const double initial = std::ceil((w.npercent / 100.0) * double(p.k));
  OLA_ENFORCE(initial >= 0 && initial < double(p.k), "VPTQ empty grouped layout.");
  p.outliers = outlier ? static_cast<int64_t>(initial) : 0;
  OLA_ENFORCE((w.group_size == -1 || w.group_size > 0) && (w.group_num == -1 || w.group_num > 0) &&
                  (w.group_size == -1 || w.group_num == -1),
              "VPTQ grouping knobs must be mutually exclusive.");
  if (w.group_num != -1) {
    p.groups = VptqPositive(w.group_num);
    OLA_ENFORCE(p.groups <= p.k - p.outliers, "VPTQ empty groups.");
    if (outlier) p.outliers += (p.k - p.outliers) % p.groups;
    p.columns = outlier ? (p.k - p.outliers) / p.groups : (p.k + p.groups - 1) / p.groups;
  } else {
    p.columns = w.group_size == -1 ? p.k - p.outliers : VptqPositive(w.group_size);
    p.groups = (p.k - p.outliers + p.columns - 1) / p.columns;
  }
  OLA_ENFORCE(p.groups > 0 && p.columns > 0 && p.groups * p.columns >= p.k - p.outliers,
              "VPTQ incomplete grouped layout.");
  auto bit_width = [](int64_t entries) {
    int b = 0;
    for (uint64_t v = (uint64_t)(entries - 1); v; v >>= 1) ++b;
    return b;
  };
  p.main_bits = bit_width(w.num_centroids[1]);
  p.residual_bits = w.num_res_centroids[1] > 1 ? bit_width(w.num_res_centroids[1]) : 0;
  OLA_ENFORCE(p.main_bits + p.residual_bits <= 32, "VPTQ index width exceeds INT32.");
  p.len1 = w.vector_lens[1];
  p.len0 = outlier ? w.vector_lens[0] : 1;
  p.nc1 = w.num_centroids[1];
  p.nr1 = w.num_res_centroids[1];
  p.vectors = (p.n + p.len1 - 1) / p.len1;
  p.words = (p.columns * (p.main_bits + p.residual_bits) + 31) / 32;
  p.dtype = dtype;
  p.norm_dim = (int)w.norm_dim;
  int64_t total = 0;
  auto spec = [&](const onnxl_amd_tensor *t, const char *name, int32_t dt, std::initializer_list<int64_t> shape) {
    int64_t bytes = dt == kInt32 || dt == kFloat ? 4 : 2;
    for (int64_t d : shape) bytes *= VptqPositive(d);
    OLA_ENFORCE(total <= kLimit && bytes <= kLimit - total, "VPTQ checkpoint exceeds max_bytes.");
    total += bytes;
    OLA_ENFORCE(!Absent(t), "VPTQ missing tensor ", name, ".");
    bool ok = t->data_type == dt && t->rank == (int32_t)shape.size() && t->size_bytes == bytes &&
              t->data != nullptr;
    int i = 0;
    for (int64_t d : shape) ok = ok && t->dims[i++] == d;
    OLA_ENFORCE(ok, "VPTQ invalid tensor type, shape or bytes: ", name, ".");
    CheckDescriptor(t, name);
  };
  spec(indices, "indices", kInt32, {p.groups, p.vectors, p.words});
  spec(centroids, "centroids.weight", dtype, {p.groups, p.nc1 * p.len1});
  if (p.residual_bits) spec(res_centroids, "res_centroids.weight", dtype, {p.groups, p.nr1 * p.len1});
  if (outlier) {
    spec(outlier_centroids, "outlier_centroids.weight", dtype, {1, w.num_centroids[0] * w.vector_lens[0]});
    spec(outlier_indices, "outlier_indices", kInt32, {1, (p.n + p.len0 - 1) / p.len0, p.outliers});
  }
  if (w.enable_norm) {
    spec(weight_scale, "weight_scale", dtype, {w.norm_dim == 0 ? p.k : p.n});
    spec(weight_bias, "weight_bias", dtype, {w.norm_dim == 0 ? p.k : p.n});
  }
  if (w.enable_perm) spec(perm, "perm", kInt32, {p.k});
  OLA_ENFORCE(y != nullptr && QqqDtype(y->data_type), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16.");
  CheckDescriptor(y, "y");
  const int64_t yw = y->data_type == kDouble ? 8 : (y->data_type == kFloat ? 4 : 2);
  OLA_ENFORCE(y->rank == 2 && y->dims[0] == p.n && y->dims[1] == p.k && y->size_bytes == p.n * p.k * yw &&
                  y->data != nullptr,
              "VPTQ: y must be [out_features, in_features] of its dtype.");
  Ctx();
  Staging st(stream, 256,
             {indices, centroids, p.residual_bits ? res_centroids : nullptr, outlier ? outlier_centroids : nullptr,
              outlier ? outlier_indices : nullptr, w.enable_norm ? weight_scale : nullptr,
              w.enable_norm ? weight_bias : nullptr, w.enable_perm ? perm : nullptr},
             {y});
  p.indices = static_cast<const uint32_t *>(st.In(indices));
  p.centroids = st.In(centroids);
  p.res_centroids = p.residual_bits ? st.In(res_centroids) : nullptr;
  p.outlier_centroids = outlier ? st.In(outlier_centroids) : nullptr;
  p.outlier_indices = outlier ? static_cast<const int32_t *>(st.In(outlier_indices)) : nullptr;
  p.scale = w.enable_norm ? st.In(weight_scale) : nullptr;
  p.bias = w.enable_norm ? st.In(weight_bias) : nullptr;
  p.perm = w.enable_perm ? static_cast<const int32_t *>(st.In(perm)) : nullptr;
  p.flag = static_cast<unsigned *>(st.Extra());
  hipLaunchKernelGGL(ZeroWordsKernel, dim3(1), dim3(256), 0, stream, p.flag, (size_t)3);
  onnxl_amd_tensor fd{};
  fd.data_type = kInt32, fd.rank = 1, fd.dims[0] = 3, fd.data = p.flag, fd.size_bytes = 12;
  fd.location = ONNXL_AMD_DEVICE;
  LaunchVptqIndexCheck(p, stream);
  OLA_HIP(hipGetLastError());
  unsigned flag = 0;
  ReadOnStream(stream, fd, &flag, 4);
  OLA_ENFORCE(!(flag & kVptqBadIndex), "VPTQ index exceeds codebook.");
  if (outlier) {
    std::vector<uint32_t> oi((size_t)NumElements(*outlier_indices));
    ReadOnStream(stream, *outlier_indices, oi.data(), oi.size() * 4);
    for (uint32_t v : oi)
      OLA_ENFORCE(v <= (uint32_t)std::numeric_limits<int32_t>::max() && (int64_t)v < w.num_centroids[0],
                  "VPTQ outlier index exceeds codebook.");
  }
  if (w.enable_perm) {
    std::vector<uint32_t> pv((size_t)p.k);
    ReadOnStream(stream, *perm, pv.data(), pv.size() * 4);
    std::vector<uint8_t> seen((size_t)p.k, 0);
    for (uint32_t v : pv) {
      OLA_ENFORCE(v <= (uint32_t)std::numeric_limits<int32_t>::max() && (int64_t)v < p.k && !seen[v],
                  "VPTQ invalid permutation.");
      seen[v] = 1;
    }
  }
  LaunchVptqDecode(p, y->data_type, st.Out(y), stream);
  OLA_HIP(hipGetLastError());
  unsigned first[3] = {0, 0, 0};  // WriteFloat's first failure in output order
  ReadOnStream(stream, fd, first, 12);
  if (first[1] || first[2]) {
    const bool nonfinite = first[1] && (!first[2] || ~first[1] < ~first[2]);
    OLA_ENFORCE(!nonfinite, "Dequantization produced a nonfinite value.");
    OLA_ENFORCE(false, "Dequantization output dtype overflow.");
  }
  st.Finish();
  return ONNXL_AMD_OK;
}

int DequantizeGptqFp8(int64_t k, int64_t n, const char *method_name, const int64_t *block, int32_t block_rank,
                      const onnxl_amd_tensor *weight, const onnxl_amd_tensor *scale, onnxl_amd_tensor *y,
                      hipStream_t stream) {
  constexpr int64_t kLimit = int64_t(1) << 30;
  OLA_ENFORCE(k > 0 && n > 0, "GPTQModel FP8 requires nonempty [N,K] weights and positive max_bytes.");
  OLA_ENFORCE(k <= kLimit / 4 / n, "GPTQModel FP8 logical FLOAT weights exceed max_bytes.");
  OLA_ENFORCE(!Absent(weight) && (weight->data_type == kFloat8E4M3FN || weight->data_type == kFloat8E4M3FNUZ ||
                                  weight->data_type == kFloat8E5M2 || weight->data_type == kFloat8E5M2FNUZ ||
                                  weight->data_type == kFloat8E8M0),
              "GPTQModel FP8 unsupported scalar format.");
  const std::string method = method_name ? method_name : "";
  OLA_ENFORCE(block_rank == 0 || (block_rank == 2 && block && block[0] > 0 && block[1] > 0),
              "GPTQModel FP8 invalid weight_block_size.");
  OLA_ENFORCE(method == "block" || block_rank == 0, "GPTQModel FP8 non-block scaling forbids weight_block_size.");
  GptqFp8Params p{};
  p.n = n, p.k = k, p.b0 = 1, p.b1 = 1;
  Shape scale_shape;
  if (method == "tensor") {
    p.method = 0;
  } else if (method == "row") {
    p.method = 1;
    scale_shape = {n};
  } else {
    OLA_ENFORCE(method == "block" && block_rank == 2 && n % block[0] == 0 && k % block[1] == 0,
                "GPTQModel FP8 requires divisible two-axis blocks.");
    p.method = 2;
    p.b0 = block[0], p.b1 = block[1], p.scale_cols = k / block[1];
    scale_shape = {n / block[0], k / block[1]};
  }
  const int64_t scales = NumElements(scale_shape);
  OLA_ENFORCE(n * k <= kLimit && scales * 4 <= kLimit - n * k, "GPTQModel FP8 checkpoint exceeds max_bytes.");
  OLA_ENFORCE(weight->rank == 2 && weight->dims[0] == n && weight->dims[1] == k && weight->size_bytes == n * k &&
                  weight->data != nullptr && !Absent(scale) && scale->data_type == kFloat &&
                  ShapeOf(*scale) == scale_shape && scale->size_bytes == scales * 4 && scale->data != nullptr,
              "GPTQModel FP8 invalid tensor dtype, shape or byte extent.");
  CheckDescriptor(weight, "weight");
  CheckDescriptor(scale, "weight_scale_inv");
  OLA_ENFORCE(y != nullptr && QqqDtype(y->data_type), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16.");
  CheckDescriptor(y, "y");
  const int64_t width = y->data_type == kDouble ? 8 : (y->data_type == kFloat ? 4 : 2);
  OLA_ENFORCE(y->rank == 2 && y->dims[0] == n && y->dims[1] == k && y->size_bytes == n * k * width &&
                  y->data != nullptr,
              "GPTQModel FP8: y must be [out_features, in_features] of its dtype.");
  Ctx();
  Staging st(stream, 256, {weight, scale}, {y});
  p.codes = static_cast<const uint8_t *>(st.In(weight));
  p.scales = static_cast<const float *>(st.In(scale));
  p.flag = static_cast<unsigned *>(st.Extra());
  hipLaunchKernelGGL(ZeroWordsKernel, dim3(1), dim3(256), 0, stream, p.flag, (size_t)1);
  LaunchGptqFp8Decode(p, weight->data_type, y->data_type, st.Out(y), stream);
  OLA_HIP(hipGetLastError());
  onnxl_amd_tensor fd{};
  fd.data_type = kInt32, fd.rank = 1, fd.dims[0] = 1, fd.data = p.flag, fd.size_bytes = 4;
  fd.location = ONNXL_AMD_DEVICE;
  unsigned flag = 0;
  ReadOnStream(stream, fd, &flag, 4);
  OLA_ENFORCE(!(flag & kGptqFp8BadScale), "GPTQModel FP8 inverse scales must be finite and positive.");
  OLA_ENFORCE(!(flag & kGptqFp8BadValue), "GPTQModel FP8 nonfinite weight or reconstruction.");
  OLA_ENFORCE(!(flag & kGptqFp8BadOutput), "Dequantization output dtype overflow.");
  st.Finish();
  return ONNXL_AMD_OK;
}

// ---------------------------------------------------------------------------
// QQQ weights (onnx_core/runtime/qqq.cc): the geometry and tensor checks of
// Geometry / CheckTensor (:38-56, :136-141) with limit 1 << 30 (DecodeValues,
// quantization.cc:2002-2008), CheckData (:204-218) and the reconstruction
// (:185-202) on the device, WriteFloat's output check
// (quantization.cc:184-201), and the fused operands.

struct QqqGeometry {
  int64_t k, n;
  bool grouped;
};

void QqqTensor(const onnxl_amd_tensor *t, const char *name, int32_t dtype, std::initializer_list<int64_t> shape,
               int64_t bytes) {
  bool ok = !Absent(t) && t->data_type == dtype && t->rank == (int32_t)shape.size() && t->size_bytes == bytes &&
            (bytes == 0 || t->data != nullptr);
  int d = 0;
  for (int64_t v : shape) ok = ok && t->dims[d++] == v;
  OLA_ENFORCE(ok, "QQQ invalid tensor type, shape or byte extent: ", name, ".");
  CheckDescriptor(t, name);
}

QqqGeometry QqqCheck(int64_t k, int64_t n, int64_t group, int64_t bits, const onnxl_amd_tensor *B,
                     const onnxl_amd_tensor *s_channel, const onnxl_amd_tensor *s_group) {
  constexpr int64_t kLimit = int64_t(1) << 30;
  OLA_ENFORCE(k > 0 && n > 0 && k % 64 == 0 && n % 64 == 0 && bits == 4 && (group == -1 || group == 128),
              "QQQ requires four-bit, unpadded dimensions divisible by 64 and group -1/128.");
  QqqGeometry g{k, n, group == 128 && k != 128};
  OLA_ENFORCE(!g.grouped || k % 128 == 0, "QQQ incomplete 128-element group.");
  OLA_ENFORCE(k <= kLimit / 4 / n, "QQQ logical FLOAT weights exceed max_bytes.");
  const int64_t gb = g.grouped ? k / 128 * n * 2 : 0;
  OLA_ENFORCE(k * n / 2 + 4 * n + gb <= kLimit, "QQQ checkpoint exceeds max_bytes.");
  QqqTensor(B, "B", kInt32, {k / 16, 2 * n}, k * n / 2);
  QqqTensor(s_channel, "s_channel", kFloat, {1, n}, 4 * n);
  if (g.grouped || !Absent(s_group)) {
    if (g.grouped)
      QqqTensor(s_group, "s_group", kFloat16, {k / 128, n}, gb);
    else
      QqqTensor(s_group, "s_group", kFloat16, {0}, 0);
  }
  return g;
}

// The device work of one QQQ call: staged inputs, the flag word and `extra`
// bytes of scratch after it.
struct QqqRun {
  QqqParams p{};
  std::unique_ptr<Staging> st;
  onnxl_amd_tensor flag_desc{};

  QqqRun(hipStream_t stream, const QqqGeometry &g, size_t extra, const onnxl_amd_tensor *B,
         const onnxl_amd_tensor *s_channel, const onnxl_amd_tensor *s_group, onnxl_amd_tensor *y) {
    st.reset(new Staging(stream, 256 + extra, {B, s_channel, s_group}, {y}));
    p.k = g.k;
    p.n = g.n;
    p.grouped = g.grouped ? 1 : 0;
    p.codes = static_cast<const uint8_t *>(st->In(B));
    p.channel = static_cast<const float *>(st->In(s_channel));
    p.group = g.grouped ? static_cast<const uint16_t *>(st->In(s_group)) : nullptr;
    p.flag = static_cast<unsigned *>(st->Extra());
    hipLaunchKernelGGL(ZeroWordsKernel, dim3(1), dim3(256), 0, stream, p.flag, (size_t)1);
    flag_desc.data_type = kInt32;
    flag_desc.rank = 1;
    flag_desc.dims[0] = 1;
    flag_desc.data = p.flag;
    flag_desc.size_bytes = 4;
    flag_desc.location = ONNXL_AMD_DEVICE;
  }
  void *Extra() const { return static_cast<char *>(st->Extra()) + 256; }
  unsigned Flag(hipStream_t stream) {
    unsigned v = 0;
    ReadOnStream(stream, flag_desc, &v, 4);
    return v;
  }
  // CheckData's failures, then WriteFloat's, in the reference's order
  static void Raise(unsigned flag) {
    OLA_ENFORCE(!(flag & kQqqBadChannel), "QQQ nonfinite or negative channel scale.");
    OLA_ENFORCE(!(flag & kQqqBadGroup), "QQQ nonfinite or negative group scale.");
    OLA_ENFORCE(!(flag & kQqqBadValue), "QQQ FLOAT reconstruction overflow.");
    OLA_ENFORCE(!(flag & kQqqBadOutput), "Dequantization output dtype overflow.");
  }
};

bool QqqDtype(int32_t dt) { return dt == kFloat || dt == kFloat16 || dt == kBfloat16 || dt == kDouble; }

int DequantizeQqq(int64_t k, int64_t n, int64_t group, int64_t bits, const onnxl_amd_tensor *B,
                  const onnxl_amd_tensor *s_channel, const onnxl_amd_tensor *s_group, onnxl_amd_tensor *y,
                  hipStream_t stream) {
  const QqqGeometry g = QqqCheck(k, n, group, bits, B, s_channel, s_group);
  OLA_ENFORCE(y != nullptr && QqqDtype(y->data_type), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16.");
  CheckDescriptor(y, "y");
  const int64_t width = y->data_type == kDouble ? 8 : (y->data_type == kFloat ? 4 : 2);
  OLA_ENFORCE(y->rank == 2 && y->dims[0] == n && y->dims[1] == k && y->size_bytes == n * k * width,
              "QQQ: y must be [out_features, in_features] of its dtype.");
  OLA_ENFORCE(y->data != nullptr, "QQQ: y has no data.");
  Ctx();
  QqqRun run(stream, g, 0, B, s_channel, s_group, y);
  LaunchQqqDecode(run.p, y->data_type, run.st->Out(y), stream);
  OLA_HIP(hipGetLastError());
  QqqRun::Raise(run.Flag(stream));
  run.st->Finish();
  return ONNXL_AMD_OK;
}

int64_t QqqWeightBytes(const QqqGeometry &g) { return g.grouped ? g.k * g.n : TiledInt4Bytes(g.k, g.n); }

int PrepareQqq(int64_t k, int64_t n, int64_t group, int64_t bits, const onnxl_amd_tensor *B,
               const onnxl_amd_tensor *s_channel, const onnxl_amd_tensor *s_group, int32_t dtype,
               onnxl_amd_tensor *weight, onnxl_amd_tensor *scale, hipStream_t stream) {
  const QqqGeometry g = QqqCheck(k, n, group, bits, B, s_channel, s_group);
  OLA_ENFORCE(QqqDtype(dtype), "Dequantize dtype must be FLOAT, DOUBLE, FLOAT16 or BFLOAT16.");
  OLA_ENFORCE(weight && scale, "prepare_qqq: weight and scale are required.");
  const int64_t wb = QqqWeightBytes(g);
  for (const onnxl_amd_tensor *t : {static_cast<const onnxl_amd_tensor *>(weight),
                                    static_cast<const onnxl_amd_tensor *>(scale)})
    OLA_ENFORCE(t->location == ONNXL_AMD_DEVICE && t->data != nullptr &&
                    reinterpret_cast<uintptr_t>(t->data) % 16 == 0,
                "prepare_qqq: weight and scale must be 16-byte aligned device buffers.");
  OLA_ENFORCE(weight->size_bytes >= wb && scale->size_bytes >= 4 * n, "prepare_qqq: weight holds ",
              weight->size_bytes, " bytes and scale ", scale->size_bytes, "; they need ", wb, " and ", 4 * n);
  Ctx();
  QqqRun run(stream, g, g.grouped ? 0 : (size_t)(k * n / 2), B, s_channel, s_group, nullptr);
  LaunchQqqDecode(run.p, dtype, nullptr, stream);  // the checks alone, in the Dequantize dtype
  OLA_HIP(hipGetLastError());
  QqqRun::Raise(run.Flag(stream));
  uint8_t *packed = g.grouped ? static_cast<uint8_t *>(weight->data) : static_cast<uint8_t *>(run.Extra());
  LaunchQqqPack(run.p, packed, static_cast<float *>(scale->data), stream);
  if (!g.grouped) LaunchTileInt4(packed, k, n, 1, static_cast<uint32_t *>(weight->data), stream);
  OLA_HIP(hipGetLastError());
  if (run.Flag(stream) & kQqqBadPrepared)
    throw Unsupported("QQQ: 16 x a channel scale overflows FLOAT, so the INT4 operand has no finite scale "
                      "(onnxl_amd_dequantize_qqq decodes such a weight)");
  run.st->Finish();
  weight->data_type = g.grouped ? kInt8 : kInt4;
  weight->rank = 2;
  for (int i = 0; i < ONNXL_AMD_MAX_RANK; ++i) weight->dims[i] = i == 0 ? k : (i == 1 ? n : 0);
  weight->layout = g.grouped ? ONNXL_AMD_LAYOUT_ONNX : ONNXL_AMD_LAYOUT_TILED_INT4;
  scale->data_type = kFloat;
  scale->rank = 1;
  for (int i = 0; i < ONNXL_AMD_MAX_RANK; ++i) scale->dims[i] = i == 0 ? n : 0;
  scale->layout = ONNXL_AMD_LAYOUT_ONNX;
  return ONNXL_AMD_OK;
}

// Validation runs before any device work, so argument errors are reported
// even before onnxl_amd_init (the first device access then raises
// NotInitialized).
template <typename F> int Guard(F &&f) {
  try {
    std::lock_guard<std::mutex> lk(g_mu);
    if (Initialized()) OLA_HIP(hipSetDevice(g_ctx.device));
    return f();
  } catch (const NotInitialized &e) {
    g_last_error = e.what();
    return ONNXL_AMD_NOT_INITIALIZED;
  } catch (const InvalidArgument &e) {
    g_last_error = e.what();
    return ONNXL_AMD_INVALID_ARGUMENT;
  } catch (const Unsupported &e) {
    g_last_error = e.what();
    return ONNXL_AMD_UNSUPPORTED;
  } catch (const std::exception &e) {
    g_last_error = e.what();
    return ONNXL_AMD_DEVICE_ERROR;
  }
}

}  // namespace
}  // namespace onnxl_amd

using namespace onnxl_amd;

extern "C" {

int onnxl_amd_init(int device_ordinal) {
  try {
    std::lock_guard<std::mutex> lk(g_mu);
    int n = 0;
    OLA_HIP(hipGetDeviceCount(&n));
    OLA_ENFORCE(device_ordinal >= 0 && device_ordinal < n, "onnxl_amd_init: device ", device_ordinal,
                " out of range (", n, " devices)");
    OLA_HIP(hipSetDevice(device_ordinal));
    hipDeviceProp_t prop;
    OLA_HIP(hipGetDeviceProperties(&prop, device_ordinal));
    const std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
      throw Unsupported(Cat("onnxl_amd_init: device is ", arch, ", kernels are built for gfx950"));
    if (g_init.load() && g_ctx.device != device_ordinal) g_ctx.ws.Release();
    g_ctx.device = device_ordinal;
    SetUpNoAllocScratch(device_ordinal);
    g_ctx.num_cus = prop.multiProcessorCount;
    g_init.store(true);
    return ONNXL_AMD_OK;
  } catch (const InvalidArgument &e) {
    g_last_error = e.what();
    return ONNXL_AMD_INVALID_ARGUMENT;
  } catch (const Unsupported &e) {
    g_last_error = e.what();
    return ONNXL_AMD_UNSUPPORTED;
  } catch (const std::exception &e) {
    g_last_error = e.what();
    return ONNXL_AMD_DEVICE_ERROR;
  }
}

int onnxl_amd_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_init.load()) {
    (void)hipSetDevice(g_ctx.device);
    (void)hipDeviceSynchronize();
    g_ctx.ws.Release();
  }
  if (g_pinned) {
    (void)hipHostFree(g_pinned);
    g_pinned = nullptr;
  }
  g_init.store(false);
  return ONNXL_AMD_OK;
}

const char *onnxl_amd_last_error(void) { return g_last_error.c_str(); }

const char *onnxl_amd_version(void) { return "onnxl_amd 0.1.0 (gfx950)"; }

int onnxl_amd_matmul_shape(const int64_t *a_dims, int32_t a_rank, const int64_t *b_dims,
                           int32_t b_rank, int64_t *out_dims, int32_t *out_rank) {
  try {
    OLA_ENFORCE(a_rank >= 0 && b_rank >= 0 && a_rank <= ONNXL_AMD_MAX_RANK &&
                    b_rank <= ONNXL_AMD_MAX_RANK,
                "onnxl_amd_matmul_shape: rank out of range");
    const MatMulPlan p = MakeMatMulPlan(Shape(a_dims, a_dims + a_rank), Shape(b_dims, b_dims + b_rank),
                                        "kernel::MatMul", " does not accept rank-0 inputs.",
                                        " got incompatible inner dimensions.",
                                        " inputs are not broadcast-compatible on batch dimensions.");
    OLA_ENFORCE((int)p.out_shape.size() <= ONNXL_AMD_MAX_RANK, "output rank too large");
    for (size_t i = 0; i < p.out_shape.size(); ++i) out_dims[i] = p.out_shape[i];
    *out_rank = (int32_t)p.out_shape.size();
    return ONNXL_AMD_OK;
  } catch (const InvalidArgument &e) {
    g_last_error = e.what();
    return ONNXL_AMD_INVALID_ARGUMENT;
  }
}

int onnxl_amd_matmul_integer(const onnxl_amd_tensor *a, const onnxl_amd_tensor *b,
                             const onnxl_amd_tensor *a_zero_point,
                             const onnxl_amd_tensor *b_zero_point, onnxl_amd_tensor *y,
                             void *stream) {
  return Guard([&] {
    return MatMulInteger(a, b, a_zero_point, b_zero_point, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_qlinear_matmul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *a_scale,
                             const onnxl_amd_tensor *a_zero_point, const onnxl_amd_tensor *b,
                             const onnxl_amd_tensor *b_scale,
                             const onnxl_amd_tensor *b_zero_point,
                             const onnxl_amd_tensor *y_scale,
                             const onnxl_amd_tensor *y_zero_point, onnxl_amd_tensor *y,
                             void *stream) {
  return Guard([&] {
    return QLinearMatMul(a, a_scale, a_zero_point, b, b_scale, b_zero_point, y_scale, y_zero_point, y,
                         static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_linear(const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale,
                                const onnxl_amd_tensor *x_zero_point, int64_t axis,
                                onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DequantizeLinear(x, x_scale, x_zero_point, axis, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_packed(const onnxl_amd_tensor *x, const char *format, const int64_t *shape, int32_t rank,
                                int64_t output_dtype, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DequantizePacked(x, format, shape, rank, output_dtype, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_packed_matmul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x, const char *format,
                                       const int64_t *shape, int32_t rank, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DequantizePackedMatMul(a, x, format, shape, rank, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_conv_shape(const int64_t *x_dims, int32_t x_rank, const int64_t *w_dims, int32_t w_rank,
                         const onnxl_amd_conv_attrs *attrs, int64_t *y_dims, int32_t *y_rank) {
  return Guard([&] {
    OLA_ENFORCE(x_dims && w_dims && y_dims && y_rank && x_rank >= 0 && x_rank <= ONNXL_AMD_MAX_RANK &&
                    w_rank >= 0 && w_rank <= ONNXL_AMD_MAX_RANK,
                "conv_shape: invalid arguments.");
    const Shape xs(x_dims, x_dims + x_rank), ws(w_dims, w_dims + w_rank);
    const ConvResolved r = ResolveConv(xs, ws, attrs, "kernel::Conv");
    OLA_ENFORCE(attrs->group >= 1 && ws[0] % attrs->group == 0 && xs[1] == ws[1] * attrs->group,
                "kernel::Conv: x.shape[1] must equal w.shape[1] * group.");
    y_dims[0] = xs[0];
    y_dims[1] = ws[0];
    for (size_t i = 0; i < r.out.size(); ++i) y_dims[2 + i] = r.out[i];
    *y_rank = (int32_t)(2 + r.out.size());
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_conv_integer(const onnxl_amd_tensor *x, const onnxl_amd_tensor *w,
                           const onnxl_amd_tensor *x_zero_point, const onnxl_amd_tensor *w_zero_point,
                           const onnxl_amd_conv_attrs *attrs, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return ConvInteger(x, w, x_zero_point, w_zero_point, attrs, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_qlinear_conv(const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale,
                           const onnxl_amd_tensor *x_zero_point, const onnxl_amd_tensor *w,
                           const onnxl_amd_tensor *w_scale, const onnxl_amd_tensor *w_zero_point,
                           const onnxl_amd_tensor *y_scale, const onnxl_amd_tensor *y_zero_point,
                           const onnxl_amd_tensor *B, const onnxl_amd_conv_attrs *attrs, onnxl_amd_tensor *y,
                           void *stream) {
  return Guard([&] {
    return QLinearConv(x, x_scale, x_zero_point, w, w_scale, w_zero_point, y_scale, y_zero_point, B, attrs, y,
                       static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_quantize_linear(const onnxl_amd_tensor *x, const onnxl_amd_tensor *y_scale,
                              const onnxl_amd_tensor *y_zero_point, int64_t axis, int32_t output_dtype,
                              onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return QuantizeLinear(x, y_scale, y_zero_point, axis, output_dtype, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dynamic_quantize_linear(const onnxl_amd_tensor *x, onnxl_amd_tensor *y, onnxl_amd_tensor *y_scale,
                                      onnxl_amd_tensor *y_zero_point, void *stream) {
  return Guard([&] {
    return DynamicQuantizeLinear(x, y, y_scale, y_zero_point, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_matmul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *b, onnxl_amd_tensor *y,
                     void *stream) {
  return Guard([&] { return MatMul(a, b, y, static_cast<hipStream_t>(stream)); });
}

int onnxl_amd_grouped_matmul(const onnxl_amd_tensor *input, const onnxl_amd_tensor *weights,
                             const onnxl_amd_tensor *group_indices, const onnxl_amd_tensor *bias, int64_t transB,
                             onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return GroupedMatMul(input, weights, group_indices, bias, transB, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_linear_grouped_matmul(const onnxl_amd_tensor *input, const onnxl_amd_tensor *x,
                                               const onnxl_amd_tensor *x_scale, const onnxl_amd_tensor *x_zero_point,
                                               int64_t axis, int32_t cast_to, const onnxl_amd_tensor *group_indices,
                                               const onnxl_amd_tensor *bias, int64_t transB, onnxl_amd_tensor *y,
                                               void *stream) {
  return Guard([&] {
    return DqGroupedMatMul(input, x, x_scale, x_zero_point, axis, cast_to, group_indices, bias, transB, y,
                           static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_prepare_matmul_nbits_size(int64_t K, int64_t N, int64_t bits, int64_t block_size, int has_zero_points,
                                        int64_t *weight_bytes, int64_t *scale_bytes, int64_t *zero_point_bytes) {
  return Guard([&] {
    OLA_ENFORCE(weight_bytes && scale_bytes && zero_point_bytes, "prepare_matmul_nbits_size: null output");
    const NbitsLayout l = PlanNbits(K, N, bits, block_size, has_zero_points != 0);
    *weight_bytes = l.weight_bytes;
    *scale_bytes = l.scale_bytes;
    *zero_point_bytes = l.zp_bytes;
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_prepare_matmul_nbits(const onnxl_amd_tensor *B, const onnxl_amd_tensor *scales,
                                   const onnxl_amd_tensor *zero_points, int64_t K, int64_t N, int64_t bits,
                                   int64_t block_size, onnxl_amd_tensor *weight, onnxl_amd_tensor *scale,
                                   onnxl_amd_tensor *zero_point, void *stream) {
  return Guard([&] {
    return PrepareMatMulNbits(B, scales, zero_points, K, N, bits, block_size, weight, scale, zero_point,
                              static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_prepare_awq_size(const char *variant, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                               int32_t scale_dtype, int64_t *weight_bytes, int64_t *scale_bytes,
                               int64_t *zero_point_bytes) {
  return Guard([&] {
    OLA_ENFORCE(weight_bytes && scale_bytes && zero_point_bytes, "prepare_awq_size: null output");
    const CkptSizes sz = CkptPreparedSizes(PlanAwq(variant, K, N, bits, group_size, scale_dtype));
    *weight_bytes = sz.weight;
    *scale_bytes = sz.scale;
    *zero_point_bytes = sz.zp;
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_prepare_awq(const char *variant, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                          const onnxl_amd_tensor *scales, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                          onnxl_amd_tensor *weight, onnxl_amd_tensor *scale, onnxl_amd_tensor *zero_point,
                          void *stream) {
  return Guard([&] {
    return PrepareAwq(variant, qweight, qzeros, scales, K, N, bits, group_size, weight, scale, zero_point,
                      static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_awq(const char *variant, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                             const onnxl_amd_tensor *scales, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                             onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    CkptPlan p = AwqFromTensors(variant, scales, K, N, bits, group_size);
    CheckAwqTensors(p, qweight, qzeros, scales);
    CkptHost h = CheckAwqValues(p, qweight, qzeros, scales);
    return DecodeCkpt(p, h, qweight, qzeros, scales, nullptr, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_prepare_gptq_size(const char *format, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                                int32_t word_dtype, int32_t scale_dtype, int64_t *weight_bytes, int64_t *scale_bytes,
                                int64_t *zero_point_bytes) {
  return Guard([&] {
    OLA_ENFORCE(weight_bytes && scale_bytes && zero_point_bytes, "prepare_gptq_size: null output");
    const CkptSizes sz = CkptPreparedSizes(PlanGptq(format, K, N, bits, group_size, word_dtype, scale_dtype));
    *weight_bytes = sz.weight;
    *scale_bytes = sz.scale;
    *zero_point_bytes = sz.zp;
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_prepare_gptq(const char *format, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                           const onnxl_amd_tensor *scales, const onnxl_amd_tensor *g_idx, int64_t K, int64_t N,
                           int64_t bits, int64_t group_size, onnxl_amd_tensor *weight, onnxl_amd_tensor *scale,
                           onnxl_amd_tensor *zero_point, void *stream) {
  return Guard([&] {
    return PrepareGptq(format, qweight, qzeros, scales, g_idx, K, N, bits, group_size, weight, scale, zero_point,
                       static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_gptq(const char *format, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                              const onnxl_amd_tensor *scales, const onnxl_amd_tensor *g_idx, int64_t K, int64_t N,
                              int64_t bits, int64_t group_size, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    CkptPlan p = GptqFromTensors(format, qweight, qzeros, scales, g_idx, K, N, bits, group_size);
    CkptHost h = CheckGptqValues(p, qweight, qzeros, scales, g_idx);
    return DecodeCkpt(p, h, qweight, qzeros, scales, g_idx, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_bitblas(const char *method, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *scales,
                                 const onnxl_amd_tensor *qzeros, int64_t K, int64_t N, int64_t bits,
                                 int64_t group_size, int32_t symmetric, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    CkptPlan p = BitblasFromTensors(method, qweight, scales, qzeros, K, N, bits, group_size, symmetric);
    CkptHost h = CheckBitblasValues(p, qzeros, scales);
    return DecodeCkpt(p, h, qweight, p.L.signed_codes ? nullptr : qzeros, scales, nullptr, y,
                      static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_prepare_bitblas_size(const char *method, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                                   int32_t symmetric, int64_t *weight_bytes, int64_t *scale_bytes,
                                   int64_t *zero_point_bytes) {
  return Guard([&] {
    OLA_ENFORCE(weight_bytes && scale_bytes && zero_point_bytes, "prepare_bitblas_size: null output");
    const CkptSizes sz = CkptPreparedSizes(PlanBitblas(method, K, N, bits, group_size, symmetric, kFloat16));
    *weight_bytes = sz.weight;
    *scale_bytes = sz.scale;
    *zero_point_bytes = sz.zp;
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_prepare_bitblas(const char *method, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *scales,
                              const onnxl_amd_tensor *qzeros, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                              int32_t symmetric, onnxl_amd_tensor *weight, onnxl_amd_tensor *scale,
                              onnxl_amd_tensor *zero_point, void *stream) {
  return Guard([&] {
    CkptPlan p = BitblasFromTensors(method, qweight, scales, qzeros, K, N, bits, group_size, symmetric);
    CheckBitblasValues(p, qzeros, scales);
    return PrepareCkpt("prepare_bitblas", p, qweight, p.L.signed_codes ? nullptr : qzeros, scales, weight, scale,
                       zero_point, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_transpose_2d(const onnxl_amd_tensor *x, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] { return Transpose2d(x, y, static_cast<hipStream_t>(stream)); });
}

int onnxl_amd_cast(const onnxl_amd_tensor *x, int32_t to, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] { return Cast(x, to, y, static_cast<hipStream_t>(stream)); });
}

int onnxl_amd_dequantize_linear_matmul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x,
                                       const onnxl_amd_tensor *x_scale,
                                       const onnxl_amd_tensor *x_zero_point, int64_t axis,
                                       int32_t cast_to, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DqMatMul(a, x, x_scale, x_zero_point, axis, cast_to, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_linear_matmul_noalloc(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x,
                                               const onnxl_amd_tensor *x_scale,
                                               const onnxl_amd_tensor *x_zero_point, int64_t axis,
                                               int32_t cast_to, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DqMatMulNoAlloc(a, x, x_scale, x_zero_point, axis, cast_to, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_prepare_weight_size(const onnxl_amd_tensor *x, int64_t *bytes) {
  return Guard([&] {
    OLA_ENFORCE(!Absent(x) && bytes, "prepare_weight: x and bytes are required.");
    CheckDescriptor(x, "x");
    OLA_ENFORCE(IsFourBit(x->data_type) && x->rank == 2,
                "prepare_weight: only 2-D INT4 / UINT4 weights have a prepared layout.");
    *bytes = TiledInt4Bytes(x->dims[0], x->dims[1]);
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_prepare_weight(const onnxl_amd_tensor *x, onnxl_amd_tensor *prepared, void *stream) {
  return Guard([&] {
    OLA_ENFORCE(!Absent(x) && prepared, "prepare_weight: x and prepared are required.");
    CheckDescriptor(x, "x");
    OLA_ENFORCE(IsFourBit(x->data_type) && x->rank == 2,
                "prepare_weight: only 2-D INT4 / UINT4 weights have a prepared layout.");
    const int64_t K = x->dims[0], N = x->dims[1];
    const int64_t need = TiledInt4Bytes(K, N);
    OLA_ENFORCE(prepared->location == ONNXL_AMD_DEVICE, "prepare_weight: prepared must be device memory.");
    OLA_ENFORCE(prepared->size_bytes >= need, "prepare_weight: prepared holds ", prepared->size_bytes,
                " bytes, the tiled weight needs ", need);
    OLA_ENFORCE(need == 0 || (prepared->data != nullptr && reinterpret_cast<uintptr_t>(prepared->data) % 16 == 0),
                "prepare_weight: prepared must be a 16-byte aligned device buffer.");
    hipStream_t s = static_cast<hipStream_t>(stream);
    Ctx();
    Staging st(s, 0, {x}, {});
    LaunchTileInt4(static_cast<const uint8_t *>(st.In(x)), K, N, x->data_type == kInt4,
                   static_cast<uint32_t *>(prepared->data), s);
    prepared->data_type = x->data_type;
    prepared->rank = 2;
    for (int i = 0; i < ONNXL_AMD_MAX_RANK; ++i) prepared->dims[i] = i < 2 ? x->dims[i] : 0;
    prepared->layout = ONNXL_AMD_LAYOUT_TILED_INT4;
    st.Finish();
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_dequantize_bitsandbytes(int32_t format, int64_t rows, int64_t cols, int64_t block_size,
                                      int64_t nested_block_size, float nested_offset, const onnxl_amd_tensor *weight,
                                      const onnxl_amd_tensor *absmax, const onnxl_amd_tensor *quant_map,
                                      const onnxl_amd_tensor *nested_absmax,
                                      const onnxl_amd_tensor *nested_quant_map, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DequantizeBnb(format, rows, cols, block_size, nested_block_size, nested_offset, weight, absmax,
                         quant_map, nested_absmax, nested_quant_map, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_prepare_bitsandbytes_size(int32_t format, int64_t rows, int64_t cols, int64_t block_size,
                                        int64_t *scale_bytes) {
  return Guard([&] {
    OLA_ENFORCE(scale_bytes, "prepare_bitsandbytes_size: null output");
    OLA_ENFORCE(rows > 0 && cols > 0 && (format == 2 || (format >= 0 && format <= 1 && block_size > 0)),
                "prepare_bitsandbytes_size: invalid format or dimensions");
    *scale_bytes = BnbBlocks(format, rows, cols, block_size) * 4;
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_prepare_bitsandbytes(int32_t format, int64_t rows, int64_t cols, int64_t block_size,
                                   int64_t nested_block_size, float nested_offset, const onnxl_amd_tensor *weight,
                                   const onnxl_amd_tensor *absmax, const onnxl_amd_tensor *quant_map,
                                   const onnxl_amd_tensor *nested_absmax, const onnxl_amd_tensor *nested_quant_map,
                                   int32_t reconstruction_dtype, onnxl_amd_tensor *scales, void *stream) {
  return Guard([&] {
    return PrepareBnb(format, rows, cols, block_size, nested_block_size, nested_offset, weight, absmax, quant_map,
                      nested_absmax, nested_quant_map, reconstruction_dtype, scales, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_bitsandbytes_matmul(const onnxl_amd_tensor *a, int32_t format, int64_t rows, int64_t cols,
                                  int64_t block_size, const onnxl_amd_tensor *weight, const onnxl_amd_tensor *scales,
                                  onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return BnbMatMul(a, format, rows, cols, block_size, weight, scales, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_vptq(const onnxl_amd_vptq_config *config, const onnxl_amd_tensor *indices,
                              const onnxl_amd_tensor *centroids, const onnxl_amd_tensor *res_centroids,
                              const onnxl_amd_tensor *outlier_centroids, const onnxl_amd_tensor *outlier_indices,
                              const onnxl_amd_tensor *weight_scale, const onnxl_amd_tensor *weight_bias,
                              const onnxl_amd_tensor *perm, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DequantizeVptq(config, indices, centroids, res_centroids, outlier_centroids, outlier_indices,
                          weight_scale, weight_bias, perm, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_mx_weights(const char *format, const onnxl_amd_tensor *weight,
                                    const onnxl_amd_tensor *weight_scale, float weight_global_scale,
                                    onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DequantizeMx(format, weight, weight_scale, weight_global_scale, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_exl3(const onnxl_amd_tensor *trellis, const onnxl_amd_tensor *suh,
                              const onnxl_amd_tensor *svh, const onnxl_amd_tensor *mcg, const onnxl_amd_tensor *mul1,
                              onnxl_amd_tensor *y, void *stream) {
  return Guard([&] { return DequantizeExl3(trellis, suh, svh, mcg, mul1, y, static_cast<hipStream_t>(stream)); });
}

int onnxl_amd_dequantize_gptqmodel_fp8(int64_t in_features, int64_t out_features, const char *weight_scale_method,
                                       const int64_t *weight_block_size, int32_t block_rank,
                                       const onnxl_amd_tensor *weight, const onnxl_amd_tensor *weight_scale_inv,
                                       onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DequantizeGptqFp8(in_features, out_features, weight_scale_method, weight_block_size, block_rank, weight,
                             weight_scale_inv, y, static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_dequantize_qqq(int64_t in_features, int64_t out_features, int64_t group_size, int64_t bits,
                             const onnxl_amd_tensor *B, const onnxl_amd_tensor *s_channel,
                             const onnxl_amd_tensor *s_group, onnxl_amd_tensor *y, void *stream) {
  return Guard([&] {
    return DequantizeQqq(in_features, out_features, group_size, bits, B, s_channel, s_group, y,
                         static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_prepare_qqq_size(int64_t in_features, int64_t out_features, int64_t group_size, int64_t bits,
                               int64_t *weight_bytes, int64_t *scale_bytes) {
  return Guard([&] {
    OLA_ENFORCE(weight_bytes && scale_bytes, "prepare_qqq_size: null output");
    OLA_ENFORCE(in_features > 0 && out_features > 0 && in_features % 64 == 0 && out_features % 64 == 0 &&
                    bits == 4 && (group_size == -1 || group_size == 128),
                "QQQ requires four-bit, unpadded dimensions divisible by 64 and group -1/128.");
    const QqqGeometry g{in_features, out_features, group_size == 128 && in_features != 128};
    *weight_bytes = QqqWeightBytes(g);
    *scale_bytes = 4 * out_features;
    return ONNXL_AMD_OK;
  });
}

int onnxl_amd_prepare_qqq(int64_t in_features, int64_t out_features, int64_t group_size, int64_t bits,
                          const onnxl_amd_tensor *B, const onnxl_amd_tensor *s_channel,
                          const onnxl_amd_tensor *s_group, int32_t dtype, onnxl_amd_tensor *weight,
                          onnxl_amd_tensor *scale, void *stream) {
  return Guard([&] {
    return PrepareQqq(in_features, out_features, group_size, bits, B, s_channel, s_group, dtype, weight, scale,
                      static_cast<hipStream_t>(stream));
  });
}

int onnxl_amd_synchronize(void *stream) {
  return Guard([&] {
    OLA_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return ONNXL_AMD_OK;
  });
}

}  // extern "C"
