// Graph rewrites that route the quantized-weight chains to the fused MI355X
// kernels registered by register_mi355x.cc:
//
//   DequantizeLinearMatMulGpu:
//     W, s[, zp] (constants) -> DequantizeLinear(axis) -> [Cast(to = FLOAT16 |
//     BFLOAT16)] -> MatMul(A, .)
//     => ai.rt.amd:DequantizeLinearMatMul(A, W, s[, zp]; axis, cast_to)
//   DequantizePackedMatMulGpu:
//     x (constant) -> DequantizePacked(format, shape = [N, K], FLOAT16) ->
//     Transpose(perm = [1, 0]) -> MatMul(A, .)
//     => ai.rt.amd:DequantizePackedMatMul(A, x; format, shape)
//   DequantizeEncodedMatMulGpu: ai.rt:Dequantize -> Transpose -> MatMul
//     => ai.rt.amd:DequantizeEncodedMatMul(A, Q)
//   DequantizeLinearGroupedMatMulGpu: constant experts -> DequantizeLinear ->
//     [Cast] -> GroupedMatMul(input, ., group_indices[, bias])
//     => ai.rt.amd:DequantizeLinearGroupedMatMul
//
// All are core::builder::PatternOptimization subclasses
// (onnx_core/builder/pattern_optimization.h:164-224) registered opt-in with
// RegisterPattern(name, factory, false) (onnx_core/builder/pattern_registry.h:
// 36-37), so the default pattern set is unchanged and a caller enables them by
// name (CreateRegisteredPattern) when the MI355X kernels are registered.  A
// rewrite only fires where the fused kernel accepts the node, so a graph that
// runs unfused never becomes one that raises: the checks read the constants'
// declared type and shape (GetConstantMetadata, no payload load) and A's
// element type.  The same rules, with the same no-match reasons, are
// onnx-light_amd/patterns.py, whose tests pin them.
//
// Compiled inside the onnx-light tree next to the adapter.
#include "onnx_core/builder/graph_graph.h"
#include "onnx_core/builder/pattern_optimization.h"
#include "onnx_core/builder/pattern_registry.h"
#include "onnx_core/symbolic/sym_tensor.h"
#include "onnx_proto/onnx.h"
#include "onnx_proto/onnx_helper.h"
#include "onnx_proto/type_helper.h"

#include <cstdint>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

namespace mi355x_patterns {

namespace ol = ONNX_LIGHT_NAMESPACE;
namespace builder = ONNX_LIGHT_NAMESPACE::core::builder;
namespace sym = ONNX_LIGHT_NAMESPACE::core::symbolic;
using ol::AttributeProto;
using ol::NodeProto;
using ol::TensorProto;
using TensorType = ol::onnx_proto::TensorType;

constexpr const char *kFusedDomain = "ai.rt.amd";
// ONNX element types
constexpr int32_t kFloat = 1, kUint8 = 2, kInt8 = 3, kFloat16 = 10, kBfloat16 = 16, kFloat8E4M3FN = 17,
                  kUint4 = 21, kInt4 = 22;

bool IsOnnxOp(const NodeProto &node, const char *op_type) {
  return node.op_type().value() == op_type && ol::NormaliseDomain(node.domain().value()) == ol::kDefaultOnnxDomain;
}

const std::string &In(const NodeProto &node, int i) { return node.input()[i].value(); }
const std::string &Out(const NodeProto &node, int i) { return node.output()[i].value(); }

std::vector<std::string> Outputs(const NodeProto &node) {
  std::vector<std::string> out;
  for (int i = 0; i < node.output_size(); ++i) out.push_back(Out(node, i));
  return out;
}

// `name` feeds one input slot of `user` only and is not a graph output.
bool SingleUse(builder::GraphGraph &graph, const std::string &name, const NodeProto &user) {
  if (graph.IsUsedMoreThanOnce(name) || graph.IsOutput(name)) return false;
  int slots = 0;
  for (int i = 0; i < user.input_size(); ++i) slots += In(user, i) == name;
  return slots == 1;
}

bool OnlyAttributes(const NodeProto &node, const std::set<std::string> &allowed) {
  for (const auto &a : node.attribute())
    if (allowed.count(std::string(a.name().value())) == 0) return false;
  return true;
}

std::vector<int64_t> Dims(const TensorProto &t) {
  std::vector<int64_t> d;
  for (int i = 0; i < t.dims_size(); ++i) d.push_back(t.dims(i));
  return d;
}

void AddInt(NodeProto &node, const char *name, int64_t value) {
  AttributeProto *a = node.add_attribute();
  a->set_name(name);
  a->set_type(AttributeProto::AttributeType::INT);
  a->set_i(value);
}

// Values per block of the 27 GGUF profiles of DequantizePacked
// (dequantize_packed.cc:27-36), 0 for any other format.  The fused node runs
// all of them on the GPU.
int64_t PackedBlockValues(const std::string &format) {
  static const std::map<std::string, int64_t> kBlock = {
      {"gguf:q4_0", 32},     {"gguf:q4_1", 32},    {"gguf:q5_0", 32},    {"gguf:q5_1", 32},   {"gguf:q8_0", 32},
      {"gguf:q8_1", 32},     {"gguf:iq4_nl", 32},  {"gguf:mxfp4", 32},   {"gguf:q2_k", 256},  {"gguf:q3_k", 256},
      {"gguf:q4_k", 256},    {"gguf:q5_k", 256},   {"gguf:q6_k", 256},   {"gguf:q8_k", 256},  {"gguf:iq2_xxs", 256},
      {"gguf:iq2_xs", 256},  {"gguf:iq3_xxs", 256}, {"gguf:iq1_s", 256}, {"gguf:iq3_s", 256}, {"gguf:iq2_s", 256},
      {"gguf:iq4_xs", 256},  {"gguf:iq1_m", 256},  {"gguf:tq1_0", 256},  {"gguf:tq2_0", 256}, {"gguf:nvfp4", 64},
      {"gguf:q2_0", 64},     {"gguf:q1_0", 128}};
  const auto it = kBlock.find(format);
  return it == kBlock.end() ? 0 : it->second;
}

// ---------------------------------------------------------------------------
class DequantizeLinearMatMulGpuPattern : public builder::PatternOptimization {
public:
  explicit DequantizeLinearMatMulGpuPattern(bool fp8_scaled_sums = false)
      : builder::PatternOptimization(1, "DequantizeLinearMatMulGpu", sym::Device::kGPU0),
        fp8_scaled_sums_(fp8_scaled_sums) {}

  std::set<std::string> FastOpType() const override { return {"MatMul"}; }

  builder::MatchResult Match(builder::GraphGraph &graph, const NodeProto &candidate) const override {
    if (!IsOnnxOp(candidate, "MatMul") || candidate.input_size() != 2) return NoMatch(candidate, "not a MatMul");
    const NodeProto *cast = nullptr;
    const NodeProto *prod = graph.NodeBefore(In(candidate, 1));
    int64_t cast_to = 0;
    if (prod != nullptr && IsOnnxOp(*prod, "Cast")) {
      cast_to = ol::GetAttributeOr<int64_t>(*prod, "to", 0);
      if (cast_to != kFloat16 && cast_to != kBfloat16)
        return NoMatch(candidate, "Cast target is not FLOAT16 or BFLOAT16");
      if (!SingleUse(graph, Out(*prod, 0), candidate)) return NoMatch(candidate, "Cast output has another consumer");
      cast = prod;
      prod = graph.NodeBefore(In(*prod, 0));
    }
    if (prod == nullptr || !IsOnnxOp(*prod, "DequantizeLinear"))
      return NoMatch(candidate, "MatMul's second input is not a DequantizeLinear output");
    if (!OnlyAttributes(*prod, {"axis"})) return NoMatch(candidate, "DequantizeLinear attribute other than axis");
    std::vector<const TensorProto *> meta;
    for (int i = 0; i < prod->input_size(); ++i) {
      if (In(*prod, i).empty()) continue;
      if (!graph.IsConstant(In(*prod, i))) return NoMatch(candidate, "DequantizeLinear inputs are not all initializers");
      meta.push_back(graph.GetConstantMetadata(In(*prod, i)));
    }
    if (meta.size() < 2) return NoMatch(candidate, "DequantizeLinear inputs are not all initializers");
    if (!SingleUse(graph, Out(*prod, 0), cast != nullptr ? *cast : candidate))
      return NoMatch(candidate, "DequantizeLinear output has another consumer");
    for (const TensorProto *m : meta)
      if (m == nullptr) return NoMatch(candidate, "type or shape of a DequantizeLinear input unknown");

    // The fused entry point's checks (the DequantizeLinear rules of
    // kq/kernel_dequantizelinear.cc:522-565, then the fused kernel's limits).
    const int32_t w_t = meta[0]->data_type(), s_t = meta[1]->data_type();
    const std::vector<int64_t> w = Dims(*meta[0]), s = Dims(*meta[1]);
    if (w_t != kInt4 && w_t != kUint4 && w_t != kInt8 && w_t != kUint8 && w_t != kFloat8E4M3FN)
      return NoMatch(candidate, "weight type has no fused kernel");
    if (w.size() != 2) return NoMatch(candidate, "weight is not 2-D");
    if (s_t != kFloat && s_t != kFloat16) return NoMatch(candidate, "scale is not FLOAT or FLOAT16");
    const bool has_zp = meta.size() > 2;
    if (has_zp && (meta[2]->data_type() != w_t || Dims(*meta[2]) != s))
      return NoMatch(candidate, "zero point type or shape does not match");
    const int64_t axis = ol::GetAttributeOr<int64_t>(*prod, "axis", 1);
    int64_t count = 1;
    for (int64_t d : s) count *= d;
    const bool per_tensor = count == 1;
    if (!per_tensor) {
      if (axis < 0 || axis >= 2) return NoMatch(candidate, "axis out of range");
      if (s.size() == 2) {
        for (int d = 0; d < 2; ++d)
          if (s[d] <= 0 || w[d] % s[d] != 0 || (d != axis && s[d] != w[d]))
            return NoMatch(candidate, "blocked scale does not fit the weight");
        if (axis != 0) return NoMatch(candidate, "scales blocked along N");
      } else if (s.size() == 1) {
        if (count != w[axis]) return NoMatch(candidate, "scale size differs from the axis dimension");
        if (axis != 1) return NoMatch(candidate, "per-row (axis 0) scales");
      } else {
        return NoMatch(candidate, "scale rank above 2");
      }
    }
    if (cast_to != 0 && s_t != kFloat) return NoMatch(candidate, "Cast of a FLOAT16 DequantizeLinear output");
    const int64_t run_type = cast_to != 0 ? cast_to : s_t;
    if (run_type != kFloat16 && run_type != kBfloat16) return NoMatch(candidate, "MatMul would run in FLOAT");
    if (w_t == kFloat8E4M3FN && cast_to == kBfloat16 && s_t == kFloat && !has_zp && (per_tensor || s.size() == 1) &&
        !fp8_scaled_sums_)
      return NoMatch(candidate, "FLOAT8E4M3FN -> BFLOAT16 chain would scale the sums (fp8_scaled_sums=True allows it)");

    std::vector<const NodeProto *> nodes{prod};
    if (cast != nullptr) nodes.push_back(cast);
    nodes.push_back(&candidate);
    return builder::MatchResult{this, nodes, &candidate};
  }

  ol::utils::RepeatedProtoField<NodeProto> Apply(builder::GraphGraph &graph,
                                                 const std::vector<const NodeProto *> &nodes) const override {
    const builder::MatchResult verified = nodes.empty() || nodes.back() == nullptr
                                              ? builder::MatchResult{}
                                              : Match(graph, *nodes.back());
    if (verified.pattern == nullptr || verified.nodes != nodes)
      throw builder::BuilderError("DequantizeLinearMatMulGpuPattern::Apply received an unsafe or inconsistent match.");
    const NodeProto &dq = *nodes.front(), &matmul = *nodes.back();
    const int64_t cast_to = nodes.size() == 3 ? ol::GetAttributeOr<int64_t>(*nodes[1], "to", 0) : 0;
    std::vector<std::string> inputs{In(matmul, 0)};
    for (int i = 0; i < dq.input_size(); ++i) inputs.push_back(In(dq, i));
    while (inputs.size() > 1 && inputs.back().empty()) inputs.pop_back();
    const std::string name = "DequantizeLinearMatMulGpu--" + std::string(matmul.name().value());
    NodeProto fused = ol::MakeNode("DequantizeLinearMatMul", inputs, Outputs(matmul), kFusedDomain, name.c_str());
    AddInt(fused, "axis", ol::GetAttributeOr<int64_t>(dq, "axis", 1));
    AddInt(fused, "cast_to", cast_to);
    ol::utils::RepeatedProtoField<NodeProto> out;
    out.push_back(std::move(fused));
    return out;
  }

private:
  bool fp8_scaled_sums_;
};

// ---------------------------------------------------------------------------
class DequantizePackedMatMulGpuPattern : public builder::PatternOptimization {
public:
  DequantizePackedMatMulGpuPattern()
      : builder::PatternOptimization(1, "DequantizePackedMatMulGpu", sym::Device::kGPU0) {}

  std::set<std::string> FastOpType() const override { return {"MatMul"}; }

  builder::MatchResult Match(builder::GraphGraph &graph, const NodeProto &candidate) const override {
    if (!IsOnnxOp(candidate, "MatMul") || candidate.input_size() != 2) return NoMatch(candidate, "not a MatMul");
    const NodeProto *tr = graph.NodeBefore(In(candidate, 1));
    if (tr == nullptr || !IsOnnxOp(*tr, "Transpose"))
      return NoMatch(candidate, "MatMul's second input is not a Transpose output");
    std::vector<int64_t> perm;
    if (ol::GetAttributeInts(*tr, "perm", perm) && perm != std::vector<int64_t>{1, 0})
      return NoMatch(candidate, "Transpose is not a 2-D transpose");
    if (!SingleUse(graph, Out(*tr, 0), candidate)) return NoMatch(candidate, "Transpose output has another consumer");
    const NodeProto *dp = graph.NodeBefore(In(*tr, 0));
    if (dp == nullptr || !IsOnnxOp(*dp, "DequantizePacked"))
      return NoMatch(candidate, "Transpose input is not a DequantizePacked output");
    if (!SingleUse(graph, Out(*dp, 0), *tr)) return NoMatch(candidate, "DequantizePacked output has another consumer");
    if (!graph.IsConstant(In(*dp, 0))) return NoMatch(candidate, "packed weight is not an initializer");
    const std::string format = ol::GetAttributeOr<std::string>(*dp, "format", "");
    const int64_t k_multiple = PackedBlockValues(format);
    if (k_multiple == 0) return NoMatch(candidate, "unknown packed format");
    std::vector<int64_t> shape;
    ol::GetAttributeInts(*dp, "shape", shape);
    if (shape.size() != 2) return NoMatch(candidate, "DequantizePacked shape is not [N, K]");
    if (ol::GetAttributeOr<int64_t>(*dp, "output_dtype", kFloat) != kFloat16)
      return NoMatch(candidate, "DequantizePacked output is not FLOAT16");
    if (shape[1] % k_multiple != 0) return NoMatch(candidate, "K is not a whole number of blocks");
    if (!graph.HasType(In(candidate, 0))) return NoMatch(candidate, "type of A unknown");
    if (graph.GetType(In(candidate, 0)) != TensorType::kFloat16) return NoMatch(candidate, "A is not FLOAT16");
    return builder::MatchResult{this, {dp, tr, &candidate}, &candidate};
  }

  ol::utils::RepeatedProtoField<NodeProto> Apply(builder::GraphGraph &graph,
                                                 const std::vector<const NodeProto *> &nodes) const override {
    const builder::MatchResult verified =
        nodes.size() != 3 || nodes[2] == nullptr ? builder::MatchResult{} : Match(graph, *nodes[2]);
    if (verified.pattern == nullptr || verified.nodes != nodes)
      throw builder::BuilderError("DequantizePackedMatMulGpuPattern::Apply received an unsafe or inconsistent match.");
    const NodeProto &dp = *nodes[0], &matmul = *nodes[2];
    const std::string name = "DequantizePackedMatMulGpu--" + std::string(matmul.name().value());
    NodeProto fused = ol::MakeNode("DequantizePackedMatMul", {In(matmul, 0), In(dp, 0)}, Outputs(matmul),
                                   kFusedDomain, name.c_str());
    for (const auto &a : dp.attribute()) {
      const std::string n(a.name().value());
      if (n == "format" || n == "shape") *fused.add_attribute() = a;
    }
    ol::utils::RepeatedProtoField<NodeProto> out;
    out.push_back(std::move(fused));
    return out;
  }
};

// ---------------------------------------------------------------------------
// ai.rt:Dequantize(Q; dtype) over a constant encoded weight Q (logical
// [N, K]) -> Transpose(perm = [1, 0]) -> MatMul(A, .), A of the same FLOAT16 /
// BFLOAT16 dtype -> ai.rt.amd:DequantizeEncodedMatMul(A, Q).  The encoding
// (AWQ, GPTQ or another) is resolved by the session kernel.
class DequantizeEncodedMatMulGpuPattern : public builder::PatternOptimization {
public:
  DequantizeEncodedMatMulGpuPattern()
      : builder::PatternOptimization(1, "DequantizeEncodedMatMulGpu", sym::Device::kGPU0) {}

  std::set<std::string> FastOpType() const override { return {"MatMul"}; }

  builder::MatchResult Match(builder::GraphGraph &graph, const NodeProto &candidate) const override {
    if (!IsOnnxOp(candidate, "MatMul") || candidate.input_size() != 2) return NoMatch(candidate, "not a MatMul");
    const NodeProto *tr = graph.NodeBefore(In(candidate, 1));
    if (tr == nullptr || !IsOnnxOp(*tr, "Transpose"))
      return NoMatch(candidate, "MatMul's second input is not a Transpose output");
    std::vector<int64_t> perm;
    if (ol::GetAttributeInts(*tr, "perm", perm) && perm != std::vector<int64_t>{1, 0})
      return NoMatch(candidate, "Transpose is not a 2-D transpose");
    if (!SingleUse(graph, Out(*tr, 0), candidate)) return NoMatch(candidate, "Transpose output has another consumer");
    const NodeProto *dq = graph.NodeBefore(In(*tr, 0));
    if (dq == nullptr || dq->op_type().value() != "Dequantize" || dq->domain().value() != "ai.rt")
      return NoMatch(candidate, "Transpose input is not an ai.rt Dequantize output");
    if (!SingleUse(graph, Out(*dq, 0), *tr)) return NoMatch(candidate, "Dequantize output has another consumer");
    if (!graph.IsConstant(In(*dq, 0))) return NoMatch(candidate, "encoded weight is not an initializer");
    const int64_t dtype = ol::GetAttributeOr<int64_t>(*dq, "dtype", 0);
    if (dtype != kFloat16 && dtype != kBfloat16) return NoMatch(candidate, "Dequantize dtype is not FLOAT16 or BFLOAT16");
    if (!graph.HasType(In(candidate, 0))) return NoMatch(candidate, "type of A unknown");
    const TensorType a_type = graph.GetType(In(candidate, 0));
    if ((dtype == kFloat16 && a_type != TensorType::kFloat16) || (dtype == kBfloat16 && a_type != TensorType::kBfloat16))
      return NoMatch(candidate, "type of A differs from the Dequantize dtype");
    return builder::MatchResult{this, {dq, tr, &candidate}, &candidate};
  }

  ol::utils::RepeatedProtoField<NodeProto> Apply(builder::GraphGraph &graph,
                                                 const std::vector<const NodeProto *> &nodes) const override {
    const builder::MatchResult verified =
        nodes.size() != 3 || nodes[2] == nullptr ? builder::MatchResult{} : Match(graph, *nodes[2]);
    if (verified.pattern == nullptr || verified.nodes != nodes)
      throw builder::BuilderError("DequantizeEncodedMatMulGpuPattern::Apply received an unsafe or inconsistent match.");
    const NodeProto &dq = *nodes[0], &matmul = *nodes[2];
    const std::string name = "DequantizeEncodedMatMulGpu--" + std::string(matmul.name().value());
    NodeProto fused = ol::MakeNode("DequantizeEncodedMatMul", {In(matmul, 0), In(dq, 0)}, Outputs(matmul),
                                   kFusedDomain, name.c_str());
    ol::utils::RepeatedProtoField<NodeProto> out;
    out.push_back(std::move(fused));
    return out;
  }
};

// ---------------------------------------------------------------------------
// W, s[, zp] (constant quantized experts [G, K, N] or [G, N, K]) ->
// DequantizeLinear(axis) -> [Cast(to = FLOAT16 | BFLOAT16)] ->
// GroupedMatMul(input, ., group_indices[, bias]; transB)
// => ai.rt.amd:DequantizeLinearGroupedMatMul(input, W, s, zp | "",
//    group_indices[, bias]; axis, cast_to, transB)
class DequantizeLinearGroupedMatMulGpuPattern : public builder::PatternOptimization {
public:
  explicit DequantizeLinearGroupedMatMulGpuPattern(bool fp8_scaled_sums = false)
      : builder::PatternOptimization(1, "DequantizeLinearGroupedMatMulGpu", sym::Device::kGPU0),
        fp8_scaled_sums_(fp8_scaled_sums) {}

  std::set<std::string> FastOpType() const override { return {"GroupedMatMul"}; }

  builder::MatchResult Match(builder::GraphGraph &graph, const NodeProto &candidate) const override {
    if (!IsOnnxOp(candidate, "GroupedMatMul") || candidate.input_size() < 3 || candidate.input_size() > 4)
      return NoMatch(candidate, "not a GroupedMatMul");
    if (!OnlyAttributes(candidate, {"transB"})) return NoMatch(candidate, "GroupedMatMul attribute other than transB");
    const int64_t trans_b = ol::GetAttributeOr<int64_t>(candidate, "transB", 0);
    const NodeProto *cast = nullptr;
    const NodeProto *prod = graph.NodeBefore(In(candidate, 1));
    int64_t cast_to = 0;
    if (prod != nullptr && IsOnnxOp(*prod, "Cast")) {
      cast_to = ol::GetAttributeOr<int64_t>(*prod, "to", 0);
      if (cast_to != kFloat16 && cast_to != kBfloat16)
        return NoMatch(candidate, "Cast target is not FLOAT16 or BFLOAT16");
      if (!SingleUse(graph, Out(*prod, 0), candidate)) return NoMatch(candidate, "Cast output has another consumer");
      cast = prod;
      prod = graph.NodeBefore(In(*prod, 0));
    }
    if (prod == nullptr || !IsOnnxOp(*prod, "DequantizeLinear"))
      return NoMatch(candidate, "GroupedMatMul's weights are not a DequantizeLinear output");
    if (!OnlyAttributes(*prod, {"axis"})) return NoMatch(candidate, "DequantizeLinear attribute other than axis");
    std::vector<const TensorProto *> meta;
    for (int i = 0; i < prod->input_size(); ++i) {
      if (In(*prod, i).empty()) continue;
      if (!graph.IsConstant(In(*prod, i))) return NoMatch(candidate, "DequantizeLinear inputs are not all initializers");
      meta.push_back(graph.GetConstantMetadata(In(*prod, i)));
    }
    if (meta.size() < 2) return NoMatch(candidate, "DequantizeLinear inputs are not all initializers");
    if (!SingleUse(graph, Out(*prod, 0), cast != nullptr ? *cast : candidate))
      return NoMatch(candidate, "DequantizeLinear output has another consumer");
    for (const TensorProto *m : meta)
      if (m == nullptr) return NoMatch(candidate, "type or shape of a DequantizeLinear input unknown");

    // The fused entry point's checks: DequantizeLinear's rules for 3-D
    // experts, the Cast's, and the 16-bit GroupedMatMul.
    const int32_t w_t = meta[0]->data_type(), s_t = meta[1]->data_type();
    const std::vector<int64_t> w = Dims(*meta[0]), s = Dims(*meta[1]);
    if (w_t != kInt4 && w_t != kUint4 && w_t != kInt8 && w_t != kUint8 && w_t != kFloat8E4M3FN)
      return NoMatch(candidate, "weight type has no fused kernel");
    if (w.size() != 3) return NoMatch(candidate, "experts are not 3-D");
    if (s_t != kFloat && s_t != kFloat16) return NoMatch(candidate, "scale is not FLOAT or FLOAT16");
    const bool has_zp = meta.size() > 2;
    if (has_zp && (meta[2]->data_type() != w_t || Dims(*meta[2]) != s))
      return NoMatch(candidate, "zero point type or shape does not match");
    const int64_t axis = ol::GetAttributeOr<int64_t>(*prod, "axis", 1);
    int64_t count = 1;
    for (int64_t d : s) count *= d;
    bool along_k = false;  // the scale varies along K inside an expert
    if (count != 1) {
      if (axis < 0 || axis >= 3) return NoMatch(candidate, "axis out of range");
      if (s.size() == 3) {
        for (int d = 0; d < 3; ++d)
          if (s[d] <= 0 || w[d] % s[d] != 0 || (d != axis && s[d] != w[d]))
            return NoMatch(candidate, "blocked scale does not fit the weight");
        along_k = !(axis == 1 && s[1] == 1);
      } else if (s.size() == 1) {
        if (count != w[axis]) return NoMatch(candidate, "scale size differs from the axis dimension");
        along_k = axis == 1;
      } else {
        return NoMatch(candidate, "scale rank is neither 1 nor 3");
      }
    }
    if (cast_to != 0 && s_t != kFloat) return NoMatch(candidate, "Cast of a FLOAT16 DequantizeLinear output");
    const int64_t run_type = cast_to != 0 ? cast_to : s_t;
    if (run_type != kFloat16 && run_type != kBfloat16) return NoMatch(candidate, "GroupedMatMul would run in FLOAT");
    if (w_t == kFloat8E4M3FN && cast_to == kBfloat16 && s_t == kFloat && !has_zp && trans_b == 0 && !along_k &&
        !fp8_scaled_sums_)
      return NoMatch(candidate, "FLOAT8E4M3FN -> BFLOAT16 chain would scale the sums (fp8_scaled_sums=True allows it)");

    std::vector<const NodeProto *> nodes{prod};
    if (cast != nullptr) nodes.push_back(cast);
    nodes.push_back(&candidate);
    return builder::MatchResult{this, nodes, &candidate};
  }

  ol::utils::RepeatedProtoField<NodeProto> Apply(builder::GraphGraph &graph,
                                                 const std::vector<const NodeProto *> &nodes) const override {
    const builder::MatchResult verified = nodes.empty() || nodes.back() == nullptr
                                              ? builder::MatchResult{}
                                              : Match(graph, *nodes.back());
    if (verified.pattern == nullptr || verified.nodes != nodes)
      throw builder::BuilderError(
          "DequantizeLinearGroupedMatMulGpuPattern::Apply received an unsafe or inconsistent match.");
    const NodeProto &dq = *nodes.front(), &gmm = *nodes.back();
    const int64_t cast_to = nodes.size() == 3 ? ol::GetAttributeOr<int64_t>(*nodes[1], "to", 0) : 0;
    std::vector<std::string> inputs{In(gmm, 0), In(dq, 0), In(dq, 1), dq.input_size() > 2 ? In(dq, 2) : "",
                                    In(gmm, 2)};
    if (gmm.input_size() > 3) inputs.push_back(In(gmm, 3));
    while (inputs.size() > 1 && inputs.back().empty()) inputs.pop_back();
    const std::string name = "DequantizeLinearGroupedMatMulGpu--" + std::string(gmm.name().value());
    NodeProto fused = ol::MakeNode("DequantizeLinearGroupedMatMul", inputs, Outputs(gmm), kFusedDomain, name.c_str());
    AddInt(fused, "axis", ol::GetAttributeOr<int64_t>(dq, "axis", 1));
    AddInt(fused, "cast_to", cast_to);
    AddInt(fused, "transB", ol::GetAttributeOr<int64_t>(gmm, "transB", 0));
    ol::utils::RepeatedProtoField<NodeProto> out;
    out.push_back(std::move(fused));
    return out;
  }

private:
  bool fp8_scaled_sums_;
};

}  // namespace mi355x_patterns

// Makes the four rewrites available by name; none is enabled by default.
void RegisterMi355xPatterns() {
  namespace builder = ONNX_LIGHT_NAMESPACE::core::builder;
  builder::RegisterPattern(
      "DequantizeLinearMatMulGpu",
      []() -> std::unique_ptr<builder::PatternOptimization> {
        return std::make_unique<mi355x_patterns::DequantizeLinearMatMulGpuPattern>();
      },
      /*enabled_by_default=*/false);
  builder::RegisterPattern(
      "DequantizePackedMatMulGpu",
      []() -> std::unique_ptr<builder::PatternOptimization> {
        return std::make_unique<mi355x_patterns::DequantizePackedMatMulGpuPattern>();
      },
      /*enabled_by_default=*/false);
  builder::RegisterPattern(
      "DequantizeEncodedMatMulGpu",
      []() -> std::unique_ptr<builder::PatternOptimization> {
        return std::make_unique<mi355x_patterns::DequantizeEncodedMatMulGpuPattern>();
      },
      /*enabled_by_default=*/false);
  builder::RegisterPattern(
      "DequantizeLinearGroupedMatMulGpu",
      []() -> std::unique_ptr<builder::PatternOptimization> {
        return std::make_unique<mi355x_patterns::DequantizeLinearGroupedMatMulGpuPattern>();
      },
      /*enabled_by_default=*/false);
}
