"""Graph rewrites that hand DequantizeLinear -> [Cast] -> MatMul and
DequantizePacked -> Transpose -> MatMul to the fused GPU kernels.

Mirrors the reference's pattern interface: a pattern's ``match`` returns the
nodes of a rewrite in the order ``apply`` expects, or a no-match carrying the
reason (PatternOptimization::Match / Apply / NoMatch,
onnx_core/builder/pattern_optimization.h:142-224), and patterns are
registered by name with an opt-in flag (RegisterPattern,
onnx_core/builder/pattern_registry.h:36-37; CreateRegisteredPatterns with a
device filter, :65-72).  Sessions of the reference apply no patterns, so a
caller rewrites the in-memory model before binding it; the file on disk is
unchanged.

The graph here is a plain node list: each node names its inputs and outputs,
initializers are the names of constant tensors.  The rewrite:

    W, s[, zp] (initializers) -> DequantizeLinear(axis) -> [Cast(to=FLOAT16 |
    BFLOAT16)] -> MatMul(A, .)

becomes one node ``ai.rt.amd:DequantizeLinearMatMul(A, W, s[, zp])`` with
attributes ``axis`` and ``cast_to`` (0 when there is no Cast), computed by
``dequantize_linear_matmul``.  The intermediate tensors must have no other
consumer and must not be graph outputs.

The rewrite only fires where the fused kernel accepts the node, so a graph
that runs unfused never becomes one that raises.  That needs the element type
and shape of W, s and zp (``Graph.value_info``, as an ONNX model's
initializers carry them); a chain without them is left alone.  The checks are
those of the fused entry point (DequantizeLinear's own, kq/kernel_
dequantizelinear.cc:522-565, then the fused kernel's limits): W is a 2-D
INT4 / UINT4 / INT8 / UINT8 / FLOAT8E4M3FN tensor; s is FLOAT or FLOAT16 and
either a scalar, 1-D along axis 1 (per output column) or 2-D blocked along
axis 0 (K); zp matches W's type and s's shape; the MatMul runs in FLOAT16 or
BFLOAT16 (a FLOAT DequantizeLinear needs the Cast, a FLOAT16 one must not
have one).  FLOAT8E4M3FN weights with a FLOAT per-tensor / per-column scale,
no zero point and a Cast to BFLOAT16 take the matrix-core path that scales
the fp32 sums instead of rounding each scaled weight to bfloat16; the pattern
rewrites such chains only when built with ``fp8_scaled_sums=True``.
"""
from __future__ import annotations

import dataclasses
from typing import Callable, Dict, List, Optional, Sequence

FUSED_DOMAIN = "ai.rt.amd"
FUSED_OP = "DequantizeLinearMatMul"
PACKED_FUSED_OP = "DequantizePackedMatMul"
ENCODED_FUSED_OP = "DequantizeEncodedMatMul"
GROUPED_FUSED_OP = "DequantizeLinearGroupedMatMul"
# the 27 GGUF profiles of DequantizePacked (format: values per block); the
# fused node runs every one of them on the GPU (decode GEMVs for q4_0, q8_0,
# q2_k, q3_k, q4_k, q5_k, q6_k and iq4_xs, the decoded weight through the
# MFMA GEMM otherwise)
_PACKED_FORMATS = {f: 32 for f in ("gguf:q4_0", "gguf:q4_1", "gguf:q5_0", "gguf:q5_1", "gguf:q8_0", "gguf:q8_1",
                                   "gguf:iq4_nl", "gguf:mxfp4")}
_PACKED_FORMATS.update({f: 256 for f in ("gguf:q2_k", "gguf:q3_k", "gguf:q4_k", "gguf:q5_k", "gguf:q6_k",
                                         "gguf:q8_k", "gguf:iq2_xxs", "gguf:iq2_xs", "gguf:iq3_xxs", "gguf:iq1_s",
                                         "gguf:iq3_s", "gguf:iq2_s", "gguf:iq4_xs", "gguf:iq1_m", "gguf:tq1_0",
                                         "gguf:tq2_0")})
_PACKED_FORMATS.update({"gguf:nvfp4": 64, "gguf:q2_0": 64, "gguf:q1_0": 128})
_ONNX_DOMAINS = ("", "ai.onnx")
_CAST_TARGETS = (10, 16)  # FLOAT16, BFLOAT16: the types the fused kernel rounds to
FLOAT, UINT8, INT8, FLOAT16, BFLOAT16, FLOAT8E4M3FN, UINT4, INT4 = 1, 2, 3, 10, 16, 17, 21, 22
_WEIGHT_TYPES = (INT4, UINT4, INT8, UINT8, FLOAT8E4M3FN)
_SCALE_TYPES = (FLOAT, FLOAT16)


@dataclasses.dataclass
class Node:
    op_type: str
    inputs: List[str]
    outputs: List[str]
    domain: str = ""
    attrs: Dict[str, object] = dataclasses.field(default_factory=dict)
    name: str = ""


@dataclasses.dataclass
class Graph:
    nodes: List[Node]
    initializers: set = dataclasses.field(default_factory=set)
    inputs: List[str] = dataclasses.field(default_factory=list)
    outputs: List[str] = dataclasses.field(default_factory=list)
    # name -> (ONNX element type, shape) for the tensors whose types are known
    value_info: Dict[str, tuple] = dataclasses.field(default_factory=dict)

    def producer(self, name: str) -> Optional[Node]:
        for n in self.nodes:
            if name in n.outputs:
                return n
        return None

    def consumers(self, name: str) -> List[Node]:
        return [n for n in self.nodes if name in n.inputs]


@dataclasses.dataclass
class MatchResult:
    """nodes: the rewrite's nodes in the order ``apply`` expects (empty on no
    match); reason: why the candidate did not match."""
    nodes: List[Node]
    reason: str = ""

    def __bool__(self) -> bool:
        return bool(self.nodes)


class PatternOptimization:
    """Base class: ``match`` a candidate node, ``apply`` a match."""
    device: Optional[str] = None  # None: device-independent

    def fast_op_type(self) -> set:
        return set()

    def match(self, graph: Graph, candidate: Node) -> MatchResult:
        raise NotImplementedError

    def apply(self, graph: Graph, nodes: Sequence[Node]) -> List[Node]:
        raise NotImplementedError

    @staticmethod
    def no_match(reason: str) -> MatchResult:
        return MatchResult([], reason)


def _is_onnx(node: Node, op_type: str) -> bool:
    return node.op_type == op_type and node.domain in _ONNX_DOMAINS


class DequantizeLinearMatMulPattern(PatternOptimization):
    """DequantizeLinear over constant inputs, an optional Cast to FLOAT16 or
    BFLOAT16, then MatMul's second input -> one fused node."""
    device = "gpu"

    def fast_op_type(self) -> set:
        return {"MatMul"}

    def __init__(self, fp8_scaled_sums: bool = False):
        self.fp8_scaled_sums = fp8_scaled_sums

    @staticmethod
    def _single_use(graph: Graph, name: str, user: Node) -> bool:
        """name feeds exactly one input slot in the graph, an input of `user`,
        and is not a graph output (MatMul(Wd, Wd) uses Wd twice)."""
        slots = [n for n in graph.nodes for i in n.inputs if i == name]
        return len(slots) == 1 and slots[0] is user and name not in graph.outputs

    def _check_types(self, graph: Graph, dq: Node, cast_to: int) -> str:
        """Why the fused kernel would refuse this chain ("" if it accepts it)."""
        info = graph.value_info
        names = [i for i in dq.inputs if i]
        if any(i not in info for i in names):
            return "type or shape of a DequantizeLinear input unknown"
        (w_t, w_shape), (s_t, s_shape) = info[names[0]], info[names[1]]
        zp = info[names[2]] if len(names) > 2 else None
        w_shape, s_shape = tuple(w_shape), tuple(s_shape)
        if w_t not in _WEIGHT_TYPES:
            return "weight type has no fused kernel"
        if len(w_shape) != 2:
            return "weight is not 2-D"
        if s_t not in _SCALE_TYPES:
            return "scale is not FLOAT or FLOAT16"
        if zp is not None and (zp[0] != w_t or tuple(zp[1]) != s_shape):
            return "zero point type or shape does not match"
        axis = int(dq.attrs.get("axis", 1))
        count = 1
        for d in s_shape:
            count *= d
        per_tensor = count == 1
        if not per_tensor:
            if not 0 <= axis < 2:
                return "axis out of range"
            if len(s_shape) == 2:
                if any(s_shape[d] <= 0 or w_shape[d] % s_shape[d] or (d != axis and s_shape[d] != w_shape[d])
                       for d in range(2)):
                    return "blocked scale does not fit the weight"
                if axis != 0:
                    return "scales blocked along N"
            elif len(s_shape) == 1:
                if count != w_shape[axis]:
                    return "scale size differs from the axis dimension"
                if axis != 1:
                    return "per-row (axis 0) scales"
            else:
                return "scale rank above 2"
        if cast_to and s_t != FLOAT:
            return "Cast of a FLOAT16 DequantizeLinear output"
        if (cast_to or s_t) not in (FLOAT16, BFLOAT16):
            return "MatMul would run in FLOAT"
        if (w_t == FLOAT8E4M3FN and cast_to == BFLOAT16 and s_t == FLOAT and zp is None
                and (per_tensor or len(s_shape) == 1) and not self.fp8_scaled_sums):
            return "FLOAT8E4M3FN -> BFLOAT16 chain would scale the sums (fp8_scaled_sums=True allows it)"
        return ""

    def match(self, graph: Graph, candidate: Node) -> MatchResult:
        if not _is_onnx(candidate, "MatMul") or len(candidate.inputs) != 2:
            return self.no_match("not a MatMul")
        cast = None
        prod = graph.producer(candidate.inputs[1])
        if prod is not None and _is_onnx(prod, "Cast"):
            if int(prod.attrs.get("to", 0)) not in _CAST_TARGETS:
                return self.no_match("Cast target is not FLOAT16 or BFLOAT16")
            if not self._single_use(graph, prod.outputs[0], candidate):
                return self.no_match("Cast output has another consumer")
            cast, prod = prod, graph.producer(prod.inputs[0])
        if prod is None or not _is_onnx(prod, "DequantizeLinear"):
            return self.no_match("MatMul's second input is not a DequantizeLinear output")
        if set(prod.attrs) - {"axis"}:
            return self.no_match("DequantizeLinear attribute other than axis")
        consts = [i for i in prod.inputs if i]
        if len(consts) < 2 or any(i not in graph.initializers for i in consts):
            return self.no_match("DequantizeLinear inputs are not all initializers")
        if not self._single_use(graph, prod.outputs[0], cast if cast is not None else candidate):
            return self.no_match("DequantizeLinear output has another consumer")
        why = self._check_types(graph, prod, int(cast.attrs["to"]) if cast is not None else 0)
        if why:
            return self.no_match(why)
        return MatchResult([prod] + ([cast] if cast is not None else []) + [candidate])

    def apply(self, graph: Graph, nodes: Sequence[Node]) -> List[Node]:
        dq, matmul = nodes[0], nodes[-1]
        cast_to = int(nodes[1].attrs["to"]) if len(nodes) == 3 else 0
        inputs = [matmul.inputs[0]] + [i for i in dq.inputs]
        while inputs and not inputs[-1]:
            inputs.pop()
        return [Node(FUSED_OP, inputs, list(matmul.outputs), FUSED_DOMAIN,
                     {"axis": int(dq.attrs.get("axis", 1)), "cast_to": cast_to},
                     matmul.name or dq.name)]


class DequantizePackedMatMulPattern(PatternOptimization):
    """DequantizePacked(x; format, shape = [N, K], output_dtype = FLOAT16) over
    a constant x -> Transpose(perm = [1, 0]) -> MatMul's second input, with a
    FLOAT16 A -> one fused node ``ai.rt.amd:DequantizePackedMatMul(A, x)``
    with attributes format and shape, computed by
    ``dequantize_packed_matmul``, which runs every GGUF profile and row count
    on the device (fused decode GEMVs up to 8 rows of A, the decoded weight
    through the MFMA GEMM otherwise)."""
    device = "gpu"

    def fast_op_type(self) -> set:
        return {"MatMul"}

    def match(self, graph: Graph, candidate: Node) -> MatchResult:
        if not _is_onnx(candidate, "MatMul") or len(candidate.inputs) != 2:
            return self.no_match("not a MatMul")
        tr = graph.producer(candidate.inputs[1])
        if tr is None or not _is_onnx(tr, "Transpose"):
            return self.no_match("MatMul's second input is not a Transpose output")
        if [int(p) for p in tr.attrs.get("perm", [1, 0])] != [1, 0]:
            return self.no_match("Transpose is not a 2-D transpose")
        if not DequantizeLinearMatMulPattern._single_use(graph, tr.outputs[0], candidate):
            return self.no_match("Transpose output has another consumer")
        dp = graph.producer(tr.inputs[0])
        if dp is None or not _is_onnx(dp, "DequantizePacked"):
            return self.no_match("Transpose input is not a DequantizePacked output")
        if not DequantizeLinearMatMulPattern._single_use(graph, dp.outputs[0], tr):
            return self.no_match("DequantizePacked output has another consumer")
        if dp.inputs[0] not in graph.initializers:
            return self.no_match("packed weight is not an initializer")
        fmt = dp.attrs.get("format")
        if fmt not in _PACKED_FORMATS:
            return self.no_match("unknown packed format")
        shape = [int(d) for d in dp.attrs.get("shape", [])]
        if len(shape) != 2:
            return self.no_match("DequantizePacked shape is not [N, K]")
        if int(dp.attrs.get("output_dtype", FLOAT)) != FLOAT16:
            return self.no_match("DequantizePacked output is not FLOAT16")
        if shape[1] % _PACKED_FORMATS[fmt]:
            return self.no_match("K is not a whole number of blocks")
        a_info = graph.value_info.get(candidate.inputs[0])
        if a_info is None:
            return self.no_match("type of A unknown")
        if a_info[0] != FLOAT16:
            return self.no_match("A is not FLOAT16")
        return MatchResult([dp, tr, candidate])

    def apply(self, graph: Graph, nodes: Sequence[Node]) -> List[Node]:
        dp, _, matmul = nodes
        return [Node(PACKED_FUSED_OP, [matmul.inputs[0], dp.inputs[0]], list(matmul.outputs), FUSED_DOMAIN,
                     {"format": dp.attrs["format"], "shape": [int(d) for d in dp.attrs["shape"]]},
                     matmul.name or dp.name)]


class DequantizeEncodedMatMulPattern(PatternOptimization):
    """ai.rt:Dequantize(Q; dtype) over a constant encoded weight Q (logical
    [N, K]) -> Transpose(perm = [1, 0]) -> MatMul's second input, with A of
    the same FLOAT16 / BFLOAT16 dtype -> one fused node
    ``ai.rt.amd:DequantizeEncodedMatMul(A, Q)``.  The session kernel prepares
    an AWQ or GPTQ weight once for the fused DequantizeLinear -> MatMul
    kernels and computes the chain for any other encoding (the encoding is
    resolved from the model's struct types at run time, not here)."""
    device = "gpu"

    def fast_op_type(self) -> set:
        return {"MatMul"}

    def match(self, graph: Graph, candidate: Node) -> MatchResult:
        if not _is_onnx(candidate, "MatMul") or len(candidate.inputs) != 2:
            return self.no_match("not a MatMul")
        tr = graph.producer(candidate.inputs[1])
        if tr is None or not _is_onnx(tr, "Transpose"):
            return self.no_match("MatMul's second input is not a Transpose output")
        if [int(p) for p in tr.attrs.get("perm", [1, 0])] != [1, 0]:
            return self.no_match("Transpose is not a 2-D transpose")
        if not DequantizeLinearMatMulPattern._single_use(graph, tr.outputs[0], candidate):
            return self.no_match("Transpose output has another consumer")
        dq = graph.producer(tr.inputs[0])
        if dq is None or dq.op_type != "Dequantize" or dq.domain != "ai.rt":
            return self.no_match("Transpose input is not an ai.rt Dequantize output")
        if not DequantizeLinearMatMulPattern._single_use(graph, dq.outputs[0], tr):
            return self.no_match("Dequantize output has another consumer")
        if dq.inputs[0] not in graph.initializers:
            return self.no_match("encoded weight is not an initializer")
        dtype = int(dq.attrs.get("dtype", 0))
        if dtype not in (FLOAT16, BFLOAT16):
            return self.no_match("Dequantize dtype is not FLOAT16 or BFLOAT16")
        a_info = graph.value_info.get(candidate.inputs[0])
        if a_info is None:
            return self.no_match("type of A unknown")
        if a_info[0] != dtype:
            return self.no_match("type of A differs from the Dequantize dtype")
        return MatchResult([dq, tr, candidate])

    def apply(self, graph: Graph, nodes: Sequence[Node]) -> List[Node]:
        dq, _, matmul = nodes
        return [Node(ENCODED_FUSED_OP, [matmul.inputs[0], dq.inputs[0]], list(matmul.outputs), FUSED_DOMAIN, {},
                     matmul.name or dq.name)]


class DequantizeLinearGroupedMatMulPattern(PatternOptimization):
    """DequantizeLinear over constant quantized experts x [G, K, N] ([G, N, K]
    with transB), an optional Cast to FLOAT16 or BFLOAT16, then
    GroupedMatMul's weights -> one fused node
    ``ai.rt.amd:DequantizeLinearGroupedMatMul(input, x, scale, zero_point,
    group_indices[, bias])`` with attributes axis, cast_to and transB,
    computed by ``dequantize_linear_grouped_matmul``.  As for the 2-D rewrite,
    fp8 experts whose Cast to BFLOAT16 the fused kernel replaces by scaled
    sums match only with ``fp8_scaled_sums``."""
    device = "gpu"

    def fast_op_type(self) -> set:
        return {"GroupedMatMul"}

    def __init__(self, fp8_scaled_sums: bool = False):
        self.fp8_scaled_sums = fp8_scaled_sums

    def _check_types(self, graph: Graph, dq: Node, cast_to: int, trans_b: int) -> str:
        """Why the fused entry point would refuse this chain ("" if it accepts it)."""
        info = graph.value_info
        names = [i for i in dq.inputs if i]
        if any(i not in info for i in names):
            return "type or shape of a DequantizeLinear input unknown"
        (w_t, w_shape), (s_t, s_shape) = info[names[0]], info[names[1]]
        zp = info[names[2]] if len(names) > 2 else None
        w_shape, s_shape = tuple(w_shape), tuple(s_shape)
        if w_t not in _WEIGHT_TYPES:
            return "weight type has no fused kernel"
        if len(w_shape) != 3:
            return "experts are not 3-D"
        if s_t not in _SCALE_TYPES:
            return "scale is not FLOAT or FLOAT16"
        if zp is not None and (zp[0] != w_t or tuple(zp[1]) != s_shape):
            return "zero point type or shape does not match"
        axis = int(dq.attrs.get("axis", 1))
        count = 1
        for d in s_shape:
            count *= d
        per_tensor = count == 1
        along_k = False  # the scale varies along K inside an expert
        if not per_tensor:
            if not 0 <= axis < 3:
                return "axis out of range"
            if len(s_shape) == 3:
                if any(s_shape[d] <= 0 or w_shape[d] % s_shape[d] or (d != axis and s_shape[d] != w_shape[d])
                       for d in range(3)):
                    return "blocked scale does not fit the weight"
                along_k = not (axis == 1 and s_shape[1] == 1)
            elif len(s_shape) == 1:
                if count != w_shape[axis]:
                    return "scale size differs from the axis dimension"
                along_k = axis == 1
            else:
                return "scale rank is neither 1 nor 3"
        if cast_to and s_t != FLOAT:
            return "Cast of a FLOAT16 DequantizeLinear output"
        if (cast_to or s_t) not in (FLOAT16, BFLOAT16):
            return "GroupedMatMul would run in FLOAT"
        if (w_t == FLOAT8E4M3FN and cast_to == BFLOAT16 and s_t == FLOAT and zp is None and not trans_b
                and not along_k and not self.fp8_scaled_sums):
            return "FLOAT8E4M3FN -> BFLOAT16 chain would scale the sums (fp8_scaled_sums=True allows it)"
        return ""

    def match(self, graph: Graph, candidate: Node) -> MatchResult:
        if not _is_onnx(candidate, "GroupedMatMul") or not 3 <= len(candidate.inputs) <= 4:
            return self.no_match("not a GroupedMatMul")
        if set(candidate.attrs) - {"transB"}:
            return self.no_match("GroupedMatMul attribute other than transB")
        cast = None
        prod = graph.producer(candidate.inputs[1])
        if prod is not None and _is_onnx(prod, "Cast"):
            if int(prod.attrs.get("to", 0)) not in _CAST_TARGETS:
                return self.no_match("Cast target is not FLOAT16 or BFLOAT16")
            if not DequantizeLinearMatMulPattern._single_use(graph, prod.outputs[0], candidate):
                return self.no_match("Cast output has another consumer")
            cast, prod = prod, graph.producer(prod.inputs[0])
        if prod is None or not _is_onnx(prod, "DequantizeLinear"):
            return self.no_match("GroupedMatMul's weights are not a DequantizeLinear output")
        if set(prod.attrs) - {"axis"}:
            return self.no_match("DequantizeLinear attribute other than axis")
        consts = [i for i in prod.inputs if i]
        if len(consts) < 2 or any(i not in graph.initializers for i in consts):
            return self.no_match("DequantizeLinear inputs are not all initializers")
        if not DequantizeLinearMatMulPattern._single_use(graph, prod.outputs[0],
                                                          cast if cast is not None else candidate):
            return self.no_match("DequantizeLinear output has another consumer")
        why = self._check_types(graph, prod, int(cast.attrs["to"]) if cast is not None else 0,
                                int(candidate.attrs.get("transB", 0)))
        if why:
            return self.no_match(why)
        return MatchResult([prod] + ([cast] if cast is not None else []) + [candidate])

    def apply(self, graph: Graph, nodes: Sequence[Node]) -> List[Node]:
        dq, gmm = nodes[0], nodes[-1]
        cast_to = int(nodes[1].attrs["to"]) if len(nodes) == 3 else 0
        zp = dq.inputs[2] if len(dq.inputs) > 2 else ""
        inputs = [gmm.inputs[0], dq.inputs[0], dq.inputs[1], zp, gmm.inputs[2]] + list(gmm.inputs[3:4])
        while inputs and not inputs[-1]:
            inputs.pop()
        return [Node(GROUPED_FUSED_OP, inputs, list(gmm.outputs), FUSED_DOMAIN,
                     {"axis": int(dq.attrs.get("axis", 1)), "cast_to": cast_to,
                      "transB": int(gmm.attrs.get("transB", 0))}, gmm.name or dq.name)]


# ---- registry --------------------------------------------------------------

_REGISTRY: Dict[str, tuple] = {}


def register_pattern(name: str, factory: Callable[[], PatternOptimization], enabled_by_default: bool = True):
    """Registers a pattern factory under a unique, non-empty name; order of
    registration is the order of ``create_registered_patterns``."""
    if not name or name in _REGISTRY:
        raise ValueError(f"pattern name {name!r} is empty or already registered")
    _REGISTRY[name] = (factory, enabled_by_default)


def registered_pattern_names(include_opt_in: bool = True) -> List[str]:
    return [n for n, (_, on) in _REGISTRY.items() if on or include_opt_in]


def create_registered_pattern(name: str) -> PatternOptimization:
    return _REGISTRY[name][0]()


def create_registered_patterns(device: Optional[str] = None) -> List[PatternOptimization]:
    """Patterns enabled by default; with a device, the device-independent ones
    and those for that device."""
    out = []
    for factory, on in _REGISTRY.values():
        if not on:
            continue
        p = factory()
        if p.device is None or (device is not None and p.device == device):
            out.append(p)
    return out


register_pattern("DequantizeLinearMatMulGpu", DequantizeLinearMatMulPattern, enabled_by_default=False)
register_pattern("DequantizePackedMatMulGpu", DequantizePackedMatMulPattern, enabled_by_default=False)
register_pattern("DequantizeEncodedMatMulGpu", DequantizeEncodedMatMulPattern, enabled_by_default=False)
register_pattern("DequantizeLinearGroupedMatMulGpu", DequantizeLinearGroupedMatMulPattern, enabled_by_default=False)


def optimize(graph: Graph, patterns: Sequence[PatternOptimization]) -> int:
    """Applies the patterns until none matches; returns the rewrite count.
    Each rewrite replaces its nodes, in place, at the position of the last."""
    count = 0
    changed = True
    while changed:
        changed = False
        for pat in patterns:
            fast = pat.fast_op_type()
            for cand in list(graph.nodes):
                if fast and cand.op_type not in fast:
                    continue
                m = pat.match(graph, cand)
                if not m:
                    continue
                new = pat.apply(graph, m.nodes)
                at = max(i for i, n in enumerate(graph.nodes) if any(n is x for x in m.nodes))
                keep = [n for i, n in enumerate(graph.nodes) if not any(n is x for x in m.nodes) or i == at]
                pos = next(i for i, n in enumerate(keep) if n is graph.nodes[at])
                graph.nodes = keep[:pos] + new + keep[pos + 1:]
                count += 1
                changed = True
                break
            if changed:
                break
    return count
