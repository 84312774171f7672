"""Graph rewrite that hands DequantizeLinear -> [Cast] -> MatMul to the fused
GPU kernel.

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
"""
from __future__ import annotations

import dataclasses
from typing import Callable, Dict, List, Optional, Sequence

FUSED_DOMAIN = "ai.rt.amd"
FUSED_OP = "DequantizeLinearMatMul"
_ONNX_DOMAINS = ("", "ai.onnx")
_CAST_TARGETS = (10, 16)  # FLOAT16, BFLOAT16: the types the fused kernel rounds to


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

    def _single_use(self, graph: Graph, name: str, user: Node) -> bool:
        users = graph.consumers(name)
        return len(users) == 1 and users[0] is user and name not in graph.outputs

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
