"""Static checks of the onnx-light adapter (adapter/register_mi355x.cc).

The adapter compiles inside the onnx-light tree only (the reference's headers
need a newer C++ library than this image has), so these CPU tests check its
text: every entry point the C ABI declares is called from it, with the
declared number of arguments; every operator of the path has a KernelBase
subclass that is registered; the preparation hooks are overridden; and, where
the reference sources are present, every runtime helper and header it uses
exists there."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "onnxl_amd.h")
ADAPTER = os.path.join(ROOT, "adapter", "register_mi355x.cc")
REFERENCE = "/root/reference/onnx_light"

OPERATORS = ["MatMulInteger", "QLinearMatMul", "DequantizeLinear", "MatMul", "QuantizeLinear",
             "DynamicQuantizeLinear", "ConvInteger", "QLinearConv", "Cast", "DequantizePacked",
             "GroupedMatMul", "MatMulNBits", "DequantizeLinearMatMul", "DequantizePackedMatMul", "Dequantize",
             "DequantizeEncodedMatMul", "DequantizeLinearGroupedMatMul"]


def _strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _args(text, open_idx):
    """Top-level arguments of the call whose '(' is at open_idx."""
    depth, start, out = 0, open_idx + 1, []
    for i in range(open_idx, len(text)):
        ch = text[i]
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
            if depth == 0:
                last = text[start:i].strip()
                if last or out:
                    out.append(last)
                return out
        elif ch == "," and depth == 1:
            out.append(text[start:i].strip())
            start = i + 1
    raise AssertionError("unbalanced call")


def _declarations():
    text = _strip_comments(open(HEADER).read())
    decls = {}
    for m in re.finditer(r"\b(?:int|const char \*)\s*(onnxl_amd_\w+)\s*\(", text):
        args = _args(text, m.end() - 1)
        decls[m.group(1)] = 0 if args == ["void"] else len(args)
    return decls


def _adapter():
    return _strip_comments(open(ADAPTER).read())


def test_header_declares_entry_points():
    decls = _declarations()
    assert len(decls) >= 20
    assert "onnxl_amd_dequantize_linear_matmul_noalloc" in decls


def test_every_entry_point_is_called_with_its_arity():
    decls = _declarations()
    text = _adapter()
    called = {}
    for m in re.finditer(r"\b(onnxl_amd_\w+)\s*\(", text):
        name = m.group(1)
        if name not in decls:
            continue
        called.setdefault(name, []).append(len(_args(text, m.end() - 1)))
    missing = sorted(set(decls) - set(called))
    assert not missing, f"entry points not called from the adapter: {missing}"
    for name, counts in called.items():
        assert all(c == decls[name] for c in counts), (name, counts, decls[name])


@pytest.mark.parametrize("op", OPERATORS)
def test_operator_has_registered_kernel_class(op):
    text = _adapter()
    cls = f"Mi355x{op}"
    assert re.search(rf"class {cls} : public Mi355xKernel\b", text), cls
    assert re.search(rf'static constexpr const char \*name = "onnxl_amd:CPU:[\w.]+:{op}";', text), cls
    assert re.search(rf"void Run\(rt::RuntimeContext &ctx\) override", text)
    domain = ("kFusedDomain" if op.endswith("MatMul") and op.startswith("Dequantize")
              else '"com.microsoft"' if op == "MatMulNBits" else '"ai.rt"' if op == "Dequantize" else '""')
    assert re.search(rf'Register<{cls}>\({re.escape(domain)}, "{op}"\);', text), cls


def test_preparation_hooks_and_entry():
    text = _adapter()
    assert "bool HasPreparations(const std::unordered_set<std::string> &immutable_inputs) const override" in text
    assert ("void DeclarePreparations(const std::unordered_set<std::string> &immutable_inputs,\n"
            "                           std::vector<rt::KernelPreparation> &preparations) override") in text
    assert re.search(r"const char \*RegisterMi355xKernelFunctions\(int device_ordinal = 0\)", text)
    assert "sym::Device::kCPU" in text
    assert "/*overwrite=*/true);" in open(ADAPTER).read()


def test_fused_pattern_names_match_adapter(olamd):
    """The fused node the Python pattern writes is the one the adapter
    registers (domain and op type)."""
    import importlib
    pat = importlib.import_module("onnx_light_amd.patterns")
    text = _adapter()
    assert f'constexpr const char *kFusedDomain = "{pat.FUSED_DOMAIN}";' in text
    assert f'Register<Mi355x{pat.FUSED_OP}>(kFusedDomain, "{pat.FUSED_OP}");' in text
    assert f'Register<Mi355x{pat.PACKED_FUSED_OP}>(kFusedDomain, "{pat.PACKED_FUSED_OP}");' in text


@pytest.mark.skipif(not os.path.isdir(REFERENCE), reason="reference sources not present")
def test_pattern_reference_names_exist():
    """Every header and GraphGraph / PatternOptimization member the C++
    patterns use exists in the reference."""
    raw = open(PATTERNS_CC).read()
    for inc in re.findall(r'#include "(onnx_core/[^"]+|onnx_proto/[^"]+)"', raw):
        if inc.startswith("onnx_proto/"):
            path = os.path.join(os.path.dirname(REFERENCE), "onnx_proto", "include", inc)
        else:
            path = os.path.join(REFERENCE, inc)
        assert os.path.isfile(path), inc
    graph_h = open(os.path.join(REFERENCE, "onnx_core/builder/graph_graph.h")).read()
    for m in sorted(set(re.findall(r"\bgraph\.(\w+)\(", _strip_comments(raw)))):
        assert re.search(rf"\b{m}\(", graph_h), f"GraphGraph::{m}"
    helper_h = open(os.path.join(os.path.dirname(REFERENCE), "onnx_proto/include/onnx_proto/onnx_helper.h")).read()
    for m in sorted(set(re.findall(r"\bol::(\w+)", _strip_comments(raw)))):
        if m in ("utils", "onnx_proto", "AttributeProto", "NodeProto", "TensorProto"):
            continue
        assert re.search(rf"\b{m}\b", helper_h), f"{m} not in onnx_helper.h"
    pat_h = open(os.path.join(REFERENCE, "onnx_core/builder/pattern_optimization.h")).read()
    for m in ("FastOpType", "Match", "Apply", "NoMatch", "MatchResult"):
        assert re.search(rf"\b{m}\b", pat_h), m
    reg_h = open(os.path.join(REFERENCE, "onnx_core/builder/pattern_registry.h")).read()
    assert "void RegisterPattern(const std::string &name, PatternFactory factory" in reg_h


@pytest.mark.skipif(not os.path.isdir(REFERENCE), reason="reference sources not present")
def test_reference_names_exist():
    """Every onnx-light header the adapter includes exists, and every runtime
    helper it calls through rt:: is declared in the reference's headers."""
    raw = open(ADAPTER).read()
    for inc in re.findall(r'#include "(onnx_core/[^"]+|onnx_proto/[^"]+)"', raw):
        if inc.startswith("onnx_proto/"):
            path = os.path.join(os.path.dirname(REFERENCE), "onnx_proto", "include", inc)
        else:
            path = os.path.join(REFERENCE, inc)
        assert os.path.isfile(path), inc
    headers = ""
    for rel in ["onnx_core/runtime/kernels/node_helpers.h", "onnx_core/runtime/kernels/kernel_dispatch_table.h",
                "onnx_core/runtime/kernels/kernel_context.h", "onnx_core/runtime/memory/simple_tensor.h",
                "onnx_core/runtime/runtime_context.h", "onnx_core/runtime/quantization.h",
                "onnx_core/runtime/runtime_value.h", "onnx_core/runtime/kernels/cast_helper.h"]:
        headers += open(os.path.join(REFERENCE, rel)).read()
    text = _adapter()
    used = set(re.findall(r"\brt::(\w+)", text))
    for name in sorted(used):
        assert re.search(rf"\b{name}\b", headers), f"rt::{name} not declared in the reference headers"
    for method in ["MakeOutputTensor", "MakeTemporaryTensor", "mutable_bytes", "size_bytes", "Get"]:
        assert re.search(rf"\b{method}\(", headers), method


PATTERNS_CC = os.path.join(ROOT, "adapter", "pattern_dequantize_linear_matmul.cc")


def _python_reasons():
    text = open(os.path.join(ROOT, "onnx-light_amd", "patterns.py")).read()
    i0 = text.index("class DequantizeLinearMatMulPattern")
    i1 = text.index("class DequantizePackedMatMulPattern")
    i2 = text.index("class DequantizeEncodedMatMulPattern")
    i3 = text.index("# ---- registry")
    pick = lambda part: set(re.findall(r'(?:no_match\(|return )"([^"]+)"', part))  # noqa: E731
    return pick(text[i0:i1]), pick(text[i1:i2]), pick(text[i2:i3])


def _cpp_reasons():
    text = _strip_comments(open(PATTERNS_CC).read())
    i1 = text.index("class DequantizePackedMatMulGpuPattern")
    i2 = text.index("class DequantizeEncodedMatMulGpuPattern")
    pick = lambda part: set(re.findall(r'NoMatch\(candidate,\s*"([^"]+)"\)', part))  # noqa: E731
    return pick(text[:i1]), pick(text[i1:i2]), pick(text[i2:])


def test_cpp_patterns_give_the_python_reasons():
    """The C++ PatternOptimization subclasses reject exactly the chains the
    Python mirror rejects, with the same reasons (the Python tests pin those)."""
    for cc, py in zip(_cpp_reasons(), _python_reasons()):
        assert cc == py, sorted(cc ^ py)


def test_cpp_patterns_registered_opt_in(olamd):
    import importlib
    pat = importlib.import_module("onnx_light_amd.patterns")
    text = _strip_comments(open(PATTERNS_CC).read())
    raw = open(PATTERNS_CC).read()
    for name in ("DequantizeLinearMatMulGpu", "DequantizePackedMatMulGpu", "DequantizeEncodedMatMulGpu",
                 "DequantizeLinearGroupedMatMulGpu"):
        assert name in pat.registered_pattern_names() and name not in pat.registered_pattern_names(False)
        assert re.search(rf'builder::RegisterPattern\(\s*"{name}",', text)
    assert raw.count("/*enabled_by_default=*/false);") == 4
    for op in (pat.ENCODED_FUSED_OP, pat.GROUPED_FUSED_OP):
        assert f'MakeNode("{op}",' in text
        assert f'Register<Mi355x{op}>(kFusedDomain, "{op}");' in _adapter()
    assert 'AddInt(fused, "transB",' in text
    assert f'kFusedDomain = "{pat.FUSED_DOMAIN}"' in text
    assert f'MakeNode("{pat.FUSED_OP}",' in text and f'MakeNode("{pat.PACKED_FUSED_OP}",' in text
    assert 'AddInt(fused, "axis",' in text and 'AddInt(fused, "cast_to", cast_to)' in text
