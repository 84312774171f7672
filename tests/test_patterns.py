"""DequantizeLinear -> [Cast] -> MatMul rewrite (host logic, no GPU)."""
import importlib

import pytest


@pytest.fixture(scope="module")
def pt(olamd):
    return importlib.import_module("onnx_light_amd.patterns")


def _graph(pt, cast_to=None, zp=True, extra_use=False, dq_is_output=False, w_const=True, axis=1):
    N = pt.Node
    nodes = [N("DequantizeLinear", ["W", "s", "z" if zp else ""], ["Wd"], attrs={"axis": axis}, name="dq")]
    b = "Wd"
    if cast_to is not None:
        nodes.append(N("Cast", ["Wd"], ["Wc"], attrs={"to": cast_to}, name="cast"))
        b = "Wc"
    nodes.append(N("MatMul", ["A", b], ["Y"], name="mm"))
    if extra_use:
        nodes.append(N("Relu", ["Wd"], ["R"], name="relu"))
    init = {"s", "z"} | ({"W"} if w_const else set())
    outs = ["Y"] + (["Wd"] if dq_is_output else []) + (["R"] if extra_use else [])
    return pt.Graph(nodes, init, ["A"] + ([] if w_const else ["W"]), outs)


def _pattern(pt):
    return pt.create_registered_pattern("DequantizeLinearMatMulGpu")


@pytest.mark.parametrize("cast_to,zp", [(None, True), (None, False), (10, True), (16, False)])
def test_rewrite(pt, olamd, cast_to, zp):
    g = _graph(pt, cast_to, zp, axis=0)
    assert pt.optimize(g, [_pattern(pt)]) == 1
    assert len(g.nodes) == 1
    n = g.nodes[0]
    assert (n.domain, n.op_type) == (pt.FUSED_DOMAIN, pt.FUSED_OP)
    assert n.inputs == ["A", "W", "s"] + (["z"] if zp else [])
    assert n.outputs == ["Y"]
    assert n.attrs == {"axis": 0, "cast_to": cast_to or 0}
    assert f"{n.domain}:{n.op_type}" in olamd.KERNELS


@pytest.mark.parametrize("kw,reason", [
    (dict(extra_use=True), "another consumer"),
    (dict(dq_is_output=True), "another consumer"),
    (dict(w_const=False), "initializers"),
    (dict(cast_to=1), "FLOAT16 or BFLOAT16"),
])
def test_no_match(pt, kw, reason):
    g = _graph(pt, **kw)
    mm = next(n for n in g.nodes if n.op_type == "MatMul")
    m = _pattern(pt).match(g, mm)
    assert not m and reason in m.reason
    before = [n.op_type for n in g.nodes]
    assert pt.optimize(g, [_pattern(pt)]) == 0
    assert [n.op_type for n in g.nodes] == before


def test_first_input_and_other_attrs_do_not_match(pt):
    N = pt.Node
    g = pt.Graph([N("DequantizeLinear", ["W", "s"], ["Wd"]), N("MatMul", ["Wd", "B"], ["Y"])], {"W", "s"},
                 ["B"], ["Y"])
    assert pt.optimize(g, [_pattern(pt)]) == 0
    g = pt.Graph([N("DequantizeLinear", ["W", "s"], ["Wd"], attrs={"block_size": 32}),
                  N("MatMul", ["A", "Wd"], ["Y"])], {"W", "s"}, ["A"], ["Y"])
    m = _pattern(pt).match(g, g.nodes[1])
    assert not m and "attribute" in m.reason


def test_two_chains_and_order(pt):
    """Two independent chains are both rewritten; each fused node sits where
    its MatMul was, after the nodes it depends on."""
    N = pt.Node
    g = pt.Graph([N("Relu", ["X"], ["A"]),
                  N("DequantizeLinear", ["W1", "s1"], ["D1"]), N("MatMul", ["A", "D1"], ["H"]),
                  N("DequantizeLinear", ["W2", "s2"], ["D2"]), N("Cast", ["D2"], ["C2"], attrs={"to": 16}),
                  N("MatMul", ["H", "C2"], ["Y"])],
                 {"W1", "s1", "W2", "s2"}, ["X"], ["Y"])
    assert pt.optimize(g, [_pattern(pt)]) == 2
    assert [n.op_type for n in g.nodes] == ["Relu", pt.FUSED_OP, pt.FUSED_OP]
    assert g.nodes[1].outputs == ["H"] and g.nodes[2].inputs[0] == "H" and g.nodes[2].attrs["cast_to"] == 16


def test_registry(pt):
    names = pt.registered_pattern_names()
    assert "DequantizeLinearMatMulGpu" in names
    assert "DequantizeLinearMatMulGpu" not in pt.registered_pattern_names(include_opt_in=False)
    assert not any(isinstance(p, pt.DequantizeLinearMatMulPattern) for p in pt.create_registered_patterns("gpu"))
    with pytest.raises(ValueError):
        pt.register_pattern("DequantizeLinearMatMulGpu", pt.DequantizeLinearMatMulPattern)
    with pytest.raises(ValueError):
        pt.register_pattern("", pt.DequantizeLinearMatMulPattern)
