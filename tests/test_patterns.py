"""DequantizeLinear -> [Cast] -> MatMul rewrite (host logic, no GPU)."""
import importlib

import pytest


@pytest.fixture(scope="module")
def pt(olamd):
    return importlib.import_module("onnx_light_amd.patterns")


def _graph(pt, cast_to=None, zp=True, extra_use=False, dq_is_output=False, w_const=True, axis=1,
           w_type=None, s_type=None, w_shape=(64, 32), s_shape=None):
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
    w_type = pt.INT8 if w_type is None else w_type
    # a FLOAT16 scale makes a FLOAT16 MatMul; a FLOAT one needs the Cast
    s_type = (pt.FLOAT16 if cast_to is None else pt.FLOAT) if s_type is None else s_type
    if s_shape is None:
        s_shape = (w_shape[0] // 32, w_shape[1]) if axis == 0 else (w_shape[1],)
    info = {"W": (w_type, w_shape), "s": (s_type, s_shape), "z": (w_type, s_shape)}
    return pt.Graph(nodes, init, ["A"] + ([] if w_const else ["W"]), outs, info)


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


@pytest.mark.parametrize("kw,reason", [
    # a FLOAT DequantizeLinear into a FLOAT MatMul: the fused kernel needs 16-bit A
    (dict(s_type=1), "MatMul would run in FLOAT"),
    # an FLOAT16 DequantizeLinear output followed by a Cast
    (dict(cast_to=16, s_type=10), "Cast of a FLOAT16"),
    (dict(w_type=5), "no fused kernel"),                      # INT16 weight
    (dict(w_type=4), "no fused kernel"),                      # UINT16 weight
    (dict(w_type=6), "no fused kernel"),                      # INT32 weight
    (dict(axis=0, s_shape=(64,)), "per-row (axis 0)"),        # 1-D scale along K
    (dict(axis=1, s_shape=(64, 2)), "blocked along N"),
    (dict(axis=0, s_shape=(3, 32)), "does not fit"),          # 64 rows in blocks of 3 scales
    (dict(axis=1, s_shape=(31,)), "differs from the axis"),
    (dict(axis=2, s_shape=(32,)), "axis out of range"),
    (dict(w_shape=(2, 64, 32), s_shape=(32,)), "not 2-D"),
    (dict(s_type=11), "not FLOAT or FLOAT16"),                # DOUBLE scale
    (dict(w_type=17, cast_to=16, zp=False), "scale the sums"),  # fp8 scaled-sum path, not opted in
])
def test_no_match_types(pt, kw, reason):
    g = _graph(pt, **kw)
    mm = next(n for n in g.nodes if n.op_type == "MatMul")
    m = _pattern(pt).match(g, mm)
    assert not m and reason in m.reason, m.reason
    assert pt.optimize(g, [_pattern(pt)]) == 0


def test_zero_point_mismatch_and_unknown_types(pt):
    g = _graph(pt, zp=True)
    g.value_info["z"] = (pt.UINT8, g.value_info["s"][1])
    assert "zero point" in _pattern(pt).match(g, g.nodes[-1]).reason
    g = _graph(pt, zp=True)
    del g.value_info["s"]
    assert "unknown" in _pattern(pt).match(g, g.nodes[-1]).reason


def test_fp8_scaled_sums_opt_in(pt):
    g = _graph(pt, w_type=17, cast_to=16, zp=False)
    assert pt.optimize(g, [pt.DequantizeLinearMatMulPattern(fp8_scaled_sums=True)]) == 1
    # with a zero point or a FLOAT16 target the chain keeps the exact rounding and is fused by default
    g = _graph(pt, w_type=17, cast_to=16, zp=True)
    assert pt.optimize(g, [_pattern(pt)]) == 1
    g = _graph(pt, w_type=17, cast_to=10, zp=False)
    assert pt.optimize(g, [_pattern(pt)]) == 1


def test_same_tensor_twice_is_two_uses(pt):
    """MatMul(Wd, Wd): the DequantizeLinear output feeds two input slots, so
    removing the DequantizeLinear would leave A dangling."""
    N = pt.Node
    g = pt.Graph([N("DequantizeLinear", ["W", "s"], ["Wd"], attrs={"axis": 1}), N("MatMul", ["Wd", "Wd"], ["Y"])],
                 {"W", "s"}, [], ["Y"], {"W": (pt.INT8, (32, 32)), "s": (pt.FLOAT16, (32,))})
    m = _pattern(pt).match(g, g.nodes[1])
    assert not m and "another consumer" in m.reason
    assert pt.optimize(g, [_pattern(pt)]) == 0


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
                 {"W1", "s1", "W2", "s2"}, ["X"], ["Y"],
                 {"W1": (pt.INT4, (64, 32)), "s1": (pt.FLOAT16, (32,)), "W2": (pt.UINT8, (32, 16)),
                  "s2": (pt.FLOAT, ())})
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


# ---- DequantizePacked -> Transpose -> MatMul --------------------------------

def _packed_graph(pt, fmt="gguf:q4_0", shape=(96, 128), odt=None, perm=None, a_type=None, extra=None,
                  const=True):
    N = pt.Node
    dattrs = {"format": fmt, "shape": list(shape), "output_dtype": pt.FLOAT16 if odt is None else odt}
    tattrs = {} if perm is None else {"perm": perm}
    nodes = [N("DequantizePacked", ["X"], ["Wd"], attrs=dattrs), N("Transpose", ["Wd"], ["Wt"], attrs=tattrs),
             N("MatMul", ["A", "Wt"], ["Y"])] + (extra or [])
    info = {"A": (pt.FLOAT16 if a_type is None else a_type, (4, shape[1]))}
    return pt.Graph(nodes, {"X"} if const else set(), ["A"] + ([] if const else ["X"]), ["Y"], info)


def test_packed_rewrite(pt):
    g = _packed_graph(pt)
    assert pt.optimize(g, [pt.create_registered_pattern("DequantizePackedMatMulGpu")]) == 1
    (node,) = g.nodes
    assert (node.domain, node.op_type) == (pt.FUSED_DOMAIN, pt.PACKED_FUSED_OP)
    assert node.inputs == ["A", "X"] and node.outputs == ["Y"]
    assert node.attrs == {"format": "gguf:q4_0", "shape": [96, 128]}


@pytest.mark.parametrize("kw,reason", [
    ({"fmt": "gguf:q9_9"}, "unknown packed format"),
    ({"shape": (96, 48)}, "K is not a whole number of blocks"),
    ({"fmt": "gguf:q6_k", "shape": (96, 128)}, "K is not a whole number of blocks"),
    ({"shape": (2, 96, 128)}, "DequantizePacked shape is not [N, K]"),
    ({"odt": 1}, "DequantizePacked output is not FLOAT16"),
    ({"perm": [0, 1]}, "Transpose is not a 2-D transpose"),
    ({"a_type": 16}, "A is not FLOAT16"),
    ({"const": False}, "packed weight is not an initializer"),
])
def test_packed_no_match(pt, kw, reason):
    g = _packed_graph(pt, **kw)
    pat = pt.create_registered_pattern("DequantizePackedMatMulGpu")
    m = pat.match(g, g.nodes[2])
    assert not m and m.reason == reason
    assert pt.optimize(g, [pat]) == 0


@pytest.mark.parametrize("fmt,block", [("gguf:q5_k", 256), ("gguf:iq2_xxs", 256), ("gguf:mxfp4", 32),
                                       ("gguf:q1_0", 128), ("gguf:nvfp4", 64), ("gguf:q4_1", 32)])
def test_packed_rewrite_every_format(pt, fmt, block):
    """Every GGUF profile runs fused on the GPU (the decode GEMVs or the
    decoded weight through the MFMA GEMM): each format with K a whole number
    of its blocks is rewritten."""
    g = _packed_graph(pt, fmt=fmt, shape=(96, 2 * block))
    assert pt.optimize(g, [pt.create_registered_pattern("DequantizePackedMatMulGpu")]) == 1
    assert g.nodes[0].attrs == {"format": fmt, "shape": [96, 2 * block]}


def test_packed_shared_intermediate_is_left_alone(pt):
    N = pt.Node
    g = _packed_graph(pt, extra=[N("Relu", ["Wt"], ["R"])])
    m = pt.create_registered_pattern("DequantizePackedMatMulGpu").match(g, g.nodes[2])
    assert not m and m.reason == "Transpose output has another consumer"
    g = _packed_graph(pt, extra=[N("Relu", ["Wd"], ["R"])])
    m = pt.create_registered_pattern("DequantizePackedMatMulGpu").match(g, g.nodes[2])
    assert not m and m.reason == "DequantizePacked output has another consumer"


def test_packed_registry(pt):
    assert "DequantizePackedMatMulGpu" in pt.registered_pattern_names()
    assert "DequantizePackedMatMulGpu" not in pt.registered_pattern_names(include_opt_in=False)


# ---- ai.rt:Dequantize (encoded weight) -> Transpose -> MatMul ----------------

def _encoded_graph(pt, dtype=10, a_type=10, perm=(1, 0), q_const=True, extra_use=False, domain="ai.rt"):
    N = pt.Node
    nodes = [N("Dequantize", ["Q"], ["Wd"], domain=domain, attrs={"dtype": dtype}, name="dq"),
             N("Transpose", ["Wd"], ["Wt"], attrs={"perm": list(perm)}, name="tr"),
             N("MatMul", ["A", "Wt"], ["Y"], name="mm")]
    if extra_use:
        nodes.append(N("Relu", ["Wd"], ["R"], name="relu"))
    outs = ["Y"] + (["R"] if extra_use else [])
    info = {} if a_type is None else {"A": (a_type, (8, 4096))}
    return pt.Graph(nodes, {"Q"} if q_const else set(), ["A"] + ([] if q_const else ["Q"]), outs, info)


@pytest.mark.parametrize("dtype", [10, 16])
def test_encoded_rewrite(pt, dtype):
    g = _encoded_graph(pt, dtype, dtype)
    assert pt.optimize(g, [pt.create_registered_pattern("DequantizeEncodedMatMulGpu")]) == 1
    assert len(g.nodes) == 1
    n = g.nodes[0]
    assert (n.domain, n.op_type, n.inputs, n.outputs) == (pt.FUSED_DOMAIN, pt.ENCODED_FUSED_OP, ["A", "Q"], ["Y"])


@pytest.mark.parametrize("kw,reason", [
    (dict(dtype=1, a_type=1), "Dequantize dtype is not FLOAT16 or BFLOAT16"),
    (dict(a_type=16), "type of A differs from the Dequantize dtype"),
    (dict(a_type=None), "type of A unknown"),
    (dict(perm=(0, 1)), "Transpose is not a 2-D transpose"),
    (dict(q_const=False), "encoded weight is not an initializer"),
    (dict(extra_use=True), "Dequantize output has another consumer"),
    (dict(domain=""), "Transpose input is not an ai.rt Dequantize output"),
])
def test_encoded_no_match(pt, kw, reason):
    g = _encoded_graph(pt, **kw)
    mm = next(n for n in g.nodes if n.op_type == "MatMul")
    m = pt.create_registered_pattern("DequantizeEncodedMatMulGpu").match(g, mm)
    assert not m and m.reason == reason
    assert pt.optimize(g, [pt.create_registered_pattern("DequantizeEncodedMatMulGpu")]) == 0


# ---- DequantizeLinear -> [Cast] -> GroupedMatMul ----------------------------

def _grouped_graph(pt, cast_to=16, zp=False, bias=True, w_type=None, s_type=None, w_shape=(4, 64, 32),
                   s_shape=(4, 1, 32), axis=1, trans_b=0, extra_use=False, gmm_attrs=None):
    N = pt.Node
    nodes = [N("DequantizeLinear", ["W", "s", "z" if zp else ""], ["Wd"], attrs={"axis": axis}, name="dq")]
    w = "Wd"
    if cast_to is not None:
        nodes.append(N("Cast", ["Wd"], ["Wc"], attrs={"to": cast_to}, name="cast"))
        w = "Wc"
    attrs = {"transB": trans_b} if gmm_attrs is None else gmm_attrs
    nodes.append(N("GroupedMatMul", ["X", w, "I"] + (["B"] if bias else []), ["Y"], attrs=attrs, name="gmm"))
    if extra_use:
        nodes.append(N("Relu", ["Wd"], ["R"], name="relu"))
    w_type = pt.FLOAT8E4M3FN if w_type is None else w_type
    s_type = pt.FLOAT if s_type is None else s_type
    info = {"W": (w_type, w_shape), "s": (s_type, s_shape), "z": (w_type, s_shape)}
    return pt.Graph(nodes, {"W", "s", "z"}, ["X", "I"] + (["B"] if bias else []),
                    ["Y"] + (["R"] if extra_use else []), info)


def _grouped_pattern(pt, fp8_scaled_sums=False):
    p = pt.create_registered_pattern("DequantizeLinearGroupedMatMulGpu")
    p.fp8_scaled_sums = fp8_scaled_sums
    return p


@pytest.mark.parametrize("cast_to,zp,bias,w_type,s_type,s_shape,axis,trans_b", [
    (16, False, True, 17, 1, (4, 1, 32), 1, 0),    # fp8 experts, per (expert, column): scaled sums (opt-in)
    (16, False, False, 17, 1, (4,), 0, 0),          # per expert
    (None, True, True, 22, 10, (4, 2, 32), 1, 0),   # INT4 blocked along K, FLOAT16 scales
    (10, True, False, 2, 1, (32,), 1, 1),           # UINT8 per column ([G, N, K]: axis 1), transB
])
def test_grouped_rewrite(pt, olamd, cast_to, zp, bias, w_type, s_type, s_shape, axis, trans_b):
    w_shape = (4, 32, 64) if trans_b else (4, 64, 32)
    g = _grouped_graph(pt, cast_to, zp, bias, w_type, s_type, w_shape, s_shape, axis, trans_b)
    assert pt.optimize(g, [_grouped_pattern(pt, fp8_scaled_sums=True)]) == 1
    (n,) = g.nodes
    assert (n.domain, n.op_type) == (pt.FUSED_DOMAIN, pt.GROUPED_FUSED_OP)
    assert n.inputs == ["X", "W", "s", "z" if zp else "", "I"] + (["B"] if bias else [])
    assert n.outputs == ["Y"]
    assert n.attrs == {"axis": axis, "cast_to": cast_to or 0, "transB": trans_b}
    assert f"{n.domain}:{n.op_type}" in olamd.KERNELS


@pytest.mark.parametrize("kw,reason", [
    (dict(), "fp8_scaled_sums=True allows it"),
    (dict(extra_use=True), "another consumer"),
    (dict(cast_to=1), "FLOAT16 or BFLOAT16"),
    (dict(cast_to=None), "would run in FLOAT"),
    (dict(w_shape=(64, 32), s_shape=(32,), axis=1), "not 3-D"),
    (dict(w_type=3, s_shape=(4, 1, 16)), "blocked scale does not fit"),
    (dict(w_type=3, s_shape=(31,), axis=2), "differs from the axis dimension"),
    (dict(w_type=3, s_shape=(4, 32), axis=2), "neither 1 nor 3"),
    (dict(w_type=3, s_shape=(32,), axis=3), "axis out of range"),
    (dict(w_type=7), "no fused kernel"),
    (dict(s_type=10), "Cast of a FLOAT16"),
    (dict(gmm_attrs={"transB": 0, "alpha": 1}), "attribute other than transB"),
])
def test_grouped_no_match(pt, kw, reason):
    g = _grouped_graph(pt, **kw)
    gmm = next(n for n in g.nodes if n.op_type == "GroupedMatMul")
    m = _grouped_pattern(pt).match(g, gmm)
    assert not m and reason in m.reason, m.reason


def test_grouped_fp8_exact_layouts_need_no_opt_in(pt):
    """fp8 experts whose scale varies along K, or transposed, take the
    dequantizing path (the chain's roundings): no opt-in needed."""
    for kw in (dict(s_shape=(4, 2, 32), axis=1), dict(s_shape=(64,), axis=1),
               dict(w_shape=(4, 32, 64), s_shape=(4, 32, 1), axis=2, trans_b=1)):
        g = _grouped_graph(pt, **kw)
        assert pt.optimize(g, [_grouped_pattern(pt)]) == 1, kw
