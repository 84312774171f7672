"""VPTQ weights on the GPU against the oracle (oracle.vptq_reconstruct,
pinned by the upstream dequantize's outputs in test_oracle_vptq.py):
onnxl_amd_dequantize_vptq reproduces the reference's 10 golden cases and the
oracle bit for bit in FLOAT, FLOAT16, BFLOAT16 and DOUBLE, from host and
device inputs; random larger weights with every feature (residual,
outliers, groups by size and count, norm on either dim, permutation); the
index, outlier-index, permutation, nonfinite and range errors in the
reference's order."""
import numpy as np
import pytest
import torch

from test_gpu_float import tensor_bits
from test_oracle_vptq import golden, vptq_cases

pytestmark = pytest.mark.gpu

DTYPES = [1, 10, 16, 11]
INT_TENSORS = ("indices", "outlier_indices", "perm")


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _bits(t):
    if t.dtype in (torch.float32, torch.float64):
        a = t.cpu().numpy()
        return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)
    return tensor_bits(t)


def _ref_bits(a, code):
    return a.view(np.uint32) if code == 1 else (a.view(np.uint64) if code == 11 else a)


def _on(tensors, dev, host):
    if host:
        return {k: np.ascontiguousarray(v) for k, v in tensors.items()}
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in tensors.items()}


def _raises(olamd, fn, message):
    with pytest.raises(olamd.InvalidArgument) as e:
        fn()
    assert message in str(e.value), str(e.value)


def _params(cfg):
    return dict(in_features=cfg.k, out_features=cfg.n, vector_lens=list(cfg.vector_lens),
                num_centroids=list(cfg.num_centroids), num_res_centroids=list(cfg.num_res_centroids),
                npercent=cfg.npercent, group_size=cfg.group_size, group_num=cfg.group_num,
                enable_norm=bool(cfg.enable_norm), norm_dim=cfg.norm_dim, enable_perm=bool(cfg.enable_perm))


def _check(olamd, oracle, dev, cfg, tensors, host=False, what=""):
    config = olamd.VptqConfig.of(_params(cfg))
    for out in DTYPES:
        rc, ref = oracle.vptq_reconstruct(cfg, tensors, out_dtype=out)
        call = lambda: olamd.dequantize_vptq(config, _on(tensors, dev, host), cfg.dtype, out)
        if rc:
            _raises(olamd, call, oracle.VPTQ_ERRORS[rc])
            continue
        assert np.array_equal(_bits(call()), _ref_bits(ref, out)), (what, out)


@pytest.mark.parametrize("f", vptq_cases(), ids=lambda f: f["name"])
@pytest.mark.parametrize("host", [False, True])
def test_golden_decode(olamd, oracle, dev, f, host):
    cfg, tensors, expected = golden(f)
    got = olamd.dequantize_vptq(olamd.VptqConfig.of(f["parameters"]), _on(tensors, dev, host), cfg.dtype, 1)
    assert np.array_equal(_bits(got), expected.view(np.uint32)), f["name"]
    _check(olamd, oracle, dev, cfg, tensors, host, f["name"])


def _random(oracle, rng, k, n, dtype, vl=(2, 4), nc=(16, 256), nr=(-1, 16), npercent=5.0, group_size=-1,
            group_num=-1, norm=True, norm_dim=0, perm=True):
    p = dict(in_features=k, out_features=n, vector_lens=list(vl), num_centroids=list(nc),
             num_res_centroids=list(nr), npercent=npercent, group_size=group_size, group_num=group_num,
             enable_norm=norm, norm_dim=norm_dim, enable_perm=perm)
    cfg = oracle.vptq_config(p, dtype)
    # the layout as the reference derives it
    outliers = int(np.ceil(npercent / 100 * k)) if npercent > 0 else 0
    if group_num != -1:
        groups = group_num
        if outliers:
            outliers += (k - outliers) % groups
        columns = (k - outliers) // groups if outliers else -(-k // groups)
    else:
        columns = k - outliers if group_size == -1 else group_size
        groups = -(-(k - outliers) // columns)
    mb = int(nc[1] - 1).bit_length()
    rb = int(nr[1] - 1).bit_length() if nr[1] > 1 else 0
    vectors, words = -(-n // vl[1]), -(-(columns * (mb + rb)) // 32)
    idx = rng.integers(0, nc[1], (groups, vectors, columns)).astype(np.uint64)
    if rb:
        idx |= rng.integers(0, nr[1], (groups, vectors, columns)).astype(np.uint64) << mb
    words_arr = np.zeros((groups, vectors, words + 1), np.uint64)
    for j in range(columns):
        bit = j * (mb + rb)
        words_arr[:, :, bit // 32] |= (idx[:, :, j] << np.uint64(bit % 32)) & np.uint64(0xFFFFFFFF)
        words_arr[:, :, bit // 32 + 1] |= idx[:, :, j] >> np.uint64(32 - bit % 32)
    t = {"indices": words_arr[:, :, :words].astype(np.uint32).view(np.int32)}
    cb = (lambda shape: rng.standard_normal(shape).astype(np.float32)) if dtype == 1 else (
        lambda shape: oracle.f32_to_f16_bits(rng.standard_normal(shape).astype(np.float32)) if dtype == 10 else
        (rng.standard_normal(shape).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16))
    t["centroids.weight"] = cb((groups, nc[1] * vl[1]))
    if rb:
        t["res_centroids.weight"] = cb((groups, nr[1] * vl[1]))
    if outliers:
        t["outlier_centroids.weight"] = cb((1, nc[0] * vl[0]))
        t["outlier_indices"] = rng.integers(0, nc[0], (1, -(-n // vl[0]), outliers)).astype(np.int32)
    if norm:
        t["weight_scale"] = cb((k if norm_dim == 0 else n,))
        t["weight_bias"] = cb((k if norm_dim == 0 else n,))
    if perm:
        t["perm"] = rng.permutation(k).astype(np.int32)
    return cfg, t


@pytest.mark.parametrize("k,n,dtype,kw", [(1024, 256, 10, dict()), (777, 130, 16, dict(group_num=5, norm_dim=1)),
                                          (512, 96, 1, dict(group_size=100, nr=(-1, -1), npercent=0.0,
                                                            vl=(-1, 8), nc=(-1, 4096))),
                                          (300, 64, 10, dict(npercent=0.0, vl=(-1, 6), nc=(-1, 64), perm=False,
                                                             norm=False))])
def test_random_decode(olamd, oracle, dev, k, n, dtype, kw):
    rng = np.random.default_rng(k + n)
    cfg, t = _random(oracle, rng, k, n, dtype, **kw)
    _check(olamd, oracle, dev, cfg, t, what=(k, n, dtype))


def test_errors(olamd, oracle, dev):
    f = next(f for f in vptq_cases() if f["name"] == "combined_float16_norm0_perm_tails")
    cfg, tensors, _ = golden(f)
    config = olamd.VptqConfig.of(f["parameters"])
    dq = lambda t, out=1: olamd.dequantize_vptq(config, _on(t, dev, False), cfg.dtype, out)
    bad_idx = dict(tensors, indices=np.full_like(tensors["indices"], -1))
    small = olamd.VptqConfig.of(dict(f["parameters"], num_centroids=[5, 7]))
    with pytest.raises(olamd.InvalidArgument):  # 7 entries: the tensor shapes no longer match
        olamd.dequantize_vptq(small, _on(bad_idx, dev, False), cfg.dtype, 1)
    oi = tensors["outlier_indices"].copy()
    oi.reshape(-1)[1] = 5
    p = tensors["perm"].copy()
    p[0] = p[1]
    _raises(olamd, lambda: dq(dict(tensors, outlier_indices=oi, perm=p)), "VPTQ outlier index exceeds codebook.")
    _raises(olamd, lambda: dq(dict(tensors, perm=p)), "VPTQ invalid permutation.")
    big = tensors["centroids.weight"].copy()
    big[:] = 0x7BFF  # 65504: the norm steps push values past FLOAT16
    rc16, _ = oracle.vptq_reconstruct(cfg, dict(tensors, **{"centroids.weight": big}), out_dtype=10)
    if rc16:
        _raises(olamd, lambda: dq(dict(tensors, **{"centroids.weight": big}), 10), oracle.VPTQ_ERRORS[rc16])
    nan = tensors["centroids.weight"].copy()
    nan[0, 3] = 0x7E00
    rc, _ = oracle.vptq_reconstruct(cfg, dict(tensors, **{"centroids.weight": nan}))
    if rc:
        _raises(olamd, lambda: dq(dict(tensors, **{"centroids.weight": nan})), oracle.VPTQ_ERRORS[rc])
