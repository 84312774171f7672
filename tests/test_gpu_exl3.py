"""EXL3 weights on the GPU against the oracle (oracle.exl3_reconstruct,
pinned in test_oracle_exl3.py by the reference test's zero-trellis values
and an independent restatement of the format): onnxl_amd_dequantize_exl3
bit for bit in FLOAT, FLOAT16, BFLOAT16 and DOUBLE for every rate and
codebook, every state, random streams at 512 x 1024 from host and device
inputs; Validate's checks and WriteFloat's range in the reference's order."""
import numpy as np
import pytest
import torch

from test_gpu_float import T
from test_gpu_gptq_fp8 import _bits, _ref_bits, _raises
from test_oracle_exl3 import fixture

pytestmark = pytest.mark.gpu

DTYPES = [1, 10, 16, 11]
MARKERS = {1: 0xCBAC1FED, 2: 0x83DCD12D}


@pytest.fixture(scope="module")
def dev(olamd):
    olamd.init(0)
    return torch.device("cuda:0")


def _marker(book):
    return np.array(MARKERS[book], np.uint32).view(np.int32).reshape(())


def _dev_scalar(m, dev):
    """A 0-d device tensor (T() would give shape [1])."""
    return torch.tensor(int(m), dtype=torch.int32, device=dev)


def _call(olamd, dev, trellis, suh, svh, book, out, host=False):
    put = (lambda a: np.ascontiguousarray(a)) if host else (lambda a: T(a, dev))
    put0 = (lambda m: m) if host else (lambda m: _dev_scalar(m, dev))
    mcg = put0(_marker(1)) if book == 1 else None
    mul1 = put0(_marker(2)) if book == 2 else None
    return olamd.dequantize_exl3(put(trellis), put(suh), put(svh), mcg, mul1, out)


def _check(olamd, oracle, dev, trellis, suh, svh, book, host=False, dtypes=DTYPES):
    for out in dtypes:
        rc, ref = oracle.exl3_reconstruct(trellis, suh, svh, book, out_dtype=out)
        if rc:
            _raises(olamd, lambda: _call(olamd, dev, trellis, suh, svh, book, out, host), oracle.EXL3_ERRORS[rc])
            continue
        y = _call(olamd, dev, trellis, suh, svh, book, out, host)
        assert np.array_equal(np.asarray(_bits(y)).reshape(-1), _ref_bits(ref, out).reshape(-1)), (book, out)


@pytest.mark.parametrize("book", [0, 1, 2])
@pytest.mark.parametrize("bits", range(1, 9))
def test_rates_and_codebooks(olamd, oracle, dev, bits, book):
    trellis, suh, svh, _ = fixture(bits, book)
    _check(olamd, oracle, dev, trellis, suh, svh, book)


@pytest.mark.parametrize("book", [0, 1, 2])
def test_every_state(olamd, oracle, dev, book):
    trellis, suh, svh, _ = fixture(8, book, cols=1024, exhaustive=True)
    _check(olamd, oracle, dev, trellis, suh, svh, book, dtypes=[1])


@pytest.mark.parametrize("bits,book,host", [(2, 0, False), (4, 1, True), (3, 2, False), (8, 0, True)])
def test_random_streams(olamd, oracle, dev, bits, book, host):
    rng = np.random.default_rng(bits * 10 + book)
    k, n = 512, 1024
    trellis = rng.integers(-32768, 32768, (k // 16, n // 16, 16 * bits)).astype(np.int16)
    suh = rng.uniform(-3, 3, k).astype(np.float16)
    svh = rng.uniform(-3, 3, n).astype(np.float16)
    _check(olamd, oracle, dev, trellis, suh, svh, book, host=host)


def test_errors_in_reference_order(olamd, oracle, dev):
    trellis, suh, svh, _ = fixture(3, 1)
    inf_suh = suh.copy()
    inf_suh[5] = np.float16(np.inf)
    call = lambda t=trellis, u=suh, v=svh, mcg=_marker(1), mul1=None: olamd.dequantize_exl3(
        T(t, dev), T(u, dev), T(v, dev), None if mcg is None else _dev_scalar(mcg, dev),
        None if mul1 is None else _dev_scalar(mul1, dev))
    _raises(olamd, lambda: call(u=inf_suh, v=svh[:100]), "EXL3 nonfinite scale.")
    _raises(olamd, lambda: call(v=svh[:100]), "EXL3 invalid tensor type, shape or byte extent.")
    bad = _marker(1).copy()
    bad[()] ^= 1
    _raises(olamd, lambda: call(mcg=bad), "EXL3 invalid codebook marker.")
    _raises(olamd, lambda: call(mul1=_marker(2)), "EXL3 unexpected side tensors or conflicting codebooks.")
    _raises(olamd, lambda: call(t=trellis[:4]), "EXL3 dimensions must be positive multiples of 128.")
    _raises(olamd, lambda: call(t=trellis[:, :, :17]), "EXL3 invalid trellis dimensions.")
    _raises(olamd, lambda: call(t=np.zeros((8, 16, 16 * 9), np.int16)), "EXL3 unsupported trellis rate.")
    big = np.full(128, 60000, np.float16)
    _check(olamd, oracle, dev, trellis, big, np.full(256, 60000, np.float16), 1, dtypes=[10])
