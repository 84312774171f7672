"""The GroupedMatMul oracle (oracle.grouped_matmul) pinned by the reference's
own backend cases, by the separately pinned MatMul oracle (each selection is
one row of a MatMul with the selected weight, summed in the same order), by
exact integer arithmetic, and by a float64 bound on random inputs."""
import numpy as np
import pytest

from grouped_cases import BFLOAT16, DOUBLE, FLOAT, FLOAT16, expand


@pytest.fixture(scope="module")
def cases(oracle):
    return expand(oracle)


def test_reference_backend_cases(oracle, cases):
    assert len(cases) == 90
    for name, dt, x, w, idx, bias, tb, want in cases:
        got = oracle.grouped_matmul(x, w, idx, bias, tb, dt)
        assert got.shape == want.shape, name
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), name


def test_invalid_index_raises(oracle):
    x = np.ones((2, 3), np.float32)
    w = np.ones((2, 3, 4), np.float32)
    for bad in (-1, 2):
        with pytest.raises(ValueError, match=r"\[0,G\)"):
            oracle.grouped_matmul(x, w, np.array([[0], [bad]]), None, 0, FLOAT)


@pytest.mark.parametrize("dt", [FLOAT16, BFLOAT16])
@pytest.mark.parametrize("tb", [0, 1])
def test_rows_equal_matmul_oracle(oracle, dt, tb):
    """Without a bias each selection's row is the MatMul oracle's row for the
    selected weight (same fp32 order, same final rounding), bit for bit."""
    rng = np.random.default_rng(31 + dt + tb)
    M, K, N, G, S = 5, 37, 11, 3, 2
    enc = oracle.f32_to_f16_bits if dt == FLOAT16 else oracle.f32_to_bf16_bits
    x = enc(rng.standard_normal((M, K)).astype(np.float32))
    w = enc(rng.standard_normal((G, N, K) if tb else (G, K, N)).astype(np.float32))
    idx = rng.integers(0, G, (M, S))
    y = oracle.grouped_matmul(x, w, idx, None, tb, dt)
    for m in range(M):
        for s in range(S):
            wg = np.ascontiguousarray(w[idx[m, s]].T if tb else w[idx[m, s]])
            ref = oracle.matmul_half(x[m:m + 1], wg, dt)
            assert np.array_equal(y[m, s], ref[0]), (m, s)


def test_integer_values_exact(oracle):
    """Small integers: every product and partial sum is exact in fp32, so the
    result equals the int64 contraction exactly (bias added after the first
    rounding, also exact)."""
    rng = np.random.default_rng(5)
    M, K, N, G, S = 7, 64, 9, 4, 3
    x = rng.integers(-3, 4, (M, K))
    w = rng.integers(-3, 4, (G, K, N))
    b = rng.integers(-5, 6, (G, N))
    idx = rng.integers(0, G, (M, S))
    want = np.einsum("mk,mskn->msn", x, w[idx]) + b[idx]
    for dt in (FLOAT, DOUBLE, FLOAT16):
        enc = {FLOAT: lambda a: a.astype(np.float32), DOUBLE: lambda a: a.astype(np.float64),
               FLOAT16: lambda a: oracle.f32_to_f16_bits(a.astype(np.float32))}[dt]
        y = oracle.grouped_matmul(enc(x), enc(w), idx, enc(b), 0, dt)
        yv = oracle.f16_bits_to_f32(y) if dt == FLOAT16 else y
        assert np.array_equal(yv.astype(np.int64), want), dt


def test_float_within_rounding_bound(oracle):
    """FLOAT: |y - exact| <= K * 2^-24 * sum |x w| (in-order fp32 summation)."""
    rng = np.random.default_rng(9)
    M, K, N, G, S = 6, 300, 13, 5, 2
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((G, N, K)).astype(np.float32)
    idx = rng.integers(0, G, (M, S))
    y = oracle.grouped_matmul(x, w, idx, None, 1, FLOAT)
    wt = np.transpose(w, (0, 2, 1)).astype(np.float64)[idx]          # [M, S, K, N]
    exact = np.einsum("mk,mskn->msn", x.astype(np.float64), wt)
    mag = np.einsum("mk,mskn->msn", np.abs(x.astype(np.float64)), np.abs(wt))
    assert np.all(np.abs(y - exact) <= K * 2.0 ** -24 * mag)
