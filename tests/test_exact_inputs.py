"""CPU checks of the dyadic inputs behind the bit-exact GPU tests
(tests/test_gpu_exact.py): for each generator, at the GPU tests' K,

- the exactness premise holds: every fp32 partial sum of a @ W is exact, and
  the oracle chain (k-sequential fp32 sums, km/kernel_matmul.cc:136-141, and
  the reference's weight rounding) gives exactly the once-rounded exact sum,
  so any summation order must reproduce it bit for bit;
- the bit-exact check rejects a wrong answer: with one nonzero k-term removed
  from every row, the rounded outputs that term touched change in at least
  99% of the cases (so a kernel that drops or repeats a k-term fails).
"""
import numpy as np
import pytest

import dyadic as dy


def _chain(oracle, case):
    """The oracle chain's output bits for a case: the weight as the chain
    rounds it, then oracle.matmul_half."""
    dt = case["out"]
    w_bits = dy.enc(oracle, case["w"], dt)  # asserts the chain's weight rounding is exact
    code = oracle.BFLOAT16 if dt == "bf16" else oracle.FLOAT16
    return oracle.matmul_half(case["a_bits"], w_bits, code, nthreads=8)


def _check(oracle, case, seed):
    dy.check_premise(case["a"].astype(np.float64), case["w"].astype(np.float64))
    want = dy.exact_out_bits(oracle, case["a"], case["w"], case["out"])
    got = _chain(oracle, case)
    assert np.array_equal(got, want), "the oracle's k-sequential sum is the exact sum"
    frac, wrong = dy.visible_drop_fraction(oracle, case, np.random.default_rng(seed))
    assert not np.array_equal(wrong, got), "the bit-exact check rejects a dropped k-term"
    assert frac >= 0.99, f"a dropped term shows in only {frac:.4f} of the outputs it touches"
    return frac


def test_fp8_case_c4_depth(oracle):
    """Configuration 4's K = 4096 (the GPU test runs the full 4096 x 14336)."""
    case = dy.fp8_case(oracle, np.random.default_rng(1), 48, 4096, 256)
    _check(oracle, case, 11)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_half_case(oracle, dt):
    case = dy.half_case(oracle, np.random.default_rng(2), 32, 4096, 192, dt)
    _check(oracle, case, 12)


@pytest.mark.parametrize("dt,signed,zp,block", [("f16", True, False, 32), ("f16", False, True, 128),
                                                 ("bf16", True, False, 32), ("bf16", False, True, 64)])
def test_int4_case_c3_depth(oracle, dt, signed, zp, block):
    case = dy.int4_case(oracle, np.random.default_rng(3), 8, 4096, 256, block, signed, zp, dt)
    _check(oracle, case, 13)


@pytest.mark.parametrize("fmt", ["gguf:q4_0", "gguf:q8_0", "gguf:q2_k", "gguf:q3_k", "gguf:q4_k", "gguf:q5_k",
                                 "gguf:q6_k", "gguf:iq4_xs"])
def test_gguf_case(oracle, fmt):
    case = dy.gguf_case(oracle, np.random.default_rng(4), 4, 4096, 256, fmt)
    _check(oracle, case, 14)


@pytest.mark.parametrize("kind,dt", [("awq", "f16"), ("awq", "bf16"), ("gptq4", "bf16"), ("gptq8", "f16"),
                                     ("gptq8", "bf16"), ("nbits2", "f16"), ("nbits4", "f16"),
                                     ("nbits8", "f16")])
def test_checkpoint_case(oracle, kind, dt):
    case = dy.ckpt_case(oracle, np.random.default_rng(6), kind, 8, 4096, 256, 128, dt)
    _check(oracle, case, 16)


def test_lsb_exponent():
    assert dy.lsb_exponent([0.0, 1.5, -3.0]) == -1
    assert dy.lsb_exponent([2.0 ** -20, 7.0]) == -20
    assert dy.lsb_exponent([96.0]) == 5


def test_premise_rejects_inexact_inputs(oracle):
    rng = np.random.default_rng(5)
    a = np.ones((2, 4096))
    w = np.full((4096, 2), 2.0 ** 10 + 2.0 ** -14)  # sums need > 24 bits
    with pytest.raises(AssertionError, match="premise"):
        dy.check_premise(a, w)
    with pytest.raises(AssertionError):
        dy.enc(oracle, np.array([1.0 + 2.0 ** -9], np.float32), "bf16")
    del rng
