"""CPU check of the constants of the fused erf-GELU epilogue of the
weight-transposed FP16 GEMM (kernels/gemm_fp16_nt.hip, GeluErfAs): the
polynomial coefficients are read from the kernel source, the same FP32
evaluation order is replayed in numpy, and the result is compared with
scipy's erf in float64. A mistyped coefficient or a wrong scaling of the
Abramowitz & Stegun 7.1.28 constants fails here before any GPU run."""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
from scipy.special import erf

SOURCE = Path(__file__).resolve().parents[1] / "cutriton_amd" / "kernels" / "gemm_fp16_nt.hip"


def _coefficients() -> list[float]:
    text = SOURCE.read_text()
    body = text[text.index("float GeluErfAs(float a) {"):]
    body = body[:body.index("\n}\n")]
    lead = re.search(r"float p = ([0-9.e+-]+)f;", body)
    rest = re.findall(r"p = __builtin_fmaf\(p, x, ([0-9.e+-]+)f\);", body)
    assert lead and len(rest) == 6, "GeluErfAs no longer has the degree-6 Horner form this check reads"
    return [float(lead.group(1))] + [float(c) for c in rest]  # highest degree first


def _gelu_fp32(a: np.ndarray, coeffs: list[float]) -> np.ndarray:
    a = a.astype(np.float32)
    x = np.abs(a)
    p = np.full_like(x, np.float32(coeffs[0]))
    for c in coeffs[1:]:
        p = (p * x + np.float32(c)).astype(np.float32)
    for _ in range(4):
        p = (p * p).astype(np.float32)
    with np.errstate(over="ignore", divide="ignore"):
        q = (np.float32(1.0) / p).astype(np.float32)
    return (np.maximum(a, np.float32(0.0)) - np.minimum(x, np.float32(16.0)) * q).astype(np.float32)


def test_coefficients_are_scaled_a_and_s_7_1_28():
    # a_i of A&S 7.1.28 over sqrt(2)^i, times 2^(1/16) (the leading 1 too).
    a = [1.0, 0.0705230784, 0.0422820123, 0.0092705272, 0.0001520143, 0.0002765672, 0.0000430638]
    want = [a[i] / np.sqrt(2.0) ** i * 2.0 ** (1.0 / 16.0) for i in range(7)][::-1]
    got = _coefficients()
    assert np.allclose(got, want, rtol=2e-7, atol=0.0), (got, want)


def test_epilogue_formula_within_1e6_of_erf_gelu():
    pre = np.concatenate([np.linspace(-12.0, 12.0, 200001), [0.0, 1e-6, -1e-6, 16.0, -16.0, 40.0, -40.0]])
    got = _gelu_fp32(pre, _coefficients()).astype(np.float64)
    want = 0.5 * pre * (1.0 + erf(pre / np.sqrt(2.0)))
    assert np.max(np.abs(got - want)) < 1e-6
    # the tails: exactly max(a, 0) far out, +inf kept
    big = np.float32(1e30)
    assert _gelu_fp32(np.array([np.inf, big, -big]), _coefficients()).tolist() == [np.inf, float(big), 0.0]


def test_a_mistyped_coefficient_is_caught():
    coeffs = _coefficients()
    coeffs[3] *= 1.01  # the x^3 term one percent off
    pre = np.linspace(-12.0, 12.0, 20001)
    got = _gelu_fp32(pre, coeffs).astype(np.float64)
    want = 0.5 * pre * (1.0 + erf(pre / np.sqrt(2.0)))
    assert np.max(np.abs(got - want)) > 1e-6
