"""tj_gelu16, the gelu of GEMM epilogues whose outputs are bf16 / fp16 (CPU only).

Its constants are read from the device prelude itself, so a mistyped one fails here:
they must be the published ones of Abramowitz & Stegun 7.1.25 and, evaluated in float64,
stay within that formula's published bound (|error| <= 2.5e-5) of ``math.erf``.  The
device function's rearranged form, 0.5 (x + |x|) - a q, is then evaluated step by step
in float32 and must stay within 1.3e-5 |x| (half the erf bound, as gelu halves it) plus
fp32 rounding of the exact gelu, which a dropped factor or a flipped sign breaks.  The
GPU test of the same function through a bf16 GEMM epilogue is in test_hip_gpu.py.
"""
import math
import re

import numpy as np
import pytest

from tensorjit.backends.hip_prelude import PRELUDE

A_S_7_1_25 = (0.47047, [0.3480242, -0.0958798, 0.7478556])   # p, a1..a3 (A&S, 1964)


def _body() -> str:
    m = re.search(r"float tj_gelu16\(float x\) \{(.*?)\n\}", PRELUDE, re.S)
    assert m, "tj_gelu16 missing from the prelude"
    return m.group(1)


def _constants() -> tuple[float, list[float]]:
    body = _body()
    p = float(re.search(r"__builtin_fmaf\((-?[0-9.]+)f \* 0\.70710678118654752f, a, 1\.0f\)", body).group(1))
    coeffs = [float(c) for c in re.findall(r"0\.5f \* (-?[0-9.]+)f", body)[:3]]
    return p, coeffs


def _erf_7_1_25(z: np.ndarray, p: float, coeffs: list[float]) -> np.ndarray:
    t = 1.0 / (1.0 + p * z)
    poly = np.zeros_like(z)
    for c in reversed(coeffs):
        poly = c + t * poly
    return 1.0 - t * poly * np.exp(-z * z)


def test_prelude_constants_are_a_and_s_7_1_25():
    assert _constants() == A_S_7_1_25


def test_constants_meet_the_published_bound_against_math_erf():
    p, coeffs = _constants()
    z = np.linspace(0.0, 6.0, 120001)
    exact = np.array([math.erf(v) for v in z])
    err = np.abs(_erf_7_1_25(z, p, coeffs) - exact)
    assert err.max() <= 2.5e-5
    # a planted mistake in one coefficient (a3 off by 2e-4) no longer meets the bound
    bad = [coeffs[0], coeffs[1], coeffs[2] + 2e-4]
    assert np.abs(_erf_7_1_25(z, p, bad) - exact).max() > 2.5e-5


def _gelu16_f32(x: np.ndarray, p: float, coeffs: list[float]) -> np.ndarray:
    """The device function's steps in float32 (transcendentals in float64, rounded)."""
    f = np.float32
    x = x.astype(np.float32)
    a = np.minimum(np.abs(x), f(5.656854249))
    t = (1.0 / (f(p) * f(0.70710678118654752) * a + f(1.0)).astype(np.float64)).astype(np.float32)
    c = [f(0.5) * f(v) for v in coeffs]
    q = t * (c[0] + t * (c[1] + t * c[2]))
    e = np.exp2((a * a * (f(-0.5) * f(1.4426950408889634))).astype(np.float64)).astype(np.float32)
    return f(0.5) * (x + np.abs(x)) - a * (q * e)


@pytest.mark.parametrize("lo,hi", [(-9.0, -2.0), (-2.0, 0.0), (0.0, 2.0), (2.0, 9.0)])
def test_rearranged_form_stays_within_the_bound_of_the_exact_gelu(lo, hi):
    p, coeffs = _constants()
    x = np.linspace(lo, hi, 40001).astype(np.float32)
    exact = np.array([0.5 * float(v) * math.erfc(-float(v) / math.sqrt(2.0)) for v in x])
    got = _gelu16_f32(x, p, coeffs).astype(np.float64)
    bound = 1.3e-5 * np.abs(x) + 4 * np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64) + 1e-12
    assert np.all(np.abs(got - exact) <= bound)


def test_special_values_follow_tj_gelu():
    p, coeffs = _constants()
    with np.errstate(invalid="ignore"):
        got = _gelu16_f32(np.array([np.inf, -np.inf, np.nan, 0.0], dtype=np.float32), p, coeffs)
    assert got[0] == np.inf and np.isnan(got[1]) and np.isnan(got[2]) and got[3] == 0.0


@pytest.mark.parametrize("dt,fast", [("bf16", True), ("f16", True), ("f32", False)])
def test_gemm_epilogues_take_tj_gelu16_only_for_16_bit_outputs(dt, fast):
    import tensorjit as tj
    from tensorjit import compiler as C
    from tensorjit.backends import hip_backend as hb
    from tensorjit.ir import DType, TensorType

    d = {"bf16": DType.bf16, "f16": DType.f16, "f32": DType.f32}[dt]
    fn = lambda x, w, b: tj.gelu(tj.linear(x, w, b))  # noqa: E731
    p = C.lower(tj.trace(fn, [TensorType(s, d) for s in [(512, 256), (768, 256), (768,)]]), "hip")
    src, _ = hb.generate(p)
    kernels = src[len(hb.PRELUDE):]
    assert ("tj_gelu16(" in kernels) == fast and ("tj_gelu(" in kernels) != fast
    # the pointwise family keeps the reference's formula at every dtype
    q = C.lower(tj.trace(lambda x: tj.gelu(x) * 2.0, [TensorType((512, 256), d)]), "hip")
    src, _ = hb.generate(q)
    assert "tj_gelu(" in src[len(hb.PRELUDE):] and "tj_gelu16(" not in src[len(hb.PRELUDE):]
