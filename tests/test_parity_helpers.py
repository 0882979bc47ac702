"""The GPU tests' parity bounds (tests/parity.py) fail on the mistakes they exist to catch.

CPU only.  Each planted error is one a kernel bug could plausibly make: one wrong row of
256 (a row kernel's stage or a GEMM tile row off by 1%), one dropped 64-deep K tile of an
8192-deep product (a lost LDS stage), an error of 5x the fp32 bar on every element of a
large tensor (which an atol scaled by the maximum over millions of elements lets pass),
one element off by half, and NaN where the reference is finite.  The correct outputs
(fp32 sums in another order, one bf16 rounding) must pass the same bounds.
"""
import pytest
import torch

from parity import close_f32, close_lowp


def _bf16(t):
    return t.to(torch.bfloat16).double()


def _rows(seed=0, shape=(256, 1024)):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64)


def test_one_row_of_256_off_by_one_percent_fails_both_helpers():
    ref = _rows()
    ok32 = ref.float().double()
    close_f32(ok32, ref)
    close_lowp(_bf16(ref), ref)
    bad = ref.clone()
    bad[137] *= 1.01
    with pytest.raises(AssertionError, match="elementwise"):
        close_f32(bad.float().double(), ref)
    with pytest.raises(AssertionError, match="row 137"):
        close_lowp(_bf16(bad), ref)


def _product(drop_tile=None):
    g = torch.Generator().manual_seed(1)
    a = torch.randn(256, 8192, generator=g).to(torch.bfloat16).float()
    b = (0.02 * torch.randn(8192, 256, generator=g)).to(torch.bfloat16).float()
    ref = a.double() @ b.double()
    if drop_tile is not None:
        keep = torch.ones(8192, dtype=torch.bool)
        keep[64 * drop_tile:64 * (drop_tile + 1)] = False
        a, b = a[:, keep], b[keep]
    return a @ b, ref


def test_dropped_64_deep_k_tile_of_an_8192_deep_product_fails_both_helpers():
    out, ref = _product()
    close_f32(out, ref)
    close_lowp(_bf16(out), ref)
    out, ref = _product(drop_tile=77)
    with pytest.raises(AssertionError):
        close_f32(out, ref)
    with pytest.raises(AssertionError):
        close_lowp(_bf16(out), ref)


def test_dropped_k_tile_in_one_output_tile_fails_the_bf16_helper():
    """The realistic race: one 64x64 output tile misses one K tile, the rest is right."""
    out, ref = _product()
    bad, _ = _product(drop_tile=5)
    out[64:128, 128:192] = bad[64:128, 128:192]
    with pytest.raises(AssertionError):
        close_lowp(_bf16(out), ref)


def test_small_error_on_every_element_of_a_large_tensor_fails_fp32():
    g = torch.Generator().manual_seed(2)
    ref = torch.randn(2**22, generator=g)
    # an absolute error of 4e-5 everywhere (5e-5 of a typical element's size, 5x the fp32
    # bar) is what an atol of 1e-5 * max|ref| (~5 rms over 4M Gaussians) lets through
    bad = ref + 4e-5 * torch.sign(ref)
    assert float(((bad - ref).abs() - (1e-5 * ref.abs().max() + 1e-5 * ref.abs())).max()) <= 0
    with pytest.raises(AssertionError, match="elementwise"):
        close_f32(bad, ref)
    close_f32(ref * (1 + 2e-6), ref)


def test_one_element_off_by_half_and_nan_fail():
    ref = _rows(3)
    bad = ref.clone()
    bad[200, 999] *= 1.5
    with pytest.raises(AssertionError):
        close_lowp(_bf16(bad), ref)
    bad = ref.clone()
    bad[3, 4] = float("nan")
    with pytest.raises(AssertionError, match="non-finite"):
        close_f32(bad, ref)


def test_row_floor_keeps_near_zero_rows_at_the_tensor_scale():
    """A row whose reference is ~0 (say gelu of very negative inputs) is held to the
    tensor's RMS, not to its own vanishing norm."""
    ref = _rows(4)
    ref[10] *= 1e-9
    out = ref.clone()
    out[10] += 1e-6 * float(ref.pow(2).mean().sqrt())
    close_f32(out, ref)
