"""Parity bounds shared by the GPU tests (and pinned on the CPU by test_parity_helpers.py).

Each comparison of a kernel's output with its reference applies three bounds, all scaled
by the reference's root-mean-square value rather than its maximum (over 1e8 Gaussian
elements the maximum is ~6x the RMS and grows with the tensor, so a max-scaled absolute
tolerance goes blind at full size):

* elementwise: ``|out - ref| <= atol + rtol * |ref|`` with ``atol = scale * rms(ref)``;
* norm-wise:   ``||out - ref||_2 <= norm * ||ref||_2`` over the whole tensor;
* row-wise:    the same ratio for every row (last axis), with the row's norm floored at
  ``rms(ref) * sqrt(N)`` so a row of near-zero reference values is not held to a bound
  below the tensor's own scale.  One wrong row of 256 moves the whole-tensor norm by only
  1/16 of its own error; the row bound sees it.

fp32 (the north star's 1e-5): ``rtol = scale = norm = 1e-5``; a reduction over n terms
passes ``scale = 1e-5 * sqrt(n / n0)`` and the norm bound follows it.
bf16 / fp16 outputs against the fp32 oracle: elementwise 2e-2 (the north star's GEMM
bound) and norm / row 5e-3.  One round-to-nearest bf16 store leaves an RMS relative
error of 2^-7 * sqrt(E[1/m^2]) / sqrt(12) = 1.66e-3 (mantissa m log-uniform on [1, 2)),
so 5e-3 is three such roundings; chains that store bf16 intermediates between kernels
pass a wider ``norm`` with the reason at the call.

With ``TJ_PARITY_LOG=<file>`` every comparison appends one JSON line with the observed
fraction of each bound, so the margins of a whole GPU run can be read afterwards.
"""
from __future__ import annotations

import json
import math
import os

import torch

F32_TOL = 1e-5
LOWP_ELEM = 2e-2
LOWP_NORM = 5e-3


def _host32(t: torch.Tensor) -> torch.Tensor:
    t = t.detach()
    if t.is_cuda:
        t = t.cpu()
    return t.double() if t.numel() < 2**25 else t.float()


def _log(record: dict) -> None:
    path = os.environ.get("TJ_PARITY_LOG")
    if not path:
        return
    record["test"] = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    with open(path, "a") as fh:
        fh.write(json.dumps(record) + "\n")


def compare(out, ref, *, rtol: float, scale: float, norm: float, what: str = "") -> dict:
    """Apply the three bounds; return the fraction of each bound used (<= 1 passes)."""
    out, ref = _host32(out), _host32(ref)
    assert out.shape == ref.shape, (what, tuple(out.shape), tuple(ref.shape))
    fin_o, fin_r = torch.isfinite(out), torch.isfinite(ref)
    assert torch.equal(fin_o, fin_r), f"{what}: non-finite values differ ({int((fin_o != fin_r).sum())} elements)"
    if not bool(fin_r.all()):
        assert torch.equal(out[~fin_r], ref[~fin_r]), f"{what}: non-finite values differ"
        out, ref = out[fin_r], ref[fin_r]
    if ref.numel() == 0:
        return {}
    n = ref.shape[-1] if ref.dim() >= 1 else 1
    d = out - ref
    rows_d = d.reshape(-1, n)
    rows_r = ref.reshape(-1, n)
    rows_err = torch.linalg.vector_norm(rows_d, dim=-1, dtype=torch.float64)
    rows_ref = torch.linalg.vector_norm(rows_r, dim=-1, dtype=torch.float64)
    err_norm = float(torch.linalg.vector_norm(rows_err))
    ref_norm = float(torch.linalg.vector_norm(rows_ref))
    rms = ref_norm / math.sqrt(ref.numel())
    tiny = 1e-30
    atol = max(scale * rms, tiny)
    excess = d.abs() - rtol * ref.abs()
    elem = float(excess.max()) / atol
    whole = err_norm / max(norm * ref_norm, tiny)
    floor = rms * math.sqrt(n)
    row = float((rows_err / (norm * rows_ref.clamp(min=floor)).clamp(min=tiny)).max())
    rec = {"what": what, "numel": ref.numel(), "rms": rms, "elem": elem, "norm": whole, "row": row,
           "rtol": rtol, "scale": scale, "norm_bound": norm}
    _log(rec)
    worst = int(torch.argmax(excess.reshape(-1)))
    assert elem <= 1.0, (f"{what}: elementwise bound exceeded {elem:.3g}x (atol {atol:.3e} = {scale:g} * rms "
                         f"{rms:.3e}, rtol {rtol:g}); worst at flat index {worst}: "
                         f"{float(out.reshape(-1)[worst]):.6g} vs {float(ref.reshape(-1)[worst]):.6g}")
    assert whole <= 1.0, f"{what}: ||out-ref|| / ||ref|| = {err_norm / max(ref_norm, tiny):.3e} > {norm:g}"
    assert row <= 1.0, (f"{what}: row {int(torch.argmax(rows_err / rows_ref.clamp(min=floor)))} of {rows_r.shape[0]} "
                        f"off by {row * norm:.3e} of its norm > {norm:g}")
    return rec


def close_f32(out, ref, rtol: float = F32_TOL, scale: float = F32_TOL, norm: float | None = None, what: str = ""):
    """fp32 output against its fp32 / float64 reference."""
    return compare(out, ref, rtol=rtol, scale=scale, norm=max(rtol, scale) if norm is None else norm, what=what)


def close_lowp(out, ref, tol: float = LOWP_ELEM, norm: float = LOWP_NORM, what: str = ""):
    """bf16 / fp16 output against the fp32 reference of the same (upcast) inputs."""
    return compare(out, ref, rtol=tol, scale=tol, norm=norm, what=what)


def stored(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``t`` (float64) as a kernel stores it in ``dtype``: rounded to fp32 where the kernel
    computes, then to ``dtype`` (round to nearest even), back in float64."""
    return t.float().to(dtype).double()


def attention_plan_reference(q, k, v, scores, dtype) -> torch.Tensor:
    """The reference plan's unfused attention (scores kernel -> softmax row kernel -> PV
    kernel) in float64 with its two intermediate stores rounded to the storage type:
    ``scores(q @ k^T)`` and ``softmax(.)``.  At bf16 a stored logit ``s`` is off by up to
    2^-8 |s|, which moves its probability by that much relative: for logits of a few units
    this error exceeds the output's own rounding several times over, so a plan that stores
    scores is compared with this emulation rather than with the fp32 oracle alone."""
    qd, kd, vd = (t.detach().cpu().double() for t in (q, k, v))
    s = stored(scores(qd @ kd.transpose(-1, -2).contiguous()), dtype)
    p = stored(torch.softmax(s, dim=-1), dtype)
    return p @ vd
