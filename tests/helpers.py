"""Tolerances and error metrics shared by the parity tests.

Gates (from the north star): fp32 within rtol 1e-5 and bf16/fp16 within rtol
2e-2 of the float reference. Every comparison also carries an absolute
floor for elements near zero, stated here: fp32 atol = 1e-5 * max|expected|
(at least 1e-6), 16-bit atol = 1e-2 * max|expected|.
"""
import torch

RTOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
ATOL_SCALE = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def error_metrics(actual, expected):
    """max abs error and relative RMS error (reference st/tools/validate.py:59-63)."""
    a, e = actual.detach().double().cpu(), expected.detach().double().cpu()
    finite = torch.isfinite(e)
    diff = (a - e).abs()[finite]
    rms = e[finite].square().mean().sqrt().clamp_min(1e-12)
    return {"max_abs": float(diff.max()) if diff.numel() else 0.0,
            "relative_rms": float(diff.square().mean().sqrt() / rms) if diff.numel() else 0.0}


def assert_close(actual, expected, dtype, name=""):
    """|a - e| <= atol + rtol |e| elementwise with the tolerances above; -inf
    entries must match exactly."""
    a, e = actual.detach().double().cpu(), expected.detach().double().cpu()
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    inf_e, inf_a = torch.isinf(e), torch.isinf(a)
    assert torch.equal(inf_e, inf_a) and torch.equal(a[inf_e], e[inf_e]), f"{name}: infinite entries differ"
    assert not torch.isnan(a).any(), f"{name}: NaN in result"
    fin = ~inf_e
    scale = float(e[fin].abs().max()) if fin.any() else 0.0
    atol = max(ATOL_SCALE[dtype] * scale, 1e-6 if dtype == torch.float32 else 0.0)
    torch.testing.assert_close(a[fin], e[fin], rtol=RTOL[dtype], atol=atol,
                               msg=lambda m: f"{name}: {m} ({error_metrics(a[fin], e[fin])})")
