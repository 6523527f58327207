"""Both halves of the tolerance definition the conv tests use.

(i)  norm-wise relative error  max|y - r| / max|r|
(ii) per-element allclose with atol = rtol * rms(r):  |y - r| <= rtol * rms(r) + rtol * |r| for
     every element (the reference's allclose, src/validation/compare.ts:17-23, with that atol).

r is an fp32 / fp64 result computed from the same rounded inputs and weights.  A test passes when
(i) <= rtol; it also asserts (ii) and prints both, with the worst element's ratio
|y - r| / (atol + rtol * |r|) (<= 1 means allclose holds everywhere).
"""
from __future__ import annotations

import numpy as np
import torch


def errors(got, ref, rtol: float) -> dict:
    """{'normwise', 'allclose', 'worst_ratio', 'rms'} for tensors or arrays of the same shape."""
    if isinstance(got, torch.Tensor) or isinstance(ref, torch.Tensor):
        g = torch.as_tensor(got).double()
        r = torch.as_tensor(ref).double().to(g.device)
        d = (g - r).abs()
        rms = float(r.pow(2).mean().sqrt())
        normwise = float(d.max() / max(float(r.abs().max()), 1e-30))
        worst = float((d / (rtol * rms + rtol * r.abs()).clamp_min(1e-300)).max())
    else:
        g = np.asarray(got, np.float64)
        r = np.asarray(ref, np.float64)
        d = np.abs(g - r)
        rms = float(np.sqrt(np.mean(r * r)))
        normwise = float(d.max() / max(np.abs(r).max(), 1e-30))
        worst = float((d / np.maximum(rtol * rms + rtol * np.abs(r), 1e-300)).max())
    return {"normwise": normwise, "allclose": worst <= 1.0, "worst_ratio": worst, "rms": rms}


def check(got, ref, rtol: float, label: str = "") -> dict:
    e = errors(got, ref, rtol)
    print(f"  {label} norm-wise {e['normwise']:.3e} (tol {rtol:g}); per-element allclose "
          f"atol=rtol*rms: worst ratio {e['worst_ratio']:.3f}", flush=True)
    assert e["normwise"] <= rtol, e
    assert e["allclose"], e
    return e
