"""Comparison helpers shared by the parity tests."""
from __future__ import annotations

import json
import os

import torch


def record_audit(what: str, stats: dict) -> None:
    """Append one parity-audit record (JSON line) to the file named by
    JO_ULP_AUDIT, when that variable is set."""
    path = os.environ.get("JO_ULP_AUDIT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(dict(what=what, **stats)) + "\n")


def bf16_ulp(ref: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |ref| (8 significant bits), floored at the smallest normal."""
    a = ref.abs().float().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def assert_bf16_within_ulp(out: torch.Tensor, ref_f32: torch.Tensor, floor_scale=None,
                           n_ulp: float = 1.0, what: str = "", floor_cap: float | None = None):
    """|out - ref| <= n_ulp bf16 ulps of ref, element-wise.

    The fp32 reference and the kernel accumulate in different orders; where a
    result is the difference of nearly equal terms (a rotated pair, x - mean)
    the fp32 rounding of the terms dominates a tiny result. `floor_scale`
    (a tensor broadcastable to ref, e.g. the row/head max |ref|) floors the
    ulp at that of floor_scale * 2^-10 to absorb that cancellation.

    Returns the audit of that floor: `floor_only`, the number of finite
    elements within n_ulp of the floored ulp but not of their own bf16 ulp,
    and `floor_only_max_ulps`, the largest error among them in bf16 ulps of
    the element itself. With `floor_cap` set, at most that fraction of the
    elements may pass through the floor alone.
    """
    out = out.float().cpu()
    ref = ref_f32.float().cpu()
    own = bf16_ulp(ref)
    ulp = own
    if floor_scale is not None:
        ulp = torch.maximum(own, bf16_ulp(floor_scale.float().cpu() * 2.0 ** -10))
    err = (out - ref).abs()
    nan_ok = torch.isnan(out) == torch.isnan(ref)
    assert bool(nan_ok.all()), f"{what}: NaN pattern differs"
    fin = torch.isfinite(ref)
    bad = (err > n_ulp * ulp) & fin
    if bool(bad.any()):
        i = int(bad.reshape(-1).nonzero()[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} elements beyond {n_ulp} bf16 ulp; first at flat index {i}: "
            f"out={out.reshape(-1)[i].item()!r} ref={ref.reshape(-1)[i].item()!r} "
            f"ulp={ulp.reshape(-1)[i].item()!r}; max err/ulp={(err / ulp)[fin].max().item():.3f}")
    floor_only = (err > n_ulp * own) & fin
    n_floor = int(floor_only.sum())
    stats = {"elements": ref.numel(), "floor_only": n_floor,
             "floor_only_frac": n_floor / max(1, ref.numel()),
             "floor_only_max_ulps": float((err / own)[floor_only].max()) if n_floor else 0.0}
    if floor_scale is not None and n_floor:
        # the same errors relative to the floor's scale (the head / row maximum):
        # meaningful where the reference itself is 0 or nearly so
        rel = err / floor_scale.float().cpu().expand_as(err).clamp_min(2.0 ** -126)
        stats["floor_only_max_rel"] = float(rel[floor_only].max())
    record_audit(what, stats)
    if floor_cap is not None:
        assert n_floor <= floor_cap * ref.numel(), (
            f"{what}: {n_floor} of {ref.numel()} elements pass only through the 2^-10 floor "
            f"(cap {floor_cap:g}); largest error among them {stats['floor_only_max_ulps']:.1f} "
            "bf16 ulps of the element")
    return stats


def f32_ulp(v: torch.Tensor) -> torch.Tensor:
    a = v.abs().float().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 23)


MANTISSA_BITS = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}


def assert_within_ulp(out: torch.Tensor, ref_f32: torch.Tensor, dtype, floor_scale=None,
                      n_ulp: float = 1.0, what: str = ""):
    """Like assert_bf16_within_ulp for any output dtype (bf16: 7, fp16: 10,
    fp32: 23 fraction bits). fp32 outputs are allowed n_ulp * 8 ulps, the
    spread of fp32 sums accumulated in different orders, and their ulp is
    floored at the ulp of floor_scale itself: a modulated output that cancels
    to near zero keeps the absolute rounding error of its O(floor_scale)
    terms (fused vs separate multiply-add)."""
    mb = MANTISSA_BITS[dtype]
    out = out.float().cpu()
    ref = ref_f32.float().cpu()

    def ulp_of(v):
        a = v.abs().clamp_min(2.0 ** -126)
        return torch.exp2(torch.floor(torch.log2(a)) - mb)

    ulp = ulp_of(ref)
    if floor_scale is not None:
        shift = 0 if dtype == torch.float32 else 10
        ulp = torch.maximum(ulp, ulp_of(floor_scale.float().cpu() * 2.0 ** -shift))
    if dtype == torch.float32:
        n_ulp = n_ulp * 8
    err = (out - ref).abs()
    fin = torch.isfinite(ref)
    assert bool((torch.isnan(out) == torch.isnan(ref)).all()), f"{what}: NaN pattern differs"
    bad = (err > n_ulp * ulp) & fin
    if bool(bad.any()):
        i = int(bad.reshape(-1).nonzero()[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.numel()} elements beyond {n_ulp} ulp ({dtype}); "
            f"first at flat index {i}: out={out.reshape(-1)[i].item()!r} "
            f"ref={ref.reshape(-1)[i].item()!r}; max err/ulp={(err / ulp)[fin].max().item():.3f}")
