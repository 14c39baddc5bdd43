"""Parity metrics and the north-star tolerances (bf16 HIP path vs fp32/fp64 oracle)."""

import json
import os

import torch

MAX_ABS = 2e-2    # layer / op outputs, max |a - b|
MEAN_REL = 5e-3   # mean |a - b| / mean |b|


def metrics(actual, expected):
    a = actual.detach().double().cpu()
    b = expected.detach().double().cpu()
    diff = (a - b).abs()
    return {
        "max_abs": diff.max().item() if diff.numel() else 0.0,
        "mean_rel": (diff.mean() / b.abs().mean().clamp_min(1e-30)).item() if diff.numel() else 0.0,
        "rrms": (diff.norm() / b.norm().clamp_min(1e-30)).item() if diff.numel() else 0.0,
    }


def assert_close(actual, expected, max_abs=MAX_ABS, mean_rel=MEAN_REL, what=""):
    m = metrics(actual, expected)
    log = os.environ.get("CYFA_PARITY_LOG")
    if log:  # record the margins of every comparison (one JSON object per line)
        with open(log, "a") as f:
            f.write(json.dumps({"what": what, **m}) + "\n")
    assert m["max_abs"] <= max_abs and m["mean_rel"] <= mean_rel, f"{what} parity failed: {m}"
    return m
