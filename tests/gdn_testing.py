"""Shared helpers of the test-suite: error measures and case naming."""

from __future__ import annotations

import sys

import numpy as np
import torch


def rel_err(got, want) -> float:
    """max |got - want| / max |want| (float64)."""
    got = np.asarray(got.detach().cpu().double() if torch.is_tensor(got) else got, dtype=np.float64)
    want = np.asarray(want.detach().cpu().double() if torch.is_tensor(want) else want, dtype=np.float64)
    scale = np.abs(want).max() if want.size else 0.0
    return float(np.abs(got - want).max() / scale) if scale > 0 else float(np.abs(got - want).max(initial=0.0))


def max_abs(got, want) -> float:
    got = got.detach().cpu().double() if torch.is_tensor(got) else torch.as_tensor(got, dtype=torch.float64)
    want = want.detach().cpu().double() if torch.is_tensor(want) else torch.as_tensor(want, dtype=torch.float64)
    return float((got - want).abs().max()) if got.numel() else 0.0


def announce(msg: str) -> None:
    """Name the case on stderr before a GPU step, flushed, so a fault can be attributed."""
    print(f"[case] {msg}", file=sys.stderr, flush=True)
