"""Accent adapter shifts of the GDN mixer's projections on the HIP kernel.

The reference adds a per-row low-rank shift to ``in_proj`` and ``wo`` of every adapted op
(``servers/sgl/src/zonos3_sgl/layers/accent.py:25-62``; ``models/gdn.py:400-401, 448-449``):
``y + ((x @ down.T) * mask) @ up`` with the op's ``_accent = (down [K, in], up [K, out])`` and the batch's
``[rows, K]`` mask. ``accent_shift`` / ``apply_accent`` keep those names, arguments and results
(``apply_accent`` returns ``y`` itself for an op without adapters or without a mask), computed by one
``zgdn_accent_shift`` call: two launches instead of two GEMMs, a product and a sum. Rows are computed
independently in a fixed order, so ``_accent_block_rows`` (the reference's fixed-shape row blocks for batch
invariance) is not needed and is ignored.

``AccentHooks(mask_source)`` is the object ``serving.OriginalGDN(accent=...)`` takes (``accent_mask()`` and
``apply_accent(op, x, y, mask)``); ``patch(module)`` rebinds ``accent_shift`` in a module such as
``zonos3_sgl.layers.accent``, whose ``apply_accent`` then runs the kernel.
"""

from __future__ import annotations

import importlib
from typing import Callable, Optional

ops = importlib.import_module(__package__ + ".ops")


def accent_shift(op, x, mask):
    """``((x @ down.T) * mask) @ up`` for an adapted op (accent.py:25-45), as a new tensor."""
    down, up = op._accent
    return ops.accent_shift(x, down, up, mask)


def apply_accent(op, x, y, mask):
    """``y`` plus the op's per-row shift (accent.py:48-62) as a new tensor; ``y`` itself when the op has no
    adapters or ``mask`` is None."""
    if op.__dict__.get("_accent") is None or mask is None:
        return y
    down, up = op._accent
    return ops.accent_shift(x, down, up, mask, y=y)


class AccentHooks:
    """``accent_mask()`` from ``mask_source`` (the engine's current [tokens, K] mask, or None) and
    ``apply_accent`` on the kernel: the ``accent`` argument of ``serving.OriginalGDN``."""

    def __init__(self, mask_source: Optional[Callable] = None):
        self._mask_source = mask_source

    def accent_mask(self):
        return None if self._mask_source is None else self._mask_source()

    def apply_accent(self, op, x, y, mask=None):
        if mask is None:
            mask = self.accent_mask()
        return apply_accent(op, x, y, mask)


def patch(module) -> None:
    """Rebind ``module.accent_shift`` (e.g. ``zonos3_sgl.layers.accent``) to the kernel."""
    module.accent_shift = accent_shift
