"""Drop-in for the LM's residual routing, ``full_attnres_route(sources, query, eps)``
(``model/src/zonos3/reference/lm.py:384-389``; ``servers/sgl/src/zonos3_sgl/models/zonos3.py:99-113``), on
the HIP kernel ``zgdn_attnres_route``: the mix of all residual sources that every GDN (and attention / FFN)
sublayer reads.

``sources`` is lm.py's list of [T, dim] tensors or the serving layer's stacked [S, T, dim] bank; both are
read in place (a list is not stacked, a bank may be a slice of a preallocated buffer). ``patch(module)``
rebinds the function of a reference module (``zonos3.reference.lm`` or ``zonos3_sgl.models.zonos3``), whose
forward passes look it up by name.
"""

from __future__ import annotations

from . import ops


def full_attnres_route(sources, query, eps):
    """Per token: softmax over the sources of rms_norm(x_s) . query (fp32), then the weighted sum of the raw
    sources. Returns [T, dim] in the sources' dtype."""
    return ops.attnres_route(sources, query, eps)


def patch(module) -> None:
    """Point ``module.full_attnres_route`` at this implementation."""
    module.full_attnres_route = full_attnres_route
