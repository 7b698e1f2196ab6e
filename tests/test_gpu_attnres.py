"""Residual routing kernel (zgdn_attnres_route, the drop-in for full_attnres_route of
model/src/zonos3/reference/lm.py:384-389) against the oracle's torch restatement and its float64 statement.

Tolerances: float32 sources -> 1e-5 relative to the float64 statement; bfloat16 sources -> 2e-2 x
max(1, max |output|) max-abs to the torch restatement (both round keys, key-query products, weights and
weighted rows to bf16 as lm.py does; they differ in summation order and rsqrt), i.e. within a couple of
bf16 rounding steps of outputs that reach several units, and a mean |error| below 2e-3 x mean |output|
(most elements round identically, a rounding step is 2^-8 relative: a wrong weight of a percent or more
fails this bound)."""

from __future__ import annotations

import importlib

import pytest
import torch

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _case(S, T, D, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    srcs = [(torch.randn(T, D, generator=gen) * (0.5 + i % 3)).to(dtype) for i in range(S)]
    q = (torch.randn(D, generator=gen) * 0.3).to(dtype)
    return srcs, q


@pytest.mark.parametrize("S,T,D", [(1, 5, 64), (3, 7, 256), (23, 300, 1024), (7, 33, 1536), (64, 4, 2048),
                                   (2, 1, 8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_route_against_the_oracle(gdn, cuda, S, T, D, dtype):
    announce(f"attnres route S={S} T={T} D={D} {dtype}")
    srcs, q = _case(S, T, D, dtype, seed=7000 + S + D)
    attnres = importlib.import_module("zonos3-mini_amd.attnres")
    out = attnres.full_attnres_route([s.to(cuda) for s in srcs], q.to(cuda), 1e-5)
    torch.cuda.synchronize()
    assert out.shape == (T, D) and out.dtype == dtype
    if dtype == torch.float32:
        assert rel_err(out.cpu(), O.attnres_route_np(srcs, q, 1e-5)) < 1e-5
    else:
        ref = O.attnres_route(srcs, q, 1e-5)
        tol = 2e-2 * max(1.0, float(ref.float().abs().max()))
        assert max_abs(out.cpu(), ref) < tol
        _mean_close(out.cpu(), ref)


def _mean_close(out, ref):
    err = (out.float() - ref.float()).abs().mean().item()
    scale = ref.float().abs().mean().item()
    print(f"mean |err| {err:.3e}, mean |ref| {scale:.3e}, differing elements {(out != ref).float().mean():.3f}")
    assert err < 2e-3 * scale, (err, scale)


def test_bank_slices_and_lists_agree(gdn, cuda):
    """A [S, T, dim] bank (the serving layer's form) read in place, also as a slice of a wider preallocated
    buffer (row stride > dim), gives the list form's result exactly."""
    announce("attnres route: bank slice vs list")
    gen = torch.Generator().manual_seed(7101)
    buf = torch.randn(30, 50, 1024 + 64, generator=gen).to(torch.bfloat16).to(cuda)
    bank = buf[:23, :, :1024]
    q = (0.3 * torch.randn(1024, generator=gen)).to(torch.bfloat16).to(cuda)
    a = gdn.ops.attnres_route(bank, q, 1e-6)
    b = gdn.ops.attnres_route([bank[i].contiguous() for i in range(23)], q, 1e-6)
    c = torch.ops.zgdn.attnres_route([bank[i] for i in range(23)], q, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)
    ref = O.attnres_route(bank.cpu(), q.cpu(), 1e-6)
    assert max_abs(a.cpu(), ref) < 2e-2 * max(1.0, float(ref.float().abs().max()))
    _mean_close(a.cpu(), ref)


def test_patch_rebinds_a_module_function(gdn, cuda):
    import types

    attnres = importlib.import_module("zonos3-mini_amd.attnres")
    mod = types.SimpleNamespace(full_attnres_route=O.attnres_route)
    attnres.patch(mod)
    srcs, q = _case(3, 4, 128, torch.float32, 7201)
    out = mod.full_attnres_route([s.to(cuda) for s in srcs], q.to(cuda), 1e-5)
    assert out.is_cuda and rel_err(out.cpu(), O.attnres_route(srcs, q, 1e-5)) < 1e-5
