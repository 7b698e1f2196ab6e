"""Accent adapter shift kernel (zgdn_accent_shift, the drop-in for accent_shift / apply_accent of
servers/sgl/src/zonos3_sgl/layers/accent.py:25-62 on the GDN mixer's in_proj and wo) against the oracle.

Shapes cover both down kernels: the LDS-staged one (inputs of at most 1024, ranks up to 64, including a width
that is not a multiple of 32) and the unstaged one (rank 256; 1040 inputs).

Tolerances: float32 -> 1e-5 relative to the float64 statement; bfloat16 -> 2e-2 x max(1, max |ref|) max-abs to
the torch restatement (both round x @ down.T, the masked product, the @ up product and the sum with y to
bf16; they differ in summation order), i.e. within a couple of bf16 rounding steps. Batch invariance (the
property the reference's ensure_batch_invariance checks, models/accent_adapters.py:318-348), zero-mask rows,
in-place updates and strided rows are bit-exact."""

from __future__ import annotations

import importlib
from types import SimpleNamespace

import pytest
import torch

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _case(rows, n_in, n_out, K, dtype, seed, zero_rows=()):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, n_in, generator=gen)
    down = torch.randn(K, n_in, generator=gen) / n_in**0.5
    up = torch.randn(K, n_out, generator=gen) / K**0.5
    y = torch.randn(rows, n_out, generator=gen)
    # two adapters of half the columns each; every row on one of them at a strength in [0.5, 1.5)
    mask = torch.zeros(rows, K)
    pick = torch.randint(0, 2, (rows,), generator=gen)
    alpha = 0.5 + torch.rand(rows, generator=gen)
    for r in range(rows):
        lo, hi = (0, K // 2) if pick[r] == 0 else (K // 2, K)
        mask[r, lo:hi] = alpha[r]
    for r in zero_rows:
        mask[r] = 0.0
    return [t.to(dtype) for t in (x, down, up, mask, y)]


def _check(got, x, down, up, mask, y, dtype):
    if dtype == torch.float32:
        assert rel_err(got.cpu(), O.accent_shift_np(x, down, up, mask, y)) < 1e-5
    else:
        ref = O.accent_shift(x, down, up, mask, y)
        assert max_abs(got.cpu(), ref) < 2e-2 * max(1.0, float(ref.float().abs().max()))


@pytest.mark.parametrize("rows,n_in,n_out,K", [(1, 1024, 2056, 64), (7, 1024, 2056, 16), (300, 512, 1024, 40),
                                               (130, 1024, 2056, 256), (65, 64, 1032, 8), (33, 1000, 520, 64),
                                               (17, 1040, 264, 32)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_shift_against_the_oracle(gdn, cuda, rows, n_in, n_out, K, dtype):
    announce(f"accent shift rows={rows} in={n_in} out={n_out} K={K} {dtype}")
    x, down, up, mask, y = _case(rows, n_in, n_out, K, dtype, seed=8000 + rows + K)
    d = [t.to(cuda) for t in (x, down, up, mask, y)]
    got = gdn.ops.accent_shift(*d[:4], y=d[4])
    shift = gdn.ops.accent_shift(*d[:4])
    torch.cuda.synchronize()
    _check(got, x, down, up, mask, y, dtype)
    _check(shift, x, down, up, mask, None, dtype)


def test_batch_invariance_zero_rows_in_place_and_strides(gdn, cuda):
    """Rows computed in one call equal the same rows computed alone or in any sub-batch; rows with a zero mask
    keep y's bits; out=y updates in place; x, y, out as slices of wider rows (aligned or not) change nothing."""
    announce("accent shift: batch invariance, zero rows, in place, strides")
    x, down, up, mask, y = (t.to(cuda) for t in _case(300, 1024, 2056, 48, torch.bfloat16, 8101,
                                                      zero_rows=(0, 5, 77)))
    full = gdn.ops.accent_shift(x, down, up, mask, y=y)
    for n in (1, 2, 3, 4, 5, 8, 16, 64, 256):
        assert torch.equal(gdn.ops.accent_shift(x[:n], down, up, mask[:n], y=y[:n]), full[:n]), n
    assert torch.equal(gdn.ops.accent_shift(x[100:137], down, up, mask[100:137], y=y[100:137]), full[100:137])
    for r in (0, 5, 77):
        assert torch.equal(full[r], y[r])
    y2 = y.clone()
    assert gdn.ops.accent_shift(x, down, up, mask, y=y2, out=y2) is y2
    assert torch.equal(y2, full)
    xw = torch.zeros(300, 1024 + 64, dtype=torch.bfloat16, device=cuda)
    xw[:, 8:1032] = x
    for pad in (8, 1):  # y rows 2064 (8-byte aligned) and 2057 (not) elements apart
        yw = torch.zeros(300, 2056 + pad, dtype=torch.bfloat16, device=cuda)
        yw[:, :2056] = y
        out = torch.zeros_like(yw)
        gdn.ops.accent_shift(xw[:, 8:1032], down, up, mask, y=yw[:, :2056], out=out[:, :2056])
        assert torch.equal(out[:, :2056], full), pad
    torch.cuda.synchronize()


def test_drop_in_functions_and_torch_op(gdn, cuda):
    accent = importlib.import_module("zonos3-mini_amd.accent")
    x, down, up, mask, y = (t.to(cuda) for t in _case(20, 512, 1024, 32, torch.bfloat16, 8201))
    op = SimpleNamespace(_accent=(down, up))
    plain = SimpleNamespace()
    assert accent.apply_accent(plain, x, y, mask) is y  # an op without adapters
    assert accent.apply_accent(op, x, y, None) is y  # no mask: no adapters in the batch
    a = accent.apply_accent(op, x, y, mask)
    b = y + accent.accent_shift(op, x, mask)
    c = torch.ops.zgdn.accent_shift(x, down, up, mask, y)
    hooks = accent.AccentHooks(lambda: mask)
    d = hooks.apply_accent(op, x, y)
    torch.cuda.synchronize()
    assert torch.equal(a, c) and torch.equal(a, d)
    assert max_abs(a.cpu(), b.cpu()) < 2e-2 * max(1.0, float(a.float().abs().max()))
    module = SimpleNamespace(accent_shift=None)
    accent.patch(module)
    assert module.accent_shift is accent.accent_shift


def test_serving_packed_pass_with_accents(gdn, cuda):
    """OriginalGDN._run_packed with accent hooks on in_proj and wo: the native shift against the same pass
    whose hooks compute the shift with torch ops on the GPU (the reference's accent_shift)."""
    announce("serving packed pass with accent adapters: native vs torch shifts")
    serving = importlib.import_module("zonos3-mini_amd.serving")
    accent = importlib.import_module("zonos3-mini_amd.accent")
    gen = torch.Generator().manual_seed(8301)
    bf, hid, K = torch.bfloat16, 256, 32
    rows = [70, 1, 130]
    n = sum(rows)
    layer = serving.OriginalGDN(SimpleNamespace(hidden_size=hid), 0)
    layer.in_proj.weight = (0.05 * torch.randn(2056, hid, generator=gen)).to(bf).to(cuda)
    layer.conv.weight = (0.2 * torch.randn(1536, 1, 4, generator=gen)).to(bf).to(cuda)
    layer.out_weight = (1 + 0.1 * torch.randn(128, generator=gen)).to(bf).to(cuda)
    layer.A_log, layer.dt_bias = (0.2 * torch.randn(4, generator=gen)).to(cuda), (0.2 * torch.randn(4, generator=gen)).to(cuda)
    layer.wo.weight = (0.05 * torch.randn(hid, 512, generator=gen)).to(bf).to(cuda)
    for op, (n_in, n_out) in ((layer.in_proj, (hid, 2056)), (layer.wo, (512, hid))):
        op._accent = ((0.1 * torch.randn(K, n_in, generator=gen)).to(bf).to(cuda),
                      (0.1 * torch.randn(K, n_out, generator=gen)).to(bf).to(cuda))
    mask = torch.zeros(n, K)
    mask[:70, :16] = 0.8
    mask[71:, 16:] = 1.3  # the one-row request has no accent
    mask = mask.to(bf).to(cuda)
    x = torch.randn(n, hid, generator=gen).to(bf).to(cuda)
    cu, chunks = serving.chunk_tables(rows, cuda)
    conv = torch.zeros(3, 1536, 4, dtype=bf, device=cuda)
    rec = torch.zeros(3, 4, 128, 128, device=cuda)

    class TorchHooks:
        def apply_accent(self, op, xx, yy, m):
            down, up = op._accent
            return yy + ((xx @ down.T) * m) @ up

    layer._accent = accent.AccentHooks(lambda: mask)
    native = layer._run_packed(x, cu, chunks, conv, rec, mask=mask)
    layer._accent = TorchHooks()
    ref = layer._run_packed(x, cu, chunks, conv, rec, mask=mask)
    layer._accent = None
    plain = layer._run_packed(x, cu, chunks, conv, rec)
    torch.cuda.synchronize()
    scale = float(ref[0].float().abs().max())
    assert max_abs(native[0].cpu(), ref[0].cpu()) < 3e-2 * max(1.0, scale)
    assert rel_err(native[2].cpu(), ref[2].cpu()) < 2e-2
    assert torch.equal(native[0][70], plain[0][70])  # the request without an accent: no shift at all
    assert max_abs(native[0].cpu(), plain[0].cpu()) > 1e-3  # the others are shifted
