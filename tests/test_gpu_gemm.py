"""The layer's projection kernels: ``gemm_nt`` (zgdn_gemm_nt) against fp32 products, and the fused in_proj + conv
(zgdn_in_proj_conv) against the GEMM followed by the conv kernel (bit for bit) and against the oracle's conv
(lm.py:561-568).

Tolerances: a bf16 GEMM output within one bf16 rounding of the fp32 product (max |y - ref| / max |ref| < 4e-3, and
at least 99 % of the elements equal to the product rounded to bf16; the rest differ by the summation order); the
fused projection bit-identical to its two-kernel composition; against the oracle (CPU bf16 F.linear + F.conv1d)
2e-2 max-abs.
"""

from __future__ import annotations

import pytest
import torch

from gdn_testing import announce, max_abs
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _operands(M, N, K, seed, cuda, x_extra=0):
    gen = torch.Generator().manual_seed(seed)
    xw = torch.randn(M, K + x_extra, generator=gen).to(torch.bfloat16).to(cuda)
    w = (0.03 * torch.randn(N, K, generator=gen)).to(torch.bfloat16).to(cuda)
    return xw[:, :K], w


@pytest.mark.parametrize("M,N,K", [(4096, 2056, 1024), (4096, 1024, 512), (1000, 2056, 1024), (1, 2056, 1024),
                                   (37, 1024, 512), (300, 264, 256), (513, 128, 128)])
def test_gemm_nt_against_fp32_products(gdn, cuda, M, N, K):
    announce(f"gemm_nt M={M} N={N} K={K}")
    x, w = _operands(M, N, K, 5000 + M + N, cuda, x_extra=24)  # x: a column slice of wider rows
    y = gdn.ops.gemm_nt(x, w)
    torch.cuda.synchronize()
    ref = x.float() @ w.float().T
    err = float((y.float() - ref).abs().max() / ref.abs().max())
    exact = float((y == ref.to(torch.bfloat16)).float().mean())
    assert err < 4e-3 and exact > 0.99, (err, exact)


def _conv_two_kernels(gdn, x, w, conv_w, C, hist):
    proj = gdn.ops.gemm_nt(x, w)
    h0 = None if hist is None else hist.unsqueeze(0)
    conv, fin = gdn.ops.causal_conv1d(proj[:, :C].unsqueeze(0), conv_w, initial_state=h0, activation="silu",
                                      state_width=3)
    return proj, conv[0], fin[0]


@pytest.mark.parametrize("M", [1, 2, 3, 100, 256, 257, 1000, 4096])
@pytest.mark.parametrize("history", [False, True])
def test_in_proj_conv_equals_gemm_then_conv(gdn, cuda, M, history):
    """The fused kernel computes the same projection (the conv tiles' halo rows included) and the same conv as
    the two kernels: every output bit and the new history equal."""
    announce(f"in_proj_conv M={M} history={history}")
    N, K, C = 2056, 1024, 1536
    x, w = _operands(M, N, K, 5100 + M, cuda)
    gen = torch.Generator().manual_seed(5200 + M)
    conv_w = (0.2 * torch.randn(C, 4, generator=gen)).to(torch.bfloat16).to(cuda)
    hist = (0.5 * torch.randn(C, 3, generator=gen)).to(torch.bfloat16).to(cuda) if history else None
    y, fin = gdn.ops.in_proj_conv(x, w, conv_w, C, initial_state=hist)
    proj, conv, fin2 = _conv_two_kernels(gdn, x, w, conv_w, C, hist)
    torch.cuda.synchronize()
    assert torch.equal(y[:, :C], conv)
    assert torch.equal(y[:, C:], proj[:, C:])
    assert torch.equal(fin, fin2)


def test_in_proj_conv_against_the_oracle(gdn, cuda):
    """The release shapes (hidden 1024, 4 heads x 128: in_proj [2056, 1024], conv [1536, 1, 4]) on a 300-row
    prompt with a history, against the oracle's bf16 F.linear + conv + SiLU on the CPU."""
    announce("in_proj_conv vs oracle, 300 rows")
    M, N, K, C = 300, 2056, 1024, 1536
    x, w = _operands(M, N, K, 5301, cuda)
    gen = torch.Generator().manual_seed(5302)
    conv_w = (0.2 * torch.randn(C, 1, 4, generator=gen)).to(torch.bfloat16)
    hist = (0.5 * torch.randn(C, 3, generator=gen)).to(torch.bfloat16)
    y, fin = gdn.ops.in_proj_conv(x, w, conv_w.to(cuda), C, initial_state=hist.to(cuda))
    torch.cuda.synchronize()
    proj = torch.nn.functional.linear(x.cpu(), w.cpu())
    conv_ref, fin_ref = O.causal_conv1d(proj[:, :C], conv_w, hist)
    assert max_abs(y[:, :C].cpu(), conv_ref) < 2e-2
    assert max_abs(y[:, C:].cpu(), proj[:, C:]) < 2e-2
    assert max_abs(fin.cpu(), fin_ref) < 2e-2


def test_in_proj_conv_rows_of_a_short_prompt_keep_the_old_history(gdn, cuda):
    """Fewer rows than the conv width: the new history is the old one shifted by the rows (taken from the two
    kernels' result, which the conv kernel's own tests pin), and no rows pass the history through."""
    announce("in_proj_conv short prompts")
    N, K, C = 2056, 1024, 1536
    gen = torch.Generator().manual_seed(5401)
    conv_w = (0.2 * torch.randn(C, 4, generator=gen)).to(torch.bfloat16).to(cuda)
    hist = (0.5 * torch.randn(C, 3, generator=gen)).to(torch.bfloat16).to(cuda)
    x, w = _operands(2, N, K, 5402, cuda)
    y, fin = gdn.ops.in_proj_conv(x, w, conv_w, C, initial_state=hist)
    proj = gdn.ops.gemm_nt(x, w)
    torch.cuda.synchronize()
    assert torch.equal(fin[:, 0], hist[:, 2]) and torch.equal(fin[:, 1:], proj[:, :C].T)
    y0, fin0 = gdn.ops.in_proj_conv(x[:0], w, conv_w, C, initial_state=hist)
    y1, fin1 = gdn.ops.in_proj_conv(x[:0], w, conv_w, C)
    torch.cuda.synchronize()
    assert y0.shape == (0, N) and torch.equal(fin0, hist) and torch.equal(fin1, torch.zeros_like(hist))
