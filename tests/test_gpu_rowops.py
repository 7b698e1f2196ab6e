"""Row-local kernels (conv1d, L2-norm, sigmoid, gated RMSNorm) and the fused q/k L2-norm / in-kernel gate
options of the recurrent and chunked kernels, against the CPU oracle."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("state_width", [3, 4])
def test_conv_packed_sequences_and_history(gdn, cuda, dtype, state_width):
    lengths = [1, 2, 70, 0, 130, 64]
    cu, _ = O.chunk_tables(lengths)
    announce(f"conv varlen {lengths} sw={state_width} {dtype}")
    gen = torch.Generator().manual_seed(3001)
    D = 200
    x = torch.randn(1, sum(lengths), D, generator=gen).to(dtype)
    w = (0.3 * torch.randn(D, 4, generator=gen)).to(dtype)
    s0 = torch.randn(len(lengths), D, state_width, generator=gen).to(dtype)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    state = s0.to(cuda)
    y, fin = gdn.ops.causal_conv1d(x.to(cuda), w.to(cuda), initial_state=state, final_state=state,
                                   activation="silu", cu_seqlens=cu_t, state_width=state_width)
    torch.cuda.synchronize()
    for i in range(len(lengths)):
        lo, hi = cu[i], cu[i + 1]
        full = torch.cat((s0[i], x[0, lo:hi].T), -1)
        assert torch.equal(fin[i].cpu(), full[:, -state_width:]), i  # in place, exact copy of raw inputs
        if hi > lo:
            y_ref, hist = O.causal_conv1d(x[0, lo:hi], w, s0[i][:, state_width - 3:])
            tol = 1e-5 if dtype == torch.float32 else 1e-2
            assert max_abs(y[0, lo:hi].cpu(), y_ref) <= tol * max(1.0, float(y_ref.abs().max())), i
            assert torch.equal(hist, fin[i].cpu()[:, state_width - 3:])


def test_conv_batched_no_state(gdn, cuda):
    announce("conv batched B=3 T=100 no state")
    gen = torch.Generator().manual_seed(3002)
    x = torch.randn(3, 100, 64, generator=gen)
    w = torch.randn(64, 4, generator=gen)
    y, fin = gdn.ops.causal_conv1d(x.to(cuda), w.to(cuda), activation=None, state_width=3)
    for b in range(3):
        ref = F.conv1d(torch.cat((torch.zeros(64, 3), x[b].T), -1)[None], w[:, None, :], groups=64)[0].T
        assert max_abs(y[b].cpu(), ref) < 1e-4
        assert torch.equal(fin[b].cpu(), x[b, -3:].T)


def test_l2norm_sigmoid_gated_norm(gdn, cuda):
    announce("l2norm / sigmoid / gated rmsnorm")
    gen = torch.Generator().manual_seed(3003)
    x = 3 * torch.randn(37, 4, 128, generator=gen)
    y, rstd = gdn.ops.l2norm(x.to(cuda), out_dtype=torch.float32)
    assert rel_err(y.cpu(), O.l2norm(x)) < 1e-6
    assert rel_err(rstd.cpu(), torch.rsqrt(x.square().sum(-1) + 1e-6)) < 1e-6
    yb, _ = gdn.ops.l2norm(x.to(torch.bfloat16).to(cuda))
    assert yb.dtype == torch.bfloat16 and max_abs(yb.cpu(), O.l2norm(x.to(torch.bfloat16))) < 4e-3
    b = torch.randn(1000, generator=gen)
    assert rel_err(gdn.ops.sigmoid(b.to(cuda), scale=0.5).cpu(), 0.5 * b.sigmoid()) < 1e-6
    for dt in (torch.float32, torch.bfloat16):
        o = torch.randn(50, 4, 128, generator=gen).to(dt)
        z = torch.randn(50, 4, 128, generator=gen).to(dt)
        nw = (1 + 0.1 * torch.randn(128, generator=gen)).to(dt)
        got, _ = gdn.ops.gated_rmsnorm(o.to(cuda), z.to(cuda), nw.to(cuda), eps=1e-5)
        want = O.gated_rmsnorm(o, z, nw, 1e-5, dt)
        assert max_abs(got.cpu(), want) < (1e-5 if dt == torch.float32 else 2e-2), dt


def _raw_qk(d, gen):
    """Raw (un-normalised) q, k rows as a layer's conv output would hand them over, bf16."""
    q = (torch.randn(d["q"].shape, generator=gen) * 0.7).to(torch.bfloat16)
    k = (torch.randn(d["k"].shape, generator=gen) * 0.7).to(torch.bfloat16)
    return q, k


@pytest.mark.parametrize("path", ["chunk", "recurrent"])
def test_fused_l2norm_and_gate(gdn, cuda, path):
    """use_qk_l2norm + A_log/dt_bias: the kernels normalise raw q, k in fp32 and form the decay themselves;
    compared with the oracle fed the fp32-normalised rows (lm.py:570-573), never rounded to bf16."""
    announce(f"fused l2norm + gate, {path}")
    gen = torch.Generator().manual_seed(3004)
    d = O.make_inputs(1, 300, 4, 4, 128, 128, seed=3005, dtype=torch.bfloat16, state_std=0.02)
    q, k = _raw_qk(d, gen)
    a = torch.randn(1, 300, 4, generator=gen)
    braw = torch.randn(1, 300, 4, generator=gen)
    A_log, dt_bias = 0.3 * torch.randn(4, generator=gen), 0.3 * torch.randn(4, generator=gen)
    beta = braw.sigmoid()
    dev = lambda t: t.to(cuda)  # noqa: E731
    kw = dict(initial_state=dev(d["s0"]), A_log=dev(A_log), dt_bias=dev(dt_bias), use_qk_l2norm=True)
    if path == "chunk":
        o, s = gdn.chunk_fwd(dev(q), dev(k), dev(d["v"]), dev(a), dev(beta), **kw)
    else:
        o, s = gdn.recurrent_fwd(dev(q), dev(k), dev(d["v"]), dev(a), dev(beta), **kw)
    torch.cuda.synchronize()
    g_log = -A_log.exp() * F.softplus(a + dt_bias)
    o_ref, s_ref = O.gated_delta_recurrence(O.l2norm(q), O.l2norm(k), d["v"], g_log, beta, None, d["s0"])
    assert max_abs(o.cpu(), o_ref) < 2e-2
    assert rel_err(s.cpu(), s_ref) < 1e-3, rel_err(s.cpu(), s_ref)
    if path == "recurrent":
        assert rel_err(s.cpu(), s_ref) < 1e-5  # the recurrent kernel is plain fp32 arithmetic


def test_rows_read_in_place(gdn, cuda):
    """The conv's input, the L2 norm's rows and the gated norm's gate as column slices of wider rows (the
    input projection, the conv output): bit-identical to the same values handed over dense. The conv input
    also at an odd element offset (no channel pairs) and as packed sequences with states."""
    announce("row kernels read slices in place")
    gen = torch.Generator().manual_seed(3101)
    T, D = 150, 96
    buf = torch.randn(1, T, 260, generator=gen).to(torch.bfloat16).to(cuda)
    w = (0.3 * torch.randn(D, 4, generator=gen)).to(torch.bfloat16).to(cuda)
    s0 = torch.randn(2, D, 4, generator=gen).to(torch.bfloat16).to(cuda)
    cu = torch.tensor([0, 70, T], dtype=torch.int32, device=cuda)
    for off in (0, 1):
        x = buf[..., off: off + D]
        for kw in (dict(state_width=3), dict(initial_state=s0, cu_seqlens=cu, state_width=4)):
            y1, f1 = gdn.ops.causal_conv1d(x, w, activation="silu", **kw)
            y2, f2 = gdn.ops.causal_conv1d(x.contiguous(), w, activation="silu", **kw)
            assert torch.equal(y1, y2) and torch.equal(f1, f2), (off, sorted(kw))
    rows = buf[0, :, :256].unflatten(-1, (2, 128))  # [T, 2, 128], token stride 260
    for dt in (torch.float32, torch.bfloat16):
        y1, r1 = gdn.ops.l2norm(rows, out_dtype=dt)
        y2, r2 = gdn.ops.l2norm(rows.contiguous(), out_dtype=dt)
        assert torch.equal(y1, y2) and torch.equal(r1, r2)
    o = torch.randn(T, 2, 128, generator=gen).to(torch.bfloat16).to(cuda)
    nw = (1 + 0.1 * torch.randn(128, generator=gen)).to(torch.bfloat16).to(cuda)
    g1, _ = gdn.ops.gated_rmsnorm(o, rows, nw, eps=1e-5)
    g2, _ = gdn.ops.gated_rmsnorm(o, rows.contiguous(), nw, eps=1e-5)
    torch.cuda.synchronize()
    assert torch.equal(g1, g2)


def test_gated_norm_many_rows(gdn, cuda):
    """Many rows (4101 tokens x 4 heads, 1026 workgroups with a ragged last one), the gate read in place from
    wider rows: within the bf16 tolerance of the oracle, rstd the row's 1/rms, and every row bit-identical to
    the same row normed in a small call."""
    announce("gated rmsnorm, many rows")
    gen = torch.Generator().manual_seed(3211)
    T = 4101
    o = torch.randn(T, 4, 128, generator=gen).to(torch.bfloat16).to(cuda)
    buf = torch.randn(T, 4 * 128 + 24, generator=gen).to(torch.bfloat16).to(cuda)
    z = buf[:, :512].unflatten(-1, (4, 128))
    nw = (1 + 0.1 * torch.randn(128, generator=gen)).to(torch.bfloat16).to(cuda)
    got, rstd = gdn.ops.gated_rmsnorm(o, z, nw, eps=1e-5)
    want = O.gated_rmsnorm(o.cpu(), z.cpu(), nw.cpu(), 1e-5, torch.bfloat16)
    assert max_abs(got.cpu(), want) < 2e-2
    assert rel_err(rstd.cpu(), torch.rsqrt(o.float().square().mean(-1) + 1e-5).cpu()) < 1e-5
    for sl in (slice(0, 20), slice(2000, 2013), slice(T - 21, T)):
        g2, r2 = gdn.ops.gated_rmsnorm(o[sl], z[sl], nw, eps=1e-5)
        torch.cuda.synchronize()
        assert torch.equal(got[sl], g2) and torch.equal(rstd[sl], r2), sl
