"""Chunked prefill in fp32 arithmetic (zgdn_chunk_fwd with fp32 q/k/v, or 64-wide heads) against the oracle.

Tolerances: fp32 inputs, outputs and final states within 1e-4 relative (max|err| / max|ref|) of the fp32 token
loop of lm.py:574-583 (``O.gated_delta_recurrence``); bf16 inputs (64-wide heads), outputs within 2e-2 max-abs
and float32 states within 1e-3 relative.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4


def _check_f32(o, s, o_ref, s_ref):
    eo, es = rel_err(o, o_ref), rel_err(s, s_ref)
    assert eo < F32_TOL and es < F32_TOL, (eo, es)
    return eo, es


def _run(gdn, d, cuda, **kw):
    x = {n: d[n].to(cuda) for n in ("q", "k", "v", "g", "beta")}
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], **kw)
    torch.cuda.synchronize()
    return o, s


def test_config1_fp32_d64(gdn, cuda):
    """The CPU-oracle configuration: B=1, T=256, H=4, dk=dv=64, fp32, zero initial state."""
    announce("chunk f32 config 1: T=256 H=4 d=64")
    d = O.make_inputs(1, 256, 4, 4, 64, 64, seed=1001)
    o, s = _run(gdn, d, cuda)
    assert o.dtype == torch.float32 and o.shape == (1, 256, 4, 64) and s.shape == (1, 4, 64, 64)
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"])
    _check_f32(o.cpu(), s.cpu(), o_ref, s_ref)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 64, 2), (2, 65, 3), (1, 200, 2), (2, 130, 4)])
def test_fp32_shapes_with_initial_state(gdn, cuda, D, B, T, H):
    announce(f"chunk f32 D={D} B={B} T={T} H={H}")
    d = O.make_inputs(B, T, H, H, D, D, seed=3000 + 7 * T + H + D, state_std=0.02)
    o, s = _run(gdn, d, cuda, initial_state=d["s0"].to(cuda))
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"])
    _check_f32(o.cpu(), s.cpu(), o_ref, s_ref)


def test_fp32_prefill_T4096_H16_d128(gdn, cuda):
    """The prefill workload's shape in fp32: B=1, T=4096, H=16, dk=dv=128, zero initial state."""
    announce("chunk f32 T=4096 H=16 d=128")
    d = O.make_inputs(1, 4096, 16, 16, 128, 128, seed=1003)
    o, s = _run(gdn, d, cuda)
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"])
    eo, es = _check_f32(o.cpu(), s.cpu(), o_ref, s_ref)
    print(f"fp32 T=4096 H=16: output rel err {eo:.2e}, state rel err {es:.2e}")


@pytest.mark.parametrize("D", [64, 128])
def test_fp32_packed_sequences(gdn, cuda, D):
    lengths = [64, 1, 130, 0, 70, 200, 63, 65]
    cu, _ = O.chunk_tables(lengths)
    announce(f"chunk f32 varlen D={D} lengths={lengths}")
    d = O.make_inputs(1, sum(lengths), 2, 4, D, D, seed=3101 + D, state_std=0.02, n_states=len(lengths))
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    o, s = _run(gdn, d, cuda, initial_state=d["s0"].to(cuda), cu_seqlens=cu_t)
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"], cu_seqlens=cu)
    _check_f32(o.cpu(), s.cpu(), o_ref, s_ref)
    assert torch.equal(s[3].cpu(), d["s0"][3])  # the empty sequence keeps its state


@pytest.mark.parametrize("D", [64, 128])
def test_fp32_gate_in_kernel_l2norm_beta_logits_rows_in_place(gdn, cuda, D):
    """Grouped heads (Hk=2 -> Hv=4), q/k/v as column slices of one wider fp32 row, raw a with A_log / dt_bias,
    beta as logits, q/k L2-normalised in the kernel: against the oracle given the normalised rows, the decay
    exp(-exp(A_log) softplus(a + dt_bias)) and sigmoid(b) (lm.py:569-573)."""
    announce(f"chunk f32 D={D} gate + l2norm + logits + strided rows")
    gen = torch.Generator().manual_seed(3201 + D)
    B, T, Hk, Hv = 2, 150, 2, 4
    width = (2 * Hk + Hv) * D
    conv = torch.randn(B, T, width + 12, generator=gen)  # 12 extra columns: a row stride of width + 12
    proj = torch.randn(B, T, 24, generator=gen)
    q = conv[..., : Hk * D].unflatten(-1, (Hk, D))
    k = conv[..., Hk * D: 2 * Hk * D].unflatten(-1, (Hk, D))
    v = conv[..., 2 * Hk * D: width].unflatten(-1, (Hv, D))
    a, b = proj[..., 3: 3 + Hv], proj[..., 12: 12 + Hv]
    A_log, dt_bias = 0.3 * torch.randn(Hv, generator=gen), 0.3 * torch.randn(Hv, generator=gen)
    s0 = 0.02 * torch.randn(B, Hv, D, D, generator=gen)
    conv_d, proj_d = conv.to(cuda), proj.to(cuda)
    qd = conv_d[..., : Hk * D].unflatten(-1, (Hk, D))
    kd = conv_d[..., Hk * D: 2 * Hk * D].unflatten(-1, (Hk, D))
    vd = conv_d[..., 2 * Hk * D: width].unflatten(-1, (Hv, D))
    ad, bd = proj_d[..., 3: 3 + Hv], proj_d[..., 12: 12 + Hv]
    o, s = gdn.chunk_fwd(qd, kd, vd, ad, bd, initial_state=s0.to(cuda), A_log=A_log.to(cuda),
                         dt_bias=dt_bias.to(cuda), use_qk_l2norm=True, beta_is_logit=True)
    torch.cuda.synchronize()
    g_log = -A_log.exp() * F.softplus(a + dt_bias)
    o_ref, s_ref = O.gated_delta_recurrence(O.l2norm(q), O.l2norm(k), v.contiguous(), g_log, torch.sigmoid(b),
                                            None, s0)
    _check_f32(o.cpu(), s.cpu(), o_ref, s_ref)


@pytest.mark.parametrize("B,T,H", [(1, 64, 2), (2, 200, 3), (1, 1, 1)])
def test_bf16_d64(gdn, cuda, B, T, H):
    """bf16 inputs at 64-wide heads run in fp32 arithmetic; bf16 tolerances."""
    announce(f"chunk bf16 d=64 B={B} T={T} H={H}")
    d = O.make_inputs(B, T, H, H, 64, 64, seed=3300 + T + H, dtype=torch.bfloat16, state_std=0.02)
    o, s = _run(gdn, d, cuda, initial_state=d["s0"].to(cuda))
    assert o.dtype == torch.bfloat16
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"])
    eo, es = max_abs(o.cpu(), o_ref), rel_err(s.cpu(), s_ref)
    assert eo < 2e-2 and es < 1e-3, (eo, es)


def test_fp32_bit_identical_repeats_and_in_place(gdn, cuda):
    """Two calls give the same bits (fixed summation order); the state may be updated in place."""
    announce("chunk f32 repeat + in place")
    d = O.make_inputs(1, 777, 4, 8, 128, 128, seed=3401, state_std=0.02)
    o1, s1 = _run(gdn, d, cuda, initial_state=d["s0"].to(cuda))
    state = d["s0"].to(cuda)
    o2, s2 = _run(gdn, d, cuda, initial_state=state, final_state=state)
    assert s2 is state
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_fp32_chunked_agrees_with_recurrent_kernel(gdn, cuda):
    """The chunked and the token-loop HIP paths agree in fp32 on a long prompt with grouped heads."""
    announce("chunk f32 vs recurrent T=2000 Hk=4 Hv=8")
    d = O.make_inputs(1, 2000, 4, 8, 128, 128, seed=3501, state_std=0.02)
    x = {n: d[n].to(cuda) for n in ("q", "k", "v", "g", "beta", "s0")}
    o_c, s_c = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"])
    o_r, s_r = gdn.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], None, x["s0"])
    torch.cuda.synchronize()
    _check_f32(o_c.cpu(), s_c.cpu(), o_r.cpu(), s_r.cpu())
