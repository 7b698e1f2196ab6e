"""Recurrent / decode kernel (zgdn_recurrent_fwd) against the CPU oracle on seeded inputs.

Tolerances: float32 inputs -> outputs and final states within 1e-4 relative; bfloat16 inputs -> outputs
within 2e-2 max-abs and float32 states within 1e-3 relative (relative = max|err| / max|ref|).
"""

from __future__ import annotations

import pytest
import torch

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _run(gdn, cuda, d, scale=None, cu=None, gb_dtype=torch.float32, inplace=False):
    q, k, v = (d[n].to(cuda) for n in ("q", "k", "v"))
    g, b = d["g"].to(cuda, gb_dtype), d["beta"].to(cuda, gb_dtype)
    s0 = d["s0"].to(cuda)
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=cuda)
    if inplace:
        o, s = gdn.recurrent_fwd(q, k, v, g, b, scale, s0, cu_seqlens=cu_t, final_state=s0)
        assert s is s0
    else:
        o, s = gdn.recurrent_fwd(q, k, v, g, b, scale, s0, cu_seqlens=cu_t)
    torch.cuda.synchronize()
    return o.cpu(), s.cpu()


def _oracle(d, scale=None, cu=None, gb_dtype=torch.float32):
    g = d["g"].to(gb_dtype).float()
    b = d["beta"].to(gb_dtype).float()
    return O.gated_delta_recurrence(d["q"], d["k"], d["v"], g, b, scale, d["s0"], cu_seqlens=cu)


def _check(o, s, o_ref, s_ref, bf16):
    if bf16:
        assert max_abs(o, o_ref) < 2e-2, max_abs(o, o_ref)
        assert rel_err(s, s_ref) < 1e-3, rel_err(s, s_ref)
    else:
        assert rel_err(o, o_ref) < 1e-4, rel_err(o, o_ref)
        assert rel_err(s, s_ref) < 1e-4, rel_err(s, s_ref)


def test_fp32_sequence_B1_T256_H4_d64(gdn, cuda):
    """Single-layer op on the reference's CPU-runnable shape: B=1, T=256, H=4, dk=dv=64, fp32, zero state."""
    announce("recurrent fp32 B=1 T=256 H=4 d=64")
    d = O.make_inputs(1, 256, 4, 4, 64, 64, seed=1001)
    o, s = _run(gdn, cuda, d)
    o_ref, s_ref = _oracle(d)
    _check(o, s, o_ref, s_ref, bf16=False)


def test_bf16_decode_B64_H16_d128(gdn, cuda):
    """Single-token decode batch: B=64 streams, H=16, dk=dv=128, bf16 q/k/v, state ~N(0, 0.02)."""
    announce("decode bf16 B=64 H=16 d=128")
    d = O.make_inputs(64, 1, 16, 16, 128, 128, seed=1002, dtype=torch.bfloat16, state_std=0.02)
    o, s = _run(gdn, cuda, d)
    o_ref, s_ref = _oracle(d)
    _check(o, s, o_ref, s_ref, bf16=True)
    assert rel_err(s, s_ref) < 1e-5  # the state update itself is exact float32 arithmetic


def test_decode_step_in_place_chain_equals_recurrence(gdn, cuda):
    announce("decode_step chain bf16 B=8 H=4 d=128 x6")
    d = O.make_inputs(8, 6, 4, 4, 128, 128, seed=1003, dtype=torch.bfloat16, state_std=0.02)
    state = d["s0"].to(cuda)
    outs = []
    for t in range(6):
        outs.append(gdn.decode_step(d["q"][:, t].to(cuda), d["k"][:, t].to(cuda), d["v"][:, t].to(cuda),
                                    d["g"][:, t].to(cuda), d["beta"][:, t].to(cuda), state).cpu())
    o_ref, s_ref = _oracle(d)
    _check(torch.stack(outs, 1), state.cpu(), o_ref, s_ref, bf16=True)


@pytest.mark.parametrize("hk,hv", [(1, 2), (2, 4), (8, 16)])
def test_grouped_value_heads(gdn, cuda, hk, hv):
    announce(f"recurrent grouped heads Hk={hk} Hv={hv}")
    d = O.make_inputs(3, 20, hk, hv, 128, 128, seed=1004 + hv, dtype=torch.bfloat16, state_std=0.02)
    o, s = _run(gdn, cuda, d)
    o_ref, s_ref = _oracle(d)
    _check(o, s, o_ref, s_ref, bf16=True)


def test_packed_sequences_with_an_empty_one(gdn, cuda):
    lengths = [5, 64, 0, 1, 70]
    cu, _ = O.chunk_tables(lengths)
    announce(f"recurrent varlen lengths={lengths}")
    d = O.make_inputs(1, sum(lengths), 2, 2, 128, 128, seed=1005, dtype=torch.bfloat16, state_std=0.02,
                      n_states=len(lengths))
    o, s = _run(gdn, cuda, d, cu=cu)
    o_ref, s_ref = _oracle(d, cu=cu)
    _check(o, s, o_ref, s_ref, bf16=True)
    assert torch.equal(s[2], d["s0"][2])  # an empty sequence passes its state through unchanged


def test_bf16_gates_and_in_place_state(gdn, cuda):
    announce("recurrent bf16 g/beta, in-place state")
    d = O.make_inputs(2, 33, 2, 2, 64, 64, seed=1006, dtype=torch.bfloat16, state_std=0.02)
    o, s = _run(gdn, cuda, d, gb_dtype=torch.bfloat16, inplace=True)
    o_ref, s_ref = _oracle(d, gb_dtype=torch.bfloat16)
    _check(o, s, o_ref, s_ref, bf16=True)


def test_ragged_value_rows_and_custom_scale(gdn, cuda):
    """V = 40 is not a multiple of the rows a workgroup owns: the tail rows are masked."""
    announce("recurrent fp32 K=64 V=40 scale=0.3")
    d = O.make_inputs(2, 17, 1, 1, 64, 40, seed=1007, state_std=0.1)
    o, s = _run(gdn, cuda, d, scale=0.3)
    o_ref, s_ref = _oracle(d, scale=0.3)
    _check(o, s, o_ref, s_ref, bf16=False)


def test_no_final_state_and_no_initial_state(gdn, cuda):
    announce("recurrent without states")
    d = O.make_inputs(2, 9, 2, 2, 128, 128, seed=1008)
    q, k, v, g, b = (d[n].to(cuda) for n in ("q", "k", "v", "g", "beta"))
    o, s = gdn.recurrent_fwd(q, k, v, g, b, output_final_state=False)
    assert s is None
    o_ref, _ = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"])
    assert rel_err(o.cpu(), o_ref) < 1e-4


@pytest.mark.parametrize("case", ["fp32_k64_v40", "bf16_gva_bf16_gates", "gate_l2norm", "no_states", "b256",
                                  "k64_tiled", "fp32_tiled"])
def test_single_token_step(gdn, cuda, case):
    """T = 1 without cu_seqlens runs the persistent single-token kernel: every input variant it takes (the
    general form), small batches (one row group per item), and batches that take the tiled form (four row
    groups sharing one q/k load), including one where each wave walks many tiles (B=256, H=16)."""
    announce(f"single-token step {case}")
    B, hk, hv, K, V, dtype, gb = 5, 2, 2, 128, 128, torch.bfloat16, torch.float32
    if case == "fp32_k64_v40":
        B, hk, hv, K, V, dtype = 3, 1, 1, 64, 40, torch.float32
    elif case == "bf16_gva_bf16_gates":
        B, hk, hv, gb = 7, 2, 8, torch.bfloat16
    elif case == "b256":
        B, hk, hv = 256, 16, 16
    elif case == "k64_tiled":
        B, hk, hv, K, V = 128, 8, 16, 64, 64
    elif case == "fp32_tiled":
        B, hk, hv, dtype = 64, 16, 16, torch.float32
    d = O.make_inputs(B, 1, hk, hv, K, V, seed=1010, dtype=dtype, state_std=0.02)
    if case == "gate_l2norm":
        gen = torch.Generator().manual_seed(1011)
        q = (2 * torch.randn(B, 1, hk, K, generator=gen)).to(dtype)
        k = (2 * torch.randn(B, 1, hk, K, generator=gen)).to(dtype)
        a = torch.randn(B, 1, hv, generator=gen)
        A_log, dt_bias = 0.3 * torch.randn(hv, generator=gen), 0.3 * torch.randn(hv, generator=gen)
        o, s = gdn.recurrent_fwd(q.to(cuda), k.to(cuda), d["v"].to(cuda), a.to(cuda), d["beta"].to(cuda),
                                 initial_state=d["s0"].to(cuda), A_log=A_log.to(cuda), dt_bias=dt_bias.to(cuda),
                                 use_qk_l2norm=True)
        torch.cuda.synchronize()
        g_log = -A_log.exp() * torch.nn.functional.softplus(a + dt_bias)
        o_ref, s_ref = O.gated_delta_recurrence(O.l2norm(q), O.l2norm(k), d["v"], g_log, d["beta"], None, d["s0"])
        o, s = o.cpu(), s.cpu()
    elif case == "no_states":
        q, k, v, g, b = (d[n].to(cuda) for n in ("q", "k", "v", "g", "beta"))
        o, s = gdn.recurrent_fwd(q, k, v, g, b, output_final_state=False)
        torch.cuda.synchronize()
        assert s is None
        o_ref, _ = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"])
        assert max_abs(o.cpu(), o_ref) < 2e-2
        return
    else:
        o, s = _run(gdn, cuda, d, gb_dtype=gb, inplace=case == "b256")
        o_ref, s_ref = _oracle(d, gb_dtype=gb)
    _check(o, s, o_ref, s_ref, bf16=dtype == torch.bfloat16)
    assert rel_err(s, s_ref) < 1e-5  # the state update is plain fp32 arithmetic


def test_single_token_step_matches_token_loop_kernel(gdn, cuda):
    """The same single-token batch through the persistent step kernel (B streams, T=1) and through the
    token-loop kernel (packed as B one-token sequences): the same fp32 arithmetic, so equal to rounding."""
    announce("single-token step vs token-loop kernel B=64 H=16")
    d = O.make_inputs(64, 1, 8, 16, 128, 128, seed=1012, dtype=torch.bfloat16, state_std=0.02)
    o1, s1 = _run(gdn, cuda, d)
    d1 = {n: d[n] if n == "s0" else d[n].reshape(1, 64, *d[n].shape[2:]) for n in d}
    o2, s2 = _run(gdn, cuda, d1, cu=list(range(65)))
    assert rel_err(s1, s2) < 1e-6
    assert rel_err(o1.reshape(o2.shape).float(), o2.float()) < 4e-3  # at most one bf16 rounding step apart
