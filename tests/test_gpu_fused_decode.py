"""Fused streaming-decode block (zgdn_fused_decode_step) against the CPU oracle, carrying conv cache and
state across consecutive steps. Tolerances: bf16 outputs 2e-2 max-abs, float32 states 1e-3 relative
(fp32 inputs: 1e-4 relative for both); the rolling conv cache is exact (a copy of raw inputs)."""

from __future__ import annotations

import pytest
import torch

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(B, hk, hv, steps, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    K = 128
    C = 2 * hk * K + hv * K
    return {
        "x": torch.randn(steps, B, C, generator=g).to(dtype),
        "z": torch.randn(steps, B, hv, K, generator=g).to(dtype),
        "a": torch.randn(steps, B, hv, generator=g).to(dtype),
        "b": torch.randn(steps, B, hv, generator=g).to(dtype),
        "w": (0.2 * torch.randn(C, 4, generator=g)).to(dtype),
        "nw": (1 + 0.1 * torch.randn(K, generator=g)).to(dtype),
        "A_log": 0.3 * torch.randn(hv, generator=g),
        "dt_bias": 0.3 * torch.randn(hv, generator=g),
        "cache": (0.5 * torch.randn(B, C, 3, generator=g)).to(dtype),
        "s0": 0.02 * torch.randn(B, hv, K, K, generator=g),
    }


def _run_case(gdn, cuda, B, hk, hv, steps, seed, dtype, round_qk=False):
    d = _inputs(B, hk, hv, steps, seed, dtype)
    dev = {k: v.to(cuda) for k, v in d.items()}
    cache, state = dev["cache"].clone(), dev["s0"].clone()
    c_ref, s_ref = d["cache"].clone(), d["s0"].clone()
    bf16 = dtype == torch.bfloat16
    for t in range(steps):
        out = gdn.fused_decode_step(dev["x"][t], dev["z"][t], dev["a"][t], dev["b"][t], dev["w"], cache, state,
                                    dev["nw"], dev["A_log"], dev["dt_bias"], eps=1e-6, round_qk=round_qk)
        torch.cuda.synchronize()
        o_ref, c_ref, s_ref = O.fused_decode_step(d["x"][t], d["z"][t], d["a"][t], d["b"][t], d["w"], c_ref, s_ref,
                                                  d["nw"], d["A_log"], d["dt_bias"], hk, eps=1e-6, round_qk=round_qk)
        assert torch.equal(cache.cpu(), c_ref), f"conv cache differs at step {t}"
        if bf16:
            assert max_abs(out.cpu(), o_ref) < 2e-2, (t, max_abs(out.cpu(), o_ref))
            assert rel_err(state.cpu(), s_ref) < 1e-3, (t, rel_err(state.cpu(), s_ref))
        else:
            assert rel_err(out.cpu(), o_ref) < 1e-4, (t, rel_err(out.cpu(), o_ref))
            assert rel_err(state.cpu(), s_ref) < 1e-4, (t, rel_err(state.cpu(), s_ref))


def test_streaming_block_B256_Hk8_Hv16(gdn, cuda):
    """The streaming-decode workload's shape: B=256 streams, 8 q/k heads shared by 16 v heads, bf16."""
    announce("fused decode B=256 Hk=8 Hv=16 bf16 x3 steps")
    _run_case(gdn, cuda, 256, 8, 16, 3, seed=5001, dtype=torch.bfloat16)


@pytest.mark.parametrize("hk,hv", [(1, 1), (2, 4), (1, 4)])
def test_group_sizes_bf16(gdn, cuda, hk, hv):
    announce(f"fused decode B=5 Hk={hk} Hv={hv} bf16 x4 steps")
    _run_case(gdn, cuda, 5, hk, hv, 4, seed=5100 + hv, dtype=torch.bfloat16)


def test_rounded_qk_like_the_serving_operators(gdn, cuda):
    """round_qk: the normalised q, k rounded to bf16 (the serving layer's l2norm operator output); the
    serving layer's head shape (4 q/k heads, 4 v heads). The rounding changes the state (so it is applied)."""
    announce("fused decode B=6 Hk=Hv=4 bf16 x4 steps, q/k rounded")
    _run_case(gdn, cuda, 6, 4, 4, 4, seed=5300, dtype=torch.bfloat16, round_qk=True)
    d = _inputs(2, 4, 4, 1, 5301, torch.bfloat16)
    dev = {k: v.to(cuda) for k, v in d.items()}
    states = []
    for r in (False, True):
        cache, state = dev["cache"].clone(), dev["s0"].clone()
        gdn.fused_decode_step(dev["x"][0], dev["z"][0], dev["a"][0], dev["b"][0], dev["w"], cache, state,
                              dev["nw"], dev["A_log"], dev["dt_bias"], round_qk=r)
        states.append(state)
    torch.cuda.synchronize()
    assert not torch.equal(states[0], states[1])


def test_float32_block(gdn, cuda):
    announce("fused decode B=4 Hk=2 Hv=4 fp32 x4 steps")
    _run_case(gdn, cuda, 4, 2, 4, 4, seed=5200, dtype=torch.float32)
