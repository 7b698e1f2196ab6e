"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): the CPU
oracle reproduces them (CPU), and the HIP kernels reproduce them to the path's tolerances (GPU)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / f"{name}.npz") as z:
        return {k: torch.from_numpy(z[k].copy()) for k in z.files}


def test_fixtures_present():
    names = {p.stem for p in GOLDEN.glob("*.npz")}
    assert {"recurrent_fp32_T40_H2_d64", "decode_bf16_B2_H1_d128", "chunk_varlen_bf16_H1to2_d128",
            "fused_block_B2_Hk1_Hv2", "conv_varlen_D16"} <= names


def test_oracle_reproduces_recurrence_fixtures():
    f = _load("recurrent_fp32_T40_H2_d64")
    o, s = O.gated_delta_recurrence(f["q"], f["k"], f["v"], f["g"], f["beta"], None, f["s0"])
    assert rel_err(o, f["o"]) < 1e-5 and rel_err(s, f["s"]) < 1e-5
    f = _load("chunk_varlen_bf16_H1to2_d128")
    o, s = O.gated_delta_recurrence(f["q"], f["k"], f["v"], f["g"], f["beta"], None, f["s0"],
                                    cu_seqlens=f["cu"].tolist())
    assert rel_err(o, f["o"]) < 1e-5 and rel_err(s, f["s"]) < 1e-5
    assert f["chunks"].tolist() == O.chunk_tables([70, 5, 0])[1]


def test_oracle_reproduces_conv_and_block_fixtures():
    f = _load("conv_varlen_D16")
    cu = f["cu"].tolist()
    for i in range(len(cu) - 1):
        y, hist = O.causal_conv1d(f["x"][0, cu[i]:cu[i + 1]], f["w"], f["s0"][i][:, 1:])
        assert max_abs(y, f["y"][0, cu[i]:cu[i + 1]]) < 1e-5
        assert torch.equal(hist, f["fin"][i][:, 1:])
    f = _load("fused_block_B2_Hk1_Hv2")
    bf = torch.bfloat16
    cache, state = f["cache0"].to(bf), f["s0"]
    for t in range(2):
        out, cache, state = O.fused_decode_step(f["x"][t].to(bf), f["z"][t].to(bf), f["a"][t].to(bf),
                                                f["b"][t].to(bf), f["w"].to(bf), cache, state, f["nw"].to(bf),
                                                f["A_log"], f["dt_bias"], 1, eps=1e-6)
        assert torch.equal(out.float(), f["out"][t])
    assert torch.equal(cache.float(), f["cache"]) and rel_err(state, f["s"]) < 1e-6


@pytest.mark.gpu
def test_kernels_reproduce_fixtures(gdn, cuda):
    announce("golden fixtures on the kernels")
    bf = torch.bfloat16
    f = _load("recurrent_fp32_T40_H2_d64")
    d = {k: v.to(cuda) for k, v in f.items()}
    o, s = gdn.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"])
    assert rel_err(o.cpu(), f["o"]) < 1e-4 and rel_err(s.cpu(), f["s"]) < 1e-4
    f = _load("decode_bf16_B2_H1_d128")
    d = {k: v.to(cuda) for k, v in f.items()}
    state = d["s0"].clone()
    o = gdn.decode_step(d["q"][:, 0].to(bf), d["k"][:, 0].to(bf), d["v"][:, 0].to(bf), d["g"][:, 0], d["beta"][:, 0],
                        state)
    assert max_abs(o.cpu(), f["o"][:, 0]) < 2e-2 and rel_err(state.cpu(), f["s"]) < 1e-3
    f = _load("chunk_varlen_bf16_H1to2_d128")
    d = {k: v.to(cuda) for k, v in f.items()}
    o, s = gdn.chunk_fwd(d["q"].to(bf), d["k"].to(bf), d["v"].to(bf), d["g"], d["beta"], initial_state=d["s0"],
                         cu_seqlens=d["cu"], chunk_indices=d["chunks"])
    assert max_abs(o.cpu(), f["o"]) < 2e-2 and rel_err(s.cpu(), f["s"]) < 1e-3
    f = _load("conv_varlen_D16")
    d = {k: v.to(cuda) for k, v in f.items()}
    st = d["s0"].clone()
    y, fin = gdn.ops.causal_conv1d(d["x"], d["w"], initial_state=st, final_state=st, activation="silu",
                                   cu_seqlens=d["cu"], state_width=4)
    assert max_abs(y.cpu(), f["y"]) < 1e-5 and torch.equal(fin.cpu(), f["fin"])
    f = _load("fused_block_B2_Hk1_Hv2")
    d = {k: (v.to(cuda) if k in ("A_log", "dt_bias", "s0") else v.to(cuda, bf)) for k, v in f.items()}
    cache, state = d["cache0"].clone(), d["s0"].clone()
    for t in range(2):
        out = gdn.fused_decode_step(d["x"][t], d["z"][t], d["a"][t], d["b"][t], d["w"], cache, state, d["nw"],
                                    d["A_log"], d["dt_bias"], eps=1e-6)
        assert max_abs(out.cpu(), f["out"][t]) < 2e-2
    assert torch.equal(cache.float().cpu(), f["cache"]) and rel_err(state.cpu(), f["s"]) < 1e-3
