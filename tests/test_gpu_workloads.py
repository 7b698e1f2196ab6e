"""The benchmark workloads themselves against the oracle, at their own sizes and through the library's default
launch choices: the packed prefill of 32 sequences (30,526 tokens, 16 heads) and 512 carried steps of the fused
streaming-decode block at B=256 with 8 key heads shared by 16 value heads.

Tolerances (bf16 inputs): outputs within 2e-2 max-abs, float32 states within 1e-3 relative (max|err| /
max|ref|, per sequence or stream), conv caches exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def test_varlen_workload_32_sequences(gdn, cuda):
    """The packed-prefill workload exactly as the bench runs it (the seed-1004 lengths in [64, 2048], Hk = Hv =
    16, per-sequence initial states ~N(0, 0.02), the library's default launch), every output row and all 32
    final states checked against the float64 chunked statement of the recurrence (itself pinned to the
    brute-force loop), sequence by sequence (gdn.py:418-434 with cu_seqlens and chunk_indices)."""
    lengths, d = bench.varlen_inputs(torch)
    cu, chunks = O.chunk_tables(lengths)
    announce(f"varlen workload n={len(lengths)} tokens={sum(lengths)} H=16")
    x = {n: d[n].to(cuda) for n in ("q", "k", "v", "g", "beta", "s0")}
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    ch_t = torch.tensor(chunks, dtype=torch.int32, device=cuda)
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"], cu_seqlens=cu_t,
                         chunk_indices=ch_t)
    torch.cuda.synchronize()
    assert gdn.ops.chunk_status() == 0
    o, s = o.float().cpu()[0], s.cpu()
    worst_o = worst_s = 0.0
    for i in range(len(lengths)):
        a, b = cu[i], cu[i + 1]
        o_ref, s_ref = O.chunked_np(d["q"][0, a:b], d["k"][0, a:b], d["v"][0, a:b], d["g"][0, a:b],
                                    d["beta"][0, a:b], 128**-0.5, d["s0"][i])
        eo = float(np.abs(o[a:b].double().numpy() - o_ref).max())
        es = rel_err(s[i], torch.from_numpy(s_ref))
        assert eo < 2e-2 and es < 1e-3, (i, lengths[i], eo, es)
        worst_o, worst_s = max(worst_o, eo), max(worst_s, es)
    print(f"varlen workload: worst output max-abs {worst_o:.3e}, worst state rel {worst_s:.3e}")


CHECK_STEPS = (1, 64, 128, 192, 256, 320, 384, 448, 512)  # after these many steps
STREAMS = (0, 1, 100, 255)                                  # the streams carried on the CPU


def test_streaming_block_512_steps(gdn, cuda):
    """The streaming-decode workload exactly as the bench runs it (B=256 streams, Hk=8 -> Hv=16, 512 consecutive
    steps carrying the conv cache and the fp32 state from zero, A_log = dt_bias = 0, eps 1e-6): all 256 streams
    on the GPU, four of them carried step by step through the oracle's fused block (lm.py:563-587 per new row)
    on the CPU; outputs, states and conv caches compared after steps 1, 64, ..., 512."""
    announce("fused decode workload B=256 Hk=8 Hv=16 x512 steps")
    xs, zs, as_, bs, w, nw, A_log, dt_bias, cache, state = bench.fused_inputs(torch, cuda)
    sel = torch.tensor(STREAMS, device=cuda)
    snaps = {}
    for t in range(bench.FUSED["steps"]):
        out = gdn.fused_decode_step(xs[t], zs[t], as_[t], bs[t], w, cache, state, nw, A_log, dt_bias, eps=1e-6)
        if t + 1 in CHECK_STEPS:
            snaps[t + 1] = (out.index_select(0, sel).cpu(), cache.index_select(0, sel).cpu(),
                            state.index_select(0, sel).cpu())
    torch.cuda.synchronize()
    # the oracle, on the selected streams' inputs
    x_c, z_c, a_c, b_c = (t.index_select(1, sel).cpu() for t in (xs, zs, as_, bs))
    w_c, nw_c, A_c, dt_c = w.cpu(), nw.cpu(), A_log.cpu(), dt_bias.cpu()
    c_ref = torch.zeros(len(STREAMS), *cache.shape[1:], dtype=cache.dtype)
    s_ref = torch.zeros(len(STREAMS), *state.shape[1:])
    hk = bench.FUSED["Hk"]
    for t in range(bench.FUSED["steps"]):
        o_ref, c_ref, s_ref = O.fused_decode_step(x_c[t], z_c[t], a_c[t], b_c[t], w_c, c_ref, s_ref, nw_c, A_c,
                                                  dt_c, hk, eps=1e-6)
        if t + 1 in snaps:
            o_g, c_g, s_g = snaps[t + 1]
            assert torch.equal(c_g, c_ref), f"conv cache differs after step {t + 1}"
            eo = max_abs(o_g, o_ref)
            es = max(rel_err(s_g[i], s_ref[i]) for i in range(len(STREAMS)))
            assert eo < 2e-2 and es < 1e-3, (t + 1, eo, es)


def test_overlapped_wait_give_up_is_reported(gdn, cuda):
    """The overlapped launch's bounded wait: with every ready flag read as unready (a host test switch) and a
    bound of 4 tries, each state job's wait runs out and carries on, every kernel ends, and the sticky device
    status word reports it (ops.check_chunk_status raises). With the switch off again the same call succeeds,
    leaves the word clear and matches the two-launch form bit for bit."""
    announce("chunk overlapped: forced wait give-up is reported")
    d = O.make_inputs(1, 4096, 16, 16, 128, 128, seed=1003, dtype=torch.bfloat16)
    x = {n: d[n].to(cuda) for n in ("q", "k", "v", "g", "beta")}
    gdn.ops.chunk_status(clear=True)
    lib = gdn._native.lib()
    form0 = lib.zgdn_chunk_get_launch_form()  # the form at the start (ZGDN_CHUNK_OVERLAP may have set it)
    try:
        gdn._native.call("zgdn_chunk_set_wait_limit", 4, 1)
        with gdn.ops.launch_form(1):
            gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"])
        st = gdn.ops.chunk_status(clear=False)
        assert st & gdn._native.STATUS_WAIT_GAVE_UP, st
        with pytest.raises(RuntimeError, match="gave up"):
            gdn.ops.check_chunk_status()
        assert gdn.ops.chunk_status() == 0  # check_chunk_status cleared it
    finally:
        gdn._native.call("zgdn_chunk_set_wait_limit", 0, 0)
    with gdn.ops.launch_form(1):
        o1, s1 = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"])
    with gdn.ops.launch_form(0):
        o0, s0 = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"])
    assert lib.zgdn_chunk_get_launch_form() == form0
    assert gdn.ops.chunk_status() == 0
    assert torch.equal(o1, o0) and torch.equal(s1, s0)


def test_zero_length_batch_passes_the_state_through(gdn, cuda):
    """T = 0 (a 0-row slice of real tensors): no chunk, the final state is the initial state, o is empty."""
    announce("chunk T=0 pass-through")
    d = O.make_inputs(2, 8, 2, 2, 128, 128, seed=1010, dtype=torch.bfloat16, state_std=0.02)
    x = {n: d[n].to(cuda) for n in ("q", "k", "v", "g", "beta", "s0")}
    o, s = gdn.chunk_fwd(x["q"][:, :0], x["k"][:, :0], x["v"][:, :0], x["g"][:, :0], x["beta"][:, :0],
                         initial_state=x["s0"])
    torch.cuda.synchronize()
    assert o.shape == (2, 0, 2, 128)
    assert torch.equal(s.cpu(), d["s0"])
