"""Writes the golden fixtures of the gated-DeltaNet path (run from the repository root:
``python tests/golden/make_golden.py``).

Each ``.npz`` holds seeded inputs and expected outputs. The recurrence cases are computed in float64 by the
oracle's mathematics-only statements (``recurrence_np``, the brute-force token loop, cross-checked here
against ``chunked_np``, the chunked WY form); the conv case by a float64 ``F.conv1d``; the fused-block case
by the torch restatement of lm.py:563-587 (a regression fixture: its pins are the CPU tests that rebuild it
from the float64 loop). Arrays are stored as float32 (bf16 inputs are stored as the float32 values of the
bf16 numbers, so they round-trip exactly).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import gdn_oracle as O  # noqa: E402


def _f32(t):
    return t.detach().float().numpy() if torch.is_tensor(t) else np.asarray(t, dtype=np.float32)


def _sequences(d, lengths, scale, g_override=None):
    """Expected o and final states per packed sequence via the float64 loop (checked against the WY form)."""
    cu = np.cumsum([0] + lengths)
    q, k, v = (d[n][0].double().numpy() for n in ("q", "k", "v"))
    g = d["g"][0].double().numpy() if g_override is None else g_override
    b = d["beta"][0].double().numpy()
    o = np.zeros(v.shape)
    finals = []
    for i in range(len(lengths)):
        lo, hi = cu[i], cu[i + 1]
        oi, si = O.recurrence_np(q[lo:hi], k[lo:hi], v[lo:hi], g[lo:hi], b[lo:hi], scale, d["s0"][i])
        oc, sc = O.chunked_np(q[lo:hi], k[lo:hi], v[lo:hi], g[lo:hi], b[lo:hi], scale, d["s0"][i])
        assert np.abs(oi - oc).max(initial=0) < 1e-9 and np.abs(si - sc).max() < 1e-9
        o[lo:hi] = oi
        finals.append(si)
    return o, np.stack(finals)


def recurrent_fp32():
    d = O.make_inputs(1, 40, 2, 2, 64, 64, seed=9001, state_std=0.1)
    o, s = _sequences(d, [40], 64**-0.5)
    return dict(q=_f32(d["q"]), k=_f32(d["k"]), v=_f32(d["v"]), g=_f32(d["g"]), beta=_f32(d["beta"]),
                s0=_f32(d["s0"]), o=_f32(o[None]), s=_f32(s))


def decode_bf16():
    d = O.make_inputs(2, 1, 1, 1, 128, 128, seed=9002, dtype=torch.bfloat16, state_std=0.02)
    outs, states = [], []
    for b in range(2):
        o, s = O.recurrence_np(d["q"][b].double().numpy(), d["k"][b].double().numpy(), d["v"][b].double().numpy(),
                               d["g"][b].double().numpy(), d["beta"][b].double().numpy(), 128**-0.5, d["s0"][b])
        outs.append(o)
        states.append(s)
    return dict(q=_f32(d["q"]), k=_f32(d["k"]), v=_f32(d["v"]), g=_f32(d["g"]), beta=_f32(d["beta"]),
                s0=_f32(d["s0"]), o=_f32(np.stack(outs)), s=_f32(np.stack(states)))


def chunk_varlen_bf16():
    lengths = [70, 5, 0]
    d = O.make_inputs(1, sum(lengths), 1, 2, 128, 128, seed=9003, dtype=torch.bfloat16, state_std=0.02,
                      n_states=len(lengths))
    o, s = _sequences(d, lengths, 128**-0.5)
    cu, chunks = O.chunk_tables(lengths)
    return dict(q=_f32(d["q"]), k=_f32(d["k"]), v=_f32(d["v"]), g=_f32(d["g"]), beta=_f32(d["beta"]),
                s0=_f32(d["s0"]), o=_f32(o[None]), s=_f32(s), cu=np.asarray(cu, np.int32),
                chunks=np.asarray(chunks, np.int32).reshape(-1, 2))


def fused_block():
    """Two steps of the whole block for 2 streams (Hk=1, Hv=2) from the float64 pieces."""
    gen = torch.Generator().manual_seed(9004)
    B, hk, hv, K = 2, 1, 2, 128
    C = 2 * hk * K + hv * K
    x = torch.randn(2, B, C, generator=gen).to(torch.bfloat16)
    z = torch.randn(2, B, hv, K, generator=gen).to(torch.bfloat16)
    a = torch.randn(2, B, hv, generator=gen).to(torch.bfloat16)
    b = torch.randn(2, B, hv, generator=gen).to(torch.bfloat16)
    w = (0.2 * torch.randn(C, 4, generator=gen)).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(K, generator=gen)).to(torch.bfloat16)
    A_log, dt_bias = 0.3 * torch.randn(hv, generator=gen), 0.3 * torch.randn(hv, generator=gen)
    cache0 = (0.5 * torch.randn(B, C, 3, generator=gen)).to(torch.bfloat16)
    s0 = 0.02 * torch.randn(B, hv, K, K, generator=gen)
    cache, state = cache0.clone(), s0.clone()
    outs = []
    for t in range(2):
        o, cache, state = O.fused_decode_step(x[t], z[t], a[t], b[t], w, cache, state, nw, A_log, dt_bias, hk,
                                              eps=1e-6)
        outs.append(o)
    return dict(x=_f32(x), z=_f32(z), a=_f32(a), b=_f32(b), w=_f32(w), nw=_f32(nw), A_log=_f32(A_log),
                dt_bias=_f32(dt_bias), cache0=_f32(cache0), s0=_f32(s0), out=_f32(torch.stack(outs)),
                cache=_f32(cache), s=_f32(state))


def conv_varlen():
    lengths = [1, 3, 70]
    gen = torch.Generator().manual_seed(9005)
    D = 16
    x = torch.randn(1, sum(lengths), D, generator=gen)
    w = 0.3 * torch.randn(D, 4, generator=gen)
    s0 = torch.randn(len(lengths), D, 4, generator=gen)
    cu = np.cumsum([0] + lengths)
    ys, fins = [], []
    for i in range(len(lengths)):
        seq = torch.cat((s0[i][:, 1:], x[0, cu[i]:cu[i + 1]].T), -1).double()
        y = F.conv1d(seq[None], w.double()[:, None, :], groups=D)[0].T
        ys.append(F.silu(y))
        fins.append(torch.cat((s0[i], x[0, cu[i]:cu[i + 1]].T), -1)[:, -4:])
    return dict(x=_f32(x), w=_f32(w), s0=_f32(s0), y=_f32(torch.cat(ys)[None]), fin=_f32(torch.stack(fins)),
                cu=np.asarray(cu, np.int32))


CASES = {
    "recurrent_fp32_T40_H2_d64": recurrent_fp32,
    "decode_bf16_B2_H1_d128": decode_bf16,
    "chunk_varlen_bf16_H1to2_d128": chunk_varlen_bf16,
    "fused_block_B2_Hk1_Hv2": fused_block,
    "conv_varlen_D16": conv_varlen,
}


def main():
    for name, fn in CASES.items():
        arrays = fn()
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        size = (HERE / f"{name}.npz").stat().st_size
        print(f"{name}.npz  {size} bytes")


if __name__ == "__main__":
    main()
