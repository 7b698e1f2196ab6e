"""Chunked prefill kernel (zgdn_chunk_fwd) against the CPU oracle on seeded inputs.

Tolerances (bf16 inputs): outputs within 2e-2 max-abs, float32 final states within 1e-3 relative
(max|err| / max|ref|).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _dev(d, cuda, gb_dtype=torch.float32):
    x = {n: d[n].to(cuda) for n in ("q", "k", "v", "s0")}
    x["g"], x["beta"] = d["g"].to(cuda, gb_dtype), d["beta"].to(cuda, gb_dtype)
    return x


def _check(o, s, o_ref, s_ref):
    eo, es = max_abs(o, o_ref), rel_err(s, s_ref)
    print(f"[errors] output max-abs {eo:.3e}, state rel {es:.3e}")
    assert eo < 2e-2 and es < 1e-3, (eo, es)
    return eo, es


@pytest.mark.parametrize("B,T,H", [(1, 64, 2), (1, 65, 2), (2, 200, 3), (1, 1, 1), (1, 130, 4)])
def test_small_shapes(gdn, cuda, B, T, H):
    announce(f"chunk B={B} T={T} H={H}")
    d = O.make_inputs(B, T, H, H, 128, 128, seed=2000 + T + H, dtype=torch.bfloat16, state_std=0.02)
    x = _dev(d, cuda)
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"])
    torch.cuda.synchronize()
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"])
    _check(o.cpu(), s.cpu(), o_ref, s_ref)


def test_prefill_T4096_H16(gdn, cuda):
    """Chunked prefill workload: B=1, T=4096, H=16, dk=dv=128, bf16, zero initial state."""
    announce("chunk prefill T=4096 H=16")
    d = O.make_inputs(1, 4096, 16, 16, 128, 128, seed=1003, dtype=torch.bfloat16)
    x = _dev(d, cuda)
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"])
    torch.cuda.synchronize()
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"])
    _check(o.cpu(), s.cpu(), o_ref, s_ref)


def test_prefill_T16384_H16(gdn, cuda):
    """A prompt four times the prefill workload's (B=1, T=16384, H=16, dk=dv=128, bf16, initial states
    ~N(0, 0.02)): 256 chunks a chain, within the same tolerance (the state error does not grow with T)."""
    announce("chunk prefill T=16384 H=16")
    d = O.make_inputs(1, 16384, 16, 16, 128, 128, seed=1016, dtype=torch.bfloat16, state_std=0.02)
    x = _dev(d, cuda)
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"])
    torch.cuda.synchronize()
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"])
    _check(o.cpu(), s.cpu(), o_ref, s_ref)


def test_prefill_T65536_H4_segmented(gdn, cuda):
    """A 65,536-token prompt at the release model's 4 heads (initial states ~N(0, 0.02)): the segmented state
    pass at its longest segments (4 segments of 256 chunks, three combine steps). Against the token-loop
    recurrent kernel (fp32 state; itself checked against the oracle) within the oracle tolerance: the state
    error does not grow with the segment length."""
    announce("chunk prefill T=65536 H=4 (segmented)")
    assert int(gdn._native.lib().zgdn_chunk_segment_workspace_size(1, 65536, 4)) > 0  # the path is taken
    d = O.make_inputs(1, 65536, 4, 4, 128, 128, seed=1065, dtype=torch.bfloat16, state_std=0.02)
    x = _dev(d, cuda)
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"])
    o_ref, s_ref = gdn.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"],
                                     out_dtype=torch.float32)
    torch.cuda.synchronize()
    _check(o.cpu(), s.cpu(), o_ref.cpu(), s_ref.cpu())


def test_packed_sequences(gdn, cuda):
    lengths = [64, 1, 130, 0, 70, 200, 63]
    cu, _ = O.chunk_tables(lengths)
    announce(f"chunk varlen lengths={lengths}")
    d = O.make_inputs(1, sum(lengths), 4, 4, 128, 128, seed=2101, dtype=torch.bfloat16, state_std=0.02,
                      n_states=len(lengths))
    x = _dev(d, cuda)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"], cu_seqlens=cu_t)
    torch.cuda.synchronize()
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"], cu_seqlens=cu)
    _check(o.cpu(), s.cpu(), o_ref, s_ref)
    assert torch.equal(s[3].cpu(), d["s0"][3])  # the empty sequence keeps its state


def test_many_short_packed_sequences(gdn, cuda):
    """300 packed sequences, most of 0-3 tokens and some at the chunk edges, with one of 2,000 tokens in the
    middle, grouped heads (2 key, 4 value): more sequences than the overlapped launch takes and 1,200 chains
    (two value blocks per state workgroup). Against the oracle; empty sequences keep their states."""
    gen = torch.Generator().manual_seed(2131)
    pool = [0, 1, 2, 3, 1, 2, 63, 64, 65]
    lengths = [pool[int(i)] for i in torch.randint(0, len(pool), (300,), generator=gen)]
    lengths[150] = 2000
    cu, _ = O.chunk_tables(lengths)
    announce(f"chunk varlen {len(lengths)} sequences, {sum(lengths)} tokens")
    d = O.make_inputs(1, sum(lengths), 2, 4, 128, 128, seed=2132, dtype=torch.bfloat16, state_std=0.02,
                      n_states=len(lengths))
    x = _dev(d, cuda)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"], cu_seqlens=cu_t)
    torch.cuda.synchronize()
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"], cu_seqlens=cu)
    _check(o.cpu(), s.cpu(), o_ref, s_ref)
    for i, n in enumerate(lengths):
        if n == 0:
            assert torch.equal(s[i].cpu(), d["s0"][i])


def test_grouped_heads_gate_in_kernel_and_bf16_gates(gdn, cuda):
    """Hk=8 -> Hv=16; the decay formed in the kernel from raw a, A_log, dt_bias; bf16 a and beta."""
    announce("chunk GVA 8->16, in-kernel gate, bf16 gates")
    gen = torch.Generator().manual_seed(2202)
    d = O.make_inputs(1, 300, 8, 16, 128, 128, seed=2201, dtype=torch.bfloat16, state_std=0.02)
    a = torch.randn(1, 300, 16, generator=gen).to(torch.bfloat16)
    A_log = 0.3 * torch.randn(16, generator=gen)
    dt_bias = 0.3 * torch.randn(16, generator=gen)
    beta = d["beta"].to(torch.bfloat16)
    o, s = gdn.chunk_fwd(d["q"].to(cuda), d["k"].to(cuda), d["v"].to(cuda), a.to(cuda), beta.to(cuda),
                         initial_state=d["s0"].to(cuda), A_log=A_log.to(cuda), dt_bias=dt_bias.to(cuda))
    torch.cuda.synchronize()
    g_log = -A_log.exp() * F.softplus(a.float() + dt_bias)
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], g_log, beta.float(), None, d["s0"])
    _check(o.cpu(), s.cpu(), o_ref, s_ref)


def test_chunked_equals_recurrent_kernel_and_in_place(gdn, cuda):
    """The two HIP paths agree on the full prefill shape; the chunked one can update the state in place."""
    announce("chunk vs recurrent T=4096 H=16, in-place")
    d = O.make_inputs(1, 4096, 16, 16, 128, 128, seed=2301, dtype=torch.bfloat16, state_std=0.02)
    x = _dev(d, cuda)
    o_r, s_r = gdn.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], None, x["s0"])
    state = x["s0"].clone()
    o_c, s_c = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=state, final_state=state)
    torch.cuda.synchronize()
    assert s_c is state
    _check(o_c.cpu(), s_c.cpu(), o_r.float().cpu(), s_r.cpu())


@pytest.mark.parametrize("packed", [False, True])
def test_rows_read_in_place_and_beta_logits(gdn, cuda, packed):
    """q, k, v as column slices of one wider row (the conv output) and g, beta as columns of another (the
    input projection), beta given as logits: bit-identical to the same values handed over dense with beta =
    sigmoid(b) from the sigmoid kernel; a row stride the kernel cannot take (not a multiple of 8) is copied
    first, same result."""
    announce(f"chunk rows in place, beta logits, packed={packed}")
    gen = torch.Generator().manual_seed(2401)
    B, T, Hk, Hv = (1, 333, 2, 4) if packed else (2, 150, 2, 4)
    width = (2 * Hk + Hv) * 128
    conv = (0.7 * torch.randn(B, T, width + 64, generator=gen)).to(torch.bfloat16).to(cuda)
    proj = torch.randn(B, T, 40, generator=gen).to(torch.bfloat16).to(cuda)
    q = conv[..., : Hk * 128].unflatten(-1, (Hk, 128))
    k = conv[..., Hk * 128: 2 * Hk * 128].unflatten(-1, (Hk, 128))
    v = conv[..., 2 * Hk * 128: width].unflatten(-1, (Hv, 128))
    a, b = proj[..., 3: 3 + Hv], proj[..., 20: 20 + Hv]
    A_log, dt_bias = (0.3 * torch.randn(Hv, generator=gen)).to(cuda), (0.3 * torch.randn(Hv, generator=gen)).to(cuda)
    s0 = (0.02 * torch.randn(B if not packed else 3, Hv, 128, 128, generator=gen)).to(cuda)
    kw = dict(A_log=A_log, dt_bias=dt_bias, use_qk_l2norm=True)
    if packed:
        cu = torch.tensor([0, 100, 100 + 64, T], dtype=torch.int32, device=cuda)
        kw["cu_seqlens"] = cu
    o1, s1 = gdn.chunk_fwd(q, k, v, a, b, initial_state=s0, beta_is_logit=True, **kw)
    beta = gdn.ops.sigmoid(b.contiguous(), out_dtype=torch.float32)
    o2, s2 = gdn.chunk_fwd(q.contiguous(), k.contiguous(), v.contiguous(), a.float().contiguous(), beta,
                           initial_state=s0, **kw)
    wide = torch.zeros(B, T, width + 4, dtype=torch.bfloat16, device=cuda)  # row stride 4 mod 8: copied
    wide[..., :width] = conv[..., :width]
    qm = wide[..., : Hk * 128].unflatten(-1, (Hk, 128))
    o3, s3 = gdn.chunk_fwd(qm, k, v, a, b, initial_state=s0, beta_is_logit=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    assert torch.equal(o1, o3) and torch.equal(s1, s3)
    # and the values themselves against the oracle, sequence by sequence
    g_log = -A_log.exp().cpu() * F.softplus(a.float().cpu() + dt_bias.cpu())
    qn, kn = O.l2norm(q.float().cpu()), O.l2norm(k.float().cpu())
    bounds = [(0, 100), (100, 164), (164, T)] if packed else None
    for i in range(len(s0)):
        bi, (lo, hi) = (0, bounds[i]) if packed else (i, (0, T))
        o_ref, s_ref = O.gated_delta_recurrence(qn[bi:bi + 1, lo:hi], kn[bi:bi + 1, lo:hi],
                                                v[bi:bi + 1, lo:hi].float().cpu(), g_log[bi:bi + 1, lo:hi],
                                                beta.cpu()[bi:bi + 1, lo:hi], None, s0[i:i + 1].cpu())
        _check(o1[bi:bi + 1, lo:hi].cpu(), s1[i:i + 1].cpu(), o_ref, s_ref)


def _plain_pass(gdn, cuda, q, k, v, g, beta, s0, fin):
    """zgdn_chunk_fwd with only the phase-1 workspace: the plain (unsegmented) state pass."""
    native = gdn._native
    B, T, Hk, _ = q.shape
    Hv = v.shape[2]
    nch = B * (-(-T // 64))
    ws_bytes = int(native.lib().zgdn_chunk_workspace_size(nch, Hv))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=cuda)
    o = torch.empty(B, T, Hv, 128, dtype=torch.bfloat16, device=cuda)
    stream = torch.cuda.current_stream().cuda_stream
    native.call("zgdn_chunk_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), native.BF16, g.data_ptr(),
                beta.data_ptr(), native.F32, None, None, 0, None if s0 is None else s0.data_ptr(), fin.data_ptr(),
                o.data_ptr(), None, None, B, nch, B, T, Hk, Hv, 128, 128, Hk * 128, Hk * 128, Hv * 128, Hv, 0,
                128**-0.5, ws.data_ptr(), ws_bytes, stream)
    return o


@pytest.mark.parametrize("B,T,Hk,Hv,with_state", [(1, 4096, 4, 4, True), (2, 2600, 1, 2, True),
                                                  (1, 3000, 2, 4, False), (1, 4096, 1, 1, True),
                                                  (1, 8192, 1, 1, False)])
def test_segmented_state_pass(gdn, cuda, B, T, Hk, Hv, with_state):
    """Few sequences and heads, long enough: the state pass runs each sequence as segments at once (from zero
    states and, for the segment maps, from the identity) and combines them -- here 4 segments (the last ones
    ragged, two sequences, grouped heads), 5 and 8. Against the oracle, against the plain pass (same inputs,
    phase-1 workspace only), and with the final state written over the initial one."""
    announce(f"chunk segmented pass B={B} T={T} Hk={Hk} Hv={Hv} state={with_state}")
    assert int(gdn._native.lib().zgdn_chunk_segment_workspace_size(B, T, Hv)) > 0  # the path is taken
    d = O.make_inputs(B, T, Hk, Hv, 128, 128, seed=2500 + T + Hv, dtype=torch.bfloat16, state_std=0.02)
    x = _dev(d, cuda)
    s0 = x["s0"] if with_state else None
    o, s = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=s0)
    fin_plain = torch.empty(B, Hv, 128, 128, device=cuda)
    o_plain = _plain_pass(gdn, cuda, x["q"], x["k"], x["v"], x["g"], x["beta"], s0, fin_plain)
    state = x["s0"].clone() if with_state else torch.zeros_like(x["s0"])
    o2, s2 = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=state, final_state=state)
    torch.cuda.synchronize()
    assert s2 is state and torch.equal(o2, o) and torch.equal(s2, s)
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None,
                                            d["s0"] if with_state else None)
    _check(o.cpu(), s.cpu(), o_ref, s_ref)
    _check(o_plain.cpu(), fin_plain.cpu(), o_ref, s_ref)
    assert max_abs(o.cpu(), o_plain.cpu()) < 2e-2 and rel_err(s.cpu(), fin_plain.cpu()) < 1e-3


@pytest.mark.parametrize("B,T,Hk,Hv,gate,with_state", [(1, 4096, 16, 16, False, False),
                                                       (2, 1000, 4, 8, True, True),
                                                       (4, 700, 8, 8, False, True),
                                                       (1, 192, 8, 8, True, False),
                                                       (1, 100, 16, 16, False, True),
                                                       (4, 500, 16, 16, True, True)])
def test_overlapped_launch(gdn, cuda, B, T, Hk, Hv, gate, with_state):
    """The overlapped launch (phase 1 and the state pass in one kernel, linked by per-chunk ready flags on each
    XCD), forced with launch form 1 (by default it is taken only where it measured faster). It runs the
    same arithmetic as the two launches, so the results are bit-identical to them (launch form 0), on
    two calls in a row (the control block is reset per call), and within tolerance of the oracle. Shapes: the prefill workload, two
    sequences with grouped heads and a ragged last chunk, the largest (32 chains) and smallest (8) batches of
    the few-chains order, a sequence shorter than two chunks, and 64 chains (the many-chains order)."""
    announce(f"chunk overlapped B={B} T={T} Hk={Hk} Hv={Hv} gate={gate} state={with_state}")
    gen = torch.Generator().manual_seed(2600 + T + Hv)
    d = O.make_inputs(B, T, Hk, Hv, 128, 128, seed=2600 + B + T, dtype=torch.bfloat16, state_std=0.02)
    x = _dev(d, cuda)
    s0 = x["s0"] if with_state else None
    kw = {}
    g_in, g_log = x["g"], d["g"]
    if gate:
        a = torch.randn(B, T, Hv, generator=gen)
        A_log, dt_bias = 0.3 * torch.randn(Hv, generator=gen), 0.3 * torch.randn(Hv, generator=gen)
        kw = dict(A_log=A_log.to(cuda), dt_bias=dt_bias.to(cuda))
        g_in, g_log = a.to(cuda), -A_log.exp() * F.softplus(a + dt_bias)
    runs = []
    for form in (1, 1, 0):
        with gdn.ops.launch_form(form):
            runs.append(gdn.chunk_fwd(x["q"], x["k"], x["v"], g_in, x["beta"], initial_state=s0, **kw))
    torch.cuda.synchronize()
    (o1, s1), (o2, s2), (o0, s0_) = runs
    assert torch.equal(o1, o0) and torch.equal(s1, s0_)
    assert torch.equal(o2, o0) and torch.equal(s2, s0_)
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], g_log, d["beta"], None,
                                            d["s0"] if with_state else None)
    _check(o1.cpu(), s1.cpu(), o_ref, s_ref)


@pytest.mark.parametrize("lengths,Hk,Hv", [([64, 1, 130, 0, 70, 200, 63, 128], 2, 4),
                                          ([700, 64, 1000, 3, 512, 129, 66, 2048, 300, 90, 1, 450], 8, 16),
                                          ([100] * 40, 4, 8)])
def test_overlapped_launch_packed(gdn, cuda, lengths, Hk, Hv):
    """Packed sequences (and their empty, one-token and ragged members) in the overlapped launch's many-chains
    order (forced): bit-identical to the two launches, within tolerance of the oracle, initial states carried
    and the empty sequence's state passed through."""
    announce(f"chunk overlapped packed n={len(lengths)} Hk={Hk} Hv={Hv}")
    cu, chunks = O.chunk_tables(lengths)
    d = O.make_inputs(1, sum(lengths), Hk, Hv, 128, 128, seed=2700 + len(lengths), dtype=torch.bfloat16,
                      state_std=0.02, n_states=len(lengths))
    x = _dev(d, cuda)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    ch_t = torch.tensor(chunks, dtype=torch.int32, device=cuda)
    runs = []
    for form in (1, 1, 0):
        with gdn.ops.launch_form(form):
            runs.append(gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"],
                                      cu_seqlens=cu_t, chunk_indices=ch_t))
    torch.cuda.synchronize()
    (o1, s1), (o2, s2), (o0, s0_) = runs
    assert torch.equal(o1, o0) and torch.equal(s1, s0_)
    assert torch.equal(o2, o0) and torch.equal(s2, s0_)
    o_ref, s_ref = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"], cu_seqlens=cu)
    _check(o1.cpu(), s1.cpu(), o_ref, s_ref)
    for i, n in enumerate(lengths):
        if n == 0:
            assert torch.equal(s1[i].cpu(), d["s0"][i])


def _random_case(rng: "torch.Generator"):
    """One seeded batch: 1-9 packed sequences whose lengths mix the chunk edges (0, 1, 63, 64, 65, 128) with
    uniform draws up to 900 tokens, 1-8 key heads with 1 or 2 value heads each, and random switches for the
    initial states, the in-kernel gate, bf16 gate inputs, beta given as logits and the in-kernel L2 norm."""
    def pick(n):
        return int(torch.randint(0, n, (1,), generator=rng))
    edges = [0, 1, 63, 64, 65, 128]
    n = 1 + pick(9)
    lengths = [edges[pick(len(edges))] if pick(2) else 1 + pick(900) for _ in range(n)]
    if sum(lengths) == 0:
        lengths[0] = 1 + pick(200)
    hk = [1, 2, 4, 8][pick(4)]
    return dict(lengths=lengths, Hk=hk, Hv=hk * (1 + pick(2)), state=bool(pick(2)), gate=bool(pick(2)),
                bf16_gates=bool(pick(2)), beta_logit=bool(pick(2)), l2=bool(pick(2)))


@pytest.mark.parametrize("case", range(8))
def test_random_packed_batches(gdn, cuda, case):
    """Seeded random packed batches through the library's own choice of launch form, against the oracle, and
    bit-identical to the overlapped launch (launch form 1) and the two-launch form (0). The inputs are drawn
    as for the configurations, except that with the in-kernel L2 norm q and k are raw N(0,1) rows, g is
    the raw gate input when the gate is in the kernel, and beta is its logit when so flagged; the oracle
    takes the rows normalised, the log decay and sigmoid(beta) formed from the same inputs in float32."""
    rng = torch.Generator().manual_seed(3100 + case)
    c = _random_case(rng)
    lengths, Hk, Hv = c["lengths"], c["Hk"], c["Hv"]
    announce(f"chunk random case={case} {c}")
    cu, chunks = O.chunk_tables(lengths)
    T, N = sum(lengths), len(lengths)
    d = O.make_inputs(1, T, Hk, Hv, 128, 128, seed=3200 + case, dtype=torch.bfloat16, state_std=0.02, n_states=N)
    q_ref, k_ref = d["q"].float(), d["k"].float()
    if c["l2"]:  # raw rows in, normalised in the kernel; the oracle normalises the same bf16 rows
        d["q"] = torch.randn(1, T, Hk, 128, generator=rng).to(torch.bfloat16)
        d["k"] = torch.randn(1, T, Hk, 128, generator=rng).to(torch.bfloat16)
        q_ref, k_ref = O.l2norm(d["q"]), O.l2norm(d["k"])
    g_log, beta_ref = d["g"].float(), d["beta"].float()
    gdt = torch.bfloat16 if c["bf16_gates"] else torch.float32
    kw = {}
    g_in, beta_in = d["g"].to(gdt), d["beta"].to(gdt)
    if c["gate"]:
        a = torch.randn(1, T, Hv, generator=rng).to(gdt)
        A_log, dt_bias = 0.3 * torch.randn(Hv, generator=rng), 0.3 * torch.randn(Hv, generator=rng)
        kw.update(A_log=A_log.to(cuda), dt_bias=dt_bias.to(cuda))
        g_in = a
        g_log = -A_log.exp() * F.softplus(a.float() + dt_bias)
    elif c["bf16_gates"]:
        g_log = g_in.float()
    if c["beta_logit"]:
        b = torch.randn(1, T, Hv, generator=rng).to(gdt)
        beta_in, beta_ref = b, torch.sigmoid(b.float())
        kw["beta_is_logit"] = True
    elif c["bf16_gates"]:
        beta_ref = beta_in.float()
    s0 = d["s0"].to(cuda) if c["state"] else None
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    ch_t = torch.tensor(chunks, dtype=torch.int32, device=cuda)
    args = (d["q"].to(cuda), d["k"].to(cuda), d["v"].to(cuda), g_in.to(cuda), beta_in.to(cuda))
    runs = []
    for form in (-1, 1, 0):
        with gdn.ops.launch_form(form):
            runs.append(gdn.chunk_fwd(*args, initial_state=s0, cu_seqlens=cu_t, chunk_indices=ch_t,
                                      use_qk_l2norm=c["l2"], **kw))
    torch.cuda.synchronize()
    (o1, s1), (o2, s2), (o0, s0_) = runs
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    assert torch.equal(o1, o0) and torch.equal(s1, s0_)
    o_ref, s_ref = O.gated_delta_recurrence(q_ref, k_ref, d["v"].float(), g_log, beta_ref, None,
                                            d["s0"] if c["state"] else None, cu_seqlens=cu)
    _check(o1.cpu(), s1.cpu(), o_ref, s_ref)
