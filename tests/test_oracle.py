"""Pins of the CPU oracle (no GPU): closed forms, invariants, brute force and the reference's literal tables.

Each statement of the oracle is checked against something the mathematics fixes, so that a plausible
transcription mistake (a dropped decay, a transposed state, a wrong grouped-head index) fails at least one
check; ``test_planted_mistakes_are_caught`` plants such mistakes in copies of the oracle and asserts that.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gdn_testing import rel_err
from oracle import gdn_oracle as O


def _seq(T, hk, hv, K, V, seed, state_std=0.1):
    d = O.make_inputs(1, T, hk, hv, K, V, seed=seed, state_std=state_std)
    return d["q"][0], d["k"][0], d["v"][0], d["g"][0], d["beta"][0], d["s0"][0]


# ------------------------------------------------------------------------------------------ known answers


def test_beta_zero_is_pure_decay():
    q, k, v, g, b, s0 = _seq(37, 2, 2, 16, 8, seed=1)
    b = torch.zeros_like(b)
    o, s = O.gated_delta_sequence(q, k, v, g.exp(), b, 0.3, s0)
    G = torch.cumsum(g.double(), 0)  # [T, H]
    want_s = torch.exp(G[-1])[:, None, None] * s0.double()
    want_o = 0.3 * torch.exp(G)[:, :, None] * torch.einsum("hvk,thk->thv", s0.double(), q.double())
    assert rel_err(s, want_s) < 1e-5 and rel_err(o, want_o) < 1e-5


def test_one_token_from_zero_state():
    q, k, v, g, b, _ = _seq(1, 3, 3, 16, 12, seed=2)
    o, s = O.gated_delta_sequence(q, k, v, g.exp(), b, 0.25, torch.zeros(3, 12, 16))
    kq = (k[0] * q[0]).sum(-1)  # [H]
    assert rel_err(o[0], (b[0] * kq * 0.25)[:, None] * v[0]) < 1e-6
    assert rel_err(s, b[0][:, None, None] * v[0][:, :, None] * k[0][:, None, :]) < 1e-6


def test_beta_one_with_unit_key_writes_the_value():
    q, k, v, g, b, s0 = _seq(9, 2, 2, 32, 8, seed=3)
    k = k.double() / k.double().norm(dim=-1, keepdim=True)
    S = s0.double()
    for t in range(9):
        _, S = O.gated_delta_sequence(q[t : t + 1].double(), k[t : t + 1], v[t : t + 1].double(),
                                      g[t : t + 1].double().exp(), torch.ones(1, 2, dtype=torch.float64), 1.0, S)
        assert torch.allclose(torch.einsum("hvk,hk->hv", S, k[t]), v[t].double(), atol=1e-12)


def test_unit_decay_zero_beta_leaves_the_state():
    q, k, v, g, b, s0 = _seq(11, 2, 4, 16, 16, seed=4)
    _, s = O.gated_delta_sequence(q, k, v, torch.ones_like(g), torch.zeros_like(b), 1.0, s0)
    assert torch.equal(s, s0)


# --------------------------------------------------------------------------- independent float64 statements


@pytest.mark.parametrize("T,hk,hv,K,V", [(1, 1, 1, 8, 8), (50, 2, 2, 16, 8), (70, 1, 2, 16, 16), (33, 2, 4, 8, 4)])
def test_torch_restatement_matches_brute_force(T, hk, hv, K, V):
    q, k, v, g, b, s0 = _seq(T, hk, hv, K, V, seed=T + hk)
    o_t, s_t = O.gated_delta_sequence(q, k, v, g.exp(), b, K**-0.5, s0)
    o_n, s_n = O.recurrence_np(q, k, v, g, b, K**-0.5, s0)
    assert rel_err(o_t, o_n) < 1e-5 and rel_err(s_t, s_n) < 1e-5


@pytest.mark.parametrize("T", [1, 5, 63, 64, 65, 130, 200])
@pytest.mark.parametrize("chunk", [64, 16])
def test_chunked_form_equals_recurrence(T, chunk):
    q, k, v, g, b, s0 = _seq(T, 2, 4, 16, 8, seed=T)
    o_r, s_r = O.recurrence_np(q, k, v, g, b, 0.25, s0)
    o_c, s_c = O.chunked_np(q, k, v, g, b, 0.25, s0, chunk=chunk)
    assert np.abs(o_r - o_c).max() < 1e-12 * max(1.0, np.abs(o_r).max())
    assert np.abs(s_r - s_c).max() < 1e-12 * max(1.0, np.abs(s_r).max())


def test_split_invariance_prefill_then_decode_steps():
    """prefill(T) == prefill(T - k) followed by k single-token steps (model/tests/test_reference_lm.py:126-136)."""
    q, k, v, g, b, s0 = _seq(40, 2, 2, 16, 16, seed=5)
    o_full, s_full = O.gated_delta_sequence(q, k, v, g.exp(), b, 0.25, s0)
    o_a, s = O.gated_delta_sequence(q[:35], k[:35], v[:35], g[:35].exp(), b[:35], 0.25, s0)
    parts = [o_a]
    for t in range(35, 40):
        o_t, s = O.gated_delta_sequence(q[t : t + 1], k[t : t + 1], v[t : t + 1], g[t : t + 1].exp(),
                                        b[t : t + 1], 0.25, s)
        parts.append(o_t)
    torch.testing.assert_close(torch.cat(parts), o_full, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(s, s_full, rtol=1e-5, atol=1e-5)


def test_segments_combine_through_their_state_maps():
    """The algebra of the segmented state pass, on the oracle: a segment's map M is its run from the identity
    state with zero values, its local part L the run from zero; the end state is S_start M + L and each output
    o_local + S_start (M_t q_t), M_t q_t being the identity run's output. Chained over three segments (V = K)
    against one run over the whole sequence."""
    T, H, K = 90, 2, 16
    d = O.make_inputs(1, T, H, H, K, K, seed=77, state_std=0.3)
    d["g"] = 0.02 * d["g"]  # decays near 0.99 a token, so that the maps carry weight
    q, k, v, g, beta = (d[n][0] for n in ("q", "k", "v", "g", "beta"))
    scale = K**-0.5
    o_full, s_full = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"])
    S = d["s0"][0]
    eye = torch.eye(K).expand(H, K, K)
    for lo, hi in ((0, 40), (40, 70), (70, T)):
        args = (q[lo:hi], k[lo:hi])
        o_loc, L = O.gated_delta_sequence(*args, v[lo:hi], g[lo:hi].exp(), beta[lo:hi], scale, torch.zeros(H, K, K))
        o_map, M = O.gated_delta_sequence(*args, torch.zeros_like(v[lo:hi]), g[lo:hi].exp(), beta[lo:hi], scale, eye)
        o_seg = o_loc + torch.einsum("hvk,thk->thv", S, o_map)
        assert rel_err(o_seg, o_full[0, lo:hi]) < 1e-5, (lo, hi)
        S = S @ M + L
    assert rel_err(S, s_full[0]) < 1e-5


def test_grouped_heads_read_key_head_h_div_group():
    """Hv = 2 Hk equals the ungrouped rule on k/q heads repeated (gdn_kernel.py:16-18)."""
    q, k, v, g, b, s0 = _seq(20, 2, 4, 16, 8, seed=6)
    o_g, s_g = O.gated_delta_sequence(q, k, v, g.exp(), b, 0.5, s0)
    rq, rk = q.repeat_interleave(2, 1), k.repeat_interleave(2, 1)
    o_r, s_r = O.gated_delta_sequence(rq, rk, v, g.exp(), b, 0.5, s0)
    assert torch.equal(o_g, o_r) and torch.equal(s_g, s_r)
    # and differs from the interleaved (h % Hk) assignment
    o_w, _ = O.gated_delta_sequence(q.repeat(1, 2, 1), k.repeat(1, 2, 1), v, g.exp(), b, 0.5, s0)
    assert rel_err(o_w, o_g) > 1e-2


def test_packed_sequences_equal_separate_calls():
    lengths = [5, 64, 1, 70]
    cu, _ = O.chunk_tables(lengths)
    d = O.make_inputs(1, sum(lengths), 2, 2, 16, 8, seed=7, state_std=0.05, n_states=len(lengths))
    o, s = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], 0.25, d["s0"], cu_seqlens=cu)
    for i in range(len(lengths)):
        lo, hi = cu[i], cu[i + 1]
        o_i, s_i = O.gated_delta_sequence(d["q"][0, lo:hi], d["k"][0, lo:hi], d["v"][0, lo:hi],
                                          d["g"][0, lo:hi].exp(), d["beta"][0, lo:hi], 0.25, d["s0"][i])
        assert torch.equal(o[0, lo:hi], o_i) and torch.equal(s[i], s_i)


# ------------------------------------------------------------------------------------------ row-local parts


def test_conv_one_hot_taps_shift_the_input_and_keep_the_last_raw_rows():
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(10, 6, generator=gen)
    hist = torch.randn(6, 3, generator=gen)
    full = torch.cat((hist.T, x))  # [13, 6] oldest first
    for tap in range(4):
        w = torch.zeros(6, 1, 4)
        w[:, 0, tap] = 1.0
        y, new_hist = O.causal_conv1d(x, w, hist)
        # tap j multiplies x_{t - 3 + j}
        assert torch.allclose(y, F.silu(full[tap : tap + 10]), atol=1e-6)
        assert torch.equal(new_hist, full[-3:].T)
    # fewer rows than the history: the new history still ends with the newest raw rows
    y, new_hist = O.causal_conv1d(x[:2], torch.ones(6, 1, 4), hist)
    assert torch.equal(new_hist, torch.cat((hist[:, 2:], x[:2].T), -1))


def test_l2norm_closed_form():
    x = torch.randn(7, 3, 64, generator=torch.Generator().manual_seed(9)) * 3
    y = O.l2norm(x)
    n = x.double().norm(dim=-1)
    assert torch.allclose(y.double().norm(dim=-1), n / torch.sqrt(n**2 + 1e-6), rtol=1e-6)
    assert torch.allclose(y / y.norm(dim=-1, keepdim=True), x / x.norm(dim=-1, keepdim=True), atol=1e-6)


def test_gate_closed_form():
    a = torch.tensor([-3.0, 0.0, 2.0, 25.0])
    b = torch.tensor([-2.0, 0.0, 1.0, 4.0])
    decay, beta = O.gate(a, b, torch.zeros(4), torch.zeros(4))
    want = [math.exp(-math.log1p(math.exp(x))) if x <= 20 else math.exp(-x) for x in a.tolist()]
    assert torch.allclose(decay.double(), torch.tensor(want, dtype=torch.float64), rtol=1e-6)
    assert torch.allclose(beta, 1 / (1 + torch.exp(-b)))
    # A_log scales the log decay by exp(A_log); dt_bias shifts a
    d2, _ = O.gate(a, b, torch.full((4,), math.log(2.0)), torch.ones(4))
    assert torch.allclose(d2.log(), -2 * F.softplus(a + 1), rtol=1e-5)


def test_gated_norm_limits():
    gen = torch.Generator().manual_seed(10)
    o = torch.randn(5, 4, 32, generator=gen)
    w = 1 + 0.1 * torch.randn(32, generator=gen)
    big = torch.full((5, 4, 32), 60.0)
    y = O.gated_rmsnorm(o, big, w, 1e-5, torch.float32)
    rms = o.pow(2).mean(-1, keepdim=True).add(1e-5).rsqrt()
    assert torch.allclose(y, o * rms * w * 60.0, rtol=1e-5)
    assert torch.equal(O.gated_rmsnorm(o, torch.zeros_like(o), w, 1e-5, torch.float32), torch.zeros_like(o))


def test_chunk_tables_match_the_reference_literals():
    """Expected values of servers/sgl/tests/test_gdn_graph_support.py:17-30."""
    cu, chunks = O.chunk_tables([64] * 4)
    assert cu == [0, 64, 128, 192, 256] and chunks == [[0, 0], [1, 0], [2, 0], [3, 0]]
    assert O.chunk_tables([64])[0] == [0, 64]
    for lengths in ([1], [64], [65], [5, 63, 64, 130], [200, 1, 128]):
        cu, chunks = O.chunk_tables(lengths)
        assert cu == np.cumsum([0] + lengths).tolist()
        want = [[i, j] for i, n in enumerate(lengths) for j in range(math.ceil(n / 64))]
        assert chunks == want


# ------------------------------------------------------------------------------------------- whole layer


def _layer_weights(heads, hd, dim, seed):
    gen = torch.Generator().manual_seed(seed)
    inner = heads * hd
    return {
        "in_proj": 0.2 * torch.randn(4 * inner + 2 * heads, dim, generator=gen),
        "conv": 0.2 * torch.randn(3 * inner, 1, 4, generator=gen),
        "out_weight": 1 + 0.1 * torch.randn(hd, generator=gen),
        "A_log": 0.2 * torch.randn(heads, generator=gen),
        "dt_bias": 0.2 * torch.randn(heads, generator=gen),
        "wo": 0.2 * torch.randn(dim, inner, generator=gen),
    }


@pytest.mark.parametrize("k", [1, 3, 5])
def test_layer_prefill_equals_prefill_plus_decode_steps(k):
    """The layer-level form of model/tests/test_reference_lm.py:126-136 (rtol = atol = 1e-5)."""
    w = _layer_weights(2, 16, 24, seed=11)
    x = torch.randn(12, 24, generator=torch.Generator().manual_seed(12))
    full, conv_f, state_f, _ = O.gdn_layer(x, w, heads=2, head_dim=16)
    y, conv, state, _ = O.gdn_layer(x[: 12 - k], w, heads=2, head_dim=16)
    parts = [y]
    for row in range(12 - k, 12):
        y, conv, state, _ = O.gdn_layer(x[row : row + 1], w, conv, state, heads=2, head_dim=16)
        parts.append(y)
    torch.testing.assert_close(torch.cat(parts), full, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(state, state_f, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(conv, conv_f, rtol=1e-5, atol=1e-5)  # in_proj over 1 vs 12 rows rounds apart


def test_layer_captures_are_named_like_the_golden_dump():
    w = _layer_weights(2, 16, 24, seed=13)
    _, _, _, cap = O.gdn_layer(torch.randn(3, 24), w, heads=2, head_dim=16)
    for name in ("gdn_conv", "gdn_q", "gdn_k", "gdn_v", "gdn_decay", "gdn_beta", "gdn_recurrent", "gdn_gated",
                 "gdn_state", "gdn_conv_state"):
        assert name in cap


def test_fused_decode_step_equals_the_layer_parts():
    """One step of the fused block == conv -> L2 -> gate -> recurrence -> gated norm, stated per stream."""
    gen = torch.Generator().manual_seed(14)
    B, hk, hv, K = 3, 1, 2, 16
    C = 2 * hk * K + hv * K
    x = torch.randn(B, C, generator=gen)
    z = torch.randn(B, hv, K, generator=gen)
    a, b = torch.randn(B, hv, generator=gen), torch.randn(B, hv, generator=gen)
    w = 0.2 * torch.randn(C, 4, generator=gen)
    cache = torch.randn(B, C, 3, generator=gen)
    s0 = 0.02 * torch.randn(B, hv, K, K, generator=gen)
    nw = 1 + 0.1 * torch.randn(K, generator=gen)
    out, new_cache, s = O.fused_decode_step(x, z, a, b, w, cache, s0, nw, torch.zeros(hv), torch.zeros(hv), hk)
    for i in range(B):
        conv = F.silu((torch.cat((cache[i], x[i][:, None]), -1) * w).sum(-1))
        q = O.l2norm(conv[: hk * K].view(1, hk, K))
        kk = O.l2norm(conv[hk * K : 2 * hk * K].view(1, hk, K))
        v = conv[2 * hk * K :].view(1, hv, K)
        o, st = O.recurrence_np(q, kk, v, -F.softplus(a[i : i + 1]), b[i : i + 1].sigmoid(), K**-0.5, s0[i])
        y = torch.tensor(o[0], dtype=torch.float32)
        y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + 1e-6) * nw * F.silu(z[i])
        assert rel_err(out[i], y) < 1e-5 and rel_err(s[i], st) < 1e-5
        assert torch.equal(new_cache[i], torch.cat((cache[i][:, 1:], x[i][:, None]), -1))


# ----------------------------------------------------------------------------------------- planted mistakes


def _mutant(kind):
    """Copies of gated_delta_sequence with one plausible mistake each."""

    def run(q, k, v, decay, beta, scale, state):
        hk, hv = k.shape[1], v.shape[1]
        q, k, v = q.float(), k.float(), v.float()
        if hv != hk:
            if kind == "interleaved_groups":
                q, k = q.repeat(1, hv // hk, 1), k.repeat(1, hv // hk, 1)
            else:
                q, k = q.repeat_interleave(hv // hk, 1), k.repeat_interleave(hv // hk, 1)
        outs = []
        for t in range(q.shape[0]):
            if kind != "prediction_before_decay":
                state = state * decay[t, :, None, None]
            if kind == "key_major_state":
                pred = (state * k[t, :, :, None]).sum(-2)
            else:
                pred = (state * k[t, :, None, :]).sum(-1)
            if kind == "prediction_before_decay":
                state = state * decay[t, :, None, None]
            delta = beta[t, :, None] * (v[t] - pred)
            if kind == "no_beta":
                delta = v[t] - pred
            state = state + delta[:, :, None] * k[t, :, None, :]
            read = state if kind != "read_before_update" else state - delta[:, :, None] * k[t, :, None, :]
            outs.append((read * (q[t] * scale)[:, None, :]).sum(-1))
        return torch.stack(outs), state

    return run


def _pins_pass(fn) -> bool:
    """The brute-force and grouped-head pins applied to a candidate recurrence."""
    q, k, v, g, b, s0 = _seq(24, 2, 4, 16, 16, seed=15)
    o, s = fn(q, k, v, g.exp(), b, 0.25, s0)
    o_n, s_n = O.recurrence_np(q, k, v, g, b, 0.25, s0)
    return rel_err(o, o_n) < 1e-5 and rel_err(s, s_n) < 1e-5


@pytest.mark.parametrize("kind", ["interleaved_groups", "prediction_before_decay", "key_major_state", "no_beta",
                                  "read_before_update"])
def test_planted_mistakes_are_caught(kind):
    assert _pins_pass(O.gated_delta_sequence)
    assert not _pins_pass(_mutant(kind))


# ------------------------------------------------------------------------------ residual routing (lm.py:384)


def test_attnres_route_closed_forms():
    gen = torch.Generator().manual_seed(91)
    srcs = [torch.randn(5, 64, generator=gen) for _ in range(4)]
    q = torch.randn(64, generator=gen)
    # one source: softmax over one logit is 1
    assert torch.allclose(O.attnres_route(srcs[:1], q, 1e-5), srcs[0], atol=1e-6)
    # zero query: equal weights, the mean of the sources
    assert torch.allclose(O.attnres_route(srcs, torch.zeros(64), 1e-5), torch.stack(srcs).mean(0), atol=1e-6)
    # a query along one source's direction of one token, scaled up: that source wins for that token
    big = 200.0 * srcs[2][3] / srcs[2][3].norm()
    assert torch.allclose(O.attnres_route(srcs, big, 1e-5)[3], srcs[2][3], atol=1e-4)
    # the order of the sources does not matter
    perm = [srcs[i] for i in (2, 0, 3, 1)]
    assert torch.allclose(O.attnres_route(srcs, q, 1e-5), O.attnres_route(perm, q, 1e-5), atol=1e-6)
    # torch restatement == float64 statement (fp32 inputs)
    assert rel_err(O.attnres_route(srcs, q, 1e-5), O.attnres_route_np(srcs, q, 1e-5)) < 1e-6
    # a stacked bank is the same as the list
    assert torch.equal(O.attnres_route(torch.stack(srcs), q, 1e-5), O.attnres_route(srcs, q, 1e-5))


def test_accent_shift_pins():
    """The accent shift restatement (layers/accent.py:37, 62) against what the mathematics fixes."""
    gen = torch.Generator().manual_seed(93)
    rows, n_in, n_out, ranks = 6, 48, 40, (4, 8)
    K = sum(ranks)
    x = torch.randn(rows, n_in, generator=gen)
    W = torch.randn(n_out, n_in, generator=gen)
    down, up = torch.randn(K, n_in, generator=gen), torch.randn(K, n_out, generator=gen)
    y = x @ W.T
    # a zero mask row leaves y exactly as it was
    assert torch.equal(O.accent_shift(x, down, up, torch.zeros(rows, K), y), y)
    # one-hot factors: adapter column k reads input i and writes 2 x its masked value to output j
    d1, u1 = torch.zeros(K, n_in), torch.zeros(K, n_out)
    d1[3, 7], u1[3, 11] = 1.0, 2.0
    m = torch.zeros(rows, K)
    m[:, 3] = torch.arange(rows, dtype=torch.float32) - 2.0
    want = torch.zeros(rows, n_out)
    want[:, 11] = 2.0 * m[:, 3] * x[:, 7]
    assert torch.equal(O.accent_shift(x, d1, u1, m), want)
    # a constant mask row alpha on adapter a's columns is the merged weight W + alpha * up_a^T down_a
    alpha = torch.tensor([0.5, -1.25, 0.0, 2.0, 1.0, 0.75], dtype=torch.float64)
    cols = slice(ranks[0], K)  # the second adapter
    mask = torch.zeros(rows, K, dtype=torch.float64)
    mask[:, cols] = alpha[:, None]
    merged = np.stack([O._f64(x[r]) @ (O._f64(W) + alpha[r].item() * O._f64(up[cols]).T @ O._f64(down[cols])).T
                       for r in range(rows)])
    got = O.accent_shift_np(x, down, up, mask.numpy(), O._f64(x) @ O._f64(W).T)
    assert np.abs(got - merged).max() < 1e-9 * np.abs(merged).max()
    # adapters on disjoint columns add
    ma, mb = torch.zeros(rows, K), torch.zeros(rows, K)
    ma[:, : ranks[0]] = torch.rand(rows, 1, generator=gen)
    mb[:, ranks[0]:] = torch.rand(rows, 1, generator=gen)
    both = O.accent_shift_np(x, down, up, (ma + mb).numpy())
    assert np.abs(both - O.accent_shift_np(x, down, up, ma.numpy()) - O.accent_shift_np(x, down, up, mb.numpy())).max() < 1e-9
    # the torch restatement (fp32) agrees with the float64 statement
    assert rel_err(O.accent_shift(x, down, up, ma + mb, y), O.accent_shift_np(x, down, up, ma + mb, y)) < 1e-5


# ---------------------------------------------------------------------- whole layer: a known answer (lm.py:556)


def _kat_layer():
    """A layer whose answer is fixed by hand: 2 heads of 4, in_proj = identity (the input row is the projection
    q|k|v | z | a | b in lm.py:562's order), conv taking only the current input (newest tap 1), A_log =
    dt_bias = 0, wo = identity. Three tokens:
      1. a = -30, b = +30 (decay 1, beta 1), q = k = 3 e_h (unit after SiLU and L2), small v: from the zero
         state o_h = beta (k.q) scale silu(v_h), small enough that the norm's eps (1e-5) matters;
      2. the same k, a new v, beta 1: the delta rule overwrites, S_h = silu(v2_h) k_h^T; head 0 reads along
         k (o = S k scale), head 1 reads along an orthogonal q (o = 0);
      3. a = 0 (decay exp(-softplus(0)) = 1/2), b = -30 (beta 0): S halves, q = k.
    Returns (x, weights, expected y, expected final state, expected conv history (the three raw inputs))."""
    heads, hd = 2, 4
    inner = heads * hd
    e = torch.eye(hd, dtype=torch.float64)
    s3 = 3.0 * torch.sigmoid(torch.tensor(3.0, dtype=torch.float64))  # silu(3)
    c = s3 / torch.sqrt(s3 * s3 + 1e-6)  # |l2norm(silu(3) e)|
    silu = lambda t: t * torch.sigmoid(t)  # noqa: E731
    v1 = torch.tensor([[0.02, -0.01, 0.03, 0.01], [0.01, 0.02, -0.02, 0.005]], dtype=torch.float64)
    v2 = torch.tensor([[0.03, 0.01, -0.02, 0.02], [-0.01, 0.015, 0.02, 0.01]], dtype=torch.float64)
    v3 = torch.tensor([[0.5, -0.5, 0.5, 0.5], [0.2, 0.1, 0.3, -0.4]], dtype=torch.float64)
    z = torch.tensor([[[1.0, -1.0, 2.0, 0.5], [0.5, 1.0, -2.0, 3.0]],
                      [[-0.5, 2.0, 1.0, 1.0], [1.0, 1.0, 1.0, 1.0]],
                      [[2.0, 0.25, -1.0, 1.5], [-1.5, 0.5, 2.5, 1.0]]], dtype=torch.float64)
    k_dirs = [e[0], e[1]]
    q_rows = [[e[0], e[1]], [e[0], e[2]], [e[0], e[1]]]
    v_rows = [v1, v2, v3]
    ab = [(-30.0, 30.0), (-30.0, 30.0), (0.0, -30.0)]
    rows = []
    for t in range(3):
        q = torch.cat([3.0 * q_rows[t][h] for h in range(heads)])
        k = torch.cat([3.0 * k_dirs[h] for h in range(heads)])
        rows.append(torch.cat([q, k, v_rows[t].reshape(-1), z[t].reshape(-1), torch.tensor([ab[t][0]] * heads,
                    dtype=torch.float64), torch.tensor([ab[t][1]] * heads, dtype=torch.float64)]))
    x = torch.stack(rows)
    w_out = torch.tensor([1.0, 2.0, 0.5, 1.5], dtype=torch.float64)
    conv = torch.zeros(3 * inner, 1, 4, dtype=torch.float64)
    conv[:, 0, 3] = 1.0
    weights = {"in_proj": torch.eye(x.shape[1], dtype=torch.float64), "conv": conv, "out_weight": w_out,
               "A_log": torch.zeros(heads, dtype=torch.float64), "dt_bias": torch.zeros(heads, dtype=torch.float64),
               "wo": torch.eye(inner, dtype=torch.float64)}
    # closed forms: beta = sigmoid(30) and decay = exp(-softplus(-30)) are 1 to 1e-13; scale = 1/2
    scale = hd**-0.5
    half = torch.exp(-torch.log(torch.tensor(2.0, dtype=torch.float64)))  # exp(-softplus(0))
    o = torch.zeros(3, heads, hd, dtype=torch.float64)
    for h in range(heads):
        o[0, h] = silu(v1[h]) * c * c * scale
    o[1, 0] = silu(v2[0]) * c * c * scale  # q along k
    o[1, 1] = 0.0  # q orthogonal to k
    for h in range(heads):
        o[2, h] = half * silu(v2[h]) * c * c * scale
    y = o / torch.sqrt(o.pow(2).mean(-1, keepdim=True) + 1e-5) * w_out * silu(z)
    state = torch.stack([half * torch.outer(silu(v2[h]), c * k_dirs[h]) for h in range(heads)])
    history = x[:, : 3 * inner].T  # the last W-1 = 3 raw q|k|v inputs, oldest first
    return x, weights, y.reshape(3, inner), state, history


def _layer_variant(kind):
    """gdn_layer's composition with one plausible mistake (its ops from the oracle's own parts)."""

    def run(x, w, heads=2, head_dim=4, eps=1e-5):
        hd, inner = head_dim, heads * head_dim
        projection = F.linear(x, w["in_proj"])
        qkv, z, aa, b = projection.split((3 * inner, inner, heads, heads), -1)
        if kind == "a_b_swapped":
            aa, b = b, aa
        conv, conv_state = O.causal_conv1d(qkv, w["conv"], None)
        if kind == "no_conv_silu":
            conv = F.silu(conv)  # a second SiLU stands for a misplaced one
        q, k, v = [part.reshape(len(x), heads, hd).double() for part in conv.split(inner, -1)]
        if kind == "q_k_swapped":
            q, k = k, q
        q = q * torch.rsqrt(q.square().sum(-1, keepdim=True) + 1e-6)
        k = k * torch.rsqrt(k.square().sum(-1, keepdim=True) + 1e-6)
        decay, beta = O.gate(aa, b, w["A_log"], w["dt_bias"])
        o, state = O.gated_delta_sequence(q, k, v, decay.double(), beta.double(),
                                          1.0 if kind == "no_scale" else hd**-0.5,
                                          torch.zeros(heads, hd, hd, dtype=torch.float64))
        o = o.double()
        zz = z.reshape(len(x), heads, hd)
        norm = o / torch.sqrt(o.pow(2).mean(-1, keepdim=True) + (1e-6 if kind == "eps_1e-6" else eps))
        gate_z = zz if kind == "z_not_silu" else F.silu(zz)
        return (norm * w["out_weight"] * gate_z).reshape(len(x), inner), state, conv_state

    return run


def test_layer_known_answer():
    """gdn_layer against the hand-fixed answer of _kat_layer: outputs, final state and conv history."""
    x, w, y_want, s_want, hist_want = _kat_layer()
    y, conv_state, state, cap = O.gdn_layer(x, w, heads=2, head_dim=4)
    # (gdn_layer runs the recurrence in float32, as lm.py:569 does: agreement to float32 rounding)
    assert rel_err(y, y_want) < 1e-6, rel_err(y, y_want)
    assert rel_err(state, s_want) < 1e-6
    assert torch.equal(conv_state, hist_want)
    assert rel_err(cap["gdn_gated"], y_want) < 1e-6  # wo = identity


@pytest.mark.parametrize("kind", ["a_b_swapped", "eps_1e-6", "z_not_silu", "q_k_swapped", "no_conv_silu",
                                  "no_scale"])
def test_layer_planted_mistakes_fail_the_known_answer(kind):
    x, w, y_want, s_want, _ = _kat_layer()
    y, state, _ = _layer_variant("none")(x, w)
    assert rel_err(y, y_want) < 1e-6 and rel_err(state, s_want) < 1e-6  # the unmutated composition passes
    y, state, _ = _layer_variant(kind)(x, w)
    assert rel_err(y, y_want) > 1e-3 or rel_err(state, s_want) > 1e-3, kind
