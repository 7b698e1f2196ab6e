"""CPU restatement of ZONOS3-Mini's gated-DeltaNet (GDN) layer -- TEST INFRASTRUCTURE, not product code.

Used only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg, to check results.

Two independent statements of the same mathematics live here:

* ``torch`` restatements that follow the reference's own PyTorch code op for op (same ops, same order, same
  dtype casts), so that on identical inputs they round like the reference:
  ``model/src/zonos3/reference/lm.py:556-602`` (``Zonos3LM._gdn``), generalised to batches, packed
  (``cu_seqlens``) sequences and grouped value heads (v-head ``h`` reads k-head ``h // (Hv // Hk)``, the
  mapping of ``servers/mlx/src/zonos3_mlx/models/gdn_kernel.py:16-18``).
* ``numpy`` float64 statements written from the mathematics instead of the reference's code: a plain triple
  loop (``recurrence_np``) and the chunked WY/UT form (``chunked_np``) that FLA's
  ``chunk_gated_delta_rule_fwd`` computes (called at ``servers/sgl/src/zonos3_sgl/models/gdn.py:418-434``).
  Agreement between the loop and the chunked form is a mathematical identity, and the tests use it to pin
  both.

The residual routing that feeds and consumes each GDN layer (``attnres_route``, ``lm.py:384-389``) has a
torch restatement and a float64 one (``attnres_route_np``); its pins are closed forms (one source returns
it, a zero query averages the sources, a dominant logit selects its source, order of sources is
irrelevant) and the float64 statement.

The accent adapter shift of the mixer's projections (``accent_shift``, ``layers/accent.py:25-62``) has a
torch restatement and a float64 one (``accent_shift_np``); pins: a zero mask leaves y unchanged, one-hot
factors move a scaled input column to an output column, adapters on disjoint columns add, and a constant
mask row equals the merged weight ``W + alpha * up_a^T down_a`` (the "base + alpha * adapter" merge of
``models/accent_adapters.py:5-8``).

Conventions (all from the reference):
  q, k   [.., T, Hk, K]       v [.., T, Hv, V]       g (log decay), beta [.., T, Hv]
  state  [N, Hv, V, K] float32, value-major (FLA ``state_v_first=True``; lm.py:577, gdn.py:427)
  conv history [D, W-1], oldest column first (lm.py:563-568; servers/web/src/gpu/kernels/gdn_conv.wgsl:1-3)
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "CHUNK",
    "chunk_tables",
    "causal_conv1d",
    "l2norm",
    "gate",
    "gated_delta_sequence",
    "gated_delta_recurrence",
    "gated_rmsnorm",
    "gdn_layer",
    "fused_decode_step",
    "attnres_route",
    "attnres_route_np",
    "accent_shift",
    "accent_shift_np",
    "recurrence_np",
    "chunked_np",
    "make_inputs",
]

CHUNK = 64  # servers/sgl/src/zonos3_sgl/models/gdn.py:46


# ----------------------------------------------------------------------------------------------- index tables


def chunk_tables(lengths: list[int], chunk: int = CHUNK) -> tuple[list[int], list[list[int]]]:
    """(cu_seqlens [n+1], chunk indices [chunks, 2] = (sequence, chunk within it)) of packed sequences.

    Follows ``servers/sgl/src/zonos3_sgl/models/gdn.py:49-59`` (the values FLA's ``prepare_chunk_indices``
    derives); returned as plain lists (the reference copies them to the device as int32)."""
    cu = [0]
    chunks: list[list[int]] = []
    for i, n in enumerate(lengths):
        cu.append(cu[-1] + n)
        for j in range(-(-n // chunk)):
            chunks.append([i, j])
    return cu, chunks


# ------------------------------------------------------------------------------------- row-local parts (torch)


def causal_conv1d(x: torch.Tensor, weight: torch.Tensor, history: torch.Tensor | None = None):
    """Depthwise causal conv + SiLU of one sequence, and the new history.

    ``lm.py:563-568``: x [T, D] (raw q|k|v channels), weight [D, 1, W] or [D, W] with ``weight[..., 0]`` the
    oldest tap, history [D, W-1] (oldest first, zeros when absent). Returns (silu(conv) [T, D] in x.dtype,
    new history [D, W-1] = the last W-1 raw inputs)."""
    if weight.dim() == 2:
        weight = weight.unsqueeze(1)
    channels, _, kernel = weight.shape
    if history is None:
        history = torch.zeros(channels, kernel - 1, dtype=x.dtype, device=x.device)
    sequence = torch.cat((history, x.T), -1)
    conv = F.conv1d(sequence.unsqueeze(0), weight, groups=channels)
    conv = F.silu(conv.squeeze(0).T)
    return conv, sequence[:, -(kernel - 1) :].clone()


def l2norm(x: torch.Tensor) -> torch.Tensor:
    """``x * rsqrt(sum(x^2) + 1e-6)`` over the last dim in float32 (``lm.py:569-571``)."""
    x = x.float()
    return x * torch.rsqrt(x.square().sum(-1, keepdim=True) + 1e-6)


def gate(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """(decay alpha, beta) in float32: ``exp(-exp(A_log) * softplus(a + dt_bias))``, ``sigmoid(b)``
    (``lm.py:572-573``; softplus is torch's, identity above 20)."""
    decay = torch.exp(-A_log.float().exp() * F.softplus(a.float() + dt_bias.float()))
    return decay, b.float().sigmoid()


def gated_rmsnorm(o: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float, dtype: torch.dtype):
    """Output gate ``rms_norm(o.to(dtype)) * w * silu(z)``, product in float32 then cast (``lm.py:584-587``).

    o, z [..., V]; weight [V]. The norm runs in ``dtype`` (``F.rms_norm`` on the cast recurrent output)."""
    recurrent = o.to(dtype)
    normalized = F.rms_norm(recurrent, (recurrent.shape[-1],), weight=weight.to(dtype), eps=eps)
    return (normalized.float() * F.silu(z.float())).to(dtype)


# ----------------------------------------------------------------------------------------- recurrence (torch)


def gated_delta_sequence(q, k, v, decay, beta, scale: float, state):
    """The token loop of ``lm.py:574-583`` for one sequence, with grouped value heads.

    q, k [T, Hk, K]; v [T, Hv, V]; decay, beta [T, Hv] float32; state [Hv, V, K] float32.
    Per token: ``S *= decay; p = S.k; delta = beta (v - p); S += delta k^T; o = S.(q scale)``.
    Returns (o [T, Hv, V] float32, final state)."""
    hk, hv = k.shape[1], v.shape[1]
    if hv % hk:
        raise ValueError("value heads must be a multiple of key heads")
    q, k, v = q.float(), k.float(), v.float()
    if hv != hk:  # gdn_kernel.py:16-18: v-head h reads k-head h // (Hv // Hk)
        q = q.repeat_interleave(hv // hk, dim=1)
        k = k.repeat_interleave(hv // hk, dim=1)
    outputs = []
    for token in range(q.shape[0]):
        state = state * decay[token, :, None, None]
        prediction = (state * k[token, :, None, :]).sum(-1)
        delta = beta[token, :, None] * (v[token] - prediction)
        state = state + delta[:, :, None] * k[token, :, None, :]
        outputs.append((state * (q[token] * scale)[:, None, :]).sum(-1))
    if outputs:
        out = torch.stack(outputs)
    else:
        out = torch.zeros(0, hv, v.shape[-1])
    return out, state


def gated_delta_recurrence(q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None):
    """Batched / packed form of ``gated_delta_sequence`` in FLA's calling convention (gdn.py:418-434).

    q, k [B, T, Hk, K]; v [B, T, Hv, V]; g = log decay and beta [B, T, Hv]; initial_state [N, Hv, V, K]
    (N = B, or the number of packed sequences when ``cu_seqlens`` is given with B == 1); zeros when None.
    Returns (o [B, T, Hv, V] float32, final state [N, Hv, V, K] float32)."""
    B, T, hk, K = k.shape
    hv, V = v.shape[2], v.shape[3]
    scale = K**-0.5 if scale is None else scale
    if cu_seqlens is None:
        bounds = [(b, 0, T) for b in range(B)]
    else:
        if B != 1:
            raise ValueError("packed sequences need B == 1")
        cu = [int(c) for c in cu_seqlens]
        bounds = [(0, cu[i], cu[i + 1]) for i in range(len(cu) - 1)]
    n = len(bounds)
    if initial_state is None:
        initial_state = torch.zeros(n, hv, V, K)
    out = torch.zeros(B, T, hv, V)
    finals = []
    for i, (b, lo, hi) in enumerate(bounds):
        o, s = gated_delta_sequence(
            q[b, lo:hi], k[b, lo:hi], v[b, lo:hi], g[b, lo:hi].float().exp(), beta[b, lo:hi].float(), scale,
            initial_state[i].float(),
        )
        out[b, lo:hi] = o
        finals.append(s)
    return out, torch.stack(finals)


# ------------------------------------------------------------------------------------------ whole layer (torch)


def gdn_layer(x, weights: dict, conv_state=None, gdn_state=None, heads=4, head_dim=128, eps=1e-5):
    """The whole GDN layer of ``lm.py:556-602`` for one sequence (same ops, same casts).

    weights: ``in_proj`` [4*inner + 2*heads, dim], ``conv`` [3*inner, 1, W], ``out_weight`` [head_dim],
    ``A_log`` [heads], ``dt_bias`` [heads], ``wo`` [dim, inner]. Returns (y [T, dim], conv_state [3*inner, W-1],
    gdn_state [heads, V, K] float32, captures dict named as lm.py:588-601)."""
    hd, inner = head_dim, heads * head_dim
    projection = F.linear(x, weights["in_proj"])
    qkv, z, aa, b = projection.split((3 * inner, inner, heads, heads), -1)
    conv, conv_state = causal_conv1d(qkv, weights["conv"], conv_state)
    q, k, v = [part.reshape(len(x), heads, hd).float() for part in conv.split(inner, -1)]
    q = q * torch.rsqrt(q.square().sum(-1, keepdim=True) + 1e-6)
    k = k * torch.rsqrt(k.square().sum(-1, keepdim=True) + 1e-6)
    decay, beta = gate(aa, b, weights["A_log"], weights["dt_bias"])
    if gdn_state is None:
        gdn_state = torch.zeros(heads, hd, hd, dtype=torch.float32, device=x.device)
    o, state = gated_delta_sequence(q, k, v, decay, beta, hd**-0.5, gdn_state)
    recurrent = o.to(x.dtype)
    gated = gated_rmsnorm(recurrent, z.reshape(len(x), heads, hd), weights["out_weight"], eps, x.dtype)
    gated = gated.reshape(len(x), inner)
    captures = {
        "gdn_conv": conv, "gdn_q": q, "gdn_k": k, "gdn_v": v, "gdn_decay": decay, "gdn_beta": beta,
        "gdn_recurrent": recurrent, "gdn_gated": gated, "gdn_state": state, "gdn_conv_state": conv_state,
    }
    return F.linear(gated, weights["wo"]), conv_state, state, captures


def fused_decode_step(x_qkv, z, a, b, conv_w, conv_cache, state, norm_w, A_log, dt_bias, hk, eps=1e-6,
                      scale=None, round_qk=False):
    """One single-token step of the GDN block for a batch of independent streams (``lm.py:563-587`` with
    T = 1 per stream, grouped value heads).

    x_qkv [B, Hk*K + Hk*K + Hv*V] raw projected q|k|v; z [B, Hv, V]; a, b [B, Hv]; conv_w [C, W];
    conv_cache [B, C, W-1] (oldest first); state [B, Hv, V, K] float32; norm_w [V]. ``round_qk``: the
    normalised q, k rounded to x's dtype, as the serving layer's l2norm operator returns them
    (servers/sgl/src/zonos3_sgl/models/gdn.py:416-417).
    Returns (out [B, Hv, V] in x's dtype, new conv cache, new state)."""
    B, C = x_qkv.shape
    hv, V = z.shape[1], z.shape[2]
    K = (C - hv * V) // (2 * hk)
    scale = K**-0.5 if scale is None else scale
    outs, caches, states = [], [], []
    for i in range(B):
        conv, hist = causal_conv1d(x_qkv[i : i + 1], conv_w, conv_cache[i])
        conv = conv[0]
        q = l2norm(conv[: hk * K].reshape(1, hk, K))
        k = l2norm(conv[hk * K : 2 * hk * K].reshape(1, hk, K))
        if round_qk:
            q, k = q.to(x_qkv.dtype).float(), k.to(x_qkv.dtype).float()
        v = conv[2 * hk * K :].reshape(1, hv, V).float()
        decay, beta = gate(a[i : i + 1], b[i : i + 1], A_log, dt_bias)
        o, s = gated_delta_sequence(q, k, v, decay, beta, scale, state[i].float())
        outs.append(gated_rmsnorm(o[0], z[i], norm_w, eps, x_qkv.dtype))
        caches.append(hist)
        states.append(s)
    return torch.stack(outs), torch.stack(caches), torch.stack(states)


def attnres_route(sources, query, eps):
    """Full Attention-Residual routing, ``lm.py:384-389`` (same ops, same casts): the sources stacked, keys =
    weightless rms_norm of each source, logits = sum(keys * query) in float32, softmax over the sources cast
    back to the sources' dtype, the weighted sum of the raw sources. sources: a list of [T, dim] tensors or a
    [S, T, dim] tensor."""
    bank = torch.stack(list(sources)) if not torch.is_tensor(sources) else sources
    keys = F.rms_norm(bank, (bank.shape[-1],), eps=eps)
    scores = (keys * query).sum(-1, dtype=torch.float32)
    weights = scores.softmax(0).to(bank.dtype)
    return (bank * weights.unsqueeze(-1)).sum(0)


def attnres_route_np(sources, query, eps) -> np.ndarray:
    """The same equation in float64 with no intermediate rounding (an independent statement)."""
    bank = np.stack([_f64(s) for s in sources])
    q = _f64(query)
    keys = bank / np.sqrt((bank**2).mean(-1, keepdims=True) + eps)
    logits = (keys * q).sum(-1)
    w = np.exp(logits - logits.max(0, keepdims=True))
    w /= w.sum(0, keepdims=True)
    return (bank * w[..., None]).sum(0)


def accent_shift(x, down, up, mask, y=None):
    """The accent adapter shift of a projection output, ``servers/sgl/src/zonos3_sgl/layers/accent.py:37``
    (``((x @ down.T) * mask) @ up``, same ops in the inputs' dtype), added to ``y`` as ``apply_accent`` does
    (``accent.py:62``) when ``y`` is given."""
    shift = ((x @ down.T) * mask) @ up
    return shift if y is None else y + shift


def accent_shift_np(x, down, up, mask, y=None) -> np.ndarray:
    """The same equation in float64 with no intermediate rounding (an independent statement)."""
    shift = ((_f64(x) @ _f64(down).T) * _f64(mask)) @ _f64(up)
    return shift if y is None else _f64(y) + shift


# ---------------------------------------------------------------------------- float64 statements (numpy)


def _f64(x) -> np.ndarray:
    if torch.is_tensor(x):
        return x.detach().cpu().double().numpy().copy()
    return np.array(x, dtype=np.float64)


def _group(hk: int, hv: int) -> int:
    if hv % hk:
        raise ValueError("value heads must be a multiple of key heads")
    return hv // hk


def recurrence_np(q, k, v, g, beta, scale, state):
    """Brute-force float64 triple loop of the delta rule for one sequence, written from the update
    ``S_t = a_t S_{t-1} (I - b_t k_t k_t^T) + b_t v_t k_t^T``, ``o_t = scale S_t q_t`` (state [Hv, V, K]).

    q, k [T, Hk, K]; v [T, Hv, V]; g (log decay), beta [T, Hv]. Returns (o [T, Hv, V], state)."""
    q, k, v, g, beta, S = (_f64(t) for t in (q, k, v, g, beta, state))
    T, hk, K = k.shape
    hv, V = v.shape[1], v.shape[2]
    rep = _group(hk, hv)
    o = np.zeros((T, hv, V))
    for t in range(T):
        for h in range(hv):
            kk, qq = k[t, h // rep], q[t, h // rep]
            a = math.exp(g[t, h])
            for j in range(V):
                row = S[h, j] * a
                p = float(np.dot(row, kk))
                row = row + beta[t, h] * (v[t, h, j] - p) * kk
                S[h, j] = row
                o[t, h, j] = scale * float(np.dot(row, qq))
    return o, S


def chunked_np(q, k, v, g, beta, scale, state, chunk=CHUNK):
    """The chunked WY/UT form of the same recurrence in float64, one sequence (state [Hv, V, K]).

    Per chunk of L <= ``chunk`` tokens with in-chunk cumulative log decay G (G_i = g_1 + .. + g_i), start
    state S0 and, per head:
      A[i, j] = beta_i exp(G_i - G_j) k_i.k_j (j < i),  T = (I + A)^-1
      W = T diag(beta exp(G)) K,   Ubar = T diag(beta) V,   U = Ubar - W S0^T       (the corrected values)
      O = scale (diag(exp(G)) Q S0^T + (Q K^T * exp(G_i - G_j) [j <= i]) U)
      S_L = exp(G_L) S0 + U^T diag(exp(G_L - G)) K
    This is the algorithm FLA's chunk_gated_delta_rule_fwd runs (gdn.py:418-434, chunk_size=64)."""
    q, k, v, g, beta, S = (_f64(t) for t in (q, k, v, g, beta, state))
    T, hk, K = k.shape
    hv, V = v.shape[1], v.shape[2]
    rep = _group(hk, hv)
    o = np.zeros((T, hv, V))
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        L = c1 - c0
        for h in range(hv):
            Q, Kc, Vc = q[c0:c1, h // rep], k[c0:c1, h // rep], v[c0:c1, h]
            G = np.cumsum(g[c0:c1, h])
            bt = beta[c0:c1, h]
            diff = G[:, None] - G[None, :]
            lower = np.tril(np.ones((L, L)), -1)
            gam = np.exp(np.where(lower > 0, diff, -np.inf))
            A = bt[:, None] * gam * (Kc @ Kc.T)
            Tm = np.linalg.inv(np.eye(L) + A)
            W = Tm @ ((bt * np.exp(G))[:, None] * Kc)
            Ubar = Tm @ (bt[:, None] * Vc)
            S0 = S[h]
            U = Ubar - W @ S0.T
            incl = np.exp(np.where(np.tril(np.ones((L, L))) > 0, diff, -np.inf))
            o[c0:c1, h] = scale * (np.exp(G)[:, None] * (Q @ S0.T) + ((Q @ Kc.T) * incl) @ U)
            S[h] = math.exp(G[-1]) * S0 + U.T @ (np.exp(G[-1] - G)[:, None] * Kc)
    return o, S


# ------------------------------------------------------------------------------------------ seeded inputs


def make_inputs(B, T, hk, hv, K, V, seed, dtype=torch.float32, state_std=0.0, n_states=None):
    """Seeded synthetic inputs of the configurations: q, k ~ N(0,1) then L2-normalised in float32
    (``rsqrt(sum x^2 + 1e-6)``); v ~ N(0,1); g = -softplus(N(0,1)); beta = sigmoid(N(0,1)); initial state
    ~ N(0, state_std) (zeros when 0). q, k, v are cast to ``dtype`` after normalisation; g, beta stay float32.
    Returns a dict of CPU tensors."""
    gen = torch.Generator().manual_seed(seed)
    q = l2norm(torch.randn(B, T, hk, K, generator=gen)).to(dtype)
    k = l2norm(torch.randn(B, T, hk, K, generator=gen)).to(dtype)
    v = torch.randn(B, T, hv, V, generator=gen).to(dtype)
    g = -F.softplus(torch.randn(B, T, hv, generator=gen))
    beta = torch.randn(B, T, hv, generator=gen).sigmoid()
    n = B if n_states is None else n_states
    if state_std:
        s0 = torch.randn(n, hv, V, K, generator=gen) * state_std
    else:
        s0 = torch.zeros(n, hv, V, K)
    return {"q": q, "k": k, "v": v, "g": g, "beta": beta, "s0": s0}
