"""Drop-in for the reference model's GDN layer, ``Zonos3LM._gdn(self, x, layer, cache)``
(``model/src/zonos3/reference/lm.py:556-602``), on the MI355X kernels.

``gdn(self, x, layer, cache)`` has the method's signature and effects: it reads the layer's weights from
``self.layers[layer].attention`` (``in_proj``, ``conv``, ``out_weight``, ``A_log``, ``dt_bias``, ``wo``),
runs the projections through ``self._lin`` (so accent adapters still apply), replaces
``cache.conv_state[layer]`` ([3 * inner, W - 1], x's dtype, oldest first) and ``cache.gdn_state[layer]``
([heads, V, K] float32, value-major) with new tensors, saves the same ``gdn_*`` captures when
``self._capture`` is set, and returns the ``wo`` projection. Bind it with ``patch(model)`` (one instance)
or ``Zonos3LM._gdn = gdn`` (the class).

Data path: one row (decode) -> the fused decode-block kernel (conv, SiLU, L2, gate, update, gated norm in
one launch); more rows -> the conv kernel, then the chunked kernels (bf16 MFMA for bf16 at head size 128, fp32
arithmetic for fp32 and for 64-wide heads; the recurrent kernel for other head sizes), with the q/k L2-norm and
the gate formed in the kernel, then the gated-RMSNorm kernel. A bf16 model without accent adapters (``_lin`` is
then F.linear, lm.py:505-507) runs its projections on this package's GEMM, in_proj with the conv fused into its
epilogue.
"""

from __future__ import annotations

import types

import torch
import torch.nn.functional as F

from . import ops


def _weights(a):
    heads = a.A_log.numel()
    hd = a.out_weight.numel()
    conv_w = a.conv.weight
    return heads, hd, conv_w.reshape(conv_w.shape[0], conv_w.shape[-1])


def gdn(self, x: torch.Tensor, layer: int, cache) -> torch.Tensor:
    """``Zonos3LM._gdn`` (lm.py:556-602) on the HIP kernels: x [T, dim] -> [T, dim]."""
    a, p = self.layers[layer].attention, f"layers.{layer}.attention."
    heads, hd, conv_w = _weights(a)
    inner = heads * hd
    channels = 3 * inner
    kernel = conv_w.shape[-1]
    n = len(x)
    dev, dt = x.device, x.dtype
    # the package's projections: a bf16 model whose _lin is plain F.linear (no accent adapters loaded), shapes the
    # GEMM takes (K a multiple of 128, the conv over whole 128-column tiles)
    own_proj = (dt == torch.bfloat16 and getattr(self, "_accents", None) is None and kernel == 4 and n > 1
                and x.shape[-1] % 128 == 0 and inner % 128 == 0 and a.in_proj.weight.dtype == dt
                and a.wo.weight.dtype == dt)
    history = cache.conv_state.get(layer)  # None before the first call: the kernels read zeros
    state = cache.gdn_state.get(layer)
    A_log, dt_bias = a.A_log.float().contiguous(), a.dt_bias.float().contiguous()
    conv_w = conv_w.to(dt).contiguous()
    norm_w = a.out_weight.to(dt).contiguous()
    capture = getattr(self, "_capture", None) is not None

    if own_proj:
        h0 = None if history is None else history.reshape(channels, kernel - 1).to(dt).contiguous()
        projection, new_hist = ops.in_proj_conv(x, a.in_proj.weight, conv_w, channels, initial_state=h0)
        conv2d = projection[:, :channels]  # silu(conv(q|k|v)): the conv ran in the projection's epilogue
        _, z, aa, b = projection.split((3 * inner, inner, heads, heads), -1)
    else:
        projection = self._lin(p + "in_proj", x, a.in_proj.weight)
        qkv, z, aa, b = projection.split((3 * inner, inner, heads, heads), -1)

    if n == 1 and hd == 128 and kernel == 4 and not capture:
        # the fused decode block updates conv history and state in place: work on fresh copies
        if history is None:
            new_hist = torch.zeros(1, channels, kernel - 1, dtype=dt, device=dev)
        else:
            new_hist = history.reshape(1, channels, kernel - 1).clone()
        if state is None:
            new_state = torch.zeros(1, heads, hd, hd, dtype=torch.float32, device=dev)
        else:
            new_state = state.reshape(1, heads, hd, hd).float().clone()
        gated = ops.fused_decode_step(qkv.contiguous(), z.reshape(1, heads, hd).contiguous(),
                                      aa.contiguous(), b.contiguous(), conv_w, new_hist, new_state, norm_w, A_log,
                                      dt_bias, eps=1e-5)
        cache.conv_state[layer] = new_hist.reshape(channels, kernel - 1)
        cache.gdn_state[layer] = new_state.reshape(heads, hd, hd)
        return self._lin(p + "wo", gated.reshape(1, inner), a.wo.weight)

    # q|k|v, z, a and b are read in place from the projection rows; the conv output's q, k, v column slices
    # likewise
    if not own_proj:
        h0 = None if history is None else history.reshape(1, channels, kernel - 1).contiguous()
        conv, new_hist = ops.causal_conv1d(qkv.unsqueeze(0), conv_w, initial_state=h0, activation="silu",
                                           state_width=kernel - 1)
        conv2d = conv[0]
    q, k, v = (part.unflatten(-1, (heads, hd)).unsqueeze(0) for part in conv2d.split(inner, -1))
    s0 = None if state is None else state.reshape(1, heads, hd, hd).float().contiguous()
    kw = dict(initial_state=s0, A_log=A_log, dt_bias=dt_bias, use_qk_l2norm=True)
    if dt in (torch.bfloat16, torch.float32) and hd in (64, 128):
        o, new_state = ops.chunk_fwd(q, k, v, aa.unsqueeze(0), b.unsqueeze(0), beta_is_logit=True, **kw)
        beta = None
    else:
        beta = ops.sigmoid(b.contiguous(), out_dtype=torch.float32).reshape(1, n, heads)
        o, new_state = ops.recurrent_fwd(q.contiguous(), k.contiguous(), v.contiguous(),
                                         aa.float().reshape(1, n, heads).contiguous(), beta, out_dtype=dt, **kw)
    recurrent = o.reshape(n, heads, hd).to(dt)
    gated, _ = ops.gated_rmsnorm(recurrent, z.unflatten(-1, (heads, hd)), norm_w, eps=1e-5)
    gated = gated.reshape(n, inner)
    cache.conv_state[layer] = new_hist.reshape(channels, kernel - 1)
    cache.gdn_state[layer] = new_state.reshape(heads, hd, hd)
    if capture:
        qn, _ = ops.l2norm(q.reshape(n, heads, hd).contiguous(), out_dtype=torch.float32)
        kn, _ = ops.l2norm(k.reshape(n, heads, hd).contiguous(), out_dtype=torch.float32)
        if beta is None:
            beta = ops.sigmoid(b.contiguous(), out_dtype=torch.float32)
        decay = torch.exp(-A_log.exp() * F.softplus(aa.float() + dt_bias))  # diagnostics only
        for name, tensor in (
            ("gdn_conv", conv2d), ("gdn_q", qn), ("gdn_k", kn), ("gdn_v", v.reshape(n, heads, hd).float()),
            ("gdn_decay", decay), ("gdn_beta", beta.reshape(n, heads)), ("gdn_recurrent", recurrent),
            ("gdn_gated", gated), ("gdn_state", cache.gdn_state[layer]),
            ("gdn_conv_state", cache.conv_state[layer]),
        ):
            self._save(f"{name}_{layer}", tensor)
    if own_proj:
        return ops.gemm_nt(gated, a.wo.weight)
    return self._lin(p + "wo", gated, a.wo.weight)


def patch(model) -> None:
    """Route one model instance's GDN layers through ``gdn``."""
    model._gdn = types.MethodType(gdn, model)
