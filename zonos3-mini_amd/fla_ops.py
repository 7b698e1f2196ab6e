"""The serving layer's operator seam, on the MI355X kernels.

``OriginalGDN`` binds five FLA forward functions as instance attributes
(``servers/sgl/src/zonos3_sgl/models/gdn.py:123-133``) and calls them from ``_run_packed``
(``gdn.py:395-450``); the reference's own test swaps exactly these attributes
(``servers/sgl/tests/test_accent_adapters.py:593-631``). The functions below keep those keyword
signatures and return arities, so ``install(layer)`` makes an ``OriginalGDN`` run on this package:

  _conv_fwd        causal_conv1d_fwd(x, weight, bias, residual, initial_state, output_final_state,
                                     activation, cu_seqlens, chunk_indices, BT) -> (y, final_state)
  _l2norm_fwd      l2norm_fwd(x) -> (y, rstd)
  _beta_fwd        fused_beta_sigmoid_fwd(b, scale) -> beta
  _delta_rule_fwd  chunk_gated_delta_rule_fwd(q, k, v, g, beta, scale, initial_state, ...) -> 6-tuple with
                   o at [1] and the final state at [3]
  _norm_fwd        layer_norm_gated_fwd(x, g, weight, bias, activation, eps, residual, residual_dtype,
                                        is_rms_norm) -> tuple with y at [0]

Unsupported options (a residual, a norm bias, layer norm instead of RMS norm, key-major states, chunks
other than 64) raise ``RuntimeError`` instead of computing something else.
"""

from __future__ import annotations

import torch

from . import ops

CHUNK = ops.CHUNK


def causal_conv1d_fwd(x, weight, bias=None, residual=None, initial_state=None, output_final_state=False,
                      activation=None, cu_seqlens=None, chunk_indices=None, BT=64, **unsupported):
    """Depthwise causal conv1d (+ SiLU) over packed sequences (gdn.py:403-414).

    x [B, T, D] (packed: B == 1 with ``cu_seqlens``); weight [D, W]; initial_state [N, D, W] holds the last W
    raw inputs before each sequence (oldest first; the last W-1 are the taps' history). Returns
    (y [B, T, D], final state [N, D, W] or None)."""
    if residual is not None:
        raise RuntimeError("causal_conv1d_fwd: a residual input is not supported")
    if unsupported:
        raise RuntimeError(f"causal_conv1d_fwd: unsupported arguments {sorted(unsupported)}")
    if BT != CHUNK and chunk_indices is not None:
        raise RuntimeError(f"causal_conv1d_fwd: chunk indices of {BT}-row chunks (supported: {CHUNK})")
    W = weight.shape[-1]
    return ops.causal_conv1d(x, weight, bias, initial_state=initial_state, output_final_state=output_final_state,
                             activation=activation, cu_seqlens=cu_seqlens, chunk_indices=chunk_indices, state_width=W)


def l2norm_fwd(x, eps=1e-6, output_dtype=None):
    """x * rsqrt(sum x^2 + eps) over the last dim (gdn.py:416-417). Returns (y, rstd)."""
    return ops.l2norm(x, eps=eps, out_dtype=output_dtype)


def fused_beta_sigmoid_fwd(b, scale=1.0):
    """beta = sigmoid(b) * scale (gdn.py:423), in float32 (the reference recurrence's beta is float32,
    ``model/src/zonos3/reference/lm.py:573``)."""
    return ops.sigmoid(b, scale=scale, out_dtype=torch.float32)


def chunk_gated_delta_rule_fwd(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=True,
                               state_v_first=True, cu_seqlens=None, chunk_indices=None, use_gate_in_kernel=False,
                               A_log=None, dt_bias=None, chunk_size=64, use_qk_l2norm_in_kernel=False,
                               **unsupported):
    """Gated delta rule over packed sequences (gdn.py:418-434). Returns a 6-tuple whose [1] is o
    [B, T, Hv, V] (q's dtype) and [3] the final state [N, Hv, V, K] float32 (value-major).

    bf16 or fp32 inputs with K == V of 64 or 128 run the chunked kernels; other head sizes the recurrent one."""
    if unsupported:
        raise RuntimeError(f"chunk_gated_delta_rule_fwd: unsupported arguments {sorted(unsupported)}")
    if not state_v_first:
        raise RuntimeError("chunk_gated_delta_rule_fwd: only value-major states (state_v_first=True)")
    if chunk_size != CHUNK:
        raise RuntimeError(f"chunk_gated_delta_rule_fwd: chunk_size {chunk_size} (supported: {CHUNK})")
    if use_gate_in_kernel != (A_log is not None):
        raise RuntimeError("chunk_gated_delta_rule_fwd: use_gate_in_kernel needs A_log and dt_bias")
    if g.dtype != beta.dtype:  # the kernels take one dtype for both ([T, H] tensors)
        g, beta = g.float().contiguous(), beta.float().contiguous()
    if initial_state is not None and initial_state.dtype != torch.float32:
        initial_state = initial_state.float()
    kw = dict(scale=scale, initial_state=initial_state, output_final_state=output_final_state,
              cu_seqlens=cu_seqlens, A_log=A_log, dt_bias=dt_bias, use_qk_l2norm=use_qk_l2norm_in_kernel)
    chunked = (q.dtype in (torch.bfloat16, torch.float32) and q.shape[-1] == v.shape[-1]
               and q.shape[-1] in (64, 128))
    if chunked:
        o, final = ops.chunk_fwd(q, k, v, g, beta, chunk_indices=chunk_indices, **kw)
    else:
        o, final = ops.recurrent_fwd(q, k, v, g, beta, out_dtype=q.dtype, **kw)
    return None, o, None, final, None, None


def layer_norm_gated_fwd(x, g, weight, bias=None, activation="swish", eps=1e-5, residual=None,
                         residual_dtype=None, is_rms_norm=True, **unsupported):
    """Gated RMSNorm y = (rms_norm(x) * weight) * silu(g) (gdn.py:435-445). Returns (y, None, rstd, None)."""
    if unsupported:
        raise RuntimeError(f"layer_norm_gated_fwd: unsupported arguments {sorted(unsupported)}")
    if bias is not None or residual is not None or not is_rms_norm:
        raise RuntimeError("layer_norm_gated_fwd: supported is RMS norm without bias or residual")
    if activation not in ("swish", "silu"):
        raise RuntimeError(f"layer_norm_gated_fwd: activation {activation!r} (supported: swish)")
    y, rstd = ops.gated_rmsnorm(x, g, weight.to(x.dtype), eps=eps)
    return y, None, rstd, None


def install(layer) -> None:
    """Point an ``OriginalGDN``'s five operator attributes (gdn.py:129-133) at this package."""
    layer._conv_fwd = causal_conv1d_fwd
    layer._l2norm_fwd = l2norm_fwd
    layer._beta_fwd = fused_beta_sigmoid_fwd
    layer._delta_rule_fwd = chunk_gated_delta_rule_fwd
    layer._norm_fwd = layer_norm_gated_fwd
