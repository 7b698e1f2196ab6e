"""The kernels as PyTorch operators: ``torch.ops.zgdn.*``.

Each operator is a thin registration (``torch.library.custom_op``) over the C-ABI call in ``ops.py``: the
real implementation validates, allocates with the caching allocator and launches on the current stream;
the fake (meta) implementation states the output shapes, so the operators trace under ``torch.compile`` /
``FakeTensorMode`` and can be captured into graphs like any aten op. Operators that update a cache or a
state in place declare it in ``mutates_args``.

| operator | replaces |
|---|---|
| ``zgdn::recurrent_fwd`` | token loop lm.py:574-583 (and serving decode windows, gdn.py:329-355) |
| ``zgdn::decode_step`` | one lm.py:574-583 step for B streams, state in place |
| ``zgdn::chunk_fwd`` | FLA ``chunk_gated_delta_rule_fwd`` (gdn.py:418-434) |
| ``zgdn::fused_decode_step`` | lm.py:563-587 for one new row per stream, conv cache and state in place |
| ``zgdn::serving_decode_step`` | the serving layer's static decode (gdn.py:329-355) on per-slot caches in place |
| ``zgdn::attnres_route`` | ``full_attnres_route`` (lm.py:384-389; zonos3.py:99-113) |
| ``zgdn::accent_shift`` | ``accent_shift`` / ``apply_accent`` (layers/accent.py:25-62) |
| ``zgdn::causal_conv1d`` | FLA ``causal_conv1d_fwd`` (gdn.py:403-414); lm.py:563-568 |
| ``zgdn::l2norm`` | FLA ``l2norm_fwd`` (gdn.py:416-417); lm.py:570-571 |
| ``zgdn::sigmoid`` | FLA ``fused_beta_sigmoid_fwd`` (gdn.py:423); lm.py:573 |
| ``zgdn::gated_rmsnorm`` | FLA ``layer_norm_gated_fwd`` (gdn.py:435-445); lm.py:584-587 |
"""

from __future__ import annotations

import importlib
from typing import List, Optional, Tuple

import torch
from torch import Tensor

ops = importlib.import_module(__package__ + ".ops")

NS = "zgdn"


def _n_states(B: int, cu_seqlens: Optional[Tensor]) -> int:
    return B if cu_seqlens is None else cu_seqlens.shape[0] - 1


# ------------------------------------------------------------------------------------------ recurrent path


@torch.library.custom_op(f"{NS}::recurrent_fwd", mutates_args=())
def recurrent_fwd(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, scale: Optional[float] = None,
                  initial_state: Optional[Tensor] = None, cu_seqlens: Optional[Tensor] = None,
                  A_log: Optional[Tensor] = None, dt_bias: Optional[Tensor] = None,
                  use_qk_l2norm: bool = False) -> Tuple[Tensor, Tensor]:
    return ops.recurrent_fwd(q, k, v, g, beta, scale=scale, initial_state=initial_state, cu_seqlens=cu_seqlens,
                             A_log=A_log, dt_bias=dt_bias, use_qk_l2norm=use_qk_l2norm)


@recurrent_fwd.register_fake
def _(q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None, A_log=None, dt_bias=None,
      use_qk_l2norm=False):
    B, T, Hk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    return (v.new_empty(B, T, Hv, V), q.new_empty(_n_states(B, cu_seqlens), Hv, V, K, dtype=torch.float32))


@torch.library.custom_op(f"{NS}::decode_step", mutates_args=("state",))
def decode_step(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, state: Tensor,
                scale: Optional[float] = None) -> Tensor:
    return ops.decode_step(q, k, v, g, beta, state, scale=scale)


@decode_step.register_fake
def _(q, k, v, g, beta, state, scale=None):
    return v.new_empty(v.shape)


# -------------------------------------------------------------------------------------------- chunked path


@torch.library.custom_op(f"{NS}::chunk_fwd", mutates_args=())
def chunk_fwd(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, scale: Optional[float] = None,
              initial_state: Optional[Tensor] = None, cu_seqlens: Optional[Tensor] = None,
              chunk_indices: Optional[Tensor] = None, A_log: Optional[Tensor] = None,
              dt_bias: Optional[Tensor] = None, use_qk_l2norm: bool = False) -> Tuple[Tensor, Tensor]:
    return ops.chunk_fwd(q, k, v, g, beta, scale=scale, initial_state=initial_state, cu_seqlens=cu_seqlens,
                         chunk_indices=chunk_indices, A_log=A_log, dt_bias=dt_bias, use_qk_l2norm=use_qk_l2norm)


@chunk_fwd.register_fake
def _(q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None, chunk_indices=None, A_log=None,
      dt_bias=None, use_qk_l2norm=False):
    B, T, Hk, K = q.shape
    Hv, V = v.shape[2], v.shape[3]
    return (v.new_empty(B, T, Hv, V, dtype=torch.bfloat16),
            q.new_empty(_n_states(B, cu_seqlens), Hv, V, K, dtype=torch.float32))


# -------------------------------------------------------------------------------------------- fused block


@torch.library.custom_op(f"{NS}::fused_decode_step", mutates_args=("conv_cache", "state"))
def fused_decode_step(x_qkv: Tensor, z: Tensor, a: Tensor, b: Tensor, conv_weight: Tensor, conv_cache: Tensor,
                      state: Tensor, norm_weight: Tensor, A_log: Tensor, dt_bias: Tensor, eps: float = 1e-6,
                      scale: Optional[float] = None, round_qk: bool = False) -> Tensor:
    return ops.fused_decode_step(x_qkv, z, a, b, conv_weight, conv_cache, state, norm_weight, A_log, dt_bias,
                                 eps=eps, scale=scale, round_qk=round_qk)


@fused_decode_step.register_fake
def _(x_qkv, z, a, b, conv_weight, conv_cache, state, norm_weight, A_log, dt_bias, eps=1e-6, scale=None,
      round_qk=False):
    return z.new_empty(z.shape, dtype=x_qkv.dtype)


@torch.library.custom_op(f"{NS}::serving_decode_step",
                         mutates_args=("conv_live", "conv_commit", "state_live", "state_commit", "window", "win_len"))
def serving_decode_step(mixed: Tensor, x_hidden: Tensor, slots: Tensor, conv_weight: Tensor, conv_live: Tensor,
                        conv_commit: Tensor, state_live: Tensor, state_commit: Tensor, window: Tensor,
                        win_len: Tensor, norm_weight: Tensor, A_log: Tensor, dt_bias: Tensor, eps: float = 1e-5,
                        scale: Optional[float] = None, round_qk: bool = True) -> Tensor:
    return ops.serving_decode_step(mixed, x_hidden, slots, conv_weight, conv_live, conv_commit, state_live,
                                   state_commit, window, win_len, norm_weight, A_log, dt_bias, eps=eps, scale=scale,
                                   round_qk=round_qk)


@serving_decode_step.register_fake
def _(mixed, x_hidden, slots, conv_weight, conv_live, conv_commit, state_live, state_commit, window, win_len,
      norm_weight, A_log, dt_bias, eps=1e-5, scale=None, round_qk=True):
    return mixed.new_empty(mixed.shape[0], state_live.shape[1], state_live.shape[3])


@torch.library.custom_op(f"{NS}::attnres_route", mutates_args=())
def attnres_route(sources: List[Tensor], query: Tensor, eps: float) -> Tensor:
    return ops.attnres_route(sources, query, eps)


@attnres_route.register_fake
def _(sources, query, eps):
    return sources[0].new_empty(sources[0].shape)


@torch.library.custom_op(f"{NS}::accent_shift", mutates_args=())
def accent_shift(x: Tensor, down: Tensor, up: Tensor, mask: Tensor, y: Optional[Tensor] = None) -> Tensor:
    return ops.accent_shift(x, down, up, mask, y=y)


@accent_shift.register_fake
def _(x, down, up, mask, y=None):
    return x.new_empty(x.shape[0], up.shape[1])


# --------------------------------------------------------------------------------------------- row ops


@torch.library.custom_op(f"{NS}::causal_conv1d", mutates_args=())
def causal_conv1d(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None, initial_state: Optional[Tensor] = None,
                  cu_seqlens: Optional[Tensor] = None, chunk_indices: Optional[Tensor] = None,
                  activation: Optional[str] = "silu", state_width: Optional[int] = None) -> Tuple[Tensor, Tensor]:
    return ops.causal_conv1d(x, weight, bias=bias, initial_state=initial_state, output_final_state=True,
                             activation=activation, cu_seqlens=cu_seqlens, chunk_indices=chunk_indices,
                             state_width=state_width)


@causal_conv1d.register_fake
def _(x, weight, bias=None, initial_state=None, cu_seqlens=None, chunk_indices=None, activation="silu",
      state_width=None):
    W = weight.shape[-1]
    sw = W if state_width is None else int(state_width)
    return x.new_empty(x.shape), x.new_empty(_n_states(x.shape[0], cu_seqlens), x.shape[2], sw)


@torch.library.custom_op(f"{NS}::l2norm", mutates_args=())
def l2norm(x: Tensor, eps: float = 1e-6) -> Tuple[Tensor, Tensor]:
    return ops.l2norm(x, eps=eps)


@l2norm.register_fake
def _(x, eps=1e-6):
    return x.new_empty(x.shape), x.new_empty(x.shape[:-1], dtype=torch.float32)


@torch.library.custom_op(f"{NS}::sigmoid", mutates_args=())
def sigmoid(x: Tensor, scale: float = 1.0) -> Tensor:
    return ops.sigmoid(x, scale=scale)


@sigmoid.register_fake
def _(x, scale=1.0):
    return x.new_empty(x.shape, dtype=torch.float32)


@torch.library.custom_op(f"{NS}::gated_rmsnorm", mutates_args=())
def gated_rmsnorm(x: Tensor, g: Tensor, weight: Tensor, eps: float = 1e-5) -> Tuple[Tensor, Tensor]:
    return ops.gated_rmsnorm(x, g, weight, eps=eps)


@gated_rmsnorm.register_fake
def _(x, g, weight, eps=1e-5):
    return x.new_empty(x.shape), x.new_empty(x.shape[:-1], dtype=torch.float32)


OPERATORS = ("recurrent_fwd", "decode_step", "chunk_fwd", "fused_decode_step", "serving_decode_step",
             "attnres_route", "accent_shift", "causal_conv1d", "l2norm", "sigmoid", "gated_rmsnorm")
