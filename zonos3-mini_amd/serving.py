"""The serving layer's GDN mixer with request-local state, on the MI355X kernels.

Mirrors ``OriginalGDN`` (``servers/sgl/src/zonos3_sgl/models/gdn.py:115-450``): the per-slot caches
(``allocate_cache``, gdn.py:150-160), the ragged eager path (``forward``, gdn.py:235-327), the static-shape
decode and prefill paths that CUDA/HIP graphs capture (gdn.py:329-393), the engine hooks (gdn.py:163-233)
and ``_run_packed`` (gdn.py:395-450) through the five operator attributes, which are bound to this
package's kernels (``fla_ops``).

Exactness model (the reference's, kept): committed per-slot states end at a multiple of 64 rows of the
request, and an eager forward replays the unfinished chunk (the tail, kept raw in a per-slot 64-row window)
in front of the new rows, so prefill/extend cuts never change the chunk boundaries.

The decode fast path. The reference's static decode recomputes each request's whole 64-row window through
the chunk kernels on every step (gdn.py:329-355). Here every slot also keeps its *live* states, the conv
history and the recurrent state after the request's last row, and a decode step (static or eager) is one
single-row pass from them: ``in_proj`` on the new rows, one serving decode launch (conv/SiLU/L2/gate/delta
rule/gated norm on the slots' caches in place, q/k rounded like the serving operators return them), ``wo``.
The same launch writes the raw row into the slot's window and, when the window fills up, the new live states
to the committed ones, so the eager path's tail replay stays what it was. Window rows past the fill are
unspecified (only the eager replay reads windows, and only their filled rows). Live states are
set by every path: the eager passes' final states (the uncommitted tail pass included: it has exact
lengths), and the static prefill's window pass, whose zero padding rows are made exact no-ops of the state
(decay 1, beta 0) so its final state is the state after the real rows.

Engine integration: ``batch_source`` is a zero-argument callable returning the current batch (in the
reference, ``get_global_ctx().batch``, gdn.py:236); ``accent`` optionally supplies the accent adapters'
``accent_mask()`` / ``apply_accent(op, x, y, mask)`` (``zonos3_sgl.layers.accent``). Batches and requests
are read by the reference's attribute names: ``is_decode``, ``padded_size``, ``gdn_prefill``, ``reqs``,
``padded_reqs``; ``table_idx``, ``extend_len``, ``cached_len``, ``device_len``, ``uid``, ``is_cfg_uncond``.
"""

from __future__ import annotations

import importlib
from dataclasses import dataclass
from typing import Callable, Optional

import torch
import torch.nn.functional as F

ops = importlib.import_module(__package__ + ".ops")
fla_ops = importlib.import_module(__package__ + ".fla_ops")

CHUNK = 64  # the training kernel's chunk length (gdn.py:46)
HEADS, HEAD_DIM = 4, 128
CONV_CHANNELS, CONV_WIDTH = 3 * HEADS * HEAD_DIM, 4  # q | k | v channels of the depthwise conv
SPLIT = [CONV_CHANNELS, HEADS * HEAD_DIM, HEADS, HEADS]  # in_proj rows: q|k|v, z, a, b (gdn.py:402)
NORM_EPS = 1e-5  # the gated RMSNorm's eps in the serving layer (gdn.py:441)
_MASKED_GATE = -30000.0  # a, b of padding rows: softplus -> 0 (decay 1) and sigmoid -> 0 (beta 0)


def device_tensor(values, dtype: torch.dtype, device) -> torch.Tensor:
    """A host list as a ``device`` tensor in one non-blocking copy from pinned memory (the reference's
    ``make_device_tensor``, ``servers/sgl/src/zonos3_sgl/utils/torch_utils.py:23-37``)."""
    host = torch.tensor(values, dtype=dtype)
    device = torch.device(device)
    if device.type == "cpu":
        return host
    return host.pin_memory().to(device, non_blocking=True)


def chunk_tables(lengths: list[int], device) -> tuple[torch.Tensor, torch.Tensor]:
    """(cu_seqlens int32 [n + 1], chunk indices int32 [chunks, 2] = (sequence, chunk within it)) of packed
    sequences of ``lengths`` rows, in one non-blocking copy (gdn.py:49-59)."""
    cu = [0]
    pairs: list[int] = []
    for i, n in enumerate(lengths):
        cu.append(cu[-1] + n)
        for j in range(-(-n // CHUNK)):
            pairs += (i, j)
    packed = device_tensor(cu + pairs, torch.int32, device)
    return packed[: len(cu)], packed[len(cu):].view(-1, 2)


@dataclass(frozen=True)
class PrefillLayout:
    """Static tables of a padded prefill (gdn.py:62-104): request i owns ``CHUNK * (whole[i] + 1)`` batch
    rows from its start, its ``whole[i]`` complete chunks, then a 64-row window for its last ``n_i % 64``
    rows (zeros after them)."""

    whole_rows: Optional[torch.Tensor]  # [sum 64 * whole] long: batch rows of the complete chunks
    whole_reqs: Optional[torch.Tensor]  # [k] long: batch index of each request with complete chunks
    whole_cu: Optional[torch.Tensor]
    whole_chunks: Optional[torch.Tensor]
    window_rows: torch.Tensor  # [b * 64] long: batch rows of the windows
    window_base: torch.Tensor  # [b] long: 64 * whole[i], the request's rows before its window
    window_cu: torch.Tensor
    window_chunks: torch.Tensor

    @classmethod
    def build(cls, whole: list[int], device) -> "PrefillLayout":
        starts, at = [], 0
        for w in whole:
            starts.append(at)
            at += CHUNK * (w + 1)
        with_whole = [i for i, w in enumerate(whole) if w]
        whole_rows = [r for i in with_whole for r in range(starts[i], starts[i] + CHUNK * whole[i])]
        window_rows = [r for i, w in enumerate(whole)
                       for r in range(starts[i] + CHUNK * w, starts[i] + CHUNK * (w + 1))]
        whole_cu = whole_chunks = None
        if with_whole:
            whole_cu, whole_chunks = chunk_tables([CHUNK * whole[i] for i in with_whole], device)
        window_cu, window_chunks = chunk_tables([CHUNK] * len(whole), device)
        return cls(
            whole_rows=device_tensor(whole_rows, torch.long, device) if with_whole else None,
            whole_reqs=device_tensor(with_whole, torch.long, device) if with_whole else None,
            whole_cu=whole_cu,
            whole_chunks=whole_chunks,
            window_rows=device_tensor(window_rows, torch.long, device),
            window_base=device_tensor([CHUNK * w for w in whole], torch.long, device),
            window_cu=window_cu,
            window_chunks=window_chunks,
        )

    def tensors(self) -> list[torch.Tensor]:
        """The static index tensors of the layout (what a captured graph reads)."""
        return [t for t in (self.whole_cu, self.whole_chunks, self.window_cu, self.window_chunks) if t is not None]


@dataclass
class PrefillInputs:
    """A padded prefill's inputs (the batch's ``gdn_prefill``): the layout and the per-replay buffers."""

    layout: PrefillLayout
    slots: torch.Tensor  # [b] long: the requests' table slots
    lengths: torch.Tensor  # [b] long: the requests' real rows


class _Weight:
    def __init__(self, shape):
        self.weight = torch.empty(shape)


class OriginalGDN:
    """The four-head GDN mixer with per-slot inference state (gdn.py:115-450). Weights are plain
    attributes with the reference's names and shapes, set by the caller's loader."""

    def __init__(self, config, layer_id: int, batch_source: Optional[Callable] = None, accent=None):
        fla_ops.install(self)  # _conv_fwd, _l2norm_fwd, _beta_fwd, _delta_rule_fwd, _norm_fwd
        self._layer_id = layer_id
        self._hidden = config.hidden_size
        self.in_proj = _Weight((sum(SPLIT), config.hidden_size))
        self.conv = _Weight((CONV_CHANNELS, 1, CONV_WIDTH))
        self.out_weight = torch.empty(HEAD_DIM)
        self.A_log = torch.empty(HEADS, dtype=torch.float32)
        self.dt_bias = torch.empty(HEADS, dtype=torch.float32)
        self.wo = _Weight((config.hidden_size, HEADS * HEAD_DIM))
        self._batch_source = batch_source
        self._accent = accent
        self._capacity = 0
        self._static_mode = False
        self._graph_slots: Optional[torch.Tensor] = None
        self._static_rows: dict[int, torch.Tensor] = {}

    # ------------------------------------------------------------------------------------------ caches

    def allocate_cache(self, capacity: int, device, dtype: torch.dtype) -> None:
        """Per-slot buffers (gdn.py:150-160) plus the live states of the decode fast path."""
        if self._capacity:
            raise RuntimeError("GDN cache already allocated")
        z = dict(device=device)
        self._conv_state = torch.zeros((capacity, CONV_CHANNELS, CONV_WIDTH), dtype=dtype, **z)
        self._recurrent_state = torch.zeros((capacity, HEADS, HEAD_DIM, HEAD_DIM), dtype=torch.float32, **z)
        self._window = torch.zeros((capacity, CHUNK, self._hidden), dtype=dtype, **z)  # rows [0, win_len) real
        self._win_len = torch.zeros((capacity,), dtype=torch.int32, **z)
        self._live_conv = torch.zeros_like(self._conv_state)
        self._live_state = torch.zeros_like(self._recurrent_state)
        self._owners: list = [None] * capacity
        self._lengths = [0] * capacity
        self._capacity = capacity

    # ----------------------------------------------------------------------------------- engine hooks

    @staticmethod
    def static_tables(device, bs_list) -> dict[int, tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
        """Per batch size: (cu_seqlens of bs 64-row windows, their chunk indices, row offsets bs * 64)
        (gdn.py:163-172). The fast decode path reads only the row offsets."""
        tables = {}
        for bs in bs_list:
            cu, chunks = chunk_tables([CHUNK] * bs, device)
            tables[bs] = (cu, chunks, torch.arange(bs, device=device, dtype=torch.long) * CHUNK)
        return tables

    def enable_graph_decode(self, slots: torch.Tensor, tables) -> None:
        """``slots``: the engine's static [max_bs] int64 buffer of table slots of the padded decode batch,
        filled before every capture / replay; ``tables`` from ``static_tables`` (gdn.py:174-183)."""
        self._graph_slots = slots
        for bs, (_, _, rows) in tables.items():
            self._static_rows[bs] = rows

    @staticmethod
    def pin_fla_cache(static_tensors, pinned: dict) -> int:
        """The reference keeps FLA's memoised index tensors alive for captured graphs (gdn.py:185-222).
        These operators memoise nothing, so there is nothing to pin: returns 0."""
        return 0

    def set_static_mode(self, enabled: bool) -> None:
        """While set, decode batches take the static-shape path (graph warm-up and capture)."""
        self._static_mode = bool(enabled)

    def note_graph_forward(self, reqs) -> None:
        """Host-side mirrors after a replayed decode step or prefill (gdn.py:228-233)."""
        for r in reqs:
            self._owners[r.table_idx] = (r.uid, r.is_cfg_uncond)
            self._lengths[r.table_idx] = r.device_len

    # ----------------------------------------------------------------------------------------- forward

    def _current_batch(self):
        if self._batch_source is None:
            raise RuntimeError("GDN forward needs a batch source (the engine's current batch)")
        return self._batch_source()

    def _accent_mask(self):
        return None if self._accent is None else self._accent.accent_mask()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """gdn.py:235-327: static decode / static prefill when the batch asks for them, else the ragged
        eager path over the batch's requests (validated before any cache changes)."""
        batch = self._current_batch()
        if batch.is_decode and self._static_mode:
            return self._forward_decode_static(x, batch.padded_size)
        if getattr(batch, "gdn_prefill", None) is not None:
            return self._forward_prefill_static(x, batch.gdn_prefill)
        if x.is_cuda and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("GDN ragged path cannot be captured; graphs use the static window / prefill paths")
        reqs = batch.reqs
        if len(batch.padded_reqs) != len(reqs):
            raise RuntimeError("GDN eager path does not accept dummy graph-padding requests")
        slots = [r.table_idx for r in reqs]
        lengths = [r.extend_len for r in reqs]
        if (not self._capacity or len(set(slots)) != len(slots)
                or any(s < 0 or s >= self._capacity for s in slots)
                or any(n <= 0 for n in lengths) or sum(lengths) != x.shape[0]):
            raise RuntimeError("Invalid GDN request slots or packed lengths")
        if batch.is_decode and any(n != 1 for n in lengths):
            raise RuntimeError("GDN decode expects one new token per request")
        owners = [(r.uid, r.is_cfg_uncond) for r in reqs]
        for r, owner in zip(reqs, owners):  # a KV-only prefix hit has no recurrent state: rejected
            s = r.table_idx
            if r.cached_len and (self._owners[s] != owner or self._lengths[s] != r.cached_len):
                raise RuntimeError(
                    f"GDN layer {self._layer_id}: missing/stale state at slot {s}; "
                    f"expected {(owner, r.cached_len)}, found {(self._owners[s], self._lengths[s])}")
        mask = self._accent_mask()
        if mask is not None:  # one [K] row per request: its first new row's
            starts = [sum(lengths[:i]) for i in range(len(lengths))]
            mask = mask.index_select(0, device_tensor(starts, torch.long, mask.device))
        fresh = [r.table_idx for r in reqs if r.cached_len == 0]
        if fresh:
            self._reset_slots(device_tensor(fresh, torch.long, x.device))
        if batch.is_decode:
            y = self._decode_rows(x, device_tensor(slots, torch.long, x.device), mask)
        else:
            y = self._extend(x, reqs, slots, lengths, mask)
        for r, owner in zip(reqs, owners):
            self._owners[r.table_idx] = owner
            self._lengths[r.table_idx] = r.device_len
        return y

    def _reset_slots(self, idx: torch.Tensor) -> None:
        for t in (self._conv_state, self._recurrent_state, self._live_conv, self._live_state, self._window,
                  self._win_len):
            t.index_fill_(0, idx, 0)

    def _extend(self, x, reqs, slots, lengths, mask):
        """The eager prefill / extend (gdn.py:271-327): replay each request's tail in front of its new rows;
        complete chunks in a committed pass, the rest in an uncommitted pass whose final states are the
        live ones."""
        pieces = x.split(lengths)
        combined, old_tail, complete = [], [], []
        for r, new in zip(reqs, pieces):
            tail = self._window[r.table_idx, : r.cached_len % CHUNK] if r.cached_len else new[:0]
            old_tail.append(len(tail))
            joined = torch.cat((tail, new)) if len(tail) else new
            combined.append(joined)
            complete.append(len(joined) // CHUNK * CHUNK)
        outputs: list[list[torch.Tensor]] = [[] for _ in reqs]

        def run(which, values, commit):
            idx = device_tensor([slots[i] for i in which], torch.long, x.device)
            rows = None if mask is None else torch.cat([mask[i].expand(len(v), -1) for i, v in zip(which, values)])
            cu, chunks = chunk_tables([len(v) for v in values], x.device)
            out, conv_final, final = self._run_packed(
                torch.cat(values), cu, chunks, self._conv_state.index_select(0, idx),
                self._recurrent_state.index_select(0, idx), rows)
            for i, y in zip(which, out.split([len(v) for v in values])):
                outputs[i].append(y)
            final = final.float()
            if commit:
                self._conv_state.index_copy_(0, idx, conv_final)
                self._recurrent_state.index_copy_(0, idx, final)
            self._live_conv.index_copy_(0, idx, conv_final)
            self._live_state.index_copy_(0, idx, final)

        whole = [i for i, n in enumerate(complete) if n]
        if whole:
            run(whole, [combined[i][: complete[i]] for i in whole], True)
        partial = [i for i, v in enumerate(combined) if complete[i] < len(v)]
        if partial:
            run(partial, [combined[i][complete[i]:] for i in partial], False)
        tails = []
        for i, r in enumerate(reqs):
            tail = combined[i][complete[i]:]
            self._window[r.table_idx, : len(tail)] = tail
            self._window[r.table_idx, len(tail):].zero_()
            tails.append(len(tail))
        self._win_len.index_copy_(0, device_tensor(slots, torch.long, x.device),
                                  device_tensor(tails, torch.int32, x.device))
        return torch.cat([torch.cat(parts)[n:] for parts, n in zip(outputs, old_tail)])

    def _forward_decode_static(self, x: torch.Tensor, bs: int) -> torch.Tensor:
        """One new row per padded request (gdn.py:329-355); every shape depends on ``bs`` only, so the step
        can be captured into a graph and replayed."""
        if self._graph_slots is None or bs not in self._static_rows:
            raise RuntimeError(f"GDN static decode is not prepared for batch size {bs}")
        mask = self._accent_mask()
        return self._decode_rows(x, self._graph_slots[:bs], mask)

    def _decode_rows(self, x, slots, mask):
        """The decode fast path: one row per slot from the live states, in one fused kernel launch; the raw
        row goes to the slot's window, and a window that fills commits the live states."""
        bs = slots.shape[0]
        x = x.contiguous()
        mixed = F.linear(x, self.in_proj.weight)
        if mask is not None:
            mixed = self._accent.apply_accent(self.in_proj, x, mixed, mask)
        o = ops.serving_decode_step(mixed, x, slots, self.conv.weight, self._live_conv, self._conv_state,
                                    self._live_state, self._recurrent_state, self._window, self._win_len,
                                    self.out_weight.to(x.dtype), self.A_log.float(), self.dt_bias.float(),
                                    eps=NORM_EPS, scale=HEAD_DIM**-0.5, round_qk=True)
        out = o.reshape(bs, HEADS * HEAD_DIM)
        y = F.linear(out, self.wo.weight)
        if mask is not None:
            y = self._accent.apply_accent(self.wo, out, y, mask)
        return y

    def _forward_prefill_static(self, x: torch.Tensor, inputs: PrefillInputs) -> torch.Tensor:
        """A padded prefill of fresh requests (gdn.py:357-393): the committed pass over the complete chunks,
        then each request's last ``n % 64`` rows as a 64-row window with zeros after them. The window's
        padding rows get decay 1 and beta 0, so its final states are the live ones."""
        if self._accent_mask() is not None:
            raise RuntimeError("GDN static prefill does not take accent adapters")
        layout, slots = inputs.layout, inputs.slots
        bs = slots.numel()
        self._reset_slots(slots)
        y = torch.empty_like(x)
        if layout.whole_rows is not None:
            whole_slots = slots.index_select(0, layout.whole_reqs)
            out, conv_final, final = self._run_packed(
                x.index_select(0, layout.whole_rows), layout.whole_cu, layout.whole_chunks,
                self._conv_state.index_select(0, whole_slots), self._recurrent_state.index_select(0, whole_slots))
            self._conv_state.index_copy_(0, whole_slots, conv_final)
            self._recurrent_state.index_copy_(0, whole_slots, final.float())
            y.index_copy_(0, layout.whole_rows, out)
        tail = inputs.lengths - layout.window_base  # real rows in each window
        real = torch.arange(CHUNK, device=x.device).view(1, CHUNK) < tail.view(bs, 1)
        win = x.index_select(0, layout.window_rows).masked_fill(~real.view(-1, 1), 0)
        conv0 = self._conv_state.index_select(0, slots)
        out, _, final, mixed = self._run_packed(win, layout.window_cu, layout.window_chunks, conv0,
                                                self._recurrent_state.index_select(0, slots),
                                                valid=real.view(-1), return_mixed=True)
        y.index_copy_(0, layout.window_rows, out)
        # live conv: the last four raw inputs before the window's padding (committed history first)
        raw = mixed[:, :CONV_CHANNELS].reshape(bs, CHUNK, CONV_CHANNELS).transpose(1, 2)
        hist = torch.cat((conv0, raw), dim=-1)  # [bs, C, 4 + 64]
        pick = (tail.view(bs, 1, 1) + torch.arange(CONV_WIDTH, device=x.device).view(1, 1, -1)).expand(
            bs, CONV_CHANNELS, CONV_WIDTH)
        self._live_conv.index_copy_(0, slots, torch.gather(hist, 2, pick))
        self._live_state.index_copy_(0, slots, final.float())
        self._window.index_copy_(0, slots, win.view(bs, CHUNK, self._hidden))
        self._win_len.index_copy_(0, slots, tail.to(torch.int32))
        return y

    def _run_packed(self, x, cu, chunks, conv, recurrent, mask=None, valid=None, return_mixed=False):
        """Packed sequences ``cu`` (chunk indices ``chunks``) from states ``conv`` / ``recurrent``
        (gdn.py:395-450), through the five operator attributes. ``mask``: per-row accent mask; ``valid``
        [rows] bool: rows outside it leave the recurrent state unchanged (decay 1, beta 0)."""
        mixed = F.linear(x, self.in_proj.weight)
        if mask is not None:
            mixed = self._accent.apply_accent(self.in_proj, x, mixed, mask)
        qkv, z, a, b = mixed.unsqueeze(0).split(SPLIT, dim=-1)
        if valid is not None:
            keep = valid.view(1, -1, 1)
            a = a.masked_fill(~keep, _MASKED_GATE)
            b = b.masked_fill(~keep, _MASKED_GATE)
        if self._own_operators() and mixed.dtype == torch.bfloat16:
            result, conv_final, final = self._run_packed_in_place(x, qkv, z, a, b, cu, chunks, conv, recurrent, mask)
            return (result, conv_final, final, mixed) if return_mixed else (result, conv_final, final)
        qkv, conv_final = self._conv_fwd(x=qkv.contiguous(), weight=self.conv.weight.squeeze(1), bias=None,
                                         residual=None, initial_state=conv, output_final_state=True,
                                         activation="silu", cu_seqlens=cu, chunk_indices=chunks, BT=CHUNK)
        q, k, v = [t.unflatten(-1, (HEADS, HEAD_DIM)).contiguous() for t in qkv.split(HEADS * HEAD_DIM, dim=-1)]
        q, _ = self._l2norm_fwd(q)
        k, _ = self._l2norm_fwd(k)
        _, output, _, final, _, _ = self._delta_rule_fwd(
            q=q, k=k, v=v, g=a.contiguous(), beta=self._beta_fwd(b.contiguous(), 1.0), scale=HEAD_DIM**-0.5,
            initial_state=recurrent, output_final_state=True, state_v_first=True, cu_seqlens=cu,
            chunk_indices=chunks, use_gate_in_kernel=True, A_log=self.A_log.float(), dt_bias=self.dt_bias.float(),
            chunk_size=CHUNK)
        output = self._norm_fwd(x=output.to(q.dtype).reshape(-1, HEAD_DIM), g=z.reshape(-1, HEAD_DIM).contiguous(),
                                weight=self.out_weight, bias=None, activation="swish", eps=NORM_EPS, residual=None,
                                residual_dtype=None, is_rms_norm=True)[0]
        output = output.reshape(x.shape[0], HEADS * HEAD_DIM)
        result = F.linear(output, self.wo.weight)
        if mask is not None:
            result = self._accent.apply_accent(self.wo, output, result, mask)
        if return_mixed:
            return result, conv_final, final, mixed
        return result, conv_final, final

    def _own_operators(self) -> bool:
        return (self._conv_fwd is fla_ops.causal_conv1d_fwd and self._l2norm_fwd is fla_ops.l2norm_fwd
                and self._beta_fwd is fla_ops.fused_beta_sigmoid_fwd
                and self._delta_rule_fwd is fla_ops.chunk_gated_delta_rule_fwd
                and self._norm_fwd is fla_ops.layer_norm_gated_fwd)

    def _run_packed_in_place(self, x, qkv, z, a, b, cu, chunks, conv, recurrent, mask):
        """``_run_packed``'s operator sequence with this package's operators, the copies left out: the
        conv reads q|k|v, the chunked kernel a and b (sigmoid(b) taken in the kernel), the gated norm z in
        place from the projection rows, and the L2 norms and the chunked kernel read q, k, v as column slices
        of the conv output. Each operator computes what the seam's does (q, k still rounded to bf16 after
        their norm, as the l2norm operator returns them), so results are bit-identical to the seam route."""
        y, conv_final = ops.causal_conv1d(qkv, self.conv.weight.squeeze(1), initial_state=conv, activation="silu",
                                          cu_seqlens=cu, chunk_indices=chunks, state_width=CONV_WIDTH)
        q, k, v = [t.unflatten(-1, (HEADS, HEAD_DIM)) for t in y.split(HEADS * HEAD_DIM, dim=-1)]
        q, _ = ops.l2norm(q[0])
        k, _ = ops.l2norm(k[0])
        o, final = ops.chunk_fwd(q.unsqueeze(0), k.unsqueeze(0), v, a, b, beta_is_logit=True, scale=HEAD_DIM**-0.5,
                                 initial_state=recurrent.float(), cu_seqlens=cu, chunk_indices=chunks,
                                 A_log=self.A_log.float(), dt_bias=self.dt_bias.float())
        output, _ = ops.gated_rmsnorm(o[0], z[0].unflatten(-1, (HEADS, HEAD_DIM)),
                                      self.out_weight.to(o.dtype), eps=NORM_EPS)
        output = output.reshape(x.shape[0], HEADS * HEAD_DIM)
        result = F.linear(output, self.wo.weight)
        if mask is not None:
            result = self._accent.apply_accent(self.wo, output, result, mask)
        return result, conv_final, final
