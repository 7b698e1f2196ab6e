"""The serving layer's GDN mixer with request-local state, on the MI355X kernels.

A drop-in for ``OriginalGDN`` (``servers/sgl/src/zonos3_sgl/models/gdn.py:115-450``): the same class,
method and attribute names, the per-slot caches of ``allocate_cache`` (gdn.py:150-160), the engine hooks
(gdn.py:163-233), the static-shape decode and prefill entries that graphs capture (gdn.py:329-393), the
eager ragged forward (gdn.py:235-327) and ``_run_packed`` (gdn.py:395-450) through the five operator
attributes, which are bound to this package's kernels (``fla_ops``).

Exactness model (the serving contract, kept): a slot's committed states end at a multiple of 64 rows of its
request, and the request's unfinished chunk is kept raw in the slot's 64-row window, so a later call
replays it in front of its new rows and prefill/extend/decode cuts never move a chunk boundary.

Design of this module.
- Eager calls are planned on the host first (``plan_extend``): every request's replayed window rows and
  new rows form one joined run, cut after its last complete chunk; the complete part goes to a committed
  pass, the rest to an open pass. The plan is a set of index lists (source rows, output rows, window rows)
  uploaded in one pinned copy; the device work is then one gather per pass, the packed pass itself and one
  scatter of the outputs, whatever the number of requests.
- ``_pass`` is the one place a packed pass touches the caches: it runs ``_run_packed`` from the slots'
  committed states and stores the final states as live (and as committed for a committed pass). The eager
  and static prefill paths both use it.
- Decode never replays a window. Every slot also keeps *live* states (conv history and recurrent state
  after the request's last row); a decode step (static or eager) is ``in_proj``, one serving decode launch
  (conv/SiLU/L2/gate/delta rule/gated norm on the slots' caches in place, q/k rounded like the serving
  operators return them) and ``wo``. The launch appends the raw row to the slot's window and, when the
  window fills up, copies the live states to the committed ones.
- Window rows past a slot's fill are unspecified: only the eager replay reads windows, and only their
  filled rows. Padding rows of a static prefill window are made exact no-ops of the state (decay 1,
  beta 0), so that pass's final state is the live state after the real rows.

Engine integration: ``batch_source`` is a zero-argument callable returning the current batch (in the
reference, ``get_global_ctx().batch``, gdn.py:236); ``accent`` optionally supplies the accent adapters'
``accent_mask()`` / ``apply_accent(op, x, y, mask)`` (``zonos3_sgl.layers.accent``). Batches and requests
are read by the reference's attribute names: ``is_decode``, ``padded_size``, ``gdn_prefill``, ``reqs``,
``padded_reqs``; ``table_idx``, ``extend_len``, ``cached_len``, ``device_len``, ``uid``, ``is_cfg_uncond``.
"""

from __future__ import annotations

import importlib
import itertools
from dataclasses import dataclass, field
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


def upload(lists: list[list[int]], dtype: torch.dtype, device) -> list[torch.Tensor]:
    """Several host lists as contiguous 1-D ``device`` tensors, all in one transfer."""
    flat = device_tensor([v for values in lists for v in values], dtype, device)
    return list(flat.split([len(values) for values in lists]))


def _table_lists(lengths: list[int]) -> tuple[list[int], list[int]]:
    """cu_seqlens of packed sequences of ``lengths`` rows and their flattened (sequence, chunk) rows."""
    cu = list(itertools.accumulate(lengths, initial=0))
    pairs = [v for i, n in enumerate(lengths) for j in range(-(-n // CHUNK)) for v in (i, j)]
    return cu, pairs


def chunk_tables(lengths: list[int], device) -> tuple[torch.Tensor, torch.Tensor]:
    """(cu_seqlens int32 [n + 1], chunk indices int32 [chunks, 2] = (sequence, chunk within it)) of packed
    sequences of ``lengths`` rows, in one non-blocking copy (the tables of gdn.py:49-59)."""
    cu, pairs = upload(list(_table_lists(lengths)), torch.int32, device)
    return cu, pairs.view(-1, 2)


@dataclass(frozen=True)
class PrefillLayout:
    """Static tables of a padded prefill (the engine builds one per tuple of complete-chunk counts,
    gdn.py:62-104): request i owns ``CHUNK * (whole[i] + 1)`` consecutive batch rows, its ``whole[i]``
    complete chunks and then a 64-row window that holds its last ``n_i % 64`` rows."""

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
        """All tables from ``whole`` in two transfers (the int64 row tables, the int32 chunk tables)."""
        owned = [CHUNK * w for w in whole]  # complete-chunk rows of each request
        cut = list(itertools.accumulate((n + CHUNK for n in owned), initial=0))  # row after request i - 1
        window_at = [c + n for c, n in zip(cut, owned)]  # first window row of each request
        with_whole = [i for i, n in enumerate(owned) if n]
        rows = upload([list(itertools.chain.from_iterable(range(cut[i], window_at[i]) for i in with_whole)),
                       with_whole,
                       [r for w in window_at for r in range(w, w + CHUNK)],
                       owned], torch.long, device)
        whole_cu, whole_pairs = _table_lists([owned[i] for i in with_whole])
        window_cu, window_pairs = _table_lists([CHUNK] * len(whole))
        tables = upload([whole_cu, whole_pairs, window_cu, window_pairs], torch.int32, device)
        has_whole = bool(with_whole)
        return cls(
            whole_rows=rows[0] if has_whole else None,
            whole_reqs=rows[1] if has_whole else None,
            whole_cu=tables[0] if has_whole else None,
            whole_chunks=tables[1].view(-1, 2) if has_whole else None,
            window_rows=rows[2],
            window_base=rows[3],
            window_cu=tables[2],
            window_chunks=tables[3].view(-1, 2),
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


# --------------------------------------------------------------------------------- eager-call planning

@dataclass(frozen=True)
class Request:
    """One request of an eager call as the mixer uses it (read from the engine's request object)."""

    slot: int
    owner: tuple  # (uid, is_cfg_uncond)
    cached: int  # rows the slot already holds (committed states + window fill)
    new: int  # rows in this call

    @property
    def replay(self) -> int:
        """Rows of the unfinished chunk, replayed from the slot's window in front of the new rows."""
        return self.cached % CHUNK

    @property
    def end(self) -> int:
        return self.cached + self.new


@dataclass
class PackedPass:
    """One packed pass of an eager call as host index lists. Source rows index the call's source: the
    replayed window rows of all requests in request order, then the call's rows ``x``."""

    commit: bool  # complete chunks (states committed) or the open remainders (live states only)
    members: list[int] = field(default_factory=list)  # request index of each packed sequence
    lengths: list[int] = field(default_factory=list)  # rows of each packed sequence
    src: list[int] = field(default_factory=list)  # source row of each pass row
    member_of_row: list[int] = field(default_factory=list)  # member request of each pass row
    out_rows: list[int] = field(default_factory=list)  # pass rows that are new rows of the call ...
    dest: list[int] = field(default_factory=list)  # ... and their rows in x (and in the result)
    window: list[int] = field(default_factory=list)  # open pass: flat window row (slot * 64 + j) of each row


def plan_extend(reqs: list[Request]) -> tuple[list[int], PackedPass, PackedPass]:
    """(flat window rows to replay, the committed pass, the open pass) of an eager call. Request i's joined
    run is its ``replay`` window rows then its ``new`` rows; its first ``joined // 64 * 64`` rows go to the
    committed pass and the rest to the open pass, whose rows become the slot's new window."""
    replayed = [r.slot * CHUNK + j for r in reqs for j in range(r.replay)]
    first_new = len(replayed)
    committed, open_ = PackedPass(commit=True), PackedPass(commit=False)
    at_replay = at_new = 0
    for i, r in enumerate(reqs):
        joined = list(range(at_replay, at_replay + r.replay)) + list(range(first_new + at_new,
                                                                           first_new + at_new + r.new))
        cut = len(joined) - len(joined) % CHUNK
        for part, lo, hi in ((committed, 0, cut), (open_, cut, len(joined))):
            if hi == lo:
                continue
            part.members.append(i)
            part.lengths.append(hi - lo)
            for p in range(lo, hi):
                if p >= r.replay:
                    part.out_rows.append(len(part.src))
                    part.dest.append(at_new + p - r.replay)
                if not part.commit:
                    part.window.append(r.slot * CHUNK + p - lo)
                part.src.append(joined[p])
                part.member_of_row.append(i)
        at_replay += r.replay
        at_new += r.new
    return replayed, committed, open_


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
        self._status: Optional[ops.StatusWatch] = None

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

    def _reset_slots(self, idx: torch.Tensor) -> None:
        for t in (self._conv_state, self._recurrent_state, self._live_conv, self._live_state, self._window,
                  self._win_len):
            t.index_fill_(0, idx, 0)

    # ----------------------------------------------------------------------------------- engine hooks

    @staticmethod
    def static_tables(device, bs_list) -> dict[int, tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
        """Per batch size bs: the chunk tables of bs 64-row windows and each window's first row
        (the contract of gdn.py:163-172). The fast decode path reads only the first rows."""
        def windows(bs):
            cu, chunks = chunk_tables([CHUNK] * bs, device)
            return cu, chunks, cu[:-1].to(torch.long)

        return {bs: windows(bs) for bs in bs_list}

    def enable_graph_decode(self, slots: torch.Tensor, tables) -> None:
        """``slots``: the engine's static [max_bs] int64 buffer of table slots of the padded decode batch,
        filled before every capture / replay; ``tables`` from ``static_tables`` (gdn.py:174-183)."""
        self._graph_slots = slots
        self._static_rows.update({bs: entry[2] for bs, entry in tables.items()})

    @staticmethod
    def pin_fla_cache(static_tensors, pinned: dict) -> int:
        """The reference keeps FLA's memoised index tensors alive for captured graphs (gdn.py:185-222).
        These operators memoise nothing, so there is nothing to pin: returns 0."""
        return 0

    def set_static_mode(self, enabled: bool) -> None:
        """While set, decode batches take the static-shape path (graph warm-up and capture)."""
        self._static_mode = bool(enabled)

    def note_graph_forward(self, reqs) -> None:
        """Host-side mirrors after a replayed decode step or prefill (gdn.py:228-233); raises RuntimeError
        when an earlier chunked launch of this layer recorded a device error, and arms the next check."""
        self._status_check()
        for r in reqs:
            self._owners[r.table_idx] = (r.uid, r.is_cfg_uncond)
            self._lengths[r.table_idx] = r.device_len
        self._status_arm()

    def _status_check(self) -> None:
        """RuntimeError when a chunked launch before the last armed status copy recorded an error (the
        overlapped launch's bounded wait ran out: that call's states are undefined), read without a sync."""
        if self._status is not None:
            self._status.check()

    def _status_arm(self) -> None:
        if self._status is None and self._capacity and self._recurrent_state.is_cuda:
            self._status = ops.StatusWatch(self._recurrent_state.device)
        if self._status is not None:
            self._status.arm()

    # ----------------------------------------------------------------------------------------- forward

    def _current_batch(self):
        if self._batch_source is None:
            raise RuntimeError("GDN forward needs a batch source (the engine's current batch)")
        return self._batch_source()

    def _accent_mask(self):
        return None if self._accent is None else self._accent.accent_mask()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Static decode / static prefill when the batch asks for them, else the eager path over the
        batch's requests, which checks the whole batch before it changes any cache (gdn.py:235-327)."""
        batch = self._current_batch()
        if batch.is_decode and self._static_mode:
            return self._forward_decode_static(x, batch.padded_size)
        if getattr(batch, "gdn_prefill", None) is not None:
            return self._forward_prefill_static(x, batch.gdn_prefill)
        if x.is_cuda and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("GDN ragged path cannot be captured; graphs use the static window / prefill paths")
        self._status_check()
        reqs = self._admit(batch, x.shape[0])
        mask = self._accent_mask()
        if mask is not None:  # a request's adapters: the mask row of its first new row
            firsts = list(itertools.accumulate((r.new for r in reqs[:-1]), initial=0))
            mask = mask.index_select(0, device_tensor(firsts, torch.long, mask.device))
        fresh = [r.slot for r in reqs if r.cached == 0]
        if fresh:
            self._reset_slots(device_tensor(fresh, torch.long, x.device))
        if batch.is_decode:
            y = self._decode_rows(x, device_tensor([r.slot for r in reqs], torch.long, x.device), mask)
        else:
            y = self._extend(x, reqs, mask)
        for r in reqs:
            self._owners[r.slot] = r.owner
            self._lengths[r.slot] = r.end
        if not batch.is_decode:
            self._status_arm()
        return y

    def _admit(self, batch, rows: int) -> list[Request]:
        """The eager batch's requests after every check (a failed check raises RuntimeError before any
        cache changes). A request that continues a slot must find the slot holding exactly its rows: a
        prefix matched in the KV cache alone has no recurrent state here and is refused."""
        where = f"GDN layer {self._layer_id} eager call"
        if not self._capacity:
            raise RuntimeError(f"{where}: allocate_cache was not called")
        if len(batch.padded_reqs) != len(batch.reqs):
            raise RuntimeError(f"{where}: {len(batch.padded_reqs) - len(batch.reqs)} dummy graph-padding "
                               f"requests (only the static paths take them)")
        reqs, taken = [], set()
        for r in batch.reqs:
            s, n = r.table_idx, r.extend_len
            if not 0 <= s < self._capacity:
                raise RuntimeError(f"{where}: slot {s} outside the {self._capacity} slots of the cache")
            if s in taken:
                raise RuntimeError(f"{where}: slot {s} named by two requests")
            taken.add(s)
            if n <= 0:
                raise RuntimeError(f"{where}: the request in slot {s} brings {n} rows")
            if batch.is_decode and n != 1:
                raise RuntimeError(f"{where}: a decode batch takes one new row per request, slot {s} has {n}")
            owner = (r.uid, r.is_cfg_uncond)
            if r.cached_len and (self._owners[s] != owner or self._lengths[s] != r.cached_len):
                raise RuntimeError(f"{where}: slot {s} has no state for {owner} at row {r.cached_len} "
                                   f"(it holds {self._owners[s]} at row {self._lengths[s]})")
            reqs.append(Request(slot=s, owner=owner, cached=r.cached_len, new=n))
        if sum(r.new for r in reqs) != rows:
            raise RuntimeError(f"{where}: {rows} rows given for requests of {sum(r.new for r in reqs)} rows")
        return reqs

    def _pass(self, rows, cu, chunks, slots, commit: bool, mask=None, valid=None, live_conv=True):
        """``_run_packed`` over packed sequences from the committed states of ``slots``; the final states
        become the slots' live states and, for a committed pass, their committed states. Returns the
        output rows and the projection rows (``mixed``)."""
        out, conv_final, final, mixed = self._run_packed(
            rows, cu, chunks, self._conv_state.index_select(0, slots), self._recurrent_state.index_select(0, slots),
            mask, valid=valid, return_mixed=True)
        final = final.float()
        if commit:
            self._conv_state.index_copy_(0, slots, conv_final)
            self._recurrent_state.index_copy_(0, slots, final)
        if live_conv:
            self._live_conv.index_copy_(0, slots, conv_final)
        self._live_state.index_copy_(0, slots, final)
        return out, mixed

    def _extend(self, x, reqs: list[Request], mask):
        """An eager prefill / extend (gdn.py:271-327) by the host plan: the committed pass, then the open
        pass (from the states the committed pass left), then the new windows."""
        replayed, *passes = plan_extend(reqs)
        passes = [p for p in passes if p.members]
        dev, hid = x.device, self._hidden
        idx = iter(upload([replayed] + [lst for p in passes for lst in (
            p.src, p.member_of_row, p.out_rows, p.dest, p.window, [reqs[i].slot for i in p.members])]
            + [[r.slot for r in reqs], [r.end % CHUNK for r in reqs]], torch.long, dev))
        tables = iter(upload([lst for p in passes for lst in _table_lists(p.lengths)], torch.int32, dev))
        src = x
        replay_idx = next(idx)
        if replayed:  # gathered before any window is rewritten
            src = torch.cat((self._window.view(-1, hid).index_select(0, replay_idx), x))
        y = torch.empty_like(x)
        for p in passes:
            src_idx, member_of_row, out_rows, dest, window, slots = (next(idx) for _ in range(6))
            cu, pairs = next(tables), next(tables)
            rows = src.index_select(0, src_idx)
            out, _ = self._pass(rows, cu, pairs.view(-1, 2), slots, p.commit,
                                mask=None if mask is None else mask.index_select(0, member_of_row))
            y.index_copy_(0, dest, out if len(p.out_rows) == len(p.src) else out.index_select(0, out_rows))
            if not p.commit:
                self._window.view(-1, hid).index_copy_(0, window, rows)
        all_slots, fill = next(idx), next(idx)
        self._win_len.index_copy_(0, all_slots, fill.to(torch.int32))
        return y

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
        """A padded prefill of fresh requests on the layout's fixed shapes (the contract of gdn.py:357-393):
        a committed pass over the complete chunks, then an open pass over every request's 64-row window, in
        which the rows past the request's real rows are zeroed and made state no-ops. The final states of
        the open pass are the live ones; the windows keep the rows."""
        if self._accent_mask() is not None:
            raise RuntimeError("GDN static prefill does not take accent adapters")
        layout, slots = inputs.layout, inputs.slots
        bs = slots.numel()
        self._reset_slots(slots)
        y = torch.empty_like(x)
        if layout.whole_rows is not None:
            out, _ = self._pass(x.index_select(0, layout.whole_rows), layout.whole_cu, layout.whole_chunks,
                                slots.index_select(0, layout.whole_reqs), commit=True)
            y.index_copy_(0, layout.whole_rows, out)
        fill = (inputs.lengths - layout.window_base).to(torch.int32)  # real rows of each window
        # a padding row is a state no-op only if its values are finite (beta 0 multiplies them): zero them
        real = torch.arange(CHUNK, device=x.device, dtype=torch.int32).unsqueeze(0) < fill.unsqueeze(1)
        win = torch.where(real.view(-1, 1), x.index_select(0, layout.window_rows), x.new_zeros(()))
        out, mixed = self._pass(win, layout.window_cu, layout.window_chunks, slots, commit=False,
                                valid=real.view(-1), live_conv=False)
        y.index_copy_(0, layout.window_rows, out)
        # live conv history: the last CONV_WIDTH conv inputs up to each window's last real row, the
        # committed history (zero for fresh requests, or the complete chunks' end) standing before row 0
        raw = mixed[:, :CONV_CHANNELS].reshape(bs, CHUNK, CONV_CHANNELS).transpose(1, 2)
        hist = torch.cat((self._conv_state.index_select(0, slots), raw), dim=-1)  # [bs, C, CONV_WIDTH + 64]
        take = fill.to(torch.long).view(bs, 1, 1) + torch.arange(CONV_WIDTH, device=x.device).view(1, 1, -1)
        self._live_conv.index_copy_(0, slots, hist.gather(2, take.expand(bs, CONV_CHANNELS, CONV_WIDTH)))
        self._window.index_copy_(0, slots, win.view(bs, CHUNK, self._hidden))
        self._win_len.index_copy_(0, slots, fill)
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
