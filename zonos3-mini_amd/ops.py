"""Torch-level entry points of the gated-DeltaNet kernels (validation, allocation, stream plumbing).

Every function validates shapes, dtypes, devices and contiguity and raises ``RuntimeError`` on a mismatch
(the reference layer's error style, ``servers/sgl/src/zonos3_sgl/models/gdn.py:152, 242, 255``), allocates
outputs with torch's caching allocator, and launches on the current HIP stream of the tensors' device
without synchronising the host, so every call can be captured into a HIP graph. There is no CPU path.
"""

from __future__ import annotations

import ctypes
import os

import torch

from . import _native
from ._native import BF16, F32

_CODES = {torch.float32: F32, torch.bfloat16: BF16}


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _code(t: torch.Tensor, name: str) -> int:
    _require(t.dtype in _CODES, f"{name}: dtype {t.dtype} not supported (float32 or bfloat16)")
    return _CODES[t.dtype]


def _on_gpu(name: str, t: torch.Tensor, device: torch.device | None = None) -> None:
    _require(isinstance(t, torch.Tensor), f"{name}: expected a tensor")
    _require(t.is_cuda, f"{name}: must be a GPU tensor (got device {t.device}); there is no CPU path")
    _require(t.is_contiguous(), f"{name}: must be contiguous")
    if device is not None:
        _require(t.device == device, f"{name}: on {t.device}, expected {device}")


def _row_stride(t: torch.Tensor, inner_dims: int) -> int | None:
    """Elements between consecutive rows of ``t`` when its last ``inner_dims`` dims are one dense row and its
    leading dims step in whole rows (a column slice of a wider row-major buffer qualifies); None otherwise."""
    shape, stride = t.shape, t.stride()
    lead = t.dim() - inner_dims
    if t.numel() == 0:  # no rows to read: any stride will do
        w = 1
        for n in shape[lead:]:
            w *= n
        return w
    width = 1
    for d in range(t.dim() - 1, lead - 1, -1):
        if shape[d] != 1 and stride[d] != width:
            return None
        width *= shape[d]
    ld, rows = None, 1
    for d in range(lead - 1, -1, -1):
        if shape[d] == 1:
            continue
        if ld is None:
            ld = stride[d]
        elif stride[d] != rows * ld:
            return None
        rows *= shape[d]
    if ld is None:
        return width
    return ld if ld >= width else None


def _rows_in_place(name: str, t: torch.Tensor, inner_dims: int, device, multiple: int = 1, align: int = 1):
    """(t, row stride) when the kernels can read t's rows in place -- row stride a multiple of ``multiple``
    elements, base aligned to ``align`` bytes -- else (a contiguous copy, dense row width)."""
    _require(isinstance(t, torch.Tensor), f"{name}: expected a tensor")
    _require(t.is_cuda, f"{name}: must be a GPU tensor (got device {t.device}); there is no CPU path")
    if device is not None:
        _require(t.device == device, f"{name}: on {t.device}, expected {device}")
    ld = _row_stride(t, inner_dims)
    if ld is None or ld % multiple or t.data_ptr() % align:
        t = t.contiguous()
        ld = _row_stride(t, inner_dims)
    return t, ld


def _head_rows(name: str, t: torch.Tensor, device=None):
    """(t, group, stride) for the row kernels: t's rows of its last dim D, row r starting at
    (r / group) * stride + (r % group) * D -- the dims after the first dense (a token's heads), the first
    stepping by ``stride`` (a column slice of wider rows qualifies). Layouts outside that are copied first."""
    t, ld = _rows_in_place(name, t, max(t.dim() - 1, 1) if isinstance(t, torch.Tensor) else 1, device)
    if t.dim() < 2:
        return t, 1, t.shape[-1] if t.dim() else 1
    group = 1
    for n in t.shape[1:-1]:
        group *= n
    return t, group, ld


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _gate_check(A_log, dt_bias, Hv: int, device) -> None:
    if (A_log is None) != (dt_bias is None):
        raise RuntimeError("A_log and dt_bias go together")
    if A_log is not None:
        for name, t in (("A_log", A_log), ("dt_bias", dt_bias)):
            _on_gpu(name, t, device)
            _require(t.dtype == torch.float32 and t.shape == (Hv,), f"{name}: expected float32 [{Hv}]")


def check_cu_seqlens(cu: list[int], total: int) -> None:
    """Raise RuntimeError unless ``cu`` (host values of cu_seqlens) starts at 0, never decreases and ends at
    ``total`` tokens -- the packed-length checks the serving layer makes before any launch
    (``servers/sgl/src/zonos3_sgl/models/gdn.py:247-255``; empty sequences are allowed here, as FLA's tables
    allow them)."""
    _require(len(cu) >= 2, f"cu_seqlens: {len(cu)} entries, need at least 2")
    _require(cu[0] == 0, f"cu_seqlens: starts at {cu[0]}, expected 0")
    for i in range(len(cu) - 1):
        _require(cu[i + 1] >= cu[i], f"cu_seqlens: decreases at entry {i} ({cu[i]} -> {cu[i + 1]})")
    _require(cu[-1] == total, f"cu_seqlens: ends at {cu[-1]}, but the batch holds {total} tokens")


def _table_rows(cu: list[int]) -> list[tuple[int, int]]:
    return [(i, j) for i in range(len(cu) - 1) for j in range(-(-(cu[i + 1] - cu[i]) // CHUNK))]


def check_chunk_indices(rows, cu: list[int]) -> None:
    """Raise RuntimeError unless ``rows`` (host values of the [n_chunks, 2] chunk table) is exactly the
    (sequence, chunk within it) table of ``gdn.py:49-59`` for the sequences of ``cu``."""
    expect = _table_rows(cu)
    got = [tuple(int(x) for x in r) for r in rows]
    if got != expect:
        first = next((i for i, (a, b) in enumerate(zip(got, expect)) if a != b), min(len(got), len(expect)))
        raise RuntimeError(f"chunk_indices: {len(got)} rows do not match the {len(expect)} chunks of cu_seqlens "
                           f"(first difference at row {first})")


def _cu_check(cu_seqlens: torch.Tensor, total: int, device) -> int:
    """Type checks of a device cu_seqlens. Its values stay on the device (no host read, so the call can be
    captured into a graph); the kernels clamp each sequence's token range into the batch, so a malformed
    device table cannot make them touch rows outside it."""
    _on_gpu("cu_seqlens", cu_seqlens, device)
    _require(cu_seqlens.dtype == torch.int32, "cu_seqlens: must be int32")
    _require(cu_seqlens.dim() == 1 and cu_seqlens.numel() >= 2, "cu_seqlens: must be 1-D with >= 2 entries")
    return cu_seqlens.numel() - 1


def _on_host(t) -> bool:
    return t is not None and (not isinstance(t, torch.Tensor) or not t.is_cuda)


def host_tables(cu_seqlens, chunk_indices, total: int, device=None):
    """Packed tables held on the host (lists or CPU tensors), as the reference builds them (gdn.py:49-59):
    checked (``check_cu_seqlens``, ``check_chunk_indices``; the chunk table is built when None), then copied
    to ``device`` in one transfer. Returns int32 (cu_seqlens [N+1], chunk_indices [n_chunks, 2]); raises
    RuntimeError before any copy or launch when a table is malformed."""
    cu = cu_seqlens.tolist() if isinstance(cu_seqlens, torch.Tensor) else [int(x) for x in cu_seqlens]
    check_cu_seqlens(cu, total)
    if chunk_indices is None:
        rows = _table_rows(cu)
    else:
        rows = chunk_indices.tolist() if isinstance(chunk_indices, torch.Tensor) else list(chunk_indices)
        check_chunk_indices(rows, cu)
    flat = torch.tensor(cu + [int(x) for r in rows for x in r], dtype=torch.int32)
    if device is not None:
        flat = flat.to(device)
    return flat[: len(cu)], flat[len(cu):].view(-1, 2)


def recurrent_fwd(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=True, cu_seqlens=None,
                  final_state=None, A_log=None, dt_bias=None, use_qk_l2norm=False, out_dtype=None):
    """Token-by-token gated delta rule (lm.py:574-583 in FLA's calling convention).

    q, k [B, T, Hk, K]; v [B, T, Hv, V]; g and beta [B, T, Hv], float32 or bfloat16; g is the log decay, or
    the raw gate input when ``A_log``/``dt_bias`` (float32 [Hv]) are given (lm.py:572). ``use_qk_l2norm``
    L2-normalises q and k in the kernel in fp32 (lm.py:570-571). initial_state [N, Hv, V, K] float32 or None
    (zeros); cu_seqlens int32 [N+1] with B == 1 for packed sequences. ``final_state`` may name an existing
    float32 tensor to write (it may be ``initial_state`` itself: an in-place update). Returns
    (o [B, T, Hv, V] in ``out_dtype`` (default v's dtype), final state or None)."""
    _on_gpu("q", q)
    dev = q.device
    for name, t in (("k", k), ("v", v), ("g", g), ("beta", beta)):
        _on_gpu(name, t, dev)
    _require(q.dim() == 4 and k.shape == q.shape, f"q, k: expected equal [B, T, Hk, K], got {tuple(q.shape)}, "
                                                  f"{tuple(k.shape)}")
    B, T, Hk, K = q.shape
    _require(v.dim() == 4 and v.shape[:2] == (B, T), f"v: expected [B={B}, T={T}, Hv, V], got {tuple(v.shape)}")
    Hv, V = v.shape[2], v.shape[3]
    _require(Hv % Hk == 0, f"value heads ({Hv}) must be a multiple of key heads ({Hk})")
    _require(g.shape == (B, T, Hv) and beta.shape == (B, T, Hv), f"g, beta: expected [{B}, {T}, {Hv}]")
    _require(q.dtype == k.dtype == v.dtype, "q, k, v: must share a dtype")
    _require(g.dtype == beta.dtype, "g, beta: must share a dtype")
    qkv_code, gb_code = _code(q, "q"), _code(g, "g")
    _gate_check(A_log, dt_bias, Hv, dev)
    n_seqs = B
    if cu_seqlens is not None:
        _require(B == 1, "cu_seqlens: packed sequences need B == 1")
        if _on_host(cu_seqlens):  # a host table: checked here, then copied
            cu_seqlens, _ = host_tables(cu_seqlens, None, T, dev)
        n_seqs = _cu_check(cu_seqlens, T, dev)
    if initial_state is not None:
        _on_gpu("initial_state", initial_state, dev)
        _require(initial_state.dtype == torch.float32, "initial_state: must be float32")
        _require(initial_state.shape == (n_seqs, Hv, V, K),
                 f"initial_state: expected [{n_seqs}, {Hv}, {V}, {K}], got {tuple(initial_state.shape)}")
    if final_state is not None:
        _on_gpu("final_state", final_state, dev)
        _require(final_state.dtype == torch.float32 and final_state.shape == (n_seqs, Hv, V, K),
                 f"final_state: expected float32 [{n_seqs}, {Hv}, {V}, {K}]")
    elif output_final_state:
        final_state = torch.empty(n_seqs, Hv, V, K, device=dev, dtype=torch.float32)
    o = torch.empty(B, T, Hv, V, device=dev, dtype=v.dtype if out_dtype is None else out_dtype)
    scale = K**-0.5 if scale is None else float(scale)
    _native.call(
        "zgdn_recurrent_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), qkv_code, g.data_ptr(), beta.data_ptr(),
        gb_code, _ptr(A_log), _ptr(dt_bias), int(bool(use_qk_l2norm)), _ptr(initial_state), _ptr(final_state),
        o.data_ptr(), _code(o, "o"), _ptr(cu_seqlens), n_seqs, B, T, Hk, Hv, K, V, scale, _stream(dev),
    )
    return o, final_state


def decode_step(q, k, v, g, beta, state, scale=None):
    """One single-token step for B independent streams, updating ``state`` in place.

    q, k [B, Hk, K]; v [B, Hv, V]; g (log decay), beta [B, Hv]; state [B, Hv, V, K] float32.
    Returns o [B, Hv, V] in v's dtype (the recurrence of lm.py:574-583 at T = 1)."""
    _require(q.dim() == 3 and v.dim() == 3, "decode_step: q, k [B, Hk, K] and v [B, Hv, V] expected")
    o, _ = recurrent_fwd(q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1), g.unsqueeze(1), beta.unsqueeze(1),
                         scale=scale, initial_state=state, final_state=state)
    return o.squeeze(1)


CHUNK = 64  # chunk length of the chunked kernels (servers/sgl/src/zonos3_sgl/models/gdn.py:46)


def chunk_indices_from_cu(cu_seqlens: torch.Tensor, total: int | None = None) -> torch.Tensor:
    """(sequence, chunk within it) int32 [n_chunks, 2] of packed sequences (gdn.py:49-59). Reads
    ``cu_seqlens`` on the host (one device->host copy) and checks it there (``check_cu_seqlens``, against
    ``total`` tokens when given); callers that already hold the lengths on the host build the table there, as
    the reference does."""
    cu = cu_seqlens.tolist()
    check_cu_seqlens(cu, cu[-1] if total is None and cu else total)
    t = torch.tensor(_table_rows(cu), dtype=torch.int32).reshape(-1, 2)
    return t.to(cu_seqlens.device)


class launch_form:
    """Context manager setting the chunked path's launch form for the process (``zgdn_chunk_set_launch_form``:
    -1 the library's choice, 0 two launches, 1 the overlapped launch wherever eligible) and restoring the
    previous form on exit. Every form gives the same results bit for bit."""

    def __init__(self, form: int):
        self.form = int(form)
        self.prev = None

    def __enter__(self):
        self.prev = int(_native.lib().zgdn_chunk_get_launch_form())
        _native.call("zgdn_chunk_set_launch_form", self.form)
        return self

    def __exit__(self, *exc):
        _native.call("zgdn_chunk_set_launch_form", self.prev)
        return False


def chunk_status(clear: bool = True) -> int:
    """Bits of the chunked path's sticky device status word (0 = no error): ``_native.STATUS_WAIT_GAVE_UP``
    when an overlapped launch's bounded wait ran out, leaving that call's outputs undefined. Synchronises the
    device; ``clear`` resets the word."""
    out = ctypes.c_int(0)
    _native.call("zgdn_chunk_status", ctypes.byref(out), int(bool(clear)))
    return out.value


def check_chunk_status() -> None:
    """Raise RuntimeError when the chunked path's device status word records an error (and clear it)."""
    st = chunk_status(clear=True)
    if st:
        raise RuntimeError(f"chunked prefill: device status {st:#x} (a state pass gave up waiting for its chunk's "
                           "phase-1 results; the outputs and final states of that call are undefined)")


class StatusWatch:
    """The chunked path's device status word read without stalling the host, for a caller that launches from
    one stream again and again (the serving layer): ``arm()`` enqueues an asynchronous copy of the word into
    page-locked host memory on the current stream, with an event behind it; ``check()`` looks at the last armed
    copy only once its event has completed (a non-blocking query) and raises RuntimeError, clearing the word,
    when a launch before it recorded an error. Neither call synchronises; both do nothing while the stream is
    being captured into a graph."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.event = None

    def arm(self) -> None:
        if torch.cuda.is_current_stream_capturing():
            return
        _native.call("zgdn_chunk_status_async", self.host.data_ptr(), _stream(self.device))
        self.event = torch.cuda.Event()
        self.event.record(torch.cuda.current_stream(self.device))

    def check(self) -> None:
        if self.event is None or torch.cuda.is_current_stream_capturing() or not self.event.query():
            return
        self.event = None
        if int(self.host[0]):
            check_chunk_status()


# Validation mode (ZGDN_VALIDATE=1 in the environment, read once at import): every chunk_fwd then synchronises
# the device after its launch and raises RuntimeError when the device status word records an error. Off by
# default, so that calls stay asynchronous and capturable.
VALIDATE = os.environ.get("ZGDN_VALIDATE", "0") not in ("", "0")


def chunk_fwd(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=True, cu_seqlens=None,
              chunk_indices=None, A_log=None, dt_bias=None, final_state=None, use_qk_l2norm=False,
              beta_is_logit=False):
    """Chunked gated delta rule (64-token chunks, fp32 state): the prefill core.

    The operator behind FLA's ``chunk_gated_delta_rule_fwd`` as the serving layer calls it
    (``servers/sgl/src/zonos3_sgl/models/gdn.py:418-434``), in the layer's dtype (``lm.py:556-602``): q, k
    [B, T, Hk, K], v [B, T, Hv, V] with K == V of 64 or 128, all bfloat16 or all float32 (bf16 at 128 runs on
    bf16 MFMA; fp32, and 64-wide heads, in fp32 arithmetic); g, beta [B, T, Hv] float32 or bfloat16. With ``A_log``/``dt_bias`` (float32 [Hv]) g is the raw gate input
    and the decay is formed in the kernel (``use_gate_in_kernel=True``). ``use_qk_l2norm``: q, k are the raw
    rows, L2-normalised in the kernel with fp32 factors (never rounded after the norm). ``beta_is_logit``: beta
    holds the raw input b and the kernel takes sigmoid(b) in fp32 (what ``sigmoid`` returns, FLA's
    fused_beta_sigmoid_fwd at gdn.py:423). Packed sequences: B == 1, ``cu_seqlens`` int32 [N+1] and optionally
    ``chunk_indices`` int32 [n_chunks, 2]. q, k, v, g, beta may be column slices of wider rows (the conv output,
    the input projection): rows whose stride the kernel can take are read in place, others are copied first.
    Returns (o [B, T, Hv, V] in q's dtype, final state [N, Hv, V, K] float32 or None)."""
    dev = q.device if isinstance(q, torch.Tensor) else None
    ve = 4 if isinstance(q, torch.Tensor) and q.dtype == torch.float32 else 8  # elements in 16 bytes
    q, q_ld = _rows_in_place("q", q, 2, dev, ve, 16)
    k, k_ld = _rows_in_place("k", k, 2, dev, ve, 16)
    v, v_ld = _rows_in_place("v", v, 2, dev, ve, 16)
    _require(q.dim() == 4 and k.shape == q.shape, f"q, k: expected equal [B, T, Hk, K], got {tuple(q.shape)}, "
                                                  f"{tuple(k.shape)}")
    B, T, Hk, K = q.shape
    _require(v.dim() == 4 and v.shape[:2] == (B, T), f"v: expected [B={B}, T={T}, Hv, V], got {tuple(v.shape)}")
    Hv, V = v.shape[2], v.shape[3]
    g, gb_ld = _rows_in_place("g", g, 1, dev)
    beta, beta_ld = _rows_in_place("beta", beta, 1, dev)
    if beta_ld != gb_ld:  # one row stride serves both
        g, gb_ld = g.contiguous(), Hv
        beta = beta.contiguous()
    _require(K == V and K in (64, 128), f"chunk_fwd: head dims K={K}, V={V}; the chunked kernels take K == V, "
                                         f"64 or 128")
    _require(Hv % Hk == 0, f"value heads ({Hv}) must be a multiple of key heads ({Hk})")
    _require(q.dtype == k.dtype == v.dtype and q.dtype in (torch.bfloat16, torch.float32),
             "chunk_fwd: q, k, v must all be bfloat16 or all float32")
    _require(g.shape == (B, T, Hv) and beta.shape == (B, T, Hv), f"g, beta: expected [{B}, {T}, {Hv}]")
    _require(g.dtype == beta.dtype, "g, beta: must share a dtype")
    gb_code = _code(g, "g")
    _gate_check(A_log, dt_bias, Hv, dev)
    n_seqs = B
    n_chunks = B * (-(-T // CHUNK))
    if cu_seqlens is not None:
        _require(B == 1, "cu_seqlens: packed sequences need B == 1")
        if _on_host(cu_seqlens):  # host tables: checked here, then copied
            cu_seqlens, chunk_indices = host_tables(cu_seqlens, chunk_indices, T, dev)
        n_seqs = _cu_check(cu_seqlens, T, dev)
        if chunk_indices is None:
            chunk_indices = chunk_indices_from_cu(cu_seqlens, T)
        _on_gpu("chunk_indices", chunk_indices, dev)
        _require(chunk_indices.dtype == torch.int32 and chunk_indices.dim() == 2 and chunk_indices.shape[1] == 2,
                 "chunk_indices: expected int32 [n_chunks, 2]")
        n_chunks = chunk_indices.shape[0]
    elif chunk_indices is not None:
        raise RuntimeError("chunk_indices without cu_seqlens")
    if initial_state is not None:
        _on_gpu("initial_state", initial_state, dev)
        _require(initial_state.dtype == torch.float32 and initial_state.shape == (n_seqs, Hv, V, K),
                 f"initial_state: expected float32 [{n_seqs}, {Hv}, {V}, {K}], got {tuple(initial_state.shape)}")
    if final_state is not None:
        _on_gpu("final_state", final_state, dev)
        _require(final_state.dtype == torch.float32 and final_state.shape == (n_seqs, Hv, V, K),
                 f"final_state: expected float32 [{n_seqs}, {Hv}, {V}, {K}]")
    elif output_final_state:
        final_state = torch.empty(n_seqs, Hv, V, K, device=dev, dtype=torch.float32)
    o = torch.empty(B, T, Hv, V, device=dev, dtype=q.dtype)
    qkv_code = _code(q, "q")
    ws_bytes = int(_native.lib().zgdn_chunk_workspace_bytes(n_chunks, Hv, K, V, qkv_code))
    if cu_seqlens is None and qkv_code == BF16 and K == 128:  # room for the segmented state pass when taken
        ws_bytes += int(_native.lib().zgdn_chunk_segment_workspace_size(B, T, Hv))
    workspace = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    scale = K**-0.5 if scale is None else float(scale)
    _native.call(
        "zgdn_chunk_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), qkv_code, g.data_ptr(), beta.data_ptr(), gb_code,
        _ptr(A_log), _ptr(dt_bias), int(bool(use_qk_l2norm)), _ptr(initial_state), _ptr(final_state), o.data_ptr(),
        _ptr(cu_seqlens),
        _ptr(chunk_indices), n_seqs, n_chunks, B, T, Hk, Hv, K, V, q_ld, k_ld, v_ld, gb_ld, int(bool(beta_is_logit)),
        scale, workspace.data_ptr(), ws_bytes, _stream(dev),
    )
    if VALIDATE:
        check_chunk_status()
    return o, final_state


def fused_decode_step(x_qkv, z, a, b, conv_weight, conv_cache, state, norm_weight, A_log, dt_bias, eps=1e-6,
                      scale=None, round_qk=False):
    """One single-token step of the whole GDN block for B streams (lm.py:563-587 for one new row each).

    x_qkv [B, 2*Hk*128 + Hv*128] raw q|k|v channels; z [B, Hv, 128]; a, b [B, Hv] (raw gate inputs);
    conv_weight [C, 4] or [C, 1, 4]; norm_weight [128] -- all bfloat16 or all float32. conv_cache [B, C, 3]
    (same dtype, oldest first) and state [B, Hv, 128, 128] float32 are updated in place; A_log, dt_bias
    float32 [Hv]. ``round_qk``: round the L2-normalised q, k to the input dtype (the serving layer's l2norm
    operator returns them so, gdn.py:416-417) instead of keeping them fp32 (lm.py:569-571). Returns the gated,
    normalised output [B, Hv, 128]."""
    _on_gpu("x_qkv", x_qkv)
    dev = x_qkv.device
    _require(x_qkv.dim() == 2, f"x_qkv: expected [B, C], got {tuple(x_qkv.shape)}")
    B, C = x_qkv.shape
    _require(z.dim() == 3 and z.shape[0] == B, f"z: expected [B={B}, Hv, V], got {tuple(z.shape)}")
    Hv, V = z.shape[1], z.shape[2]
    K = V
    _require(K == 128, f"fused_decode_step: head size {V}; the fused kernel needs 128")
    _require((C - Hv * V) > 0 and (C - Hv * V) % (2 * K) == 0, f"x_qkv: {C} channels do not split into "
                                                                f"q|k|v with Hv={Hv}, head size {K}")
    Hk = (C - Hv * V) // (2 * K)
    _require(Hv % Hk == 0 and Hv // Hk in (1, 2, 4), f"Hv/Hk = {Hv}/{Hk}: supported groups are 1, 2, 4")
    if conv_weight.dim() == 3:
        conv_weight = conv_weight.squeeze(1)
    dt = x_qkv.dtype
    for name, t, shape in (("z", z, (B, Hv, V)), ("a", a, (B, Hv)), ("b", b, (B, Hv)),
                           ("conv_weight", conv_weight, (C, 4)), ("conv_cache", conv_cache, (B, C, 3)),
                           ("norm_weight", norm_weight, (V,))):
        _on_gpu(name, t, dev)
        _require(t.dtype == dt, f"{name}: dtype {t.dtype}, expected {dt} (the dtype of x_qkv)")
        _require(tuple(t.shape) == shape, f"{name}: expected {list(shape)}, got {list(t.shape)}")
    _on_gpu("state", state, dev)
    _require(state.dtype == torch.float32 and state.shape == (B, Hv, V, K),
             f"state: expected float32 [{B}, {Hv}, {V}, {K}]")
    for name, t in (("A_log", A_log), ("dt_bias", dt_bias)):
        _on_gpu(name, t, dev)
        _require(t.dtype == torch.float32 and t.shape == (Hv,), f"{name}: expected float32 [{Hv}]")
    out = torch.empty(B, Hv, V, device=dev, dtype=dt)
    scale = K**-0.5 if scale is None else float(scale)
    _native.call(
        "zgdn_fused_decode_step", x_qkv.data_ptr(), z.data_ptr(), a.data_ptr(), b.data_ptr(), _code(x_qkv, "x_qkv"),
        conv_weight.data_ptr(), conv_cache.data_ptr(), A_log.data_ptr(), dt_bias.data_ptr(), norm_weight.data_ptr(),
        state.data_ptr(), out.data_ptr(), B, Hk, Hv, K, V, 4, float(eps), scale, int(bool(round_qk)), _stream(dev),
    )
    return out


def serving_decode_step(mixed, x_hidden, slots, conv_weight, conv_live, conv_commit, state_live, state_commit,
                        window, win_len, norm_weight, A_log, dt_bias, eps=1e-5, scale=None, round_qk=True):
    """The serving layer's single-row decode for B requests in table slots, in place on the per-slot caches
    (the fast path of ``servers/sgl/src/zonos3_sgl/models/gdn.py:329-355``; C ABI ``zgdn_serving_decode_step``).

    mixed [B, >= C + Hv*128 + 2*Hv] in_proj rows (q|k|v | z | a | b, unit stride within a row); x_hidden
    [B, hidden] the raw rows; slots int64 [B], table slots (a slot repeated later in the batch -- the spare
    slot of a padded graph replay -- is served by its first entry only; the later entries' rows of the result
    are unspecified). Caches over ``cap`` slots: conv_live,
    conv_commit [cap, C, 4] and window [cap, R, hidden] in mixed's dtype; state_live, state_commit
    [cap, Hv, 128, 128] float32; win_len int32 [cap]. conv_weight [C, 4] or [C, 1, 4], norm_weight [128] in
    mixed's dtype; A_log, dt_bias float32 [Hv]. Returns the gated, normalised output [B, Hv, 128]."""
    _on_gpu("mixed", mixed)
    dev = mixed.device
    _require(mixed.dim() == 2 and mixed.stride(1) == 1, f"mixed: expected [B, L] rows, got {tuple(mixed.shape)}")
    B = mixed.shape[0]
    _require(conv_live.dim() == 3, f"conv_live: expected [cap, C, 4], got {tuple(conv_live.shape)}")
    cap, C, W = conv_live.shape
    _require(W == 4, f"conv_live: conv width {W} (supported: 4)")
    _require(state_live.dim() == 4 and state_live.shape[0] == cap and state_live.shape[2:] == (128, 128),
             f"state_live: expected [{cap}, Hv, 128, 128], got {tuple(state_live.shape)}")
    Hv, K = state_live.shape[1], 128
    _require((C - Hv * K) > 0 and (C - Hv * K) % (2 * K) == 0, f"conv_live: {C} channels do not split into "
                                                                f"q|k|v with Hv={Hv}, head size {K}")
    Hk = (C - Hv * K) // (2 * K)
    _require(mixed.shape[1] >= C + Hv * K + 2 * Hv, f"mixed: {mixed.shape[1]} columns hold no q|k|v ({C}), z "
                                                    f"({Hv * K}), a, b ({Hv} each)")
    if conv_weight.dim() == 3:
        conv_weight = conv_weight.squeeze(1)
    dt = mixed.dtype
    _require(window.dim() == 3 and window.shape[0] == cap, f"window: expected [{cap}, R, hidden]")
    hidden = window.shape[2]
    for name, t, shape in (("x_hidden", x_hidden, (B, hidden)), ("conv_weight", conv_weight, (C, 4)),
                           ("conv_live", conv_live, (cap, C, 4)), ("norm_weight", norm_weight, (K,)),
                           ("window", window, tuple(window.shape))):
        _on_gpu(name, t, dev)
        _require(t.dtype == dt, f"{name}: dtype {t.dtype}, expected {dt} (the dtype of mixed)")
        _require(tuple(t.shape) == shape and t.is_contiguous(), f"{name}: expected contiguous {list(shape)}")
    _on_gpu("conv_commit", conv_commit, dev)
    _require(conv_commit.dtype == dt and conv_commit.shape == conv_live.shape and conv_commit.is_contiguous()
             and conv_live.is_contiguous(), f"conv_live, conv_commit: contiguous {dt} [{cap}, {C}, 4]")
    for name, t in (("state_live", state_live), ("state_commit", state_commit)):
        _on_gpu(name, t, dev)
        _require(t.dtype == torch.float32 and t.shape == (cap, Hv, K, K) and t.is_contiguous(),
                 f"{name}: expected contiguous float32 [{cap}, {Hv}, {K}, {K}]")
    _on_gpu("slots", slots, dev)
    _require(slots.dtype == torch.int64 and slots.shape == (B,) and slots.is_contiguous(), f"slots: int64 [{B}]")
    _on_gpu("win_len", win_len, dev)
    _require(win_len.dtype == torch.int32 and win_len.shape == (cap,), f"win_len: int32 [{cap}]")
    for name, t in (("A_log", A_log), ("dt_bias", dt_bias)):
        _on_gpu(name, t, dev)
        _require(t.dtype == torch.float32 and t.shape == (Hv,), f"{name}: expected float32 [{Hv}]")
    out = torch.empty(B, Hv, K, device=dev, dtype=dt)
    scale = K**-0.5 if scale is None else float(scale)
    _native.call(
        "zgdn_serving_decode_step", mixed.data_ptr(), mixed.stride(0), x_hidden.data_ptr(), hidden,
        _code(mixed, "mixed"), slots.data_ptr(), cap, B, Hk, Hv, K, K, 4, conv_weight.data_ptr(),
        conv_live.data_ptr(), conv_commit.data_ptr(), state_live.data_ptr(), state_commit.data_ptr(),
        window.data_ptr(), win_len.data_ptr(), window.shape[1], A_log.data_ptr(), dt_bias.data_ptr(),
        norm_weight.data_ptr(), out.data_ptr(), float(eps), scale, int(bool(round_qk)), _stream(dev),
    )
    return out


def attnres_route(sources, query, eps):
    """Full Attention-Residual routing (lm.py:384-389): per token, softmax over the sources of
    rms_norm(x_s) . query (fp32), then the weighted sum of the raw sources.

    sources: a list of [T, dim] tensors (lm.py) or one [S, T, dim] bank (the serving layer, zonos3.py:99-113),
    read in place (no stacking); query [dim]; one dtype (float32 / bfloat16). Returns [T, dim]."""
    if torch.is_tensor(sources):
        _require(sources.dim() == 3, f"sources: expected [S, T, dim], got {tuple(sources.shape)}")
        sources = list(sources.unbind(0))
    _require(len(sources) >= 1, "sources: at least one source")
    first = sources[0]
    _require(isinstance(first, torch.Tensor) and first.is_cuda,
             "sources[0]: must be a GPU tensor; there is no CPU path")
    dev = first.device
    _require(first.dim() == 2, f"sources: expected [T, dim] rows, got {tuple(first.shape)}")
    T, D = first.shape
    rows = []
    for i, s in enumerate(sources):  # rows may be strided (a bank's slices, a wider tensor's columns)
        _require(isinstance(s, torch.Tensor) and s.device == dev, f"sources[{i}]: expected a tensor on {dev}")
        _require(s.shape == first.shape and s.dtype == first.dtype,
                 f"sources[{i}]: {tuple(s.shape)} {s.dtype}, expected {tuple(first.shape)} {first.dtype}")
        rows.append(s)
    stride = first.stride(0) if T > 1 else D
    if any(s.stride(1) != 1 or (T > 1 and s.stride(0) != stride) for s in rows):
        rows = [s.contiguous() for s in rows]
        stride = D
    _on_gpu("query", query, dev)
    _require(query.shape == (D,) and query.dtype == first.dtype and query.is_contiguous(),
             f"query: expected contiguous [{D}] {first.dtype}")
    out = torch.empty(T, D, device=dev, dtype=first.dtype)
    ptrs = (ctypes.c_void_p * len(rows))(*[s.data_ptr() for s in rows])
    _native.call("zgdn_attnres_route", ptrs, len(rows), T, D, stride, _code(first, "sources"), query.data_ptr(),
                 float(eps), out.data_ptr(), _stream(dev))
    return out


def causal_conv1d(x, weight, bias=None, initial_state=None, output_final_state=True, activation="silu",
                  cu_seqlens=None, chunk_indices=None, state_width=None, final_state=None):
    """Depthwise causal conv1d with a rolling history over (packed) sequences (lm.py:563-568; the operator
    behind FLA's causal_conv1d_fwd at gdn.py:403-414).

    x [B, T, D]; weight [D, W] or [D, 1, W] (tap 0 oldest); bias [D] or None; all one dtype. State rows
    [N, D, state_width] (default W: the serving layer's [N, D, W]; lm.py keeps W-1): the raw inputs before
    each sequence, oldest first. Returns (y [B, T, D] dense, new state [N, D, state_width] or None);
    ``final_state`` may name the tensor to write, ``initial_state`` itself included. x may be a column slice of
    wider rows (the q|k|v columns of the input projection), read in place."""
    dev = x.device if isinstance(x, torch.Tensor) else None
    x, x_ld = _rows_in_place("x", x, 1, dev)
    _require(x.dim() == 3, f"x: expected [B, T, D], got {tuple(x.shape)}")
    B, T, D = x.shape
    if weight.dim() == 3:
        weight = weight.squeeze(1)
    _on_gpu("weight", weight, dev)
    _require(weight.dim() == 2 and weight.shape[0] == D, f"weight: expected [{D}, W], got {tuple(weight.shape)}")
    W = weight.shape[1]
    sw = W if state_width is None else int(state_width)
    _require(W - 1 <= sw <= 4 and 1 <= W <= 4, f"conv width {W} / state width {sw}: need W <= 4, W-1 <= sw <= 4")
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None:
            _on_gpu(name, t, dev)
            _require(t.dtype == x.dtype, f"{name}: dtype {t.dtype}, expected {x.dtype}")
    if bias is not None:
        _require(bias.shape == (D,), f"bias: expected [{D}]")
    _require(activation in (None, "silu", "swish"), f"activation {activation!r}: supported None, 'silu'")
    n_seqs, n_chunks = B, 0
    if cu_seqlens is not None:
        _require(B == 1, "cu_seqlens: packed sequences need B == 1")
        if _on_host(cu_seqlens):  # host tables: checked here, then copied
            cu_seqlens, chunk_indices = host_tables(cu_seqlens, chunk_indices, T, dev)
        n_seqs = _cu_check(cu_seqlens, T, dev)
        if chunk_indices is None:
            chunk_indices = chunk_indices_from_cu(cu_seqlens, T)
        _on_gpu("chunk_indices", chunk_indices, dev)
        _require(chunk_indices.dtype == torch.int32 and chunk_indices.dim() == 2 and chunk_indices.shape[1] == 2,
                 "chunk_indices: expected int32 [n_chunks, 2]")
        n_chunks = chunk_indices.shape[0]
    for name, t in (("initial_state", initial_state), ("final_state", final_state)):
        if t is not None:
            _on_gpu(name, t, dev)
            _require(t.dtype == x.dtype and t.shape == (n_seqs, D, sw),
                     f"{name}: expected {x.dtype} [{n_seqs}, {D}, {sw}], got {t.dtype} {tuple(t.shape)}")
    if final_state is None and output_final_state:
        final_state = torch.empty(n_seqs, D, sw, device=dev, dtype=x.dtype)
    y = torch.empty(B, T, D, device=dev, dtype=x.dtype)
    _native.call(
        "zgdn_causal_conv1d_fwd", x.data_ptr(), weight.data_ptr(), _ptr(bias), _code(x, "x"), _ptr(initial_state),
        _ptr(final_state), sw, y.data_ptr(), _ptr(cu_seqlens), _ptr(chunk_indices), n_seqs, n_chunks, B, T, D, W,
        1 if activation in ("silu", "swish") else 0, x_ld, _stream(dev),
    )
    return y, final_state


def l2norm(x, eps=1e-6, out_dtype=None):
    """x * rsqrt(sum x^2 + eps) over the last dim (<= 1024); returns (y in ``out_dtype`` (default x's),
    rstd float32 [...]) -- lm.py:570-571 / FLA l2norm_fwd (gdn.py:416-417). x may be a column slice of wider
    rows whose dims after the first are dense (q or k of the conv output, [T, H, D]), read in place; y is
    dense."""
    x, group, ld = _head_rows("x", x)
    D = x.shape[-1]
    rows = x.numel() // D if D else 0
    y = torch.empty(x.shape, device=x.device, dtype=x.dtype if out_dtype is None else out_dtype)
    rstd = torch.empty(x.shape[:-1], device=x.device, dtype=torch.float32)
    _native.call("zgdn_l2norm_fwd", x.data_ptr(), _code(x, "x"), y.data_ptr(), _code(y, "y"), rstd.data_ptr(),
                 rows, D, group, ld, float(eps), _stream(x.device))
    return y, rstd


def sigmoid(x, scale=1.0, out_dtype=torch.float32):
    """sigmoid(x) * scale elementwise (lm.py:573 / FLA fused_beta_sigmoid_fwd at gdn.py:423), in ``out_dtype``."""
    _on_gpu("x", x)
    y = torch.empty(x.shape, device=x.device, dtype=out_dtype)
    _native.call("zgdn_sigmoid_fwd", x.data_ptr(), _code(x, "x"), y.data_ptr(), _code(y, "y"), x.numel(),
                 float(scale), _stream(x.device))
    return y


def gated_rmsnorm(x, g, weight, eps=1e-5):
    """(rms_norm(x) * weight).to(dtype) * silu(g), product in fp32, over rows of the last dim (<= 1024)
    (lm.py:584-587 / FLA layer_norm_gated_fwd at gdn.py:435-445). Returns (y, rstd float32 [...]). g may be a
    column slice of wider rows whose dims after the first are dense (z of the input projection, [T, Hv, V]),
    read in place."""
    _on_gpu("x", x)
    dev = x.device
    D = x.shape[-1]
    _on_gpu("weight", weight, dev)
    _require(weight.dtype == x.dtype, f"weight: dtype {weight.dtype}, expected {x.dtype}")
    g, group, g_ld = _head_rows("g", g, dev)
    _require(g.dtype == x.dtype, f"g: dtype {g.dtype}, expected {x.dtype}")
    _require(g.shape == x.shape and weight.shape == (D,), "gated_rmsnorm: g like x, weight [D]")
    rows = x.numel() // D if D else 0
    y = torch.empty_like(x)
    rstd = torch.empty(x.shape[:-1], device=dev, dtype=torch.float32)
    _native.call("zgdn_gated_rmsnorm_fwd", x.data_ptr(), g.data_ptr(), weight.data_ptr(), _code(x, "x"), y.data_ptr(),
                 rstd.data_ptr(), rows, D, group, g_ld, float(eps), _stream(dev))
    return y, rstd


def accent_shift(x, down, up, mask, y=None, out=None):
    """Accent adapter shift of a projection output: ``y + ((x @ down.T) * mask) @ up`` per row
    (``servers/sgl/src/zonos3_sgl/layers/accent.py:25-62``), the bf16 roundings of those torch ops kept.

    x [rows, in]; down [K, in], up [K, out] (an op's ``_accent``); mask [rows, K]; y [rows, out] or None (the
    shift alone); all one dtype, K <= 256. x, mask and y may be column slices of wider rows. ``out``: the tensor
    to write ([rows, out]; may be ``y`` for an in-place update), else a new one. Rows are independent: a row's
    result does not depend on the other rows of the call."""
    dev = x.device if isinstance(x, torch.Tensor) else None
    bf = isinstance(x, torch.Tensor) and x.dtype == torch.bfloat16
    x, x_ld = _rows_in_place("x", x, 1, dev, 8 if bf else 1, 16 if bf else 1)
    _require(x.dim() == 2, f"x: expected [rows, in], got {tuple(x.shape)}")
    rows, n_in = x.shape
    code = _code(x, "x")
    for name, t in (("down", down), ("up", up)):
        _on_gpu(name, t, dev)
        _require(t.dtype == x.dtype, f"{name}: dtype {t.dtype}, expected {x.dtype}")
    _require(down.dim() == 2 and down.shape[1] == n_in, f"down: expected [K, {n_in}], got {tuple(down.shape)}")
    K = down.shape[0]
    _require(up.dim() == 2 and up.shape[0] == K, f"up: expected [{K}, out], got {tuple(up.shape)}")
    n_out = up.shape[1]
    mask, mask_ld = _rows_in_place("mask", mask, 1, dev)
    _require(mask.dtype == x.dtype and tuple(mask.shape) == (rows, K),
             f"mask: expected {x.dtype} [{rows}, {K}], got {mask.dtype} {tuple(mask.shape)}")
    y_ld = 0
    if y is not None:
        y, y_ld = _rows_in_place("y", y, 1, dev)
        _require(y.dtype == x.dtype and tuple(y.shape) == (rows, n_out),
                 f"y: expected {x.dtype} [{rows}, {n_out}], got {y.dtype} {tuple(y.shape)}")
    if out is None:
        out = torch.empty(rows, n_out, device=dev, dtype=x.dtype)
    _require(isinstance(out, torch.Tensor) and out.is_cuda and out.device == dev and out.dtype == x.dtype
             and tuple(out.shape) == (rows, n_out), f"out: expected {x.dtype} [{rows}, {n_out}] on {dev}")
    out_ld = _row_stride(out, 1)
    _require(out_ld is not None, "out: rows must be contiguous")
    ws_bytes = int(_native.lib().zgdn_accent_workspace_size(rows, n_out, K, code))
    workspace = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    _native.call("zgdn_accent_shift", x.data_ptr(), x_ld, down.data_ptr(), up.data_ptr(), mask.data_ptr(), mask_ld,
                 _ptr(y), y_ld, out.data_ptr(), out_ld, rows, n_in, n_out, K, code, workspace.data_ptr(), ws_bytes,
                 _stream(dev))
    return out


def _gemm_operands(name, x, w, dev):
    x, x_ld = _rows_in_place(name, x, 1, dev, 8, 16)
    _require(x.dim() == 2, f"{name}: expected [M, K], got {tuple(x.shape)}")
    _on_gpu("w", w, dev)
    _require(w.dim() == 2 and w.shape[1] == x.shape[1], f"w: expected [N, {x.shape[1]}], got {tuple(w.shape)}")
    _require(x.dtype == w.dtype == torch.bfloat16, "the projection kernels take bfloat16 operands")
    return x, x_ld


def gemm_nt(x, w, out=None):
    """y = x . w^T (F.linear without bias) on bf16 MFMA with fp32 accumulation, rounded to bf16: the GDN layer's
    projections (in_proj lm.py:561 / gdn.py:399, wo lm.py:602 / gdn.py:447; C ABI ``zgdn_gemm_nt``).

    x [M, K] bfloat16 (rows may be a strided slice), w [N, K] bfloat16 (dense); K a multiple of 128, N of 8.
    Returns y [M, N] bfloat16 (``out``, when given, is written and returned)."""
    dev = x.device if isinstance(x, torch.Tensor) else None
    x, x_ld = _gemm_operands("x", x, w, dev)
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    _require(out.shape == (M, N) and out.dtype == torch.bfloat16 and out.stride(1) == 1,
             f"out: expected bfloat16 [{M}, {N}] with unit column stride")
    _native.call("zgdn_gemm_nt", x.data_ptr(), x_ld, w.data_ptr(), out.data_ptr(), out.stride(0), M, N, K, BF16,
                 _stream(dev))
    return out


def in_proj_conv(x, w, conv_weight, channels, initial_state=None, output_final_state=True):
    """The GDN layer's in_proj with the depthwise causal conv + SiLU of its q|k|v columns fused in, for one
    sequence (lm.py:561-568; C ABI ``zgdn_in_proj_conv``): y[:, :C] = silu(conv(x . w[:C]^T)) with the width-4
    conv over rows (history: the last 3 raw inputs before row 0, oldest first), y[:, C:] = x . w[C:]^T raw.

    x [M, K], w [N, K], conv_weight [C, 4] or [C, 1, 4] bfloat16; ``channels`` = C (a multiple of 128);
    initial_state [C, 3] bfloat16 or None (zeros). Returns (y [M, N] bfloat16, new history [C, 3] or None)."""
    dev = x.device if isinstance(x, torch.Tensor) else None
    x, x_ld = _gemm_operands("x", x, w, dev)
    M, K = x.shape
    N, C = w.shape[0], int(channels)
    if conv_weight.dim() == 3:
        conv_weight = conv_weight.squeeze(1)
    _on_gpu("conv_weight", conv_weight, dev)
    _require(conv_weight.shape == (C, 4) and conv_weight.dtype == torch.bfloat16,
             f"conv_weight: expected bfloat16 [{C}, 4], got {conv_weight.dtype} {tuple(conv_weight.shape)}")
    conv_weight = conv_weight.contiguous()
    if initial_state is not None:
        _on_gpu("initial_state", initial_state, dev)
        _require(initial_state.shape == (C, 3) and initial_state.dtype == torch.bfloat16,
                 f"initial_state: expected bfloat16 [{C}, 3], got {initial_state.dtype} {tuple(initial_state.shape)}")
        initial_state = initial_state.contiguous()
    final = torch.empty(C, 3, device=dev, dtype=torch.bfloat16) if output_final_state else None
    y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    _native.call("zgdn_in_proj_conv", x.data_ptr(), x_ld, w.data_ptr(), y.data_ptr(), N, M, N, K,
                 conv_weight.data_ptr(), C, _ptr(initial_state), _ptr(final), BF16, _stream(dev))
    return y, final
