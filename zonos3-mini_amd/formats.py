"""On-disk formats around the GDN layer: GGUF weight names and the ``state.npz`` state snapshot.

* GGUF: the release LM's GDN tensors are stored under the names of the reference's name contract
  (``tools/convert_gguf.py:111-132``: ``blk.{L}.gdn_in.weight`` for ``attention.in_proj.weight``,
  ``gdn_norm`` for ``out_weight``, ``gdn_A_log``, ``gdn_dt_bias``, ``gdn_conv`` (the conv weight without its
  middle axis), ``attn_output`` for ``wo``) with the ``gdn.head_count`` / ``gdn.head_dim`` /
  ``gdn.conv_kernel`` metadata (``convert_gguf.py:476-478``). ``read_gguf`` parses a GGUF v2/v3 file (its
  published layout: header, typed key/value metadata, tensor infos, aligned data) for the tensor types those
  weights use (F32, F16, BF16, Q8_0), and ``gdn_layer_weights`` returns one layer's weights under the names
  and shapes the layer drop-ins take (``in_proj``, ``conv`` [C, 1, W], ``out_weight``, ``A_log``, ``dt_bias``,
  ``wo``).
* ``state.npz``: the reference's snapshot of a model cache for split-run continuation
  (``tools/dump_golden.py:223-272``) holds, per GDN layer, ``gdn_state_{L}`` ([H, V, K] float32) and
  ``gdn_conv_state_{L}`` ([3 * inner, W - 1], float32 on disk, the model dtype in memory), and ``position``.
  ``gdn_state_arrays`` / ``save_gdn_state`` write those entries from the caches ``layer.gdn`` keeps (device
  tensors are copied to the host), ``load_gdn_state`` checks and loads them (entries of attention layers,
  ``kv_k_{L}`` / ``kv_v_{L}``, belong to the attention caches and are left to their owner).
"""

from __future__ import annotations

import mmap
import struct
from typing import Iterable

import numpy as np
import torch

# ------------------------------------------------------------------------------------------------------- GGUF

# (model parameter of layer L, GGUF name of layer L): the GDN part of the release LM's name contract
GDN_GGUF_NAMES = (
    ("layers.{L}.attention.in_proj.weight", "blk.{L}.gdn_in.weight"),
    ("layers.{L}.attention.out_weight", "blk.{L}.gdn_norm.weight"),
    ("layers.{L}.attention.A_log", "blk.{L}.gdn_A_log"),
    ("layers.{L}.attention.dt_bias", "blk.{L}.gdn_dt_bias"),
    ("layers.{L}.attention.conv.weight", "blk.{L}.gdn_conv.weight"),  # stored as [C, W] (middle axis dropped)
    ("layers.{L}.attention.wo.weight", "blk.{L}.attn_output.weight"),
)
GDN_GGUF_METADATA = ("gdn.head_count", "gdn.head_dim", "gdn.conv_kernel")

# ggml tensor types used by these weights: code -> (name, elements per block, bytes per block)
GGML_TYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 8: ("Q8_0", 32, 34), 30: ("BF16", 1, 2)}

_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
_STRING, _ARRAY = 8, 9


class _Cursor:
    def __init__(self, buf):
        self.buf, self.at = buf, 0

    def take(self, fmt):
        value = struct.unpack_from(fmt, self.buf, self.at)[0]
        self.at += struct.calcsize(fmt)
        return value

    def string(self):
        n = self.take("<Q")
        s = bytes(self.buf[self.at:self.at + n]).decode("utf-8")
        self.at += n
        return s

    def value(self, vtype):
        if vtype in _SCALARS:
            return self.take(_SCALARS[vtype])
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            etype, n = self.take("<I"), self.take("<Q")
            return [self.value(etype) for _ in range(n)]
        raise ValueError(f"GGUF: unknown metadata value type {vtype}")


class GGUFTensor:
    """One tensor of a GGUF file: ``shape`` in torch order (the reverse of ggml's ne), its ggml type, and
    ``data``, a read-only view of its bytes in the file."""

    def __init__(self, name, shape, ggml_type, data):
        self.name, self.shape, self.ggml_type, self.data = name, shape, ggml_type, data

    @property
    def type_name(self) -> str:
        return GGML_TYPES[self.ggml_type][0] if self.ggml_type in GGML_TYPES else f"type {self.ggml_type}"

    def numpy(self) -> np.ndarray:
        """The tensor as float32 (Q8_0 blocks dequantised: 32 int8 values times their fp16 scale)."""
        if self.ggml_type not in GGML_TYPES:
            raise ValueError(f"GGUF tensor {self.name}: ggml type {self.ggml_type} is not supported here")
        n = int(np.prod(self.shape)) if self.shape else 1
        raw = np.frombuffer(self.data, dtype=np.uint8)
        kind = GGML_TYPES[self.ggml_type][0]
        if kind == "F32":
            out = raw.view("<f4").copy()
        elif kind == "F16":
            out = raw.view("<f2").astype(np.float32)
        elif kind == "BF16":
            out = (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
        else:  # Q8_0
            blocks = raw.reshape(-1, 34)
            scale = blocks[:, :2].copy().view("<f2").astype(np.float32)
            out = (blocks[:, 2:].view(np.int8).astype(np.float32) * scale).reshape(-1)
        if out.size != n:
            raise ValueError(f"GGUF tensor {self.name}: {out.size} values for shape {self.shape}")
        return out.reshape(self.shape)


def read_gguf(path) -> tuple[dict, dict]:
    """(metadata, tensors by name) of a GGUF v2 / v3 file; tensor data is memory-mapped, not copied."""
    with open(path, "rb") as f:
        buf = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    cur = _Cursor(buf)
    if bytes(buf[:4]) != b"GGUF":
        raise ValueError(f"{path}: not a GGUF file")
    cur.at = 4
    version = cur.take("<I")
    if version not in (2, 3):
        raise ValueError(f"{path}: GGUF version {version} (supported: 2, 3)")
    n_tensors, n_kv = cur.take("<Q"), cur.take("<Q")
    meta = {}
    for _ in range(n_kv):
        key = cur.string()
        meta[key] = cur.value(cur.take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = cur.string()
        ndim = cur.take("<I")
        ne = [cur.take("<Q") for _ in range(ndim)]
        infos.append((name, tuple(reversed(ne)), cur.take("<I"), cur.take("<Q")))
    align = int(meta.get("general.alignment", 32))
    base = (cur.at + align - 1) // align * align
    view = memoryview(buf)
    tensors = {}
    for name, shape, ggml_type, offset in infos:
        count = int(np.prod(shape)) if shape else 1
        if ggml_type in GGML_TYPES:
            _, per_block, block_bytes = GGML_TYPES[ggml_type]
            if count % per_block:
                raise ValueError(f"GGUF tensor {name}: {count} values do not fill {per_block}-value blocks")
            nbytes = count // per_block * block_bytes
        else:
            nbytes = 0  # listed, but not readable here
        start = base + offset
        if start + nbytes > len(buf):
            raise ValueError(f"GGUF tensor {name}: data past the end of the file")
        tensors[name] = GGUFTensor(name, shape, ggml_type, view[start:start + nbytes])
    return meta, tensors


def gdn_layer_weights(tensors: dict, layer: int) -> dict:
    """One GDN layer's weights from GGUF tensors (as ``read_gguf`` returns them) as float32 torch tensors
    under the layer drop-ins' names: in_proj [4*inner + 2*H, dim], conv [3*inner, 1, W], out_weight [V],
    A_log [H], dt_bias [H], wo [dim, inner]."""
    out = {}
    for param, gguf_name in GDN_GGUF_NAMES:
        name = gguf_name.format(L=layer)
        if name not in tensors:
            raise KeyError(f"GGUF file has no {name} (layer {layer} is not a GDN layer?)")
        t = torch.from_numpy(tensors[name].numpy())
        key = param.format(L=layer).split(".attention.")[1].removesuffix(".weight")
        out[key] = t.unsqueeze(1) if key == "conv" else t
    return out


# -------------------------------------------------------------------------------------------------- state.npz


def gdn_state_arrays(cache, layers: Iterable[int]) -> dict:
    """The GDN entries of a ``state.npz`` snapshot from a cache holding ``gdn_state`` / ``conv_state`` per
    layer (``[H, V, K]`` float32 and ``[3 * inner, W - 1]``), as float32 host arrays."""
    arrays = {}
    for layer in layers:
        arrays[f"gdn_conv_state_{layer}"] = cache.conv_state[layer].detach().float().cpu().numpy()
        arrays[f"gdn_state_{layer}"] = cache.gdn_state[layer].detach().float().cpu().numpy()
    return arrays


def save_gdn_state(path, cache, layers: Iterable[int], position: int, extra: dict | None = None) -> None:
    """Write a ``state.npz`` with the GDN layers' entries, ``position`` (int64) and any ``extra`` entries
    (the attention layers' ``kv_k_{L}`` / ``kv_v_{L}``, owned by their caches)."""
    arrays = gdn_state_arrays(cache, layers)
    arrays.update(extra or {})
    np.savez(path, position=np.asarray(position, dtype=np.int64), **arrays)


def load_gdn_state(path, cache, layers: Iterable[int], dtype: torch.dtype, device, heads: int = 4,
                   head_dim: int = 128, conv_kernel: int = 4) -> int:
    """Load the GDN entries of a ``state.npz`` into ``cache.gdn_state`` (float32) / ``cache.conv_state``
    (``dtype``) on ``device``; returns ``position``. Every GDN entry must be present, finite and of its
    shape (``ValueError`` otherwise); entries other than the GDN ones and ``position`` are ignored."""
    with np.load(path, allow_pickle=False) as state:
        position = np.asarray(state["position"])
        if position.shape != () or int(position) < 0 or int(position) != position:
            raise ValueError("state.npz: invalid position")
        inner = heads * head_dim
        for layer in layers:
            for name, shape, tdt in ((f"gdn_state_{layer}", (heads, head_dim, head_dim), torch.float32),
                                     (f"gdn_conv_state_{layer}", (3 * inner, conv_kernel - 1), dtype)):
                if name not in state.files:
                    raise ValueError(f"state.npz: missing {name}")
                arr = state[name]
                if arr.shape != shape or not np.isfinite(arr).all():
                    raise ValueError(f"state.npz: invalid {name}: expected {shape}, got {arr.shape}")
                t = torch.from_numpy(arr.copy()).to(device=device, dtype=tdt)
                (cache.gdn_state if name.startswith("gdn_state") else cache.conv_state)[layer] = t
    return int(position)

