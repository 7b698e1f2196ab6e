"""Shared helpers of the test-suite: error measures, case naming, a GGUF writer."""

from __future__ import annotations

import struct
import sys
from pathlib import Path

import numpy as np
import torch


def rel_err(got, want) -> float:
    """max |got - want| / max |want| (float64)."""
    got = np.asarray(got.detach().cpu().double() if torch.is_tensor(got) else got, dtype=np.float64)
    want = np.asarray(want.detach().cpu().double() if torch.is_tensor(want) else want, dtype=np.float64)
    scale = np.abs(want).max() if want.size else 0.0
    return float(np.abs(got - want).max() / scale) if scale > 0 else float(np.abs(got - want).max(initial=0.0))


def max_abs(got, want) -> float:
    got = got.detach().cpu().double() if torch.is_tensor(got) else torch.as_tensor(got, dtype=torch.float64)
    want = want.detach().cpu().double() if torch.is_tensor(want) else torch.as_tensor(want, dtype=torch.float64)
    return float((got - want).abs().max()) if got.numel() else 0.0


def announce(msg: str) -> None:
    """Name the case on stderr before a GPU step, flushed, so a fault can be attributed."""
    print(f"[case] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------------------------------------ a GGUF writer


def _gguf_string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _gguf_value(v) -> bytes:
    if isinstance(v, bool):
        return struct.pack("<I?", 7, v)
    if isinstance(v, int):
        return struct.pack("<II", 4, v)
    if isinstance(v, float):
        return struct.pack("<If", 6, v)
    if isinstance(v, str):
        return struct.pack("<I", 8) + _gguf_string(v)
    assert isinstance(v, list) and all(isinstance(x, int) for x in v)
    return struct.pack("<IIQ", 9, 5, len(v)) + b"".join(struct.pack("<i", x) for x in v)


def write_gguf(path, meta: dict, tensors: dict, align=32) -> None:
    """GGUF v3 with ``tensors`` = name -> (ggml type code, raw bytes, torch-order shape)."""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta) + 1)
    kv = _gguf_string("general.alignment") + struct.pack("<II", 4, align)
    kv += b"".join(_gguf_string(k) + _gguf_value(v) for k, v in meta.items())
    infos, blobs, offset = b"", b"", 0
    for name, (code, raw, shape) in tensors.items():
        pad = (-offset) % align
        blobs += b"\0" * pad
        offset += pad
        infos += _gguf_string(name) + struct.pack("<I", len(shape)) + b"".join(
            struct.pack("<Q", d) for d in reversed(shape)) + struct.pack("<IQ", code, offset)
        blobs += raw
        offset += len(raw)
    body = head + kv + infos
    body += b"\0" * ((-len(body)) % align)
    Path(path).write_bytes(body + blobs)


def q8_0(values: np.ndarray) -> bytes:
    """Q8_0 blocks: per 32 values an fp16 scale max|x|/127 and the int8 round(x / scale)."""
    out = b""
    for blk in values.reshape(-1, 32):
        d = np.float16(np.abs(blk).max() / 127.0)
        q = np.clip(np.rint(blk / np.float32(d)), -127, 127).astype(np.int8) if d else np.zeros(32, np.int8)
        out += d.tobytes() + q.tobytes()
    return out
