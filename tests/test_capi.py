"""The C ABI without a GPU: the library loads, exports every declared entry point, and rejects bad
arguments with a status and a message before touching the device."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(zgdn_\w+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    assert {"zgdn_last_error", "zgdn_abi_version", "zgdn_recurrent_fwd"} <= _declared()


def test_library_exports_every_declared_symbol(gdn):
    from importlib import import_module

    native = import_module("zonos3-mini_amd._native")
    lib = native.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(native.SIGNATURES) == _declared()
    assert lib.zgdn_abi_version() == 1


def test_bad_arguments_fail_with_a_message(gdn):
    from importlib import import_module

    native = import_module("zonos3-mini_amd._native")
    lib = native.lib()
    p = ctypes.c_void_p(16)
    # null pointers
    st = lib.zgdn_recurrent_fwd(None, p, p, 1, p, p, 0, None, None, p, 1, None, 1, 1, 1, 1, 1, 128, 128, 1.0, None)
    assert st == native.EINVAL and b"null" in lib.zgdn_last_error()
    # grouped heads that do not divide
    st = lib.zgdn_recurrent_fwd(p, p, p, 1, p, p, 0, None, None, p, 1, None, 1, 1, 1, 3, 4, 128, 128, 1.0, None)
    assert st == native.EINVAL and b"multiple" in lib.zgdn_last_error()
    # unsupported head size
    st = lib.zgdn_recurrent_fwd(p, p, p, 1, p, p, 0, None, None, p, 1, None, 1, 1, 1, 1, 1, 96, 128, 1.0, None)
    assert st == native.EUNSUPPORTED and b"K=96" in lib.zgdn_last_error()
    # packed sequences need B == 1
    st = lib.zgdn_recurrent_fwd(p, p, p, 1, p, p, 0, None, None, p, 1, p, 2, 2, 1, 1, 1, 128, 128, 1.0, None)
    assert st == native.EINVAL and b"cu_seqlens" in lib.zgdn_last_error()
    with pytest.raises(RuntimeError, match="null"):
        native.call("zgdn_recurrent_fwd", None, p, p, 1, p, p, 0, None, None, p, 1, None, 1, 1, 1, 1, 1, 128, 128,
                    1.0, None)


def test_host_validation_refuses_cpu_tensors(gdn):
    import torch

    q = torch.zeros(1, 2, 1, 128)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        gdn.recurrent_fwd(q, q, q, torch.zeros(1, 2, 1), torch.zeros(1, 2, 1))
