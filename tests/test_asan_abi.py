"""The C ABI's argument validation under AddressSanitizer, on the CPU: every library source is built with
AddressSanitizer on its host code and linked into tests/asan/abi_checks.cpp, which calls each entry point of
include/zonos3_gdn.h with arguments its checks reject (null pointers, unsupported sizes, short workspaces, bad
strides, a source-pointer array of exactly the size passed) and checks the status codes and messages. An
out-of-bounds host access is an AddressSanitizer report and a non-zero exit."""

from __future__ import annotations

import importlib.util
import os
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _builder():
    spec = importlib.util.spec_from_file_location("zgdn_build", ROOT / "zonos3-mini_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_validation_paths_under_address_sanitizer():
    exe = _builder().build_asan()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0")  # (the HIP runtime keeps its state)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert "AddressSanitizer" not in res.stderr, res.stderr[-4000:]
    assert res.returncode == 0, res.stderr[-4000:]
    assert "0 failed checks" in res.stderr
