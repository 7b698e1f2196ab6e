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
    assert {"zgdn_last_error", "zgdn_abi_version", "zgdn_recurrent_fwd", "zgdn_chunk_fwd", "zgdn_chunk_workspace_size",
            "zgdn_fused_decode_step", "zgdn_causal_conv1d_fwd", "zgdn_l2norm_fwd", "zgdn_sigmoid_fwd",
            "zgdn_gated_rmsnorm_fwd", "zgdn_serving_decode_step", "zgdn_attnres_route", "zgdn_accent_workspace_size",
            "zgdn_accent_shift", "zgdn_chunk_segment_workspace_size", "zgdn_chunk_set_launch_form",
            "zgdn_chunk_get_launch_form", "zgdn_chunk_status", "zgdn_chunk_set_wait_limit",
            "zgdn_chunk_status_async", "zgdn_chunk_overlap_queues",
            "zgdn_chunk_noalloc_max_bytes", "zgdn_chunk_fwd_noalloc", "zgdn_chunk_workspace_bytes", "zgdn_gemm_nt",
            "zgdn_in_proj_conv"} == _declared()


def test_library_exports_every_declared_symbol(gdn):
    from importlib import import_module

    native = import_module("zonos3-mini_amd._native")
    lib = native.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(native.SIGNATURES) == _declared()
    assert lib.zgdn_abi_version() == native.ABI_VERSION == 2


def test_segment_workspace_follows_the_plan(gdn):
    """Sizing of the segmented state pass (no device: 256 CUs assumed). Short prompts, many heads or many
    sequences take the plain pass (no extra bytes); one 4096-token sequence of 4 heads runs 4 segments: Q'P^T
    (bf16, a token and head) plus, a head, 4 local end states (fp32), 3 maps (bf16 hi and lo) and 3 segment
    start states (bf16)."""
    from importlib import import_module

    lib = import_module("zonos3-mini_amd._native").lib()
    f = lib.zgdn_chunk_segment_workspace_size
    assert f(1, 1024, 4) == 0 and f(1, 2048, 4) == 0 and f(1, 4096, 16) == 0 and f(8, 4096, 4) == 0
    hs = 128 * 128
    assert f(1, 4096, 4) == 4096 * 4 * 128 * 2 + 4 * hs * (4 * 4 + 4 * 3 + 2 * 3)
    assert f(1, 3072, 4) > 0 and f(2, 4096, 4) > 0


def _rec_args(**over):
    """Arguments of zgdn_recurrent_fwd by name (pointers are dummies: every call here fails validation)."""
    p = ctypes.c_void_p(16)
    a = dict(q=p, k=p, v=p, qkv_dtype=1, g=p, beta=p, gb_dtype=0, A_log=None, dt_bias=None, qk_l2norm=0,
             s_in=None, s_out=None, o=p, o_dtype=1, cu=None, n_seqs=1, B=1, T=1, Hk=1, Hv=1, K=128, V=128,
             scale=1.0, stream=None)
    a.update(over)
    return list(a.values())


def test_bad_arguments_fail_with_a_message(gdn):
    from importlib import import_module

    native = import_module("zonos3-mini_amd._native")
    lib = native.lib()
    p = ctypes.c_void_p(16)
    cases = [
        (_rec_args(q=None), native.EINVAL, b"null"),
        (_rec_args(Hk=3, Hv=4), native.EINVAL, b"multiple"),
        (_rec_args(K=96), native.EUNSUPPORTED, b"K=96"),
        (_rec_args(cu=p, n_seqs=2, B=2), native.EINVAL, b"cu_seqlens"),
        (_rec_args(A_log=p), native.EINVAL, b"together"),
        (_rec_args(gb_dtype=7), native.EINVAL, b"dtype"),
    ]
    for args, code, msg in cases:
        assert lib.zgdn_recurrent_fwd(*args) == code
        assert msg in lib.zgdn_last_error()
    with pytest.raises(RuntimeError, match="null"):
        native.call("zgdn_recurrent_fwd", *_rec_args(q=None))
    # chunked prefill: head size, dtype and workspace checks
    chunk = [p, p, p, 1, p, p, 0, None, None, 0, None, None, p, None, None, 1, 0, 1, 64, 1, 1, 128, 128,
             128, 128, 128, 1, 0, 1.0, p, 0, None]
    assert lib.zgdn_chunk_fwd(*chunk) == native.EINVAL and b"workspace" in lib.zgdn_last_error()
    chunk[23] = 1536 + 4  # q row stride not a multiple of 8 elements
    assert lib.zgdn_chunk_fwd(*chunk) == native.EINVAL and b"row strides" in lib.zgdn_last_error()
    chunk[23], chunk[26] = 128, 0  # g/beta rows narrower than the heads
    assert lib.zgdn_chunk_fwd(*chunk) == native.EINVAL and b"row strides" in lib.zgdn_last_error()
    chunk[26] = 1
    chunk[21] = 96  # K
    assert lib.zgdn_chunk_fwd(*chunk) == native.EUNSUPPORTED and b"K=96" in lib.zgdn_last_error()
    chunk[21], chunk[22] = 64, 128  # K != V
    assert lib.zgdn_chunk_fwd(*chunk) == native.EUNSUPPORTED and b"K=64 V=128" in lib.zgdn_last_error()
    chunk[21], chunk[3] = 128, 5  # q/k/v dtype code
    assert lib.zgdn_chunk_fwd(*chunk) == native.EINVAL and b"dtype code 5" in lib.zgdn_last_error()
    # fp32 q/k/v (and 64-wide heads) take the fp32-arithmetic path: its workspace, its row-stride multiple
    chunk[3] = 0
    assert lib.zgdn_chunk_fwd(*chunk) == native.EINVAL and b"workspace" in lib.zgdn_last_error()
    chunk[23] = 1536 + 4  # a multiple of 4 fp32 elements: accepted by the stride check (then the workspace)
    assert lib.zgdn_chunk_fwd(*chunk) == native.EINVAL and b"workspace" in lib.zgdn_last_error()
    chunk[23] = 1536 + 2
    assert lib.zgdn_chunk_fwd(*chunk) == native.EINVAL and b"multiples of 4" in lib.zgdn_last_error()
    chunk[23], chunk[3] = 128, 1
    # projection kernels: dtype, K multiple of 128, strides, conv channels, in-place history
    # (every call here fails validation or has no rows: none launches with these dummy pointers)
    gemm = [p, 1024, p, p, 2056, 64, 2056, 1000, 1, None]
    assert lib.zgdn_gemm_nt(*gemm) == native.EINVAL and b"K=1000" in lib.zgdn_last_error()
    gemm[7], gemm[8] = 1024, 0
    assert lib.zgdn_gemm_nt(*gemm) == native.EUNSUPPORTED and b"bf16 only" in lib.zgdn_last_error()
    gemm[8], gemm[5] = 1, 0
    assert lib.zgdn_gemm_nt(*gemm) == native.OK  # no rows: nothing to launch
    proj = [p, 1024, p, p, 2056, 64, 2056, 1024, p, 1500, None, None, 1, None]
    assert lib.zgdn_in_proj_conv(*proj) == native.EINVAL and b"C=1500" in lib.zgdn_last_error()
    proj[9], proj[10], proj[11] = 1536, p, p
    assert lib.zgdn_in_proj_conv(*proj) == native.EINVAL and b"in place" in lib.zgdn_last_error()
    # per-dtype workspace: the bf16 path's at 128; 5 fp32 blocks of 64 x D + 256 bytes an item otherwise
    wb = lib.zgdn_chunk_workspace_bytes
    assert wb(64, 16, 128, 128, 1) == lib.zgdn_chunk_workspace_size(64, 16)
    assert wb(64, 16, 128, 128, 0) == 64 * 16 * (5 * 64 * 128 * 4 + 256) == 64 * 16 * 164096
    assert wb(4, 4, 64, 64, 0) == wb(4, 4, 64, 64, 1) == 16 * (5 * 64 * 64 * 4 + 256) == 16 * 82176
    assert wb(4, 4, 96, 96, 0) == 0 and wb(4, 4, 64, 128, 1) == 0 and wb(4, 4, 128, 128, 3) == 0
    # items, then the control block of the overlapped launch (45 x 256 bytes: tickets, per-CU arrival counts;
    # then one 4-byte flag per item)
    assert lib.zgdn_chunk_workspace_size(64, 16) == 64 * 16 * 98560 + 256 * 45 + 64 * 16 * 4
    # conv width, state width; row-op sizes; fused block group size
    conv = [p, p, None, 1, None, None, 4, p, None, None, 1, 0, 1, 8, 16, 5, 1, 16, None]
    assert lib.zgdn_causal_conv1d_fwd(*conv) == native.EUNSUPPORTED and b"width 5" in lib.zgdn_last_error()
    conv[15], conv[6] = 4, 2
    assert lib.zgdn_causal_conv1d_fwd(*conv) == native.EINVAL and b"state width" in lib.zgdn_last_error()
    conv[6], conv[17] = 4, 8
    assert lib.zgdn_causal_conv1d_fwd(*conv) == native.EINVAL and b"row stride" in lib.zgdn_last_error()
    assert lib.zgdn_l2norm_fwd(p, 1, p, 1, None, 4, 2048, 1, 2048, 1e-6, None) == native.EUNSUPPORTED
    assert lib.zgdn_l2norm_fwd(p, 1, p, 1, None, 8, 128, 4, 256, 1e-6, None) == native.EINVAL
    assert b"x rows" in lib.zgdn_last_error()
    assert lib.zgdn_gated_rmsnorm_fwd(p, None, p, 1, p, None, 4, 128, 1, 128, 1e-5, None) == native.EINVAL
    assert lib.zgdn_gated_rmsnorm_fwd(p, p, p, 1, p, None, 4, 128, 4, 500, 1e-5, None) == native.EINVAL
    assert b"gate rows" in lib.zgdn_last_error()
    assert lib.zgdn_sigmoid_fwd(p, 5, p, 0, 10, 1.0, None) == native.EINVAL
    fused = [p, p, p, p, 1, p, p, p, p, p, p, p, 2, 1, 8, 128, 128, 4, 1e-6, 1.0, 0, None]
    assert lib.zgdn_fused_decode_step(*fused) == native.EUNSUPPORTED and b"Hv/Hk=8" in lib.zgdn_last_error()
    fused[14], fused[17] = 2, 3
    assert lib.zgdn_fused_decode_step(*fused) == native.EUNSUPPORTED and b"width 3" in lib.zgdn_last_error()
    # mixed, ld, x, hidden, dtype, slots, n_slots, B, Hk, Hv, K, V, W, conv_w, conv_live, conv_commit, state_live,
    # state_commit, window, win_len, window_rows, A_log, dt_bias, norm_w, out, eps, scale, qk_round, stream
    serve = [p, 2056, p, 256, 1, p, 4, 2, 4, 4, 128, 128, 4, p, p, p, p, p, p, p, 64, p, p, p, p, 1e-5, 1.0, 1, None]
    serve[1] = 2055
    assert lib.zgdn_serving_decode_step(*serve) == native.EINVAL and b"holds no q|k|v" in lib.zgdn_last_error()
    serve[1], serve[14] = 2056, None
    assert lib.zgdn_serving_decode_step(*serve) == native.EINVAL and b"null pointer" in lib.zgdn_last_error()
    serve[14], serve[9] = p, 32
    assert lib.zgdn_serving_decode_step(*serve) == native.EUNSUPPORTED and b"Hv/Hk=8" in lib.zgdn_last_error()
    serve[9], serve[6] = 4, 0
    assert lib.zgdn_serving_decode_step(*serve) == native.EINVAL and b"n_slots=0" in lib.zgdn_last_error()
    srcs = (ctypes.c_void_p * 2)(16, 16)
    assert lib.zgdn_attnres_route(srcs, 65, 4, 1024, 1024, 1, p, 1e-5, p, None) == native.EUNSUPPORTED
    assert lib.zgdn_attnres_route(srcs, 2, 4, 1028, 1028, 1, p, 1e-5, p, None) == native.EUNSUPPORTED
    assert b"multiple of 8" in lib.zgdn_last_error()
    assert lib.zgdn_attnres_route(srcs, 2, 4, 1024, 1000, 1, p, 1e-5, p, None) == native.EINVAL
    srcs[1] = None
    assert lib.zgdn_attnres_route(srcs, 2, 4, 1024, 1024, 1, p, 1e-5, p, None) == native.EINVAL
    assert b"null source 1" in lib.zgdn_last_error()
    # accent shift: x, x_ld, down, up, mask, mask_ld, y_in, y_in_ld, y_out, y_out_ld, rows, in, out, K, dtype,
    # workspace, bytes, stream (no call below passes validation, so none launches)
    assert lib.zgdn_accent_workspace_size(100, 2056, 40, 1) == 100 * 64 * 2
    assert lib.zgdn_accent_workspace_size(100, 2056, 40, 0) == 100 * 64 * 4
    acc = [p, 1024, p, p, p, 64, p, 2056, p, 2056, 100, 1024, 2056, 64, 1, p, 0, None]
    assert lib.zgdn_accent_shift(*acc) == native.EINVAL and b"workspace" in lib.zgdn_last_error()
    acc[13] = 300
    assert lib.zgdn_accent_shift(*acc) == native.EUNSUPPORTED and b"K=300" in lib.zgdn_last_error()
    acc[13], acc[12] = 64, 2052
    assert lib.zgdn_accent_shift(*acc) == native.EINVAL and b"multiples of 8" in lib.zgdn_last_error()
    acc[12], acc[5] = 2056, 32
    assert lib.zgdn_accent_shift(*acc) == native.EINVAL and b"row strides" in lib.zgdn_last_error()


def test_host_validation_refuses_cpu_tensors(gdn):
    import torch

    q = torch.zeros(1, 2, 1, 128)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        gdn.recurrent_fwd(q, q, q, torch.zeros(1, 2, 1), torch.zeros(1, 2, 1))


def test_launch_form_and_wait_limit_controls(gdn):
    """The process-wide launch-form switch (no environment read per call) and the wait-limit test switch:
    valid values are taken and restored, invalid ones rejected with a message, without a device."""
    from importlib import import_module

    native = import_module("zonos3-mini_amd._native")
    ops = import_module("zonos3-mini_amd.ops")
    lib = native.lib()
    before = lib.zgdn_chunk_get_launch_form()
    with ops.launch_form(0):
        assert lib.zgdn_chunk_get_launch_form() == 0
        with ops.launch_form(1):
            assert lib.zgdn_chunk_get_launch_form() == 1
        assert lib.zgdn_chunk_get_launch_form() == 0
    assert lib.zgdn_chunk_get_launch_form() == before
    assert lib.zgdn_chunk_set_launch_form(2) == native.EINVAL
    assert b"form 2" in lib.zgdn_last_error()
    assert lib.zgdn_chunk_set_wait_limit(-1, 0) == native.EINVAL
    assert lib.zgdn_chunk_set_wait_limit(0, 0) == native.OK
    assert lib.zgdn_chunk_status(None, 0) == native.EINVAL
    assert lib.zgdn_chunk_status_async(None, None) == native.EINVAL


def test_overlap_queue_mapping(gdn):
    """The overlapped launch's queues: one per XCD when the CUs split evenly over 1 .. 8 XCDs (MI355X: 256 CUs,
    8 XCDs), else 0 -- the two-launch form then runs (a host-only function, no GPU call)."""
    from importlib import import_module

    lib = import_module("zonos3-mini_amd._native").lib()
    assert lib.zgdn_chunk_overlap_queues(256, 8) == 8
    assert lib.zgdn_chunk_overlap_queues(32, 1) == 1    # one XCD of a partitioned device
    assert lib.zgdn_chunk_overlap_queues(128, 4) == 4
    assert lib.zgdn_chunk_overlap_queues(304, 8) == 8   # 38 CUs per XCD
    assert lib.zgdn_chunk_overlap_queues(256, 0) == 0   # unknown XCD count
    assert lib.zgdn_chunk_overlap_queues(256, 16) == 0  # more XCDs than the control block has queues
    assert lib.zgdn_chunk_overlap_queues(250, 8) == 0   # CUs that do not split evenly
    assert lib.zgdn_chunk_overlap_queues(4, 8) == 0


def test_launch_form_reads_the_environment_once_at_load():
    """ZGDN_CHUNK_OVERLAP is read when the library is loaded (a fresh process), not at each call."""
    import os
    import subprocess
    import sys

    code = ("import importlib, os; n = importlib.import_module('zonos3-mini_amd._native'); lib = n.lib(); "
            "a = lib.zgdn_chunk_get_launch_form(); os.environ['ZGDN_CHUNK_OVERLAP'] = '1'; "
            "print(a, lib.zgdn_chunk_get_launch_form())")
    env = dict(os.environ, ZGDN_CHUNK_OVERLAP="0")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.split() == ["0", "0"]
