"""zgdn_chunk_fwd_noalloc, the chunked forward for callers that cannot allocate (its workspace is the library's
per-device static scratch), called through the C ABI with caller-allocated outputs: on two calls in a row, the
second smaller, its outputs and final states equal zgdn_chunk_fwd's on the same inputs bit for bit (the same
kernels; the scratch keeps the first call's contents, so anything the second call read without writing would
show) and sit within tolerance of the oracle (bf16: outputs 2e-2 max-abs, states 1e-3 relative). The same holds
for each of the path's launch forms in the scratch: the plain two launches, the overlapped launch (whose control
block in the scratch must start each call at zero) and the segmented state pass (whose extra space follows the
workspace in the scratch); and for calls captured into a HIP graph and replayed with new inputs. A call whose
workspace exceeds the scratch is refused before any launch."""

from __future__ import annotations

import pytest
import torch

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _noalloc(gdn, x, o, final, s0, cu=None, chunks=None, A_log=None, dt_bias=None):
    """One zgdn_chunk_fwd_noalloc call through ctypes; q, k, v dense bf16, g / beta float32."""
    B, T, Hk, K = x["q"].shape
    Hv = x["v"].shape[2]
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    n_seqs = B if cu is None else cu.numel() - 1
    n_chunks = 0 if chunks is None else chunks.shape[0]
    stream = torch.cuda.current_stream().cuda_stream
    gdn._native.call("zgdn_chunk_fwd_noalloc", x["q"].data_ptr(), x["k"].data_ptr(), x["v"].data_ptr(),
                     gdn._native.BF16, x["g"].data_ptr(), x["beta"].data_ptr(), gdn._native.F32, ptr(A_log),
                     ptr(dt_bias), 0, ptr(s0), final.data_ptr(), o.data_ptr(), ptr(cu), ptr(chunks), n_seqs,
                     n_chunks, B, T, Hk, Hv, K, 128, Hk * K, Hk * K, Hv * 128, Hv, 0, K**-0.5, stream)


def _case(cuda, B, T, Hk, Hv, seed, lengths=None):
    n = B if lengths is None else len(lengths)
    d = O.make_inputs(B, T, Hk, Hv, 128, 128, seed=seed, dtype=torch.bfloat16, state_std=0.02, n_states=n)
    return d, {k: v.to(cuda) for k, v in d.items()}


def test_noalloc_matches_the_allocating_entry_on_two_calls(gdn, cuda):
    announce("chunk no-alloc: call 1 B=2 T=1000 Hk=4 Hv=8 gate")
    lib = gdn._native.lib()
    assert lib.zgdn_chunk_noalloc_max_bytes() == 64 << 20
    # call 1: two sequences, grouped heads, the in-kernel gate
    d, x = _case(cuda, 2, 1000, 4, 8, seed=7001)
    gen = torch.Generator().manual_seed(7002)
    a = torch.randn(2, 1000, 8, generator=gen)
    A_log, dt_bias = 0.3 * torch.randn(8, generator=gen), 0.3 * torch.randn(8, generator=gen)
    x["g"] = a.to(cuda)
    A_d, dt_d = A_log.to(cuda), dt_bias.to(cuda)
    o = torch.empty(2, 1000, 8, 128, dtype=torch.bfloat16, device=cuda)
    final = torch.empty(2, 8, 128, 128, device=cuda)
    _noalloc(gdn, x, o, final, x["s0"], A_log=A_d, dt_bias=dt_d)
    o_ref, s_ref = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"], A_log=A_d,
                                 dt_bias=dt_d)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(final, s_ref)
    g_log = -A_log.exp() * torch.nn.functional.softplus(a + dt_bias)
    o_cpu, s_cpu = O.gated_delta_recurrence(d["q"], d["k"], d["v"], g_log, d["beta"], None, d["s0"])
    assert max_abs(o.cpu(), o_cpu) < 2e-2 and rel_err(final.cpu(), s_cpu) < 1e-3

    # call 2, smaller: packed sequences (an empty one among them), fewer heads, in the same scratch
    announce("chunk no-alloc: call 2 packed [100, 1, 0, 64] Hk=2 Hv=4")
    lengths = [100, 1, 0, 64]
    cu, chunks = O.chunk_tables(lengths)
    d, x = _case(cuda, 1, sum(lengths), 2, 4, seed=7003, lengths=lengths)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    ch_t = torch.tensor(chunks, dtype=torch.int32, device=cuda)
    o = torch.empty(1, sum(lengths), 4, 128, dtype=torch.bfloat16, device=cuda)
    final = torch.empty(len(lengths), 4, 128, 128, device=cuda)
    _noalloc(gdn, x, o, final, x["s0"], cu=cu_t, chunks=ch_t)
    o_ref, s_ref = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"], cu_seqlens=cu_t,
                                 chunk_indices=ch_t)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(final, s_ref)
    o_cpu, s_cpu = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"], None, d["s0"],
                                            cu_seqlens=cu)
    assert max_abs(o.cpu(), o_cpu) < 2e-2 and rel_err(final.cpu(), s_cpu) < 1e-3
    assert torch.equal(final[2].cpu(), d["s0"][2])  # the empty sequence passes its state through
    assert gdn.ops.chunk_status() == 0


def test_noalloc_refuses_more_than_its_scratch(gdn, cuda):
    """T=4096, H=16 needs ~96 MiB of workspace: refused with ZGDN_EINVAL and a message, nothing launched."""
    lib = gdn._native.lib()
    p = 16  # dummy pointers: the size check comes first
    st = lib.zgdn_chunk_fwd_noalloc(p, p, p, gdn._native.BF16, p, p, gdn._native.F32, None, None, 0, None, None,
                                    p, None, None, 1, 0, 1, 4096, 16, 16, 128, 128, 2048, 2048, 2048, 16, 0,
                                    128**-0.5, None)
    assert st == gdn._native.EINVAL
    assert b"scratch" in lib.zgdn_last_error()


def _pair(gdn, cuda, B, T, H, seed):
    """One no-alloc call and one zgdn_chunk_fwd call on the same inputs (zero initial states); both results."""
    d, x = _case(cuda, B, T, H, H, seed=seed)
    o = torch.empty(B, T, H, 128, dtype=torch.bfloat16, device=cuda)
    final = torch.empty(B, H, 128, 128, device=cuda)
    _noalloc(gdn, x, o, final, None)
    o_ref, s_ref = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"])
    torch.cuda.synchronize()
    return d, o, final, o_ref, s_ref


def test_noalloc_overlapped_launch_on_two_calls(gdn, cuda):
    """The overlapped launch (forced) in the scratch: its control block (tickets, per-CU claims, ready flags)
    lies in the scratch after the workspace and must be zeroed by each call; a second, smaller call reuses it."""
    with gdn.ops.launch_form(1):
        for B, T, H, seed in [(1, 4096, 8, 7101), (1, 2048, 8, 7102)]:
            announce(f"chunk no-alloc overlapped B={B} T={T} H={H}")
            d, o, final, o_ref, s_ref = _pair(gdn, cuda, B, T, H, seed)
            assert torch.equal(o, o_ref) and torch.equal(final, s_ref)
            o_cpu, s_cpu = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"])
            assert max_abs(o.cpu(), o_cpu) < 2e-2 and rel_err(final.cpu(), s_cpu) < 1e-3
    assert gdn.ops.chunk_status() == 0


def test_noalloc_segmented_pass_on_two_calls(gdn, cuda):
    """Few long chains (one 4096- then 3072-token prompt, 4 heads) take the segmented state pass, whose local
    and transition states, Q'P^T rows and segment starts sit in the scratch after the phase-1 workspace."""
    lib = gdn._native.lib()
    for B, T, H, seed in [(1, 4096, 4, 7201), (1, 3072, 4, 7202)]:
        assert lib.zgdn_chunk_segment_workspace_size(B, T, H) > 0  # the library plans segments here
        announce(f"chunk no-alloc segmented B={B} T={T} H={H}")
        d, o, final, o_ref, s_ref = _pair(gdn, cuda, B, T, H, seed)
        assert torch.equal(o, o_ref) and torch.equal(final, s_ref)
        o_cpu, s_cpu = O.gated_delta_recurrence(d["q"], d["k"], d["v"], d["g"], d["beta"])
        assert max_abs(o.cpu(), o_cpu) < 2e-2 and rel_err(final.cpu(), s_cpu) < 1e-3


@pytest.mark.parametrize("form", [0, 1])
def test_noalloc_in_a_graph(gdn, cuda, form):
    """A no-alloc call captured into a HIP graph (two launches, or the overlapped launch with its control-block
    fill kernel) and replayed three times, with new inputs copied in and eager work in between: every replay
    equals zgdn_chunk_fwd on the same inputs bit for bit."""
    announce(f"chunk no-alloc graph form={form}")
    B, T, H = 1, 1024, 8
    _, x = _case(cuda, B, T, H, H, seed=7300)
    o = torch.empty(B, T, H, 128, dtype=torch.bfloat16, device=cuda)
    final = torch.empty(B, H, 128, 128, device=cuda)
    with gdn.ops.launch_form(form):
        _noalloc(gdn, x, o, final, x["s0"])  # first call on the device outside the capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            _noalloc(gdn, x, o, final, x["s0"])
        for r in range(3):
            _, new = _case(cuda, B, T, H, H, seed=7301 + r)
            for name in ("q", "k", "v", "g", "beta", "s0"):
                x[name].copy_(new[name])
            graph.replay()
            o_ref, s_ref = gdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"])
            torch.cuda.synchronize()
            assert torch.equal(o, o_ref) and torch.equal(final, s_ref), r
    assert gdn.ops.chunk_status() == 0
