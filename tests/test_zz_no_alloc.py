"""zgdn_chunk_fwd_noalloc, the chunked forward for callers that cannot allocate (its workspace is the library's
per-device static scratch), called through the C ABI with caller-allocated outputs: on two calls in a row, the
second smaller, its outputs and final states equal zgdn_chunk_fwd's on the same inputs bit for bit (the same
kernels; the scratch keeps the first call's contents, so anything the second call read without writing would
show) and sit within tolerance of the oracle (bf16: outputs 2e-2 max-abs, states 1e-3 relative). A call whose
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
