"""Host checks of packed-sequence tables (no device): malformed cu_seqlens / chunk_indices raise RuntimeError
before any copy or launch, as the serving layer rejects invalid packed lengths before its kernels
(servers/sgl/src/zonos3_sgl/models/gdn.py:247-255); well-formed tables match the reference's chunk_tables
(gdn.py:49-59)."""

from __future__ import annotations

from importlib import import_module

import pytest
import torch

from oracle import gdn_oracle as O

ops = import_module("zonos3-mini_amd.ops")


@pytest.mark.parametrize("cu,total,msg", [([0, 5, 3, 9], 9, "decreases at entry 1"),
                                          ([1, 5, 9], 9, "starts at 1"),
                                          ([0, 5, 9], 10, "ends at 9"),
                                          ([0, 5, 12], 9, "ends at 12"),
                                          ([0], 0, "need at least 2"),
                                          ([0, -3, 0], 0, "decreases at entry 0")])
def test_malformed_cu_seqlens_raise(cu, total, msg):
    with pytest.raises(RuntimeError, match=msg):
        ops.check_cu_seqlens(cu, total)
    with pytest.raises(RuntimeError, match=msg):
        ops.host_tables(torch.tensor(cu, dtype=torch.int32), None, total)


def test_malformed_chunk_indices_raise():
    cu = [0, 64, 65, 200]
    good = O.chunk_tables([64, 1, 135])[1]
    ops.check_chunk_indices(good, cu)
    for bad in (good[:-1], good + [[2, 3]], [[1, 0]] + good[1:], [[r[0], r[1] + 1] for r in good],
                [[0, 0], [0, 0]] + good[2:]):
        with pytest.raises(RuntimeError, match="chunk_indices"):
            ops.check_chunk_indices(bad, cu)
        with pytest.raises(RuntimeError, match="chunk_indices"):
            ops.host_tables(cu, torch.tensor(bad, dtype=torch.int32), 200)


@pytest.mark.parametrize("lengths", [[64, 1, 130, 0, 70, 200, 63], [1], [0, 0, 5], [128] * 5])
def test_host_tables_match_the_reference_tables(lengths):
    """Tables built and checked on the host equal the oracle's statement of gdn.py:49-59 (itself pinned to
    the literal tables of servers/sgl/tests/test_gdn_graph_support.py:17-30)."""
    cu, chunks = ops.host_tables(O.chunk_tables(lengths)[0], None, sum(lengths))
    ref_cu, ref_chunks = O.chunk_tables(lengths)
    assert cu.dtype == chunks.dtype == torch.int32
    assert cu.tolist() == ref_cu and chunks.tolist() == ref_chunks
    assert chunks.shape == (len(ref_chunks), 2)
