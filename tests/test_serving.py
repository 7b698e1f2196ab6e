"""Host logic of the serving-layer mixer (zonos3-mini_amd/serving.py, the counterpart of
servers/sgl/src/zonos3_sgl/models/gdn.py): static index tables and padded prefill layouts against the
reference's expected values (servers/sgl/tests/test_gdn_graph_support.py:17-42), and the eager path's
validation, which rejects a batch before touching any cache."""

from __future__ import annotations

import importlib
from types import SimpleNamespace

import pytest
import torch

from oracle import gdn_oracle as O


@pytest.fixture(scope="module")
def serving(gdn):
    return importlib.import_module("zonos3-mini_amd.serving")


def test_static_tables_describe_bs_windows_of_64_rows(serving):
    tables = serving.OriginalGDN.static_tables(torch.device("cpu"), [1, 4])
    cu, chunks, rows = tables[4]
    assert cu.tolist() == [0, 64, 128, 192, 256] and cu.dtype == torch.int32
    assert chunks.tolist() == [[0, 0], [1, 0], [2, 0], [3, 0]] and chunks.dtype == torch.int32
    assert rows.tolist() == [0, 64, 128, 192] and rows.dtype == torch.long
    assert tables[1][0].tolist() == [0, 64]


@pytest.mark.parametrize("lengths", [[1], [64], [65], [5, 63, 64, 130], [200, 1, 128]])
def test_chunk_tables(serving, lengths):
    cu, chunks = serving.chunk_tables(lengths, torch.device("cpu"))
    assert cu.tolist() == torch.tensor([0] + lengths).cumsum(0).tolist()
    want_cu, want_chunks = O.chunk_tables(lengths)
    assert cu.tolist() == want_cu and chunks.tolist() == [list(c) for c in want_chunks]
    assert chunks.dtype == torch.int32 and chunks.shape == (sum(-(-n // 64) for n in lengths), 2)


def test_prefill_layout_covers_every_padded_row_once(serving):
    whole = [0, 3, 1]
    layout = serving.PrefillLayout.build(whole, torch.device("cpu"))
    rows = sum(64 * (w + 1) for w in whole)
    covered = torch.cat([layout.whole_rows, layout.window_rows]).sort().values
    assert torch.equal(covered, torch.arange(rows))
    assert layout.whole_reqs.tolist() == [1, 2] and layout.whole_cu.tolist() == [0, 3 * 64, 4 * 64]
    assert layout.window_base.tolist() == [0, 3 * 64, 64]
    assert layout.window_rows.view(3, 64)[:, 0].tolist() == [0, 4 * 64, 6 * 64]
    assert len(layout.tensors()) == 4
    assert serving.PrefillLayout.build([0, 0], torch.device("cpu")).whole_rows is None


def test_pin_fla_cache_has_nothing_to_pin(serving):
    assert serving.OriginalGDN.pin_fla_cache([torch.zeros(3)], {}) == 0


def _layer(serving, batch):
    layer = serving.OriginalGDN(SimpleNamespace(hidden_size=32), layer_id=3, batch_source=lambda: batch)
    layer.allocate_cache(4, torch.device("cpu"), torch.float32)
    return layer


def _req(slot, cached, n, uid=None):
    return SimpleNamespace(table_idx=slot, uid=slot if uid is None else uid, is_cfg_uncond=False, cached_len=cached,
                           device_len=cached + n, extend_len=n)


def test_eager_path_rejects_bad_batches_before_any_kernel(serving):
    batch = SimpleNamespace(is_decode=False, padded_size=2, gdn_prefill=None)
    layer = _layer(serving, batch)
    with pytest.raises(RuntimeError, match="already allocated"):
        layer.allocate_cache(4, torch.device("cpu"), torch.float32)
    cases = [
        ([_req(0, 0, 3), _req(0, 0, 2)], 5, "slots or packed lengths"),  # the same slot twice
        ([_req(0, 0, 3), _req(4, 0, 2)], 5, "slots or packed lengths"),  # slot outside the cache
        ([_req(0, 0, 3), _req(1, 0, 0)], 3, "slots or packed lengths"),  # an empty request
        ([_req(0, 0, 3), _req(1, 0, 2)], 6, "slots or packed lengths"),  # rows != sum of lengths
        ([_req(0, 7, 1)], 1, "missing/stale state at slot 0"),  # no state for a cached prefix
    ]
    for reqs, rows, message in cases:
        batch.reqs = batch.padded_reqs = reqs
        with pytest.raises(RuntimeError, match=message):
            layer.forward(torch.zeros(rows, 32))
    batch.reqs, batch.padded_reqs = [_req(0, 0, 1)], [_req(0, 0, 1), _req(1, 0, 1)]
    with pytest.raises(RuntimeError, match="dummy graph-padding"):
        layer.forward(torch.zeros(1, 32))
    batch.is_decode = True
    batch.reqs = batch.padded_reqs = [_req(0, 0, 2)]
    with pytest.raises(RuntimeError, match="one new token"):
        layer.forward(torch.zeros(2, 32))
    layer.set_static_mode(True)
    with pytest.raises(RuntimeError, match="not prepared for batch size 2"):
        layer.forward(torch.zeros(2, 32))
    assert layer._owners == [None] * 4 and not layer._win_len.any()  # nothing was changed
    with pytest.raises(RuntimeError, match="batch source"):
        serving.OriginalGDN(SimpleNamespace(hidden_size=32), 0).forward(torch.zeros(1, 32))
