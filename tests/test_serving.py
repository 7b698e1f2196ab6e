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
        ([_req(0, 0, 3), _req(0, 0, 2)], 5, "slot 0 named by two requests"),
        ([_req(0, 0, 3), _req(4, 0, 2)], 5, "slot 4 outside the 4 slots"),
        ([_req(0, 0, 3), _req(1, 0, 0)], 3, "slot 1 brings 0 rows"),
        ([_req(0, 0, 3), _req(1, 0, 2)], 6, "6 rows given for requests of 5 rows"),
        ([_req(0, 7, 1)], 1, r"slot 0 has no state for \(0, False\) at row 7"),  # a cached prefix, no state
    ]
    for reqs, rows, message in cases:
        batch.reqs = batch.padded_reqs = reqs
        with pytest.raises(RuntimeError, match=message):
            layer.forward(torch.zeros(rows, 32))
    batch.reqs, batch.padded_reqs = [_req(0, 0, 1)], [_req(0, 0, 1), _req(1, 0, 1)]
    with pytest.raises(RuntimeError, match="1 dummy graph-padding requests"):
        layer.forward(torch.zeros(1, 32))
    batch.is_decode = True
    batch.reqs = batch.padded_reqs = [_req(0, 0, 2)]
    with pytest.raises(RuntimeError, match="one new row per request, slot 0 has 2"):
        layer.forward(torch.zeros(2, 32))
    layer.set_static_mode(True)
    with pytest.raises(RuntimeError, match="not prepared for batch size 2"):
        layer.forward(torch.zeros(2, 32))
    assert layer._owners == [None] * 4 and not layer._win_len.any()  # nothing was changed
    with pytest.raises(RuntimeError, match="batch source"):
        serving.OriginalGDN(SimpleNamespace(hidden_size=32), 0).forward(torch.zeros(1, 32))


def _transparent_packed(calls):
    """A stand-in for ``_run_packed`` on the CPU that makes the bookkeeping visible: output row = input row +
    its position in its packed sequence; conv / recurrent final = initial + the sum of the sequence's rows
    (so a slot's states telescope to the sum of the rows that went through them). Checks the chunk tables
    against the sequence lengths."""

    def run(x, cu, chunks, conv, recurrent, mask=None, valid=None, return_mixed=False):
        lengths = (cu[1:] - cu[:-1]).tolist()
        assert cu[0] == 0 and cu[-1] == x.shape[0] and len(lengths) == conv.shape[0] == recurrent.shape[0]
        want = [[i, j] for i, n in enumerate(lengths) for j in range(-(-n // 64))]
        assert chunks.tolist() == want
        pos = torch.cat([torch.arange(n, dtype=x.dtype) for n in lengths])
        sums = torch.stack([p.sum() for p in x.split(lengths)])
        calls.append(lengths)
        out = x + pos.view(-1, 1)
        result = (out, conv + sums.view(-1, 1, 1), recurrent + sums.view(-1, 1, 1, 1))
        return result + (None,) if return_mixed else result

    return run


def test_eager_bookkeeping_follows_the_chunk_contract(serving):
    """Eager prefills and extends of several requests through the host plan, with the packed pass replaced by
    ``_transparent_packed``: after every call each new row's output is that row plus its position in the
    pass that ran it (the committed pass takes the joined run of replayed tail + new rows up to its last 64-row
    boundary as one sequence, the open pass the rest), the committed
    states hold the sum of the request's rows up to its last 64-row boundary, the live states the sum of all
    its rows, and the window its rows past that boundary (the brute-force statement of gdn.py:271-327)."""
    hid = 8
    batch = SimpleNamespace(is_decode=False, padded_size=0, gdn_prefill=None)
    layer = serving.OriginalGDN(SimpleNamespace(hidden_size=hid), layer_id=1, batch_source=lambda: batch)
    layer.allocate_cache(5, torch.device("cpu"), torch.float64)
    calls = []
    layer._run_packed = _transparent_packed(calls)
    gen = torch.Generator().manual_seed(7)
    history = {}  # slot -> all rows of its request so far
    reqs = {}
    schedule = [  # (slot, new rows) per call
        [(0, 70), (1, 5), (2, 63), (4, 64)],
        [(2, 1), (1, 59), (0, 130)],  # slot 2 completes its chunk exactly, slot 1 reaches 64 with its tail
        [(3, 200), (1, 1), (2, 64), (0, 3)],
        [(0, 58), (3, 56), (4, 1)],
    ]
    for step in schedule:
        batch_reqs = []
        for s, n in step:
            r = reqs.setdefault(s, SimpleNamespace(table_idx=s, uid=10 + s, is_cfg_uncond=False, cached_len=0,
                                                   device_len=0, extend_len=0))
            r.cached_len, r.extend_len, r.device_len = r.device_len, n, r.device_len + n
            batch_reqs.append(r)
        batch.reqs = batch.padded_reqs = batch_reqs
        x = torch.randn(sum(n for _, n in step), hid, generator=gen, dtype=torch.float64)
        calls.clear()
        y = layer.forward(x)
        # the passes ran each request's unfinished tail and new rows once, nothing of its history before
        assert sum(map(sum, calls)) == sum(len(history.get(s, [])) % 64 + n for s, n in step)
        at = 0
        for s, n in step:
            old = history.get(s, x[:0])
            cut = len(old) // 64 * 64  # the window before the call starts here
            rows = torch.cat((old, x[at:at + n]))
            for j in range(n):  # new row j sits at position len(old) + j of the request
                p = len(old) + j
                whole = cut + (len(rows) - cut) // 64 * 64  # the committed pass runs [cut, whole) as one run
                base = cut if p < whole else whole
                assert torch.equal(y[at + j], x[at + j] + (p - base)), (step, s, j)
            history[s] = rows
            at += n
        for s, rows in history.items():
            done = len(rows) // 64 * 64
            assert torch.allclose(layer._conv_state[s], rows[:done].sum().expand(1536, 4)), s
            assert torch.allclose(layer._recurrent_state[s], rows[:done].sum().expand(4, 128, 128).float()), s
            assert torch.allclose(layer._live_conv[s], rows.sum().expand(1536, 4)), s
            assert torch.allclose(layer._live_state[s], rows.sum().expand(4, 128, 128).float()), s
            assert layer._win_len[s].item() == len(rows) - done and layer._lengths[s] == len(rows)
            assert torch.equal(layer._window[s, : len(rows) - done], rows[done:]), s


def test_plan_extend_splits_each_joined_run_at_its_last_chunk(serving):
    """The host plan for three requests: a fresh one of 70 rows, one with a 10-row tail and 54 new rows (one
    complete chunk, nothing open), one with a 3-row tail and 2 new rows (open only)."""
    R = serving.Request
    reqs = [R(slot=2, owner=(1, False), cached=0, new=70), R(slot=0, owner=(2, False), cached=74, new=54),
            R(slot=3, owner=(3, False), cached=131, new=2)]
    replayed, committed, open_ = serving.plan_extend(reqs)
    assert replayed == list(range(0, 10)) + [3 * 64 + j for j in range(3)]
    assert committed.members == [0, 1] and committed.lengths == [64, 64]
    assert committed.src == [13 + j for j in range(64)] + list(range(10)) + [13 + 70 + j for j in range(54)]
    assert committed.dest == list(range(64)) + list(range(70, 124))
    assert committed.out_rows == list(range(64)) + list(range(74, 128))
    assert open_.members == [0, 2] and open_.lengths == [6, 5]
    assert open_.src == [13 + 64 + j for j in range(6)] + [10, 11, 12, 13 + 124, 13 + 125]
    assert open_.dest == list(range(64, 70)) + [124, 125] and open_.out_rows == [0, 1, 2, 3, 4, 5, 9, 10]
    assert open_.window == [2 * 64 + j for j in range(6)] + [3 * 64 + j for j in range(5)]
    assert open_.member_of_row == [0] * 6 + [2] * 5


def test_static_prefill_bookkeeping(serving):
    """A padded static prefill (PrefillLayout of complete-chunk counts 0, 2, 1) with the packed pass replaced by
    ``_transparent_packed`` (extended with a projection stand-in, mixed = x tiled to the in_proj width):
    outputs of complete chunks and windows land on their batch rows, committed states hold the complete
    chunks' rows, live states all real rows (the padding rows' values are zeroed first, and their gate inputs
    set to the no-op values), windows keep the rows with their real count in win_len, and the live conv
    history is the last CONV_WIDTH projection rows before the padding, the committed history in front."""
    hid = 8
    batch = SimpleNamespace(is_decode=False, padded_size=0)
    layer = serving.OriginalGDN(SimpleNamespace(hidden_size=hid), layer_id=2, batch_source=lambda: batch)
    layer.allocate_cache(4, torch.device("cpu"), torch.float64)
    calls = []
    base = _transparent_packed(calls)
    seen = {}

    def run(x, cu, chunks, conv, recurrent, mask=None, valid=None, return_mixed=False):
        if valid is not None:
            seen["valid"] = valid.clone()
            assert torch.equal(x[~valid], torch.zeros_like(x[~valid]))  # padding rows arrive zeroed
        out, conv_final, final = base(x, cu, chunks, conv, recurrent)[:3]
        if valid is not None:  # decay 1, beta 0: the padding rows leave the states alone
            sums = torch.stack([p[v].sum() for p, v in zip(x.split((cu[1:] - cu[:-1]).tolist()),
                                                           valid.split((cu[1:] - cu[:-1]).tolist()))])
            final = recurrent + sums.view(-1, 1, 1, 1)
        mixed = x.repeat(1, -(-2056 // hid))[:, :2056]
        return (out, conv_final, final, mixed) if return_mixed else (out, conv_final, final)

    layer._run_packed = run
    whole, lengths, slots = [0, 2, 1], [5, 130, 64], [2, 0, 3]
    layout = serving.PrefillLayout.build(whole, torch.device("cpu"))
    rows = sum(64 * (w + 1) for w in whole)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(rows, hid, generator=gen, dtype=torch.float64)
    batch.gdn_prefill = serving.PrefillInputs(layout, torch.tensor(slots), torch.tensor(lengths))
    y = layer.forward(x)
    start = 0
    for w, n, s in zip(whole, lengths, slots):
        seg = x[start:start + 64 * (w + 1)]
        real = seg[:n]
        done = 64 * w
        if done:  # the complete chunks: one packed sequence from zero states, outputs row + position
            assert torch.equal(y[start:start + done], seg[:done] + torch.arange(done, dtype=x.dtype).view(-1, 1))
        fill = n - done
        win_out = y[start + done:start + done + fill]
        assert torch.equal(win_out, seg[done:n] + torch.arange(fill, dtype=x.dtype).view(-1, 1))
        assert torch.allclose(layer._conv_state[s], real[:done].sum().expand(1536, 4))
        assert torch.allclose(layer._recurrent_state[s], real[:done].sum().expand(4, 128, 128).float())
        assert torch.allclose(layer._live_state[s], real.sum().expand(4, 128, 128).float())
        assert layer._win_len[s].item() == fill
        assert torch.equal(layer._window[s, :fill], seg[done:n])
        # live conv: the last 4 conv inputs up to the window's last real row, the committed history first
        hist = torch.cat((layer._conv_state[s], seg[done:n].repeat(1, -(-2056 // hid))[:, :1536].T), dim=1)
        assert torch.equal(layer._live_conv[s], hist[:, fill:fill + 4])
        start += 64 * (w + 1)
    assert seen["valid"].view(3, 64).sum(1).tolist() == [n - 64 * w for w, n in zip(whole, lengths)]
