"""On-disk formats (zonos3-mini_amd/formats.py): the GGUF name contract of the GDN tensors
(tools/convert_gguf.py:123-127, 132), GGUF parsing (a file written here with the published layout,
and the reference's own dummy model file when it is present), and the state.npz GDN entries
(tools/dump_golden.py:223-272)."""

from __future__ import annotations

import importlib
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from gdn_testing import q8_0, write_gguf

DUMMY_GGUF = Path("/root/reference/servers/ggml/tests/fixtures/dummy-zonos3.gguf")


@pytest.fixture(scope="module")
def formats(gdn):
    return importlib.import_module("zonos3-mini_amd.formats")


def test_gdn_name_contract(formats):
    names = {p.format(L=3): g.format(L=3) for p, g in formats.GDN_GGUF_NAMES}
    assert names == {
        "layers.3.attention.in_proj.weight": "blk.3.gdn_in.weight",
        "layers.3.attention.out_weight": "blk.3.gdn_norm.weight",
        "layers.3.attention.A_log": "blk.3.gdn_A_log",
        "layers.3.attention.dt_bias": "blk.3.gdn_dt_bias",
        "layers.3.attention.conv.weight": "blk.3.gdn_conv.weight",
        "layers.3.attention.wo.weight": "blk.3.attn_output.weight",
    }
    assert formats.GDN_GGUF_METADATA == ("gdn.head_count", "gdn.head_dim", "gdn.conv_kernel")


def test_gguf_round_trip_of_every_supported_type(formats, tmp_path):
    rng = np.random.default_rng(7)
    a32 = rng.standard_normal((3, 5)).astype(np.float32)
    a16 = rng.standard_normal((4, 8)).astype(np.float16)
    abf = rng.standard_normal((2, 16)).astype(np.float32)
    abf_bits = (abf.view(np.uint32) >> 16).astype(np.uint16)  # truncated to bf16
    aq = rng.standard_normal((2, 64)).astype(np.float32)
    tensors = {
        "t.f32": (0, a32.tobytes(), a32.shape),
        "t.f16": (1, a16.tobytes(), a16.shape),
        "t.bf16": (30, abf_bits.tobytes(), abf.shape),
        "t.q8": (8, q8_0(aq), aq.shape),
        "t.vec": (0, np.arange(7, dtype=np.float32).tobytes(), (7,)),
    }
    meta = {"general.architecture": "zonos3", "gdn.head_count": 4, "x.scale": 0.5, "x.list": [1, -2, 3],
            "x.flag": True}
    path = tmp_path / "t.gguf"
    write_gguf(path, meta, tensors)
    got_meta, got = formats.read_gguf(path)
    assert got_meta["general.architecture"] == "zonos3" and got_meta["gdn.head_count"] == 4
    assert got_meta["x.scale"] == 0.5 and got_meta["x.list"] == [1, -2, 3] and got_meta["x.flag"] is True
    assert np.array_equal(got["t.f32"].numpy(), a32)
    assert np.array_equal(got["t.f16"].numpy(), a16.astype(np.float32))
    assert np.array_equal(got["t.bf16"].numpy(), (abf_bits.astype(np.uint32) << 16).view(np.float32))
    assert np.array_equal(got["t.vec"].numpy(), np.arange(7, dtype=np.float32))
    # Q8_0 against its definition: scale times int8, per 32-value block
    q = got["t.q8"].numpy().reshape(-1, 32)
    scales = np.abs(aq.reshape(-1, 32)).max(1) / 127.0
    assert np.allclose(q, aq.reshape(-1, 32), atol=float(scales.max()) * 0.51)
    assert got["t.q8"].shape == (2, 64) and got["t.q8"].type_name == "Q8_0"


def test_gguf_rejects_what_it_cannot_read(formats, tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + b"\0" * 32)
    with pytest.raises(ValueError, match="not a GGUF"):
        formats.read_gguf(bad)
    write_gguf(tmp_path / "q4.gguf", {}, {"t": (2, b"\0" * 18, (32,))})  # Q4_0: listed, not readable here
    _, t = formats.read_gguf(tmp_path / "q4.gguf")
    with pytest.raises(ValueError, match="not supported"):
        t["t"].numpy()


def test_gdn_layer_weights_from_a_written_file(formats, tmp_path):
    rng = np.random.default_rng(11)
    w = {"gdn_in": rng.standard_normal((2056, 64)).astype(np.float16),
         "gdn_norm": rng.standard_normal(128).astype(np.float32),
         "gdn_A_log": rng.standard_normal(4).astype(np.float32),
         "gdn_dt_bias": rng.standard_normal(4).astype(np.float32),
         "gdn_conv": rng.standard_normal((1536, 4)).astype(np.float32),
         "attn_output": rng.standard_normal((64, 512)).astype(np.float16)}
    tensors = {f"blk.2.{k}" + ("" if k in ("gdn_A_log", "gdn_dt_bias") else ".weight"):
               (1 if v.dtype == np.float16 else 0, v.tobytes(), v.shape) for k, v in w.items()}
    write_gguf(tmp_path / "m.gguf", {"gdn.head_count": 4, "gdn.head_dim": 128, "gdn.conv_kernel": 4}, tensors)
    _, t = formats.read_gguf(tmp_path / "m.gguf")
    got = formats.gdn_layer_weights(t, 2)
    assert got["conv"].shape == (1536, 1, 4) and torch.equal(got["conv"][:, 0], torch.from_numpy(w["gdn_conv"]))
    assert torch.equal(got["in_proj"], torch.from_numpy(w["gdn_in"].astype(np.float32)))
    assert torch.equal(got["wo"], torch.from_numpy(w["attn_output"].astype(np.float32)))
    assert torch.equal(got["A_log"], torch.from_numpy(w["gdn_A_log"]))
    with pytest.raises(KeyError, match="blk.1.gdn_in.weight"):
        formats.gdn_layer_weights(t, 1)


@pytest.mark.skipif(not DUMMY_GGUF.exists(), reason="the reference's dummy model file is not here")
def test_reference_dummy_model_file(formats):
    """The reference's own test model (servers/ggml/tests/fixtures/dummy-zonos3.gguf): its GDN layers parse
    into consistent layer weights (heads from A_log, q|k|v|z|a|b rows of in_proj, conv channels 3*inner)."""
    meta, t = formats.read_gguf(DUMMY_GGUF)
    assert meta["general.architecture"] == "zonos3"
    gdn_layers = sorted({int(n.split(".")[1]) for n in t if ".gdn_in." in n})
    assert gdn_layers
    for layer in gdn_layers:
        w = formats.gdn_layer_weights(t, layer)
        heads, hd = w["A_log"].numel(), w["out_weight"].numel()
        dim = w["in_proj"].shape[1]
        assert w["in_proj"].shape == (4 * heads * hd + 2 * heads, dim)
        assert w["conv"].shape == (3 * heads * hd, 1, 4) and w["wo"].shape == (dim, heads * hd)
        assert all(torch.isfinite(v).all() for v in w.values())


# ------------------------------------------------------------------------------------------------ state.npz


def test_state_npz_round_trip_and_entry_names(formats, tmp_path):
    gen = torch.Generator().manual_seed(3)
    cache = SimpleNamespace(gdn_state={0: torch.randn(4, 128, 128, generator=gen),
                                       2: torch.randn(4, 128, 128, generator=gen)},
                            conv_state={0: torch.randn(1536, 3, generator=gen).bfloat16(),
                                        2: torch.randn(1536, 3, generator=gen).bfloat16()})
    kv = {"kv_k_1": np.zeros((9, 2, 8), np.float32), "kv_v_1": np.ones((9, 2, 8), np.float32)}
    path = tmp_path / "state.npz"
    formats.save_gdn_state(path, cache, [0, 2], position=9, extra=kv)
    with np.load(path, allow_pickle=False) as f:
        assert set(f.files) == {"position", "gdn_state_0", "gdn_state_2", "gdn_conv_state_0", "gdn_conv_state_2",
                                "kv_k_1", "kv_v_1"}
        assert f["position"].dtype == np.int64 and f["gdn_conv_state_0"].dtype == np.float32
    back = SimpleNamespace(gdn_state={}, conv_state={})
    assert formats.load_gdn_state(path, back, [0, 2], torch.bfloat16, "cpu") == 9
    for layer in (0, 2):
        assert torch.equal(back.gdn_state[layer], cache.gdn_state[layer])
        assert back.conv_state[layer].dtype == torch.bfloat16
        assert torch.equal(back.conv_state[layer], cache.conv_state[layer])


def test_state_npz_validation(formats, tmp_path):
    good = {"gdn_state_0": np.zeros((4, 128, 128), np.float32), "gdn_conv_state_0": np.zeros((1536, 3), np.float32)}
    cases = [
        ({**good, "position": np.asarray(-1)}, "invalid position"),
        ({"gdn_state_0": good["gdn_state_0"], "position": np.asarray(3)}, "missing gdn_conv_state_0"),
        ({**good, "gdn_state_0": np.zeros((4, 128, 64), np.float32), "position": np.asarray(3)}, "invalid gdn_state_0"),
        ({**good, "gdn_conv_state_0": np.full((1536, 3), np.nan, np.float32), "position": np.asarray(3)},
         "invalid gdn_conv_state_0"),
    ]
    for i, (arrays, message) in enumerate(cases):
        path = tmp_path / f"s{i}.npz"
        np.savez(path, **arrays)
        with pytest.raises(ValueError, match=message):
            formats.load_gdn_state(path, SimpleNamespace(gdn_state={}, conv_state={}), [0], torch.float32, "cpu")
