"""Layer-level drop-ins against the CPU oracle: ``layer.gdn`` in place of ``Zonos3LM._gdn``
(model/src/zonos3/reference/lm.py:556-602) and the five-operator seam installed on a restatement of
``OriginalGDN._run_packed`` (servers/sgl/src/zonos3_sgl/models/gdn.py:395-450)."""

from __future__ import annotations

import importlib
from dataclasses import dataclass, field
from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gdn_testing import announce, max_abs, rel_err
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

HEADS, HD, DIM = 4, 128, 256


def _weights(seed, dtype):
    gen = torch.Generator().manual_seed(seed)
    inner = HEADS * HD
    w = {
        "in_proj": 0.05 * torch.randn(4 * inner + 2 * HEADS, DIM, generator=gen),
        "conv": 0.2 * torch.randn(3 * inner, 1, 4, generator=gen),
        "out_weight": 1 + 0.1 * torch.randn(HD, generator=gen),
        "A_log": 0.2 * torch.randn(HEADS, generator=gen),
        "dt_bias": 0.2 * torch.randn(HEADS, generator=gen),
        "wo": 0.05 * torch.randn(DIM, inner, generator=gen),
    }
    return {k: (v if k in ("A_log", "dt_bias") else v.to(dtype)) for k, v in w.items()}


@dataclass
class _Cache:  # the two fields of LMCache (lm.py:345-361) the layer touches
    gdn_state: dict = field(default_factory=dict)
    conv_state: dict = field(default_factory=dict)


class _Model:
    """The attributes Zonos3LM._gdn reads: layers[i].attention.*, _lin, _capture, _save."""

    def __init__(self, w, device):
        t = {k: v.to(device) for k, v in w.items()}
        att = SimpleNamespace(in_proj=SimpleNamespace(weight=t["in_proj"]), conv=SimpleNamespace(weight=t["conv"]),
                              out_weight=t["out_weight"], A_log=t["A_log"], dt_bias=t["dt_bias"],
                              wo=SimpleNamespace(weight=t["wo"]))
        self.layers = [SimpleNamespace(attention=att)]
        self._capture = None

    def _lin(self, name, x, weight, bias=None):
        return F.linear(x, weight, bias)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_layer_prefill_then_decode_steps(gdn, cuda, dtype):
    """Prefill 100 rows, then 3 single-row decode steps, carrying the cache (the split invariance of
    model/tests/test_reference_lm.py:126-136, each part checked against the oracle)."""
    announce(f"layer drop-in prefill 100 + 3 decode, {dtype}")
    layer = importlib.import_module("zonos3-mini_amd.layer")
    w = _weights(4001, dtype)
    model = _Model(w, cuda)
    layer.patch(model)
    x = torch.randn(103, DIM, generator=torch.Generator().manual_seed(4002)).to(dtype)
    cache = _Cache()
    conv_ref, state_ref = None, None
    for lo, hi in ((0, 100), (100, 101), (101, 102), (102, 103)):
        y = model._gdn(x[lo:hi].to(cuda), 0, cache)
        torch.cuda.synchronize()
        y_ref, conv_ref, state_ref, _ = O.gdn_layer(x[lo:hi], w, conv_ref, state_ref, heads=HEADS, head_dim=HD)
        tol_o, tol_s = (2e-2, 1e-3) if dtype == torch.bfloat16 else (1e-4, 1e-4)
        assert rel_err(y.cpu(), y_ref) < tol_o, (lo, rel_err(y.cpu(), y_ref))
        assert rel_err(cache.gdn_state[0].cpu(), state_ref) < tol_s, (lo, rel_err(cache.gdn_state[0].cpu(), state_ref))
        # the history is the raw in_proj output: GPU and CPU GEMMs round it differently
        assert rel_err(cache.conv_state[0].cpu(), conv_ref) < (1e-5 if dtype == torch.float32 else 1e-2), lo
        assert cache.conv_state[0].dtype == dtype and cache.gdn_state[0].dtype == torch.float32


def _run_packed(layer, x, cu, chunks, conv, recurrent):
    """The call sequence of OriginalGDN._run_packed (gdn.py:399-450) through the five bound operators."""
    mixed = F.linear(x, layer.in_proj)
    qkv, z, a, b = mixed.unsqueeze(0).split([1536, 512, 4, 4], dim=-1)
    qkv, conv_final = layer._conv_fwd(x=qkv.contiguous(), weight=layer.conv.squeeze(1), bias=None, residual=None,
                                      initial_state=conv, output_final_state=True, activation="silu",
                                      cu_seqlens=cu, chunk_indices=chunks, BT=64)
    q, k, v = [t.unflatten(-1, (4, 128)).contiguous() for t in qkv.split(512, dim=-1)]
    q, _ = layer._l2norm_fwd(q)
    k, _ = layer._l2norm_fwd(k)
    _, output, _, final, _, _ = layer._delta_rule_fwd(
        q=q, k=k, v=v, g=a.contiguous(), beta=layer._beta_fwd(b.contiguous(), 1.0), scale=128**-0.5,
        initial_state=recurrent, output_final_state=True, state_v_first=True, cu_seqlens=cu, chunk_indices=chunks,
        use_gate_in_kernel=True, A_log=layer.A_log, dt_bias=layer.dt_bias, chunk_size=64)
    output = layer._norm_fwd(x=output.to(q.dtype).reshape(-1, 128), g=z.reshape(-1, 128).contiguous(),
                             weight=layer.out_weight, bias=None, activation="swish", eps=1e-5, residual=None,
                             residual_dtype=None, is_rms_norm=True)[0]
    return F.linear(output.reshape(x.shape[0], 512), layer.wo), conv_final, final


def test_serving_seam_on_packed_requests(gdn, cuda):
    """Three packed requests (one crossing chunk boundaries) through the installed seam; expected values from
    the oracle's parts with the seam's own data flow (bf16 conv output, bf16 L2-normalised q, k)."""
    announce("serving seam _run_packed 3 requests")
    fla = importlib.import_module("zonos3-mini_amd.fla_ops")
    dtype = torch.bfloat16
    w = _weights(4101, dtype)
    gen = torch.Generator().manual_seed(4102)
    lengths = [70, 5, 130]
    cu, chunks = O.chunk_tables(lengths)
    N = len(lengths)
    x = torch.randn(sum(lengths), DIM, generator=gen).to(dtype)
    conv0 = (0.5 * torch.randn(N, 1536, 4, generator=gen)).to(dtype)
    rec0 = 0.02 * torch.randn(N, 4, 128, 128, generator=gen)
    layer = SimpleNamespace(in_proj=w["in_proj"].to(cuda), conv=w["conv"].to(cuda), out_weight=w["out_weight"].to(cuda),
                            A_log=w["A_log"].to(cuda), dt_bias=w["dt_bias"].to(cuda), wo=w["wo"].to(cuda))
    fla.install(layer)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda)
    ch_t = torch.tensor(chunks, dtype=torch.int32, device=cuda)
    y, conv_final, final = _run_packed(layer, x.to(cuda), cu_t, ch_t, conv0.to(cuda), rec0.to(cuda))
    torch.cuda.synchronize()
    mixed = F.linear(x, w["in_proj"])
    for i in range(N):
        lo, hi = cu[i], cu[i + 1]
        qkv, z, a, b = mixed[lo:hi].split([1536, 512, 4, 4], -1)
        conv, hist = O.causal_conv1d(qkv, w["conv"], conv0[i][:, 1:])
        q, k, v = (t.reshape(hi - lo, 4, 128) for t in conv.split(512, -1))
        q, k = O.l2norm(q).to(dtype), O.l2norm(k).to(dtype)
        decay, beta = O.gate(a, b, w["A_log"], w["dt_bias"])
        o, s = O.gated_delta_sequence(q, k, v, decay, beta, 128**-0.5, rec0[i])
        gated = O.gated_rmsnorm(o.to(dtype), z.reshape(hi - lo, 4, 128), w["out_weight"], 1e-5, dtype)
        y_ref = F.linear(gated.reshape(hi - lo, 512), w["wo"])
        assert rel_err(y[lo:hi].cpu(), y_ref) < 2e-2, (i, rel_err(y[lo:hi].cpu(), y_ref))
        assert rel_err(final[i].cpu(), s) < 1e-3, (i, rel_err(final[i].cpu(), s))
        assert torch.equal(conv_final[i].cpu()[:, 1:], hist), i
        assert torch.equal(conv_final[i].cpu(), torch.cat((conv0[i], qkv.T), -1)[:, -4:]), i


def test_seam_refuses_what_it_does_not_compute(gdn, cuda):
    fla = importlib.import_module("zonos3-mini_amd.fla_ops")
    t = torch.zeros(1, 64, 2, 128, dtype=torch.bfloat16, device=cuda)
    g = torch.zeros(1, 64, 2, device=cuda)
    with pytest.raises(RuntimeError, match="value-major"):
        fla.chunk_gated_delta_rule_fwd(t, t, t, g, g, state_v_first=False)
    with pytest.raises(RuntimeError, match="chunk_size"):
        fla.chunk_gated_delta_rule_fwd(t, t, t, g, g, chunk_size=32)
    with pytest.raises(RuntimeError, match="bias"):
        fla.layer_norm_gated_fwd(t[0, 0], t[0, 0], t[0, 0, 0], bias=t[0, 0, 0])
    with pytest.raises(RuntimeError, match="residual"):
        fla.causal_conv1d_fwd(t[0], t[0, 0, :, :4].T.contiguous(), residual=t[0])


def test_layer_with_weights_read_from_gguf(gdn, cuda, tmp_path):
    """A layer's weights stored under the GGUF GDN names (in_proj as Q8_0 blocks, wo as F16, the rest F32),
    read back by formats.read_gguf / gdn_layer_weights and run through the drop-in: against the oracle given
    the same (dequantised) weights, a 70-row prefill then a decode row."""
    from gdn_testing import q8_0, write_gguf

    announce("layer drop-in with GGUF-read weights, prefill 70 + 1 decode, bf16")
    formats = importlib.import_module("zonos3-mini_amd.formats")
    layer = importlib.import_module("zonos3-mini_amd.layer")
    w = _weights(4301, torch.float32)
    tensors = {
        "blk.0.gdn_in.weight": (8, q8_0(w["in_proj"].numpy()), tuple(w["in_proj"].shape)),
        "blk.0.gdn_norm.weight": (0, w["out_weight"].numpy().tobytes(), (128,)),
        "blk.0.gdn_A_log": (0, w["A_log"].numpy().tobytes(), (HEADS,)),
        "blk.0.gdn_dt_bias": (0, w["dt_bias"].numpy().tobytes(), (HEADS,)),
        "blk.0.gdn_conv.weight": (0, w["conv"][:, 0].contiguous().numpy().tobytes(), (3 * HEADS * HD, 4)),
        "blk.0.attn_output.weight": (1, w["wo"].numpy().astype(np.float16).tobytes(), tuple(w["wo"].shape)),
    }
    write_gguf(tmp_path / "gdn.gguf", {"gdn.head_count": HEADS, "gdn.head_dim": HD, "gdn.conv_kernel": 4}, tensors)
    _, t = formats.read_gguf(tmp_path / "gdn.gguf")
    read = {k: v.to(torch.bfloat16) if k not in ("A_log", "dt_bias") else v
            for k, v in formats.gdn_layer_weights(t, 0).items()}
    assert (read["in_proj"].float() - w["in_proj"]).abs().max() < 0.05 * w["in_proj"].abs().max()  # Q8_0 grid
    model = _Model(read, cuda)
    layer.patch(model)
    x = torch.randn(71, DIM, generator=torch.Generator().manual_seed(4302)).to(torch.bfloat16)
    cache = _Cache()
    conv_ref, state_ref = None, None
    for lo, hi in ((0, 70), (70, 71)):
        y = model._gdn(x[lo:hi].to(cuda), 0, cache)
        torch.cuda.synchronize()
        y_ref, conv_ref, state_ref, _ = O.gdn_layer(x[lo:hi], read, conv_ref, state_ref, heads=HEADS, head_dim=HD)
        assert rel_err(y.cpu(), y_ref) < 2e-2, (lo, rel_err(y.cpu(), y_ref))
        assert rel_err(cache.gdn_state[0].cpu(), state_ref) < 1e-3, lo


def _fork(cache: _Cache, deep: bool) -> _Cache:
    """LMCache.fork (lm.py:353-359) clones every tensor (deep); a shallow fork shares the tensors, so a drop-in
    that wrote into the tensors it was handed would show up in the parent."""
    if deep:
        return _Cache({k: v.clone() for k, v in cache.gdn_state.items()},
                      {k: v.clone() for k, v in cache.conv_state.items()})
    return _Cache(dict(cache.gdn_state), dict(cache.conv_state))


@pytest.mark.parametrize("deep", [True, False])
def test_fork_isolates_caches(gdn, cuda, deep):
    """model/tests/test_reference_lm.py:139-154 through the drop-in: after a 60-row prefill the cache is forked;
    the child takes two decode rows (the fused in-place kernel) and a 70-row prefill (the chunked path); the
    parent's state and conv history stay bit-identical to a snapshot, and the parent's own next decode row
    equals the child's first bit for bit. With a shallow fork the child shares the parent's tensors, so this
    also shows that no path writes into the tensors it reads."""
    announce(f"layer drop-in fork isolation deep={deep}")
    layer = importlib.import_module("zonos3-mini_amd.layer")
    w = _weights(4401, torch.bfloat16)
    model = _Model(w, cuda)
    layer.patch(model)
    x = torch.randn(133, DIM, generator=torch.Generator().manual_seed(4402)).to(torch.bfloat16).to(cuda)
    cache = _Cache()
    model._gdn(x[:60], 0, cache)
    snapshot = _fork(cache, deep=True)
    child = _fork(cache, deep)
    a = model._gdn(x[60:61], 0, child)
    model._gdn(x[61:62], 0, child)
    model._gdn(x[62:132], 0, child)
    torch.cuda.synchronize()
    assert torch.equal(cache.gdn_state[0], snapshot.gdn_state[0])
    assert torch.equal(cache.conv_state[0], snapshot.conv_state[0])
    assert not torch.equal(child.gdn_state[0], snapshot.gdn_state[0])
    b = model._gdn(x[60:61], 0, cache)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


class _CapturingModel(_Model):
    """_Model with lm.py's capture hook: _save stores float32 CPU copies under the given names (lm.py:498-500)."""

    def __init__(self, w, device):
        super().__init__(w, device)
        self._capture = {}

    def _save(self, name, tensor):
        self._capture[name] = tensor.detach().float().cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_capture_names_and_values(gdn, cuda, dtype):
    """The golden-dump hook (lm.py:588-601; tools/dump_golden.py) through the drop-in: a 40-row prefill then a
    decode row with capture on save exactly lm.py's ten gdn_*_<layer> names, and every value matches the
    oracle's captures of the same rows (fp32: 1e-4 relative; bf16: 2e-2 relative, 1e-3 on the fp32 state; the
    conv output and history compare to the GEMM's rounding, which the GPU and the CPU do differently)."""
    announce(f"layer drop-in captures {dtype}")
    layer = importlib.import_module("zonos3-mini_amd.layer")
    w = _weights(4501, dtype)
    model = _CapturingModel(w, cuda)
    layer.patch(model)
    x = torch.randn(41, DIM, generator=torch.Generator().manual_seed(4502)).to(dtype)
    cache = _Cache()
    conv_ref = state_ref = None
    names = ("gdn_conv", "gdn_q", "gdn_k", "gdn_v", "gdn_decay", "gdn_beta", "gdn_recurrent", "gdn_gated",
             "gdn_state", "gdn_conv_state")
    bf16 = dtype == torch.bfloat16
    for lo, hi in ((0, 40), (40, 41)):
        model._capture = {}
        model._gdn(x[lo:hi].to(cuda), 0, cache)
        torch.cuda.synchronize()
        _, conv_ref, state_ref, cap = O.gdn_layer(x[lo:hi], w, conv_ref, state_ref, heads=HEADS, head_dim=HD)
        assert set(model._capture) == {f"{n}_0" for n in names}
        for n in names:
            got, want = model._capture[f"{n}_0"], cap[n].float()
            assert got.shape == want.shape, (n, got.shape, want.shape)
            tol = (1e-3 if n == "gdn_state" else 2e-2) if bf16 else 1e-4
            assert rel_err(got, want) < tol, (lo, n, rel_err(got, want))
