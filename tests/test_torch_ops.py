"""The ``torch.ops.zgdn.*`` registrations: schemas and fake shapes on the CPU, the same results as the direct
ops on the GPU (they run the same kernels)."""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from gdn_testing import announce
from oracle import gdn_oracle as O

OPS = ("recurrent_fwd", "decode_step", "chunk_fwd", "fused_decode_step", "serving_decode_step", "attnres_route",
       "accent_shift", "causal_conv1d", "l2norm", "sigmoid", "gated_rmsnorm")


def test_registered_with_mutation_annotations(gdn):
    for name in OPS:
        assert hasattr(torch.ops.zgdn, name), name
    mutated = {
        name: {a.name for a in getattr(torch.ops.zgdn, name).default._schema.arguments
               if a.alias_info is not None and a.alias_info.is_write}
        for name in OPS
    }
    assert mutated["decode_step"] == {"state"}
    assert mutated["fused_decode_step"] == {"conv_cache", "state"}
    assert mutated["serving_decode_step"] == {"conv_live", "conv_commit", "state_live", "state_commit", "window",
                                              "win_len"}
    assert all(not m for n, m in mutated.items()
               if n not in ("decode_step", "fused_decode_step", "serving_decode_step"))


def test_fake_shapes(gdn):
    """Shapes and dtypes of every operator under FakeTensorMode (no kernel runs)."""
    z = torch.ops.zgdn
    with FakeTensorMode():
        q = torch.empty(1, 130, 2, 128, dtype=torch.bfloat16)
        v = torch.empty(1, 130, 4, 128, dtype=torch.bfloat16)
        g = torch.empty(1, 130, 4)
        cu = torch.empty(4, dtype=torch.int32)
        o, s = z.chunk_fwd(q, q, v, g, g, None, None, cu)
        assert o.shape == (1, 130, 4, 128) and o.dtype == torch.bfloat16
        assert s.shape == (3, 4, 128, 128) and s.dtype == torch.float32
        o, s = z.recurrent_fwd(q.float(), q.float(), v.float(), g, g)
        assert o.shape == (1, 130, 4, 128) and o.dtype == torch.float32 and s.shape == (1, 4, 128, 128)
        st = torch.empty(5, 4, 128, 128)
        assert z.decode_step(q[0, :5], q[0, :5], v[0, :5], g[0, :5], g[0, :5], st).shape == (5, 4, 128)
        x = torch.empty(6, 2 * 2 * 128 + 4 * 128, dtype=torch.bfloat16)
        zz = torch.empty(6, 4, 128, dtype=torch.bfloat16)
        ab = torch.empty(6, 4, dtype=torch.bfloat16)
        w = torch.empty(x.shape[1], 4, dtype=torch.bfloat16)
        cache = torch.empty(6, x.shape[1], 3, dtype=torch.bfloat16)
        st6 = torch.empty(6, 4, 128, 128)
        nw = torch.empty(128, dtype=torch.bfloat16)
        hv = torch.empty(4)
        assert z.fused_decode_step(x, zz, ab, ab, w, cache, st6, nw, hv, hv).shape == (6, 4, 128)
        mixed = torch.empty(3, 2056, dtype=torch.bfloat16)
        conv4 = torch.empty(5, 1536, 4, dtype=torch.bfloat16)
        st5 = torch.empty(5, 4, 128, 128)
        win = torch.empty(5, 64, 256, dtype=torch.bfloat16)
        y = z.serving_decode_step(mixed, torch.empty(3, 256, dtype=torch.bfloat16), torch.empty(3, dtype=torch.long),
                                  torch.empty(1536, 4, dtype=torch.bfloat16), conv4, conv4, st5, st5, win,
                                  torch.empty(5, dtype=torch.int32), nw, hv, hv)
        assert y.shape == (3, 4, 128) and y.dtype == torch.bfloat16
        bank = [torch.empty(9, 1024, dtype=torch.bfloat16) for _ in range(5)]
        r = z.attnres_route(bank, torch.empty(1024, dtype=torch.bfloat16), 1e-5)
        assert r.shape == (9, 1024) and r.dtype == torch.bfloat16
        xa = torch.empty(7, 1024, dtype=torch.bfloat16)
        sh = z.accent_shift(xa, torch.empty(24, 1024, dtype=torch.bfloat16), torch.empty(24, 2056, dtype=torch.bfloat16),
                            torch.empty(7, 24, dtype=torch.bfloat16))
        assert sh.shape == (7, 2056) and sh.dtype == torch.bfloat16
        xc = torch.empty(1, 130, 96)
        y, fin = z.causal_conv1d(xc, torch.empty(96, 4), None, None, cu, None, "silu", 3)
        assert y.shape == xc.shape and fin.shape == (3, 96, 3)
        y, rstd = z.l2norm(v)
        assert y.shape == v.shape and rstd.shape == (1, 130, 4) and rstd.dtype == torch.float32
        assert z.sigmoid(g.bfloat16()).dtype == torch.float32
        y, rstd = z.gated_rmsnorm(v, v, nw)
        assert y.shape == v.shape and rstd.shape == (1, 130, 4)


@pytest.mark.gpu
def test_ops_match_direct_calls(gdn, cuda):
    announce("torch.ops.zgdn vs direct ops: chunk, decode (in place), fused block")
    d = O.make_inputs(1, 150, 2, 4, 128, 128, seed=5001, dtype=torch.bfloat16, state_std=0.02)
    x = {n: d[n].to(cuda) for n in ("q", "k", "v", "g", "beta", "s0")}
    o1, s1 = gdn.ops.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["s0"])
    o2, s2 = torch.ops.zgdn.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], None, x["s0"])
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    st1, st2 = x["s0"].clone(), x["s0"].clone()
    a = gdn.ops.decode_step(x["q"][:, 0], x["k"][:, 0], x["v"][:, 0], x["g"][:, 0], x["beta"][:, 0], st1)
    b = torch.ops.zgdn.decode_step(x["q"][:, 0], x["k"][:, 0], x["v"][:, 0], x["g"][:, 0], x["beta"][:, 0], st2)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(st1, st2) and not torch.equal(st2, x["s0"])
    gen = torch.Generator().manual_seed(5003)
    B, Hk, Hv, K = 3, 1, 2, 128
    C = 2 * Hk * K + Hv * K
    xq = torch.randn(B, C, generator=gen).to(torch.bfloat16).to(cuda)
    zz = torch.randn(B, Hv, K, generator=gen).to(torch.bfloat16).to(cuda)
    ab = torch.randn(B, Hv, generator=gen).to(torch.bfloat16).to(cuda)
    w = (0.2 * torch.randn(C, 4, generator=gen)).to(torch.bfloat16).to(cuda)
    nw = (1 + 0.1 * torch.randn(K, generator=gen)).to(torch.bfloat16).to(cuda)
    hv = (0.3 * torch.randn(Hv, generator=gen)).to(cuda)
    cache0 = (0.5 * torch.randn(B, C, 3, generator=gen)).to(torch.bfloat16).to(cuda)
    state0 = (0.02 * torch.randn(B, Hv, K, K, generator=gen)).to(cuda)
    c1, c2, t1, t2 = cache0.clone(), cache0.clone(), state0.clone(), state0.clone()
    y1 = gdn.ops.fused_decode_step(xq, zz, ab, ab, w, c1, t1, nw, hv, hv)
    y2 = torch.ops.zgdn.fused_decode_step(xq, zz, ab, ab, w, c2, t2, nw, hv, hv)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(c1, c2) and torch.equal(t1, t2) and not torch.equal(c2, cache0)


@pytest.mark.gpu
def test_opcheck_decode_and_chunk(gdn, cuda):
    """torch.library.opcheck: schema, fake implementation and dispatch consistency against the real kernels."""
    announce("torch.library.opcheck decode_step, chunk_fwd, l2norm")
    d = O.make_inputs(2, 70, 2, 2, 128, 128, seed=5002, dtype=torch.bfloat16, state_std=0.02)
    x = {n: d[n].to(cuda) for n in ("q", "k", "v", "g", "beta", "s0")}
    tests = ("test_schema", "test_faketensor")
    step = [x[n][:, 0].contiguous() for n in ("q", "k", "v", "g", "beta")]  # the ops take contiguous rows
    torch.library.opcheck(torch.ops.zgdn.decode_step.default, (*step, x["s0"].clone()), test_utils=tests)
    torch.library.opcheck(torch.ops.zgdn.chunk_fwd.default, (x["q"], x["k"], x["v"], x["g"], x["beta"]),
                          test_utils=tests)
    torch.library.opcheck(torch.ops.zgdn.l2norm.default, (x["v"],), test_utils=tests)
