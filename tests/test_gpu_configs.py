"""The stacked-graft and bake-sentinel workloads at the Llama-3-8B MLP shape
(hidden 4096, base intermediate 14336), with fewer tokens than the
benchmark: the properties checked hold per token.

* Four stacked 512-neuron slices (seeds 1..4) appended after the base
  (N = 16384), forward only: explicit stacked grafts against the same
  forward over shadow-baked merged weights, and against the oracle on a
  token sample.
* shadow_bake materialising [15360,4096] / [4096,15360] baked matrices for
  several layers, then the sentinel forward (X ~N(0,1) [2048,4096]) baked
  against stacked, per layer.
"""
import numpy as np
import pytest

from helpers import assert_bf16_budget, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

D, I = 4096, 14336


def _base(torch, ops, seed=0, tid0=1):
    bf = torch.bfloat16
    wg = ops.fill_normal(torch.empty((I, D), dtype=bf, device="cuda"), seed, tid0, 0.0, 0.02)
    wu = ops.fill_normal(torch.empty((I, D), dtype=bf, device="cuda"), seed, tid0 + 1, 0.0, 0.02)
    wd = ops.fill_normal(torch.empty((D, I), dtype=bf, device="cuda"), seed, tid0 + 2, 0.0, 0.02)
    return wg, wu, wd


def _slices(torch, ops, placements, seeds):
    out = []
    for (i0, s, h0, h), seed in zip(placements, seeds):
        ms = [ops.fill_normal(torch.empty((s, h), dtype=torch.float32, device="cuda"), seed, 1 + p, 0.0, 0.02)
              for p in range(3)]
        out.append(ops.GraftSlice(i0, s, h0, h, *ms).pack())
    return out


def _baked_forward(torch, ops, wg, wu, wd, slices, x, N):
    """Materialise the merged weights with shadow_bake, then run the plain
    (non-explicit) forward over them."""
    from glt_amd import _ffi as F
    bf = torch.bfloat16
    go = torch.empty((N, D), dtype=bf, device="cuda")
    uo = torch.empty((N, D), dtype=bf, device="cuda")
    do = torch.empty((D, N), dtype=bf, device="cuda")
    flat = [[torch.cat([sl.gate.reshape(-1), sl.up.reshape(-1), sl.down.reshape(-1)])] for sl in slices]
    ops.shadow_bake(F.ModelState(0), [wg], [wu], [wd], flat, [(s.i_start, s.s, s.h_start, s.h) for s in slices],
                    D=D, I=I, N=N, materialize=True, gate_out=[go], up_out=[uo], down_out=[do])
    baked = ops.BaseMLP(go, uo, do)
    return ops.mlp_forward(baked, [], x, N, explicit=False), (go, uo, do)


def test_stacked_four_slices_vs_baked_and_oracle(dev):
    import torch
    from glt_amd import ops
    M, S = 1024, 512
    N = I + 4 * S
    placements = [(I + S * k, S, 0, D) for k in range(4)]
    wg, wu, wd = _base(torch, ops)
    slices = _slices(torch, ops, placements, seeds=(1, 2, 3, 4))
    x = ops.fill_normal(torch.empty((M, D), dtype=torch.bfloat16, device="cuda"), 100, 10, 0.0, 1.0)
    base = ops.BaseMLP(wg, wu, wd)
    y, g, u, inter = ops.mlp_forward(base, slices, x, N)
    (yb, gb, ub, ib), _ = _baked_forward(torch, ops, wg, wu, wd, slices, x, N)
    torch.cuda.synchronize()
    # appended slices: the baked rows are bf16(delta) exactly, so only the
    # accumulation order differs
    for name, a, b, q in (("gate_pre", g, gb, 2), ("up_pre", u, ub, 2), ("inter", inter, ib, 3), ("y", y, yb, 4)):
        assert_bf16_budget(to_np(a), to_np(b), q=q, what=f"stacked vs baked {name}")
    # oracle on a token sample
    T = 32
    h = lambda t: to_np(t)
    sl_np = [{"i0": s.i_start, "s": s.s, "h0": s.h_start, "h": s.h, "gate": h(s.gate), "up": h(s.up),
              "down": h(s.down)} for s in slices]
    rg, ru, ri, ry = O.mlp_fwd(h(x[:T]), h(wg), h(wu), h(wd), N, sl_np, bf16=True)
    for name, a, r, q in (("gate_pre", g, rg, 2), ("up_pre", u, ru, 2), ("inter", inter, ri, 3), ("y", y, ry, 4)):
        assert_bf16_budget(to_np(a[:T]), r, q=q, what=f"stacked vs oracle {name}")


def test_bake_sentinel_forward(dev):
    import torch
    from glt_amd import ops
    M, S, L = 2048, 1024, 2
    N = I + S
    x = ops.fill_normal(torch.empty((M, D), dtype=torch.bfloat16, device="cuda"), 100, 10, 0.0, 1.0)
    for layer in range(L):
        wg, wu, wd = _base(torch, ops, seed=0, tid0=1000 + 3 * layer)
        slices = _slices(torch, ops, [(I, S, 0, D)], seeds=(1 + layer,))
        base = ops.BaseMLP(wg, wu, wd)
        y, _, _, _ = ops.mlp_forward(base, slices, x, N)
        (yb, _, _, _), (go, uo, do) = _baked_forward(torch, ops, wg, wu, wd, slices, x, N)
        torch.cuda.synchronize()
        assert_bf16_budget(to_np(y), to_np(yb), q=4, what=f"layer {layer} baked vs stacked y")
        # baked matrices: base rows copied, graft rows bf16(delta), down graft
        # columns bf16(delta^T)
        sl = slices[0]
        assert torch.equal(go[:I], wg) and torch.equal(uo[:I], wu) and torch.equal(do[:, :I], wd)
        np.testing.assert_array_equal(to_np(go[I:]), O.bf16_round(to_np(sl.gate)))
        np.testing.assert_array_equal(to_np(do[:, I:]), O.bf16_round(to_np(sl.down)).T)
        del base, go, uo, do
        torch.cuda.empty_cache()
