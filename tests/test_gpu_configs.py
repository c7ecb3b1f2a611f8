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


def test_config2_full_size_step_properties(dev):
    """The measured workload at its full size (16384 tokens, hidden 4096, base
    14336, one appended 1024-neuron slice), checked through properties that
    hold at any size:
    * per-token outputs (y, gate/up pre-activations, inter, dX) on a token
      sample against the oracle;
    * graft weight gradients, reductions over all 16384 tokens: sampled
      entries of dW_down = inter_i^T . dy and of dW_gate = dg_i^T . x against
      an f64 computation from the step's own saved bf16 activations;
    * linearity over tokens: the two half-size steps' gradients sum to the
      full step's, and their per-token outputs equal the full step's rows
      bit for bit."""
    import torch
    from glt_amd import ops
    M, S = 16384, 1024
    N = I + S
    wg, wu, wd = _base(torch, ops)
    slices = _slices(torch, ops, [(I, S, 0, D)], seeds=(1,))
    x = ops.fill_normal(torch.empty((M, D), dtype=torch.bfloat16, device="cuda"), 100, 10, 0.0, 1.0)
    dy = ops.fill_normal(torch.empty((M, D), dtype=torch.bfloat16, device="cuda"), 200, 11, 0.0, 1.0)
    base = ops.BaseMLP(wg, wu, wd)
    y, g, u, inter = ops.mlp_forward(base, slices, x, N)
    dx, grads = ops.mlp_backward(base, slices, x, dy, N, g, u, inter)
    torch.cuda.synchronize()
    print("full-size step done", flush=True)

    # per-token outputs against the oracle on a token sample spanning the M tiles
    rows = torch.tensor([0, 1, 255, 256, 4095, 8192, 12345, 16383], device="cuda")
    h = lambda t: to_np(t)
    sl = slices[0]
    sl_np = [{"i0": sl.i_start, "s": sl.s, "h0": sl.h_start, "h": sl.h, "gate": h(sl.gate), "up": h(sl.up),
              "down": h(sl.down)}]
    xs, dys = h(x[rows]), h(dy[rows])
    wg_np, wu_np, wd_np = h(wg), h(wu), h(wd)
    rg, ru, ri, ry = O.mlp_fwd(xs, wg_np, wu_np, wd_np, N, sl_np, bf16=True)
    for name, a, r, q in (("gate_pre", g, rg, 2), ("up_pre", u, ru, 2), ("inter", inter, ri, 3), ("y", y, ry, 4)):
        assert_bf16_budget(h(a[rows]), r, q=q, what=f"full-size {name}")
    rdx, _ = O.mlp_bwd(xs, wg_np, wu_np, wd_np, N, sl_np, rg, ru, ri, dys, bf16=True)
    assert_bf16_budget(h(dx[rows]), rdx, q=4, what="full-size dX")
    del wg_np, wu_np, wd_np

    # sampled graft-gradient entries over all tokens, in f64 from the saved
    # bf16 activations
    dyf = h(dy).astype(np.float64)
    xf = h(x).astype(np.float64)
    dd = O.bf16_round(h(sl.down)).astype(np.float64)                  # bf16 mirror of the down delta [S, H]
    for s in (0, 511, 1023):
        col = I + s
        it = h(inter[:, col]).astype(np.float64)
        gt = h(g[:, col]).astype(np.float64)
        ut = h(u[:, col]).astype(np.float64)
        di = (dyf @ dd[s]).astype(np.float32)                         # dInter of graft column s (f32 accumulator)
        sg = 1.0 / (1.0 + np.exp(-gt))
        dg = O.bf16_round((di * ut * (sg * (1.0 + gt * (1.0 - sg)))).astype(np.float32)).astype(np.float64)
        for hh in (0, 2047, 4095):
            terms = it * dyf[:, hh]
            got = float(grads[0][2][s, hh])
            assert abs(got - terms.sum()) <= 1e-4 * np.abs(terms).sum() + 1e-6, ("dW_down", s, hh, got, terms.sum())
            terms = dg * xf[:, hh]
            got = float(grads[0][0][s, hh])
            assert abs(got - terms.sum()) <= 1e-2 * np.abs(terms).sum() + 1e-6, ("dW_gate", s, hh, got, terms.sum())
    del dyf, xf

    # linearity over tokens
    half = M // 2
    parts = []
    for a, b in ((0, half), (half, M)):
        ya, ga, ua, ia = ops.mlp_forward(base, slices, x[a:b].contiguous(), N)
        dxa, gra = ops.mlp_backward(base, slices, x[a:b].contiguous(), dy[a:b].contiguous(), N, ga, ua, ia)
        torch.cuda.synchronize()
        assert torch.equal(ya.view(torch.int16), y[a:b].view(torch.int16))
        assert torch.equal(dxa.view(torch.int32), dx[a:b].view(torch.int32))
        parts.append(gra)
        del ya, ga, ua, ia, dxa
    for p in range(3):
        full = grads[0][p].double()
        summed = parts[0][0][p].double() + parts[1][0][p].double()
        scale = full.abs().max().item()
        assert (summed - full).abs().max().item() <= 1e-5 * scale, p
