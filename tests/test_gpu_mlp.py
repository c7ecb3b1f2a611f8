"""GPU parity of the grafted SwiGLU MLP forward/backward against the oracle.

Shapes are chosen so the oracle finishes in seconds: aligned bf16 shapes
run the gfx950 MFMA kernel, the f32 and unaligned shapes the generic kernel.
"""
import numpy as np
import pytest

from helpers import (assert_bf16_budget, assert_f32_close, draw, make_layer, rel_l2, to_dev, to_np)
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _run(dev, D, I, N, pl, M, bf16, explicit=True, recompute=False, seed_x=100):
    import torch
    from glt_amd import ops, synth
    dt = torch.bfloat16 if bf16 else torch.float32
    wg, wu, wd, sl = make_layer(D, I, N, pl, bf16)
    x = draw((M, D), seed_x, synth.TID_X, 0, 1, bf16)
    dy = draw((M, D), 200, synth.TID_DY, 0, 1, bf16)
    base = ops.BaseMLP(to_dev(wg, dt), to_dev(wu, dt), to_dev(wd, dt))
    gs = []
    for s in sl:
        g = ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"], *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down")))
        gs.append(g.pack())
    xd, dyd = to_dev(x, dt), to_dev(dy, dt)
    y, gp, up, inter = ops.mlp_forward(base, gs, xd, N, explicit=explicit)
    dx, grads = ops.mlp_backward(base, gs, xd, dyd, N, gp, up, inter, explicit=explicit, recompute=recompute)
    torch.cuda.synchronize()
    osl = sl if explicit else []
    rg, ru, ri, ry = O.mlp_fwd(x, wg, wu, wd, N, osl, bf16=bf16)
    rdx, rgrads = O.mlp_bwd(x, wg, wu, wd, N, osl, rg, ru, ri, dy, bf16=bf16)
    return dict(y=(to_np(y), ry), g=(to_np(gp), rg), u=(to_np(up), ru), inter=(to_np(inter), ri),
                dx=(to_np(dx), rdx), grads=[[to_np(t) if t is not None else None for t in row] for row in grads],
                rgrads=rgrads)


@pytest.mark.parametrize("M,D,I,S", [(256, 256, 512, 128), (512, 512, 1024, 256)])
def test_mfma_appended_bf16(dev, M, D, I, S):
    """The appended form (the graft slice's neurons after the base rows, as in the
    benchmarked layer) on the MFMA path."""
    N = I + S
    r = _run(dev, D, I, N, [(I, S, 0, D)], M, bf16=True)
    for k, q in (("g", 2), ("u", 2), ("inter", 3), ("y", 4)):
        assert_bf16_budget(*r[k], q=q, what=k)
    assert_bf16_budget(*r["dx"], q=4, what="dx")
    for p, name in enumerate(("gate", "up", "down")):
        assert_bf16_budget(r["grads"][0][p], r["rgrads"][0][p], q=2, what=f"dW_{name}")


def test_mfma_many_tiles_per_workgroup(dev):
    """More tiles than CUs (576 gate/up, 288 dInter tiles) with a ragged last
    M-tile: the persistent kernel carries its load stream across tiles."""
    M, D, I, S = 2112, 512, 7936, 256
    N = I + S
    r = _run(dev, D, I, N, [(I, S, 0, D)], M, bf16=True)
    for k, q in (("g", 2), ("u", 2), ("inter", 3), ("y", 4), ("dx", 4)):
        assert_bf16_budget(*r[k], q=q, what=k)
    for p, name in enumerate(("gate", "up", "down")):
        assert_bf16_budget(r["grads"][0][p], r["rgrads"][0][p], q=2, what=f"dW_{name}")


def test_weight_gradients_over_many_tokens(dev):
    """Few weight-gradient tiles over many tokens (6 tiles, 64 K-steps of
    4096 tokens each): an appended slice and an in-place slice with an H
    offset, dX and every gradient against the oracle."""
    M, D, I = 4096, 256, 512
    pl = [(I, 128, 0, 256), (64, 128, 128, 128)]
    N = I + 128
    r = _run(dev, D, I, N, pl, M, bf16=True)
    assert_bf16_budget(*r["dx"], q=4, what="dx")
    for j in range(2):
        for p, name in enumerate(("gate", "up", "down")):
            assert_bf16_budget(r["grads"][j][p], r["rgrads"][j][p], q=2, what=f"slice {j} dW_{name}")


def test_mfma_many_tiles_explicit_off(dev):
    """Graft columns without a segment (explicit off) are zero-K tiles
    interleaved with full ones in each workgroup's tile sequence."""
    M, D, I, S = 1024, 256, 7936, 2048
    N = I + S
    r = _run(dev, D, I, N, [(I, S, 0, D)], M, bf16=True, explicit=False)
    for k, q in (("g", 2), ("u", 2), ("inter", 3), ("y", 4), ("dx", 4)):
        assert_bf16_budget(*r[k], q=q, what=k)
    assert np.all(r["inter"][0][:, I:] == 0)


def test_mfma_inplace_and_stacked_bf16(dev):
    """In-place slices (domain-sliced, the reference's CLI form) plus an
    appended slice, all on the MFMA path (64-aligned)."""
    M, D, I, N = 256, 512, 1024, 1152
    pl = [(0, 128, 0, 256), (512, 256, 256, 256), (1024, 128, 64, 448)]
    r = _run(dev, D, I, N, pl, M, bf16=True)
    for k, q in (("g", 2), ("u", 2), ("inter", 3), ("y", 4), ("dx", 4)):
        assert_bf16_budget(*r[k], q=q, what=k)
    for j in range(len(pl)):
        for p in range(3):
            assert_bf16_budget(r["grads"][j][p], r["rgrads"][j][p], q=2, what=f"slice{j} proj{p}")


def test_eight_slices_the_most_one_call_takes(dev):
    """Eight slices (the limit of glt_mlp_fwd/bwd, glt_shadow_bake and the
    graft AdamW step): six in place over different neuron and hidden ranges,
    two appended; 18 K-segments in the dX GEMM. The forward against the
    oracle; the backward against the oracle's backward fed by the kernel's
    own saved activations (so that a pre-activation one bf16 ulp away from
    the oracle's at a rounding boundary, which moves inter and through it
    the small dW_down entries, is not counted against the backward)."""
    import torch
    from glt_amd import ops, synth
    M, D, I = 256, 256, 512
    pl = [(0, 64, 0, 128), (64, 64, 128, 128), (128, 64, 64, 192), (192, 64, 0, 256),
          (320, 64, 192, 64), (448, 64, 0, 64), (512, 64, 0, 256), (576, 128, 64, 128)]
    N = 704
    bf = torch.bfloat16
    wg, wu, wd, sl = make_layer(D, I, N, pl, True)
    x = draw((M, D), 100, synth.TID_X, 0, 1, True)
    dy = draw((M, D), 200, synth.TID_DY, 0, 1, True)
    base = ops.BaseMLP(to_dev(wg, bf), to_dev(wu, bf), to_dev(wd, bf))
    gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"],
                         *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack() for s in sl]
    xd, dyd = to_dev(x, bf), to_dev(dy, bf)
    y, gp, up, inter = ops.mlp_forward(base, gs, xd, N)
    dx, grads = ops.mlp_backward(base, gs, xd, dyd, N, gp, up, inter)
    torch.cuda.synchronize()
    rg, ru, ri, ry = O.mlp_fwd(x, wg, wu, wd, N, sl, bf16=True)
    for name, a, ref, q in (("g", gp, rg, 2), ("u", up, ru, 2), ("y", y, ry, 4)):
        assert_bf16_budget(to_np(a), ref, q=q, what=name)
    g_k, u_k, i_k = to_np(gp), to_np(up), to_np(inter)
    # inter from the kernel's own g and u: one rounding
    assert_bf16_budget(i_k, O.silu_mul(g_k, u_k), q=1, what="inter from the kernel's g, u")
    assert rel_l2(i_k, ri) <= 1e-2
    rdx, rgrads = O.mlp_bwd(x, wg, wu, wd, N, sl, g_k, u_k, i_k, dy, bf16=True)
    assert_bf16_budget(to_np(dx), rdx, q=4, what="dx")
    for j in range(len(pl)):
        for p in range(3):
            assert_bf16_budget(to_np(grads[j][p]), rgrads[j][p], q=2, what=f"slice{j} proj{p}")


def _random_layer(seed):
    """A random layer the MFMA path takes: a ragged token count, hidden and
    base widths multiples of 64, 1-4 slices in place or appended with
    neuron and hidden offsets on 32-element boundaries (so slice ranges
    straddle the 256-wide tiles and start mid-way through 64-wide K
    blocks), and 0-7 groups of 8 trailing columns that no slice covers."""
    rng = np.random.default_rng(seed)
    M = int(rng.integers(1, 700))
    D = 64 * int(rng.integers(1, 9))
    I = 64 * int(rng.integers(1, 13))
    pl, n = [], I
    for _ in range(int(rng.integers(1, 5))):
        s = 64 * int(rng.integers(1, 4))
        h = 64 * int(rng.integers(1, D // 64 + 1))
        h0 = 32 * int(rng.integers(0, (D - h) // 32 + 1))
        if rng.random() < 0.6 and s <= I:
            i0 = 32 * int(rng.integers(0, (I - s) // 32 + 1))
        else:
            i0, n = n, n + s
        pl.append((i0, s, h0, h))
    return M, D, I, n + 8 * int(rng.integers(0, 8)), pl


@pytest.mark.parametrize("seed", range(8))
def test_mfma_random_layers(dev, seed):
    """Random layer shapes (`_random_layer`) through the forward and the
    graft-only backward: the forward against the oracle, inter against
    silu(g)*u of the kernel's own pre-activations, and the backward against
    the oracle's backward fed by the kernel's saved activations (as in the
    eight-slice test)."""
    import torch
    from glt_amd import ops, synth
    M, D, I, N, pl = _random_layer(seed)
    case = f"seed {seed}: M={M} D={D} I={I} N={N} slices={pl}"
    bf = torch.bfloat16
    wg, wu, wd, sl = make_layer(D, I, N, pl, True)
    x = draw((M, D), 100 + seed, synth.TID_X, 0, 1, True)
    dy = draw((M, D), 200 + seed, synth.TID_DY, 0, 1, True)
    base = ops.BaseMLP(to_dev(wg, bf), to_dev(wu, bf), to_dev(wd, bf))
    gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"],
                         *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack() for s in sl]
    xd, dyd = to_dev(x, bf), to_dev(dy, bf)
    y, gp, up, inter = ops.mlp_forward(base, gs, xd, N)
    dx, grads = ops.mlp_backward(base, gs, xd, dyd, N, gp, up, inter)
    torch.cuda.synchronize()
    rg, ru, ri, ry = O.mlp_fwd(x, wg, wu, wd, N, sl, bf16=True)
    for name, a, ref, q in (("g", gp, rg, 2), ("u", up, ru, 2), ("y", y, ry, 4)):
        assert_bf16_budget(to_np(a), ref, q=q, what=f"{case}: {name}")
    g_k, u_k, i_k = to_np(gp), to_np(up), to_np(inter)
    assert_bf16_budget(i_k, O.silu_mul(g_k, u_k), q=1, what=f"{case}: inter from the kernel's g, u")
    assert rel_l2(i_k, ri) <= 1e-2, case
    rdx, rgrads = O.mlp_bwd(x, wg, wu, wd, N, sl, g_k, u_k, i_k, dy, bf16=True)
    assert_bf16_budget(to_np(dx), rdx, q=4, what=f"{case}: dx")
    for j in range(len(pl)):
        for p in range(3):
            assert_bf16_budget(to_np(grads[j][p]), rgrads[j][p], q=2, what=f"{case}: slice{j} proj{p}")


def test_f32_config1(dev):
    """Config 1: hidden 512, base 1408, 256 appended neurons, 4x128 tokens, fp32."""
    M, D, I, S = 512, 512, 1408, 256
    N = I + S
    r = _run(dev, D, I, N, [(I, S, 0, D)], M, bf16=False)
    for k in ("g", "u", "inter", "y", "dx"):
        assert_f32_close(*r[k], tol=1e-5, what=k)
    for p in range(3):
        assert_f32_close(r["grads"][0][p], r["rgrads"][0][p], tol=1e-5, what=f"dW{p}")


def test_unaligned_bf16_generic(dev):
    """Odd slice placements (H=513-style) go through the generic kernel."""
    M, D, I, N = 70, 100, 130, 150
    pl = [(3, 17, 5, 33), (130, 20, 0, 100)]
    r = _run(dev, D, I, N, pl, M, bf16=True)
    for k, q in (("g", 2), ("u", 2), ("inter", 3), ("y", 4), ("dx", 4)):
        assert_bf16_budget(*r[k], q=q, what=k)


@pytest.mark.parametrize("pl", [[(512, 128, 0, 256)],                            # appended
                                [(0, 128, 0, 256), (256, 128, 64, 128)]])      # in place
def test_recompute_matches_reference_recompute(dev, pl):
    """GLT_MLP_RECOMPUTE against the reference's backward fed by the
    reference's recompute_ffn (src/layer_recompute_impl.inc:8-91), which
    rebuilds each grafted slice as bf16(bf16(base) + bf16(delta)) rather than
    the forward's single rounding: dX and every slice gradient within the
    bf16 budget. (Appended slices: the two roundings coincide; in place: they
    differ by up to one bf16 ulp of the pre-activations.)"""
    import torch
    from glt_amd import ops, synth
    M, D, I = 256, 256, 512
    N = I + sum(s for i0, s, _, _ in pl if i0 >= I)
    wg, wu, wd, sl = make_layer(D, I, N, pl, True)
    x = draw((M, D), 100, synth.TID_X, 0, 1, True)
    dy = draw((M, D), 200, synth.TID_DY, 0, 1, True)
    bf = torch.bfloat16
    base = ops.BaseMLP(to_dev(wg, bf), to_dev(wu, bf), to_dev(wd, bf))
    gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"],
                         *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack() for s in sl]
    xd, dyd = to_dev(x, bf), to_dev(dy, bf)
    dx, grads = ops.mlp_backward(base, gs, xd, dyd, N, recompute=True)
    y, gp, up, inter = ops.mlp_forward(base, gs, xd, N)
    dx_saved, grads_saved = ops.mlp_backward(base, gs, xd, dyd, N, gp, up, inter)
    torch.cuda.synchronize()
    rg, ru, ri = O.mlp_recompute(x, wg, wu, N, sl)
    rdx, rgrads = O.mlp_bwd(x, wg, wu, wd, N, sl, rg, ru, ri, dy, bf16=True)
    assert_bf16_budget(to_np(dx), rdx, q=4, what="dX")
    for j in range(len(sl)):
        for p in range(3):
            assert_bf16_budget(to_np(grads[j][p]), rgrads[j][p], q=2, what=f"slice {j} dW{p}")
    if all(i0 >= I for i0, _, _, _ in pl):
        # appended: the reference's recompute equals its forward, and so do
        # the library's recompute and saved-activation backwards
        fg, fu, fi, _ = O.mlp_fwd(x, wg, wu, wd, N, sl, bf16=True)
        np.testing.assert_array_equal(rg, fg)
        assert torch.equal(dx.view(torch.int32), dx_saved.view(torch.int32))
        for p in range(3):
            assert torch.equal(grads[0][p].view(torch.int32), grads_saved[0][p].view(torch.int32))


def test_f32_upstream_gradient(dev):
    """GLT_MLP_DY_F32: the reference's backward takes an f32 gradient
    (src/layer_backward_impl.inc:48). Drawn off the bf16 grid, it is checked
    against the oracle that multiplies the f32 gradient for the base dInter
    and rounds it to bf16 for the graft GEMMs, and equals the bf16 call on
    the RNE-rounded gradient bit for bit (one rounding inside the call)."""
    import torch
    from glt_amd import ops, synth
    M, D, I, S = 512, 512, 1024, 256
    N = I + S
    wg, wu, wd, sl = make_layer(D, I, N, [(I, S, 0, D)], True)
    x = draw((M, D), 100, synth.TID_X, 0, 1, True)
    dy = draw((M, D), 200, synth.TID_DY, 0, 1, bf16=False)
    assert np.mean(O.bf16_round(dy) != dy) > 0.99
    bf = torch.bfloat16
    base = ops.BaseMLP(to_dev(wg, bf), to_dev(wu, bf), to_dev(wd, bf))
    gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"],
                         *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack() for s in sl]
    xd = to_dev(x, bf)
    y, gp, up, inter = ops.mlp_forward(base, gs, xd, N)
    dx32, g32 = ops.mlp_backward(base, gs, xd, to_dev(dy, torch.float32), N, gp, up, inter)
    dxb, gb = ops.mlp_backward(base, gs, xd, to_dev(O.bf16_round(dy), bf), N, gp, up, inter)
    dx32r, g32r = ops.mlp_backward(base, gs, xd, to_dev(dy, torch.float32), N, recompute=True)
    torch.cuda.synchronize()
    assert torch.equal(dx32.view(torch.int32), dxb.view(torch.int32))
    assert torch.equal(dx32r.view(torch.int32), dxb.view(torch.int32))
    for p in range(3):
        assert torch.equal(g32[0][p].view(torch.int32), gb[0][p].view(torch.int32))
        assert torch.equal(g32r[0][p].view(torch.int32), gb[0][p].view(torch.int32))
    rg, ru, ri, _ = O.mlp_fwd(x, wg, wu, wd, N, sl, bf16=True)
    rdx, rgrads = O.mlp_bwd(x, wg, wu, wd, N, sl, rg, ru, ri, dy, bf16=True)
    assert_bf16_budget(to_np(dx32), rdx, q=4, what="dX (f32 dy)")
    for p in range(3):
        assert_bf16_budget(to_np(g32[0][p]), rgrads[0][p], q=2, what=f"dW{p} (f32 dy)")


def test_explicit_off_is_base_only(dev):
    """use_explicit_graft=false: slices are ignored (reference
    src/layer_forward_impl.inc:76)."""
    M, D, I, S = 128, 256, 512, 128
    N = I + S
    r = _run(dev, D, I, N, [(I, S, 0, D)], M, bf16=True, explicit=False)
    assert_bf16_budget(*r["y"], q=4, what="y")
    assert np.all(r["inter"][0][:, I:] == 0)


def test_test6_f32_explicit_equals_baked(dev):
    """Reference tests/test6_stack_vs_bake_f32.cpp:43-58,199-205: two domains
    (S=3, H=2) in a D=4, F=6 base; explicit injection == baked weights,
    tol 1e-4 abs or 1e-6 rel."""
    import torch
    from glt_amd import ops
    S, H, D, F, M = 3, 2, 4, 6, 2
    gate0 = np.array([(i + 1) * 0.1 for i in range(F * D)], np.float32).reshape(F, D)
    up0 = np.array([(i + 1) * 0.07 for i in range(F * D)], np.float32).reshape(F, D)
    down0 = np.array([(i + 1) * 0.05 for i in range(D * F)], np.float32).reshape(D, F)
    x = np.arange(1, 9, dtype=np.float32).reshape(M, D)

    def mk(b, stp):
        return np.array([[b + i * stp + j for j in range(H)] for i in range(S)], np.float32)

    g0, g1, u0, u1, d0, d1 = mk(0.5, 0.1), mk(0.3, 0.2), mk(0.9, 0.15), mk(0.7, 0.05), mk(1.2, 0.08), mk(1.0, 0.12)
    dt = torch.float32
    base = ops.BaseMLP(to_dev(gate0, dt), to_dev(up0, dt), to_dev(down0, dt))
    gs = [ops.GraftSlice(0, S, 0, H, *(to_dev(a, dt) for a in (g0, u0, d0))).pack(),
          ops.GraftSlice(S, S, H, H, *(to_dev(a, dt) for a in (g1, u1, d1))).pack()]
    y, gp, up, inter = ops.mlp_forward(base, gs, to_dev(x, dt), F)
    # baked weights (path B of the reference test)
    gb, ub, db = gate0.copy(), up0.copy(), down0.copy()
    gb[0:S, 0:H] += g0; gb[S:2 * S, H:2 * H] += g1
    ub[0:S, 0:H] += u0; ub[S:2 * S, H:2 * H] += u1
    db[0:H, 0:S] += d0.T; db[H:2 * H, S:2 * S] += d1.T
    baked = ops.BaseMLP(to_dev(gb, dt), to_dev(ub, dt), to_dev(db, dt))
    yb, gpb, upb, interb = ops.mlp_forward(baked, [], to_dev(x, dt), F, explicit=False)
    torch.cuda.synchronize()
    for a, b, nm in ((gp, gpb, "gate_pre"), (up, upb, "up_pre"), (inter, interb, "inter"), (y, yb, "ffn_out")):
        a, b = to_np(a), to_np(b)
        md = np.max(np.abs(a - b))
        mv = np.max(np.maximum(np.abs(a), np.abs(b)))
        assert md < 1e-4 or md / mv < 1e-6, (nm, md, mv)


@pytest.mark.parametrize("M,D,I,S,bf16", [(512, 512, 1024, 256, True),    # MFMA path
                                          (100, 200, 300, 40, True),      # generic bf16 path
                                          (64, 128, 192, 64, False)])     # f32 path
def test_residual_fused_in_down_epilogue(dev, M, D, I, S, bf16):
    """GLT_MLP_RESIDUAL: y = round(residual + round(ffn_out)) written by the
    down GEMM's epilogue, bit-for-bit the reference's x = x + ffn_out on the
    path dtype (src/layer_forward_impl.inc:271-275) over the plain output."""
    import torch
    from glt_amd import ops, synth
    dt = torch.bfloat16 if bf16 else torch.float32
    N = I + S
    wg, wu, wd, sl = make_layer(D, I, N, [(I, S, 0, D)], bf16)
    base = ops.BaseMLP(to_dev(wg, dt), to_dev(wu, dt), to_dev(wd, dt))
    gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"],
                         *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack() for s in sl]
    x = to_dev(draw((M, D), 100, synth.TID_X, 0, 1, bf16), dt)
    res = draw((M, D), 7, 77, 0, 1, bf16)
    y, _, _, _ = ops.mlp_forward(base, gs, x, N)
    yr_in = to_dev(res, dt)
    yr, _, _, _ = ops.mlp_forward(base, gs, x, N, residual=yr_in)
    torch.cuda.synchronize()
    assert yr.data_ptr() == yr_in.data_ptr()
    ffn = to_np(y)
    if bf16:
        exp = O.f32_to_bf16_bits(res.astype(np.float32) + ffn)
        np.testing.assert_array_equal(yr.view(torch.int16).cpu().numpy().view(np.uint16), exp)
    else:
        np.testing.assert_array_equal(to_np(yr), res + ffn)


def test_pipelined_adamw_stream_matches_sequential(dev):
    """The reference's pipelined AdamW stream (grafting.hip:1165-1172): the
    backward runs on one stream, an event hands its gradients to a second
    stream that runs the graft AdamW step (with the packed-mirror refresh).
    Masters, moments and mirrors match a single-stream run bit for bit."""
    import torch
    from glt_amd import ops, synth
    M, D, I, S = 512, 512, 1024, 256
    N = I + S
    wg, wu, wd, sl = make_layer(D, I, N, [(I, S, 0, D)], True)
    s0 = sl[0]
    x = to_dev(draw((M, D), 100, synth.TID_X, 0, 1, True), torch.bfloat16)
    dy = to_dev(draw((M, D), 200, synth.TID_DY, 0, 1, True), torch.bfloat16)
    base = ops.BaseMLP(to_dev(wg, torch.bfloat16), to_dev(wu, torch.bfloat16), to_dev(wd, torch.bfloat16))

    def fresh():
        g = ops.GraftSlice(s0["i0"], s0["s"], s0["h0"], s0["h"],
                           *(to_dev(s0[p], torch.float32) for p in ("gate", "up", "down"))).pack()
        return g, torch.zeros(3 * S * D, device=dev), torch.zeros(3 * S * D, device=dev)

    def step(g, m, v, s_bwd, s_opt):
        s_bwd.wait_stream(torch.cuda.current_stream())  # inputs were made on the current stream
        with torch.cuda.stream(s_bwd):
            y, gp, up, inter = ops.mlp_forward(base, [g], x, N)
            _, grads = ops.mlp_backward(base, [g], x, dy, N, gp, up, inter)
            done = torch.cuda.Event()
            done.record(s_bwd)
        if s_opt is not s_bwd:
            s_opt.wait_event(done)
        with torch.cuda.stream(s_opt):
            flat = torch.cat([t.reshape(-1) for t in grads[0]])
            ops.adamw_graft_step([g], [flat], [m], [v], 0, 1e-3)
        torch.cuda.synchronize()

    ref = fresh()
    main = torch.cuda.current_stream()
    step(*ref, main, main)
    pip = fresh()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    step(*pip, s1, s2)
    bits = lambda t: t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)
    for a, b in zip((ref[0].gate, ref[0].up, ref[0].down, ref[1], ref[2], ref[0].packed),
                    (pip[0].gate, pip[0].up, pip[0].down, pip[1], pip[2], pip[0].packed)):
        assert torch.equal(bits(a), bits(b))
    assert torch.count_nonzero(ref[1]).item() > 0  # the step did update the moments


@pytest.mark.parametrize("M,D,I,S,n_slices", [(2048, 1024, 2048, 256, 1),   # weight gradients leave CUs idle
                                               (512, 512, 1024, 128, 0),     # no slices: no weight gradients
                                               (512, 4608, 1024, 256, 1),    # rows past 4096: not forked
                                               (1000, 1088, 1024, 128, 1)])  # 136 chunks per row: ragged lanes, ragged M
def test_mlp_rmsnorm_bwd_equals_the_two_calls(dev, M, D, I, S, n_slices):
    """glt_mlp_rmsnorm_bwd (the FFN backward with the FFN norm's backward
    beside its weight-gradient GEMM) gives glt_mlp_bwd's dx and gradients and
    glt_rmsnorm_bwd's norm gradient bit for bit, whether or not the norm's
    backward runs on the helper stream; and so do both calls with the norm's
    gradient written in place over their input gradient."""
    import torch
    from glt_amd import ops, synth
    N = I + S
    pl = [(I, S, 0, D)] if n_slices else []
    wg, wu, wd, sl = make_layer(D, I, N, pl, True)
    dt = torch.bfloat16
    base = ops.BaseMLP(to_dev(wg, dt), to_dev(wu, dt), to_dev(wd, dt))
    gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"], *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack()
          for s in sl]
    x_raw = to_dev(draw((M, D), 100, synth.TID_X, 0, 1, True), dt)
    gamma = to_dev(draw((D,), 300, synth.TID_GAMMA, 1.0, 0.02, True), dt)
    dy = to_dev(draw((M, D), 200, synth.TID_DY, 0, 1, False), torch.float32)
    x, var = ops.rms_norm(x_raw, gamma, 1e-5)
    y, gp, up, inter = ops.mlp_forward(base, gs, x, N)
    dx0, g0 = ops.mlp_backward(base, gs, x, dy, N, gp, up, inter)
    nd0 = ops.rms_norm_bwd(dx0, x_raw, gamma, var, 1e-5)
    dx1, g1, nd1 = ops.mlp_backward(base, gs, x, dy, N, gp, up, inter, norm=(x_raw, gamma, var, 1e-5))
    torch.cuda.synchronize()
    assert torch.equal(dx0, dx1)
    assert torch.equal(nd0, nd1)
    for r0, r1 in zip(g0, g1):
        for a, b in zip(r0, r1):
            assert (a is None) == (b is None) and (a is None or torch.equal(a, b))
    # in place: norm_dx == dx
    dx2, g2, nd2 = ops.mlp_backward(base, gs, x, dy, N, gp, up, inter, norm=(x_raw, gamma, var, 1e-5),
                                    norm_in_place=True)
    nd3 = dx0.clone()
    ops.rms_norm_bwd(nd3, x_raw, gamma, var, 1e-5, out=nd3)
    torch.cuda.synchronize()
    assert nd2 is dx2 and torch.equal(nd2, nd0) and torch.equal(nd3, nd0)
    for r0, r2 in zip(g0, g2):
        for a, b in zip(r0, r2):
            assert (a is None) == (b is None) and (a is None or torch.equal(a, b))


def test_mlp_rmsnorm_bwd_in_a_graph(dev):
    """glt_mlp_rmsnorm_bwd's fork onto the helper stream and its join are
    captured with the caller's stream: a graph of the call, replayed three
    times with eager work between the replays, reproduces the eager call's dx,
    gradients and norm gradient bit for bit every time."""
    import ctypes
    import torch
    from glt_amd import _ffi as F, ops, synth
    M, D, I, S = 2048, 1024, 2048, 256
    N = I + S
    wg, wu, wd, sl = make_layer(D, I, N, [(I, S, 0, D)], True)
    dt = torch.bfloat16
    base = ops.BaseMLP(to_dev(wg, dt), to_dev(wu, dt), to_dev(wd, dt))
    gsl = ops.GraftSlice(sl[0]["i0"], S, 0, D, *(to_dev(sl[0][p], torch.float32) for p in ("gate", "up", "down")))
    gs = [gsl.pack()]
    x_raw = to_dev(draw((M, D), 100, synth.TID_X, 0, 1, True), dt)
    gamma = to_dev(draw((D,), 300, synth.TID_GAMMA, 1.0, 0.02, True), dt)
    dy = to_dev(draw((M, D), 200, synth.TID_DY, 0, 1, False), torch.float32)
    x, var = ops.rms_norm(x_raw, gamma, 1e-5)
    y, gp, up, inter = ops.mlp_forward(base, gs, x, N)
    dx_e, g_e, nd_e = ops.mlp_backward(base, gs, x, dy, N, gp, up, inter, norm=(x_raw, gamma, var, 1e-5))
    torch.cuda.synchronize()

    # the same call on preallocated buffers, captured
    d, keep = ops._desc(base, gs, M, N, True, dy_f32=True)
    nbytes = F.load().glt_mlp_bwd_workspace_size(ctypes.byref(d))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dx = torch.empty((M, D), dtype=torch.float32, device="cuda")
    nd = torch.empty_like(dx)
    grads = [torch.empty((S, D), dtype=torch.float32, device="cuda") for _ in range(3)]
    garr = (F.GraftGrads * 1)()
    garr[0] = F.GraftGrads(*(t.data_ptr() for t in grads))
    b = base.c_struct()
    p = lambda t: ctypes.c_void_p(t.data_ptr())

    def call():
        F.call("glt_mlp_rmsnorm_bwd", ctypes.byref(d), ctypes.byref(b), p(x), p(dy), p(gp), p(up), p(inter), p(dx),
               garr, p(ws), nbytes, p(x_raw), p(gamma), p(var), 1e-5,
               p(nd), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()   # first call sets per-device kernel attributes and creates the helper stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep in range(3):
        for t in (dx, nd, *grads):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(dx, dx_e), rep
        assert torch.equal(nd, nd_e), rep
        for a, r in zip(grads, g_e[0]):
            assert torch.equal(a, r), rep
        _ = (x_raw.float() * 2).sum()   # eager work between replays
        torch.cuda.synchronize()


def test_outputs_past_two_gib_split_into_row_blocks(dev):
    """65536 tokens at N = 16384: the gate/up outputs and the dInter GEMM's
    outputs and saved pre-activations pass 2 GiB, beyond the MFMA kernel's
    31-bit buffer offsets, so run_gemm runs them as row blocks (65280 rows,
    then 256). Token rows on both sides of the block boundary and at the
    ends equal a call on just those tokens, bit for bit (every output row
    depends on its own token only)."""
    import torch
    from glt_amd import ops, synth
    M, D, I, S = 65536, 256, 16128, 256
    N = I + S
    wg, wu, wd, sl = make_layer(D, I, N, [(I, S, 0, D)], True)
    dt = torch.bfloat16
    base = ops.BaseMLP(to_dev(wg, dt), to_dev(wu, dt), to_dev(wd, dt))
    gs = [ops.GraftSlice(sl[0]["i0"], S, 0, D, *(to_dev(sl[0][p], torch.float32) for p in ("gate", "up", "down"))).pack()]
    x = ops.fill_normal(torch.empty((M, D), dtype=dt, device="cuda"), 100, 10, 0.0, 1.0)
    dy = ops.fill_normal(torch.empty((M, D), dtype=dt, device="cuda"), 200, 11, 0.0, 1.0)
    y, g, u, inter = ops.mlp_forward(base, gs, x, N)
    dx, _ = ops.mlp_backward(base, gs, x, dy, N, g, u, inter)
    torch.cuda.synchronize()
    for r0 in (0, 65280 - 256, 65536 - 512):
        rows = slice(r0, r0 + 512)
        ys, gss, us, iss = ops.mlp_forward(base, gs, x[rows].contiguous(), N)
        dxs, _ = ops.mlp_backward(base, gs, x[rows].contiguous(), dy[rows].contiguous(), N, gss, us, iss)
        torch.cuda.synchronize()
        for name, big, small in (("y", y, ys), ("gate_pre", g, gss), ("up_pre", u, us), ("inter", inter, iss)):
            assert torch.equal(big[rows].view(torch.int16), small.view(torch.int16)), (name, r0)
        assert torch.equal(dx[rows].view(torch.int32), dxs.view(torch.int32)), ("dx", r0)
