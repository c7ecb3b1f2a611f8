"""GPU parity of the bandwidth-bound kernels (bake, RMSNorm, RoPE, AdamW,
elementwise probes, conversions) and the graft-GEMM kinds."""
import numpy as np
import pytest

from helpers import (assert_bf16_budget, assert_f32_close, draw, packed_views, rel_l2, shuffle_b, to_dev,
                     to_np)
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bits(t):
    import torch
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


# ------------------------------------------------------------ shadow bake
def test_bake_test22_sentinel(dev):
    """Reference tests/test22_shadow_bake_sentinel.cpp:72-260: H=513 > 256,
    S=3, 2 layers, sentinel (l*100+p*10+s)*1000+h+1, orientation, h>=256
    coverage, projection mask, layer range, double-bake guard. Checked
    bit-exact against the oracle and within the test's 0.5+0.5% tolerance."""
    import torch
    from glt_amd import _ffi, ops
    S, H, L = 3, 513, 2

    def val(l, p, s, h):
        return float((l * 100 + p * 10 + s) * 1000 + h + 1)

    graft = np.zeros((L, 3, S, H), np.float32)
    for l in range(L):
        for p in range(3):
            for s in range(S):
                graft[l, p, s] = [val(l, p, s, h) for h in range(H)]

    def run(mask=7, lo=0, hi=L - 1):
        gate = [torch.zeros((S, H), dtype=torch.bfloat16, device=dev) for _ in range(L)]
        up = [torch.zeros((S, H), dtype=torch.bfloat16, device=dev) for _ in range(L)]
        down = [torch.zeros((H, S), dtype=torch.bfloat16, device=dev) for _ in range(L)]
        gr = [[torch.from_numpy(graft[l].ravel().copy()).cuda() for l in range(L)]]
        st = _ffi.ModelState(0)
        ops.shadow_bake(st, gate, up, down, gr, [(0, S, 0, H)], D=H, I=S, proj_mask=mask, layer_start=lo,
                        layer_end=hi)
        torch.cuda.synchronize()
        return st, gate, up, down, gr

    st, gate, up, down, gr = run()
    for l in range(L):
        for p, mats, mode in ((0, gate, 0), (1, up, 0), (2, down, 1)):
            ref = np.zeros((S, H) if mode == 0 else (H, S), np.uint16)
            O.bake_inplace(ref, graft[l, p], 0, 0, mode)
            got = _bits(mats[l])
            np.testing.assert_array_equal(got, ref)
            f = O.bf16_bits_to_f32(got)
            exp = np.array([[val(l, p, s, h) for h in range(H)] for s in range(S)], np.float32)
            exp = exp if mode == 0 else exp.T
            assert np.all(np.abs(f - exp) <= 0.5 + 0.005 * np.abs(exp))
    # h-loop coverage: column 300 baked
    assert np.all(O.bf16_bits_to_f32(_bits(gate[0]))[:, 300] != 0)
    # double bake on the same state is refused
    with pytest.raises(_ffi.GltError) as e:
        ops.shadow_bake(st, gate, up, down, gr, [(0, S, 0, H)], D=H, I=S)
    assert e.value.status == "GLT_ERR_ALREADY_BAKED"
    # projection mask: gate off -> untouched
    st, gate, up, down, _ = run(mask=6)
    assert np.all(_bits(gate[0]) == 0) and np.any(_bits(up[0]) != 0) and np.any(_bits(down[0]) != 0)
    # layer range: only layer 1
    st, gate, up, down, _ = run(lo=1, hi=1)
    assert np.all(_bits(gate[0]) == 0) and np.any(_bits(gate[1]) != 0)


def test_bake_test5_two_domains(dev):
    """Reference tests/test5_bake_in_sentinel.py:24-139: two domains baked
    in place into zero [6,4]/[4,6] bases; values seed+10i+j; cross-domain
    blocks stay zero; order of the two bakes does not matter."""
    import torch
    from glt_amd import _ffi, ops
    S, H = 3, 2
    F, D = 2 * S, 2 * H

    def sent(seed):
        return np.array([[seed + i * 10 + j for j in range(H)] for i in range(S)], np.float32)

    def bake(order):
        gate = [torch.zeros((F, D), dtype=torch.bfloat16, device=dev)]
        up = [torch.zeros((F, D), dtype=torch.bfloat16, device=dev)]
        down = [torch.zeros((D, F), dtype=torch.bfloat16, device=dev)]
        for dom in order:
            flat = np.stack([sent(100 + 100 * dom), sent(300 + 100 * dom), sent(500 + 100 * dom)]).ravel()
            st = _ffi.ModelState(0)  # one bake per domain: separate guard states
            ops.shadow_bake(st, gate, up, down, [[torch.from_numpy(flat).cuda()]], [(dom * S, S, dom * H, H)],
                            D=D, I=F)
        torch.cuda.synchronize()
        return [O.bf16_bits_to_f32(_bits(t[0])) for t in (gate, up, down)]

    g, u, d = bake([0, 1])
    # the bases hold bf16, so each sentinel lands as its RNE bf16 value
    # (e.g. 501 -> 500, 511 -> 512); orientation is what the test pins
    rb = O.bf16_round
    np.testing.assert_array_equal(g[0:3, 0:2], rb(sent(100)))
    np.testing.assert_array_equal(g[3:6, 2:4], rb(sent(200)))
    np.testing.assert_array_equal(u[0:3, 0:2], rb(sent(300)))
    np.testing.assert_array_equal(d[0:2, 0:3], rb(sent(500).T))
    np.testing.assert_array_equal(d[2:4, 3:6], rb(sent(600).T))
    assert np.all(g[0:3, 2:4] == 0) and np.all(g[3:6, 0:2] == 0)
    assert np.all(d[0:2, 3:6] == 0) and np.all(d[2:4, 0:3] == 0)
    g2, u2, d2 = bake([1, 0])
    np.testing.assert_array_equal(g, g2)
    np.testing.assert_array_equal(d, d2)


@pytest.mark.parametrize("gdt", ["f32", "bf16"])
def test_bake_materialize_bitexact(dev, gdt):
    """Materialised bake (appended slices into zero-extended [N,D]/[D,N])
    is bit-exact against an independent numpy construction."""
    import torch
    from glt_amd import _ffi, ops
    L, D, I = 3, 256, 384
    pl = [(384, 64, 0, 256), (448, 64, 0, 256), (40, 24, 72, 40)]
    N = 512
    rng = np.random.default_rng(7)
    bases = [[O.bf16_round(rng.normal(0, 0.02, sh).astype(np.float32)) for sh in ((I, D), (I, D), (D, I))]
             for _ in range(L)]
    grafts = []
    for (i0, s, h0, h) in pl:
        per = []
        for l in range(L):
            a = rng.normal(0, 0.02, (3, s, h)).astype(np.float32)
            per.append(O.bf16_round(a) if gdt == "bf16" else a)
        grafts.append(per)
    tdt = torch.bfloat16 if gdt == "bf16" else torch.float32
    dev_b = [[to_dev(b, torch.bfloat16) for b in lay] for lay in bases]
    outs = [[torch.empty((N, D), dtype=torch.bfloat16, device=dev) for _ in range(L)] for _ in range(2)] + \
           [[torch.empty((D, N), dtype=torch.bfloat16, device=dev) for _ in range(L)]]
    st = _ffi.ModelState(0)
    ops.shadow_bake(st, [b[0] for b in dev_b], [b[1] for b in dev_b], [b[2] for b in dev_b],
                    [[to_dev(g.ravel(), tdt) for g in per] for per in grafts], pl, D=D, I=I, N=N,
                    materialize=True, gate_out=outs[0], up_out=outs[1], down_out=outs[2])
    torch.cuda.synchronize()
    for l in range(L):
        for p in range(3):
            ref = np.zeros((N, D) if p < 2 else (D, N), np.float32)
            if p < 2:
                ref[:I] = bases[l][p]
            else:
                ref[:, :I] = bases[l][p]
            for j, (i0, s, h0, h) in enumerate(pl):
                blk = grafts[j][l][p]
                if p < 2:
                    ref[i0:i0 + s, h0:h0 + h] += blk
                else:
                    ref[h0:h0 + h, i0:i0 + s] += blk.T
            np.testing.assert_array_equal(_bits(outs[p][l]), O.f32_to_bf16_bits(ref))
            # inputs untouched
            np.testing.assert_array_equal(_bits(dev_b[l][p]), O.f32_to_bf16_bits(bases[l][p]))


@pytest.mark.parametrize("materialize", [True, False])
def test_bake_seven_slices_eighteen_layers(dev, materialize):
    """As many slices as the MLP path stacks (7) and more layers than one
    launch takes (18 > 16): materialised (4 appended + 3 in-place slices) and
    in place (7 in-place slices), bit-exact against numpy."""
    import torch
    from glt_amd import _ffi, ops
    L, D, I = 18, 256, 384
    if materialize:
        pl = [(384, 32, 0, 256), (416, 32, 64, 128), (448, 32, 0, 64), (480, 32, 32, 200),
              (0, 16, 0, 64), (40, 24, 72, 40), (100, 8, 200, 56)]
        N = 512
    else:
        pl = [(0, 16, 0, 64), (40, 24, 72, 40), (100, 8, 200, 56), (128, 64, 0, 256), (200, 40, 8, 24),
              (300, 50, 100, 156), (360, 24, 250, 6)]
        N = I
    rng = np.random.default_rng(11)
    bases = [[O.bf16_round(rng.normal(0, 0.02, sh).astype(np.float32)) for sh in ((I, D), (I, D), (D, I))]
             for _ in range(L)]
    grafts = [[rng.normal(0, 0.02, (3, sz, h)).astype(np.float32) for _ in range(L)] for (i0, sz, h0, h) in pl]
    dev_b = [[to_dev(b, torch.bfloat16) for b in lay] for lay in bases]
    st = _ffi.ModelState(0)
    if materialize:
        outs = [[torch.empty((N, D), dtype=torch.bfloat16, device=dev) for _ in range(L)] for _ in range(2)] + \
               [[torch.empty((D, N), dtype=torch.bfloat16, device=dev) for _ in range(L)]]
    else:
        outs = [[b[p] for b in dev_b] for p in range(3)]
    ops.shadow_bake(st, [b[0] for b in dev_b], [b[1] for b in dev_b], [b[2] for b in dev_b],
                    [[to_dev(g.ravel(), torch.float32) for g in per] for per in grafts], pl, D=D, I=I, N=N,
                    materialize=materialize, gate_out=outs[0] if materialize else None,
                    up_out=outs[1] if materialize else None, down_out=outs[2] if materialize else None)
    torch.cuda.synchronize()
    assert st.baked == 1
    for l in range(L):
        for p in range(3):
            ref = np.zeros((N, D) if p < 2 else (D, N), np.float32)
            if p < 2:
                ref[:I] = bases[l][p]
            else:
                ref[:, :I] = bases[l][p]
            for j, (i0, sz, h0, h) in enumerate(pl):
                blk = grafts[j][l][p]
                if p < 2:
                    ref[i0:i0 + sz, h0:h0 + h] += blk
                else:
                    ref[h0:h0 + h, i0:i0 + sz] += blk.T
            np.testing.assert_array_equal(_bits(outs[p][l]), O.f32_to_bf16_bits(ref), err_msg=f"{l} {p}")


# ---------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("M,D", [(64, 4096), (33, 513), (16, 8192)])
def test_rmsnorm(dev, M, D):
    import torch
    from glt_amd import ops
    x = draw((M, D), 1, 1)
    w = O.bf16_round(1 + draw((D,), 300, 12, 0, 0.02, bf16=False))
    dy = draw((M, D), 2, 2, bf16=False)
    y, var = ops.rms_norm(to_dev(x, torch.bfloat16), to_dev(w, torch.bfloat16), 1e-5)
    dx = ops.rms_norm_bwd(to_dev(dy, torch.float32), to_dev(x, torch.bfloat16), to_dev(w, torch.bfloat16), var, 1e-5)
    torch.cuda.synchronize()
    ry, rvar = O.rmsnorm_fwd(x, w, 1e-5)
    assert_f32_close(to_np(var), rvar, tol=1e-6, what="var")
    yy = to_np(y)
    # one RNE of x*r*w: at most one bf16 ulp away from the oracle's value
    ulp = np.abs(ry) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(yy - ry) <= ulp), np.max(np.abs(yy - ry) / ulp)
    assert np.mean(yy != ry) < 1e-3
    rdx = O.rmsnorm_bwd(dy, x, w, to_np(var), 1e-5)
    assert_f32_close(to_np(dx), rdx, tol=1e-5, what="dx")


# ------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("hd,pos0", [(128, 0), (64, 17), (40, 5)])   # 40: the element-wise kernel
def test_rope(dev, hd, pos0):
    import torch
    from glt_amd import ops
    B, T, nq, nk = 2, 96, 4, 2
    q = draw((B, T, nq, hd), 3, 3)
    k = draw((B, T, nk, hd), 4, 4)
    qd, kd = to_dev(q, torch.bfloat16), to_dev(k, torch.bfloat16)
    ops.apply_rope(qd, kd, 500000.0, pos0)
    torch.cuda.synchronize()
    for got, src in ((qd, q), (kd, k)):
        one = O.rope(src, 500000.0, pos0, exact_rounding=False)   # same single rounding
        ref = O.rope(src, 500000.0, pos0, exact_rounding=True)    # the reference's ATen roundings
        g = to_np(got)
        assert np.mean(g != one) < 2e-3
        assert_bf16_budget(g, ref, q=3, what="rope vs reference rounding")
        if pos0 == 0:
            np.testing.assert_array_equal(g[:, 0], src[:, 0])  # position 0 is the identity


# ------------------------------------------------------------------ AdamW
@pytest.mark.parametrize("clip", [0.0, 1.0])
def test_adamw(dev, clip):
    import torch
    from glt_amd import ops
    n = 100003
    w = draw((n,), 5, 5, 0, 0.02, bf16=False)
    g = draw((n,), 6, 6, 0, 0.01, bf16=False)
    m = draw((n,), 7, 7, 0, 1e-3, bf16=False)
    v = np.abs(draw((n,), 8, 8, 0, 1e-4, bf16=False))
    wd_, gd, md, vd = (to_dev(a, torch.float32) for a in (w, g, m, v))
    mir = torch.empty(n, dtype=torch.bfloat16, device=dev)
    ops.adamw_step(wd_, gd, md, vd, 3, 1e-4, clip_norm=clip, mirror=mir)
    torch.cuda.synchronize()
    rw, rm, rv = O.adamw(w, g, m, v, 3, 1e-4, 0.9, 0.999, 1e-8, 0.01, clip_norm=clip)
    assert_f32_close(to_np(wd_), rw, tol=1e-6, what="w")
    assert_f32_close(to_np(md), rm, tol=1e-5, what="m")
    assert_f32_close(to_np(vd), rv, tol=1e-5, what="v")
    np.testing.assert_array_equal(_bits(mir), O.f32_to_bf16_bits(to_np(wd_)))


@pytest.mark.parametrize("S,H", [(64, 96), (128, 192)])   # H % 64 != 0: separate passes; else the fused kernel
def test_adamw_graft_step_refreshes_packed_mirror(dev, S, H):
    import torch
    from glt_amd import ops
    ms = [torch.from_numpy(draw((S, H), 9, p, 0, 0.02, bf16=False)).cuda() for p in range(3)]
    sl = ops.GraftSlice(0, S, 0, H, *ms).pack()
    m = torch.zeros(3 * S * H, device=dev)
    v = torch.zeros(3 * S * H, device=dev)
    w = [to_np(t).copy() for t in ms]
    rm = [np.zeros((S, H), np.float32) for _ in range(3)]
    rv = [np.zeros((S, H), np.float32) for _ in range(3)]
    for step in range(2):
        grads = torch.from_numpy(draw((3 * S * H,), 10 + step, 1, 0, 0.01, bf16=False)).cuda()
        ops.adamw_graft_step([sl], [grads], [m], [v], step, 1e-4)
        torch.cuda.synchronize()
        gn = to_np(grads).reshape(3, S, H)
        for p in range(3):
            w[p], rm[p], rv[p] = O.adamw(w[p], gn[p], rm[p], rv[p], step, 1e-4, 0.9, 0.999, 1e-8, 0.01)
    rowmajor, shuf = packed_views(O.bf16_bits_to_f32(_bits(sl.packed)), S, H)
    mn, vn = to_np(m).reshape(3, S, H), to_np(v).reshape(3, S, H)
    for p in range(3):
        assert_f32_close(to_np(ms[p]), w[p], tol=1e-6)
        assert_f32_close(mn[p], rm[p], tol=1e-5, what="m")
        assert_f32_close(vn[p], rv[p], tol=1e-5, what="v")
        wb = O.bf16_round(to_np(ms[p]))
        np.testing.assert_array_equal(rowmajor[2 * p], wb)
        np.testing.assert_array_equal(rowmajor[2 * p + 1], wb.T)
        np.testing.assert_array_equal(shuf[2 * p], shuffle_b(wb))
        np.testing.assert_array_equal(shuf[2 * p + 1], shuffle_b(wb.T))


@pytest.mark.parametrize("clip", [1.0, 1e6])
def test_adamw_graft_step_global_clip(dev, clip):
    """The graft step's clip is one global L2 norm over every updated
    projection of every slice (the reference's clip over all of its deltas,
    grafting.hip:1149-1164): two slices (the fused mirror kernel and the
    separate-pass shape) against the oracle's clipped AdamW over the
    concatenated gradients; clip 1e6 leaves the update unclipped."""
    import torch
    from glt_amd import ops
    shapes = [(64, 128), (64, 96)]
    slices, grads, ms, vs, w0, gs = [], [], [], [], [], []
    for j, (S, H) in enumerate(shapes):
        masters = [torch.from_numpy(draw((S, H), 20 + j, p, 0, 0.02, bf16=False)).cuda() for p in range(3)]
        w0.append([to_np(t).copy() for t in masters])
        slices.append(ops.GraftSlice(0, S, 0, H, *masters).pack())
        g = draw((3 * S * H,), 30 + j, 1, 0, 0.05, bf16=False)   # global norm ~ 14, clipped at 1.0
        gs.append(g)
        grads.append(torch.from_numpy(g).cuda())
        ms.append(torch.zeros(3 * S * H, device=dev))
        vs.append(torch.zeros(3 * S * H, device=dev))
    ops.adamw_graft_step(slices, grads, ms, vs, 2, 1e-3, clip_norm=clip)
    torch.cuda.synchronize()
    allg = np.concatenate(gs)
    allw = np.concatenate([np.concatenate([a.ravel() for a in w]) for w in w0])
    z = np.zeros_like(allw)
    rw, rm, rv = O.adamw(allw, allg, z, z, 2, 1e-3, 0.9, 0.999, 1e-8, 0.01, clip_norm=clip)
    got_w = np.concatenate([np.concatenate([to_np(t).ravel() for t in (sl.gate, sl.up, sl.down)]) for sl in slices])
    assert_f32_close(got_w, rw, tol=1e-6, what="w")
    assert_f32_close(np.concatenate([to_np(t) for t in ms]), rm, tol=1e-5, what="m")
    assert_f32_close(np.concatenate([to_np(t) for t in vs]), rv, tol=1e-5, what="v")
    unclipped = O.adamw(allw, allg, z, z, 2, 1e-3, 0.9, 0.999, 1e-8, 0.01)[1]
    assert (np.abs(rm - unclipped).max() > 1e-3 * np.abs(unclipped).max()) == (clip == 1.0)
    for sl in slices:   # the mirrors follow the clipped masters
        rowmajor, _ = packed_views(O.bf16_bits_to_f32(_bits(sl.packed)), sl.s, sl.h)
        np.testing.assert_array_equal(rowmajor[0], O.bf16_round(to_np(sl.gate)))


@pytest.mark.parametrize("proj_mask", [7, 5])
def test_adamw_graft_step_clip_over_36_slices(dev, proj_mask):
    """One global clip over a whole model's graft: 36 slices (one per layer
    at the reference's 36 layers, grafting.hip:1149-1164 clips all L*3 deltas
    with one norm), more projections than one launch of the clip's partial
    sums or of the fused update takes, mixing the fused-mirror shape with
    the separate-pass one, against the oracle's clipped AdamW over the
    concatenated gradients of every updated projection. proj_mask 5 leaves
    the up projections out of the norm and untouched
    (src/kernels_optimizer_impl.inc:20-25)."""
    import torch
    from glt_amd import ops
    L = 36
    shapes = [(64, 96) if j % 5 == 4 else (64, 128) for j in range(L)]
    slices, grads, ms, vs, w0, gs = [], [], [], [], [], []
    for j, (S, H) in enumerate(shapes):
        masters = [torch.from_numpy(draw((S, H), 100 + j, p, 0, 0.02, bf16=False)).cuda() for p in range(3)]
        w0.append([to_np(t).copy() for t in masters])
        slices.append(ops.GraftSlice(0, S, 0, H, *masters).pack())
        g = draw((3 * S * H,), 200 + j, 1, 0, 0.01, bf16=False)
        gs.append(g.reshape(3, S * H))
        grads.append(torch.from_numpy(g).cuda())
        ms.append(torch.zeros(3 * S * H, device=dev))
        vs.append(torch.zeros(3 * S * H, device=dev))
    packed0 = [s.packed.clone() for s in slices]
    ops.adamw_graft_step(slices, grads, ms, vs, 1, 1e-3, proj_mask=proj_mask, clip_norm=1.0)
    torch.cuda.synchronize()
    upd = [p for p in range(3) if proj_mask & (1 << p)]
    allg = np.concatenate([gs[j][p] for j in range(L) for p in upd])
    allw = np.concatenate([w0[j][p].ravel() for j in range(L) for p in upd])
    z = np.zeros_like(allw)
    assert O.lib().orc_clip_scale(O._fp(allg), allg.size, 1.0) < 0.5   # the clip acts
    rw, rm, rv = O.adamw(allw, allg, z, z, 1, 1e-3, 0.9, 0.999, 1e-8, 0.01, clip_norm=1.0)
    cat = lambda per: np.concatenate([per(j, p) for j in range(L) for p in upd])
    got_w = cat(lambda j, p: to_np((slices[j].gate, slices[j].up, slices[j].down)[p]).ravel())
    sh = lambda j: shapes[j][0] * shapes[j][1]
    got_m = cat(lambda j, p: to_np(ms[j])[p * sh(j):(p + 1) * sh(j)])
    got_v = cat(lambda j, p: to_np(vs[j])[p * sh(j):(p + 1) * sh(j)])
    assert_f32_close(got_w, rw, tol=1e-6, what="w")
    assert_f32_close(got_m, rm, tol=1e-5, what="m")
    assert_f32_close(got_v, rv, tol=1e-5, what="v")
    for j, sl in enumerate(slices):
        rowmajor, shuf = packed_views(O.bf16_bits_to_f32(_bits(sl.packed)), sl.s, sl.h)
        rowmajor0, shuf0 = packed_views(O.bf16_bits_to_f32(_bits(packed0[j])), sl.s, sl.h)
        for p, t in enumerate((sl.gate, sl.up, sl.down)):
            if p in upd:
                wb = O.bf16_round(to_np(t))
                np.testing.assert_array_equal(rowmajor[2 * p], wb)
                np.testing.assert_array_equal(shuf[2 * p + 1], shuffle_b(wb.T))
            else:   # skipped projection: master, moments and mirror untouched
                np.testing.assert_array_equal(to_np(t), w0[j][p])
                assert not to_np(ms[j])[p * sh(j):(p + 1) * sh(j)].any()
                np.testing.assert_array_equal(rowmajor[2 * p], rowmajor0[2 * p])
                np.testing.assert_array_equal(shuf[2 * p], shuf0[2 * p])


def test_base_prepare_layout(dev):
    """The prepared base holds gate, up, down, down^T, gate^T, up^T in the
    fragment layout, bit for bit (ragged sizes pad with zeros)."""
    import ctypes
    import torch
    from glt_amd import _ffi as F
    from glt_amd import ops
    I, D = 96, 80
    wg = draw((I, D), 0, 1, 0, 0.02)
    wu = draw((I, D), 0, 2, 0, 0.02)
    wd = draw((D, I), 0, 3, 0, 0.02)
    base = ops.BaseMLP(*(to_dev(a, torch.bfloat16) for a in (wg, wu, wd)))
    torch.cuda.synchronize()
    got = O.bf16_bits_to_f32(_bits(base.prepared.view(torch.bfloat16)))
    off = 0
    for ref in (wg, wu, wd, wd.T, wg.T, wu.T):
        exp = shuffle_b(ref)
        np.testing.assert_array_equal(got[off:off + exp.size], exp)
        off += exp.size
    assert off * 2 == base.prepared.numel()


# -------------------------------------------------------------- elementwise
def test_silu_mul_and_gate_up_bwd(dev):
    import torch
    from glt_amd import ops
    n = 50001
    g = draw((n,), 11, 1, 0, 2.0)
    u = draw((n,), 11, 2, 0, 1.0)
    gi = draw((n,), 11, 3, 0, 1.0, bf16=False)
    out = ops.silu_mul(to_dev(g, torch.bfloat16), to_dev(u, torch.bfloat16))
    dg, du = ops.gate_up_bwd(to_dev(gi, torch.float32), to_dev(g, torch.bfloat16), to_dev(u, torch.bfloat16))
    torch.cuda.synchronize()
    ref = O.silu_mul(g, u)
    o = to_np(out)
    assert np.all(np.abs(o - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30)
    rdg, rdu = O.gate_up_bwd(gi, g, u)
    assert_f32_close(to_np(dg), rdg, tol=1e-5)
    assert_f32_close(to_np(du), rdu, tol=1e-5)


@pytest.mark.parametrize("rows,cols,dt", [(128, 192, "bf16"), (16384 // 8, 1024, "bf16"), (100, 72, "bf16"),
                                         (64, 64, "f32"), (33, 65, "f32")])
def test_transpose_exact(dev, rows, cols, dt):
    """glt_transpose: whole 64x64 bf16 tiles take the 16-byte path, other
    shapes and f32 the element path; either way a bit-exact transpose."""
    import torch
    from glt_amd import _ffi as F
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    x = torch.randn(rows, cols, device=dev).to(tdt)
    y = torch.full((cols, rows), 7.0, device=dev).to(tdt)
    F.call("glt_transpose", x.data_ptr(), y.data_ptr(), rows, cols, F.DTYPE_BF16 if dt == "bf16" else F.DTYPE_F32,
           None)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), x.cpu().t().contiguous())


@pytest.mark.parametrize("V,D", [(192, 128), (100, 96), (4096, 512)])
def test_lm_head_prepare_fragment_layout(dev, V, D):
    """glt_lm_head_prepare writes lm_head [V,D] and its transpose [D,V] in
    the MFMA fragment layout, bit for bit. Whole 64 x 64 tiles of the
    transpose go through the register-transpose path, ragged shapes through
    the LDS tile path."""
    import torch
    from glt_amd import _ffi as F
    lib = F.load()
    w = torch.from_numpy(draw((V, D), 21, V, 0, 1.0)).to(dev).to(torch.bfloat16)
    prep = torch.full((lib.glt_lm_head_prepared_size(V, D),), 0x55, dtype=torch.uint8, device=dev)
    F.call("glt_lm_head_prepare", w.data_ptr(), V, D, prep.data_ptr(), None)
    torch.cuda.synchronize()
    wf = w.float().cpu().numpy()
    n_fwd = (-(-V // 32) * 32) * (-(-D // 64) * 64)
    off = -(-(n_fwd * 2) // 256) * 256
    n_t = (-(-D // 32) * 32) * (-(-V // 64) * 64)
    got = prep.cpu().numpy()
    fwd = got[:n_fwd * 2].view(np.uint16)
    tr = got[off:off + n_t * 2].view(np.uint16)
    np.testing.assert_array_equal(fwd, O.f32_to_bf16_bits(shuffle_b(wf)))
    np.testing.assert_array_equal(tr, O.f32_to_bf16_bits(shuffle_b(wf.T)))


def test_f32_to_bf16_bitexact(dev):
    import torch
    from glt_amd import ops
    x = np.concatenate([draw((10007,), 12, 1, 0, 3.0, bf16=False),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -1e-40, 65504.0], np.float32)])
    b = ops.f32_to_bf16(to_dev(x, torch.float32))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(b), O.f32_to_bf16_bits(x))


def test_fill_normal_matches_host_generator(dev):
    import torch
    from glt_amd import ops, synth
    n = 1 << 16
    t = torch.empty(n, dtype=torch.float32, device=dev)
    ops.fill_normal(t, 100, 10, 0.0, 1.0)
    torch.cuda.synchronize()
    ref = synth.normal((n,), 100, 10)
    got = to_np(t)
    assert np.mean(got != ref) < 1e-4
    assert np.max(np.abs(got - ref)) < 1e-5


# ----------------------------------------------------------- graft GEMMs
def _golden():
    import json, os
    with open(os.path.join(os.path.dirname(__file__), "golden", "golden_vectors.json")) as f:
        return json.load(f)


def test_graft_gemm_contract_audit_golden(dev):
    """All six graft GEMM kinds on the S=3, H=2, M=2 vectors of the reference's
    docs/test_contract_audit.py:8-46 (expected outputs transcribed there)."""
    import torch
    from glt_amd import _ffi, ops
    G = _golden()["contract_audit"]
    S, H, M = G["S"], G["H"], G["M"]
    bf = lambda a: to_dev(np.array(a, np.float32), torch.bfloat16)
    f3 = lambda a: to_dev(np.array(a, np.float32), torch.float32)
    x_h, x_i = bf(G["x_h"]), bf(G["x_i"])
    dexp = f3(G["delta_exp"])
    dctr = f3(np.array(G["delta_ctr_math"], np.float32).T.copy())  # storage [S,H] = math [H,S]^T
    cases = [
        (_ffi.GEMM_EXPAND_FWD, (M, S), dict(a=x_h, lda=H, delta=dexp), "expand_fwd"),
        (_ffi.GEMM_EXPAND_WGRAD, (S, H), dict(a=x_h, lda=H, dy=f3(G["dy_s"])), "expand_wgrad"),
        (_ffi.GEMM_EXPAND_IGRAD, (M, H), dict(delta=dexp, dy=f3(G["dy_s"])), "expand_igrad"),
        (_ffi.GEMM_CONTRACT_FWD, (M, H), dict(a=x_i, lda=S, delta=dctr), "contract_fwd"),
        (_ffi.GEMM_CONTRACT_WGRAD, (S, H), dict(a=x_i, lda=S, dy=f3(G["dx_h"])), "contract_wgrad_storage"),
        (_ffi.GEMM_CONTRACT_IGRAD, (M, S), dict(delta=dctr, dy=f3(G["dx_h"])), "contract_igrad"),
    ]
    for kind, shape, kw, name in cases:
        out = torch.zeros(shape, dtype=torch.float32, device=dev)
        ops.graft_gemm(kind, M, S, H, out, **kw)
        torch.cuda.synchronize()
        np.testing.assert_allclose(to_np(out), np.array(G["expected"][name], np.float32), atol=1e-5, err_msg=name)


def test_graft_gemm_contract_probe_golden(dev):
    """Reference --contract-probe (src/graft_ops_impl.inc:158-212): sparse
    one-hot contract forward, expected out[0,11]=14, out[1,23]=65."""
    import torch
    from glt_amd import _ffi, ops
    G = _golden()["contract_probe"]
    M, S, H, ld = G["M"], G["S"], G["H"], G["input_stride"]
    a = np.zeros((M, ld), np.float32)
    for (r, c, v) in G["input"]:
        a[r, c] = v
    w = np.zeros((S, H), np.float32)
    for (r, c, v) in G["weight"]:
        w[r, c] = v
    out = torch.zeros((M, H), dtype=torch.float32, device=dev)
    ops.graft_gemm(_ffi.GEMM_CONTRACT_FWD, M, S, H, out, a=to_dev(a, torch.bfloat16), lda=ld,
                   delta=to_dev(w, torch.float32))
    torch.cuda.synchronize()
    o = to_np(out)
    exp = np.zeros((M, H), np.float32)
    for (r, c, v) in G["expected_nonzero"]:
        exp[r, c] = v
    np.testing.assert_array_equal(o, exp)


def test_down_orientation_and_checkpoint_golden(dev):
    """Reference tests/down_orientation_roundtrip.cpp:63-116,136-217 (strided
    input ld=6, storage [S,H] wgrad) and tests/test4_down_checkpoint_roundtrip.cpp:148."""
    import torch
    from glt_amd import _ffi, ops
    G = _golden()["down_orientation"]
    S, H, M, ld = G["S"], G["H"], G["M"], G["input_stride"]
    w = np.array(G["w_storage"], np.float32)
    x = np.zeros((M, ld), np.float32)
    x[:, :S] = np.array(G["x"], np.float32)
    out = torch.zeros((M, H), dtype=torch.float32, device=dev)
    ops.graft_gemm(_ffi.GEMM_CONTRACT_FWD, M, S, H, out, a=to_dev(x, torch.bfloat16), lda=ld,
                   delta=to_dev(w, torch.float32))
    g = torch.zeros((S, H), dtype=torch.float32, device=dev)
    ops.graft_gemm(_ffi.GEMM_CONTRACT_WGRAD, M, S, H, g, a=to_dev(np.array(G["x"], np.float32), torch.bfloat16), lda=S,
                   dy=to_dev(np.array(G["dy"], np.float32), torch.float32))
    torch.cuda.synchronize()
    np.testing.assert_allclose(to_np(out).ravel(), G["expected_forward"], atol=1e-4)
    np.testing.assert_allclose(to_np(g).ravel(), G["expected_wgrad_storage"], atol=1e-4)


@pytest.mark.parametrize("kind", range(6))
def test_graft_gemm_random_vs_oracle(dev, kind):
    import torch
    from glt_amd import ops
    M, S, H = 77, 45, 61
    lda = {0: H + 3, 1: S + 5, 2: H, 3: S + 2, 4: 0, 5: 0}[kind]
    arows = M
    a = draw((arows, max(lda, 1)), 13, kind)
    delta = draw((S, H), 14, kind, 0, 0.5, bf16=False)
    dys = {2: (M, S), 3: (M, H), 4: (M, S), 5: (M, H)}
    dy = draw(dys.get(kind, (1, 1)), 15, kind, bf16=False)
    outshape = {0: (M, S), 1: (M, H), 2: (S, H), 3: (S, H), 4: (M, H), 5: (M, S)}[kind]
    init = draw(outshape, 16, kind, bf16=False)
    out = to_dev(init, torch.float32)
    ops.graft_gemm(kind, M, S, H, out, a=to_dev(a, torch.bfloat16), lda=lda, delta=to_dev(delta, torch.float32),
                   dy=to_dev(dy, torch.float32), alpha=0.75, beta=0.5)
    torch.cuda.synchronize()
    ref = O.graft_gemm(kind, M, S, H, a=a, lda=lda, delta=delta, dy=dy, out=init.copy(), ldo=outshape[1],
                       alpha=0.75, beta=0.5)
    assert_f32_close(to_np(out), ref, tol=1e-5, what=f"kind {kind}")


# ------------------------------------------------------------ checkpoint
def test_grft_checkpoint_device_path(dev, tmp_path):
    """glt_grft_save / glt_grft_load on device memory: the same file as the
    host path writes, and the loaded storage equals the RNE bf16 values."""
    import torch
    from glt_amd import ops
    L_, S_, H_ = 3, 64, 96
    w = np.random.default_rng(9).normal(0, 0.02, L_ * 3 * S_ * H_).astype(np.float32)
    dpath, hpath = tmp_path / "dev.grft", tmp_path / "host.grft"
    ops.grft_save(dpath, torch.from_numpy(w).cuda(), L_, S_, H_, hidden_dim=96, domain_id=1, session_id="x")
    ops.grft_save(hpath, torch.from_numpy(w), L_, S_, H_, hidden_dim=96, domain_id=1, session_id="x")
    assert dpath.read_bytes() == hpath.read_bytes()
    out = torch.zeros(L_ * 3 * S_ * H_, device=dev)
    ops.grft_load(dpath, out, L_, S_, H_, domain_id=1, session_id="x")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), O.f32_to_bf16_bits(w).astype(np.uint32) << 16)


def test_safetensors_model_device_path(dev, tmp_path):
    """glt_st_load_layer / glt_st_load_head / glt_st_read into device memory:
    the same bits as the host path delivers (stored BF16, F32 and F16)."""
    import torch
    from safetensors.torch import save_file
    from glt_amd import ops
    D_, I_, hq, hkv, hd, V_ = 64, 96, 4, 2, 16, 80
    g = torch.Generator().manual_seed(4)
    p = "model.layers.0."
    t = {p + "input_layernorm.weight": torch.randn(D_, generator=g),
         p + "self_attn.q_proj.weight": torch.randn(hq * hd, D_, generator=g).to(torch.bfloat16),
         p + "self_attn.k_proj.weight": torch.randn(hkv * hd, D_, generator=g).to(torch.float16),
         p + "self_attn.v_proj.weight": torch.randn(hkv * hd, D_, generator=g).to(torch.bfloat16),
         p + "self_attn.o_proj.weight": torch.randn(D_, hq * hd, generator=g).to(torch.bfloat16),
         p + "post_attention_layernorm.weight": torch.randn(D_, generator=g).to(torch.bfloat16),
         p + "mlp.gate_proj.weight": torch.randn(I_, D_, generator=g).to(torch.bfloat16),
         p + "mlp.up_proj.weight": torch.randn(I_, D_, generator=g).to(torch.bfloat16),
         p + "mlp.down_proj.weight": torch.randn(D_, I_, generator=g).to(torch.bfloat16),
         "model.embed_tokens.weight": torch.randn(V_, D_, generator=g).to(torch.bfloat16),
         "model.norm.weight": torch.randn(D_, generator=g).to(torch.bfloat16),
         "lm_head.weight": torch.randn(D_, V_, generator=g).to(torch.bfloat16)}
    save_file(t, str(tmp_path / "m.safetensors"))
    with ops.SafetensorsModel(tmp_path / "m.safetensors") as m:
        wd = m.load_layer(0, D_, I_, hq, hkv, hd, device=dev)
        wh = m.load_layer(0, D_, I_, hq, hkv, hd, device="cpu")
        hd_ = m.load_head(V_, D_, device=dev)
        hh = m.load_head(V_, D_, device="cpu")
        td = m.read(p + "mlp.down_proj.weight", torch.float32, transpose=True, device=dev)
        torch.cuda.synchronize()
        for k in wd:
            assert torch.equal(wd[k].cpu().view(torch.int16), wh[k].view(torch.int16)), k
        for a, b in zip(hd_, hh):
            assert torch.equal(a.cpu(), b)
        assert torch.equal(td.cpu(), t[p + "mlp.down_proj.weight"].float().t())
