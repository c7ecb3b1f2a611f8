"""The workloads at the Llama-3-8B shape (hidden 4096, base intermediate
14336) at their full sizes, checked through per-token oracle samples and
size-independent properties:

* Four stacked 512-neuron slices (seeds 1..4) appended after the base
  (N = 16384), 4 x 4096 tokens, forward only: explicit stacked grafts
  against the same forward over shadow-baked merged weights on every token,
  and against the oracle on one token of every 256-token tile.
* shadow_bake materialising [15360,4096] / [4096,15360] baked matrices for
  several layers, then the sentinel forward (X ~N(0,1) [2048,4096]) baked
  against stacked, per layer.
* The measured MLP step (16384 tokens) and the decoder layer with recompute
  (2 x 4096 tokens, 32/8 heads).
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
    M, S = 16384, 512
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
    # oracle on one token of each of the 64 M-tiles (a different row of the tile each time)
    rows = torch.tensor([256 * t + (37 * t) % 256 for t in range(M // 256)], device="cuda")
    h = lambda t: to_np(t)
    sl_np = [{"i0": s.i_start, "s": s.s, "h0": s.h_start, "h": s.h, "gate": h(s.gate), "up": h(s.up),
              "down": h(s.down)} for s in slices]
    rg, ru, ri, ry = O.mlp_fwd(h(x[rows]), h(wg), h(wu), h(wd), N, sl_np, bf16=True)
    for name, a, r, q in (("gate_pre", g, rg, 2), ("up_pre", u, ru, 2), ("inter", inter, ri, 3), ("y", y, ry, 4)):
        assert_bf16_budget(to_np(a[rows]), r, q=q, what=f"stacked vs oracle {name}")


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
            assert abs(got - terms.sum()) <= 1e-3 * np.abs(terms).sum() + 1e-6, ("dW_gate", s, hh, got, terms.sum())
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

    # the backward with the FFN norm's backward beside the weight-gradient
    # GEMM (192 tiles: the norm runs on the other CUs), as bench.py's step
    # runs it: bit for bit the two separate calls
    del parts
    gamma = ops.fill_normal(torch.empty(D, dtype=torch.bfloat16, device="cuda"), 300, 12, 1.0, 0.02)
    xn, var = ops.rms_norm(x, gamma, 1e-5)
    dx2, g2 = ops.mlp_backward(base, slices, xn, dy, N, g, u, inter)
    nd2 = ops.rms_norm_bwd(dx2, x, gamma, var, 1e-5)
    dx3, g3, nd3 = ops.mlp_backward(base, slices, xn, dy, N, g, u, inter, norm=(x, gamma, var, 1e-5))
    torch.cuda.synchronize()
    assert torch.equal(dx2, dx3) and torch.equal(nd2, nd3)
    for a, b in zip(g2[0], g3[0]):
        assert torch.equal(a, b)


def test_config5_decoder_layer_full_size(dev):
    """The decoder layer at its workload (2 x 4096 tokens, hidden 4096, 32
    query / 8 kv heads of 128, RoPE theta 500000, causal; base intermediate
    14336 plus an appended 1024-neuron slice), forward then the graft-only
    backward with recompute on an f32 upstream gradient:
    * forward: the layer output and the MLP input on 8 tokens (both
      sequences, several query blocks, the last token) against the oracle's
      composition of the reference's forward_layer (k/v of every token from
      f64 products, attention over each sampled query's causal prefix);
    * backward: per-token dX on those tokens against the oracle's
      recompute (the reference's rounding) and backward; sampled dW entries
      against f64 sums over all 8192 tokens; the two sequences' backwards
      give the same per-token dX bit for bit and gradients that sum to the
      whole batch's."""
    import torch
    from glt_amd import ops
    bf = torch.bfloat16
    B, T, Hq, Hkv, hd, S = 2, 4096, 32, 8, 128, 1024
    M, N, theta, eps = B * T, I + S, 500000.0, 1e-5
    fill = lambda shape, seed, tid, mean, std, dt=bf: ops.fill_normal(torch.empty(shape, dtype=dt, device="cuda"),
                                                                       seed, tid, mean, std)
    x = fill((M, D), 100, 10, 0.0, 1.0)
    wq, wk, wv = fill((Hq * hd, D), 0, 30, 0.0, 0.02), fill((Hkv * hd, D), 0, 31, 0.0, 0.02), \
        fill((Hkv * hd, D), 0, 32, 0.0, 0.02)
    wo = fill((D, Hq * hd), 0, 33, 0.0, 0.02)
    ln_in, ln_post = fill((D,), 300, 12, 1.0, 0.02), fill((D,), 300, 13, 1.0, 0.02)
    wg, wu, wd = _base(torch, ops)
    slices = _slices(torch, ops, [(I, S, 0, D)], seeds=(1,))
    base = ops.BaseMLP(wg, wu, wd)
    layer = ops.DecoderLayer(B, T, Hq, Hkv, wq, wk, wv, wo, ln_in, ln_post, base, slices, N, rope_theta=theta,
                             rms_eps=eps)
    x_in = x.clone()
    out, x_ffn, _ = layer.forward(x)
    dy = fill((M, D), 200, 11, 0.0, 1.0, torch.float32)
    dx, grads = ops.mlp_backward(base, slices, x_ffn, dy, N, recompute=True)
    torch.cuda.synchronize()
    print("config-5 layer forward + backward done", flush=True)

    h = lambda t: to_np(t)
    rb = O.bf16_round
    bi = np.array([0, 0, 0, 0, 1, 1, 1, 1])
    ti = np.array([0, 127, 128, 2049, 1, 1000, 3968, 4095])
    idx = bi * T + ti
    rows = torch.tensor(idx, device="cuda")
    xn, _ = O.rmsnorm_fwd(h(x_in), h(ln_in), eps)
    f64 = lambda a: np.asarray(a, np.float64)
    kv = [O.rope(rb((f64(xn) @ f64(h(w)).T).astype(np.float32)).reshape(B, T, Hkv, hd), theta, 0,
                 exact_rounding=False) if j == 0 else rb((f64(xn) @ f64(h(w)).T).astype(np.float32)).reshape(B, T, Hkv, hd)
          for j, w in enumerate((wk, wv))]
    q = rb((f64(xn[idx]) @ f64(h(wq)).T).astype(np.float32)).reshape(-1, Hq, hd)
    q = np.stack([O.rope(q[i][None, None], theta, int(ti[i]), exact_rounding=False)[0, 0] for i in range(len(idx))])
    a = rb(O.attention_rows(q, kv[0], kv[1], bi, ti).astype(np.float32)).reshape(len(idx), Hq * hd)
    x1 = rb(h(x_in[rows]) + rb((f64(a) @ f64(h(wo)).T).astype(np.float32)))
    ref_ffn, _ = O.rmsnorm_fwd(x1, h(ln_post), eps)
    sl = slices[0]
    sl_np = [{"i0": sl.i_start, "s": sl.s, "h0": sl.h_start, "h": sl.h, "gate": h(sl.gate), "up": h(sl.up),
              "down": h(sl.down)}]
    wg_np, wu_np, wd_np = h(wg), h(wu), h(wd)
    _, _, _, y = O.mlp_fwd(ref_ffn, wg_np, wu_np, wd_np, N, sl_np, bf16=True)
    assert_bf16_budget(h(x_ffn[rows]), ref_ffn, q=4, what="config-5 MLP input")
    assert_bf16_budget(h(out[rows]), rb(x1 + y), q=4, what="config-5 layer output")
    del xn, kv

    # backward on the sampled tokens, from the layer's own MLP input
    xs = h(x_ffn[rows])
    rg, ru, ri = O.mlp_recompute(xs, wg_np, wu_np, N, sl_np)
    rdx, _ = O.mlp_bwd(xs, wg_np, wu_np, wd_np, N, sl_np, rg, ru, ri, h(dy[rows]), bf16=True)
    assert_bf16_budget(h(dx[rows]), rdx, q=4, what="config-5 dX")
    del wg_np, wu_np, wd_np

    # sampled gradient entries over all tokens: the slice's activations (the
    # forward's equal the recompute's for an appended slice) in f64
    _, g, u, inter = ops.mlp_forward(base, slices, x_ffn, N)
    torch.cuda.synchronize()
    dyb = rb(h(dy)).astype(np.float64)                                # the graft GEMMs read bf16(dy)
    xf = h(x_ffn).astype(np.float64)
    dd = rb(h(sl.down)).astype(np.float64)
    for s_ in (0, 700, 1023):
        col = I + s_
        it, gt, ut = (h(t[:, col]).astype(np.float64) for t in (inter, g, u))
        di = (dyb @ dd[s_]).astype(np.float32)
        sg = 1.0 / (1.0 + np.exp(-gt))
        dgc = rb((di * ut * (sg * (1.0 + gt * (1.0 - sg)))).astype(np.float32)).astype(np.float64)
        for hh in (0, 1234, 4095):
            terms = it * dyb[:, hh]
            got = float(grads[0][2][s_, hh])
            assert abs(got - terms.sum()) <= 1e-4 * np.abs(terms).sum() + 1e-6, ("dW_down", s_, hh, got)
            terms = dgc * xf[:, hh]
            got = float(grads[0][0][s_, hh])
            assert abs(got - terms.sum()) <= 1e-3 * np.abs(terms).sum() + 1e-6, ("dW_gate", s_, hh, got)
    del dyb, xf, g, u, inter

    # the two sequences separately
    parts = []
    for b in range(B):
        xb = x_ffn[b * T:(b + 1) * T].contiguous()
        dxb, grb = ops.mlp_backward(base, slices, xb, dy[b * T:(b + 1) * T].contiguous(), N, recompute=True)
        torch.cuda.synchronize()
        assert torch.equal(dxb.view(torch.int32), dx[b * T:(b + 1) * T].view(torch.int32))
        parts.append(grb)
    for p in range(3):
        full = grads[0][p].double()
        summed = parts[0][0][p].double() + parts[1][0][p].double()
        assert (summed - full).abs().max().item() <= 1e-5 * full.abs().max().item(), p


def test_config2_adamw_clip_full_size(dev):
    """The measured step's optimizer leg at its size: one appended slice of
    S 1024 x H 4096 (3 x 4,194,304 = 12,582,912 gradients, so the clip's
    partial sums run with a 25,600-element chunk over 492 workgroups, every
    16-byte load of their unrolled loops live, and the update sums 492
    partials) with the reference's clip 1.0 (grafting.hip:1149-1172,
    src/kernels_optimizer_impl.inc:11-77), over steps 0 and 1. The workspace
    form is checked against the oracle's clipped AdamW over the concatenated
    gradients, the allocation-free form against it bit for bit, and every
    orientation of the packed mirror against the new masters bit for bit."""
    import torch
    from glt_amd import _ffi as F
    from glt_amd import ops
    from helpers import assert_f32_close, packed_views, shuffle_b
    S, H = 1024, D
    n = 3 * S * H
    a = _slices(torch, ops, [(I, S, 0, H)], seeds=(1,))
    b = [ops.GraftSlice(s.i_start, s.s, s.h_start, s.h, s.gate.clone(), s.up.clone(), s.down.clone()) for s in a]
    for sa, sb in zip(a, b):
        sb.packed.copy_(sa.packed)
    ma, va = torch.zeros(n, device=dev), torch.zeros(n, device=dev)
    mb, vb = torch.zeros(n, device=dev), torch.zeros(n, device=dev)
    w = np.concatenate([to_np(t).ravel() for t in (a[0].gate, a[0].up, a[0].down)])
    rm = np.zeros(n, np.float32)
    rv = np.zeros(n, np.float32)
    ws_bytes = F.load().glt_adamw_workspace_size(0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    lr, clip = 1e-4, 1.0
    for step in (0, 1):
        print("config-2 AdamW step", step, flush=True)
        g = ops.fill_normal(torch.empty(n, dtype=torch.float32, device=dev), 400 + step, 1, 0.0, 0.01)
        ops.adamw_graft_step(a, [g], [ma], [va], step, lr, clip_norm=clip, workspace=ws)
        F.call("glt_adamw_graft_step_noalloc", ops._slices_array(b), 1, F.ptr_array([g.data_ptr()]),
               F.ptr_array([mb.data_ptr()]), F.ptr_array([vb.data_ptr()]), F.ptr_array([b[0].packed.data_ptr()]),
               7, step, lr, 0.9, 0.999, 1e-8, 0.01, clip, ops._stream())
        torch.cuda.synchronize()
        gn = to_np(g)
        assert O.lib().orc_clip_scale(O._fp(gn), n, clip) < 0.05     # norm ~ 35: the clip acts
        w, rm, rv = O.adamw(w, gn, rm, rv, step, lr, 0.9, 0.999, 1e-8, 0.01, clip_norm=clip)
        got = np.concatenate([to_np(t).ravel() for t in (a[0].gate, a[0].up, a[0].down)])
        assert_f32_close(got, w, tol=1e-6, what=f"w step {step}")
        assert_f32_close(to_np(ma), rm, tol=1e-5, what=f"m step {step}")
        assert_f32_close(to_np(va), rv, tol=1e-5, what=f"v step {step}")
        i32 = lambda t: t.view(torch.int32)
        for x, y in ((a[0].gate, b[0].gate), (a[0].up, b[0].up), (a[0].down, b[0].down), (ma, mb), (va, vb)):
            assert torch.equal(i32(x), i32(y))
        assert torch.equal(a[0].packed.view(torch.int16), b[0].packed.view(torch.int16))
        bits = a[0].packed.view(torch.int16).cpu().numpy().view(np.uint16)
        rowmajor, shuf = packed_views(O.bf16_bits_to_f32(bits), S, H)
        for p, t in enumerate((a[0].gate, a[0].up, a[0].down)):
            wb = O.bf16_round(to_np(t))
            np.testing.assert_array_equal(rowmajor[2 * p], wb)
            np.testing.assert_array_equal(rowmajor[2 * p + 1], wb.T)
            np.testing.assert_array_equal(shuf[2 * p], shuffle_b(wb))
            np.testing.assert_array_equal(shuf[2 * p + 1], shuffle_b(wb.T))
        del g, bits, rowmajor, shuf
