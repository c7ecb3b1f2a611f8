"""Pins the CPU oracle (oracle/glt_oracle.c) before it is trusted as the
checker: golden vectors from the reference's tests, closed forms, library
routines (torch CPU, numpy) and brute force on tiny inputs. CPU only."""
import json
import os

import numpy as np
import pytest
import torch

from helpers import draw
from oracle import oracle as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden_vectors.json")))


# ------------------------------------------------------------------ bf16
def test_bf16_rne_known_answers():
    # ties go to even: 1+2^-8 -> 1.0, 1+3*2^-8 -> 1+2^-6; halfway negative likewise
    x = np.array([1.0, 1.00390625, 1.01171875, -1.00390625, 0.0, -0.0, 3.0e38, 1e-40], np.float32)
    b = O.f32_to_bf16_bits(x)
    assert list(b[:6]) == [0x3F80, 0x3F80, 0x3F82, 0xBF80, 0x0000, 0x8000]
    # 3e38 = 0x7F61B1E6: lower half 0xB1E6 > 0x8000, so it rounds up to 0x7F62
    assert b[6] == 0x7F62
    assert b[7] == 0x0001  # 1e-40 (subnormal 0x000116C2) -> 0x0001


def test_bf16_rne_matches_torch():
    x = np.concatenate([draw((100000,), 1, 1, 0, 3.0, bf16=False), draw((1000,), 1, 2, 0, 1e-30, bf16=False)])
    ours = O.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, ref)


# ------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("form", ["nt", "tn", "nn"])
def test_gemm_vs_numpy(form):
    rng = np.random.default_rng(0)
    M, N, K = 13, 17, 29
    A = rng.normal(size=(M, K)).astype(np.float32)
    B = rng.normal(size=(N, K)).astype(np.float32)
    if form == "nt":
        C = O.gemm_strided(M, N, K, A, K, 1, B, K, 1)
    elif form == "tn":
        At = A.T.copy()
        C = O.gemm_strided(M, N, K, At, 1, M, B, K, 1)
    else:
        Bt = B.T.copy()
        C = O.gemm_strided(M, N, K, A, K, 1, Bt, 1, N)
    np.testing.assert_allclose(C, A.astype(np.float64) @ B.T.astype(np.float64), rtol=1e-6, atol=1e-6)


def test_graft_ops_contract_audit_golden():
    G = GOLDEN["contract_audit"]
    S, H, M = G["S"], G["H"], G["M"]
    x_h, x_i = np.array(G["x_h"], np.float32), np.array(G["x_i"], np.float32)
    dexp = np.array(G["delta_exp"], np.float32)
    dctr = np.array(G["delta_ctr_math"], np.float32).T.copy()
    dy_s, dx_h = np.array(G["dy_s"], np.float32), np.array(G["dx_h"], np.float32)
    E = G["expected"]
    got = {
        "expand_fwd": O.graft_gemm(0, M, S, H, a=x_h, lda=H, delta=dexp),
        "contract_fwd": O.graft_gemm(1, M, S, H, a=x_i, lda=S, delta=dctr),
        "expand_wgrad": O.graft_gemm(2, M, S, H, a=x_h, lda=H, dy=dy_s),
        "contract_wgrad_storage": O.graft_gemm(3, M, S, H, a=x_i, lda=S, dy=dx_h),
        "expand_igrad": O.graft_gemm(4, M, S, H, delta=dexp, dy=dy_s),
        "contract_igrad": O.graft_gemm(5, M, S, H, delta=dctr, dy=dx_h),
    }
    for k, v in got.items():
        np.testing.assert_allclose(v, np.array(E[k], np.float32), atol=1e-6, err_msg=k)
    # the storage-canonical contract wgrad is the transpose of its math view
    np.testing.assert_allclose(got["contract_wgrad_storage"].T, np.array(E["contract_wgrad_math"]), atol=1e-6)


def test_contract_probe_golden():
    G = GOLDEN["contract_probe"]
    a = np.zeros((G["M"], G["input_stride"]), np.float32)
    for r, c, v in G["input"]:
        a[r, c] = v
    w = np.zeros((G["S"], G["H"]), np.float32)
    for r, c, v in G["weight"]:
        w[r, c] = v
    out = O.graft_gemm(1, G["M"], G["S"], G["H"], a=a, lda=G["input_stride"], delta=w)
    exp = np.zeros_like(out)
    for r, c, v in G["expected_nonzero"]:
        exp[r, c] = v
    np.testing.assert_array_equal(out, exp)


def test_down_orientation_golden():
    G = GOLDEN["down_orientation"]
    x = np.zeros((G["M"], G["input_stride"]), np.float32)
    x[:, :G["S"]] = G["x"]
    out = O.graft_gemm(1, G["M"], G["S"], G["H"], a=x, lda=G["input_stride"], delta=np.array(G["w_storage"]))
    np.testing.assert_allclose(out.ravel(), G["expected_forward"])
    g = O.graft_gemm(3, G["M"], G["S"], G["H"], a=np.array(G["x"], np.float32), lda=G["S"], dy=np.array(G["dy"]))
    np.testing.assert_allclose(g.ravel(), G["expected_wgrad_storage"])
    # checkpoint roundtrip: f32 -> bf16 -> f32 keeps these values exactly
    w = np.array(G["w_storage"], np.float32)
    np.testing.assert_array_equal(O.bf16_round(w), w)


# ------------------------------------------------------------------ bake
def test_bake_sentinel_and_orientation():
    S, H = 3, 513
    val = lambda l, p, s, h: float((l * 100 + p * 10 + s) * 1000 + h + 1)
    for p, mode in ((0, 0), (2, 1)):
        g = np.array([[val(1, p, s, h) for h in range(H)] for s in range(S)], np.float32)
        base = np.zeros((S, H) if mode == 0 else (H, S), np.uint16)
        O.bake_inplace(base, g, 0, 0, mode)
        f = O.bf16_bits_to_f32(base)
        exp = g if mode == 0 else g.T
        assert np.all(np.abs(f - exp) <= 0.5 + 0.005 * np.abs(exp))
        np.testing.assert_array_equal(base, O.f32_to_bf16_bits(exp))


def test_bake_single_rounding_vs_torch():
    rng = np.random.default_rng(3)
    base = O.bf16_round(rng.normal(0, 0.02, (40, 50)).astype(np.float32))
    g = rng.normal(0, 0.02, (7, 9)).astype(np.float32)
    bits = O.f32_to_bf16_bits(base)
    O.bake_inplace(bits, g, 5, 11, 0)
    ref = torch.from_numpy(base.copy())
    ref[5:12, 11:20] += torch.from_numpy(g)
    np.testing.assert_array_equal(O.bf16_bits_to_f32(bits), ref.to(torch.bfloat16).float().numpy())


# --------------------------------------------------------------- RMSNorm
def test_rmsnorm_vs_torch():
    x = draw((9, 130), 2, 1)
    w = O.bf16_round(1 + draw((130,), 2, 2, 0, 0.02, bf16=False))
    y, var = O.rmsnorm_fwd(x, w, 1e-5)
    xt = torch.from_numpy(x).double()
    rvar = (xt ** 2).mean(-1)
    np.testing.assert_allclose(var, rvar.numpy(), rtol=1e-6)
    r = torch.rsqrt(rvar + 1e-5).float()
    ref = (torch.from_numpy(x) * r[:, None] * torch.from_numpy(w)).to(torch.bfloat16).float().numpy()
    assert np.mean(y != ref) < 0.01 and np.max(np.abs(y - ref)) <= 2.0 ** -7 * np.max(np.abs(ref))
    # backward vs autograd (f64) of the same normalisation
    dy = draw((9, 130), 2, 3, bf16=False)
    xr = torch.from_numpy(x).double().requires_grad_()
    yy = xr * torch.rsqrt((xr ** 2).mean(-1, keepdim=True) + 1e-5) * torch.from_numpy(w).double()
    yy.backward(torch.from_numpy(dy).double())
    dx = O.rmsnorm_bwd(dy, x, w, var, 1e-5)
    np.testing.assert_allclose(dx, xr.grad.numpy(), rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------ RoPE
def _torch_reference_rope(t, theta):
    """The reference's ATen sequence (src/rope_impl.inc:8-39) in torch CPU bf16."""
    B, T, nh, hd = t.shape
    i = torch.arange(0, hd, 2, dtype=torch.float32)
    inv = 1.0 / torch.pow(theta, i / hd)
    ang = torch.arange(T, dtype=torch.float32)[:, None] * inv[None]
    emb = torch.cat([ang, ang], -1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    x = torch.from_numpy(t).to(torch.bfloat16)
    half = hd // 2
    x1, x2 = x[..., :half], x[..., half:]
    cs, sn = cos[None, :, None], sin[None, :, None]
    r1 = x1 * cs[..., :half] - x2 * sn[..., :half]
    r2 = x2 * cs[..., half:] + x1 * sn[..., half:]
    return torch.cat([r1, r2], -1).float().numpy()


def test_rope_matches_aten_sequence_and_invariants():
    t = draw((2, 33, 3, 64), 4, 1)
    got = O.rope(t, 500000.0, 0, exact_rounding=True)
    ref = _torch_reference_rope(t, 500000.0)
    assert np.mean(got != ref) < 1e-3  # torch f32 cos/sin vs libm may differ in rare last bits
    np.testing.assert_array_equal(got[:, 0], t[:, 0])  # position 0 is the identity
    one = O.rope(t, 500000.0, 0, exact_rounding=False)
    n0 = np.linalg.norm(t.reshape(-1, 64), axis=1)
    n1 = np.linalg.norm(one.reshape(-1, 64), axis=1)
    assert np.max(np.abs(n1 - n0) / n0) < 2e-2  # rotation preserves the norm up to bf16 c/s
    # pos_offset shifts positions
    a = O.rope(t[:, 5:], 500000.0, 5, exact_rounding=True)
    np.testing.assert_array_equal(a, got[:, 5:])


# ------------------------------------------------------------ attention
def test_attention_closed_forms():
    """Pins what a plausible mistake would change: the causal mask direction
    (key <= query), the GQA head map (repeat_interleave: query head h uses kv
    head h // rep, not h % Hkv), the scale, and T = 1."""
    B, T, Hq, Hkv, hd = 2, 7, 4, 2, 8
    rng = np.random.default_rng(3)
    v = rng.normal(size=(B, T, Hkv, hd))
    k = rng.normal(size=(B, T, Hkv, hd))
    # q = 0: uniform weights over the allowed keys -> causal prefix mean of v
    out = O.attention(np.zeros((B, T, Hq, hd)), k, v, causal=True)
    for h in range(Hq):
        g = h // (Hq // Hkv)
        prefix = np.cumsum(v[:, :, g], axis=1) / np.arange(1, T + 1)[None, :, None]
        np.testing.assert_allclose(out[:, :, h], prefix, rtol=1e-12, atol=1e-12)
    # non-causal: the full mean for every query
    full = O.attention(np.zeros((B, T, Hq, hd)), k, v, causal=False)
    np.testing.assert_allclose(full[:, :, 1], np.broadcast_to(v[:, :, 0].mean(axis=1, keepdims=True), (B, T, hd)),
                               rtol=1e-12, atol=1e-12)
    # a query aligned with one earlier key at a large scale picks that key's value
    kk = np.zeros((1, 4, 1, 4))
    kk[0, :, 0, :] = np.eye(4)
    vv = np.arange(16, dtype=np.float64).reshape(1, 4, 1, 4)
    qq = np.zeros((1, 4, 1, 4))
    qq[0, 3, 0, 1] = 1.0  # query 3 matches key 1
    sharp = O.attention(qq, kk, vv, causal=True, scale=200.0)
    np.testing.assert_allclose(sharp[0, 3, 0], vv[0, 1, 0], atol=1e-9)
    # T = 1: the output is v whatever q is
    one = O.attention(rng.normal(size=(1, 1, 2, 8)), rng.normal(size=(1, 1, 1, 8)), v[:1, :1, :1], causal=True)
    np.testing.assert_allclose(one[0, 0, 1], v[0, 0, 0], rtol=1e-12)


def test_attention_matches_torch_sdpa():
    """torch's CPU scaled_dot_product_attention (a library routine, float64)
    on repeat_interleave'd k/v, as the reference calls it."""
    import torch
    B, T, Hq, Hkv, hd = 2, 19, 6, 2, 16
    rng = np.random.default_rng(5)
    q, k, v = (rng.normal(size=(B, T, H, hd)) for H in (Hq, Hkv, Hkv))
    for causal in (True, False):
        got = O.attention(q, k, v, causal=causal)
        tq, tk, tv = (torch.from_numpy(a).transpose(1, 2) for a in (q, k, v))
        tk = tk.repeat_interleave(Hq // Hkv, 1)
        tv = tv.repeat_interleave(Hq // Hkv, 1)
        ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal).transpose(1, 2).numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


# ----------------------------------------------------------------- AdamW
def test_adamw_closed_form_step0_and_torch():
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, 1000).astype(np.float32)
    g = rng.normal(0, 0.01, 1000).astype(np.float32)
    z = np.zeros_like(w)
    nw, m, v = O.adamw(w, g, z, z, 0, 1e-3, 0.9, 0.999, 1e-8, 0.01)
    # step 0: m_hat = g, v_hat = g^2
    exp = w - 1e-3 * g / (np.abs(g) + 1e-8) - 1e-3 * 0.01 * w
    np.testing.assert_allclose(nw, exp, rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(m, 0.1 * g, rtol=1e-6)
    # three steps against torch.optim.AdamW
    p = torch.nn.Parameter(torch.from_numpy(w.copy()))
    opt = torch.optim.AdamW([p], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    ww, mm, vv = w.copy(), z.copy(), z.copy()
    for step in range(3):
        gs = rng.normal(0, 0.01, 1000).astype(np.float32)
        p.grad = torch.from_numpy(gs.copy())
        opt.step()
        ww, mm, vv = O.adamw(ww, gs, mm, vv, step, 1e-3, 0.9, 0.999, 1e-8, 0.01)
    np.testing.assert_allclose(ww, p.detach().numpy(), rtol=1e-5, atol=1e-8)


def test_clip_scale():
    g = np.full(100, 0.5, np.float32)  # norm 5
    nw, m, _ = O.adamw(np.zeros(100, np.float32), g, np.zeros(100, np.float32), np.zeros(100, np.float32), 0, 1.0,
                       0.9, 0.999, 1e-8, 0.0, clip_norm=1.0)
    np.testing.assert_allclose(m, 0.1 * g * (1.0 / np.sqrt(25 + 1e-8)), rtol=1e-6)


# ----------------------------------------------------------- elementwise
def test_silu_and_derivative_finite_difference():
    g = np.linspace(-6, 6, 1001).astype(np.float32)
    u = np.linspace(2, -1, 1001).astype(np.float32)
    gi = np.ones_like(g)
    dg, du = O.gate_up_bwd(gi, g, u)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    f = lambda a, b: a / (1 + np.exp(-a)) * b
    h = 1e-5
    np.testing.assert_allclose(dg, (f(gd + h, ud) - f(gd - h, ud)) / (2 * h), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(du, gd / (1 + np.exp(-gd)), rtol=1e-5, atol=1e-6)
    s = O.silu_mul(g, u, round_out=False)
    np.testing.assert_allclose(s, f(gd, ud), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------- MLP layer
def _torch_mlp(x, wg, wu, wd, N, slices):
    """Independent restatement: materialise W_eff = zero-extended base +
    scattered deltas, run the f64 SwiGLU MLP under autograd."""
    I, D = wg.shape
    xt = torch.from_numpy(x).double().requires_grad_()
    deltas = []
    Wg = torch.zeros(N, D, dtype=torch.float64)
    Wu = torch.zeros(N, D, dtype=torch.float64)
    Wd = torch.zeros(D, N, dtype=torch.float64)
    Wg[:I], Wu[:I], Wd[:, :I] = (torch.from_numpy(a).double() for a in (wg, wu, wd))
    for s in slices:
        i0, S, h0, H = s["i0"], s["s"], s["h0"], s["h"]
        dg, du, dd = (torch.from_numpy(s[p]).double().requires_grad_() for p in ("gate", "up", "down"))
        deltas.append((dg, du, dd))
        pad = lambda d, r0, c0, shape: torch.nn.functional.pad(d, (c0, shape[1] - c0 - d.shape[1], r0, shape[0] - r0 - d.shape[0]))
        Wg = Wg + pad(dg, i0, h0, (N, D))
        Wu = Wu + pad(du, i0, h0, (N, D))
        Wd = Wd + pad(dd.T, h0, i0, (D, N))
    g = xt @ Wg.T
    u = xt @ Wu.T
    inter = torch.nn.functional.silu(g) * u
    y = inter @ Wd.T
    return xt, deltas, g, u, inter, y


@pytest.mark.parametrize("pl", [[(0, 3, 0, 2), (3, 3, 2, 2)], [(20, 8, 0, 12)], [(2, 5, 3, 6), (20, 8, 0, 12)]])
def test_mlp_f32_vs_autograd(pl):
    D, I, N, M = 12, 20, 28, 7
    rng = np.random.default_rng(11)
    x = rng.normal(size=(M, D)).astype(np.float32)
    wg, wu = rng.normal(0, 0.3, (I, D)).astype(np.float32), rng.normal(0, 0.3, (I, D)).astype(np.float32)
    wd = rng.normal(0, 0.3, (D, I)).astype(np.float32)
    slices = [{"i0": a, "s": b, "h0": c, "h": d, **{p: rng.normal(0, 0.3, (b, d)).astype(np.float32)
                                                   for p in ("gate", "up", "down")}} for a, b, c, d in pl]
    g, u, inter, y = O.mlp_fwd(x, wg, wu, wd, N, slices, bf16=False)
    xt, deltas, tg, tu, ti, ty = _torch_mlp(x, wg, wu, wd, N, slices)
    np.testing.assert_allclose(g, tg.detach().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(inter, ti.detach().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(y, ty.detach().numpy(), rtol=1e-5, atol=1e-6)
    dy = rng.normal(size=(M, D)).astype(np.float32)
    ty.backward(torch.from_numpy(dy).double())
    dx, grads = O.mlp_bwd(x, wg, wu, wd, N, slices, g, u, inter, dy, bf16=False)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-4, atol=1e-5)
    for j, (dg, du, dd) in enumerate(deltas):
        for p, t in enumerate((dg, du, dd)):
            np.testing.assert_allclose(grads[j][p], t.grad.numpy(), rtol=1e-4, atol=1e-5, err_msg=f"{j},{p}")


def test_mlp_bf16_rounding_points():
    """bf16 path: gate_pre/up/inter/y are bf16 values; base-only columns equal
    bf16 of the f32 GEMM; appended columns equal bf16(x . bf16(delta)^T)."""
    D, I, N, M = 16, 24, 32, 5
    rng = np.random.default_rng(12)
    x = O.bf16_round(rng.normal(size=(M, D)).astype(np.float32))
    wg, wu = (O.bf16_round(rng.normal(0, 0.2, (I, D)).astype(np.float32)) for _ in range(2))
    wd = O.bf16_round(rng.normal(0, 0.2, (D, I)).astype(np.float32))
    sl = [{"i0": 24, "s": 8, "h0": 0, "h": 16, **{p: rng.normal(0, 0.2, (8, 16)).astype(np.float32)
                                                  for p in ("gate", "up", "down")}}]
    g, u, inter, y = O.mlp_fwd(x, wg, wu, wd, N, sl, bf16=True)
    for a in (g, u, inter, y):
        np.testing.assert_array_equal(a, O.bf16_round(a))
    ref_g = O.bf16_round((x.astype(np.float64) @ wg.T.astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(g[:, :I], ref_g)
    tail = O.bf16_round((x.astype(np.float64) @ O.bf16_round(sl[0]["gate"]).T.astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(g[:, I:], tail)


def test_test6_f32_explicit_equals_baked_oracle():
    G = GOLDEN["test6_f32"]
    S, H, D, F, M = G["S"], G["H"], G["D"], G["F"], G["M"]
    gate0 = np.array([(i + 1) * 0.1 for i in range(F * D)], np.float32).reshape(F, D)
    up0 = np.array([(i + 1) * 0.07 for i in range(F * D)], np.float32).reshape(F, D)
    down0 = np.array([(i + 1) * 0.05 for i in range(D * F)], np.float32).reshape(D, F)
    x = np.array(G["x"], np.float32).reshape(M, D)
    mk = lambda b, stp: np.array([[b + i * stp + j for j in range(H)] for i in range(S)], np.float32)
    dl = {k: mk(*v) for k, v in G["deltas"].items()}
    sl = [{"i0": 0, "s": S, "h0": 0, "h": H, "gate": dl["g0"], "up": dl["u0"], "down": dl["d0"]},
          {"i0": S, "s": S, "h0": H, "h": H, "gate": dl["g1"], "up": dl["u1"], "down": dl["d1"]}]
    a = O.mlp_fwd(x, gate0, up0, down0, F, sl, bf16=False)
    gb, ub, db = gate0.copy(), up0.copy(), down0.copy()
    gb[0:S, 0:H] += dl["g0"]; gb[S:, H:] += dl["g1"]
    ub[0:S, 0:H] += dl["u0"]; ub[S:, H:] += dl["u1"]
    db[0:H, 0:S] += dl["d0"].T; db[H:, S:] += dl["d1"].T
    b = O.mlp_fwd(x, gb, ub, db, F, [], bf16=False)
    for u, v in zip(a, b):
        md = np.max(np.abs(u - v))
        assert md < G["tol_abs"] or md / np.max(np.abs(v)) < G["tol_rel"]


def test_attention_rows_equals_full_attention():
    """The sampled-query form gives the full form's rows (causal and not)."""
    B, T, Hq, Hkv, hd = 2, 23, 4, 2, 8
    rng = np.random.default_rng(9)
    q, k, v = (rng.normal(size=(B, T, H, hd)) for H in (Hq, Hkv, Hkv))
    bi, ti = np.array([0, 0, 1, 1, 1]), np.array([0, 11, 3, 21, 22])
    for causal in (True, False):
        full = O.attention(q, k, v, causal=causal)
        rows = O.attention_rows(q[bi, ti], k, v, bi, ti, causal=causal)
        np.testing.assert_allclose(rows, full[bi, ti], rtol=1e-12, atol=1e-14)


def test_mlp_recompute_matches_aten_bf16_sequence():
    """The reference's recompute (src/layer_recompute_impl.inc:20-64) rebuilds
    each grafted slice of the bf16 pre-activation with torch's bf16 in-place
    add of the cached delta cast to bf16. The oracle's recompute equals that
    sequence run with torch's CPU bf16 kernels on the oracle's own base
    pre-activations and delta GEMMs; the forward (one rounding of the f32
    delta) differs from it on in-place slices and equals it on appended ones."""
    D, I, N, M = 32, 48, 64, 40
    rng = np.random.default_rng(21)
    x = O.bf16_round(rng.normal(size=(M, D)).astype(np.float32))
    wg, wu = (O.bf16_round(rng.normal(0, 0.2, (I, D)).astype(np.float32)) for _ in range(2))
    wd = O.bf16_round(rng.normal(0, 0.2, (D, I)).astype(np.float32))
    sl = [{"i0": 8, "s": 16, "h0": 4, "h": 20},      # in place
          {"i0": 48, "s": 16, "h0": 0, "h": 32}]     # appended
    for s in sl:
        for p in ("gate", "up", "down"):
            s[p] = rng.normal(0, 0.3, (s["s"], s["h"])).astype(np.float32)
    g, u, inter = O.mlp_recompute(x, wg, wu, N, sl)
    gb, ub, _, _ = O.mlp_fwd(x, wg, wu, wd, N, [], bf16=True)        # base pre-activations (bf16)
    for name, got, base in (("gate", g, gb), ("up", u, ub)):
        t = torch.from_numpy(base.copy()).to(torch.bfloat16)
        for s in sl:
            # the cached expand output: f32 delta of the forward (graft GEMM kind 0)
            delta = O.graft_gemm(0, M, s["s"], s["h"], a=x[:, s["h0"]:s["h0"] + s["h"]].copy(), lda=s["h"],
                                 delta=s[name])
            t[:, s["i0"]:s["i0"] + s["s"]].add_(torch.from_numpy(delta).to(torch.bfloat16))
        np.testing.assert_array_equal(got, t.float().numpy(), err_msg=name)
    np.testing.assert_array_equal(inter, O.silu_mul(g, u))
    gf, uf, _, _ = O.mlp_fwd(x, wg, wu, wd, N, sl, bf16=True)
    np.testing.assert_array_equal(g[:, I:], gf[:, I:])                 # appended: one rounding either way
    assert np.any(g[:, 8:24] != gf[:, 8:24])                           # in place: the double rounding shows
    assert np.max(np.abs(g - gf)) <= 2 ** -7 * np.max(np.abs(gf))      # within one bf16 ulp of the forward
