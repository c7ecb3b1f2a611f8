"""GPU parity of the whole-model pieces against the oracle: embedding,
LM head, forward_model (reference grafting.hip:224-271) with the graft path
on and off, and the shadow-eval statistics (grafting.hip:504-547)."""
import numpy as np
import pytest

from helpers import assert_bf16_budget, draw, make_layer, to_dev, to_np
from oracle import oracle as O
from test_gpu_layer import _oracle_layer

pytestmark = pytest.mark.gpu


def test_embedding_gathers_rows(dev):
    import torch
    from glt_amd import ops
    V, D = 50, 96
    table = draw((V, D), 0, 7, 0, 1.0)
    ids = np.array([0, 49, 3, 3, 17, -1, 50, 8], np.int32)
    out = ops.embedding(torch.tensor(ids).cuda(), to_dev(table, torch.bfloat16))
    torch.cuda.synchronize()
    ref = np.where(((ids >= 0) & (ids < V))[:, None], table[np.clip(ids, 0, V - 1)], 0.0)
    np.testing.assert_array_equal(to_np(out), ref)


@pytest.mark.parametrize("M,D,V", [(100, 256, 1000), (64, 200, 77)])
def test_lm_head_matches_oracle(dev, M, D, V):
    import torch
    from glt_amd import ops
    x = draw((M, D), 0, 1, 0, 1.0)
    w = draw((V, D), 0, 2, 0, 0.02)
    out = ops.lm_head_fwd(to_dev(x, torch.bfloat16), to_dev(w, torch.bfloat16))
    torch.cuda.synchronize()
    assert_bf16_budget(to_np(out), O.lm_head(x, w), q=1, what="logits")


@pytest.mark.parametrize("explicit", [True, False])
def test_model_forward_matches_oracle(dev, explicit):
    import torch
    from glt_amd import ops
    bf = torch.bfloat16
    B, T, D, Hq, Hkv, I, S, V, L = 1, 96, 256, 4, 2, 512, 128, 1000, 2
    hd, theta, eps = 128, 500000.0, 1e-5
    N = I + S
    embed = draw((V, D), 0, 90, 0, 0.05)
    final_norm = O.bf16_round(1 + draw((D,), 300, 91, 0, 0.02, bf16=False))
    ids = np.random.default_rng(5).integers(0, V, (B, T)).astype(np.int32)
    layers, refs = [], []
    for l in range(L):
        wq = draw((Hq * hd, D), 0, 30 + 10 * l, 0, 0.02)
        wk = draw((Hkv * hd, D), 0, 31 + 10 * l, 0, 0.02)
        wv = draw((Hkv * hd, D), 0, 32 + 10 * l, 0, 0.02)
        wo = draw((D, Hq * hd), 0, 33 + 10 * l, 0, 0.02)
        ln_in = O.bf16_round(1 + draw((D,), 300, 12 + 10 * l, 0, 0.02, bf16=False))
        ln_post = O.bf16_round(1 + draw((D,), 300, 13 + 10 * l, 0, 0.02, bf16=False))
        wg, wu, wd, sl = make_layer(D, I, N, [(I, S, 0, D)], True, base_seed=100 + l)
        base = ops.BaseMLP(to_dev(wg, bf), to_dev(wu, bf), to_dev(wd, bf))
        gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"],
                             *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack() for s in sl]
        layers.append(ops.DecoderLayer(B, T, Hq, Hkv, *(to_dev(w, bf) for w in (wq, wk, wv, wo, ln_in, ln_post)),
                                       base, gs, N, rope_theta=theta, rms_eps=eps))
        refs.append((wq, wk, wv, wo, ln_in, ln_post, wg, wu, wd, sl if explicit else []))
    model = ops.Model(layers, to_dev(embed, bf), to_dev(final_norm, bf))
    logits = model.forward(torch.tensor(ids).cuda(), explicit=explicit)
    torch.cuda.synchronize()
    x = embed[ids.reshape(-1)]
    for (wq, wk, wv, wo, ln_in, ln_post, wg, wu, wd, sl) in refs:
        x, _ = _oracle_layer(x, wq, wk, wv, wo, ln_in, ln_post, wg, wu, wd, N, sl, B, T, Hq, Hkv, theta, eps)
    xn, _ = O.rmsnorm_fwd(x, final_norm, eps)
    ref = O.lm_head(xn, embed)     # lm_head tied to the embedding
    assert_bf16_budget(to_np(logits), ref, q=8, what="logits")


@pytest.mark.parametrize("reference_hash,extreme", [(True, False), (False, False), (True, True), (False, True)])
def test_eval_stats_match_oracle(dev, reference_hash, extreme):
    """extreme: logits of magnitude 2^70 and 2^-70, whose f32 squares overflow
    and underflow; the sum of squares is formed in f64 as the reference's
    (grafting.hip:525-547)."""
    import torch
    from glt_amd import ops
    B, T, V = 2, 33, 1500
    x = O.bf16_round(np.random.default_rng(8).normal(0, 3, (B * T, V)).astype(np.float32))
    if extreme:
        x[5, 17], x[40, 3], x[41, 1499] = 2.0 ** 70, -(2.0 ** 70), 2.0 ** -70
        x[60, :] = 2.0 ** -70
    ids = np.random.default_rng(9).integers(0, V, (B, T)).astype(np.int32)
    r = ops.eval_stats(to_dev(x, torch.bfloat16), torch.tensor(ids).cuda(), reference_hash=reference_hash)
    ref = O.eval_stats(x.reshape(B, T, V), ids, reference_hash=reference_hash)
    assert r["logits_hash"] == ref["logits_hash"]
    assert r["count"] == ref["count"]
    assert r["total_nll"] == pytest.approx(ref["total_nll"], rel=1e-5)
    # +-2^70 cancel in the sum: any f64 summation order loses up to a few of
    # their ulps (2^18) there
    assert r["logits_sum"] == pytest.approx(ref["logits_sum"], rel=1e-9, abs=2.0 ** 20 if extreme else 1e-6)
    assert r["logits_sumsq"] == pytest.approx(ref["logits_sumsq"], rel=1e-12)
    assert np.isfinite(r["logits_sumsq"])


@pytest.mark.parametrize("B,T,V,ld", [(2, 3, 128256, 128256),   # the Llama-3 vocabulary, 16-byte chunks
                                      (3, 5, 1001, 1001),       # odd rows: element-wise walk
                                      (1, 2, 7, 7),             # fewer logits than chunks per row
                                      (2, 4, 96, 104),          # padded row stride
                                      (4, 512, 32000, 32000)])  # 32768 chunks: several scan workgroups
def test_eval_reference_hash_is_exact(dev, B, T, V, ld):
    """The reference's logits hash (one FNV-1a chain over every f32 logit byte,
    grafting.hip:536-546) bit for bit, from the basis and from an arbitrary
    running hash, against the oracle's sequential loop."""
    import torch
    from glt_amd import ops
    rng = np.random.default_rng(B * 1000 + V)
    x = O.bf16_round(rng.normal(0, 2, (B * T, ld)).astype(np.float32))
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    xd, idd = to_dev(x, torch.bfloat16), torch.tensor(ids).cuda()
    view = xd[:, :V]
    h0 = int(rng.integers(0, 2 ** 63)) * 2 + 1
    for hin in (O.FNV_BASIS, h0):
        r = ops.eval_stats(view, idd, hash_in=hin)
        assert r["logits_hash"] == O.eval_hash_reference(x[:, :V].reshape(B, T, V), hin), (B, T, V, hin)
    print("hash", B, T, V, hex(r["logits_hash"]), flush=True)


def test_eval_reference_hash_chains_batches(dev):
    """Batches chained as the reference's eval loop does (the running hash
    carries over): eval_batches over three batches equals the sequential
    chain over their concatenation, and nll/counts add up."""
    import torch
    from glt_amd import ops
    rng = np.random.default_rng(12)
    V, T = 5000, 17
    xs = [O.bf16_round(rng.normal(0, 3, (b, T, V)).astype(np.float32)) for b in (2, 1, 3)]
    ids = [rng.integers(0, V, (x.shape[0], T)).astype(np.int32) for x in xs]
    r = ops.eval_batches([(to_dev(x.reshape(-1, V), torch.bfloat16), torch.tensor(i).cuda()) for x, i in zip(xs, ids)])
    assert r["logits_hash"] == O.eval_hash_reference(np.concatenate(xs))
    refs = [O.eval_stats(x, i) for x, i in zip(xs, ids)]
    assert r["count"] == sum(q["count"] for q in refs)
    assert r["total_nll"] == pytest.approx(sum(q["total_nll"] for q in refs), rel=1e-5)


def test_lm_head_at_eval_size_runs_in_row_blocks(dev):
    """An LM head whose logits pass 2 GiB (16384 tokens x 128256 = 4 GiB of
    bf16) runs on the MFMA kernel in row blocks of 7936 tokens (the most
    whose output offsets fit the kernel's 31-bit buffer range: three launches
    here) instead of falling back to the strided kernel; sampled rows of every
    block match the oracle."""
    import torch
    from glt_amd import _ffi as F
    from glt_amd import ops
    M, D, V = 16384, 4096, 128256
    bf = torch.bfloat16
    x = ops.fill_normal(torch.empty((M, D), dtype=bf, device="cuda"), 100, 10, 0.0, 1.0)
    w = ops.fill_normal(torch.empty((V, D), dtype=bf, device="cuda"), 0, 60, 0.0, 0.02)
    prep = torch.empty(F.load().glt_lm_head_prepared_size(V, D), dtype=torch.uint8, device="cuda")
    F.call("glt_lm_head_prepare", ops._p(w), V, D, ops._p(prep), ops._stream())
    F.load().glt_profile_enable(1)
    F.profile_collect()
    logits = ops.lm_head_fwd(x, w, prep)
    torch.cuda.synchronize()
    prof = F.profile_collect()
    F.load().glt_profile_enable(0)
    assert prof["lm_head"][1] == 3, prof
    rows = torch.tensor([0, 4095, 7935, 7936, 12000, 15871, 15872, 16383], device="cuda")
    wn = to_np(w)
    ref = O.lm_head(to_np(x[rows]), wn)
    assert_bf16_budget(to_np(logits[rows]), ref, q=1, what="eval-size logits")


def test_certify_bake_and_reload_gates(dev):
    """The certify run on a two-layer model: A base, B explicit graft, C the
    shadow-baked weights with the graft path off, D the same base rebuilt.
    Baked equals explicit within the bake budget (gate 2) and the rebuilt
    base reproduces A's CE and logits hash (gate 3)."""
    import torch
    from glt_amd import _ffi as F
    from glt_amd import ops
    bf = torch.bfloat16
    B, T, D, Hq, Hkv, I, S, V, L = 2, 64, 256, 4, 2, 512, 128, 1000, 2
    N = I + S
    embed = to_dev(draw((V, D), 0, 90, 0, 0.05), bf)
    final_norm = to_dev(O.bf16_round(1 + draw((D,), 300, 91, 0, 0.02, bf16=False)), bf)
    ids = torch.tensor(np.random.default_rng(6).integers(0, V, (B, T)).astype(np.int32)).cuda()
    att, mlp = [], []
    for l in range(L):
        att.append([to_dev(draw(sh, 0, 40 + 10 * l + k, 0, 0.02), bf) for k, sh in
                    enumerate(((Hq * 128, D), (Hkv * 128, D), (Hkv * 128, D), (D, Hq * 128)))] +
                   [to_dev(O.bf16_round(1 + draw((D,), 300, 44 + 10 * l + k, 0, 0.02, bf16=False)), bf)
                    for k in range(2)])
        wg, wu, wd, sl = make_layer(D, I, N, [(I, S, 0, D)], True, base_seed=200 + l, graft_std=0.05)
        gs = [ops.GraftSlice(s["i0"], s["s"], s["h0"], s["h"],
                             *(to_dev(s[p], torch.float32) for p in ("gate", "up", "down"))).pack() for s in sl]
        mlp.append((to_dev(wg, bf), to_dev(wu, bf), to_dev(wd, bf), gs))

    def model(bases, slices):
        layers = [ops.DecoderLayer(B, T, Hq, Hkv, *att[l], bases[l], slices[l], N) for l in range(L)]
        return ops.Model(layers, embed, final_norm)

    def ev(m, explicit):
        return ops.eval_stats(m.forward(ids, explicit=explicit), ids)

    bases = [ops.BaseMLP(wg, wu, wd) for (wg, wu, wd, _) in mlp]
    m = model(bases, [gs for (_, _, _, gs) in mlp])
    A, Bx = ev(m, False), ev(m, True)
    baked = []
    for (wg, wu, wd, gs) in mlp:
        go = torch.empty((N, D), dtype=bf, device="cuda")
        uo = torch.empty((N, D), dtype=bf, device="cuda")
        do = torch.empty((D, N), dtype=bf, device="cuda")
        flat = [[torch.cat([s.gate.reshape(-1), s.up.reshape(-1), s.down.reshape(-1)])] for s in gs]
        ops.shadow_bake(F.ModelState(0), [wg], [wu], [wd], flat, [(s.i_start, s.s, s.h_start, s.h) for s in gs],
                        D=D, I=I, N=N, materialize=True, gate_out=[go], up_out=[uo], down_out=[do])
        baked.append(ops.BaseMLP(go, uo, do))
    C = ev(model(baked, [[] for _ in range(L)]), False)
    Dr = ev(model([ops.BaseMLP(wg, wu, wd) for (wg, wu, wd, _) in mlp], [[] for _ in range(L)]), False)
    torch.cuda.synchronize()
    r = ops.certify(A, Bx, C, Dr)
    print({k: r[k] for k in ("A_ce", "B_ce", "C_ce", "D_ce", "bake_ce_gap")}, flush=True)
    assert Bx["ce"] != A["ce"]                 # the graft changes the model
    assert r["gate_bake_equal"] == 1, r
    assert r["gate_reload_equal"] == 1, r
    assert abs(r["bake_ce_gap"]) < 2e-3


@pytest.mark.parametrize("M,V,D", [(96, 1024, 256), (40, 1000, 200)])
def test_lm_head_backward_matches_oracle(dev, M, V, D):
    """dx = grad_logits . lm_head (reference grafting.hip:1137) in f32: MFMA
    path (V a multiple of 64) and strided path."""
    import torch
    from glt_amd import ops
    g = draw((M, V), 0, 3, 0, 1e-3)
    w = draw((V, D), 0, 4, 0, 0.02)
    dx = ops.lm_head_bwd(to_dev(g, torch.bfloat16), to_dev(w, torch.bfloat16))
    torch.cuda.synchronize()
    ref = np.asarray(g, np.float64) @ np.asarray(w, np.float64)
    err = np.linalg.norm((to_np(dx) - ref).ravel()) / np.linalg.norm(ref.ravel())
    assert err < 1e-5, err
