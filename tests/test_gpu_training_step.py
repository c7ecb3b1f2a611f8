"""GPU parity of the training-step neighbours against the oracle: masked
cross-entropy with grad_logits (register-resident rows, the re-read path for
vocabularies past 131072 and for unaligned rows, in-place, masks, scale),
and the silence energy / blend kernels."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bf16(a):
    return torch.tensor(np.asarray(a, np.float32)).to(torch.bfloat16).cuda()


def _case(B, T, V, seed, ood_kind="some"):
    rng = np.random.default_rng(seed)
    x = O.bf16_round(rng.normal(0, 3, (B, T, V)).astype(np.float32))
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    ood = np.zeros((B, T), np.int32)
    if ood_kind == "some":
        ood[:, 1::3] = 1
    elif ood_kind == "all":
        ood[:] = 1
    return x, ids, ood


def _check_grad(g, ref):
    # bf16 bar: 1-ulp flips where the GPU's f32 exp/sum and the oracle's f64
    # straddle a rounding boundary; the bulk is bit-identical
    g = g.float().cpu().numpy()
    same = np.mean(g.view(np.uint32) == ref.view(np.uint32))
    assert same > 0.99, same
    scale = np.abs(ref).max()
    assert np.abs(g - ref).max() <= scale * 2.0 ** -7  # q = 2
    err = np.linalg.norm((g - ref).ravel()) / max(np.linalg.norm(ref.ravel()), 1e-30)
    assert err <= 1e-2


@pytest.mark.parametrize("B,T,V,ood_kind,scale", [
    (2, 9, 1000, "some", 1.0),        # resident rows
    (3, 4, 128256, "some", 1.0),      # Llama-3 vocabulary, resident
    (1, 3, 140000, "none", 2.0),      # past 131072: re-read path
    (2, 5, 1001, "all", 1.0),         # V % 8 != 0: re-read path, every row excluded
])
def test_masked_ce_matches_oracle(B, T, V, ood_kind, scale):
    from glt_amd import ops
    x, ids, ood = _case(B, T, V, B * 7 + V, ood_kind)
    print(f"case B={B} T={T} V={V} ood={ood_kind}", flush=True)
    stats, g, ce = ops.masked_ce(_bf16(x), torch.tensor(ids).cuda(), torch.tensor(ood).cuda(), scale,
                                 ce_per_token=True)
    torch.cuda.synchronize()
    rg, rce, rst = O.masked_ce(x, ids, ood, scale)
    _check_grad(g, rg)
    c = ce.cpu().numpy()[:B * (T - 1)]
    assert np.all(np.abs(c - rce) <= np.abs(rce) * 2.0 ** -7 + 1e-30)
    st = stats.cpu().numpy()
    assert st[3] == rst[3]
    assert st[0] == pytest.approx(rst[0], rel=2e-3, abs=1e-6)
    assert st[1] == pytest.approx(rst[1], rel=1e-5, abs=1e-5)
    assert st[2] == pytest.approx(rst[2], rel=1e-2, abs=1e-6)


def test_masked_ce_in_place_and_loss_only():
    from glt_amd import ops
    B, T, V = 2, 6, 4096
    x, ids, ood = _case(B, T, V, 11)
    logits = _bf16(x)
    stats_a, _, _ = ops.masked_ce(_bf16(x), torch.tensor(ids).cuda(), torch.tensor(ood).cuda(), want_grad=False)
    stats_b, g, _ = ops.masked_ce(logits, torch.tensor(ids).cuda(), torch.tensor(ood).cuda(), grad=logits)
    torch.cuda.synchronize()
    assert g.data_ptr() == logits.data_ptr()
    rg, _, rst = O.masked_ce(x, ids, ood, 1.0)
    _check_grad(logits, rg)
    assert np.array_equal(stats_a.cpu().numpy(), stats_b.cpu().numpy())


def test_masked_ce_single_position_rows():
    from glt_amd import ops
    x, ids, ood = _case(3, 1, 512, 5)
    stats, g, _ = ops.masked_ce(_bf16(x), torch.tensor(ids).cuda(), torch.tensor(ood).cuda())
    torch.cuda.synchronize()
    assert torch.count_nonzero(g).item() == 0
    assert stats.cpu().numpy().tolist() == [0.0, 0.0, 0.0, 1.0]


@pytest.mark.parametrize("tokens,sl", [(37, 1024), (5, 200)])
def test_silence_kernels_match_oracle(tokens, sl):
    from glt_amd import ops
    rng = np.random.default_rng(tokens + sl)
    d_g = rng.normal(0, 0.05, (tokens, sl)).astype(np.float32)
    d_u = rng.normal(0, 0.02, (tokens, sl)).astype(np.float32)
    dy = rng.normal(0, 1, (tokens, sl)).astype(np.float32)
    ood = (np.arange(tokens) % 3 == 0).astype(np.int32)
    tg = torch.tensor(d_g).cuda()
    e = ops.silence_energy(tg)
    eb = ops.silence_energy(tg.to(torch.bfloat16))
    out = ops.silence_blend(torch.tensor(dy).cuda(), tg, torch.tensor(ood).cuda(), 5.0)
    dyg, dyu = torch.tensor(dy).cuda(), torch.tensor(dy).cuda()
    eg, eu = ops.silence_blend_energy(dyg, tg, dyu, torch.tensor(d_u).cuda(), torch.tensor(ood).cuda(), 5.0)
    torch.cuda.synchronize()
    assert np.allclose(e.cpu().numpy(), O.silence_energy(d_g), rtol=1e-5)
    assert np.allclose(eb.cpu().numpy(), O.silence_energy(O.bf16_round(d_g)), rtol=1e-5)
    assert np.allclose(out.cpu().numpy(), O.silence_blend(dy, d_g, ood, 5.0), rtol=1e-5, atol=1e-6)
    rg, ru, reg, reu = O.silence_blend_energy(dy, d_g, dy, d_u, ood, 5.0)
    assert np.allclose(dyg.cpu().numpy(), rg, rtol=1e-5, atol=1e-6)
    assert np.allclose(dyu.cpu().numpy(), ru, rtol=1e-5, atol=1e-6)
    assert np.allclose(eg.cpu().numpy(), reg, rtol=1e-5) and np.allclose(eu.cpu().numpy(), reu, rtol=1e-5)


def test_masked_ce_full_size_properties():
    """The benchmarked size (4 x 4096 positions, Llama-3 vocabulary 128256):
    n counts the unmasked shifted positions exactly; the loss is the mean
    of the per-token CE over them; sampled rows' CE and gradient match the
    oracle (each row posed as its own two-position sequence, the gradient
    rescaled from the sample's n to the full n); masked rows and the last
    position of each sequence carry no gradient."""
    import torch
    from glt_amd import ops
    B, T, V = 4, 4096, 128256
    logits = ops.fill_normal(torch.empty((B, T, V), dtype=torch.bfloat16, device="cuda"), 41, 1, 0.0, 3.0)
    gen = torch.Generator().manual_seed(5)
    ids = torch.randint(0, V, (B, T), generator=gen, dtype=torch.int32)
    ood = (torch.rand((B, T), generator=gen) < 0.25).to(torch.int32)
    stats, g, ce = ops.masked_ce(logits, ids.cuda(), ood.cuda(), 1.0, ce_per_token=True)
    torch.cuda.synchronize()
    st = stats.cpu().numpy()
    valid = (1 - ood[:, 1:]).reshape(-1).numpy().astype(bool)
    n = int(valid.sum())
    assert st[3] == n
    cen = ce.cpu().numpy()[:B * (T - 1)].astype(np.float64)
    assert st[0] == pytest.approx(cen[valid].sum() / n, rel=1e-4)
    samples = [(0, 0), (0, 1), (1, 2047), (2, 4000), (3, 4094), (3, 17)]
    sv = [(b, t) for b, t in samples if not ood[b, t + 1]]
    sm = [(b, t) for b, t in samples if ood[b, t + 1]]
    assert sv, "the sample needs unmasked rows"
    x = np.stack([[logits[b, t].float().cpu().numpy(), np.zeros(V, np.float32)] for b, t in sv])
    sid = np.array([[0, ids[b, t + 1]] for b, t in sv], np.int32)
    rg, rce, rst = O.masked_ce(x, sid, None, 1.0)
    for i, (b, t) in enumerate(sv):
        assert abs(cen[b * (T - 1) + t] - rce[i]) <= abs(rce[i]) * 2.0 ** -7 + 1e-30
        got = g[b, t].float().cpu().numpy()
        ref = rg[i, 0] * (rst[3] / n)
        assert np.abs(got - ref).max() <= np.abs(ref).max() * 2.0 ** -6, (b, t)
    for b, t in sm:
        assert torch.count_nonzero(g[b, t]).item() == 0
    assert torch.count_nonzero(g[:, T - 1]).item() == 0
