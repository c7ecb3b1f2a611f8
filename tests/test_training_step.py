"""Training-step neighbours on the CPU: the oracle's masked cross-entropy,
silence terms and LR schedule pinned against torch's own CPU kernels run in
the reference's op sequence, against closed forms, and the host-side LR
schedule of libglt.so against the oracle."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O


def _reference_ops(x, ids, ood, scale):
    """The reference's masked CE and grad_logits as torch ops on bf16 CPU
    tensors, in its order (grafting.hip:1027-1050, :1122-1135)."""
    B, T, V = x.shape
    logits = torch.tensor(x, dtype=torch.bfloat16)
    labels = torch.tensor(ids[:, 1:].astype(np.int64)).reshape(-1)
    lf = logits[:, :T - 1].reshape(-1, V)
    ce = -torch.log_softmax(lf, -1).gather(-1, labels.unsqueeze(-1)).squeeze(-1)
    dm = (1 - torch.tensor(ood[:, 1:].astype(np.int32)).reshape(-1)).to(torch.float32)
    n = max(dm.sum().item(), 1.0)
    loss = (ce * dm).sum() / n
    g = torch.softmax(lf, -1)
    ar = torch.arange(labels.numel())
    g.index_put_((ar, labels), g[ar, labels] - 1.0)
    g *= dm.unsqueeze(-1)
    g /= n
    g *= scale
    full = torch.zeros((B, T, V), dtype=torch.bfloat16)
    full[:, :T - 1] = g.reshape(B, T - 1, V)
    return full.float().numpy(), ce.float().numpy(), loss.item(), n


@pytest.mark.parametrize("B,T,V,ood_kind,scale", [(2, 9, 257, "half", 1.0), (3, 5, 1000, "none", 1.0),
                                                   (1, 17, 64, "all", 1.0), (2, 6, 333, "half", 2.0)])
def test_masked_ce_oracle_matches_torch(B, T, V, ood_kind, scale):
    rng = np.random.default_rng(B * 1000 + V)
    x = O.bf16_round(rng.normal(0, 3, (B, T, V)).astype(np.float32))
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    ood = np.zeros((B, T), np.int32)
    if ood_kind == "half":
        ood[:, T // 2:] = 1
    elif ood_kind == "all":
        ood[:] = 1
    g, ce, st = O.masked_ce(x, ids, ood, scale)
    tg, tce, tloss, tn = _reference_ops(x, ids, ood, scale)
    assert st[3] == tn
    # same per-element formula; torch's CPU softmax (f32 exp and sum, its own
    # intermediate rounding; the reference's GPU kernel rounds once) and the
    # oracle's f64 may land on opposite sides of a bf16 rounding boundary now
    # and then: nearly all elements agree bit for bit, none by more than 2 ulp
    same = np.mean(g.view(np.uint32) == tg.view(np.uint32))
    assert same > 0.995, same
    assert np.all(np.abs(g - tg) <= np.abs(tg) * 2.0 ** -6 + 1e-30)
    assert np.all(np.abs(ce - tce) <= np.abs(tce) * 2.0 ** -7)
    assert st[0] == pytest.approx(tloss, rel=2e-3, abs=1e-6)


def test_masked_ce_closed_form():
    # equal logits: p = 1/V exactly where representable; ce = log V
    B, T, V = 2, 4, 64
    x = np.full((B, T, V), 0.5, np.float32)
    ids = np.tile(np.arange(T, dtype=np.int32), (B, 1))
    g, ce, st = O.masked_ce(x, ids, None, 1.0)
    n = B * (T - 1)
    p = 1.0 / V
    assert np.allclose(ce, O.bf16_round(np.float32(math.log(V))))
    assert st[0] == pytest.approx(float(O.bf16_round(np.float32(math.log(V)))), rel=1e-6)
    assert st[2] == pytest.approx(p, rel=1e-6) and st[3] == n
    lab = g[0, 0, 1]
    assert lab == O.bf16_round(O.bf16_round(np.float32(p - 1.0)) * np.float32(1.0 / n))
    assert np.all(g[:, T - 1] == 0)
    # the gradient of each scored row sums to ~0 (softmax minus one-hot)
    assert np.abs(g[:, :T - 1].astype(np.float64).sum(-1)).max() < 4.0 / (n * 64)


def test_masked_ce_masked_rows_are_zero():
    rng = np.random.default_rng(3)
    B, T, V = 1, 6, 50
    x = O.bf16_round(rng.normal(0, 1, (B, T, V)).astype(np.float32))
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    ood = np.array([[0, 1, 0, 1, 0, 0]], np.int32)  # rows t=0 and t=2 excluded (ood of t+1)
    g, _, st = O.masked_ce(x, ids, ood, 1.0)
    assert st[3] == 3
    assert np.all(g[0, 0] == 0) and np.all(g[0, 2] == 0) and np.any(g[0, 1] != 0)


def test_silence_closed_forms():
    tokens, sl = 5, 64
    c = np.linspace(-2, 2, tokens).astype(np.float32)
    c[2] = 0.5
    d = np.tile(c[:, None], (1, sl))
    e = O.silence_energy(d)
    assert np.allclose(e, np.sqrt(sl * c.astype(np.float64) ** 2 + 1e-8) / np.sqrt(sl))
    ood = np.array([1, 0, 1, 0, 1], np.int32)
    lam = 5.0
    out = O.silence_blend(np.zeros_like(d), d, ood, lam)
    # dy += lam * c / (|c| sqrt(sl) * sqrt(sl)) = lam * sign(c) / sl on OOD rows
    for t in range(tokens):
        want = lam * np.sign(c[t]) / sl if ood[t] else 0.0
        assert np.allclose(out[t], want, rtol=1e-6, atol=1e-12)
    og, ou, eg, eu = O.silence_blend_energy(np.zeros_like(d), d, np.zeros_like(d), 2 * d, ood, lam)
    assert np.allclose(eu, O.silence_energy(2 * d))
    assert np.allclose(og[0], lam * np.sign(c[0]) / sl, rtol=1e-6)


def test_lr_schedule_closed_forms_and_library():
    from glt_amd import ops
    peak, warm, total = 3e-4, 20, 200
    for step in (0, 5, 19):
        assert O.lr_schedule(step, total, warm, peak) == np.float32(np.float32(peak * (step + 1)) / warm)
    assert O.lr_schedule(warm, total, warm, peak) == pytest.approx(peak, rel=1e-7)
    assert O.lr_schedule(total, total, warm, peak) == pytest.approx(0.0, abs=1e-12)
    assert O.lr_schedule(warm + (total - warm) // 2, total, warm, peak) == pytest.approx(peak / 2, rel=1e-6)
    # total <= warmup: the denominator is clamped to 1
    assert ops.lr_schedule(5, 3, 3, peak) == pytest.approx(O.lr_schedule(5, 3, 3, peak), rel=1e-6)
    for step in range(0, total + 1, 7):
        a = np.float32(ops.lr_schedule(step, total, warm, peak))
        b = O.lr_schedule(step, total, warm, peak)
        assert abs(float(a) - float(b)) <= 2 * np.spacing(np.float32(max(abs(b), 1e-30))), (step, a, b)
