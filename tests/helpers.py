"""Shared test helpers: input drawing, bf16 handling, parity metrics."""
import numpy as np

from glt_amd import synth
from oracle import oracle as O


def draw(shape, seed, tid, mean=0.0, std=1.0, bf16=True):
    a = synth.normal(shape, seed, tid, mean, std)
    return O.bf16_round(a) if bf16 else a


def to_dev(a, dtype):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t.to(dtype).cuda()


def to_np(t):
    return t.detach().float().cpu().numpy()


def rel_l2(out, ref):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(out - ref) / (den if den > 0 else 1.0))


def max_abs(out, ref):
    return float(np.max(np.abs(np.asarray(out, np.float64) - np.asarray(ref, np.float64)))) if np.size(ref) else 0.0


def assert_bf16_budget(out, ref, q, what=""):
    """bf16 budget: rel-L2 <= 1e-2 and max-abs <= q * 2^-8 * max|ref|, q =
    number of bf16 roundings on the longest path (the reference's "~1/256
    relative per quantization step", tests/test7_bf16_error_budget.cpp:239)."""
    r = rel_l2(out, ref)
    ma = max_abs(out, ref)
    lim = q * 2.0 ** -8 * float(np.max(np.abs(ref))) if np.size(ref) else 0.0
    assert r <= 1e-2, f"{what}: rel-L2 {r:.3e} > 1e-2"
    assert ma <= lim, f"{what}: max-abs {ma:.3e} > {lim:.3e} (q={q})"
    return r, ma


def assert_f32_close(out, ref, tol=1e-5, what=""):
    """f32 path: rel-L2 <= tol and max-abs <= tol * max|ref|."""
    r = rel_l2(out, ref)
    ma = max_abs(out, ref)
    lim = tol * float(np.max(np.abs(ref))) if np.size(ref) else 0.0
    assert r <= tol, f"{what}: rel-L2 {r:.3e} > {tol:.1e}"
    assert ma <= lim, f"{what}: max-abs {ma:.3e} > {lim:.3e}"
    return r, ma


def make_layer(D, I, N, slices_pl, bf16=True, base_seed=0, graft_std=0.02):
    """Base weights ~N(0,0.02) and per-slice deltas ~N(0,graft_std) with the
    workload seeds (base seed 0, slice k seed k+1)."""
    wg = draw((I, D), base_seed, synth.TID_GATE, 0, 0.02, bf16)
    wu = draw((I, D), base_seed, synth.TID_UP, 0, 0.02, bf16)
    wd = draw((D, I), base_seed, synth.TID_DOWN, 0, 0.02, bf16)
    slices = []
    for k, (i0, s, h0, h) in enumerate(slices_pl):
        sd = {"i0": i0, "s": s, "h0": h0, "h": h}
        for p, name in enumerate(("gate", "up", "down")):
            sd[name] = synth.normal((s, h), k + 1, 1 + p, 0, graft_std)  # f32 masters
        slices.append(sd)
    return wg, wu, wd, slices


def shuffle_b(b):
    """The MFMA fragment layout of a B operand [rows, K] (the kernels' own
    weight format, written by glt_base_prepare / glt_graft_pack): 32 x 64
    blocks, row-block major; inside a block [substep 4][lane 64][8], lane l
    of substep s holding row l%32, K = 16*s + 8*(l//32) + e. Zero padded."""
    b = np.asarray(b, np.float32)
    rows, k = b.shape
    rp, kp = -(-rows // 32) * 32, -(-k // 64) * 64
    pad = np.zeros((rp, kp), np.float32)
    pad[:rows, :k] = b
    blk = pad.reshape(rp // 32, 32, kp // 64, 4, 2, 8)  # rb, r, kb, s, half, e
    return blk.transpose(0, 2, 3, 4, 1, 5).reshape(-1)


def packed_views(packed_f32, s, h):
    """Splits a packed graft mirror (as f32 values) into its six row-major
    orientations and six shuffled ones (gate, gate^T, up, up^T, down, down^T)."""
    sh = s * h
    rowmajor = [packed_f32[q * sh:(q + 1) * sh].reshape((h, s) if q & 1 else (s, h)) for q in range(6)]
    off = -(-6 * sh // 128) * 128
    shuf = []
    for q in range(6):
        r, k = (h, s) if q & 1 else (s, h)
        n = (-(-r // 32) * 32) * (-(-k // 64) * 64)
        shuf.append(packed_f32[off:off + n])
        off += n
    return rowmajor, shuf
