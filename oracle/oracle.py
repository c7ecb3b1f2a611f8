"""numpy/ctypes front end of the C oracle (glt_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg; never by the glt_amd package.

All arrays are numpy float32 holding bf16-representable values where the
reference holds bf16 (use bf16_round to get there). Citations of the
reference live beside each C function in glt_oracle.c.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build():
    subprocess.run(["sh", os.path.join(HERE, "build.sh")], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _setup(_lib)
    return _lib


_f = ctypes.POINTER(ctypes.c_float)
_u16 = ctypes.POINTER(ctypes.c_uint16)
_i64 = ctypes.c_int64
_i = ctypes.c_int
_fl = ctypes.c_float


class Slice(ctypes.Structure):
    _fields_ = [("i0", _i), ("s", _i), ("h0", _i), ("h", _i),
                ("gate", _f), ("up", _f), ("down", _f)]


def _setup(L):
    L.orc_f32_to_bf16.restype = ctypes.c_uint16
    L.orc_f32_to_bf16.argtypes = [_fl]
    L.orc_bf16_to_f32.restype = _fl
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f32_to_bf16_vec.argtypes = [_f, _u16, _i64]
    L.orc_round_bf16_vec.argtypes = [_f, _i64]
    L.orc_gemm.argtypes = [_i, _i, _i, _f, _i64, _i64, _f, _i64, _i64, _f, _i64, _fl, _fl]
    L.orc_bake_inplace.argtypes = [_u16, _i64, _f, _i, _i, _i, _i, _i]
    L.orc_rmsnorm_fwd.argtypes = [_f, _f, _f, _f, _i, _i, _fl]
    L.orc_rmsnorm_bwd.argtypes = [_f, _f, _f, _f, _f, _i, _i, _fl]
    L.orc_rope.argtypes = [_f, _i, _i, _i, _i, _fl, _i, _i]
    L.orc_clip_scale.restype = _fl
    L.orc_clip_scale.argtypes = [_f, _i64, _fl]
    L.orc_adamw.argtypes = [_f, _f, _f, _f, _i64, _i, _fl, _fl, _fl, _fl, _fl, _fl]
    L.orc_silu_mul.argtypes = [_f, _f, _f, _i64, _i]
    L.orc_gate_up_bwd.argtypes = [_f, _f, _f, _f, _f, _i64]
    L.orc_mlp_fwd.argtypes = [_i, _i, _i, _i, _i, _i, ctypes.POINTER(Slice), _f, _f, _f, _f, _f, _f, _f, _f]
    L.orc_mlp_recompute.argtypes = [_i, _i, _i, _i, _i, ctypes.POINTER(Slice), _f, _f, _f, _f, _f, _f]
    L.orc_fnv1a64.restype = ctypes.c_uint64
    L.orc_fnv1a64.argtypes = [ctypes.c_void_p, _i64, ctypes.c_uint64]
    L.orc_mlp_bwd.argtypes = [_i, _i, _i, _i, _i, _i, ctypes.POINTER(Slice), _f, _f, _f, _f, _f, _f, _f, _f,
                              _f, ctypes.POINTER(_f)]


def _fp(a):
    if a is None:
        return _f()
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------ bf16
def f32_to_bf16_bits(x):
    """RNE bf16 bit patterns (uint16) of float32 values."""
    x = _c32(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_vec(_fp(x), out.ctypes.data_as(_u16), x.size)
    return out


def bf16_bits_to_f32(b):
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_round(x):
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ------------------------------------------------------------------ GEMM
def gemm_strided(M, N, K, A, sam, sak, B, sbn, sbk, C=None, ldc=None, alpha=1.0, beta=0.0):
    A, B = _c32(A), _c32(B)
    if C is None:
        C = np.zeros((M, N), np.float32)
        ldc = N
    lib().orc_gemm(M, N, K, _fp(A), sam, sak, _fp(B), sbn, sbk, _fp(C), ldc, alpha, beta)
    return C


def graft_gemm(kind, M, S, H, a=None, lda=None, delta=None, dy=None, out=None, ldo=None, alpha=1.0, beta=0.0):
    """The six graft GEMM kinds (reference src/gemm_impl.inc:383-584) with
    their bf16 rounding of f32 operands: delta and dy are rounded, a is bf16."""
    d = bf16_round(delta) if delta is not None else None
    g = bf16_round(dy) if dy is not None else None
    a = _c32(a).ravel() if a is not None else None
    if kind == 0:    # out[M,S] = a[M,H] . d^T
        return gemm_strided(M, S, H, a, lda, 1, d, H, 1, out, ldo, alpha, beta)
    if kind == 1:    # out[M,H] = a[M,S] . d
        return gemm_strided(M, H, S, a, lda, 1, d, 1, H, out, ldo, alpha, beta)
    if kind == 2:    # out[S,H] = g[M,S]^T . a[M,H]
        return gemm_strided(S, H, M, g, 1, S, a, 1, lda, out, ldo, alpha, beta)
    if kind == 3:    # out[S,H] = a[M,S]^T . g[M,H]
        return gemm_strided(S, H, M, a, 1, lda, g, 1, H, out, ldo, alpha, beta)
    if kind == 4:    # out[M,H] = g[M,S] . d
        return gemm_strided(M, H, S, g, S, 1, d, 1, H, out, ldo, alpha, beta)
    if kind == 5:    # out[M,S] = g[M,H] . d^T
        return gemm_strided(M, S, H, g, H, 1, d, H, 1, out, ldo, alpha, beta)
    raise ValueError(kind)


# ------------------------------------------------------------ shadow bake
def bake_inplace(base_bits, graft, i0, h0, mode):
    """base_bits: uint16 2-D (modified in place); graft f32 [S,H]."""
    assert base_bits.dtype == np.uint16 and base_bits.flags["C_CONTIGUOUS"]
    graft = _c32(graft)
    S, H = graft.shape
    lib().orc_bake_inplace(base_bits.ctypes.data_as(_u16), base_bits.shape[1], _fp(graft), S, H, i0, h0, mode)
    return base_bits


# -------------------------------------------------------------- RMSNorm
def rmsnorm_fwd(x, w, eps):
    x, w = _c32(x), _c32(w)
    M, D = x.shape
    y = np.empty_like(x)
    var = np.empty(M, np.float32)
    lib().orc_rmsnorm_fwd(_fp(x), _fp(w), _fp(y), _fp(var), M, D, eps)
    return y, var


def rmsnorm_bwd(dy, x, w, var, eps):
    dy, x, w, var = _c32(dy), _c32(x), _c32(w), _c32(var)
    M, D = x.shape
    dx = np.empty_like(dy)
    lib().orc_rmsnorm_bwd(_fp(dy), _fp(x), _fp(w), _fp(var), _fp(dx), M, D, eps)
    return dx


# ----------------------------------------------------------------- RoPE
def rope(t, theta, pos_offset=0, exact_rounding=True):
    """t: f32 [B,T,nh,hd] bf16-valued; returns the rotated copy."""
    t = _c32(t).copy()
    B, T, nh, hd = t.shape
    lib().orc_rope(_fp(t), B, T, nh, hd, theta, pos_offset, int(exact_rounding))
    return t


# ------------------------------------------------------------- attention
def attention(q, k, v, causal=True, scale=None):
    """Scaled-dot-product attention in float64, the reference's base
    attention (forward_layer, src/layer_forward_impl.inc:41-49): query head h
    reads kv head h // (Hq // Hkv) (k/v repeat_interleave'd over heads,
    :46-47), softmax(scale * q.k^T) with keys after the query masked when
    causal (SDPA is_causal, :48), then . v. q [B,T,Hq,hd], k/v [B,T,Hkv,hd];
    returns [B,T,Hq,hd] float64."""
    B, T, Hq, hd = q.shape
    Hkv = k.shape[2]
    rep = Hq // Hkv
    scale = hd ** -0.5 if scale is None else scale
    out = np.zeros((B, T, Hq, hd))
    future = np.triu(np.ones((T, T), bool), 1) if causal else np.zeros((T, T), bool)
    for b in range(B):
        for h in range(Hq):
            g = h // rep
            s = (np.asarray(q[b, :, h], np.float64) @ np.asarray(k[b, :, g], np.float64).T) * scale
            s[future] = -np.inf
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, :, h] = p @ np.asarray(v[b, :, g], np.float64)
    return out


def attention_rows(q_rows, k, v, b_idx, t_idx, causal=True, scale=None):
    """attention() for selected query positions only: q_rows [n,Hq,hd] are
    the queries of positions (b_idx[i], t_idx[i]); k/v [B,T,Hkv,hd]. Same
    float64 softmax; returns [n,Hq,hd] float64."""
    n, Hq, hd = q_rows.shape
    Hkv = k.shape[2]
    rep = Hq // Hkv
    scale = hd ** -0.5 if scale is None else scale
    out = np.zeros((n, Hq, hd))
    for i in range(n):
        b, t = int(b_idx[i]), int(t_idx[i])
        end = t + 1 if causal else k.shape[1]
        for h in range(Hq):
            g = h // rep
            s = (np.asarray(k[b, :end, g], np.float64) @ np.asarray(q_rows[i, h], np.float64)) * scale
            s -= s.max()
            p = np.exp(s)
            p /= p.sum()
            out[i, h] = p @ np.asarray(v[b, :end, g], np.float64)
    return out


# ---------------------------------------------------------------- AdamW
def adamw(w, g, m, v, step, lr, b1, b2, eps, wd, clip_norm=0.0):
    w, g, m, v = _c32(w).copy(), _c32(g), _c32(m).copy(), _c32(v).copy()
    scale = lib().orc_clip_scale(_fp(g), g.size, clip_norm) if clip_norm > 0 else 1.0
    lib().orc_adamw(_fp(w), _fp(g), _fp(m), _fp(v), w.size, step, lr, b1, b2, eps, wd, scale)
    return w, m, v


# ---------------------------------------------------------- elementwise
def silu_mul(g, u, round_out=True):
    g, u = _c32(g), _c32(u)
    out = np.empty_like(g)
    lib().orc_silu_mul(_fp(g), _fp(u), _fp(out), g.size, int(round_out))
    return out


def gate_up_bwd(gi, g, u):
    gi, g, u = _c32(gi), _c32(g), _c32(u)
    dg, du = np.empty_like(gi), np.empty_like(gi)
    lib().orc_gate_up_bwd(_fp(gi), _fp(g), _fp(u), _fp(dg), _fp(du), gi.size)
    return dg, du


# ------------------------------------------------------------ MLP layer
def _slices(slices):
    """slices: list of dicts {i0, s, h0, h, gate, up, down} (f32 [S,H] or None)."""
    keep = []
    arr = (Slice * max(1, len(slices)))()
    for j, s in enumerate(slices):
        vals = {}
        for p in ("gate", "up", "down"):
            a = s.get(p)
            vals[p] = _c32(a) if a is not None else None
            keep.append(vals[p])
        arr[j] = Slice(s["i0"], s["s"], s["h0"], s["h"], _fp(vals["gate"]), _fp(vals["up"]), _fp(vals["down"]))
    return arr, keep


def mlp_fwd(x, wg, wu, wd, N, slices, bf16=True):
    x, wg, wu, wd = _c32(x), _c32(wg), _c32(wu), _c32(wd)
    M, D = x.shape
    I = wg.shape[0]
    arr, keep = _slices(slices)
    g = np.empty((M, N), np.float32)
    u = np.empty((M, N), np.float32)
    inter = np.empty((M, N), np.float32)
    y = np.empty((M, D), np.float32)
    lib().orc_mlp_fwd(M, D, I, N, int(bf16), len(slices), arr, _fp(x), _fp(wg), _fp(wu), _fp(wd), _fp(g), _fp(u),
                      _fp(inter), _fp(y))
    return g, u, inter, y


def mlp_recompute(x, wg, wu, N, slices):
    """The reference's recompute_ffn rounding (src/layer_recompute_impl.inc:8-91):
    returns (gate_pre, up_pre, inter) with each slice's delta rounded to bf16
    before it is added to the bf16 base pre-activation."""
    x, wg, wu = _c32(x), _c32(wg), _c32(wu)
    M, D = x.shape
    I = wg.shape[0]
    arr, keep = _slices(slices)
    g = np.empty((M, N), np.float32)
    u = np.empty((M, N), np.float32)
    inter = np.empty((M, N), np.float32)
    lib().orc_mlp_recompute(M, D, I, N, len(slices), arr, _fp(x), _fp(wg), _fp(wu), _fp(g), _fp(u), _fp(inter))
    return g, u, inter


def mlp_bwd(x, wg, wu, wd, N, slices, g, u, inter, dy, bf16=True, want_dx=True):
    x, wg, wu, wd = _c32(x), _c32(wg), _c32(wu), _c32(wd)
    g, u, inter, dy = _c32(g), _c32(u), _c32(inter), _c32(dy)
    M, D = x.shape
    I = wg.shape[0]
    arr, keep = _slices(slices)
    grads = []
    ptrs = (_f * (3 * max(1, len(slices))))()
    for j, s in enumerate(slices):
        row = []
        for p, name in enumerate(("gate", "up", "down")):
            if s.get(name) is not None:
                a = np.zeros((s["s"], s["h"]), np.float32)
                ptrs[3 * j + p] = _fp(a)
                row.append(a)
            else:
                row.append(None)
        grads.append(row)
    dx = np.zeros((M, D), np.float32) if want_dx else None
    lib().orc_mlp_bwd(M, D, I, N, int(bf16), len(slices), arr, _fp(x), _fp(wg), _fp(wu), _fp(wd), _fp(g), _fp(u),
                      _fp(inter), _fp(dy), _fp(dx), ptrs)
    return dx, grads


# --------------------------------------------------- training-step neighbours
def masked_ce(logits, ids, ood=None, scale=1.0):
    """Masked cross-entropy over the shifted logits and grad_logits
    (reference grafting.hip:1027-1050, :1122-1135): row (b, t), t < T-1,
    against ids[b, t+1], domain mask 1 - ood[b, t+1], n = max(sum mask, 1).
    Softmax max/sum in float64; every bf16 tensor op of the reference is a
    bf16 rounding here: p = bf16(softmax), bf16(p - 1) at the label (index_put_),
    bf16(g * mask), bf16(g * (1/n)) (ATen multiplies by the reciprocal of a
    scalar divisor), bf16(g * scale); ce = -bf16(x_label - max - log(sum))
    (log_softmax + gather). Returns (grad [B,T,V] f32 with zero rows at
    t = T-1, ce [B*(T-1)], stats [loss, mean target logit, mean target prob,
    n])."""
    x = np.asarray(logits, np.float32)
    B, T, V = x.shape
    R = B * max(T - 1, 0)
    grad = np.zeros((B, T, V), np.float32)
    if R == 0:
        return grad, np.zeros(0, np.float32), np.array([0.0, 0.0, 0.0, 1.0])
    rows = x[:, :T - 1, :].reshape(R, V).astype(np.float64)
    lab = np.asarray(ids)[:, 1:].reshape(R).astype(np.int64)
    mask = (np.ones(R, np.float32) if ood is None
            else (np.asarray(ood)[:, 1:].reshape(R) == 0).astype(np.float32))
    n = np.float32(max(float(mask.sum()), 1.0))
    inv_n = np.float32(1.0) / n
    m = rows.max(axis=1, keepdims=True)
    e = np.exp(rows - m)
    s = e.sum(axis=1, keepdims=True)
    p = bf16_round((e / s).astype(np.float32))
    ar = np.arange(R)
    g = p.copy()
    g[ar, lab] = bf16_round(g[ar, lab] - np.float32(1.0))
    g = bf16_round(g * mask[:, None])
    g = bf16_round(g * inv_n)
    g = bf16_round(g * np.float32(scale))
    grad[:, :T - 1, :] = g.reshape(B, T - 1, V)
    xl = rows[ar, lab]
    ce = -bf16_round((xl - m[:, 0] - np.log(s[:, 0])).astype(np.float32))
    pl = p[ar, lab]
    stats = np.array([(ce.astype(np.float64) * mask).sum() * inv_n,
                      (xl * mask).sum() * inv_n,
                      (pl.astype(np.float64) * mask).sum() * inv_n, float(n)])
    return grad, ce, stats


def silence_energy(delta):
    """||delta_t|| / sqrt(slice) per token row, with the reference's 1e-8
    inside the root (compute_energy_kernel,
    src/kernels_elementwise_impl.inc:222-275); float64."""
    d = np.asarray(delta, np.float64)
    return np.sqrt((d * d).sum(axis=1) + 1e-8) / np.sqrt(d.shape[1])


def silence_blend(dy, delta, ood, lam):
    """dy + lambda * delta / (||delta|| sqrt(slice)) on rows with ood != 0
    (silence_blend_kernel, src/kernels_elementwise_impl.inc:8-67)."""
    d = np.asarray(delta, np.float64)
    out = np.asarray(dy, np.float64).copy()
    norm = np.sqrt((d * d).sum(axis=1) + 1e-8)
    sel = np.asarray(ood) != 0
    out[sel] += (lam / (norm[sel] * np.sqrt(d.shape[1])))[:, None] * d[sel]
    return out


def silence_blend_energy(dy_g, d_g, dy_u, d_u, ood, lam):
    """Gate and up (fused_silence_blend_energy_kernel,
    src/kernels_elementwise_impl.inc:458-560): energies e = ||d|| /
    sqrt(slice), then on rows with ood == 1 dy += lambda / (e * sqrt(slice)
    * sqrt(slice) + 1e-8) * d. Returns (dy_g, dy_u, e_g, e_u) in float64."""
    rs = np.sqrt(np.asarray(d_g).shape[1])
    outs = []
    es = []
    sel = np.asarray(ood) == 1
    for dy, d in ((dy_g, d_g), (dy_u, d_u)):
        d = np.asarray(d, np.float64)
        e = silence_energy(d)
        o = np.asarray(dy, np.float64).copy()
        o[sel] += (lam / (e[sel] * rs * rs + 1e-8))[:, None] * d[sel]
        outs.append(o)
        es.append(e)
    return outs[0], outs[1], es[0], es[1]


def lr_schedule(step, total_steps, warmup_steps, lr_peak):
    """Linear warmup then half-cosine decay in float32 arithmetic (get_lr,
    src/config.hpp:122-129); cos of the float32-rounded argument."""
    f = np.float32
    if step < warmup_steps:
        return f(f(f(lr_peak) * f(step + 1)) / f(warmup_steps))
    den = f(total_steps - warmup_steps)
    progress = f(f(step - warmup_steps) / max(den, f(1.0)))
    c = f(np.cos(np.float64(f(np.pi * np.float64(progress)))))
    return f(f(f(lr_peak) * f(f(1.0) + c)) * f(0.5))


# ---------------------------------------------------------------- model / eval
# the reference's offset basis (grafting.hip:505) is the published FNV-1a
# 64-bit basis 14695981039346656037 with its last digit missing; its hash is
# defined with it, so this one is too
FNV_BASIS = 1469598103934665603
FNV_BASIS_PUBLISHED = 14695981039346656037
FNV_PRIME = 1099511628211
_M64 = (1 << 64) - 1


def fnv1a64(data, h=FNV_BASIS):
    """64-bit FNV-1a over bytes (the reference's logits hash step,
    grafting.hip:505, :544-547)."""
    for b in bytes(data):
        h = ((h ^ b) * FNV_PRIME) & _M64
    return h


def fnv1a64_c(data, h=FNV_BASIS):
    """fnv1a64 through the C oracle (large inputs)."""
    a = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray)
                             else data.view(np.uint8).reshape(-1))
    return int(lib().orc_fnv1a64(a.ctypes.data_as(ctypes.c_void_p), a.size, h))


def eval_hash_reference(logits, h=FNV_BASIS):
    """The reference's logits hash (grafting.hip:536-546): one FNV-1a chain
    from h over the four little-endian bytes of every f32 logit, b, t, v in
    order (logits [.., V] f32 holding the bf16 values)."""
    return fnv1a64_c(np.ascontiguousarray(np.asarray(logits, np.float32).astype("<f4")), h)


EVAL_CHUNKS = 16


def eval_row_hash(row):
    """A row's hash in the library's parallel form: the row's f32 logits in
    EVAL_CHUNKS chunks of ceil(V / EVAL_CHUNKS) elements (the last ones
    shorter or empty), each chunk's bytes hashed with FNV-1a from the basis,
    then the chunk hashes' little-endian bytes hashed in chunk order."""
    b = np.asarray(row, np.float32).astype("<f4")
    L = -(-b.size // EVAL_CHUNKS)
    h = FNV_BASIS
    for c in range(EVAL_CHUNKS):
        h = fnv1a64(int(fnv1a64(b[c * L:(c + 1) * L].tobytes())).to_bytes(8, "little"), h)
    return h


def eval_stats(logits, ids, hash_in=FNV_BASIS, reference_hash=True):
    """Shadow-eval terms (reference grafting.hip:504-547): the logits hash
    continued from hash_in, either the reference's (eval_hash_reference) or
    the library's row form (each row hashed by eval_row_hash, the row
    hashes' little-endian bytes chained in row order); f64 NLL of rows
    t < T-1 against ids[b, t+1]; f64 sum and sum of squares."""
    x = np.asarray(logits, np.float32)
    B, T = np.asarray(ids).shape
    V = x.shape[-1]
    rows = x.reshape(B * T, V)
    if reference_hash:
        h = eval_hash_reference(rows, hash_in)
    else:
        h = hash_in
        for r in rows:
            h = fnv1a64(int(eval_row_hash(r)).to_bytes(8, "little"), h)
    r64 = rows.astype(np.float64)
    scored = r64.reshape(B, T, V)[:, :T - 1].reshape(-1, V)
    lab = np.asarray(ids)[:, 1:].reshape(-1)
    m = scored.max(axis=1)
    lse = m + np.log(np.exp(scored - m[:, None]).sum(axis=1))
    nll = lse - scored[np.arange(len(lab)), lab]
    return {"total_nll": float(nll.sum()), "count": int(nll.size), "logits_sum": float(r64.sum()),
            "logits_sumsq": float((r64 * r64).sum()), "logits_hash": h}


def lm_head(x, w):
    """logits = bf16(x . w^T) (at::linear on bf16, f64 accumulation here)."""
    return bf16_round((np.asarray(x, np.float64) @ np.asarray(w, np.float64).T).astype(np.float32))
