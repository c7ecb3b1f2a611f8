"""numpy/ctypes front end of the C oracle (glt_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker; never by the glt_amd package.

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
