"""Host-side operator surface of the grafted-SwiGLU path (Python mirror of
the reference's graft ops / layer / bake / norm / RoPE / optimizer entry
points), calling libglt.so through ctypes.

torch tensors are used only as device memory and for the current stream;
all arithmetic happens in the HIP kernels behind include/glt.h. Errors come
back as glt_amd._ffi.GltError (the reference throws std::runtime_error,
src/checks.hpp:10-18).
"""
import ctypes

import torch

from . import _ffi as F

PROJ_GATE, PROJ_UP, PROJ_DOWN = 0, 1, 2


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dtype_code(dtype):
    if dtype == torch.bfloat16:
        return F.DTYPE_BF16
    if dtype == torch.float32:
        return F.DTYPE_F32
    raise TypeError(f"unsupported dtype {dtype}")


def delta_offset(layer_idx, proj_idx, slice_dim, h_slice_dim):
    """Flat offset of (layer, projection) in [L*3, S, H] graft storage
    (reference src/graft_ops_impl.inc:5-7)."""
    return (layer_idx * 3 + proj_idx) * slice_dim * h_slice_dim


class GraftSlice:
    """One graft slice of one layer: placement + f32 masters [S,H] + the
    packed bf16 mirror (every orientation the GEMMs read; reference
    GraftWeights, src/types.hpp:190-201)."""

    def __init__(self, i_start, s, h_start, h, gate=None, up=None, down=None):
        self.i_start, self.s, self.h_start, self.h = int(i_start), int(s), int(h_start), int(h)
        self.gate, self.up, self.down = gate, up, down
        for t in (gate, up, down):
            if t is not None:
                assert t.dtype == torch.float32 and tuple(t.shape) == (self.s, self.h) and t.is_contiguous()
        dev = next(t.device for t in (gate, up, down) if t is not None) if any(
            t is not None for t in (gate, up, down)) else torch.device("cuda")
        nbytes = F.load().glt_graft_packed_size(self.s, self.h)
        self.packed = torch.zeros(nbytes // 2, dtype=torch.bfloat16, device=dev)

    def c_struct(self):
        return F.GraftSlice(self.i_start, self.s, self.h_start, self.h, _p(self.gate), _p(self.up), _p(self.down),
                            _p(self.packed))

    def pack(self):
        """Refresh the bf16 mirror from the masters (reference
        refresh_graft_weight_bf16, src/gemm_impl.inc:91-95)."""
        s = self.c_struct()
        F.call("glt_graft_pack", ctypes.byref(s), _p(self.packed), _stream())
        return self


def _slices_array(slices):
    arr = (F.GraftSlice * max(1, len(slices)))()
    for j, s in enumerate(slices):
        arr[j] = s.c_struct()
    return arr


class BaseMLP:
    """Frozen base weights of one MLP layer: gate/up [I,D], down [D,I], plus
    (bf16) the prepared copy the GEMMs read, made once."""

    def __init__(self, gate, up, down, prepare=True):
        self.gate, self.up, self.down = gate, up, down
        self.I, self.D = gate.shape
        self.dtype = gate.dtype
        self.prepared = None
        if prepare and self.I > 0:
            self.prepare()

    def prepare(self):
        d = F.MlpDesc(0, self.D, self.I, self.I, _dtype_code(self.dtype), 0, 0, None, None)
        nbytes = F.load().glt_base_prepared_size(ctypes.byref(d))
        if nbytes == 0:
            return self
        self.prepared = torch.empty(nbytes, dtype=torch.uint8, device=self.gate.device)
        F.call("glt_base_prepare", ctypes.byref(d), _p(self.gate), _p(self.up), _p(self.down), _p(self.prepared),
               _stream())
        return self

    def c_struct(self):
        return F.BaseWeights(_p(self.gate), _p(self.up), _p(self.down), _p(self.prepared))


def _desc(base, slices, M, N, explicit, recompute=False, state=None, residual=False, dy_f32=False):
    arr = _slices_array(slices)
    flags = ((F.MLP_EXPLICIT if explicit else 0) | (F.MLP_RECOMPUTE if recompute else 0)
             | (F.MLP_RESIDUAL if residual else 0) | (F.MLP_DY_F32 if dy_f32 else 0))
    d = F.MlpDesc(M, base.D, base.I, N, _dtype_code(base.dtype), flags, len(slices), arr,
                  ctypes.pointer(state) if state is not None else None)
    return d, arr


def mlp_forward(base, slices, x, N, explicit=True, save=True, residual=None):
    """Grafted SwiGLU forward (reference forward_layer FFN section,
    src/layer_forward_impl.inc:61-290). Returns y, gate_pre, up_pre, inter.
    With `residual` ([M,D], updated in place and returned as y) the output is
    added to it in the down GEMM's epilogue (reference x = x + ffn_out,
    src/layer_forward_impl.inc:271-275)."""
    M = x.shape[0]
    d, keep = _desc(base, slices, M, N, explicit, residual=residual is not None)
    y = residual if residual is not None else torch.empty((M, base.D), dtype=base.dtype, device=x.device)
    inter = torch.empty((M, N), dtype=base.dtype, device=x.device)
    g = torch.empty_like(inter) if save else None
    u = torch.empty_like(inter) if save else None
    b = base.c_struct()
    F.call("glt_mlp_fwd", ctypes.byref(d), ctypes.byref(b), _p(x), _p(y), _p(g), _p(u), _p(inter), _stream())
    return y, g, u, inter


def mlp_backward_workspace(base, slices, M, N, explicit=True, recompute=False):
    d, keep = _desc(base, slices, M, N, explicit, recompute)
    return F.load().glt_mlp_bwd_workspace_size(ctypes.byref(d))


def mlp_backward(base, slices, x, dy, N, gate_pre=None, up_pre=None, inter=None, want_dx=True, explicit=True,
                 recompute=False, state=None, workspace=None, norm=None, norm_in_place=False):
    """Graft-only backward (reference backward_layer FFN section,
    src/layer_backward_impl.inc:10-361). dy is [M,D] in the path dtype or
    f32 (the reference's upstream gradient, rounded once inside on the bf16
    path). Returns dx (f32) and per-slice [gate, up, down] f32 gradients in
    [S,H] storage.

    norm = (norm_x, norm_w, var, eps): x is the output of that RMSNorm
    (reference rms_norm of the FFN input); the call then also runs its
    backward on dx (glt_mlp_rmsnorm_bwd, beside the weight-gradient GEMM)
    and returns (dx, grads, norm_dx); norm_in_place writes norm_dx over dx
    (the same tensor is returned twice)."""
    M = x.shape[0]
    if norm is not None:
        want_dx = True
    d, keep = _desc(base, slices, M, N, explicit, recompute, state, dy_f32=dy.dtype == torch.float32)
    nbytes = F.load().glt_mlp_bwd_workspace_size(ctypes.byref(d))
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    dx = torch.empty((M, base.D), dtype=torch.float32, device=x.device) if want_dx else None
    grads = []
    garr = (F.GraftGrads * max(1, len(slices)))()
    for j, s in enumerate(slices):
        row = [torch.zeros((s.s, s.h), dtype=torch.float32, device=x.device) if t is not None else None
               for t in (s.gate, s.up, s.down)]
        grads.append(row)
        garr[j] = F.GraftGrads(_p(row[0]), _p(row[1]), _p(row[2]))
    b = base.c_struct()
    if norm is not None:
        norm_x, norm_w, var, eps = norm
        norm_dx = dx if norm_in_place else torch.empty((M, base.D), dtype=torch.float32, device=x.device)
        F.call("glt_mlp_rmsnorm_bwd", ctypes.byref(d), ctypes.byref(b), _p(x), _p(dy), _p(gate_pre), _p(up_pre),
               _p(inter), _p(dx), garr, _p(workspace), nbytes, _p(norm_x), _p(norm_w), _p(var), eps, _p(norm_dx),
               _stream())
        return dx, grads, norm_dx
    F.call("glt_mlp_bwd", ctypes.byref(d), ctypes.byref(b), _p(x), _p(dy), _p(gate_pre), _p(up_pre), _p(inter),
           _p(dx), garr, _p(workspace), nbytes, _stream())
    return dx, grads


def graft_gemm(kind, M, S, H, out, a=None, lda=0, delta=None, dy=None, ldo=None, alpha=1.0, beta=0.0):
    """One of the reference's six graft GEMM kinds (src/config.hpp:31-38)."""
    F.call("glt_graft_gemm", kind, M, S, H, _p(a), lda, _p(delta), _p(dy), _p(out),
           ldo if ldo is not None else out.shape[-1], alpha, beta, _stream())
    return out


def rms_norm(x, w, eps):
    """(y, variance) like the reference rms_norm (grafting.hip:116-146)."""
    M, D = x.shape
    y = torch.empty_like(x)
    var = torch.empty(M, dtype=torch.float32, device=x.device)
    F.call("glt_rmsnorm_fwd", _p(x), _p(w), _p(y), _p(var), M, D, eps, _stream())
    return y, var


def rms_norm_bwd(dy, x, w, var, eps, out=None):
    """Reference rms_norm_bwd (grafting.hip:153-172); dy f32, returns dx f32
    (into out when given, which may be dy itself)."""
    M, D = x.shape
    dx = torch.empty((M, D), dtype=torch.float32, device=x.device) if out is None else out
    F.call("glt_rmsnorm_bwd", _p(dy), _p(x), _p(w), _p(var), _p(dx), M, D, eps, _stream())
    return dx


def apply_rope(q, k, theta, pos_offset=0):
    """In-place RoPE on q [B,T,nq,hd] and k [B,T,nk,hd] (reference apply_rope,
    src/rope_impl.inc:8-39)."""
    B, T, nq, hd = q.shape
    nk = k.shape[2] if k is not None else 0
    F.call("glt_rope_fwd", _p(q), nq, _p(k), nk, B, T, hd, theta, pos_offset, _stream())


def attention(q, k, v, causal=True, scale=None):
    """Causal GQA attention forward (the reference's SDPA call in
    forward_layer, src/layer_forward_impl.inc:41-49). q [B,T,Hq,hd],
    k/v [B,T,Hkv,hd] bf16; returns [B,T,Hq,hd]."""
    B, T, Hq, hd = q.shape
    Hkv = k.shape[2]
    if scale is None:
        scale = hd ** -0.5
    out = torch.empty_like(q)
    nb = F.load().glt_attention_workspace_size(B, T, Hkv, hd)
    ws = torch.empty(nb, dtype=torch.uint8, device=q.device)
    F.call("glt_attention_fwd", _p(q), _p(k), _p(v), _p(out), B, T, Hq, Hkv, hd, scale, 1 if causal else 0,
           _p(ws), nb, _stream())
    return out


def adamw_step(w, g, m, v, step, lr, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, clip_norm=0.0,
               mirror=None):
    """One AdamW step (reference adamw_fused_kernel + optional global clip)."""
    n = w.numel()
    ws_bytes = F.load().glt_adamw_workspace_size(n)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=w.device) if clip_norm > 0 else None
    F.call("glt_adamw_step", _p(w), _p(g), _p(m), _p(v), _p(mirror), n, step, lr, beta1, beta2, eps, weight_decay,
           clip_norm, _p(ws), ws_bytes if ws is not None else 0, _stream())


def adamw_graft_step(slices, grads, m, v, step, lr, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
                     proj_mask=7, clip_norm=0.0, workspace=None):
    """AdamW over graft slices with the packed-mirror refresh fused in and
    the optional global-L2 clip over all of their gradients (reference
    grafting.hip:1149-1164, clip 1.0 by default there).
    grads/m/v: per slice a flat f32 [3*S*H] tensor (gate, up, down)."""
    arr = _slices_array(slices)
    nbytes = F.load().glt_adamw_workspace_size(0)
    if clip_norm > 0 and workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=grads[0].device)
    F.call("glt_adamw_graft_step", arr, len(slices), F.ptr_array([g.data_ptr() for g in grads]),
           F.ptr_array([t.data_ptr() for t in m]), F.ptr_array([t.data_ptr() for t in v]),
           F.ptr_array([s.packed.data_ptr() for s in slices]), proj_mask, step, lr, beta1, beta2, eps,
           weight_decay, clip_norm, _p(workspace), nbytes if workspace is not None else 0, _stream())


def shadow_bake(state, gate, up, down, grafts, placements, *, D, I, N=None, materialize=False, gate_out=None,
                up_out=None, down_out=None, layer_start=0, layer_end=None, proj_mask=7, graft_dtype=None):
    """Bake graft deltas into bf16 base matrices (reference
    apply_graft_to_shadow, src/shadow_bake_impl.inc:58-128).

    gate/up/down: per-layer lists of bf16 tensors; grafts[j][l]: slice j's
    flat [3,S,H] deltas for layer l; placements[j] = (i0, S, h0, H)."""
    L = len(gate)
    n_sl = len(placements)
    if graft_dtype is None:
        graft_dtype = grafts[0][0].dtype if n_sl else torch.float32
    pl = (ctypes.c_int32 * max(1, 4 * n_sl))(*[int(v) for p in placements for v in p])
    gptr = F.ptr_array([grafts[j][l].data_ptr() for j in range(n_sl) for l in range(L)])
    d = F.BakeDesc(F.BAKE_MATERIALIZE if materialize else F.BAKE_IN_PLACE, L, layer_start,
                   L - 1 if layer_end is None else layer_end, proj_mask, D, I, N if N is not None else I,
                   _dtype_code(graft_dtype), n_sl, pl, gptr)

    def arr(ts):
        return F.ptr_array([t.data_ptr() for t in ts]) if ts is not None else None

    F.call("glt_shadow_bake", ctypes.byref(d), ctypes.byref(state), arr(gate), arr(up), arr(down), arr(gate_out),
           arr(up_out), arr(down_out), _stream())


def f32_to_bf16(x):
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    F.call("glt_f32_to_bf16", _p(x), _p(out), x.numel(), _stream())
    return out


def fill_normal(t, seed, tensor_id, mean=0.0, std=1.0):
    F.call("glt_fill_normal", _p(t), _dtype_code(t.dtype), t.numel(), seed, tensor_id, mean, std, _stream())
    return t


def silu_mul(g, u):
    out = torch.empty_like(g)
    F.call("glt_silu_mul", _p(g), _p(u), _p(out), g.numel(), _stream())
    return out


def gate_up_bwd(gi, g, u):
    dg = torch.empty(gi.shape, dtype=torch.float32, device=gi.device)
    du = torch.empty_like(dg)
    F.call("glt_gate_up_bwd", _p(gi), _p(g), _p(u), _p(dg), _p(du), gi.numel(), _stream())
    return dg, du


class DecoderLayer:
    """One decoder layer with the grafted MLP (reference forward_layer,
    src/layer_forward_impl.inc:15-290) over glt_layer_fwd. Projection weights
    bf16 [out, in]; base is the MLP's BaseMLP; slices its graft slices."""

    def __init__(self, B, T, n_q_heads, n_kv_heads, wq, wk, wv, wo, ln_in, ln_post, base, slices, N,
                 rope_theta=500000.0, rms_eps=1e-5, explicit=True, head_dim=128):
        self.base, self.slices = base, slices
        md, self._keep = _desc(base, slices, B * T, N, explicit)
        self.desc = F.LayerDesc(B, T, n_q_heads, n_kv_heads, head_dim, rope_theta, rms_eps, md)
        self._w = (wq, wk, wv, wo, ln_in, ln_post)
        self.prepared = torch.empty(F.load().glt_attn_prepared_size(ctypes.byref(self.desc)), dtype=torch.uint8,
                                    device=wq.device)
        self.weights = F.LayerWeights(_p(wq), _p(wk), _p(wv), _p(wo), _p(ln_in), _p(ln_post), _p(self.prepared),
                                      base.c_struct())
        F.call("glt_attn_prepare", ctypes.byref(self.desc), ctypes.byref(self.weights), _p(self.prepared), _stream())
        self.ws = torch.empty(F.load().glt_layer_fwd_workspace_size(ctypes.byref(self.desc)), dtype=torch.uint8,
                              device=wq.device)

    def forward(self, x, inter=None):
        """x [B*T, D] bf16, updated in place; returns (x, x_ffn, ffn_var)."""
        M, D = x.shape
        x_ffn = torch.empty_like(x)
        var = torch.empty(M, dtype=torch.float32, device=x.device)
        F.call("glt_layer_fwd", ctypes.byref(self.desc), ctypes.byref(self.weights), _p(x), _p(x_ffn), _p(var),
               None, None, _p(inter), _p(self.ws), self.ws.numel(), _stream())
        return x, x_ffn, var


def _grft_info(num_layers, S, H, hidden_dim=0, domain_id=0, session_id=""):
    return F.GrftInfo(num_layers, S, H, hidden_dim, domain_id, session_id.encode() if session_id else None)


def grft_save(path, weight, num_layers, S, H, hidden_dim=0, domain_id=0, session_id=""):
    """Writes the flat f32 graft storage [num_layers*3*S*H] (device or host
    tensor) as a GRFT checkpoint (reference save_safetensors,
    src/checkpoint_impl.inc:39-97)."""
    info = _grft_info(num_layers, S, H, hidden_dim, domain_id, session_id)
    F.call("glt_grft_save", str(path).encode(), ctypes.byref(info), _p(weight), int(weight.is_cuda),
           _stream() if weight.is_cuda else None)


def grft_load(path, weight, num_layers, S, H, domain_id=0, session_id="", raw_f32=False):
    """Loads a GRFT checkpoint (reference load_safetensors_checkpoint,
    src/checkpoint_impl.inc:170-285) or, with raw_f32, an --init-deltas file
    into the f32 storage tensor `weight` (device or host)."""
    info = _grft_info(num_layers, S, H, 0, domain_id, session_id)
    F.call("glt_grft_load_raw_f32" if raw_f32 else "glt_grft_load", str(path).encode(), ctypes.byref(info),
           _p(weight), int(weight.is_cuda), _stream() if weight.is_cuda else None)
    return weight

def masked_ce(logits, ids, ood=None, scale=1.0, grad=None, want_grad=True, ce_per_token=False):
    """Masked cross-entropy over the shifted logits and its gradient
    (reference loss grafting.hip:1027-1050, grad_logits :1122-1135).
    logits [B,T,V] bf16, ids [B,T] int32, ood [B,T] int32 or None.
    Returns (stats [loss, target-logit mean, target-prob mean, n] f32 on the
    device, grad [B,T,V] bf16 or None, ce [B*(T-1)] f32 or None). Pass
    grad=logits to overwrite the logits with the gradient."""
    B, T, V = logits.shape
    dev = logits.device
    stats = torch.empty(4, dtype=torch.float32, device=dev)
    if want_grad and grad is None:
        grad = torch.empty_like(logits)
    ce = torch.empty(max(B * (T - 1), 1), dtype=torch.float32, device=dev) if ce_per_token else None
    nbytes = F.load().glt_masked_ce_workspace_size(B, T)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    F.call("glt_masked_ce", _p(logits), logits.stride(1), _p(ids), _p(ood), B, T, V, scale,
           _p(grad) if want_grad else None, grad.stride(1) if want_grad else 0, _p(ce), _p(stats), _p(ws), nbytes,
           _stream())
    return stats, (grad if want_grad else None), ce


def silence_energy(delta, ld=None):
    """Per-token energy ||delta_t|| / sqrt(slice) of [tokens, slice] f32 or
    bf16 rows (reference compute_energy_kernel)."""
    tokens, slice_ = delta.shape
    out = torch.empty(tokens, dtype=torch.float32, device=delta.device)
    dt = F.DTYPE_F32 if delta.dtype == torch.float32 else F.DTYPE_BF16
    F.call("glt_silence_energy", _p(delta), dt, ld if ld is not None else delta.stride(0), tokens, slice_, _p(out),
           _stream())
    return out


def silence_blend(dy, delta, ood, lam):
    """In place: dy += lam * delta / (||delta|| sqrt(slice)) on OOD tokens
    (reference silence_blend_kernel)."""
    tokens, slice_ = delta.shape
    F.call("glt_silence_blend", _p(dy), _p(delta), _p(ood), tokens, slice_, lam, _stream())
    return dy


def silence_blend_energy(dy_gate, delta_gate, dy_up, delta_up, ood, lam, energies=True):
    """Gate and up silence blend with their energies (reference
    fused_silence_blend_energy_kernel); returns (energy_gate, energy_up)."""
    tokens, slice_ = delta_gate.shape
    eg = torch.empty(tokens, dtype=torch.float32, device=dy_gate.device) if energies else None
    eu = torch.empty(tokens, dtype=torch.float32, device=dy_gate.device) if energies else None
    F.call("glt_silence_blend_energy", _p(dy_gate), _p(delta_gate), _p(dy_up), _p(delta_up), _p(eg), _p(eu), _p(ood),
           tokens, slice_, lam, _stream())
    return eg, eu


def lr_schedule(step, total_steps, warmup_steps, lr_peak):
    """Warmup + cosine learning rate (reference get_lr, src/config.hpp:122-129)."""
    return F.load().glt_lr_schedule(step, total_steps, warmup_steps, lr_peak)


class SafetensorsModel:
    """Base-model weights in safetensors files (reference
    load_base_model_safetensors, src/model_io_impl.inc:57-190): a file or a
    directory of *.safetensors, memory-mapped by the library."""

    def __init__(self, path):
        self._h = ctypes.c_void_p()
        F.call("glt_st_open", str(path).encode(), ctypes.byref(self._h))

    def close(self):
        if self._h:
            F.load().glt_st_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __len__(self):
        return F.load().glt_st_count(self._h)

    def info(self, name):
        """(dtype code, shape) of tensor `name`."""
        dt, nd = ctypes.c_int32(), ctypes.c_int32()
        shape = (ctypes.c_int64 * 8)()
        F.call("glt_st_info", self._h, name.encode(), ctypes.byref(dt), ctypes.byref(nd), shape)
        return dt.value, tuple(shape[i] for i in range(nd.value))

    def read(self, name, dtype=torch.bfloat16, transpose=False, device="cuda"):
        """Tensor `name` as bf16 or f32, optionally transposed (2-D)."""
        _, shape = self.info(name)
        if transpose:
            shape = shape[::-1]
        out = torch.empty(shape, dtype=dtype, device=device)
        on_dev = out.is_cuda
        F.call("glt_st_read", self._h, name.encode(), _p(out), F.DTYPE_F32 if dtype == torch.float32 else F.DTYPE_BF16,
               int(transpose), int(on_dev), _stream() if on_dev else None)
        return out

    def load_layer(self, layer, D, I, n_q_heads, n_kv_heads, head_dim, device="cuda"):
        """The nine bf16 weights of decoder layer `layer` (names and shapes of
        the reference's loader); returns a dict."""
        nq, nk = n_q_heads * head_dim, n_kv_heads * head_dim
        shapes = {"q_proj": (nq, D), "k_proj": (nk, D), "v_proj": (nk, D), "o_proj": (D, nq), "ln_in": (D,),
                  "ln_post": (D,), "gate": (I, D), "up": (I, D), "down": (D, I)}
        out = {k: torch.empty(v, dtype=torch.bfloat16, device=device) for k, v in shapes.items()}
        bufs = F.LayerBuffers(*[out[k].data_ptr() for k in shapes])
        md = F.MlpDesc(1, D, I, I, F.DTYPE_BF16, 0, 0, None, None)
        ld = F.LayerDesc(1, 1, n_q_heads, n_kv_heads, head_dim, 0.0, 1e-5, md)
        on_dev = torch.device(device).type == "cuda"
        F.call("glt_st_load_layer", self._h, layer, ctypes.byref(ld), ctypes.byref(bufs), int(on_dev),
               _stream() if on_dev else None)
        return out

    def load_head(self, V, D, device="cuda"):
        """(embed [V,D], final norm [D], lm_head [V,D]) as bf16; lm_head tied
        to the embedding when the files have none."""
        embed = torch.empty((V, D), dtype=torch.bfloat16, device=device)
        norm = torch.empty(D, dtype=torch.bfloat16, device=device)
        head = torch.empty((V, D), dtype=torch.bfloat16, device=device)
        on_dev = embed.is_cuda
        F.call("glt_st_load_head", self._h, V, D, _p(embed), _p(norm), _p(head), int(on_dev),
               _stream() if on_dev else None)
        return embed, norm, head


class Model:
    """forward_model (reference grafting.hip:224-271) over DecoderLayer
    objects: embedding, the layers, final RMSNorm, LM head. embed / lm_head
    [V,D] bf16, final_norm [D] bf16."""

    def __init__(self, layers, embed, final_norm, lm_head=None):
        self.layers = layers
        self.embed, self.final_norm = embed, final_norm
        self.lm_head = embed if lm_head is None else lm_head      # tied when absent
        self.V, self.D = self.lm_head.shape
        lib = F.load()
        self.lm_prepared = torch.empty(lib.glt_lm_head_prepared_size(self.V, self.D), dtype=torch.uint8,
                                       device=self.lm_head.device)
        F.call("glt_lm_head_prepare", _p(self.lm_head), self.V, self.D, _p(self.lm_prepared), _stream())
        n = len(layers)
        self._descs = (F.LayerDesc * n)(*[l.desc for l in layers])
        self._weights = (F.LayerWeights * n)(*[l.weights for l in layers])

    def _c(self, explicit):
        return F.Model(len(self.layers), self.V, int(explicit), self._descs, self._weights, _p(self.embed),
                       _p(self.final_norm), _p(self.lm_head), _p(self.lm_prepared))

    def forward(self, ids, explicit=True):
        """ids [B,T] int32 on the device; returns logits [B*T, V] bf16."""
        m = self._c(explicit)
        M = ids.numel()
        logits = torch.empty((M, self.V), dtype=torch.bfloat16, device=ids.device)
        nbytes = F.load().glt_model_fwd_workspace_size(ctypes.byref(m))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=ids.device)
        F.call("glt_model_fwd", ctypes.byref(m), _p(ids), _p(logits), _p(ws), nbytes, _stream())
        return logits


def lm_head_fwd(x, lm_head, prepared=None):
    """logits [M,V] = x [M,D] . lm_head^T (at::linear), bf16."""
    V, D = lm_head.shape
    if prepared is None:
        prepared = torch.empty(F.load().glt_lm_head_prepared_size(V, D), dtype=torch.uint8, device=x.device)
        F.call("glt_lm_head_prepare", _p(lm_head), V, D, _p(prepared), _stream())
    out = torch.empty((x.shape[0], V), dtype=torch.bfloat16, device=x.device)
    F.call("glt_lm_head_fwd", _p(x), x.shape[0], D, _p(lm_head), _p(prepared), V, _p(out), _stream())
    return out


def lm_head_bwd(grad, lm_head, prepared=None):
    """dx [M,D] f32 = grad [M,V] . lm_head (the reference's grad_logits_full @
    lm_head, grafting.hip:1137)."""
    V, D = lm_head.shape
    if prepared is None:
        prepared = torch.empty(F.load().glt_lm_head_prepared_size(V, D), dtype=torch.uint8, device=grad.device)
        F.call("glt_lm_head_prepare", _p(lm_head), V, D, _p(prepared), _stream())
    dx = torch.empty((grad.shape[0], D), dtype=torch.float32, device=grad.device)
    F.call("glt_lm_head_bwd", _p(grad), grad.shape[0], V, _p(lm_head), _p(prepared), D, _p(dx), _stream())
    return dx


def embedding(ids, table):
    """table[ids] (at::embedding) for int32 ids, bf16 table [V,D]."""
    V, D = table.shape
    out = torch.empty((ids.numel(), D), dtype=torch.bfloat16, device=ids.device)
    F.call("glt_embedding", _p(ids), ids.numel(), _p(table), V, D, _p(out), _stream())
    return out


def eval_stats(logits, ids, hash_in=F.FNV_BASIS, reference_hash=True):
    """Shadow-eval terms of one batch (reference grafting.hip:504-547):
    dict(total_nll, count, ce, logits_sum, logits_sumsq, logits_hash).
    The hash is the reference's FNV-1a chain over every f32 logit byte,
    continued from hash_in (pass the previous batch's logits_hash to chain
    batches as the reference does); reference_hash=False gives the library's
    one-pass row form instead."""
    B, T = ids.shape
    V = logits.shape[-1]
    assert logits.stride(-1) == 1, "logits rows must be contiguous"
    ld = logits.stride(-2)
    lib = F.load()
    nbytes = lib.glt_eval_stats_workspace_size(B, T)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=logits.device)
    r = F.EvalResult()
    F.call("glt_eval_stats", _p(logits), ld, _p(ids), B, T, V,
           F.EVAL_HASH_REFERENCE if reference_hash else F.EVAL_HASH_ROWS, hash_in, ctypes.byref(r), _p(ws), nbytes,
           _stream())
    return {"total_nll": r.total_nll, "count": r.count, "ce": r.total_nll / max(r.count, 1),
            "logits_sum": r.logits_sum, "logits_sumsq": r.logits_sumsq, "logits_hash": r.logits_hash}


def eval_batches(batches, reference_hash=True):
    """The reference's whole eval loop over several (logits, ids) batches
    (grafting.hip:504-547): nll and counts summed, the logits hash chained
    from the FNV basis through every batch; returns the eval_stats dict of
    the whole set (ce = total_nll / count)."""
    out = {"total_nll": 0.0, "count": 0, "logits_sum": 0.0, "logits_sumsq": 0.0, "logits_hash": F.FNV_BASIS}
    for logits, ids in batches:
        r = eval_stats(logits, ids, out["logits_hash"], reference_hash)
        for k in ("total_nll", "count", "logits_sum", "logits_sumsq"):
            out[k] += r[k]
        out["logits_hash"] = r["logits_hash"]
    out["ce"] = out["total_nll"] / max(out["count"], 1)
    return out


def certify(A, B, C, D, ce_improve_margin=0.0, eps_ce_bake=0.02, eps_ce_reload=1e-4):
    """The A/B/C/D gates of the reference's certify step (deploy/certify.sh:28-59;
    default margins deploy/config.sh:39-41) over eval results (dicts with "ce"
    and "logits_hash"): A base, B explicit graft, C shadow-baked, D freshly
    reloaded base."""
    g1 = B["ce"] < A["ce"] - ce_improve_margin
    gap = C["ce"] - B["ce"]
    g2 = abs(gap) < eps_ce_bake
    g3 = abs(D["ce"] - A["ce"]) < eps_ce_reload and A["logits_hash"] == D["logits_hash"]
    content = "A_STANDALONE_DELTAS" if (g1 and g2) else ("B_BAKED_MISLABEL_SUSPECT" if g2 else "UNKNOWN")
    return {"A_ce": A["ce"], "B_ce": B["ce"], "C_ce": C["ce"], "D_ce": D["ce"], "A_hash": A["logits_hash"],
            "D_hash": D["logits_hash"], "gate_improve": int(g1), "gate_bake_equal": int(g2),
            "gate_reload_equal": int(g3), "bake_ce_gap": gap, "eps_ce_bake": eps_ce_bake, "content": content,
            "pass": int(g1 and g2 and g3)}
