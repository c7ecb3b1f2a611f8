"""The C-ABI library loads and exports every entry point include/glt.h
declares (no GPU calls)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "glt.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(glt_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_surface():
    names = declared_functions()
    for n in ("glt_mlp_fwd", "glt_mlp_bwd", "glt_shadow_bake", "glt_rmsnorm_fwd", "glt_rmsnorm_bwd", "glt_rope_fwd",
              "glt_adamw_step", "glt_graft_gemm", "glt_silu_mul", "glt_gate_up_bwd", "glt_f32_to_bf16"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from glt_amd import _ffi
    lib = ctypes.CDLL(_ffi.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(_ffi.SIGNATURES), "ctypes binding out of sync with glt.h"


def test_version_and_error_string():
    from glt_amd import _ffi
    lib = _ffi.load()
    assert lib.glt_version() == 4
    assert isinstance(lib.glt_last_error_string(), bytes)


def test_host_validation_errors_without_gpu():
    """Descriptor checks run before any GPU call and return distinct codes."""
    from glt_amd import _ffi as F
    lib = F.load()
    st = F.ModelState(1)
    d = F.MlpDesc(16, 64, 64, 64, F.DTYPE_BF16, F.MLP_EXPLICIT, 0, None, ctypes.pointer(st))
    w = F.BaseWeights(1, 1, 1, 1)
    rc = lib.glt_mlp_bwd(ctypes.byref(d), ctypes.byref(w), 1, 1, 1, 1, 1, None, None, None, 0, None)
    assert rc == 7  # GLT_ERR_BAKED_NO_BACKWARD (reference src/layer_backward_impl.inc:11-13)
    bd = F.BakeDesc(0, 1, 0, 0, 7, 64, 64, 64, F.DTYPE_F32, 0, None, None)
    assert lib.glt_shadow_bake(ctypes.byref(bd), ctypes.byref(st), None, None, None, None, None, None, None) == 6
    # attention supports head_dim 128 only; refused before any GPU call
    assert lib.glt_attention_fwd(1, 1, 1, 1, 1, 16, 4, 1, 64, 0.125, 1, None, 0, None) == 9  # GLT_ERR_UNSUPPORTED
    # the transposed-V workspace: B x Hkv x 128 x (T rounded up to 64) bf16; refused when short
    assert lib.glt_attention_workspace_size(2, 100, 4, 128) == 2 * 4 * 128 * 128 * 2
    assert lib.glt_attention_fwd(16, 16, 16, 16, 1, 16, 4, 1, 128, 0.125, 1, None, 0, None) == 5  # GLT_ERR_WORKSPACE
    d2 = F.MlpDesc(16, 64, 128, 64, F.DTYPE_BF16, 0, 0, None, None)  # N < I
    assert lib.glt_mlp_fwd(ctypes.byref(d2), ctypes.byref(w), 1, 1, None, None, 1, None) == 2
    d3 = F.MlpDesc(16, 64, 64, 64, 7, 0, 0, None, None)
    assert lib.glt_mlp_fwd(ctypes.byref(d3), ctypes.byref(w), 1, 1, None, None, 1, None) == 3
    assert lib.glt_rmsnorm_fwd(None, None, None, None, -1, 8, 1e-5, None) == 2
    assert lib.glt_graft_gemm(9, 1, 1, 1, None, 0, None, None, None, 0, 1.0, 0.0, None) == 1
    assert lib.glt_adamw_step(1, 1, 1, 1, None, 10, 0, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1.0, None, 0, None) == 5


def test_mlp_rmsnorm_bwd_validation_without_gpu():
    """The fused FFN + RMSNorm backward refuses a missing descriptor, a
    missing dx or norm operand and the f32 path before any GPU call."""
    from glt_amd import _ffi as F
    lib = F.load()
    desc = F.MlpDesc(16, 64, 64, 64, F.DTYPE_BF16, F.MLP_EXPLICIT, 0, None, None)
    base = F.BaseWeights(16, 16, 16, None)
    args = (ctypes.byref(base), 16, 16, 16, 16, 16)
    tail = (None, None, 0)
    assert lib.glt_mlp_rmsnorm_bwd(None, *args, 16, *tail, 16, 16, 16, 1e-5, 16, None) == 1
    assert lib.glt_mlp_rmsnorm_bwd(ctypes.byref(desc), *args, None, *tail, 16, 16, 16, 1e-5, 16, None) == 1
    assert lib.glt_mlp_rmsnorm_bwd(ctypes.byref(desc), *args, 16, *tail, 16, None, 16, 1e-5, 16, None) == 1
    desc32 = F.MlpDesc(16, 64, 64, 64, F.DTYPE_F32, F.MLP_EXPLICIT, 0, None, None)
    assert lib.glt_mlp_rmsnorm_bwd(ctypes.byref(desc32), *args, 16, *tail, 16, 16, 16, 1e-5, 16, None) == 3


def test_eval_and_graft_adamw_validation_without_gpu():
    """glt_eval_stats and the graft AdamW step refuse bad requests, and pass
    an empty batch through, before any GPU call."""
    from glt_amd import _ffi as F
    lib = F.load()
    res = F.EvalResult()
    h = 0x0123456789ABCDEF
    assert lib.glt_eval_stats(1, 8, 1, 1, 2, 8, 5, h, ctypes.byref(res), None, 0, None) == 1   # hash mode
    assert lib.glt_eval_stats(1, 4, 1, 1, 2, 8, 0, h, ctypes.byref(res), None, 0, None) == 2   # row stride < V
    assert lib.glt_eval_stats(1, 8, 1, 1, 2, 8, 0, h, ctypes.byref(res), None, 0, None) == 5   # no workspace
    # no rows: the running hash passes through unchanged (the reference's
    # chain over an empty batch), nothing counted
    assert lib.glt_eval_stats(None, 8, None, 0, 2, 8, 0, h, ctypes.byref(res), None, 0, None) == 0
    assert res.logits_hash == h and res.count == 0 and res.total_nll == 0.0
    # graft AdamW: a negative slice count (either form); a clip over more
    # projections than it has partial sums (171 slices x 3 > 512), refused
    # before any launch; the clip without its workspace
    sl = (F.GraftSlice * 171)()
    for j in range(171):
        sl[j].s, sl[j].h = 64, 64
        sl[j].master_gate = sl[j].master_up = sl[j].master_down = 4096
    arr = F.ptr_array([4096] * 171)
    args = (sl, -1, arr, arr, arr, None, 7, 0, 1e-4, 0.9, 0.999, 1e-8, 0.01)
    assert lib.glt_adamw_graft_step(*args, 0.0, None, 0, None) == 2
    assert lib.glt_adamw_graft_step_noalloc(*args, 0.0, None) == 2
    assert lib.glt_adamw_graft_step(sl, 171, arr, arr, arr, None, 7, 0, 1e-4, 0.9, 0.999, 1e-8, 0.01, 1.0,
                                    ctypes.c_void_p(4096), 1 << 20, None) == 9
    assert lib.glt_adamw_graft_step(sl, 1, arr, arr, arr, None, 7, 0, 1e-4, 0.9, 0.999, 1e-8, 0.01, 1.0, None, 0,
                                    None) == 5
