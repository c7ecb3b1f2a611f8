"""ctypes binding of libglt.so (include/glt.h).

The library is built in-tree by glt_amd/build.py; importing this module
fails loudly when it is missing. Structures mirror include/glt.h field for
field.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libglt.so")

GLT_OK = 0
STATUS_NAMES = {
    0: "GLT_OK", 1: "GLT_ERR_INVALID_ARG", 2: "GLT_ERR_SHAPE", 3: "GLT_ERR_DTYPE",
    4: "GLT_ERR_ALIGNMENT", 5: "GLT_ERR_WORKSPACE", 6: "GLT_ERR_ALREADY_BAKED",
    7: "GLT_ERR_BAKED_NO_BACKWARD", 8: "GLT_ERR_HIP", 9: "GLT_ERR_UNSUPPORTED", 10: "GLT_ERR_IO",
    11: "GLT_ERR_FORMAT", 12: "GLT_ERR_NOT_FOUND",
}
DTYPE_BF16, DTYPE_F32, DTYPE_F16 = 0, 1, 2
MLP_EXPLICIT, MLP_RECOMPUTE, MLP_RESIDUAL, MLP_DY_F32 = 1, 2, 4, 8
FNV_BASIS = 1469598103934665603
EVAL_HASH_REFERENCE, EVAL_HASH_ROWS = 0, 1
BAKE_IN_PLACE, BAKE_MATERIALIZE = 0, 1
GEMM_EXPAND_FWD, GEMM_CONTRACT_FWD, GEMM_EXPAND_WGRAD, GEMM_CONTRACT_WGRAD, GEMM_EXPAND_IGRAD, \
    GEMM_CONTRACT_IGRAD = range(6)

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t


class ModelState(ctypes.Structure):
    _fields_ = [("baked", _i32)]


class GraftSlice(ctypes.Structure):
    _fields_ = [("i_start", _i32), ("s", _i32), ("h_start", _i32), ("h", _i32),
                ("master_gate", _vp), ("master_up", _vp), ("master_down", _vp), ("packed", _vp)]


class GraftGrads(ctypes.Structure):
    _fields_ = [("gate", _vp), ("up", _vp), ("down", _vp)]


class BaseWeights(ctypes.Structure):
    _fields_ = [("gate", _vp), ("up", _vp), ("down", _vp), ("prepared", _vp)]


class MlpDesc(ctypes.Structure):
    _fields_ = [("M", _i32), ("D", _i32), ("I", _i32), ("N", _i32), ("dtype", _i32), ("flags", _i32),
                ("n_slices", _i32), ("slices", ctypes.POINTER(GraftSlice)), ("state", ctypes.POINTER(ModelState))]


class BakeDesc(ctypes.Structure):
    _fields_ = [("mode", _i32), ("num_layers", _i32), ("layer_start", _i32), ("layer_end", _i32),
                ("proj_mask", _i32), ("D", _i32), ("I", _i32), ("N", _i32), ("graft_dtype", _i32),
                ("n_slices", _i32), ("placement", ctypes.POINTER(_i32)), ("graft", ctypes.POINTER(_vp))]


class GrftInfo(ctypes.Structure):
    _fields_ = [("num_layers", _i32), ("S", _i32), ("H", _i32), ("hidden_dim", _i32), ("domain_id", _i32),
                ("session_id", ctypes.c_char_p)]


class LayerDesc(ctypes.Structure):
    _fields_ = [("B", _i32), ("T", _i32), ("n_q_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32),
                ("rope_theta", _f32), ("rms_eps", _f32), ("mlp", MlpDesc)]


class LayerWeights(ctypes.Structure):
    _fields_ = [("q_proj", _vp), ("k_proj", _vp), ("v_proj", _vp), ("o_proj", _vp), ("ln_in", _vp),
                ("ln_post", _vp), ("prepared", _vp), ("mlp", BaseWeights)]


class Model(ctypes.Structure):
    _fields_ = [("num_layers", _i32), ("V", _i32), ("use_explicit_graft", _i32), ("descs", ctypes.POINTER(LayerDesc)),
                ("layers", ctypes.POINTER(LayerWeights)), ("embed", _vp), ("final_norm", _vp), ("lm_head", _vp),
                ("lm_head_prepared", _vp)]


class EvalResult(ctypes.Structure):
    _fields_ = [("total_nll", ctypes.c_double), ("count", _i64), ("logits_sum", ctypes.c_double),
                ("logits_sumsq", ctypes.c_double), ("logits_hash", ctypes.c_uint64)]


class LayerBuffers(ctypes.Structure):
    _fields_ = [("q_proj", _vp), ("k_proj", _vp), ("v_proj", _vp), ("o_proj", _vp), ("ln_in", _vp),
                ("ln_post", _vp), ("gate", _vp), ("up", _vp), ("down", _vp)]


# name -> (restype, argtypes): every entry point declared in include/glt.h
SIGNATURES = {
    "glt_version": (_i32, []),
    "glt_last_error_string": (ctypes.c_char_p, []),
    "glt_device_info": (_i32, [_i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_i64)]),
    "glt_profile_enable": (_i32, [_i32]),
    "glt_profile_collect": (_i32, [ctypes.c_char_p, _sz, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64),
                                   _i32]),
    "glt_f32_to_bf16": (_i32, [_vp, _vp, _i64, _vp]),
    "glt_fill_normal": (_i32, [_vp, _i32, _i64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double,
                               ctypes.c_double, _vp]),
    "glt_graft_packed_size": (_sz, [_i32, _i32]),
    "glt_graft_pack": (_i32, [ctypes.POINTER(GraftSlice), _vp, _vp]),
    "glt_transpose": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp]),
    "glt_base_prepared_size": (_sz, [ctypes.POINTER(MlpDesc)]),
    "glt_base_prepare": (_i32, [ctypes.POINTER(MlpDesc), _vp, _vp, _vp, _vp, _vp]),
    "glt_graft_gemm": (_i32, [_i32, _i32, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i64, _f32, _f32, _vp]),
    "glt_mlp_fwd": (_i32, [ctypes.POINTER(MlpDesc), ctypes.POINTER(BaseWeights), _vp, _vp, _vp, _vp, _vp, _vp]),
    "glt_mlp_bwd_workspace_size": (_sz, [ctypes.POINTER(MlpDesc)]),
    "glt_mlp_bwd": (_i32, [ctypes.POINTER(MlpDesc), ctypes.POINTER(BaseWeights), _vp, _vp, _vp, _vp, _vp, _vp,
                           ctypes.POINTER(GraftGrads), _vp, _sz, _vp]),
    "glt_mlp_rmsnorm_bwd": (_i32, [ctypes.POINTER(MlpDesc), ctypes.POINTER(BaseWeights), _vp, _vp, _vp, _vp, _vp,
                                   _vp, ctypes.POINTER(GraftGrads), _vp, _sz, _vp, _vp, _vp, _f32, _vp, _vp]),
    "glt_silu_mul": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "glt_gate_up_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "glt_rmsnorm_fwd": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "glt_rmsnorm_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "glt_rope_fwd": (_i32, [_vp, _i32, _vp, _i32, _i32, _i32, _i32, _f32, _i32, _vp]),
    "glt_attention_fwd": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _vp, _sz, _vp]),
    "glt_attention_workspace_size": (_sz, [_i32, _i32, _i32, _i32]),
    "glt_grft_save": (_i32, [ctypes.c_char_p, ctypes.POINTER(GrftInfo), _vp, _i32, _vp]),
    "glt_grft_load": (_i32, [ctypes.c_char_p, ctypes.POINTER(GrftInfo), _vp, _i32, _vp]),
    "glt_grft_load_raw_f32": (_i32, [ctypes.c_char_p, ctypes.POINTER(GrftInfo), _vp, _i32, _vp]),
    "glt_attn_prepared_size": (_sz, [ctypes.POINTER(LayerDesc)]),
    "glt_attn_prepare": (_i32, [ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerWeights), _vp, _vp]),
    "glt_layer_fwd_workspace_size": (_sz, [ctypes.POINTER(LayerDesc)]),
    "glt_layer_fwd": (_i32, [ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerWeights), _vp, _vp, _vp, _vp, _vp, _vp,
                             _vp, _sz, _vp]),
    "glt_adamw_workspace_size": (_sz, [_i64]),
    "glt_adamw_step": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _f32, _f32, _f32, _f32, _f32, _f32, _vp, _sz,
                              _vp]),
    "glt_adamw_graft_step": (_i32, [ctypes.POINTER(GraftSlice), _i32, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                    ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i32, _i32, _f32, _f32, _f32, _f32,
                                    _f32, _f32, _vp, _sz, _vp]),
    "glt_adamw_graft_step_noalloc": (_i32, [ctypes.POINTER(GraftSlice), _i32, ctypes.POINTER(_vp),
                                            ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i32, _i32,
                                            _f32, _f32, _f32, _f32, _f32, _f32, _vp]),
    "glt_shadow_bake": (_i32, [ctypes.POINTER(BakeDesc), ctypes.POINTER(ModelState), ctypes.POINTER(_vp),
                               ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                               ctypes.POINTER(_vp), _vp]),
    "glt_embedding": (_i32, [_vp, _i64, _vp, _i32, _i32, _vp, _vp]),
    "glt_lm_head_prepared_size": (_sz, [_i32, _i32]),
    "glt_lm_head_prepare": (_i32, [_vp, _i32, _i32, _vp, _vp]),
    "glt_lm_head_fwd": (_i32, [_vp, _i32, _i32, _vp, _vp, _i32, _vp, _vp]),
    "glt_lm_head_bwd": (_i32, [_vp, _i32, _i32, _vp, _vp, _i32, _vp, _vp]),
    "glt_model_fwd_workspace_size": (_sz, [ctypes.POINTER(Model)]),
    "glt_model_fwd": (_i32, [ctypes.POINTER(Model), _vp, _vp, _vp, _sz, _vp]),
    "glt_eval_stats_workspace_size": (_sz, [_i32, _i32]),
    "glt_eval_stats": (_i32, [_vp, _i64, _vp, _i32, _i32, _i32, _i32, ctypes.c_uint64, ctypes.POINTER(EvalResult),
                              _vp, _sz, _vp]),
    "glt_st_open": (_i32, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "glt_st_close": (None, [_vp]),
    "glt_st_count": (_i32, [_vp]),
    "glt_st_info": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_i64)]),
    "glt_st_read": (_i32, [_vp, ctypes.c_char_p, _vp, _i32, _i32, _i32, _vp]),
    "glt_st_load_layer": (_i32, [_vp, _i32, ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerBuffers), _i32, _vp]),
    "glt_st_load_head": (_i32, [_vp, _i32, _i32, _vp, _vp, _vp, _i32, _vp]),
    "glt_masked_ce_workspace_size": (_sz, [_i32, _i32]),
    "glt_masked_ce": (_i32, [_vp, _i64, _vp, _vp, _i32, _i32, _i32, ctypes.c_float, _vp, _i64, _vp, _vp, _vp, _sz,
                             _vp]),
    "glt_silence_energy": (_i32, [_vp, _i32, _i64, _i32, _i32, _vp, _vp]),
    "glt_silence_blend": (_i32, [_vp, _vp, _vp, _i32, _i32, ctypes.c_float, _vp]),
    "glt_silence_blend_energy": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, _vp]),
    "glt_lr_schedule": (ctypes.c_float, [_i32, _i32, _i32, ctypes.c_float]),
}

_lib = None


class GltError(RuntimeError):
    def __init__(self, code, fn, msg):
        self.code = code
        self.status = STATUS_NAMES.get(code, str(code))
        super().__init__(f"{fn}: {self.status}: {msg}")


def load(path=LIB_PATH):
    """Loads libglt.so and binds every declared entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"libglt.so is not built at {path}; run `python -m glt_amd.build` "
                           "(the graft-layer path has no fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name, *args):
    """Calls an entry point and raises GltError on a non-OK status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != GLT_OK:
        raise GltError(rc, name, lib.glt_last_error_string().decode(errors="replace"))
    return rc


def profile_collect(max_labels=64):
    """{label: (total_ms, launches)} of the launches timed since the last collect."""
    lib = load()
    names = ctypes.create_string_buffer(64 * max_labels)
    tot = (ctypes.c_double * max_labels)()
    cnt = (_i64 * max_labels)()
    n = lib.glt_profile_collect(names, len(names), tot, cnt, max_labels)
    labels = names.raw.split(b"\0")[:n]
    return {labels[i].decode(): (tot[i], cnt[i]) for i in range(n)}


def ptr_array(ptrs):
    arr = (_vp * max(1, len(ptrs)))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr
