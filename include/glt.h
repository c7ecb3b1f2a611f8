/*
 * glt.h — C ABI of the MI355X (gfx950) grafted-SwiGLU layer path.
 *
 * Every entry point takes caller-owned device buffers, explicit shapes and an
 * explicit HIP stream (hipStream_t passed as void*, NULL = default stream),
 * and returns an int status. No C++ exception crosses this boundary and no
 * entry point allocates device memory; scratch space is passed in by the
 * caller (glt_mlp_bwd_workspace_size tells how much).
 *
 * bf16 values are passed as their 16-bit patterns (uint16_t storage).
 * All matrices are row-major. "[R,C]" means R rows of C contiguous elements.
 *
 * The reference implements this path as an internal C++ API with shapes held
 * in a process-global config (reference src/config.hpp:40-95, g_cfg). Here the
 * shapes travel in descriptors instead. Citations name the reference function
 * each entry point replaces.
 */
#ifndef GLT_H_
#define GLT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLT_ABI_VERSION 4

/* ------------------------------------------------------------------ status */
typedef int32_t glt_status;
#define GLT_OK                     0
#define GLT_ERR_INVALID_ARG        1  /* null pointer / bad enum / bad flag        */
#define GLT_ERR_SHAPE              2  /* inconsistent or out-of-range dimensions   */
#define GLT_ERR_DTYPE              3  /* unsupported dtype combination             */
#define GLT_ERR_ALIGNMENT          4  /* pointer or stride alignment not met       */
#define GLT_ERR_WORKSPACE          5  /* workspace missing or too small            */
#define GLT_ERR_ALREADY_BAKED      6  /* second bake on the same model state       */
#define GLT_ERR_BAKED_NO_BACKWARD  7  /* backward on a shadow-baked model          */
#define GLT_ERR_HIP                8  /* a HIP runtime call failed                 */
#define GLT_ERR_UNSUPPORTED        9  /* valid request the library does not serve  */
#define GLT_ERR_IO                10  /* a file could not be opened, read or written */
#define GLT_ERR_FORMAT            11  /* file content malformed or not the expected  */
#define GLT_ERR_NOT_FOUND         12  /* a named tensor is absent from the files     */

/* ------------------------------------------------------------------ dtypes */
#define GLT_DTYPE_BF16 0
#define GLT_DTYPE_F32  1
#define GLT_DTYPE_F16  2  /* stored dtype reported by glt_st_info only */

/* Projection indices, as in the reference flat graft storage
 * (reference src/graft_ops_impl.inc:5-7: offset = (layer*3 + proj)*S*H). */
#define GLT_PROJ_GATE 0
#define GLT_PROJ_UP   1
#define GLT_PROJ_DOWN 2
#define GLT_PROJ_MASK_ALL 7 /* bit p set = projection p grafted */

/* Shadow-bake guard state, owned by the caller (one per model instance).
 * Replaces the process-global g_shadow_baked (reference src/shadow_bake.hpp:5). */
typedef struct {
  int32_t baked; /* 0 = not baked; set to 1 by a successful glt_shadow_bake */
} glt_model_state;

/* One graft slice of one layer.
 *
 * Placement (reference src/shadow_bake_impl.inc:11-14, docs/contract_audit.md:601-612):
 *   gate/up delta [S,H] adds onto rows [i_start, i_start+S) x cols [h_start, h_start+H)
 *   of W_gate / W_up ([N,D]); the down delta is stored [S,H] too and adds onto
 *   the transposed block rows [h_start, h_start+H) x cols [i_start, i_start+S)
 *   of W_down ([D,N]).
 * An "appended" slice (i_start >= I) lives in the zero-extended tail of the
 * base, i.e. it adds new neurons; an in-place slice (i_start+S <= I) adds onto
 * existing ones (the reference's domain-sliced form).
 *
 * master_*: f32 [S,H] master deltas (reference GraftWeights.d_weight,
 *           src/types.hpp:190-201). NULL = projection not grafted.
 * packed:   bf16 mirror written by glt_graft_pack / glt_adamw_graft_step,
 *           glt_graft_packed_size(S, H) bytes, 256-byte aligned: the six
 *           orientations gate[S,H], gate^T[H,S], up[S,H], up^T[H,S],
 *           down[S,H], down^T[H,S] row-major, then the same six in the
 *           MFMA fragment layout. Read by the bf16 path; unused by f32.  */
typedef struct {
  int32_t i_start, s, h_start, h;
  const float* master_gate;
  const float* master_up;
  const float* master_down;
  const uint16_t* packed;
} glt_graft_slice;

/* Per-slice f32 weight-gradient outputs of glt_mlp_bwd, [S,H] each in the
 * same storage orientation as the master (reference d_delta_grad,
 * src/graft_ops_impl.inc:120-141, :214-228). NULL = not requested. */
typedef struct {
  float* gate;
  float* up;
  float* down;
} glt_graft_grads;

/* Frozen base weights of one MLP layer (torch Linear [out,in] layout),
 * gate/up [I,D], down [D,I], in the path dtype. prepared: the bf16 path's
 * copy of all six orientations the GEMMs multiply by (gate, up, down,
 * down^T, gate^T, up^T) in the MFMA fragment layout, made once per frozen
 * base by glt_base_prepare (glt_base_prepared_size bytes); NULL on the f32
 * path. It replaces the reference's cached f32 base copies
 * (src/model_io_impl.inc:174-177). */
typedef struct {
  const void* gate;
  const void* up;
  const void* down;
  const void* prepared;
} glt_base_weights;

/* Shape of one grafted SwiGLU MLP call.
 *   M tokens, D hidden, I base intermediate rows held by W_gate/W_up,
 *   N >= I total neurons (rows [I,N) of the base are zero: appended grafts).
 * flags: GLT_MLP_EXPLICIT applies the slices (the reference's
 * use_explicit_graft, src/layer_forward_impl.inc:76); without it the call is
 * the plain base MLP (e.g. over shadow-baked weights). */
#define GLT_MLP_EXPLICIT 1
/* GLT_MLP_RECOMPUTE: glt_mlp_bwd recomputes gate_pre/up_pre/inter from x in
 * its workspace instead of reading saved activations (the reference's
 * recompute_ffn, src/layer_recompute_impl.inc:8-91). */
#define GLT_MLP_RECOMPUTE 2
/* GLT_MLP_RESIDUAL: y holds the residual stream on entry and glt_mlp_fwd
 * adds the MLP output to it in the down GEMM's epilogue,
 * y = round(y + round(ffn_out)) (the reference's x = x + ffn_out,
 * src/layer_forward_impl.inc:271-275, on the path dtype). */
#define GLT_MLP_RESIDUAL 4
/* GLT_MLP_DY_F32: glt_mlp_bwd's dy is f32 [M,D] on the bf16 path (the
 * reference's backward receives an f32 gradient, src/layer_backward_impl.inc:48).
 * It is rounded once (RNE) to the bf16 MFMA operand inside the call; without
 * the flag dy is in the path dtype. No effect on the f32 path (dy is f32). */
#define GLT_MLP_DY_F32 8
typedef struct {
  int32_t M, D, I, N;
  int32_t dtype;   /* GLT_DTYPE_BF16 or GLT_DTYPE_F32 */
  int32_t flags;
  int32_t n_slices;               /* at most 8 (as glt_shadow_bake and the AdamW graft step) */
  const glt_graft_slice* slices;
  glt_model_state* state; /* nullable; checked for the baked guard in backward */
} glt_mlp_desc;

/* ----------------------------------------------------------- library info */
int32_t glt_version(void);                 /* GLT_ABI_VERSION */
const char* glt_last_error_string(void);   /* thread-local text of the last error */
/* Device properties the roofline needs: CU count and peak engine clock (MHz). */
glt_status glt_device_info(int32_t device, int32_t* cu_count, int32_t* clock_mhz,
                           int64_t* hbm_bytes);

/* Launch timing. While enabled, each kernel launch of the library is
 * bracketed by HIP events on its own stream, keyed by a label naming the
 * kernel's role ("gate_up", "down", "dinter", "dx", "wgrad", "bake", ...).
 * Replaces the reference's --profile-graft-gemms (src/gemm_impl.inc:153-199,
 * :408-444) without its synchronisation after every GEMM.
 * glt_profile_collect waits for the recorded events, writes up to
 * max_labels NUL-separated labels into names, their summed milliseconds and
 * launch counts, clears the records and returns the number of labels. */
glt_status glt_profile_enable(int32_t on);
int32_t glt_profile_collect(char* names, size_t names_len, double* total_ms, int64_t* counts,
                            int32_t max_labels);

/* ------------------------------------------------------------ conversions */
/* out[i] = RNE bf16 of in[i] (reference f32_to_bf16_kernel, src/gemm_impl.inc:69-89). */
glt_status glt_f32_to_bf16(const float* in, uint16_t* out, int64_t n, void* stream);

/* Synthetic inputs: counter-based normal generator keyed by (seed, tensor_id):
 * splitmix64 -> Box-Muller in f64 -> f32 (-> RNE bf16). out[i] = mean + std*z_i.
 * Not a reference function (the reference loads real weights); used so that
 * benchmarks and host checks can draw the same inputs. */
glt_status glt_fill_normal(void* out, int32_t dtype, int64_t n, uint64_t seed,
                           uint64_t tensor_id, double mean, double stdev,
                           void* stream);

/* --------------------------------------------------------------- graft ops */
/* Bytes of the packed bf16 mirror of an S x H slice (glt_graft_slice.packed). */
size_t glt_graft_packed_size(int32_t S, int32_t H);
/* Build the packed bf16 mirror of one slice from its f32 masters.
 * Replaces refresh_graft_weight_bf16 / convert_f32_to_bf16 of the reference
 * (src/gemm_impl.inc:85-95), which it ran before every graft GEMM call. */
glt_status glt_graft_pack(const glt_graft_slice* slice, uint16_t* packed, void* stream);

/* Transposed copy (dst[c,r] = src[r,c]), rows x cols. */
glt_status glt_transpose(const void* src, void* dst, int32_t rows, int32_t cols,
                         int32_t dtype, void* stream);
/* Bytes of glt_base_weights.prepared for d (0 on the f32 path). */
size_t glt_base_prepared_size(const glt_mlp_desc* d);
/* Writes the prepared copy of a frozen bf16 base (256-byte aligned buffer);
 * a no-op on the f32 path. */
glt_status glt_base_prepare(const glt_mlp_desc* d, const void* gate, const void* up,
                            const void* down, void* prepared, void* stream);

/* The six graft GEMM kinds of the reference (src/config.hpp:31-38,
 * graft_gemm_fwd / grad_gemm / grad_gemm_storage_canonical
 * src/gemm_impl.inc:388-584, graft ops src/graft_ops_impl.inc:14-228).
 * All operands bf16 except out (f32) and delta (f32 master, rounded to bf16
 * per call exactly as the reference does). S,H = slice dims; M = tokens.
 *   0 EXPAND_FWD      out[M,S]  = a[M,H](lda) . bf16(delta[S,H])^T
 *   1 CONTRACT_FWD    out[M,H]  = a[M,S](lda) . bf16(delta[S,H])
 *   2 EXPAND_WGRAD    out[S,H]  = bf16(dy[M,S])^T . a[M,H](lda)      dy f32
 *   3 CONTRACT_WGRAD  out[S,H]  = a[M,S](lda)^T . bf16(dy[M,H])      dy f32
 *   4 EXPAND_IGRAD    out[M,H]  = bf16(dy[M,S]) . bf16(delta[S,H])  dy f32
 *   5 CONTRACT_IGRAD  out[M,S]  = bf16(dy[M,H]) . bf16(delta[S,H])^T dy f32
 * out = alpha*result + beta*out, with row stride ldo. */
#define GLT_GEMM_EXPAND_FWD     0
#define GLT_GEMM_CONTRACT_FWD   1
#define GLT_GEMM_EXPAND_WGRAD   2
#define GLT_GEMM_CONTRACT_WGRAD 3
#define GLT_GEMM_EXPAND_IGRAD   4
#define GLT_GEMM_CONTRACT_IGRAD 5
glt_status glt_graft_gemm(int32_t kind, int32_t M, int32_t S, int32_t H,
                          const uint16_t* a, int64_t lda, const float* delta,
                          const float* dy, float* out, int64_t ldo, float alpha,
                          float beta, void* stream);

/* ------------------------------------------------------------- MLP layer */
/* Forward of the grafted SwiGLU MLP (reference FFN section of forward_layer,
 * src/layer_forward_impl.inc:61-290, with execute_expand_forward /
 * execute_contract_forward src/graft_ops_impl.inc:14-114):
 *   gate_pre = x . [W_gate (+) grafts]^T, up_pre likewise      [M,N]
 *   inter    = silu(gate_pre) * up_pre                          [M,N]
 *   y        = inter . [W_down (+) grafts]^T                    [M,D]
 * bf16 path: one concat-N MFMA GEMM for gate/up with the SiLU*up epilogue and
 * one K-concat GEMM for down, graft terms accumulated in fp32.
 * gate_pre/up_pre: saved for glt_mlp_bwd (nullable: then backward recomputes).
 * inter: required. Buffers are [M,N] / [M,D] of the path dtype. */
glt_status glt_mlp_fwd(const glt_mlp_desc* d, const glt_base_weights* w,
                       const void* x, void* y, void* gate_pre, void* up_pre,
                       void* inter, void* stream);

/* Graft-only backward (reference FFN section of backward_layer,
 * src/layer_backward_impl.inc:10-361; base weights frozen):
 *   dInter = dy . W_down_ext ; dgate/dup via the SiLU*up derivative;
 *   grads[j] = per-slice dW (f32, [S,H] storage); dx = d(x) f32 [M,D].
 * dy is [M,D] of the path dtype, or f32 with GLT_MLP_DY_F32. dx nullable. Returns
 * GLT_ERR_BAKED_NO_BACKWARD when d->state says the model is shadow-baked
 * (reference src/layer_backward_impl.inc:11-13). */
size_t glt_mlp_bwd_workspace_size(const glt_mlp_desc* d);
glt_status glt_mlp_bwd(const glt_mlp_desc* d, const glt_base_weights* w,
                       const void* x, const void* dy, const void* gate_pre,
                       const void* up_pre, const void* inter, float* dx,
                       const glt_graft_grads* grads, void* ws, size_t ws_bytes,
                       void* stream);
/* The FFN backward followed by the backward of the RMSNorm that produced its
 * input, as the reference's backward_layer runs them (graft-only FFN backward,
 * src/layer_backward_impl.inc:34-361, then rms_norm_bwd of the FFN norm,
 * src/kernels_rmsnorm_kernels.inc:70-126): glt_mlp_bwd(d, w, x, dy, gate_pre,
 * up_pre, inter, dx, grads, ws, ws_bytes) then glt_rmsnorm_bwd(dx, norm_x,
 * norm_w, norm_var, norm_dx, M, D, eps), with the same results bit for bit.
 * x is the RMSNorm's output (the FFN input), norm_x its input (bf16 [M,D]),
 * norm_w its weight [D], norm_var its saved mean squares [M]; dx (required)
 * receives the FFN input gradient and norm_dx (f32 [M,D], may be dx) the
 * norm input gradient. The RMSNorm backward runs on a per-device helper
 * stream, on the CUs the weight-gradient GEMM leaves idle, joined to
 * `stream` before the call's work on it ends. bf16 path only. */
glt_status glt_mlp_rmsnorm_bwd(const glt_mlp_desc* d, const glt_base_weights* w,
                               const void* x, const void* dy, const void* gate_pre,
                               const void* up_pre, const void* inter, float* dx,
                               const glt_graft_grads* grads, void* ws, size_t ws_bytes,
                               const uint16_t* norm_x, const uint16_t* norm_w,
                               const float* norm_var, float eps, float* norm_dx,
                               void* stream);

/* Unfused parity probes of the elementwise stages.
 * glt_silu_mul:  out = bf16(g*sigmoid(g)*u)   (reference fused_silu_product_kernel,
 *                src/kernels_elementwise_impl.inc:378-448)
 * glt_gate_up_bwd: dg = gi*u*s*(1+g*(1-s)), du = gi*g*s, f32 out
 *                (reference fused_gate_up_bwd_kernel, :80-124) */
glt_status glt_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n,
                        void* stream);
glt_status glt_gate_up_bwd(const float* gi, const uint16_t* g, const uint16_t* u,
                           float* dg, float* du, int64_t n, void* stream);

/* --------------------------------------------------------------- RMSNorm */
/* y = bf16(x * rsqrt(var+eps) * w), var[m] = mean(x^2) (mean-square, as the
 * reference stores it). x,y [M,D] bf16, w [D] bf16, var [M] f32.
 * Reference rms_norm / rms_norm_fwd_kernel (grafting.hip:116-146,
 * src/kernels_rmsnorm_kernels.inc:8-60). */
glt_status glt_rmsnorm_fwd(const uint16_t* x, const uint16_t* w, uint16_t* y, float* var,
                           int32_t M, int32_t D, float eps, void* stream);
/* dx = dy*r*w - x*mean(dy*x*w)*r^3, r = rsqrt(var+eps); dy,dx f32 [M,D].
 * Reference rms_norm_bwd / rms_norm_bwd_kernel (grafting.hip:153-172,
 * src/kernels_rmsnorm_kernels.inc:70-126). */
glt_status glt_rmsnorm_bwd(const float* dy, const uint16_t* x, const uint16_t* w,
                           const float* var, float* dx, int32_t M, int32_t D, float eps,
                           void* stream);

/* ------------------------------------------------------------------- RoPE */
/* In-place rotate-half RoPE on q [B,T,n_q_heads,head_dim] and k
 * [B,T,n_kv_heads,head_dim] (bf16; k nullable), positions pos_offset + t.
 * Reference apply_rope (src/rope_impl.inc:8-39): inv_freq_i = 1/theta^(2i/hd)
 * and angles in f32, cos/sin rounded to bf16, r1 = x1*c - x2*s,
 * r2 = x2*c + x1*s. Here the rotation runs in f32 with one rounding per
 * output. The caller skips layers its no-RoPE mask excludes
 * (reference src/layer_forward_impl.inc:37-39). */
glt_status glt_rope_fwd(uint16_t* q, int32_t n_q_heads, uint16_t* k, int32_t n_kv_heads,
                        int32_t B, int32_t T, int32_t head_dim, float theta,
                        int32_t pos_offset, void* stream);

/* -------------------------------------------------------------- Attention */
/* Causal GQA attention forward, the decoder layer's base attention
 * (reference forward_layer src/layer_forward_impl.inc:41-49: heads split,
 * k/v repeat_interleave'd to the query heads, at::scaled_dot_product_attention
 * with is_causal, heads merged). q/out [B,T,n_q_heads,head_dim], k/v
 * [B,T,n_kv_heads,head_dim], bf16 row-major; query head h reads kv head
 * h / (n_q_heads / n_kv_heads). scale multiplies q.k (the reference's default
 * is 1/sqrt(head_dim)); causal != 0 masks keys after the query's position.
 * Softmax in f32 (online, exp2), probabilities rounded to bf16 for the P.V
 * product, f32 accumulation, one rounding of the output. head_dim must be
 * 128; tensors 16-byte aligned. workspace (glt_attention_workspace_size
 * bytes, 256-byte aligned) receives a transposed copy of v, [B, n_kv_heads,
 * head_dim, T rounded up to 64], rewritten by every call. */
size_t glt_attention_workspace_size(int32_t B, int32_t T, int32_t n_kv_heads, int32_t head_dim);
glt_status glt_attention_fwd(const void* q, const void* k, const void* v, void* out,
                             int32_t B, int32_t T, int32_t n_q_heads, int32_t n_kv_heads,
                             int32_t head_dim, float scale, int32_t causal, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------- decoder layer */
/* One decoder layer forward with the grafted MLP (reference forward_layer,
 * src/layer_forward_impl.inc:15-290):
 *   xn = rms_norm(x, ln_in); q,k,v = xn . W^T; RoPE(q, k); a = SDPA(q,k,v)
 *   x += a . W_o^T; x_ffn = rms_norm(x, ln_post); x += grafted_mlp(x_ffn)
 * bf16 throughout; M = B*T tokens, x [M,D] is the residual stream, updated
 * in place. rope_theta <= 0 skips RoPE (the reference's no-RoPE layer mask,
 * :37-39). mlp is the MLP's descriptor (mlp.M = B*T, mlp.D = D, bf16). */
typedef struct {
  int32_t B, T;
  int32_t n_q_heads, n_kv_heads, head_dim; /* head_dim 128 */
  float rope_theta;
  float rms_eps;
  glt_mlp_desc mlp;
} glt_layer_desc;

/* Projection weights are bf16 [out, in] row-major like torch Linear (the
 * reference's q_proj/k_proj/v_proj/o_proj, src/types.hpp); ln_* are the two
 * RMSNorm weights [D]; prepared holds them in the MFMA fragment layout
 * (glt_attn_prepare); mlp is the MLP's base. */
typedef struct {
  const void* q_proj;
  const void* k_proj;
  const void* v_proj;
  const void* o_proj;
  const void* ln_in;
  const void* ln_post;
  const void* prepared;
  glt_base_weights mlp;
} glt_layer_weights;

size_t glt_attn_prepared_size(const glt_layer_desc* d);
/* Writes the four projections of w into prepared (glt_attn_prepared_size
 * bytes, 256-byte aligned); once per frozen layer. */
glt_status glt_attn_prepare(const glt_layer_desc* d, const glt_layer_weights* w, void* prepared,
                            void* stream);
size_t glt_layer_fwd_workspace_size(const glt_layer_desc* d);
/* x_ffn [M,D] bf16 and ffn_var [M] f32 (the MLP input and its RMSNorm
 * mean square) are written for the backward; gate_pre/up_pre/inter are the
 * MLP's saved activations as in glt_mlp_fwd (nullable: then they live in the
 * workspace and glt_mlp_bwd recomputes, the reference's recompute_ffn). */
glt_status glt_layer_fwd(const glt_layer_desc* d, const glt_layer_weights* w, void* x, void* x_ffn,
                         float* ffn_var, void* gate_pre, void* up_pre, void* inter, void* workspace,
                         size_t workspace_bytes, void* stream);

/* -------------------------------------------------------- graft checkpoint */
/* The GRFT graft file (reference save_safetensors / load_safetensors_checkpoint,
 * src/checkpoint_impl.inc:39-97, :170-285; magic and version
 * src/checkpoint.hpp:5-6): u32 magic 0x54465247 ("GRFT"), version byte 4, then
 * a safetensors body: u64 header size, a JSON header padded with NUL bytes to a
 * multiple of 8, the data. One tensor "delta_weights", BF16 [num_layers*3, S, H]:
 * the RNE bf16 of the flat f32 graft storage (offset (l*3+p)*S*H, p = gate, up,
 * down). __metadata__ holds session_id, domain_id, slice_dim, h_slice_dim,
 * hidden_dim and num_layers as strings. weight_on_device says whether weight
 * is device memory (copied on stream) or host memory. */
typedef struct {
  int32_t num_layers, S, H, hidden_dim, domain_id;
  const char* session_id; /* nullable = "" */
} glt_grft_info;
glt_status glt_grft_save(const char* path, const glt_grft_info* info, const float* weight,
                         int32_t weight_on_device, void* stream);
/* Loads delta_weights into the f32 storage (bf16 widened). Accepts files
 * without the magic (plain safetensors, the reference's legacy form) and
 * space- or NUL-padded headers. Checks, as the reference: dtype BF16, shape
 * [num_layers*3, S, H], session_id equal when both are non-empty, domain_id
 * equal when the file has one (a file without it loads).
 * GLT_ERR_IO / GLT_ERR_FORMAT on failure; weight is untouched then. */
glt_status glt_grft_load(const char* path, const glt_grft_info* expect, float* weight,
                         int32_t weight_on_device, void* stream);
/* Raw flat f32 storage, the reference's --init-deltas file (grafting.hip:
 * 882-901): exactly num_layers*3*S*H floats, native byte order. */
glt_status glt_grft_load_raw_f32(const char* path, const glt_grft_info* expect, float* weight,
                                 int32_t weight_on_device, void* stream);

/* ------------------------------------------------------------------ AdamW */
/* One AdamW step over n f32 params (reference adamw_fused_kernel,
 * src/kernels_optimizer_impl.inc:11-77) with bias corrections for step
 * (0-based, as the reference's step+1). clip_norm > 0 first scales grads to
 * global L2 norm <= clip_norm using sqrt(sum g^2 + 1e-8) (reference
 * reduce_l2/calc_scale/apply_scale, src/kernels_elementwise_impl.inc:133-213);
 * clip_norm <= 0 = no clip. The clip needs ws of glt_adamw_workspace_size(n)
 * bytes. bf16_mirror (nullable) receives bf16(w). g is read only (the
 * reference scales its gradient buffer in place; here the scale is applied
 * as the update reads it). */
size_t glt_adamw_workspace_size(int64_t n);
glt_status glt_adamw_step(float* w, float* g, float* m, float* v, uint16_t* bf16_mirror,
                          int64_t n, int32_t step, float lr, float beta1, float beta2,
                          float eps, float weight_decay, float clip_norm, void* ws,
                          size_t ws_bytes, void* stream);

/* AdamW over a whole graft set with the packed-mirror refresh fused in:
 * updates each slice's masters (treated as writable) and rewrites the
 * updated projections' part of its packed bf16 mirror. grads/m/v are per-slice [3,S,H]
 * f32 buffers laid out gate,up,down. proj_mask as in the reference
 * (skipped projections are untouched, src/kernels_optimizer_impl.inc:20-25).
 * clip_norm > 0 clips first by the global L2 norm over the gradients of every
 * projection the step updates, all slices together (the reference's
 * per-step clip over all of its deltas, grafting.hip:1149-1164, default
 * 1.0, src/config.hpp:85); it needs ws of glt_adamw_workspace_size(0)
 * bytes. Any number of slices; with the clip on, the norm covers at most
 * 512 projections (170 slices of gate, up and down), more return
 * GLT_ERR_UNSUPPORTED. */
glt_status glt_adamw_graft_step(const glt_graft_slice* slices, int32_t n_slices,
                                float* const* grads, float* const* m, float* const* v,
                                uint16_t* const* packed_out, int32_t proj_mask,
                                int32_t step, float lr, float beta1, float beta2,
                                float eps, float weight_decay, float clip_norm, void* ws,
                                size_t ws_bytes, void* stream);

/* glt_adamw_graft_step without a workspace argument and without allocating:
 * the clip's partial sums live in a 2 KB device array of the library (one
 * per GPU, held until the process ends). No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving or training loops). Every gradient size fits (the
 * clip uses at most 512 partial sums), and so does every slice count
 * glt_adamw_graft_step takes. Calls on one GPU share the array: calls that overlap
 * in time on one GPU (two streams) race; calls in stream order do not. */
glt_status glt_adamw_graft_step_noalloc(const glt_graft_slice* slices, int32_t n_slices,
                                        float* const* grads, float* const* m, float* const* v,
                                        uint16_t* const* packed_out, int32_t proj_mask,
                                        int32_t step, float lr, float beta1, float beta2,
                                        float eps, float weight_decay, float clip_norm,
                                        void* stream);

/* ------------------------------------------------------------ shadow bake */
/* Merge graft deltas into bf16 base matrices (reference shadow_bake_kernel /
 * apply_graft_to_shadow, src/shadow_bake_impl.inc:15-128).
 *
 * mode GLT_BAKE_IN_PLACE: base[l] += delta, in place (reference semantics);
 *   gate/up base [I,D] (row stride D), down base [D,I] (row stride I).
 * mode GLT_BAKE_MATERIALIZE: out[l] = zero-extended base (+) deltas, with
 *   gate/up out [N,D] and down out [D,N]; base matrices are read only.
 * Every output element is one RNE of f32(base) + f32(delta): bit-exact.
 *
 * graft[l] points at layer l's flat [3,S,H] deltas (gate, up, down) of the
 * given dtype, i.e. the reference's d_weight + delta_offset(l, 0).
 * Layers outside [layer_start, layer_end] and projections not in proj_mask
 * are skipped (reference should_graft_layer / should_graft_proj,
 * src/config.hpp:100-110). A second bake on the same state fails with
 * GLT_ERR_ALREADY_BAKED (reference src/shadow_bake_impl.inc:59-62). */
#define GLT_BAKE_IN_PLACE    0
#define GLT_BAKE_MATERIALIZE 1
typedef struct {
  int32_t mode;
  int32_t num_layers;
  int32_t layer_start, layer_end; /* inclusive */
  int32_t proj_mask;
  int32_t D, I, N;                /* N used by MATERIALIZE (N >= I) */
  int32_t graft_dtype;            /* GLT_DTYPE_F32 (master) or GLT_DTYPE_BF16 */
  int32_t n_slices;               /* slices baked together (stacked grafts), at most 8 */
  const int32_t* placement;       /* n_slices x {i_start, s, h_start, h} */
  const void* const* graft;       /* [n_slices * num_layers] flat [3,S,H] per layer */
} glt_bake_desc;
glt_status glt_shadow_bake(const glt_bake_desc* d, glt_model_state* state,
                           void* const* gate, void* const* up, void* const* down,
                           void* const* gate_out, void* const* up_out,
                           void* const* down_out, void* stream);

/* ------------------------------------------------------ whole model
 * forward_model (reference grafting.hip:224-271): embedding, the decoder
 * layers, final RMSNorm, LM head.
 * glt_embedding: out[t] = table[ids[t]] (at::embedding), bf16 rows of D;
 * ids outside [0, V) give zero rows (at::embedding raises).
 * glt_lm_head_prepare writes lm_head [V,D] and its transpose in the MFMA
 * fragment layout (glt_lm_head_prepared_size bytes, 256-byte aligned; once
 * per model); glt_lm_head_fwd: logits [M,V] = x [M,D] . lm_head^T, bf16 out
 * (at::linear); glt_lm_head_bwd: dx [M,D] = grad [M,V] . lm_head, f32 out
 * (the reference's dx = grad_logits_full @ lm_head, grafting.hip:1137). */
glt_status glt_embedding(const int32_t* ids, int64_t n, const uint16_t* table, int32_t V, int32_t D,
                         uint16_t* out, void* stream);
size_t glt_lm_head_prepared_size(int32_t V, int32_t D);
glt_status glt_lm_head_prepare(const uint16_t* lm_head, int32_t V, int32_t D, void* prepared, void* stream);
glt_status glt_lm_head_fwd(const uint16_t* x, int32_t M, int32_t D, const uint16_t* lm_head,
                           const void* prepared, int32_t V, uint16_t* logits, void* stream);
glt_status glt_lm_head_bwd(const uint16_t* grad, int32_t M, int32_t V, const uint16_t* lm_head,
                           const void* prepared, int32_t D, float* dx, void* stream);

/* The whole forward: layers[l] with descs[l] (per-layer graft slices; every
 * desc has the same B, T, heads and D), use_explicit_graft selects the
 * graft path of every layer's MLP (the reference's flag; off = base only,
 * e.g. over shadow-baked weights). logits [B*T, V] bf16. workspace:
 * glt_model_fwd_workspace_size bytes, 256-byte aligned. */
typedef struct {
  int32_t num_layers, V;
  int32_t use_explicit_graft;
  const glt_layer_desc* descs;       /* [num_layers] */
  const glt_layer_weights* layers;   /* [num_layers], attention prepared */
  const uint16_t* embed;             /* [V,D] */
  const uint16_t* final_norm;        /* [D] */
  const uint16_t* lm_head;           /* [V,D] */
  const void* lm_head_prepared;
} glt_model;
size_t glt_model_fwd_workspace_size(const glt_model* m);
glt_status glt_model_fwd(const glt_model* m, const int32_t* ids, uint16_t* logits, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Shadow-eval statistics of one logits batch (reference eval loop,
 * grafting.hip:504-547): over rows (b,t) of B*T bf16 logits (row stride
 * ld), the f32 cross-entropy of rows t < T-1 against ids[b,t+1] summed in
 * f64 (total_nll; mean = total_nll / count), the f64 sum and sum of squares
 * of every logit, and a 64-bit FNV-1a hash of the logits.
 *
 * hash_mode GLT_EVAL_HASH_REFERENCE: the reference's hash, bit for bit: one
 * FNV-1a chain, h = (h ^ byte) * 1099511628211 mod 2^64, over the four
 * little-endian bytes of every f32 logit in (b, t, v) order, starting from
 * hash_in (grafting.hip:536-546). The reference starts at GLT_FNV_BASIS and
 * continues the chain across its eval batches: pass the previous batch's
 * logits_hash as hash_in to do the same. Computed exactly in parallel (the
 * low byte of the state is a chain of its own, after which each chunk of
 * logits is an affine map mod 2^64).
 * hash_mode GLT_EVAL_HASH_ROWS: this library's row form: each row's f32
 * logits cut into 16 chunks of ceil(V/16) (the last ones shorter or empty),
 * each chunk hashed byte by byte from GLT_FNV_BASIS, the chunk hashes' 8
 * bytes hashed in chunk order into the row hash, and the row hashes' 8 bytes
 * chained in row order from hash_in (one pass over the logits; a different
 * value from the reference's).
 * Synchronous; workspace: glt_eval_stats_workspace_size bytes, 256-byte
 * aligned. */
#define GLT_FNV_BASIS 1469598103934665603ULL /* the reference's offset basis, grafting.hip:505 */
#define GLT_EVAL_HASH_REFERENCE 0
#define GLT_EVAL_HASH_ROWS      1
typedef struct {
  double total_nll;
  int64_t count;
  double logits_sum, logits_sumsq;
  uint64_t logits_hash;
} glt_eval_result;
size_t glt_eval_stats_workspace_size(int32_t B, int32_t T);
glt_status glt_eval_stats(const uint16_t* logits, int64_t ld, const int32_t* ids, int32_t B, int32_t T,
                          int32_t V, int32_t hash_mode, uint64_t hash_in, glt_eval_result* out,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------ base model files
 * Safetensors model weights (reference load_base_model_safetensors /
 * load_named_tensor / st_to_aten, src/model_io_impl.inc:16-190). path is a
 * .safetensors file or a directory whose *.safetensors files are used in
 * sorted order; files are memory-mapped, and a name found in several files
 * resolves to the first. Stored dtypes BF16, F32, F16 are read; tensors are
 * delivered as dst_dtype (GLT_DTYPE_BF16 or GLT_DTYPE_F32, RNE on the host),
 * optionally transposed (2-D only), to device memory on `stream`
 * (on_device = 1, waited for) or host memory. */
typedef struct glt_st_set glt_st_set;
glt_status glt_st_open(const char* path, glt_st_set** out);
void glt_st_close(glt_st_set* s);
int32_t glt_st_count(const glt_st_set* s);  /* distinct tensor names */
/* dtype (GLT_DTYPE_*), ndim and shape (up to 8 dims) of tensor `name`;
 * GLT_ERR_NOT_FOUND when absent, GLT_ERR_DTYPE for other stored dtypes */
glt_status glt_st_info(const glt_st_set* s, const char* name, int32_t* dtype, int32_t* ndim,
                       int64_t* shape);
glt_status glt_st_read(const glt_st_set* s, const char* name, void* dst, int32_t dst_dtype,
                       int32_t transpose, int32_t on_device, void* stream);
/* The nine weights of decoder layer `layer` under the reference's names
 * (model.layers.{l}.input_layernorm / self_attn.{q,k,v,o}_proj /
 * post_attention_layernorm / mlp.{gate,up,down}_proj .weight,
 * src/model_io_impl.inc:104-115), shapes checked against d (q [Hq*hd, D],
 * k/v [Hkv*hd, D], o [D, Hq*hd], norms [D], gate/up [I, D], down [D, I]),
 * delivered as bf16. */
typedef struct {
  void* q_proj; void* k_proj; void* v_proj; void* o_proj;
  void* ln_in; void* ln_post;
  void* gate; void* up; void* down;
} glt_layer_buffers;
glt_status glt_st_load_layer(const glt_st_set* s, int32_t layer, const glt_layer_desc* d,
                             const glt_layer_buffers* dst, int32_t on_device, void* stream);
/* model.embed_tokens.weight [V,D], model.norm.weight [D] and lm_head.weight
 * as [V,D] bf16: tied to the embedding when absent, transposed when stored
 * [D,V], taken as [V,D] when square (src/model_io_impl.inc:118-145). */
glt_status glt_st_load_head(const glt_st_set* s, int32_t V, int32_t D, void* embed,
                            void* final_norm, void* lm_head, int32_t on_device, void* stream);

/* ------------------------------------------------------ training step
 * Masked cross-entropy over the shifted logits and its gradient: replaces
 * the reference's ATen loss (grafting.hip:1027-1050) and grad_logits
 * (:1122-1135). logits: B*T rows of V bf16 at row stride ld (elements);
 * ids, ood: [B,T] int32 (ood != 0 marks an excluded token). Row (b,t),
 * t < T-1, is scored against ids[b,t+1] and counts when ood[b,t+1] == 0;
 * n = max(count, 1). grad (NULL = loss only; may alias logits when
 * ld_grad == ld) gets B*T rows, row (b,T-1) zero, the others
 * bf16((bf16(softmax) - onehot)*mask*(1/n)*scale) rounded after every
 * operation as the reference's bf16 tensor ops do. ce_per_token (NULL or
 * f32 [B*(T-1)]) gets -bf16(log_softmax[label]). stats (device f32[4]):
 * loss, mean target logit, mean target probability, n. Labels outside
 * [0,V) make the row's terms NaN. workspace: glt_masked_ce_workspace_size
 * bytes, 256-byte aligned. */
size_t glt_masked_ce_workspace_size(int32_t B, int32_t T);
glt_status glt_masked_ce(const uint16_t* logits, int64_t ld, const int32_t* ids,
                         const int32_t* ood, int32_t B, int32_t T, int32_t V,
                         float scale, uint16_t* grad, int64_t ld_grad,
                         float* ce_per_token, float* stats, void* workspace,
                         size_t workspace_bytes, void* stream);

/* OOD silence terms on per-token graft outputs delta [tokens, slice]
 * (row stride ld): energy[t] = sqrt(sum delta^2 + 1e-8) / sqrt(slice)
 * (compute_energy_kernel, src/kernels_elementwise_impl.inc:222-275;
 * dtype GLT_DTYPE_F32 or GLT_DTYPE_BF16, e.g. the graft columns of
 * gate_pre); glt_silence_blend adds lambda / (||delta|| sqrt(slice)) * delta
 * to dy for tokens with ood != 0 (silence_blend_kernel, :8-67);
 * glt_silence_blend_energy does gate and up together, writing both energies
 * (NULL = skip) and blending tokens with ood == 1
 * (fused_silence_blend_energy_kernel, :458-560). f32, contiguous rows. */
glt_status glt_silence_energy(const void* delta, int32_t dtype, int64_t ld, int32_t tokens,
                              int32_t slice, float* energy, void* stream);
glt_status glt_silence_blend(float* dy, const float* delta, const int32_t* ood, int32_t tokens,
                             int32_t slice, float lambda, void* stream);
glt_status glt_silence_blend_energy(float* dy_gate, const float* delta_gate, float* dy_up,
                                    const float* delta_up, float* energy_gate, float* energy_up,
                                    const int32_t* ood, int32_t tokens, int32_t slice,
                                    float lambda, void* stream);

/* Learning rate of step `step` (0-based) of total_steps: linear warmup to
 * lr_peak over warmup_steps, then half-cosine decay (get_lr,
 * src/config.hpp:122-129). Host-only. */
float glt_lr_schedule(int32_t step, int32_t total_steps, int32_t warmup_steps, float lr_peak);

#ifdef __cplusplus
}
#endif
#endif /* GLT_H_ */
