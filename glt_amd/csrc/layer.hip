// Decoder layer forward with the grafted MLP (reference forward_layer,
// src/layer_forward_impl.inc:15-290): the attention block is frozen base
// code there (ATen); here every step runs on this library's kernels.
//
//   xn   = rms_norm(x, ln_in)                       glt_rmsnorm_fwd
//   q,k,v = xn . W_{q,k,v}^T                         one MFMA launch, 3 problems
//   RoPE(q, k)                                       glt_rope_fwd
//   a    = causal GQA SDPA(q, k, v)                  glt_attention_fwd
//   x   += a . W_o^T                                 MFMA, residual epilogue
//   x_ffn = rms_norm(x, ln_post)                     glt_rmsnorm_fwd
//   x   += grafted_mlp(x_ffn)                        glt_mlp_fwd (GLT_MLP_RESIDUAL)
#include <cmath>

#include "gemm.hpp"
#include "layout.hpp"

namespace glt {

namespace {

constexpr size_t kAlign = 256;
size_t up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

struct Dims {
  int64_t M, D, nq, nk;  // tokens, hidden, q width, k/v width
};
Dims dims(const glt_layer_desc* d) {
  return {(int64_t)d->B * d->T, d->mlp.D, (int64_t)d->n_q_heads * d->head_dim,
          (int64_t)d->n_kv_heads * d->head_dim};
}

// prepared: W_q, W_k, W_v (K = D) and W_o (K = q width), each shuffled
struct Prep {
  size_t q, k, v, o, total;
};
Prep prep_layout(const glt_layer_desc* d) {
  const Dims m = dims(d);
  Prep p{};
  p.q = 0;
  p.k = up(p.q + shuf_elems(m.nq, m.D) * 2);
  p.v = up(p.k + shuf_elems(m.nk, m.D) * 2);
  p.o = up(p.v + shuf_elems(m.nk, m.D) * 2);
  p.total = up(p.o + shuf_elems(m.D, m.nq) * 2);
  return p;
}

// workspace: xn, q, k, v, attention output, RMSNorm mean squares, and the
// MLP's inter when the caller does not keep it
struct Ws {
  size_t xn, q, k, v, a, var_in, var_post, inter, total;
};
Ws ws_layout(const glt_layer_desc* d) {
  const Dims m = dims(d);
  const int64_t N = d->mlp.N;
  Ws w{};
  w.xn = 0;
  w.q = up(w.xn + m.M * m.D * 2);
  w.k = up(w.q + m.M * m.nq * 2);
  w.v = up(w.k + m.M * m.nk * 2);
  w.a = up(w.v + m.M * m.nk * 2);
  w.var_in = up(w.a + m.M * m.nq * 2);
  w.var_post = up(w.var_in + m.M * 4);
  w.inter = up(w.var_post + m.M * 4);
  w.total = up(w.inter + m.M * N * 2);
  return w;
}

glt_status check_layer(const glt_layer_desc* d, const glt_layer_weights* w, const char* who) {
  GLT_CHECK(d && w, GLT_ERR_INVALID_ARG, "%s: null descriptor/weights", who);
  GLT_CHECK(d->B >= 0 && d->T >= 0 && d->n_q_heads > 0 && d->n_kv_heads > 0 &&
                d->n_q_heads % d->n_kv_heads == 0,
            GLT_ERR_SHAPE, "%s: B=%d T=%d heads %d/%d", who, d->B, d->T, d->n_q_heads, d->n_kv_heads);
  GLT_CHECK(d->head_dim == 128, GLT_ERR_UNSUPPORTED, "%s: head_dim %d (only 128)", who, d->head_dim);
  GLT_CHECK(d->mlp.dtype == GLT_DTYPE_BF16, GLT_ERR_DTYPE, "%s: the decoder layer runs in bf16", who);
  GLT_CHECK((int64_t)d->mlp.M == (int64_t)d->B * d->T, GLT_ERR_SHAPE, "%s: mlp.M=%d != B*T=%lld", who, d->mlp.M,
            (long long)d->B * d->T);
  GLT_CHECK(w->q_proj && w->k_proj && w->v_proj && w->o_proj && w->ln_in && w->ln_post, GLT_ERR_INVALID_ARG,
            "%s: null projection / norm weight", who);
  return GLT_OK;
}

GSeg seg(const void* A, int64_t lda, int K, int N, const void* B, int64_t ldb) {
  GSeg s{};
  s.A = A; s.lda = lda; s.a_ks = 1; s.a_col = 0; s.K = K; s.n_lo = 0; s.n_hi = N;
  s.B0 = B; s.ldb0 = ldb; s.b0_row0 = 0; s.b_ks = 1;
  return s;
}
GProb prob(int64_t M, int64_t N, int mode, void* out) {
  GProb p{};
  p.M = (int)M; p.N = (int)N; p.mode = mode; p.out_f32 = 0; p.alpha = 1.f; p.beta = 0.f;
  p.out0 = out; p.ldo = N;
  return p;
}

// Runs out_j = A . W_j^T for the listed problems, on the MFMA kernel with
// the prepared (shuffled) weights when the shapes allow it, else on the
// strided kernel with the row-major weights.
struct Proj {
  const void* w;        // row-major [N, K]
  const uint16_t* shuf; // prepared
  int64_t N;
  void* out;
};
glt_status project(const void* A, int64_t M, int64_t K, const Proj* ps, int n, int mode, const char* label,
                   hipStream_t st) {
  GemmPlan plan;
  plan.label = label;
  plan.a_kind = LD_BF16;
  plan.b_kind = LD_SHUF;
  for (int j = 0; j < n; ++j) {
    plan.add_problem(prob(M, ps[j].N, mode, ps[j].out));
    plan.add_seg(seg(A, K, (int)K, (int)ps[j].N, ps[j].shuf, shuf_k(K)));
  }
  if (gemm_mfma_eligible(plan)) return run_gemm(plan, st);
  GemmPlan gen;
  gen.label = label;
  gen.a_kind = gen.b_kind = LD_BF16;
  for (int j = 0; j < n; ++j) {
    gen.add_problem(prob(M, ps[j].N, mode, ps[j].out));
    gen.add_seg(seg(A, K, (int)K, (int)ps[j].N, ps[j].w, K));
  }
  return run_gemm(gen, st, false);
}

}  // namespace

}  // namespace glt

using namespace glt;

extern "C" {

size_t glt_attn_prepared_size(const glt_layer_desc* d) { return d ? prep_layout(d).total : 0; }

glt_status glt_attn_prepare(const glt_layer_desc* d, const glt_layer_weights* w, void* prepared, void* stream) {
  glt_status s = check_layer(d, w, "glt_attn_prepare");
  if (s != GLT_OK) return s;
  GLT_CHECK(prepared && reinterpret_cast<uintptr_t>(prepared) % kAlign == 0, GLT_ERR_ALIGNMENT,
            "glt_attn_prepare: prepared must be %zu-byte aligned", kAlign);
  const Dims m = dims(d);
  const Prep p = prep_layout(d);
  uint16_t* base = static_cast<uint16_t*>(prepared);
  hipStream_t st = as_stream(stream);
  struct Job { const void* src; int64_t rows, K; size_t off; };
  const Job jobs[4] = {{w->q_proj, m.nq, m.D, p.q}, {w->k_proj, m.nk, m.D, p.k}, {w->v_proj, m.nk, m.D, p.v},
                       {w->o_proj, m.D, m.nq, p.o}};
  for (const Job& j : jobs) {
    s = shuffle_b(j.src, GLT_DTYPE_BF16, j.K, false, (int)j.rows, (int)j.K, base + j.off / 2, st);
    if (s != GLT_OK) return s;
  }
  return GLT_OK;
}

size_t glt_layer_fwd_workspace_size(const glt_layer_desc* d) { return d ? ws_layout(d).total : 0; }

glt_status glt_layer_fwd(const glt_layer_desc* d, const glt_layer_weights* w, void* x, void* x_ffn, float* ffn_var,
                         void* gate_pre, void* up_pre, void* inter, void* workspace, size_t workspace_bytes,
                         void* stream) {
  glt_status s = check_layer(d, w, "glt_layer_fwd");
  if (s != GLT_OK) return s;
  const Dims m = dims(d);
  if (m.M == 0) return GLT_OK;
  const Ws L = ws_layout(d);
  GLT_CHECK(x && x_ffn && w->prepared, GLT_ERR_INVALID_ARG, "glt_layer_fwd: null x/x_ffn/prepared");
  GLT_CHECK(workspace && workspace_bytes >= L.total && reinterpret_cast<uintptr_t>(workspace) % kAlign == 0,
            GLT_ERR_WORKSPACE, "glt_layer_fwd: needs %zu workspace bytes, %zu-byte aligned", L.total, kAlign);
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  uint16_t* xn = reinterpret_cast<uint16_t*>(ws + L.xn);
  uint16_t* q = reinterpret_cast<uint16_t*>(ws + L.q);
  uint16_t* k = reinterpret_cast<uint16_t*>(ws + L.k);
  uint16_t* v = reinterpret_cast<uint16_t*>(ws + L.v);
  uint16_t* a = reinterpret_cast<uint16_t*>(ws + L.a);
  float* var_in = reinterpret_cast<float*>(ws + L.var_in);
  float* var_post = ffn_var ? ffn_var : reinterpret_cast<float*>(ws + L.var_post);
  const Prep P = prep_layout(d);
  const uint16_t* pb = static_cast<const uint16_t*>(w->prepared);

  // attention block (reference :29-55)
  s = glt_rmsnorm_fwd(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w->ln_in), xn, var_in,
                      (int32_t)m.M, (int32_t)m.D, d->rms_eps, stream);
  if (s != GLT_OK) return s;
  const Proj qkv[3] = {{w->q_proj, pb + P.q / 2, m.nq, q}, {w->k_proj, pb + P.k / 2, m.nk, k},
                       {w->v_proj, pb + P.v / 2, m.nk, v}};
  if ((s = project(xn, m.M, m.D, qkv, 3, EPI_STORE, "qkv", st)) != GLT_OK) return s;
  if (d->rope_theta > 0.f) {
    s = glt_rope_fwd(q, d->n_q_heads, k, d->n_kv_heads, d->B, d->T, d->head_dim, d->rope_theta, 0, stream);
    if (s != GLT_OK) return s;
  }
  s = glt_attention_fwd(q, k, v, a, d->B, d->T, d->n_q_heads, d->n_kv_heads, d->head_dim,
                        1.0f / std::sqrt((float)d->head_dim), 1, stream);
  if (s != GLT_OK) return s;
  const Proj o = {w->o_proj, pb + P.o / 2, m.D, x};
  if ((s = project(a, m.M, m.nq, &o, 1, EPI_RESID, "o_proj", st)) != GLT_OK) return s;

  // grafted MLP block (reference :57-290)
  s = glt_rmsnorm_fwd(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w->ln_post),
                      static_cast<uint16_t*>(x_ffn), var_post, (int32_t)m.M, (int32_t)m.D, d->rms_eps, stream);
  if (s != GLT_OK) return s;
  glt_mlp_desc md = d->mlp;
  md.flags |= GLT_MLP_RESIDUAL;
  return glt_mlp_fwd(&md, &w->mlp, x_ffn, x, gate_pre, up_pre, inter ? inter : ws + L.inter, stream);
}

}  // extern "C"
