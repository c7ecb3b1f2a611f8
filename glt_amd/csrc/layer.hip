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
#include <algorithm>
#include <cmath>
#include <vector>

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
  size_t xn, q, k, v, a, var_in, var_post, inter, vt, total;
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
  w.vt = up(w.inter + m.M * N * 2);
  w.total = up(w.vt + glt_attention_workspace_size(d->B, d->T, d->n_kv_heads, d->head_dim));
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
  auto mfma_plan = [&](int64_t r0, int64_t rows, GemmPlan& plan) {
    plan.label = label;
    plan.a_kind = LD_BF16;
    plan.b_kind = LD_SHUF;
    for (int j = 0; j < n; ++j) {
      plan.add_problem(prob(rows, ps[j].N, mode, static_cast<char*>(ps[j].out) + r0 * ps[j].N * 2));
      plan.add_seg(seg(static_cast<const char*>(A) + r0 * K * 2, K, (int)K, (int)ps[j].N, ps[j].shuf, shuf_k(K)));
    }
  };
  {
    // on the MFMA kernel, in row blocks when the output passes 31-bit
    // offsets (run_gemm splits it)
    GemmPlan plan;
    mfma_plan(0, M, plan);
    GemmPlan probe;
    mfma_plan(0, std::min<int64_t>(M, 256), probe);
    if (gemm_mfma_eligible(plan) || gemm_mfma_eligible(probe)) return run_gemm(plan, st);
  }
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
                        1.0f / std::sqrt((float)d->head_dim), 1, ws + L.vt, L.total - L.vt, stream);
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

// ===================================================================== model
// forward_model (reference grafting.hip:224-271) and the shadow-eval
// statistics of its logits (grafting.hip:504-547).
namespace glt {
namespace {

// out[t] = table[ids[t]], 16 bytes per lane when rows allow it
__global__ void __launch_bounds__(256) embedding_kernel(const int32_t* ids, const uint16_t* table, int V, int D,
                                                        uint16_t* out, bool vec) {
  const int64_t t = blockIdx.x;
  const int id = ids[t];
  const bool ok = id >= 0 && id < V;
  const uint16_t* src = table + (int64_t)(ok ? id : 0) * D;
  uint16_t* dst = out + t * D;
  if (vec) {
    for (int c = threadIdx.x; c < D / 8; c += 256) {
      u32x4 v = reinterpret_cast<const u32x4*>(src)[c];
      if (!ok) v = u32x4{0u, 0u, 0u, 0u};
      reinterpret_cast<u32x4*>(dst)[c] = v;
    }
  } else {
    for (int c = threadIdx.x; c < D; c += 256) dst[c] = ok ? src[c] : (uint16_t)0;
  }
}

// Per-row eval terms: f64 sum / sum of squares of the f32 logits, for rows
// t < T-1 the f32 cross-entropy max + log(sum exp(x - max)) - x_label
// against ids[b, t+1], and (rows hash form only) an FNV-1a hash of the row.
struct EvalRow {
  double sum, sumsq;
  uint64_t hash;
  float nll;
  int32_t scored;
};
// the reference's offset basis (grafting.hip:505): the published FNV-1a basis
// 14695981039346656037 with its last digit missing; the hash is defined by it
constexpr uint64_t kFnvBasis = 1469598103934665603ULL;
constexpr uint64_t kFnvPrime = 1099511628211ULL;  // 2^40 + 0x1B3

// Row-hash form: every row is cut into kEvalChunks chunks of
// ceil(V / kEvalChunks) logits (the last ones shorter or empty), which
// defines that hash; one thread walks one chunk in order.
constexpr int kEvalChunks = 16;

__device__ __forceinline__ void chunk_range(int V, int c, int& v0, int& v1) {
  const int L = (V + kEvalChunks - 1) / kEvalChunks;
  v0 = min(V, c * L);
  v1 = min(V, v0 + L);
}

// The reference hash's passes cut every row into kHashChunks chunks of
// ceil(V / kHashChunks) logits rounded up to a multiple of 8 (16-byte chunk
// starts in rows that start on 16 bytes; the last chunks shorter or empty).
// Any cut gives the same hash. (64 chunks per row, 4x the threads, measured
// 2 % slower over the three passes at 16384 x 128256: the passes are bound
// by their arithmetic, not by the chunk walks' load latency.)
constexpr int kHashChunks = 16;

__device__ __forceinline__ void hash_chunk_range(int V, int c, int& v0, int& v1) {
  const int L = ((V + kHashChunks - 1) / kHashChunks + 7) & ~7;
  v0 = min(V, c * L);
  v1 = min(V, v0 + L);
}

// Calls f(bits) for the bf16 logits x[v0, v1) in order: eight 16-byte loads
// in flight per thread when the chunk is aligned, else one element a time.
template <typename F>
__device__ __forceinline__ void walk_chunk(const uint16_t* x, int v0, int v1, F&& f) {
  const bool vec = ((reinterpret_cast<uintptr_t>(x + v0) & 15) == 0) && ((v1 - v0) % 8 == 0);
  if (vec) {
    int v = v0;
    for (; v + 64 <= v1; v += 64) {
      u32x4 q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = *reinterpret_cast<const u32x4*>(x + v + 8 * i);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f(q[i][e] & 0xFFFFu);
          f(q[i][e] >> 16);
        }
    }
    for (; v < v1; v += 8) {
      const u32x4 q = *reinterpret_cast<const u32x4*>(x + v);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f(q[e] & 0xFFFFu);
        f(q[e] >> 16);
      }
    }
  } else {
    for (int v = v0; v < v1; ++v) f((uint32_t)x[v]);
  }
}

// Row-hash form: one workgroup per 16 rows, 16 threads per row: thread c of
// a row takes chunk c and accumulates its f64 sum and sum of squares, its
// maximum and the FNV-1a hash of the chunk's f32 bytes from the basis. The
// row's threads then share their maxima through LDS, sum exp(x - max) over
// their chunks, and thread 0 of the row adds the parts in chunk order and
// hashes the chunk hashes' little-endian bytes in order.
__global__ void __launch_bounds__(256) eval_rows_kernel(const uint16_t* logits, int64_t ld, const int32_t* ids, int B,
                                                        int T, int V, EvalRow* rows) {
  __shared__ float s_max[16][kEvalChunks], s_se[16][kEvalChunks];
  __shared__ double s_sum[16][kEvalChunks], s_sq[16][kEvalChunks];
  __shared__ uint64_t s_h[16][kEvalChunks];
  const int lr = threadIdx.x >> 4, c = threadIdx.x & (kEvalChunks - 1);
  const int64_t r = (int64_t)blockIdx.x * 16 + lr;
  const bool valid = r < (int64_t)B * T;
  int v0, v1;
  chunk_range(V, c, v0, v1);
  const uint16_t* x = logits + (valid ? r : 0) * ld;
  double s = 0.0, s2 = 0.0;
  float mx = -INFINITY;
  uint64_t h = kFnvBasis;
  if (valid)
    walk_chunk(x, v0, v1, [&](uint32_t h16) {
      const uint32_t bits = h16 << 16;
      const float f = __uint_as_float(bits);
      s += f;
      s2 += (double)f * f;
      mx = fmaxf(mx, f);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        h ^= (bits >> (8 * k)) & 0xFFu;
        h *= kFnvPrime;
      }
    });
  s_max[lr][c] = mx;
  __syncthreads();
  float rmx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kEvalChunks; ++k) rmx = fmaxf(rmx, s_max[lr][k]);
  const int b = valid ? (int)(r / T) : 0, t = valid ? (int)(r - (int64_t)b * T) : 0;
  const bool scored = valid && t < T - 1;
  float se = 0.f;
  if (scored) walk_chunk(x, v0, v1, [&](uint32_t h16) { se += expf(__uint_as_float(h16 << 16) - rmx); });
  s_se[lr][c] = se;
  s_sum[lr][c] = s;
  s_sq[lr][c] = s2;
  s_h[lr][c] = h;
  __syncthreads();
  if (!valid || c != 0) return;
  EvalRow o{0.0, 0.0, kFnvBasis, 0.f, 0};
  float tse = 0.f;
  for (int k = 0; k < kEvalChunks; ++k) {
    o.sum += s_sum[lr][k];
    o.sumsq += s_sq[lr][k];
    tse += s_se[lr][k];
    const uint64_t hk = s_h[lr][k];
    for (int j = 0; j < 8; ++j) {
      o.hash ^= (hk >> (8 * j)) & 0xFFu;
      o.hash *= kFnvPrime;
    }
  }
  if (scored) {
    const int label = ids[(int64_t)b * T + t + 1];
    const float xl = (label >= 0 && label < V) ? __uint_as_float((uint32_t)x[label] << 16) : NAN;
    o.nll = (rmx + logf(tse)) - xl;
    o.scored = 1;
  }
  rows[r] = o;
}

// (max, sum of exp(x - max)) pairs: the sum rescaled to the larger maximum
__device__ __forceinline__ void lse_merge(float& m, float& se, float m2, float se2) {
  const float M = fmaxf(m, m2);
  se = se * __expf(m - M) + se2 * __expf(m2 - M);
  m = M;
}

// Row statistics without the row hash (the reference hash runs in its own
// passes): one workgroup per row reads it once with coalesced 16-byte loads.
// Each thread keeps a running maximum m and the sum of exp(x - m), rescaled
// when m grows (once per 8 logits at most), and f64 sums of x and x^2; the
// threads' parts are merged by a butterfly in each wavefront and the four
// wavefront results in order.
__global__ void __launch_bounds__(256) eval_row_stats_kernel(const uint16_t* logits, int64_t ld, const int32_t* ids,
                                                             int T, int V, EvalRow* rows) {
  __shared__ float s_m[4], s_se[4];
  __shared__ double s_s[4], s_q[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t r = blockIdx.x;
  const uint16_t* x = logits + r * ld;
  double s = 0.0, s2 = 0.0;
  // The running maximum starts finite and low (-2^126: times log2(e) it
  // stays finite), so exp(-inf - m) is 0 and the first chunk's rescale of
  // the zero sum needs no test. Each chunk rescales the sum to the new
  // maximum (a factor of 1 when it did not grow), branch-free; exp(x - m)
  // is exp2(x log2(e) - m log2(e)), one fma per logit.
  constexpr float kLog2e = 1.4426950408889634f;
  float m = -8.5070592e37f, se = 0.f;
  auto add8 = [&](const u32x4& q) {
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = __uint_as_float(q[e] << 16);
      f[2 * e + 1] = __uint_as_float(q[e] & 0xFFFF0000u);
    }
    float lm = f[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) lm = fmaxf(lm, f[e]);
    const float mn = fmaxf(m, lm);
    const float mn2 = mn * kLog2e;
    se *= __builtin_amdgcn_exp2f(fmaf(m, kLog2e, -mn2));
    m = mn;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      se += __builtin_amdgcn_exp2f(fmaf(f[e], kLog2e, -mn2));
      // squared in f64 like the reference (static_cast<double>(f) * f): the
      // f32 square of a large or tiny logit overflows or underflows; the
      // product of two f32 values is exact in f64, so one fma is the
      // reference's multiply and add
      const double d = (double)f[e];
      s += d;
      s2 = __builtin_fma(d, d, s2);
    }
  };
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && V % 8 == 0) {
    const u32x4* xc = reinterpret_cast<const u32x4*>(x);
    const int nc = V >> 3;
    int c = tid;
    for (; c + 768 < nc; c += 1024) {
      u32x4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = __builtin_nontemporal_load(xc + c + 256 * u);
#pragma unroll
      for (int u = 0; u < 4; ++u) add8(q[u]);
    }
    for (; c < nc; c += 256) add8(__builtin_nontemporal_load(xc + c));
  } else {
    for (int v = tid; v < V; v += 256) {
      const float f = __uint_as_float((uint32_t)x[v] << 16);
      if (f > m) {
        se *= __expf(m - f);
        m = f;
      }
      se += __expf(f - m);
      const double d = (double)f;
      s += d;
      s2 = __builtin_fma(d, d, s2);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lse_merge(m, se, __shfl_xor(m, o, 64), __shfl_xor(se, o, 64));
    s += __shfl_xor(s, o, 64);
    s2 += __shfl_xor(s2, o, 64);
  }
  if (lane == 0) {
    s_m[tid >> 6] = m;
    s_se[tid >> 6] = se;
    s_s[tid >> 6] = s;
    s_q[tid >> 6] = s2;
  }
  __syncthreads();
  if (tid != 0) return;
  EvalRow o{s_s[0], s_q[0], kFnvBasis, 0.f, 0};
  float rmx = s_m[0], tse = s_se[0];
  for (int k = 1; k < 4; ++k) {
    o.sum += s_s[k];
    o.sumsq += s_q[k];
    lse_merge(rmx, tse, s_m[k], s_se[k]);
  }
  const int t = (int)(r % T);
  if (t < T - 1) {
    const int label = ids[r + 1];
    const float xl = (label >= 0 && label < V) ? __uint_as_float((uint32_t)x[label] << 16) : NAN;
    o.nll = (rmx + logf(tse)) - xl;
    o.scored = 1;
  }
  rows[r] = o;
}

// ------------------------------------------------ the reference's logits hash
// The reference hashes every f32 logit's four little-endian bytes in (b, t, v)
// order with one FNV-1a chain, h = (h ^ byte) * P mod 2^64 (grafting.hip:536-546),
// continued across its eval batches. That chain is computed here exactly, in
// parallel over the chunks of all rows (chunk k = row k / kHashChunks, part
// k % kHashChunks),
// in three passes:
//  * P is odd, so the low byte of h evolves on its own:
//    s' = ((s ^ byte) * P) mod 256. Bit j of s' depends only on bits 0..j of
//    s, so the low nibble is a 16-state chain. Pass 1 runs every chunk from
//    all 16 low nibbles, giving each chunk's map of 16 nibbles; an ordered
//    scan of the maps from the start hash's nibble gives every chunk's
//    starting low nibble.
//  * Pass 2 does the same for the high nibble of the low byte, each chunk's
//    16 runs starting from its known low nibble.
//  * With the low byte s of h known at every step, h ^ byte = h + ((s ^ byte)
//    - s), so a chunk maps h to h * P^(4 n) + B (n logits). Pass 3 runs every
//    chunk once from h = its starting low byte s, giving B = h_end - s P^(4n);
//    the (P^(4n), B) pairs compose in order, h <- h A + B.
// A bf16 logit widens to f32 bits w << 16: its bytes are 0, 0, lo, hi.
constexpr uint32_t kP16 = (uint32_t)(kFnvPrime & 0xFFFF);
constexpr uint32_t kP16sq = (uint32_t)((kFnvPrime * kFnvPrime) & 0xFFFF);
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_mul(uint32_t a, uint32_t k) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * (u16x2){(uint16_t)k, (uint16_t)k});
}

// Pass 1 in bit planes. Per logit the low nibble goes
//   s <- ((9 s ^ a) * 3 ^ b) * 3 mod 16   (P mod 16 = 3, a / b: low nibbles of lo / hi)
// and the 16 runs of a chunk are kept as four 16-bit planes (bit i of plane
// j = bit j of run i), two chunks of one row per thread in the two halves
// of each 32-bit plane: 9 s flips bit 3 by bit 0, 3 s = s + 2 s is a ripple
// carry over the planes, and XOR with a logit's bit is a XOR with that bit
// spread over the chunk's half. About 19 operations per logit, against 40
// for 16 runs held as 16-bit integers.
typedef short s16x2 __attribute__((ext_vector_type(2)));
struct Planes {
  uint32_t p0, p1, p2, p3;
};
// bit k of each 16-bit half of w, spread over that half (0 or 0xFFFF)
__device__ __forceinline__ uint32_t half_mask(uint32_t w, int k) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, w << (15 - k)) >> (s16x2){15, 15});
}
__device__ __forceinline__ void planes_x3(Planes& P) {
  const uint32_t c1 = P.p1 & P.p0, t = P.p2 ^ P.p1;
  const uint32_t c2 = (t & c1) | (~t & P.p2);  // carry into bit 3: majority of p2, p1, c1
  P.p3 ^= P.p2 ^ c2;
  P.p2 = t ^ c1;
  P.p1 ^= P.p0;
}
// one logit of each chunk: chunk A's 16 bits in the low half of w, B's high
__device__ __forceinline__ void planes_step(Planes& P, uint32_t w) {
  P.p3 ^= P.p0 ^ half_mask(w, 3);  // 9 s, then ^ a
  P.p0 ^= half_mask(w, 0);
  P.p1 ^= half_mask(w, 1);
  P.p2 ^= half_mask(w, 2);
  planes_x3(P);
  P.p0 ^= half_mask(w, 8);
  P.p1 ^= half_mask(w, 9);
  P.p2 ^= half_mask(w, 10);
  P.p3 ^= half_mask(w, 11);
  planes_x3(P);
}
// chunk pair kp = chunks 2 kp, 2 kp + 1 (the same row: kHashChunks is even);
// the second one is never longer than the first
static_assert(kHashChunks % 2 == 0, "chunk pairs share a row");
__global__ void __launch_bounds__(256) hash_lo_planes_kernel(const uint16_t* logits, int64_t ld, int64_t chunks, int V,
                                                             uint64_t* __restrict__ maps) {
  const int64_t kA = 2 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
  if (kA >= chunks) return;
  const uint16_t* x = logits + (kA / kHashChunks) * ld;
  int a0, a1, b0, b1;
  hash_chunk_range(V, (int)(kA & (kHashChunks - 1)), a0, a1);
  hash_chunk_range(V, (int)((kA + 1) & (kHashChunks - 1)), b0, b1);
  const int na = a1 - a0, nb = b1 - b0;
  Planes P{0xAAAAAAAAu, 0xCCCCCCCCu, 0xF0F0F0F0u, 0xFF00FF00u};  // run i starts at nibble i
  auto step2 = [&](uint32_t qa, uint32_t qb) {  // two logits of each chunk, in order
    planes_step(P, (qa & 0xFFFFu) | (qb << 16));
    planes_step(P, (qa >> 16) | (qb & 0xFFFF0000u));
  };
  int v = 0;
  const bool vec = ((reinterpret_cast<uintptr_t>(x + a0) | reinterpret_cast<uintptr_t>(x + b0)) & 15) == 0;
  if (vec) {
    const u32x4* xa = reinterpret_cast<const u32x4*>(x + a0);
    const u32x4* xb = reinterpret_cast<const u32x4*>(x + b0);
    for (; v + 32 <= nb; v += 32) {
      u32x4 qa[4], qb[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        qa[u] = xa[(v >> 3) + u];
        qb[u] = xb[(v >> 3) + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) step2(qa[u][e], qb[u][e]);
    }
    for (; v + 8 <= nb; v += 8) {
      const u32x4 qa = xa[v >> 3], qb = xb[v >> 3];
#pragma unroll
      for (int e = 0; e < 4; ++e) step2(qa[e], qb[e]);
    }
  }
  for (; v < nb; ++v) planes_step(P, (uint32_t)x[a0 + v] | ((uint32_t)x[b0 + v] << 16));
  // the rest of chunk A (B ran out): B's half of every plane is kept
  for (; v < na; ++v) {
    const Planes Q = P;
    planes_step(P, (uint32_t)x[a0 + v]);
    P.p0 = (P.p0 & 0xFFFFu) | (Q.p0 & 0xFFFF0000u);
    P.p1 = (P.p1 & 0xFFFFu) | (Q.p1 & 0xFFFF0000u);
    P.p2 = (P.p2 & 0xFFFFu) | (Q.p2 & 0xFFFF0000u);
    P.p3 = (P.p3 & 0xFFFFu) | (Q.p3 & 0xFFFF0000u);
  }
  uint64_t mA = 0, mB = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t sa = ((P.p0 >> i) & 1u) | (((P.p1 >> i) & 1u) << 1) | (((P.p2 >> i) & 1u) << 2) |
                        (((P.p3 >> i) & 1u) << 3);
    const uint32_t sb = ((P.p0 >> (16 + i)) & 1u) | (((P.p1 >> (16 + i)) & 1u) << 1) |
                        (((P.p2 >> (16 + i)) & 1u) << 2) | (((P.p3 >> (16 + i)) & 1u) << 3);
    mA |= (uint64_t)sa << (4 * i);
    mB |= (uint64_t)sb << (4 * i);
  }
  maps[kA] = mA;
  maps[kA + 1] = mB;
}

// Pass 2: 16 runs of the low-byte chain over chunk k, two per register
// (16-bit halves; the low byte of a product depends only on the operands'
// low bytes, so the high bytes may hold anything), run i starting at
// (i << 4) | the chunk's starting low nibble. maps[k] nibble i = the final
// high nibble of run i.
__global__ void __launch_bounds__(256) hash_hi_nibble_kernel(const uint16_t* logits, int64_t ld, int64_t chunks, int V,
                                                             const uint8_t* __restrict__ start_lo,
                                                             uint64_t* __restrict__ maps) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= chunks) return;
  const uint32_t base = start_lo[k];
  uint32_t st[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) st[i] = (base | ((2 * i) << 4)) | ((base | ((2 * i + 1) << 4)) << 16);
  int v0, v1;
  hash_chunk_range(V, (int)(k & (kHashChunks - 1)), v0, v1);
  walk_chunk(logits + (k / kHashChunks) * ld, v0, v1, [&](uint32_t w) {
    const uint32_t lo = (w & 0xFFu) * 0x10001u, hi = (w >> 8) * 0x10001u;
#pragma unroll
    for (int i = 0; i < 8; ++i) st[i] = pk_mul(pk_mul(pk_mul(st[i], kP16sq) ^ lo, kP16) ^ hi, kP16);
  });
  uint64_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint32_t v = (st[i] >> (16 * hh)) & 0xFFu;
      m |= (uint64_t)(v >> 4) << (4 * (2 * i + hh));
    }
  maps[k] = m;
}

// 16-nibble maps: apply, and compose (first f, then g).
__device__ __forceinline__ uint32_t nib_apply(uint64_t f, uint32_t s) { return (uint32_t)(f >> (4 * s)) & 15u; }
__device__ __forceinline__ uint64_t nib_compose(uint64_t f, uint64_t g) {
  uint64_t h = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) h |= (uint64_t)nib_apply(g, nib_apply(f, i)) << (4 * i);
  return h;
}
constexpr uint64_t kNibIdentity = 0xFEDCBA9876543210ull;
constexpr int kScanPer = 4, kScanBlock = 256 * kScanPer;  // chunks per scan workgroup

// Ordered scan of the chunk maps, step 1: each workgroup's composition of
// its kScanBlock maps (in order, by an order-preserving tree in LDS).
__global__ void __launch_bounds__(256) nib_scan_up_kernel(const uint64_t* __restrict__ maps, int64_t chunks,
                                                          uint64_t* __restrict__ agg) {
  __shared__ uint64_t s[256];
  const int t = threadIdx.x;
  uint64_t f = kNibIdentity;
  for (int i = 0; i < kScanPer; ++i) {
    const int64_t k = (int64_t)blockIdx.x * kScanBlock + t * kScanPer + i;
    if (k < chunks) f = nib_compose(f, maps[k]);
  }
  s[t] = f;
  __syncthreads();
  for (int w = 1; w < 256; w *= 2) {
    if ((t & (2 * w - 1)) == 0) s[t] = nib_compose(s[t], s[t + w]);
    __syncthreads();
  }
  if (t == 0) agg[blockIdx.x] = s[0];
}

// Step 2: the starting nibble of every workgroup, in order from `start`:
// each thread composes a run of consecutive workgroup maps, thread 0 walks
// the 256 run maps, and each thread then walks its own run.
__global__ void __launch_bounds__(256) nib_scan_top_kernel(const uint64_t* __restrict__ agg, int64_t nblocks,
                                                           uint32_t start, uint8_t* __restrict__ bstart) {
  __shared__ uint64_t run[256];
  __shared__ uint8_t rs[256];
  const int t = threadIdx.x;
  const int64_t q = (nblocks + 255) / 256;
  const int64_t b0 = min(nblocks, t * q), b1 = min(nblocks, b0 + q);
  uint64_t f = kNibIdentity;
  for (int64_t b = b0; b < b1; ++b) f = nib_compose(f, agg[b]);
  run[t] = f;
  __syncthreads();
  if (t == 0) {
    uint32_t s = start;
    for (int i = 0; i < 256; ++i) {
      rs[i] = (uint8_t)s;
      s = nib_apply(run[i], s);
    }
  }
  __syncthreads();
  uint32_t s = rs[t];
  for (int64_t b = b0; b < b1; ++b) {
    bstart[b] = (uint8_t)s;
    s = nib_apply(agg[b], s);
  }
}

// Step 3: every chunk's starting nibble. OR_SHIFT 0 writes it to out[k];
// 4 ORs it in as the high nibble (out then holds whole starting bytes).
template <int OR_SHIFT>
__global__ void __launch_bounds__(256) nib_scan_down_kernel(const uint64_t* __restrict__ maps, int64_t chunks,
                                                            const uint8_t* __restrict__ bstart,
                                                            uint8_t* __restrict__ out) {
  __shared__ uint64_t s[256];
  __shared__ uint8_t ts[256];
  const int t = threadIdx.x;
  uint64_t f = kNibIdentity;
  for (int i = 0; i < kScanPer; ++i) {
    const int64_t k = (int64_t)blockIdx.x * kScanBlock + t * kScanPer + i;
    if (k < chunks) f = nib_compose(f, maps[k]);
  }
  s[t] = f;
  __syncthreads();
  if (t == 0) {
    uint32_t st = bstart[blockIdx.x];
    for (int i = 0; i < 256; ++i) {
      ts[i] = (uint8_t)st;
      st = nib_apply(s[i], st);
    }
  }
  __syncthreads();
  uint32_t st = ts[t];
  for (int i = 0; i < kScanPer; ++i) {
    const int64_t k = (int64_t)blockIdx.x * kScanBlock + t * kScanPer + i;
    if (k >= chunks) break;
    if (OR_SHIFT == 0) out[k] = (uint8_t)st;
    else out[k] = (uint8_t)(out[k] | (st << 4));
    st = nib_apply(maps[k], st);
  }
}

// h * P mod 2^64 with P = 2^40 + 0x1B3.
__device__ __forceinline__ uint64_t fnv_mul(uint64_t h) { return (h << 40) + h * 0x1B3ull; }

struct Affine {
  uint64_t a, b;  // h -> h * a + b
};
// first x, then y
__device__ __forceinline__ Affine affine_then(Affine x, Affine y) { return Affine{x.a * y.a, x.b * y.a + y.b}; }

// Pass 3: each chunk run once from h = its starting low byte, reduced to one
// affine map per workgroup of 256 chunks (order-preserving tree).
__global__ void __launch_bounds__(256) hash_affine_kernel(const uint16_t* logits, int64_t ld, int64_t chunks, int V,
                                                          const uint8_t* __restrict__ start_byte,
                                                          Affine* __restrict__ out) {
  __shared__ uint64_t sa[256], sb[256];
  const int t = threadIdx.x;
  const int64_t k = (int64_t)blockIdx.x * 256 + t;
  Affine f{1, 0};
  if (k < chunks) {
    int v0, v1;
    hash_chunk_range(V, (int)(k & (kHashChunks - 1)), v0, v1);
    const uint64_t s0 = start_byte[k];
    uint64_t h = s0;
    walk_chunk(logits + (k / kHashChunks) * ld, v0, v1, [&](uint32_t w) {
      h = fnv_mul(fnv_mul(h));
      h = fnv_mul(h ^ (w & 0xFFu));
      h = fnv_mul(h ^ (w >> 8));
    });
    // P^(4 n) by squaring
    uint64_t a = 1, p4 = fnv_mul(fnv_mul(fnv_mul(kFnvPrime)));
    for (uint32_t n = (uint32_t)(v1 - v0); n; n >>= 1, p4 *= p4)
      if (n & 1) a *= p4;
    f = Affine{a, h - s0 * a};
  }
  sa[t] = f.a;
  sb[t] = f.b;
  __syncthreads();
  for (int w = 1; w < 256; w *= 2) {
    if ((t & (2 * w - 1)) == 0) {
      const Affine r = affine_then(Affine{sa[t], sb[t]}, Affine{sa[t + w], sb[t + w]});
      sa[t] = r.a;
      sb[t] = r.b;
    }
    __syncthreads();
  }
  if (t == 0) out[blockIdx.x] = Affine{sa[0], sb[0]};
}

struct ModelWs {
  size_t x, x_ffn, var, layer, total;
};
ModelWs model_ws(const glt_model* m) {
  const glt_layer_desc& d0 = m->descs[0];
  const int64_t M = (int64_t)d0.B * d0.T, D = d0.mlp.D;
  ModelWs w{};
  w.x = 0;
  w.x_ffn = up(w.x + M * D * 2);
  w.var = up(w.x_ffn + M * D * 2);
  w.layer = up(w.var + M * 4);
  size_t lw = 0;
  for (int l = 0; l < m->num_layers; ++l) lw = std::max(lw, glt_layer_fwd_workspace_size(&m->descs[l]));
  w.total = up(w.layer + lw);
  return w;
}

}  // namespace
}  // namespace glt

extern "C" {

glt_status glt_embedding(const int32_t* ids, int64_t n, const uint16_t* table, int32_t V, int32_t D, uint16_t* out,
                         void* stream) {
  GLT_CHECK(n >= 0 && V > 0 && D > 0, GLT_ERR_SHAPE, "glt_embedding: n=%lld V=%d D=%d", (long long)n, V, D);
  if (n == 0) return GLT_OK;
  GLT_CHECK(ids && table && out, GLT_ERR_INVALID_ARG, "glt_embedding: null pointer");
  const bool vec = D % 8 == 0 && (reinterpret_cast<uintptr_t>(table) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  GLT_LAUNCH("embedding", embedding_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream), ids, table, V, D, out,
             vec);
  GLT_LAUNCH_CHECK("embedding");
  return GLT_OK;
}

// prepared LM head: [V rows, K = D] (forward), then 256-byte aligned the
// transpose [D rows, K = V] (backward), both in the fragment layout
size_t lm_head_t_offset(int32_t V, int32_t D) { return up((size_t)shuf_elems(V, D) * 2); }

size_t glt_lm_head_prepared_size(int32_t V, int32_t D) {
  return (V > 0 && D > 0) ? lm_head_t_offset(V, D) + (size_t)shuf_elems(D, V) * 2 : 0;
}

glt_status glt_lm_head_prepare(const uint16_t* lm_head, int32_t V, int32_t D, void* prepared, void* stream) {
  GLT_CHECK(V > 0 && D > 0, GLT_ERR_SHAPE, "glt_lm_head_prepare: V=%d D=%d", V, D);
  GLT_CHECK(lm_head && prepared && reinterpret_cast<uintptr_t>(prepared) % kAlign == 0, GLT_ERR_ALIGNMENT,
            "glt_lm_head_prepare: null pointer or prepared not %zu-byte aligned", kAlign);
  hipStream_t st = as_stream(stream);
  uint16_t* p = static_cast<uint16_t*>(prepared);
  glt_status s = shuffle_b(lm_head, GLT_DTYPE_BF16, D, false, V, D, p, st);
  if (s != GLT_OK) return s;
  return shuffle_b(lm_head, GLT_DTYPE_BF16, D, true, D, V, p + lm_head_t_offset(V, D) / 2, st);
}

glt_status glt_lm_head_bwd(const uint16_t* grad, int32_t M, int32_t V, const uint16_t* lm_head, const void* prepared,
                           int32_t D, float* dx, void* stream) {
  GLT_CHECK(M >= 0 && D > 0 && V > 0, GLT_ERR_SHAPE, "glt_lm_head_bwd: M=%d D=%d V=%d", M, D, V);
  if (M == 0) return GLT_OK;
  GLT_CHECK(grad && lm_head && prepared && dx, GLT_ERR_INVALID_ARG, "glt_lm_head_bwd: null pointer");
  // dx[m, d] = sum_v grad[m, v] lm_head[v, d]: B(n = d, k = v) = lm_head^T
  const uint16_t* pt = static_cast<const uint16_t*>(prepared) + lm_head_t_offset(V, D) / 2;
  GemmPlan plan;
  plan.label = "lm_head_bwd";
  plan.a_kind = LD_BF16;
  plan.b_kind = LD_SHUF;
  GProb pr = prob(M, D, EPI_STORE, dx);
  pr.out_f32 = 1;
  plan.add_problem(pr);
  plan.add_seg(seg(grad, V, V, D, pt, shuf_k(V)));
  hipStream_t st = as_stream(stream);
  if (gemm_mfma_eligible(plan)) return run_gemm(plan, st);
  GemmPlan gen;
  gen.label = "lm_head_bwd";
  gen.a_kind = gen.b_kind = LD_BF16;
  gen.add_problem(pr);
  GSeg g = seg(grad, V, V, D, lm_head, 1);
  g.b_ks = D;  // B(n = d, k = v) = lm_head[v * D + d]
  gen.add_seg(g);
  return run_gemm(gen, st, false);
}

glt_status glt_lm_head_fwd(const uint16_t* x, int32_t M, int32_t D, const uint16_t* lm_head, const void* prepared,
                           int32_t V, uint16_t* logits, void* stream) {
  GLT_CHECK(M >= 0 && D > 0 && V > 0, GLT_ERR_SHAPE, "glt_lm_head_fwd: M=%d D=%d V=%d", M, D, V);
  if (M == 0) return GLT_OK;
  GLT_CHECK(x && lm_head && prepared && logits, GLT_ERR_INVALID_ARG, "glt_lm_head_fwd: null pointer");
  const Proj p = {lm_head, static_cast<const uint16_t*>(prepared), V, logits};
  return project(x, M, D, &p, 1, EPI_STORE, "lm_head", as_stream(stream));
}

size_t glt_model_fwd_workspace_size(const glt_model* m) {
  return (m && m->num_layers > 0 && m->descs) ? model_ws(m).total : 0;
}

glt_status glt_model_fwd(const glt_model* m, const int32_t* ids, uint16_t* logits, void* workspace,
                         size_t workspace_bytes, void* stream) {
  GLT_CHECK(m && m->num_layers > 0 && m->descs && m->layers && m->embed && m->final_norm && m->lm_head &&
                m->lm_head_prepared && m->V > 0,
            GLT_ERR_INVALID_ARG, "glt_model_fwd: incomplete model");
  const glt_layer_desc& d0 = m->descs[0];
  for (int l = 1; l < m->num_layers; ++l) {
    const glt_layer_desc& d = m->descs[l];
    GLT_CHECK(d.B == d0.B && d.T == d0.T && d.mlp.D == d0.mlp.D && d.n_q_heads == d0.n_q_heads &&
                  d.n_kv_heads == d0.n_kv_heads && d.head_dim == d0.head_dim,
              GLT_ERR_SHAPE, "glt_model_fwd: layer %d's shape differs from layer 0's", l);
  }
  const int64_t M = (int64_t)d0.B * d0.T;
  const int D = d0.mlp.D;
  if (M == 0) return GLT_OK;
  GLT_CHECK(ids && logits, GLT_ERR_INVALID_ARG, "glt_model_fwd: null ids/logits");
  const ModelWs W = model_ws(m);
  GLT_CHECK(workspace && workspace_bytes >= W.total && reinterpret_cast<uintptr_t>(workspace) % kAlign == 0,
            GLT_ERR_WORKSPACE, "glt_model_fwd: needs %zu workspace bytes, %zu-byte aligned", W.total, kAlign);
  char* ws = static_cast<char*>(workspace);
  uint16_t* x = reinterpret_cast<uint16_t*>(ws + W.x);
  uint16_t* x_ffn = reinterpret_cast<uint16_t*>(ws + W.x_ffn);
  float* var = reinterpret_cast<float*>(ws + W.var);
  glt_status s = glt_embedding(ids, M, m->embed, m->V, D, x, stream);
  if (s != GLT_OK) return s;
  for (int l = 0; l < m->num_layers; ++l) {
    glt_layer_desc d = m->descs[l];
    d.mlp.flags = m->use_explicit_graft ? (d.mlp.flags | GLT_MLP_EXPLICIT) : (d.mlp.flags & ~GLT_MLP_EXPLICIT);
    s = glt_layer_fwd(&d, &m->layers[l], x, x_ffn, var, nullptr, nullptr, nullptr, ws + W.layer,
                      W.total - W.layer, stream);
    if (s != GLT_OK) return s;
  }
  // final norm (into x_ffn) and the LM head
  s = glt_rmsnorm_fwd(x, m->final_norm, x_ffn, var, (int32_t)M, D, d0.rms_eps, stream);
  if (s != GLT_OK) return s;
  return glt_lm_head_fwd(x_ffn, (int32_t)M, D, m->lm_head, m->lm_head_prepared, m->V, logits, stream);
}

}  // extern "C"

namespace glt {
namespace {
struct EvalWs {
  size_t rows, maps, start, agg, bstart, aff, total;
  int64_t chunks, nscan, naff;
};
EvalWs eval_ws(int64_t R) {
  EvalWs w{};
  w.chunks = R * kHashChunks;
  w.nscan = cdiv(w.chunks, kScanBlock);
  w.naff = cdiv(w.chunks, 256);
  w.rows = 0;
  w.maps = up(w.rows + R * sizeof(EvalRow));
  w.start = up(w.maps + w.chunks * 8);
  w.agg = up(w.start + w.chunks);
  w.bstart = up(w.agg + w.nscan * 8);
  w.aff = up(w.bstart + w.nscan);
  w.total = up(w.aff + w.naff * sizeof(Affine));
  return w;
}

// Starting nibble of every chunk from the maps (ordered scan, three launches).
glt_status nib_scan(const EvalWs& w, char* ws, uint32_t start, bool high, hipStream_t st) {
  const uint64_t* maps = reinterpret_cast<const uint64_t*>(ws + w.maps);
  uint64_t* agg = reinterpret_cast<uint64_t*>(ws + w.agg);
  uint8_t* bstart = reinterpret_cast<uint8_t*>(ws + w.bstart);
  uint8_t* out = reinterpret_cast<uint8_t*>(ws + w.start);
  GLT_LAUNCH("eval_hash_scan", nib_scan_up_kernel, dim3((unsigned)w.nscan), dim3(256), 0, st, maps, w.chunks, agg);
  GLT_LAUNCH_CHECK("nib_scan_up");
  GLT_LAUNCH("eval_hash_scan", nib_scan_top_kernel, dim3(1), dim3(256), 0, st, agg, w.nscan, start, bstart);
  GLT_LAUNCH_CHECK("nib_scan_top");
  if (high)
    GLT_LAUNCH("eval_hash_scan", nib_scan_down_kernel<4>, dim3((unsigned)w.nscan), dim3(256), 0, st, maps, w.chunks,
               bstart, out);
  else
    GLT_LAUNCH("eval_hash_scan", nib_scan_down_kernel<0>, dim3((unsigned)w.nscan), dim3(256), 0, st, maps, w.chunks,
               bstart, out);
  GLT_LAUNCH_CHECK("nib_scan_down");
  return GLT_OK;
}
}  // namespace
}  // namespace glt

extern "C" {

size_t glt_eval_stats_workspace_size(int32_t B, int32_t T) {
  return (B > 0 && T > 0) ? eval_ws((int64_t)B * T).total : 256;
}

glt_status glt_eval_stats(const uint16_t* logits, int64_t ld, const int32_t* ids, int32_t B, int32_t T, int32_t V,
                          int32_t hash_mode, uint64_t hash_in, glt_eval_result* out, void* workspace,
                          size_t workspace_bytes, void* stream) {
  GLT_CHECK(out && B >= 0 && T >= 0 && V > 0 && ld >= V, GLT_ERR_SHAPE, "glt_eval_stats: B=%d T=%d V=%d", B, T, V);
  GLT_CHECK(hash_mode == GLT_EVAL_HASH_REFERENCE || hash_mode == GLT_EVAL_HASH_ROWS, GLT_ERR_INVALID_ARG,
            "glt_eval_stats: hash_mode %d", hash_mode);
  *out = glt_eval_result{0.0, 0, 0.0, 0.0, hash_in};
  const int64_t R = (int64_t)B * T;
  if (R == 0) return GLT_OK;
  GLT_CHECK(logits && ids, GLT_ERR_INVALID_ARG, "glt_eval_stats: null logits/ids");
  GLT_CHECK(workspace && workspace_bytes >= glt_eval_stats_workspace_size(B, T) &&
                reinterpret_cast<uintptr_t>(workspace) % kAlign == 0,
            GLT_ERR_WORKSPACE, "glt_eval_stats: needs %zu workspace bytes, %zu-byte aligned",
            glt_eval_stats_workspace_size(B, T), kAlign);
  const bool exact = hash_mode == GLT_EVAL_HASH_REFERENCE;
  const EvalWs w = eval_ws(R);
  GLT_CHECK(w.naff < INT32_MAX, GLT_ERR_SHAPE, "glt_eval_stats: %lld rows", (long long)R);
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  EvalRow* rows = reinterpret_cast<EvalRow*>(ws + w.rows);
  if (exact)
    GLT_LAUNCH("eval_rows", eval_row_stats_kernel, dim3((unsigned)R), dim3(256), 0, st, logits, ld, ids, T, V, rows);
  else
    GLT_LAUNCH("eval_rows", eval_rows_kernel, dim3((unsigned)((R + 15) / 16)), dim3(256), 0, st, logits, ld,
               ids, B, T, V, rows);
  GLT_LAUNCH_CHECK("eval_rows");
  Affine* aff = reinterpret_cast<Affine*>(ws + w.aff);
  if (exact) {
    uint64_t* maps = reinterpret_cast<uint64_t*>(ws + w.maps);
    uint8_t* start = reinterpret_cast<uint8_t*>(ws + w.start);
    const dim3 grid((unsigned)w.naff);
    GLT_LAUNCH("eval_hash_nibble", hash_lo_planes_kernel, dim3((unsigned)cdiv(w.chunks / 2, 256)), dim3(256), 0, st,
               logits, ld, w.chunks, V, maps);
    GLT_LAUNCH_CHECK("hash_nibble");
    glt_status s = nib_scan(w, ws, (uint32_t)(hash_in & 15), false, st);
    if (s != GLT_OK) return s;
    GLT_LAUNCH("eval_hash_nibble", hash_hi_nibble_kernel, grid, dim3(256), 0, st, logits, ld, w.chunks, V,
               (const uint8_t*)start, maps);
    GLT_LAUNCH_CHECK("hash_nibble");
    if ((s = nib_scan(w, ws, (uint32_t)((hash_in >> 4) & 15), true, st)) != GLT_OK) return s;
    GLT_LAUNCH("eval_hash_affine", hash_affine_kernel, grid, dim3(256), 0, st, logits, ld, w.chunks, V,
               (const uint8_t*)start, aff);
    GLT_LAUNCH_CHECK("hash_affine");
  }
  std::vector<EvalRow> h((size_t)R);
  std::vector<Affine> ha(exact ? (size_t)w.naff : 0);
  GLT_CHECK(hipMemcpyAsync(h.data(), rows, (size_t)R * sizeof(EvalRow), hipMemcpyDeviceToHost, st) == hipSuccess &&
                (!exact || hipMemcpyAsync(ha.data(), aff, ha.size() * sizeof(Affine), hipMemcpyDeviceToHost, st) ==
                               hipSuccess) &&
                hipStreamSynchronize(st) == hipSuccess,
            GLT_ERR_HIP, "glt_eval_stats: copy of the results failed");
  uint64_t hash = hash_in;
  for (const EvalRow& r : h) {
    out->logits_sum += r.sum;
    out->logits_sumsq += r.sumsq;
    if (r.scored) {
      out->total_nll += r.nll;
      ++out->count;
    }
    if (!exact)
      for (int k = 0; k < 8; ++k) {
        hash ^= (r.hash >> (8 * k)) & 0xFFu;
        hash *= kFnvPrime;
      }
  }
  for (const Affine& a : ha) hash = hash * a.a + a.b;
  out->logits_hash = hash;
  return GLT_OK;
}

}  // extern "C"
