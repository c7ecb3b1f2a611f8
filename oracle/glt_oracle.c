/*
 * glt_oracle.c — CPU restatement of the reference's grafted-SwiGLU layer path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the oracle the GPU library is
 * compared against; it is loaded by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg, and by nothing on the product path.
 *
 * Every function restates the reference's algorithm, including where it
 * rounds to bf16, and cites the reference file:line it follows. Dot products
 * accumulate in f64 (the reference accumulates in f32 inside rocBLAS/ATen in
 * an order this restatement cannot reproduce; f64 is the order-free truth the
 * tests measure both against).
 *
 * Matrices are row-major. bf16 tensors are passed as f32 arrays holding
 * bf16-representable values; rb() marks every point where the reference
 * rounds to bf16.
 *
 * Build: oracle/build.sh (gcc -O3 -fopenmp -shared).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ----------------------------------------------------------------- bf16 */
/* RNE via the 0x7FFF + lsb bias (reference src/kernels_elementwise_impl.inc:575-580,
 * src/gemm_impl.inc:69-80); widening is a 16-bit shift (:570-573). */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}
float orc_bf16_to_f32(uint16_t h) {
  uint32_t b = (uint32_t)h << 16;
  float f;
  memcpy(&f, &b, 4);
  return f;
}
static inline float rb(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

void orc_f32_to_bf16_vec(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}
void orc_round_bf16_vec(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = rb(x[i]);
}

/* ----------------------------------------------------------------- GEMM */
/* C[m*ldc + n] = alpha * sum_k A(m,k) B(n,k) + beta*C, with general strides:
 * A(m,k) = A[m*sam + k*sak], B(n,k) = B[n*sbn + k*sbk]. f64 accumulation.
 * (The six graft GEMM kinds of src/gemm_impl.inc:383-584 are all instances.) */
static float* pack_rows(int R, int K, const float* X, int64_t sr, int64_t sk) {
  /* contiguous copy X'[r*K + k] = X[r*sr + k*sk] */
  float* P = (float*)malloc(sizeof(float) * (size_t)R * (size_t)K);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < R; ++r)
    for (int k = 0; k < K; ++k) P[(int64_t)r * K + k] = X[(int64_t)r * sr + (int64_t)k * sk];
  return P;
}

void orc_gemm(int M, int N, int K, const float* A, int64_t sam, int64_t sak, const float* B, int64_t sbn,
              int64_t sbk, float* C, int64_t ldc, float alpha, float beta) {
  if ((sak != 1 || sbk != 1) && (int64_t)M * N * K > (1 << 16)) {
    /* strided operands: gather them K-contiguous once, then the NT loop */
    float* Ap = sak != 1 ? pack_rows(M, K, A, sam, sak) : NULL;
    float* Bp = sbk != 1 ? pack_rows(N, K, B, sbn, sbk) : NULL;
    orc_gemm(M, N, K, Ap ? Ap : A, Ap ? K : sam, 1, Bp ? Bp : B, Bp ? K : sbn, 1, C, ldc, alpha, beta);
    free(Ap);
    free(Bp);
    return;
  }
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      const float* a = A + (int64_t)m * sam;
      const float* b = B + (int64_t)n * sbn;
      double acc = 0.0;
      if (sak == 1 && sbk == 1) {
        double p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int k = 0;
        for (; k + 8 <= K; k += 8)
          for (int u = 0; u < 8; ++u) p[u] += (double)a[k + u] * (double)b[k + u];
        for (; k < K; ++k) acc += (double)a[k] * (double)b[k];
        acc += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      } else {
        for (int k = 0; k < K; ++k) acc += (double)a[(int64_t)k * sak] * (double)b[(int64_t)k * sbk];
      }
      float* c = C + (int64_t)m * ldc + n;
      const float r = (float)(alpha * acc);
      *c = beta != 0.f ? r + beta * *c : r;
    }
  }
}

/* NT form: C[M,N] = A[M,K] . B[N,K]^T (both K-contiguous). */
static void gemm_nt(int M, int N, int K, const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                    int64_t ldc) {
  orc_gemm(M, N, K, A, lda, 1, B, ldb, 1, C, ldc, 1.f, 0.f);
}

/* ------------------------------------------------------------ shadow bake */
/* Reference shadow_bake_kernel (src/shadow_bake_impl.inc:15-51):
 * mode 0 (expand, gate/up): base[i0+s, h0+h] = bf16(f32(base) + g[s,h])
 * mode 1 (contract, down):  base[h0+h, i0+s] = bf16(f32(base) + g[s,h])
 * base is bf16 bits with row stride ld; graft f32 [S,H]. */
void orc_bake_inplace(uint16_t* base, int64_t ld, const float* graft, int S, int H, int i0, int h0, int mode) {
  for (int s = 0; s < S; ++s)
    for (int h = 0; h < H; ++h) {
      const int64_t r = mode == 0 ? i0 + s : h0 + h;
      const int64_t c = mode == 0 ? h0 + h : i0 + s;
      uint16_t* p = base + r * ld + c;
      *p = orc_f32_to_bf16(orc_bf16_to_f32(*p) + graft[(int64_t)s * H + h]);
    }
}

/* ---------------------------------------------------------------- RMSNorm */
/* Reference rms_norm_fwd_kernel (src/kernels_rmsnorm_kernels.inc:8-60):
 * var = sum(x^2)/D (stored), r = rsqrt(var + eps), y = bf16((x*r)*w). */
void orc_rmsnorm_fwd(const float* x, const float* w, float* y, float* var, int M, int D, float eps) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    const float* xr = x + (int64_t)m * D;
    double ss = 0.0;
    for (int c = 0; c < D; ++c) ss += (double)xr[c] * xr[c];
    const float v = (float)(ss / D);
    const float r = (float)(1.0 / sqrt((double)v + (double)eps));
    var[m] = v;
    for (int c = 0; c < D; ++c) y[(int64_t)m * D + c] = rb(xr[c] * r * w[c]);
  }
}

/* Reference rms_norm_bwd_kernel (src/kernels_rmsnorm_kernels.inc:70-126):
 * r = rsqrt(var+eps), mean = sum(dy*x*w)/D, dx = dy*r*w - x*mean*r^3. */
void orc_rmsnorm_bwd(const float* dy, const float* x, const float* w, const float* var, float* dx, int M, int D,
                     float eps) {
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m) {
    const int64_t o = (int64_t)m * D;
    const double r = 1.0 / sqrt((double)var[m] + (double)eps);
    const double r3 = r * r * r;
    double acc = 0.0;
    for (int c = 0; c < D; ++c) acc += (double)dy[o + c] * x[o + c] * w[c];
    const double mean = acc / D;
    for (int c = 0; c < D; ++c) dx[o + c] = (float)(dy[o + c] * r * w[c] - x[o + c] * mean * r3);
  }
}

/* ------------------------------------------------------------------- RoPE */
/* Reference apply_rope (src/rope_impl.inc:8-39) on a bf16 tensor t
 * [B,T,nh,hd]: i2 = 2i as f32, inv = 1/pow(theta, i2/hd) (f32), ang = pos*inv
 * (f32), emb = [ang, ang]; c, s = bf16(cos/sin(emb)); then ATen bf16 ops, each
 * rounding: r1 = bf16(bf16(x1*c) - bf16(x2*s)), r2 = bf16(bf16(x2*c) + bf16(x1*s)).
 * exact_rounding = 0 gives the single-rounding form bf16(x1*c - x2*s). */
void orc_rope(float* t, int B, int T, int nh, int hd, float theta, int pos_offset, int exact_rounding) {
  const int half = hd / 2;
  float* cs = (float*)malloc(sizeof(float) * half * 2);
  for (int tt = 0; tt < T; ++tt) {
    const int pos = tt + pos_offset;
    for (int i = 0; i < half; ++i) {
      const float e = (float)(2 * i) / (float)hd;
      const float inv = 1.0f / powf(theta, e);
      const float ang = (float)pos * inv;
      cs[i] = rb(cosf(ang));
      cs[half + i] = rb(sinf(ang));
    }
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < nh; ++h) {
        float* p = t + (((int64_t)b * T + tt) * nh + h) * hd;
        for (int i = 0; i < half; ++i) {
          const float x1 = p[i], x2 = p[half + i], c = cs[i], s = cs[half + i];
          if (exact_rounding) {
            p[i] = rb(rb(x1 * c) - rb(x2 * s));
            p[half + i] = rb(rb(x2 * c) + rb(x1 * s));
          } else {
            p[i] = rb(x1 * c - x2 * s);
            p[half + i] = rb(x2 * c + x1 * s);
          }
        }
      }
  }
  free(cs);
}

/* ------------------------------------------------------------------ AdamW */
/* Global-L2 clip scale (reference reduce_l2/calc_scale, src/kernels_elementwise_impl.inc:133-197):
 * norm = sqrt(sum g^2 + 1e-8); scale = clip/norm if norm > clip else 1. */
float orc_clip_scale(const float* g, int64_t n, float clip) {
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += (double)g[i] * g[i];
  const float norm = (float)sqrt(s + 1e-8);
  return norm > clip ? clip / norm : 1.0f;
}

/* Reference adamw_fused_kernel (src/kernels_optimizer_impl.inc:27-51) with the
 * host-side bias corrections of execute_adamw_all (:64-65). */
void orc_adamw(float* w, const float* g, float* m, float* v, int64_t n, int step, float lr, float b1, float b2,
               float eps, float wd, float grad_scale) {
  const float b1c = 1.0f / (1.0f - powf(b1, (float)(step + 1)));
  const float b2c = 1.0f / (1.0f - powf(b2, (float)(step + 1)));
  for (int64_t i = 0; i < n; ++i) {
    const float gi = g[i] * grad_scale;
    const float mi = b1 * m[i] + (1.0f - b1) * gi;
    const float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const float mh = mi * b1c, vh = vi * b2c;
    const float denom = sqrtf(vh) + eps;
    w[i] = w[i] - lr * mh / denom - lr * wd * w[i];
  }
}

/* ------------------------------------------------------------- elementwise */
/* Reference fused_silu_product_kernel (src/kernels_elementwise_impl.inc:395-401):
 * sg = 1/(1+exp(-g)), out = bf16((g*sg)*u). */
void orc_silu_mul(const float* g, const float* u, float* out, int64_t n, int round_out) {
  for (int64_t i = 0; i < n; ++i) {
    const float sg = 1.0f / (1.0f + expf(-g[i]));
    const float r = g[i] * sg * u[i];
    out[i] = round_out ? rb(r) : r;
  }
}

/* Reference fused_gate_up_bwd_kernel (src/kernels_elementwise_impl.inc:107-117). */
void orc_gate_up_bwd(const float* gi, const float* g, const float* u, float* dg, float* du, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float sg = 1.0f / (1.0f + expf(-g[i]));
    const float gv = g[i] * sg;
    const float sgrad = sg * (1.0f + g[i] * (1.0f - sg));
    dg[i] = gi[i] * u[i] * sgrad;
    du[i] = gi[i] * gv;
  }
}

/* -------------------------------------------------------------- MLP layer */
typedef struct {
  int i0, s, h0, h;
  const float* gate; /* f32 [S,H] master, NULL = projection not grafted */
  const float* up;
  const float* down;
} orc_slice;

/* Forward of the reference's explicit graft path
 * (src/layer_forward_impl.inc:61-218):
 *   gate_pre = bf16(x . W_gate^T)                             (:72, ATen bf16 out)
 *   for each slice: delta = x[:, h-slice] . bf16(Dg)^T (f32)  (graft_gemm_fwd, src/gemm_impl.inc:388-445)
 *                   gate_pre[:, i-slice] = bf16(gate_pre + delta)  (fused_inject_clone_energy_kernel :314-326)
 *   up likewise (:118-139); inter = bf16((g*sg)*u)             (:156-170)
 *   y = bf16(inter . W_down^T)                                  (:180)
 *   for each slice: y[:, h-slice] = bf16(y + inter[:, i-slice] . bf16(Dd))   (:186-218)
 * Base rows [I,N) are zero (appended neurons). bf16 = 0 gives the f32 path
 * (no roundings). x [M,D], wg/wu [I,D], wd [D,I]; outputs [M,N] / [M,D]. */
void orc_mlp_fwd_mode(int M, int D, int I, int N, int bf16, int recompute, int n_slices, const orc_slice* sl,
                      const float* x, const float* wg, const float* wu, const float* wd, float* gate_pre,
                      float* up_pre, float* inter, float* y) {
  const int64_t MN = (int64_t)M * N;
  float* tmp = (float*)malloc(sizeof(float) * (size_t)M * (N > D ? N : D));
  float* dbf = NULL;
  for (int p = 0; p < 2; ++p) {
    const float* W = p == 0 ? wg : wu;
    float* out = p == 0 ? gate_pre : up_pre;
    memset(out, 0, sizeof(float) * MN);
    if (I > 0) {
      gemm_nt(M, I, D, x, D, W, D, tmp, I);
      for (int m = 0; m < M; ++m)
        for (int n = 0; n < I; ++n) out[(int64_t)m * N + n] = bf16 ? rb(tmp[(int64_t)m * I + n]) : tmp[(int64_t)m * I + n];
    }
    for (int j = 0; j < n_slices; ++j) {
      const orc_slice* s = &sl[j];
      const float* delta = p == 0 ? s->gate : s->up;
      if (!delta) continue;
      dbf = (float*)realloc(dbf, sizeof(float) * (size_t)s->s * s->h);
      for (int64_t e = 0; e < (int64_t)s->s * s->h; ++e) dbf[e] = bf16 ? rb(delta[e]) : delta[e];
      gemm_nt(M, s->s, s->h, x + s->h0, D, dbf, s->h, tmp, s->s);
      for (int m = 0; m < M; ++m)
        for (int c = 0; c < s->s; ++c) {
          float* o = out + (int64_t)m * N + s->i0 + c;
          /* forward: the f32 delta joins the bf16 base, one rounding;
           * recompute: the cached delta is cast to bf16 first and added in
           * bf16 (gate_slice.add_(delta.to(bf16))) */
          const float dv = tmp[(int64_t)m * s->s + c];
          const float r = *o + ((bf16 && recompute) ? rb(dv) : dv);
          *o = bf16 ? rb(r) : r;
        }
    }
  }
  orc_silu_mul(gate_pre, up_pre, inter, MN, bf16);
  if (!y) {
    free(dbf);
    free(tmp);
    return;
  }
  memset(y, 0, sizeof(float) * (size_t)M * D);
  if (I > 0) {
    gemm_nt(M, D, I, inter, N, wd, I, tmp, D);
    for (int64_t e = 0; e < (int64_t)M * D; ++e) y[e] = bf16 ? rb(tmp[e]) : tmp[e];
  }
  for (int j = 0; j < n_slices; ++j) {
    const orc_slice* s = &sl[j];
    if (!s->down) continue;
    dbf = (float*)realloc(dbf, sizeof(float) * (size_t)s->s * s->h);
    for (int64_t e = 0; e < (int64_t)s->s * s->h; ++e) dbf[e] = bf16 ? rb(s->down[e]) : s->down[e];
    /* contract forward: out[m,h] = sum_s inter[m, i0+s] * Dd[s,h] (src/graft_ops_impl.inc:33-114) */
    orc_gemm(M, s->h, s->s, inter + s->i0, N, 1, dbf, 1, s->h, tmp, s->h, 1.f, 0.f);
    for (int m = 0; m < M; ++m)
      for (int c = 0; c < s->h; ++c) {
        float* o = y + (int64_t)m * D + s->h0 + c;
        const float r = *o + tmp[(int64_t)m * s->h + c];
        *o = bf16 ? rb(r) : r;
      }
  }
  free(dbf);
  free(tmp);
}

void orc_mlp_fwd(int M, int D, int I, int N, int bf16, int n_slices, const orc_slice* sl, const float* x,
                 const float* wg, const float* wu, const float* wd, float* gate_pre, float* up_pre, float* inter,
                 float* y) {
  orc_mlp_fwd_mode(M, D, I, N, bf16, 0, n_slices, sl, x, wg, wu, wd, gate_pre, up_pre, inter, y);
}

/* The reference's recompute_ffn (src/layer_recompute_impl.inc:8-91): gate and
 * up from at::linear in bf16 (:20, :46), each slice's cached expand output
 * (the forward's f32 delta, acts.delta_gate_out) cast to bf16 and added into
 * the bf16 slice in place (:33-38, :59-64), i.e. bf16(bf16(base) +
 * bf16(delta)) where the forward rounds once, bf16(bf16(base) + delta)
 * (src/kernels_elementwise_impl.inc:314-326); inter = silu(gate)*up (:66-82). */
void orc_mlp_recompute(int M, int D, int I, int N, int n_slices, const orc_slice* sl, const float* x,
                       const float* wg, const float* wu, float* gate_pre, float* up_pre, float* inter) {
  orc_mlp_fwd_mode(M, D, I, N, 1, 1, n_slices, sl, x, wg, wu, NULL, gate_pre, up_pre, inter, NULL);
}

/* 64-bit FNV-1a over n bytes from h (the reference's logits hash step,
 * grafting.hip:536-546: h ^= byte; h *= 1099511628211). */
uint64_t orc_fnv1a64(const uint8_t* p, int64_t n, uint64_t h) {
  for (int64_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 1099511628211ULL;
  }
  return h;
}

/* Graft-only backward of the reference (src/layer_backward_impl.inc:34-361)
 * given the forward's gate_pre/up_pre/inter (bf16-valued in the bf16 path).
 *   gi = dy . W_down (f32 weights)                                 (:48)
 *   per slice (down): dDd[S,H] = inter_i^T . bf16(dy_h)            (:93-95, src/gemm_impl.inc:520-584)
 *                     gi[:, i-slice] += bf16(dy_h) . bf16(Dd)^T    (:144-155)
 *   dg = gi*u*sg*(1+g*(1-sg)), du = gi*g*sg (f32)                   (:165-188)
 *   per slice (gate/up): dDg = bf16(dg_i)^T . x_h, dDu likewise    (:305-330, src/gemm_impl.inc:450-514)
 *                        gx_h = bf16(dg_i).bf16(Dg) + bf16(du_i).bf16(Du)   (:311-342)
 *   dx = dg . W_gate + du . W_up (f32 weights); dx[:, h-slice] += gx_h     (:356-361)
 * grads: per slice 3 pointers (gate, up, down) [S,H], NULL = skip. */
void orc_mlp_bwd(int M, int D, int I, int N, int bf16, int n_slices, const orc_slice* sl, const float* x,
                 const float* wg, const float* wu, const float* wd, const float* gate_pre, const float* up_pre,
                 const float* inter, const float* dy, float* dx, float** grads) {
  const int64_t MN = (int64_t)M * N;
  float* gi = (float*)calloc((size_t)MN, sizeof(float));
  float* dg = (float*)malloc(sizeof(float) * (size_t)MN);
  float* du = (float*)malloc(sizeof(float) * (size_t)MN);
  float* tmp = (float*)malloc(sizeof(float) * (size_t)M * (N > D ? N : D));
  float* dyb = (float*)malloc(sizeof(float) * (size_t)M * D);
  for (int64_t e = 0; e < (int64_t)M * D; ++e) dyb[e] = bf16 ? rb(dy[e]) : dy[e];
  /* gi = dy . W_down over the base columns: gi[m, n] = sum_d dy[m,d] wd[d,n] */
  if (I > 0) {
    orc_gemm(M, I, D, dy, D, 1, wd, 1, I, tmp, I, 1.f, 0.f);
    for (int m = 0; m < M; ++m) memcpy(gi + (int64_t)m * N, tmp + (int64_t)m * I, sizeof(float) * I);
  }
  float* dbf = NULL;
  for (int j = 0; j < n_slices; ++j) {
    const orc_slice* s = &sl[j];
    if (!s->down) continue;
    if (grads && grads[3 * j + 2])
      /* dDd[s,h] = sum_m inter[m, i0+s] * bf16(dy[m, h0+h]) */
      orc_gemm(s->s, s->h, M, inter + s->i0, 1, N, dyb + s->h0, 1, D, grads[3 * j + 2], s->h, 1.f, 0.f);
    dbf = (float*)realloc(dbf, sizeof(float) * (size_t)s->s * s->h);
    for (int64_t e = 0; e < (int64_t)s->s * s->h; ++e) dbf[e] = bf16 ? rb(s->down[e]) : s->down[e];
    /* gi[m, i0+s] += sum_h bf16(dy[m,h0+h]) * bf16(Dd[s,h]) */
    orc_gemm(M, s->s, s->h, dyb + s->h0, D, 1, dbf, s->h, 1, gi + s->i0, N, 1.f, 1.f);
  }
  orc_gate_up_bwd(gi, gate_pre, up_pre, dg, du, MN);
  float* dgb = (float*)malloc(sizeof(float) * (size_t)MN);
  float* dub = (float*)malloc(sizeof(float) * (size_t)MN);
  for (int64_t e = 0; e < MN; ++e) {
    dgb[e] = bf16 ? rb(dg[e]) : dg[e];
    dub[e] = bf16 ? rb(du[e]) : du[e];
  }
  if (dx) {
    memset(dx, 0, sizeof(float) * (size_t)M * D);
    if (I > 0) {
      /* dx[m,d] = sum_n dg[m,n] wg[n,d] + du[m,n] wu[n,d] */
      orc_gemm(M, D, I, dg, N, 1, wg, 1, D, dx, D, 1.f, 0.f);
      orc_gemm(M, D, I, du, N, 1, wu, 1, D, dx, D, 1.f, 1.f);
    }
  }
  for (int j = 0; j < n_slices; ++j) {
    const orc_slice* s = &sl[j];
    const float* deltas[2] = {s->gate, s->up};
    const float* srcs[2] = {dgb, dub};
    for (int p = 0; p < 2; ++p) {
      if (!deltas[p]) continue;
      if (grads && grads[3 * j + p])
        /* dD[s,h] = sum_m bf16(d*[m, i0+s]) * x[m, h0+h] */
        orc_gemm(s->s, s->h, M, srcs[p] + s->i0, 1, N, x + s->h0, 1, D, grads[3 * j + p], s->h, 1.f, 0.f);
      if (dx) {
        dbf = (float*)realloc(dbf, sizeof(float) * (size_t)s->s * s->h);
        for (int64_t e = 0; e < (int64_t)s->s * s->h; ++e) dbf[e] = bf16 ? rb(deltas[p][e]) : deltas[p][e];
        /* dx[m, h0+h] += sum_s bf16(d*[m, i0+s]) * bf16(D[s,h]) */
        orc_gemm(M, s->h, s->s, srcs[p] + s->i0, N, 1, dbf, 1, s->h, dx + s->h0, D, 1.f, 1.f);
      }
    }
  }
  free(dbf);
  free(dgb);
  free(dub);
  free(dyb);
  free(tmp);
  free(du);
  free(dg);
  free(gi);
}
