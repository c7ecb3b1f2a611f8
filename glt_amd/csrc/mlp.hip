// Grafted SwiGLU MLP: forward, graft-only backward, graft-GEMM probes,
// base preparation. Host code that turns a glt_mlp_desc into segment-list
// GEMM launches (see gemm.hpp).
#include <algorithm>
#include <atomic>
#include <mutex>

#include "gemm.hpp"
#include "layout.hpp"
#include "norm_rope.hpp"

namespace glt {

glt_status transpose_any(const void* src, void* dst, int rows, int cols, int64_t src_ld, int dtype,
                         hipStream_t st);

static size_t esize(int dtype) { return dtype == GLT_DTYPE_F32 ? 4 : 2; }
static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Row-major packed-mirror orientation q = 2*proj + transposed (layout.hpp).
static const uint16_t* packed_block(const glt_graft_slice& s, int proj, bool transposed) {
  const int64_t sh = (int64_t)s.s * s.h;
  return s.packed + (2 * proj + (transposed ? 1 : 0)) * sh;
}
// Shuffled packed-mirror orientation.
static const uint16_t* packed_shuf(const glt_graft_slice& s, int proj, bool transposed) {
  return s.packed + packed_shuf_offset(s.s, s.h, 2 * proj + (transposed ? 1 : 0));
}
static const uint16_t* prep(const glt_mlp_desc* d, const glt_base_weights* w, int slot) {
  return static_cast<const uint16_t*>(w->prepared) + prep_offset(d->I, d->D, slot);
}

// The bf16 MLP runs on the MFMA kernel when every K is a multiple of 64,
// every output column range and every operand row offset is 32-aligned
// (whole shuffled B blocks) and the activation rows are 16-byte aligned;
// other shapes (and the f32 path) take the strided generic kernel.
static bool mlp_uses_mfma(const glt_mlp_desc* d) {
  if (d->dtype != GLT_DTYPE_BF16) return false;
  if (d->D % 64 || d->I % 64 || d->N % 8) return false;
  if (d->flags & GLT_MLP_EXPLICIT)
    for (int j = 0; j < d->n_slices; ++j) {
      const glt_graft_slice& s = d->slices[j];
      if (s.s % 64 || s.h % 64 || s.i_start % 32 || s.h_start % 32) return false;
    }
  return true;
}

static glt_status check_desc(const glt_mlp_desc* d, const glt_base_weights* w, const char* who) {
  GLT_CHECK(d && w, GLT_ERR_INVALID_ARG, "%s: null descriptor", who);
  GLT_CHECK(d->dtype == GLT_DTYPE_BF16 || d->dtype == GLT_DTYPE_F32, GLT_ERR_DTYPE, "%s: dtype %d", who, d->dtype);
  GLT_CHECK(d->M >= 0 && d->D > 0 && d->I >= 0 && d->N >= d->I && d->N > 0, GLT_ERR_SHAPE,
            "%s: bad dims M=%d D=%d I=%d N=%d", who, d->M, d->D, d->I, d->N);
  GLT_CHECK(d->n_slices >= 0 && d->n_slices <= 8, GLT_ERR_UNSUPPORTED, "%s: %d slices (max 8)", who, d->n_slices);
  GLT_CHECK(d->n_slices == 0 || d->slices, GLT_ERR_INVALID_ARG, "%s: null slices", who);
  GLT_CHECK(d->I == 0 || (w->gate && w->up && w->down), GLT_ERR_INVALID_ARG, "%s: null base weight", who);
  GLT_CHECK(d->I == 0 || !mlp_uses_mfma(d) || w->prepared, GLT_ERR_INVALID_ARG,
            "%s: the bf16 path needs the prepared base (glt_base_prepare)", who);
  const bool explicit_graft = d->flags & GLT_MLP_EXPLICIT;
  for (int j = 0; explicit_graft && j < d->n_slices; ++j) {
    const glt_graft_slice& s = d->slices[j];
    GLT_CHECK(s.i_start >= 0 && s.s > 0 && s.i_start + s.s <= d->N && s.h_start >= 0 && s.h > 0 &&
                  s.h_start + s.h <= d->D,
              GLT_ERR_SHAPE, "%s: slice %d {i0=%d S=%d h0=%d H=%d} outside N=%d D=%d", who, j, s.i_start, s.s,
              s.h_start, s.h, d->N, d->D);
    const bool any = s.master_gate || s.master_up || s.master_down;
    GLT_CHECK(d->dtype != GLT_DTYPE_BF16 || !any || s.packed, GLT_ERR_INVALID_ARG,
              "%s: slice %d has no packed bf16 mirror (glt_graft_pack)", who, j);
  }
  return GLT_OK;
}

static GSeg nt_seg(const void* A, int64_t lda, int a_col, int K, int n_lo, int n_hi, const void* B0, int64_t ldb0,
                   int b0_row0, const void* B1 = nullptr, int64_t ldb1 = 0, int b1_row0 = 0) {
  GSeg s{};
  s.A = A; s.lda = lda; s.a_ks = 1; s.a_col = a_col; s.K = K; s.n_lo = n_lo; s.n_hi = n_hi;
  s.B0 = B0; s.ldb0 = ldb0; s.b0_row0 = b0_row0; s.B1 = B1; s.ldb1 = ldb1; s.b1_row0 = b1_row0; s.b_ks = 1;
  return s;
}

static GProb prob(int M, int N, int mode, bool f32, void* o0, void* o1, void* o2, int64_t ldo,
                  const void* a0 = nullptr, const void* a1 = nullptr, int64_t ldaux = 0) {
  GProb p{};
  p.M = M; p.N = N; p.mode = mode; p.out_f32 = f32; p.alpha = 1.f; p.beta = 0.f;
  p.out0 = o0; p.out1 = o1; p.out2 = o2; p.ldo = ldo; p.aux0 = a0; p.aux1 = a1; p.ldaux = ldaux;
  return p;
}

// Operand kinds of a plan: MFMA path = bf16 A, shuffled B; otherwise the
// path dtype, strided.
static void set_kinds(GemmPlan& plan, const glt_mlp_desc* d, bool mfma) {
  plan.a_kind = d->dtype == GLT_DTYPE_F32 ? LD_F32 : LD_BF16;
  plan.b_kind = mfma ? LD_SHUF : plan.a_kind;
}

// gate/up concat-N GEMM with the SiLU*up epilogue.
static glt_status gate_up_forward(const glt_mlp_desc* d, const glt_base_weights* w, const void* x, void* g_out,
                                  void* u_out, void* inter, hipStream_t st) {
  const bool f32 = d->dtype == GLT_DTYPE_F32;
  const bool mfma = mlp_uses_mfma(d);
  GemmPlan plan;
  plan.dual = true;
  plan.label = "gate_up";
  set_kinds(plan, d, mfma);
  plan.add_problem(prob(d->M, d->N, EPI_SILU, f32, inter, g_out, u_out, d->N));
  if (d->I > 0) {
    if (mfma)
      plan.add_seg(nt_seg(x, d->D, 0, d->D, 0, d->I, prep(d, w, PREP_GATE), d->D, 0, prep(d, w, PREP_UP), d->D, 0));
    else
      plan.add_seg(nt_seg(x, d->D, 0, d->D, 0, d->I, w->gate, d->D, 0, w->up, d->D, 0));
  }
  if (d->flags & GLT_MLP_EXPLICIT) {
    for (int j = 0; j < d->n_slices; ++j) {
      const glt_graft_slice& s = d->slices[j];
      if (!s.master_gate && !s.master_up) continue;
      const void *bg, *bu;
      if (mfma) {
        bg = s.master_gate ? packed_shuf(s, 0, false) : nullptr;
        bu = s.master_up ? packed_shuf(s, 1, false) : nullptr;
      } else {
        bg = f32 ? (const void*)s.master_gate : (s.master_gate ? packed_block(s, 0, false) : nullptr);
        bu = f32 ? (const void*)s.master_up : (s.master_up ? packed_block(s, 1, false) : nullptr);
      }
      plan.add_seg(nt_seg(x, d->D, s.h_start, s.h, s.i_start, s.i_start + s.s, bg, s.h, s.i_start, bu, s.h,
                          s.i_start));
    }
  }
  return run_gemm(plan, st);
}

// down projection: K-concat of the base columns and each slice's rows.
static glt_status down_forward(const glt_mlp_desc* d, const glt_base_weights* w, const void* inter, void* y,
                               hipStream_t st) {
  const bool f32 = d->dtype == GLT_DTYPE_F32;
  const bool mfma = mlp_uses_mfma(d);
  GemmPlan plan;
  plan.label = "down";
  set_kinds(plan, d, mfma);
  plan.add_problem(prob(d->M, d->D, (d->flags & GLT_MLP_RESIDUAL) ? EPI_RESID : EPI_STORE, f32, y, nullptr, nullptr,
                        d->D));
  if (d->I > 0) plan.add_seg(nt_seg(inter, d->N, 0, d->I, 0, d->D, mfma ? prep(d, w, PREP_DOWN) : w->down, d->I, 0));
  if (d->flags & GLT_MLP_EXPLICIT) {
    for (int j = 0; j < d->n_slices; ++j) {
      const glt_graft_slice& s = d->slices[j];
      if (!s.master_down) continue;
      if (f32) {
        // B(n = h0+h, k = s) = delta_down[s, h]: read the [S,H] master strided
        GSeg g = nt_seg(inter, d->N, s.i_start, s.s, s.h_start, s.h_start + s.h, s.master_down, 1, s.h_start);
        g.b_ks = s.h;
        plan.add_seg(g);
      } else {
        plan.add_seg(nt_seg(inter, d->N, s.i_start, s.s, s.h_start, s.h_start + s.h,
                            mfma ? packed_shuf(s, 2, true) : packed_block(s, 2, true), s.s, s.h_start));
      }
    }
  }
  return run_gemm(plan, st);
}

struct BwdLayout {
  size_t dg, du, dyb, xt, dyt, g, u, inter, slice0, slice_stride, total;
  bool wgrad_mfma, dy_f32;
};

// The weight gradients reduce over the M tokens; on the MFMA kernel that K
// must be a multiple of 64 as well.
static bool wgrad_uses_mfma(const glt_mlp_desc* d) { return mlp_uses_mfma(d) && d->M % 64 == 0; }

static BwdLayout bwd_layout(const glt_mlp_desc* d) {
  BwdLayout L{};
  const size_t es = esize(d->dtype);
  const size_t MN = (size_t)d->M * d->N * es;
  L.wgrad_mfma = wgrad_uses_mfma(d);
  size_t off = 0;
  L.dg = off; off += align256(MN);
  L.du = off; off += align256(MN);
  // an f32 upstream gradient on the bf16 path is rounded once into here
  L.dy_f32 = (d->flags & GLT_MLP_DY_F32) && d->dtype == GLT_DTYPE_BF16;
  if (L.dy_f32) {
    L.dyb = off;
    off += align256((size_t)d->M * d->D * 2);
  }
  if (d->flags & GLT_MLP_RECOMPUTE) {
    L.g = off; off += align256(MN);
    L.u = off; off += align256(MN);
    L.inter = off; off += align256(MN);
  }
  const bool grads = (d->flags & GLT_MLP_EXPLICIT) && d->n_slices > 0;
  if (L.wgrad_mfma && grads) {
    // x and dy as shuffled B operands [D rows, K = M]
    L.xt = off; off += align256((size_t)shuf_elems(d->D, d->M) * 2);
    L.dyt = off; off += align256((size_t)shuf_elems(d->D, d->M) * 2);
    L.slice0 = off;
    size_t per = 0;
    for (int j = 0; j < d->n_slices; ++j) per = std::max(per, 3 * align256((size_t)d->slices[j].s * d->M * es));
    L.slice_stride = per;
    off += per * (size_t)d->n_slices;
  }
  L.total = off;
  return L;
}

}  // namespace glt

using namespace glt;

extern "C" {

size_t glt_base_prepared_size(const glt_mlp_desc* d) {
  if (!d || d->dtype != GLT_DTYPE_BF16 || d->I <= 0 || d->D <= 0) return 0;
  return (size_t)prep_bytes(d->I, d->D);
}

glt_status glt_base_prepare(const glt_mlp_desc* d, const void* gate, const void* up, const void* down,
                            void* prepared, void* stream) {
  GLT_CHECK(d, GLT_ERR_INVALID_ARG, "glt_base_prepare: null descriptor");
  GLT_CHECK(d->dtype == GLT_DTYPE_BF16 || d->dtype == GLT_DTYPE_F32, GLT_ERR_DTYPE, "glt_base_prepare: dtype");
  GLT_CHECK(d->D > 0 && d->I >= 0, GLT_ERR_SHAPE, "glt_base_prepare: dims");
  if (d->dtype == GLT_DTYPE_F32 || d->I == 0) return GLT_OK;  // the f32 path reads the base as is
  GLT_CHECK(gate && up && down && prepared, GLT_ERR_INVALID_ARG, "glt_base_prepare: null pointer");
  GLT_CHECK((reinterpret_cast<uintptr_t>(prepared) & 255) == 0, GLT_ERR_ALIGNMENT,
            "glt_base_prepare: prepared buffer must be 256-byte aligned");
  hipStream_t st = as_stream(stream);
  uint16_t* out = static_cast<uint16_t*>(prepared);
  const int I = d->I, D = d->D;
  struct Job { const void* src; int64_t ld; bool tr; int rows, K; };
  const Job jobs[6] = {
      {gate, D, false, I, D}, {up, D, false, I, D}, {down, I, false, D, I},
      {down, I, true, I, D},  {gate, D, true, D, I}, {up, D, true, D, I},
  };
  for (int q = 0; q < 6; ++q) {
    glt_status s = shuffle_b(jobs[q].src, GLT_DTYPE_BF16, jobs[q].ld, jobs[q].tr, jobs[q].rows, jobs[q].K,
                             out + prep_offset(I, D, q), st);
    if (s != GLT_OK) return s;
  }
  return GLT_OK;
}

glt_status glt_mlp_fwd(const glt_mlp_desc* d, const glt_base_weights* w, const void* x, void* y, void* gate_pre,
                       void* up_pre, void* inter, void* stream) {
  glt_status s = check_desc(d, w, "glt_mlp_fwd");
  if (s != GLT_OK) return s;
  GLT_CHECK(d->M == 0 || (x && y && inter), GLT_ERR_INVALID_ARG, "glt_mlp_fwd: null x/y/inter");
  if (d->M == 0) return GLT_OK;
  hipStream_t st = as_stream(stream);
  if ((s = gate_up_forward(d, w, x, gate_pre, up_pre, inter, st)) != GLT_OK) return s;
  return down_forward(d, w, inter, y, st);
}

size_t glt_mlp_bwd_workspace_size(const glt_mlp_desc* d) {
  if (!d) return 0;
  return bwd_layout(d).total;
}

namespace glt {
// The RMSNorm backward that glt_mlp_rmsnorm_bwd runs after the MLP backward.
struct NormBwd {
  const uint16_t* x;
  const uint16_t* w;
  const float* var;
  float eps;
  float* dx;
};

// Helper stream of the current device (created once, default priority) on
// which the RMSNorm backward runs beside the weight-gradient GEMM.
static glt_status helper_stream(hipStream_t& out) {
  static std::atomic<hipStream_t> streams[64];
  static std::mutex mu;
  int dev = 0;
  GLT_TRY_HIP(hipGetDevice(&dev));
  GLT_CHECK(dev >= 0 && dev < 64, GLT_ERR_HIP, "helper stream: device index %d out of range", dev);
  hipStream_t h = streams[dev].load(std::memory_order_acquire);
  if (!h) {
    std::lock_guard<std::mutex> lk(mu);
    h = streams[dev].load(std::memory_order_acquire);
    if (!h) {
      GLT_TRY_HIP(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
      streams[dev].store(h, std::memory_order_release);
    }
  }
  out = h;
  return GLT_OK;
}

// Starts the RMSNorm backward of dx on the helper stream once everything
// enqueued on st so far is done, on `grid` persistent workgroups; *done is
// recorded on the helper stream after it (the caller waits for it on st and
// destroys it). Both events exist before the launch, so an error after it
// can still be made to wait for the launched kernel: no work of the call is
// left running once it has returned an error.
static glt_status fork_norm_bwd(const NormBwd& nb, const float* dx, int M, int D, int grid, hipStream_t st,
                                hipEvent_t* done) {
  hipStream_t hs = nullptr;
  glt_status s = helper_stream(hs);
  if (s != GLT_OK) return s;
  hipEvent_t ready = nullptr, fin = nullptr;
  GLT_TRY_HIP(hipEventCreateWithFlags(&ready, hipEventDisableTiming));
  hipError_t e = hipEventCreateWithFlags(&fin, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(ready, st);
  if (e == hipSuccess) e = hipStreamWaitEvent(hs, ready, 0);
  const hipError_t de = hipEventDestroy(ready);
  if (e == hipSuccess) e = de;
  if (e != hipSuccess) {
    if (fin) (void)hipEventDestroy(fin);
    GLT_TRY_HIP(e);
  }
  s = rmsnorm_bwd_rows(dx, nb.x, nb.w, nb.var, nb.dx, M, D, nb.eps, grid, hs);
  e = hipEventRecord(fin, hs);
  if (s != GLT_OK || e != hipSuccess) {
    // the kernel may have been enqueued: wait for the helper stream
    const hipError_t se = hipStreamSynchronize(hs);
    (void)hipEventDestroy(fin);
    if (s != GLT_OK) return s;
    GLT_TRY_HIP(e);
    GLT_TRY_HIP(se);
  }
  *done = fin;
  return GLT_OK;
}

// glt_mlp_bwd; with nb, the RMSNorm backward of dx starts beside the
// weight-gradient GEMM when that launch leaves CUs idle (*norm_done set),
// else the caller runs it afterwards.
static glt_status mlp_bwd_impl(const glt_mlp_desc* d, const glt_base_weights* w, const void* x, const void* dy,
                               const void* gate_pre, const void* up_pre, const void* inter, float* dx,
                               const glt_graft_grads* grads, void* ws, size_t ws_bytes, hipStream_t st,
                               const NormBwd* nb, bool* norm_done) {
  glt_status s = check_desc(d, w, "glt_mlp_bwd");
  if (s != GLT_OK) return s;
  GLT_CHECK(!(d->state && d->state->baked), GLT_ERR_BAKED_NO_BACKWARD,
            "glt_mlp_bwd: backward on a shadow-baked model is forbidden");
  const bool recompute = d->flags & GLT_MLP_RECOMPUTE;
  GLT_CHECK(d->M == 0 || (x && dy && (recompute || (gate_pre && up_pre && inter))), GLT_ERR_INVALID_ARG,
            "glt_mlp_bwd: null x/dy or saved activations (set GLT_MLP_RECOMPUTE to recompute them)");
  const bool explicit_graft = d->flags & GLT_MLP_EXPLICIT;
  GLT_CHECK(!explicit_graft || d->n_slices == 0 || grads, GLT_ERR_INVALID_ARG, "glt_mlp_bwd: null grads");
  const BwdLayout L = bwd_layout(d);
  GLT_CHECK(ws_bytes >= L.total && (L.total == 0 || ws), GLT_ERR_WORKSPACE,
            "glt_mlp_bwd: workspace %zu bytes < required %zu", ws_bytes, L.total);
  if (d->M == 0) return GLT_OK;
  char* W = static_cast<char*>(ws);
  const bool f32 = d->dtype == GLT_DTYPE_F32;
  const bool mfma = mlp_uses_mfma(d);
  const int kind = f32 ? LD_F32 : LD_BF16;
  const int dt = d->dtype;
  const int M = d->M, D = d->D, I = d->I, N = d->N;
  void* dg = W + L.dg;
  void* du = W + L.du;

  const bool grads_wanted = explicit_graft && d->n_slices > 0;
  bool operands_laid_out = false;  // x and dy already in the weight-gradient fragment layout
  if (L.dy_f32) {
    // The reference multiplies its f32 upstream gradient by the f32 copy of
    // W_down (src/layer_backward_impl.inc:48) and rounds it to bf16 for the
    // graft GEMMs (src/gemm_impl.inc:454-455, :524-525). The MFMA operands
    // are bf16, so the gradient is rounded once (RNE) here and every GEMM
    // below reads that copy; when the weight gradients need x and dy in the
    // fragment layout, the same pass writes them.
    uint16_t* dyb = reinterpret_cast<uint16_t*>(W + L.dyb);
    const float* dyf = static_cast<const float*>(dy);
    uint16_t* XS = reinterpret_cast<uint16_t*>(W + L.xt);
    uint16_t* DYS = reinterpret_cast<uint16_t*>(W + L.dyt);
    if (L.wgrad_mfma && grads_wanted && shuffle_tr_pair_f32_ok(x, dyf, d->D, d->D, d->M, XS, DYS, dyb)) {
      if ((s = shuffle_tr_pair_f32(static_cast<const uint16_t*>(x), dyf, d->D, d->D, d->M, XS, DYS, dyb, st)) !=
          GLT_OK)
        return s;
      operands_laid_out = true;
    } else if ((s = convert_f32_to_bf16(dyf, dyb, (int64_t)d->M * d->D, st)) != GLT_OK) {
      return s;
    }
    dy = dyb;
  }

  if (recompute) {
    gate_pre = W + L.g;
    up_pre = W + L.u;
    inter = W + L.inter;
    if ((s = gate_up_forward(d, w, x, W + L.g, W + L.u, W + L.inter, st)) != GLT_OK) return s;
  }

  // 1) dInter = dy . [W_down | grafts] with the SiLU*up derivative epilogue
  //    (reference src/layer_backward_impl.inc:45-188).
  {
    GemmPlan plan;
    plan.label = "dinter";
    set_kinds(plan, d, mfma);
    plan.add_problem(prob(M, N, EPI_DGDU, f32, dg, du, nullptr, N, gate_pre, up_pre, N));
    if (I > 0) {
      if (mfma) {
        plan.add_seg(nt_seg(dy, D, 0, D, 0, I, prep(d, w, PREP_DOWN_T), D, 0));
      } else {
        GSeg g = nt_seg(dy, D, 0, D, 0, I, w->down, 1, 0);  // B(n, k) = W_down[k, n]
        g.b_ks = I;
        plan.add_seg(g);
      }
    }
    for (int j = 0; explicit_graft && j < d->n_slices; ++j) {
      const glt_graft_slice& sl = d->slices[j];
      if (!sl.master_down) continue;
      // B(n = i0+s, k = h) = delta_down[s, h]: the [S,H] storage is NT as is
      const void* B = f32 ? (const void*)sl.master_down : mfma ? packed_shuf(sl, 2, false) : packed_block(sl, 2, false);
      plan.add_seg(nt_seg(dy, D, sl.h_start, sl.h, sl.i_start, sl.i_start + sl.s, B, sl.h, sl.i_start));
    }
    if ((s = run_gemm(plan, st)) != GLT_OK) return s;
  }

  // 2) dX = [dgate | dup] . [W_gate ; W_up (+) grafts]  (f32 out)
  //    (reference src/layer_backward_impl.inc:307-361).
  if (dx) {
    GemmPlan plan;
    plan.label = "dx";
    set_kinds(plan, d, mfma);
    plan.add_problem(prob(M, D, EPI_STORE, true, dx, nullptr, nullptr, D));
    if (I > 0) {
      const int slots[2] = {PREP_GATE_T, PREP_UP_T};
      const void* wo[2] = {w->gate, w->up};
      const void* a[2] = {dg, du};
      for (int p = 0; p < 2; ++p) {
        if (mfma) {
          plan.add_seg(nt_seg(a[p], N, 0, I, 0, D, prep(d, w, slots[p]), I, 0));
        } else {
          GSeg g = nt_seg(a[p], N, 0, I, 0, D, wo[p], 1, 0);  // B(n, k) = W[k, n]
          g.b_ks = D;
          plan.add_seg(g);
        }
      }
    }
    for (int j = 0; explicit_graft && j < d->n_slices; ++j) {
      const glt_graft_slice& sl = d->slices[j];
      const float* mast[2] = {sl.master_gate, sl.master_up};
      const void* a[2] = {dg, du};
      for (int p = 0; p < 2; ++p) {
        if (!mast[p]) continue;
        if (f32) {
          GSeg g = nt_seg(a[p], N, sl.i_start, sl.s, sl.h_start, sl.h_start + sl.h, mast[p], 1, sl.h_start);
          g.b_ks = sl.h;  // B(n = h0+h, k = s) = delta[s, h]
          plan.add_seg(g);
        } else {
          plan.add_seg(nt_seg(a[p], N, sl.i_start, sl.s, sl.h_start, sl.h_start + sl.h,
                              mfma ? packed_shuf(sl, p, true) : packed_block(sl, p, true), sl.s, sl.h_start));
        }
      }
    }
    if ((s = run_gemm(plan, st)) != GLT_OK) return s;
  }

  // 3) per-slice weight gradients, reduced over the M tokens, [S,H] storage
  //    (reference src/graft_ops_impl.inc:120-141, :214-228):
  //      dGate = dgate_i^T . x_h, dUp = dup_i^T . x_h, dDown = inter_i^T . dy_h
  if (!explicit_graft || d->n_slices == 0) return GLT_OK;
  if (L.wgrad_mfma) {
    // K (= tokens) must be the contiguous axis of A: each slice's column
    // block of dgate/dup/inter is transposed once; x and dy become shuffled
    // B operands [D rows, K = M] once for all slices.
    uint16_t* XS = reinterpret_cast<uint16_t*>(W + L.xt);
    uint16_t* DYS = reinterpret_cast<uint16_t*>(W + L.dyt);
    if (!operands_laid_out && (s = shuffle_b_tr_pair(x, dy, dt, D, D, M, XS, DYS, st)) != GLT_OK) return s;
    const size_t es = esize(dt);
    // every slice transpose first, batched into few launches
    {
      T16Job jobs[kMaxT16Jobs];
      int nj = 0;
      for (int j = 0; j < d->n_slices; ++j) {
        const glt_graft_slice& sl = d->slices[j];
        const glt_graft_grads& gr = grads[j];
        char* base = W + L.slice0 + (size_t)j * L.slice_stride;
        const size_t blk = align256((size_t)sl.s * M * es);
        const char* srcs[3] = {static_cast<const char*>(dg), static_cast<const char*>(du),
                               static_cast<const char*>(inter)};
        const float* outs[3] = {gr.gate, gr.up, gr.down};
        const float* mast[3] = {sl.master_gate, sl.master_up, sl.master_down};
        for (int p = 0; p < 3; ++p) {
          if (!outs[p] || !mast[p]) continue;
          jobs[nj++] = T16Job{srcs[p] + (size_t)sl.i_start * es, base + p * blk, M, sl.s, (int64_t)N};
          if (nj == kMaxT16Jobs) {
            if ((s = transpose_batch(jobs, nj, dt, st)) != GLT_OK) return s;
            nj = 0;
          }
        }
      }
      if (nj > 0 && (s = transpose_batch(jobs, nj, dt, st)) != GLT_OK) return s;
    }
    GemmPlan plan;
    plan.label = "wgrad";
    plan.a_kind = LD_BF16;
    plan.b_kind = LD_SHUF;
    for (int j = 0; j < d->n_slices; ++j) {
      const glt_graft_slice& sl = d->slices[j];
      const glt_graft_grads& gr = grads[j];
      char* base = W + L.slice0 + (size_t)j * L.slice_stride;
      const size_t blk = align256((size_t)sl.s * M * es);
      float* outs[3] = {gr.gate, gr.up, gr.down};
      const float* mast[3] = {sl.master_gate, sl.master_up, sl.master_down};
      for (int p = 0; p < 3; ++p) {
        if (!outs[p] || !mast[p]) continue;
        char* AT = base + p * blk;
        if (plan.args.nprob == kMaxProb) {
          if ((s = run_gemm(plan, st)) != GLT_OK) return s;
          plan = GemmPlan();
          plan.label = "wgrad";
          plan.a_kind = LD_BF16;
          plan.b_kind = LD_SHUF;
        }
        // B row of output column h is row h0 + h of the shuffled x / dy
        plan.add_problem(prob(sl.s, sl.h, EPI_STORE, true, outs[p], nullptr, nullptr, sl.h));
        plan.add_seg(nt_seg(AT, M, 0, M, 0, sl.h, p < 2 ? XS : DYS, M, -sl.h_start));
      }
    }
    // The weight-gradient launch has few tiles (3 per slice and 256 x 256
    // block of [S,H]); the CUs it leaves idle take the RMSNorm backward,
    // which only needs dx (complete: its GEMM ran above on this stream).
    hipEvent_t norm_ev = nullptr;
    if (nb && dx && gemm_mfma_eligible(plan) &&
        rmsnorm_bwd_rows_ok(dx, nb->x, nb->w, nb->dx, d->M, d->D)) {
      int cus = 0;
      if ((s = device_cus(cus)) != GLT_OK) return s;
      const int idle = cus - gemm_mfma_tiles(plan);
      if (idle >= 16 && (s = fork_norm_bwd(*nb, dx, d->M, d->D, idle, st, &norm_ev)) != GLT_OK) return s;
    }
    // join the helper stream even when the GEMM launch failed, so that no
    // work of this call is left running after it returns an error
    const glt_status gs = run_gemm(plan, st);
    if (norm_ev) {
      hipError_t we = hipStreamWaitEvent(st, norm_ev, 0);
      // no join on st: wait for the helper stream's kernel on the host
      if (we != hipSuccess) (void)hipEventSynchronize(norm_ev);
      const hipError_t de = hipEventDestroy(norm_ev);
      GLT_TRY_HIP(we);
      GLT_TRY_HIP(de);
      *norm_done = true;
    }
    return gs;
  }
  // strided (generic) form: A(s, t) = src[t*N + i0 + s], B(h, t) = src2[t*D + h0 + h]
  GemmPlan plan;
  plan.label = "wgrad";
  plan.a_kind = plan.b_kind = kind;
  const size_t es = esize(dt);
  for (int j = 0; j < d->n_slices; ++j) {
    const glt_graft_slice& sl = d->slices[j];
    const glt_graft_grads& gr = grads[j];
    const char* srcs[3] = {static_cast<const char*>(dg), static_cast<const char*>(du),
                           static_cast<const char*>(inter)};
    const char* srcb[3] = {static_cast<const char*>(x), static_cast<const char*>(x), static_cast<const char*>(dy)};
    float* outs[3] = {gr.gate, gr.up, gr.down};
    const float* mast[3] = {sl.master_gate, sl.master_up, sl.master_down};
    for (int p = 0; p < 3; ++p) {
      if (!outs[p] || !mast[p]) continue;
      if (plan.args.nprob == kMaxProb) {
        if ((s = run_gemm(plan, st)) != GLT_OK) return s;
        plan = GemmPlan();
        plan.label = "wgrad";
        plan.a_kind = plan.b_kind = kind;
      }
      plan.add_problem(prob(sl.s, sl.h, EPI_STORE, true, outs[p], nullptr, nullptr, sl.h));
      GSeg g = nt_seg(srcs[p] + (size_t)sl.i_start * es, 1, 0, M, 0, sl.h, srcb[p] + (size_t)sl.h_start * es, 1, 0);
      g.a_ks = N;
      g.b_ks = D;
      plan.add_seg(g);
    }
  }
  return run_gemm(plan, st);
}
}  // namespace glt

glt_status glt_mlp_bwd(const glt_mlp_desc* d, const glt_base_weights* w, const void* x, const void* dy,
                       const void* gate_pre, const void* up_pre, const void* inter, float* dx,
                       const glt_graft_grads* grads, void* ws, size_t ws_bytes, void* stream) {
  bool norm_done = false;
  return mlp_bwd_impl(d, w, x, dy, gate_pre, up_pre, inter, dx, grads, ws, ws_bytes, as_stream(stream), nullptr,
                      &norm_done);
}

glt_status glt_mlp_rmsnorm_bwd(const glt_mlp_desc* d, const glt_base_weights* w, const void* x, const void* dy,
                               const void* gate_pre, const void* up_pre, const void* inter, float* dx,
                               const glt_graft_grads* grads, void* ws, size_t ws_bytes, const uint16_t* norm_x,
                               const uint16_t* norm_w, const float* norm_var, float eps, float* norm_dx,
                               void* stream) {
  GLT_CHECK(d, GLT_ERR_INVALID_ARG, "glt_mlp_rmsnorm_bwd: null descriptor");
  GLT_CHECK(d->M == 0 || (dx && norm_x && norm_w && norm_var && norm_dx), GLT_ERR_INVALID_ARG,
            "glt_mlp_rmsnorm_bwd: null dx or RMSNorm operand");
  GLT_CHECK(d->dtype == GLT_DTYPE_BF16, GLT_ERR_DTYPE, "glt_mlp_rmsnorm_bwd: bf16 path only (dtype %d)", d->dtype);
  const NormBwd nb{norm_x, norm_w, norm_var, eps, norm_dx};
  bool norm_done = false;
  hipStream_t st = as_stream(stream);
  glt_status s = mlp_bwd_impl(d, w, x, dy, gate_pre, up_pre, inter, dx, grads, ws, ws_bytes, st, &nb, &norm_done);
  if (s != GLT_OK || norm_done || d->M == 0) return s;
  return glt_rmsnorm_bwd(dx, norm_x, norm_w, norm_var, norm_dx, d->M, d->D, eps, stream);
}

glt_status glt_graft_gemm(int32_t kind, int32_t M, int32_t S, int32_t H, const uint16_t* a, int64_t lda,
                          const float* delta, const float* dy, float* out, int64_t ldo, float alpha, float beta,
                          void* stream) {
  GLT_CHECK(M >= 0 && S > 0 && H > 0, GLT_ERR_SHAPE, "glt_graft_gemm: M=%d S=%d H=%d", M, S, H);
  GLT_CHECK(kind >= GLT_GEMM_EXPAND_FWD && kind <= GLT_GEMM_CONTRACT_IGRAD, GLT_ERR_INVALID_ARG,
            "glt_graft_gemm: kind %d", kind);
  GLT_CHECK(out, GLT_ERR_INVALID_ARG, "glt_graft_gemm: null out");
  const bool needs_a = kind <= GLT_GEMM_CONTRACT_WGRAD;
  const bool needs_delta = kind == GLT_GEMM_EXPAND_FWD || kind == GLT_GEMM_CONTRACT_FWD || kind >= GLT_GEMM_EXPAND_IGRAD;
  const bool needs_dy = kind >= GLT_GEMM_EXPAND_WGRAD;
  GLT_CHECK((!needs_a || a) && (!needs_delta || delta) && (!needs_dy || dy), GLT_ERR_INVALID_ARG,
            "glt_graft_gemm: missing operand for kind %d", kind);
  GemmPlan plan;
  plan.label = "graft_gemm";
  GSeg g{};
  g.a_col = 0;
  g.n_lo = 0;
  g.b0_row0 = 0;
  int outM = M, outN = 0;
  switch (kind) {
    case GLT_GEMM_EXPAND_FWD:  // out[M,S] = a[M,H] . bf16(delta[S,H])^T
      plan.a_kind = LD_BF16; plan.b_kind = LD_F32_AS_BF16; outN = S;
      g.A = a; g.lda = lda; g.a_ks = 1; g.K = H; g.B0 = delta; g.ldb0 = H; g.b_ks = 1;
      break;
    case GLT_GEMM_CONTRACT_FWD:  // out[M,H] = a[M,S] . bf16(delta[S,H])
      plan.a_kind = LD_BF16; plan.b_kind = LD_F32_AS_BF16; outN = H;
      g.A = a; g.lda = lda; g.a_ks = 1; g.K = S; g.B0 = delta; g.ldb0 = 1; g.b_ks = H;
      break;
    case GLT_GEMM_EXPAND_WGRAD:  // out[S,H] = bf16(dy[M,S])^T . a[M,H]
      plan.a_kind = LD_F32_AS_BF16; plan.b_kind = LD_BF16; outM = S; outN = H;
      g.A = dy; g.lda = 1; g.a_ks = S; g.K = M; g.B0 = a; g.ldb0 = 1; g.b_ks = lda;
      break;
    case GLT_GEMM_CONTRACT_WGRAD:  // out[S,H] = a[M,S]^T . bf16(dy[M,H])
      plan.a_kind = LD_BF16; plan.b_kind = LD_F32_AS_BF16; outM = S; outN = H;
      g.A = a; g.lda = 1; g.a_ks = lda; g.K = M; g.B0 = dy; g.ldb0 = 1; g.b_ks = H;
      break;
    case GLT_GEMM_EXPAND_IGRAD:  // out[M,H] = bf16(dy[M,S]) . bf16(delta[S,H])
      plan.a_kind = LD_F32_AS_BF16; plan.b_kind = LD_F32_AS_BF16; outN = H;
      g.A = dy; g.lda = S; g.a_ks = 1; g.K = S; g.B0 = delta; g.ldb0 = 1; g.b_ks = H;
      break;
    default:  // CONTRACT_IGRAD: out[M,S] = bf16(dy[M,H]) . bf16(delta[S,H])^T
      plan.a_kind = LD_F32_AS_BF16; plan.b_kind = LD_F32_AS_BF16; outN = S;
      g.A = dy; g.lda = H; g.a_ks = 1; g.K = H; g.B0 = delta; g.ldb0 = H; g.b_ks = 1;
      break;
  }
  GLT_CHECK(ldo >= outN, GLT_ERR_SHAPE, "glt_graft_gemm: ldo %lld < %d", (long long)ldo, outN);
  g.n_hi = outN;
  GProb p = prob(outM, outN, EPI_STORE, true, out, nullptr, nullptr, ldo);
  p.alpha = alpha;
  p.beta = beta;
  plan.add_problem(p);
  plan.add_seg(g);
  if (outM == 0) return GLT_OK;
  return run_gemm(plan, as_stream(stream), false);
}

}  // extern "C"
