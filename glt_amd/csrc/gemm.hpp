// Segment-list GEMM shared by the graft-layer kernels.
//
// One output C[M,N] is the sum of K-segments. Segment s contributes
//   C[m, n] += sum_{k < K_s} A_s(m, a_col_s + k) * B_s(n - b_row0_s, k)
// for output columns n in [n_lo_s, n_hi_s). A base projection is one segment
// over all of its columns; every graft slice adds one more segment over the
// columns it touches. Appended slices (new neurons) therefore extend N
// (concat-N) and in-place slices add an extra K range to existing columns
// (concat-K), all in one fp32 accumulator.
//
// The dual form pairs two B operands (gate and up) over the same A tile so
// the epilogue sees gate and up pre-activations of the same (m, n) element.
#pragma once

#include "common.hpp"

namespace glt {

constexpr int kMaxSeg = 18;  // dX of 8 slices: base gate and up + 2 per slice
constexpr int kMaxProb = 8;

enum EpiMode : int {
  EPI_STORE = 0,  // out0 = alpha*acc + beta*out0
  EPI_SILU = 1,   // dual: out0 = silu(g)*u, out1 = g, out2 = u (out1/out2 nullable)
  EPI_DGDU = 2,   // out0 = acc*u*silu'(g), out1 = acc*silu(g); g = aux0, u = aux1
  EPI_RESID = 3,  // out0 = round(out0 + round(alpha*acc)): residual add of a rounded result
};

// Element kinds an operand can be read as. LD_SHUF: bf16 B operand in the
// shuffled layout of layout.hpp (MFMA kernel only).
enum LoadKind : int { LD_BF16 = 0, LD_F32 = 1, LD_F32_AS_BF16 = 2, LD_SHUF = 3 };

struct GSeg {
  const void* A;
  const void* B0;   // single / gate operand
  const void* B1;   // up operand (dual only)
  int64_t lda, a_ks;         // A(m, k) = A[m*lda + k*a_ks]
  int64_t ldb0, ldb1, b_ks;  // strided: B(n, k) = B[n*ldb + k*b_ks]; LD_SHUF: ldb = padded K of B
  int a_col, K, n_lo, n_hi, b0_row0, b1_row0;
};

struct GProb {
  int M, N;
  int seg0, nseg;
  int tiles_m, tiles_n, tile_begin;
  int mode;      // EpiMode
  int out_f32;   // element type of out*/aux*: 1 = f32, 0 = bf16
  float alpha, beta;
  void* out0;
  void* out1;
  void* out2;
  const void* aux0;
  const void* aux1;
  int64_t ldo, ldaux;
};

struct GArgs {
  int nprob, total_tiles;
  GProb p[kMaxProb];
  GSeg s[kMaxSeg];
};

// Host-side builder of one GEMM launch (up to kMaxProb problems).
struct GemmPlan {
  GArgs args{};
  bool dual = false;
  int a_kind = LD_BF16, b_kind = LD_BF16;
  const char* label = "gemm";  // launch-timing label (glt_profile_enable)
  int nseg = 0;
  int add_problem(const GProb& p) {
    args.p[args.nprob] = p;
    args.p[args.nprob].seg0 = nseg;
    args.p[args.nprob].nseg = 0;
    return args.nprob++;
  }
  void add_seg(const GSeg& s) {
    args.s[nseg++] = s;
    args.p[args.nprob - 1].nseg++;
  }
};

// Runs the plan: the gfx950 MFMA kernel when A is bf16 row-major (16-byte
// aligned rows), B is shuffled (LD_SHUF, 32-aligned row ranges) and every K
// is a multiple of 64; otherwise the strided generic kernel (f32 path,
// tiny/unaligned shapes, transposed probes). A shuffled B has no generic
// form: such a plan must be MFMA-eligible.
glt_status run_gemm(GemmPlan& plan, hipStream_t st, bool allow_mfma = true);
bool gemm_mfma_eligible(const GemmPlan& plan);
// Workgroups of the MFMA kernel's launch for this plan (one per 256 x 256
// tile, dual: 256 x 128, at most one per CU).
int gemm_mfma_tiles(const GemmPlan& plan);
// CUs of the current device (cached per device).
glt_status device_cus(int& cus);

}  // namespace glt
