// Fragment-major ("shuffled") layout of a GEMM B operand.
//
// B is [rows, K] (rows = output columns n, K = reduction). It is stored in
// blocks of 32 rows x 64 K (4 KB of bf16), block (rb, kb) at element offset
// (rb * ceil(K/64) + kb) * 2048. Inside a block the order is
// [substep s: 4][lane: 64][8 elements], element e of lane l in substep s
// holding B[32*rb + (l & 31)][64*kb + 16*s + 8*(l >> 5) + e]: exactly the
// B operand of one v_mfma_f32_32x32x16_bf16 per (s, lane). A wavefront then
// fetches a 32-row fragment of one K-substep with one fully coalesced 1 KB
// load straight into registers. Rows past `rows` and K past K are zero.
#pragma once

#include "common.hpp"

namespace glt {

// Transposes dst [cols, rows] = src [rows, cols] (rows src_ld elements
// apart) of several matrices in one launch when all are bf16 in whole,
// 16-byte-aligned 64 x 64 tiles, one launch per matrix otherwise.
constexpr int kMaxT16Jobs = 8;
struct T16Job {
  const void* src;
  void* dst;
  int rows, cols;
  int64_t src_ld;
};
glt_status transpose_batch(const T16Job* jobs, int n, int dtype, hipStream_t st);

constexpr int kShufRows = 32, kShufK = 64, kShufBlock = kShufRows * kShufK;

inline int64_t shuf_rows(int64_t rows) { return (rows + kShufRows - 1) / kShufRows * kShufRows; }
inline int64_t shuf_k(int64_t k) { return (k + kShufK - 1) / kShufK * kShufK; }
// bf16 elements of the shuffled form of a [rows, K] operand
inline int64_t shuf_elems(int64_t rows, int64_t k) { return shuf_rows(rows) * shuf_k(k); }

// Packed bf16 mirror of one graft slice (glt_graft_slice.packed), six
// orientations q = 2*proj + transposed (proj gate, up, down; [S,H] or
// [H,S]): first row-major, 6*S*H elements in the order gate, gate^T, up,
// up^T, down, down^T (read by the generic kernel), then, 256-byte aligned,
// the same six in the shuffled layout (read by the MFMA kernel).
inline int64_t packed_shuf_base(int S, int H) { return ((int64_t)6 * S * H + 127) / 128 * 128; }
inline int64_t packed_shuf_offset(int S, int H, int q) {
  int64_t off = packed_shuf_base(S, H);
  for (int i = 0; i < q; ++i) off += (i & 1) ? shuf_elems(H, S) : shuf_elems(S, H);
  return off;
}
inline int64_t packed_bytes(int S, int H) { return packed_shuf_offset(S, H, 6) * 2; }

// Prepared bf16 base of one MLP layer (glt_base_weights.prepared): the six
// shuffled B operands the MFMA path multiplies by, in the order
// gate[I,D], up[I,D] (gate/up forward), down[D,I] (down forward),
// down^T[I,D] (dInter), gate^T[D,I], up^T[D,I] (dX).
enum PrepSlot : int { PREP_GATE = 0, PREP_UP, PREP_DOWN, PREP_DOWN_T, PREP_GATE_T, PREP_UP_T };
inline int64_t prep_offset(int I, int D, int q) {
  static const bool id_shape[6] = {true, true, false, true, false, false};  // [I,D] vs [D,I]
  int64_t off = 0;
  for (int i = 0; i < q; ++i) off += id_shape[i] ? shuf_elems(I, D) : shuf_elems(D, I);
  return off;
}
inline int64_t prep_bytes(int I, int D) { return prep_offset(I, D, 6) * 2; }

// Writes the shuffled form of B[rows, K]. Source element (r, k) is
// src[r*ld + k] (transposed = false) or src[k*ld + r] (transposed = true);
// src_dtype GLT_DTYPE_BF16 or GLT_DTYPE_F32 (rounded to bf16, RNE).
// Two transposed operands of one shape (B[n][k] = src[k][n], rows x K) into
// the fragment layout in one launch when they are bf16 in whole 64 x 64
// tiles, else two shuffle_b calls.
glt_status shuffle_b_tr_pair(const void* src0, const void* src1, int src_dtype, int64_t ld, int rows, int K,
                            uint16_t* dst0, uint16_t* dst1, hipStream_t st);
glt_status shuffle_b(const void* src, int src_dtype, int64_t ld, bool transposed, int rows, int K, uint16_t* dst,
                     hipStream_t st);
// shuffle_b_tr_pair for a bf16 src0 and an f32 src1 (whole 64 x 64 tiles,
// 16-byte aligned): src1 is rounded to bf16 (RNE) and its row-major bf16
// copy is written to rm1 in the same pass.
bool shuffle_tr_pair_f32_ok(const void* src0, const float* src1, int64_t ld, int rows, int K, const void* dst0,
                            const void* dst1, const void* rm1);
glt_status shuffle_tr_pair_f32(const uint16_t* src0, const float* src1, int64_t ld, int rows, int K, uint16_t* dst0,
                               uint16_t* dst1, uint16_t* rm1, hipStream_t st);

// out[i] = RNE bf16 of in[i].
glt_status convert_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t st);

// Packed-mirror orientations q = 2*proj and 2*proj+1 (row-major and
// shuffled) of one projection from its f32 [S,H] master.
glt_status pack_projection(const float* master, int S, int H, int proj, uint16_t* packed, hipStream_t st);

}  // namespace glt
