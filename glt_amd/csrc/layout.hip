// Shuffled B layout writer (see layout.hpp).
#include "layout.hpp"

namespace glt {

template <typename TS>
__device__ __forceinline__ float ld_src(const TS* p, int64_t i) {
  if constexpr (sizeof(TS) == 4) return p[i];
  else return bf16_to_f32(p[i]);
}

// Eight consecutive source elements p[i .. i+7] as f32; `whole` = all in
// range, then one or two 16-byte loads when aligned.
template <typename TS>
__device__ __forceinline__ void ld_src8(const TS* p, int64_t i, int valid, float* v) {
  const bool al = (reinterpret_cast<uintptr_t>(p + i) & 15) == 0;
  if (valid == 8 && al) {
    if constexpr (sizeof(TS) == 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p + i);
      const f32x4 b = *reinterpret_cast<const f32x4*>(p + i + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const u32x4 q = *reinterpret_cast<const u32x4*>(p + i);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = bf16_to_f32((uint16_t)(w[e] & 0xFFFF));
        v[2 * e + 1] = bf16_to_f32((uint16_t)(w[e] >> 16));
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = e < valid ? ld_src(p, i + e) : 0.f;
}

// One workgroup per 32 x 64 block: the source tile goes through LDS (read
// coalesced along the source's contiguous axis), then every thread writes
// one 16-byte (substep, lane) chunk of the block.
template <typename TS, bool TR>
__global__ void __launch_bounds__(256) shuffle_kernel(const TS* __restrict__ src, int64_t ld, int rows, int K,
                                                      int kblocks, uint16_t* __restrict__ dst) {
  __shared__ float tile[kShufRows][kShufK + 1];
  const int blk = blockIdx.x;
  const int rb = blk / kblocks, kb = blk - rb * kblocks;
  const int r0 = rb * kShufRows, k0 = kb * kShufK;
  const int t = threadIdx.x;
  float v[8];
  if constexpr (!TR) {
    const int r = t >> 3, kc = (t & 7) * 8;  // 32 rows x 8 chunks of 8 along K
    const int valid = r0 + r < rows ? max(0, min(8, K - (k0 + kc))) : 0;
    ld_src8(src, (int64_t)(r0 + r) * ld + k0 + kc, valid, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[r][kc + e] = v[e];
  } else {
    const int kk = t >> 2, rc = (t & 3) * 8;  // 64 source rows (K) x 4 chunks of 8 along the rows of B
    const int valid = k0 + kk < K ? max(0, min(8, rows - (r0 + rc))) : 0;
    ld_src8(src, (int64_t)(k0 + kk) * ld + r0 + rc, valid, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[rc + e][kk] = v[e];
  }
  __syncthreads();
  const int s = t >> 6, lane = t & 63;
  const int rr = lane & 31, kq = 16 * s + 8 * (lane >> 5);
  u32x4 q;
  q.x = pack_bf16x2(tile[rr][kq + 0], tile[rr][kq + 1]);
  q.y = pack_bf16x2(tile[rr][kq + 2], tile[rr][kq + 3]);
  q.z = pack_bf16x2(tile[rr][kq + 4], tile[rr][kq + 5]);
  q.w = pack_bf16x2(tile[rr][kq + 6], tile[rr][kq + 7]);
  *reinterpret_cast<u32x4*>(dst + (int64_t)blk * kShufBlock + t * 8) = q;
}

// Transposed bf16 source (B[n][k] = src[k][n]) in whole 64 x 64 tiles, one
// tile per wavefront: the tile is the two 32-row fragment blocks (n0/32,
// n0/32 + 1) of K block k0/64. Lane (cb = lane & 7, kb = lane >> 3) loads
// the 8 x 8 sub-block at source rows k0 + 8 kb .. +7, columns n0 + 8 cb ..
// +7 (each load instruction covers eight whole 128-byte lines) and
// transposes it in registers: column c becomes the 16-byte chunk of B row
// n0 + 8 cb + c holding K = k0 + 8 kb .. +7, which is chunk (substep kb/2,
// lane (8 cb + c) % 32 + 32 (kb & 1)) of its block. The chunks go to their
// place in the wavefront's 8 KB of LDS and leave as contiguous 1 KB stores.
// SRC1_F32: the second source is f32; its 8 x 8 sub-blocks are rounded to
// bf16 (RNE) on load and also written row-major to rm1 (the bf16 copy the
// other GEMMs read), so one pass converts and lays out an f32 gradient.
template <bool SRC1_F32>
__global__ void __launch_bounds__(256) shuffle_tr16_kernel(const uint16_t* __restrict__ src0,
                                                           const void* __restrict__ src1, int64_t ld, int rows,
                                                           int K, int njobs, uint16_t* __restrict__ dst0,
                                                           uint16_t* __restrict__ dst1, uint16_t* __restrict__ rm1) {
  __shared__ __attribute__((aligned(16))) uint16_t stage[4][2 * kShufBlock];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  const int kt = K / 64;
  const int64_t per = (int64_t)(rows / 64) * kt;  // tiles of one matrix; a second one of the same shape follows
  if (tile >= per * njobs) return;
  const bool second = tile >= per;
  if (second) tile -= per;
  uint16_t* __restrict__ dst = second ? dst1 : dst0;
  // consecutive tiles take consecutive column bands of the same source rows
  // (the step's x and f32 gradient, 805 MB: 158 us with consecutive tiles
  // going down the rows instead, 131 us this way)
  const int ntiles_n = rows / 64;
  const int nt = (int)(tile % ntiles_n), ktile = (int)(tile / ntiles_n);
  const int n0 = nt * 64, k0 = ktile * 64;
  const int cb = lane & 7, kb = lane >> 3;
  u32x4 in[8];
  if (SRC1_F32 && second) {
    const float* __restrict__ src = static_cast<const float*>(src1);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int64_t o = (int64_t)(k0 + 8 * kb + r) * ld + n0 + 8 * cb;
      const f32x4 a = *reinterpret_cast<const f32x4*>(src + o), b = *reinterpret_cast<const f32x4*>(src + o + 4);
      in[r] = u32x4{pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w), pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w)};
      *reinterpret_cast<u32x4*>(rm1 + o) = in[r];
    }
  } else {
    const uint16_t* __restrict__ src = second ? static_cast<const uint16_t*>(src1) : src0;
#pragma unroll
    for (int r = 0; r < 8; ++r)
      in[r] = *reinterpret_cast<const u32x4*>(src + (int64_t)(k0 + 8 * kb + r) * ld + n0 + 8 * cb);
  }
  uint16_t* st = stage[wave];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = __builtin_amdgcn_perm(in[2 * w + 1][c >> 1], in[2 * w][c >> 1], sel);
    const int n = 8 * cb + c;
    const int chunk = (kb >> 1) * 64 + (n & 31) + 32 * (kb & 1);
    *reinterpret_cast<u32x4*>(st + (n >> 5) * kShufBlock + chunk * 8) = o;
  }
  // the wavefront's LDS accesses execute in order; the fences keep the
  // compiler from moving the reads above the writes
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint16_t* out = dst + ((int64_t)(2 * nt + h) * kt + ktile) * kShufBlock;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4*>(out + (i * 64 + lane) * 8) =
          *reinterpret_cast<const u32x4*>(st + h * kShufBlock + (i * 64 + lane) * 8);
  }
}

glt_status shuffle_b_tr_pair(const void* src0, const void* src1, int src_dtype, int64_t ld, int rows, int K,
                            uint16_t* dst0, uint16_t* dst1, hipStream_t st) {
  const bool fast = src_dtype == GLT_DTYPE_BF16 && rows > 0 && K > 0 && rows % 64 == 0 && K % 64 == 0 && ld % 8 == 0 &&
                    src0 && src1 && dst0 && dst1 &&
                    ((reinterpret_cast<uintptr_t>(src0) | reinterpret_cast<uintptr_t>(src1) |
                      reinterpret_cast<uintptr_t>(dst0) | reinterpret_cast<uintptr_t>(dst1)) & 15) == 0;
  if (!fast) {
    const glt_status s = shuffle_b(src0, src_dtype, ld, true, rows, K, dst0, st);
    return s != GLT_OK ? s : shuffle_b(src1, src_dtype, ld, true, rows, K, dst1, st);
  }
  const int64_t tiles = 2 * (int64_t)(rows / 64) * (K / 64);
  GLT_CHECK(tiles < (1ll << 33), GLT_ERR_SHAPE, "shuffle_b_tr_pair: %lld tiles", (long long)tiles);
  GLT_LAUNCH("shuffle_tr", shuffle_tr16_kernel<false>, dim3((unsigned)cdiv(tiles, 4)), dim3(256), 0, st,
             static_cast<const uint16_t*>(src0), src1, ld, rows, K, 2, dst0, dst1, (uint16_t*)nullptr);
  GLT_LAUNCH_CHECK("shuffle_tr");
  return GLT_OK;
}

bool shuffle_tr_pair_f32_ok(const void* src0, const float* src1, int64_t ld, int rows, int K, const void* dst0,
                            const void* dst1, const void* rm1) {
  return rows > 0 && K > 0 && rows % 64 == 0 && K % 64 == 0 && ld % 8 == 0 && src0 && src1 && dst0 && dst1 && rm1 &&
         ((reinterpret_cast<uintptr_t>(src0) | reinterpret_cast<uintptr_t>(src1) | reinterpret_cast<uintptr_t>(dst0) |
           reinterpret_cast<uintptr_t>(dst1) | reinterpret_cast<uintptr_t>(rm1)) & 15) == 0;
}

glt_status shuffle_tr_pair_f32(const uint16_t* src0, const float* src1, int64_t ld, int rows, int K, uint16_t* dst0,
                               uint16_t* dst1, uint16_t* rm1, hipStream_t st) {
  GLT_CHECK(shuffle_tr_pair_f32_ok(src0, src1, ld, rows, K, dst0, dst1, rm1), GLT_ERR_UNSUPPORTED,
            "shuffle_tr_pair_f32: shape or alignment");
  const int64_t tiles = 2 * (int64_t)(rows / 64) * (K / 64);
  GLT_CHECK(tiles < (1ll << 33), GLT_ERR_SHAPE, "shuffle_tr_pair_f32: %lld tiles", (long long)tiles);
  GLT_LAUNCH("shuffle_tr", shuffle_tr16_kernel<true>, dim3((unsigned)cdiv(tiles, 4)), dim3(256), 0, st, src0,
             static_cast<const void*>(src1), ld, rows, K, 2, dst0, dst1, rm1);
  GLT_LAUNCH_CHECK("shuffle_tr");
  return GLT_OK;
}

glt_status shuffle_b(const void* src, int src_dtype, int64_t ld, bool transposed, int rows, int K, uint16_t* dst,
                     hipStream_t st) {
  GLT_CHECK(rows >= 0 && K >= 0, GLT_ERR_SHAPE, "shuffle_b: negative shape");
  if (rows == 0 || K == 0) return GLT_OK;
  GLT_CHECK(src && dst, GLT_ERR_INVALID_ARG, "shuffle_b: null pointer");
  const int kblocks = (int)(shuf_k(K) / kShufK);
  const int64_t blocks = shuf_rows(rows) / kShufRows * kblocks;
  GLT_CHECK(blocks < (1ll << 31), GLT_ERR_SHAPE, "shuffle_b: %lld blocks", (long long)blocks);
  const dim3 grid((unsigned)blocks);
  if (src_dtype == GLT_DTYPE_F32) {
    const float* s = static_cast<const float*>(src);
    if (transposed) GLT_LAUNCH("shuffle", (shuffle_kernel<float, true>), grid, dim3(256), 0, st, s, ld, rows, K, kblocks, dst);
    else GLT_LAUNCH("shuffle", (shuffle_kernel<float, false>), grid, dim3(256), 0, st, s, ld, rows, K, kblocks, dst);
  } else {
    const uint16_t* s = static_cast<const uint16_t*>(src);
    if (transposed && rows % 64 == 0 && K % 64 == 0 && ld % 8 == 0 &&
        ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
      const int64_t tiles = (int64_t)(rows / 64) * (K / 64);
      GLT_LAUNCH("shuffle_tr", shuffle_tr16_kernel<false>, dim3((unsigned)cdiv(tiles, 4)), dim3(256), 0, st, s,
                 static_cast<const void*>(s), ld, rows, K, 1, dst, dst, (uint16_t*)nullptr);
      GLT_LAUNCH_CHECK("shuffle_tr");
      return GLT_OK;
    }
    if (transposed) GLT_LAUNCH("shuffle", (shuffle_kernel<uint16_t, true>), grid, dim3(256), 0, st, s, ld, rows, K, kblocks, dst);
    else GLT_LAUNCH("shuffle", (shuffle_kernel<uint16_t, false>), grid, dim3(256), 0, st, s, ld, rows, K, kblocks, dst);
  }
  GLT_LAUNCH_CHECK("shuffle");
  return GLT_OK;
}

}  // namespace glt
