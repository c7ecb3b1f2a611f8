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
    if (transposed) GLT_LAUNCH("shuffle", (shuffle_kernel<uint16_t, true>), grid, dim3(256), 0, st, s, ld, rows, K, kblocks, dst);
    else GLT_LAUNCH("shuffle", (shuffle_kernel<uint16_t, false>), grid, dim3(256), 0, st, s, ld, rows, K, kblocks, dst);
  }
  GLT_LAUNCH_CHECK("shuffle");
  return GLT_OK;
}

}  // namespace glt
