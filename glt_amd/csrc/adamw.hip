// AdamW over graft parameters with the optional global-L2 gradient clip and
// the bf16 mirror refresh fused into the update.
#include <cmath>

#include "common.hpp"
#include "layout.hpp"

namespace glt {


constexpr int kClipBlocks = 1024;

// Partial sums of g^2 (f32, like the reference reduce_l2_kernel,
// src/kernels_elementwise_impl.inc:141-165), one partial per workgroup.
__global__ void __launch_bounds__(256) sumsq_partial_kernel(const float* __restrict__ g, int64_t n,
                                                            float* __restrict__ partial) {
  __shared__ float wsum[4];
  float s = 0.f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) s += g[i] * g[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

// scale = clip/norm if norm > clip else 1, norm = sqrt(sum + 1e-8)
// (reference calc_scale_kernel, src/kernels_elementwise_impl.inc:193-196).
__device__ __forceinline__ float clip_scale(const float* partial, int np, float clip) {
  float s = 0.f;
  for (int i = 0; i < np; ++i) s += partial[i];
  const float norm = sqrtf(s + 1e-8f);
  return norm > clip ? clip / norm : 1.0f;
}

// One AdamW element update in the reference's operation order
// (reference adamw_fused_kernel, src/kernels_optimizer_impl.inc:27-51).
__device__ __forceinline__ float adamw_elem(float wi, float gi, float& mi, float& vi, float lr, float b1, float b2,
                                            float b1c, float b2c, float eps, float wd) {
  mi = b1 * mi + (1.0f - b1) * gi;
  vi = b2 * vi + (1.0f - b2) * gi * gi;
  const float mh = mi * b1c, vh = vi * b2c;
  const float denom = sqrtf(vh) + eps;
  return wi - lr * mh / denom - lr * wd * wi;
}

__global__ void __launch_bounds__(256) adamw_kernel(float* __restrict__ w, const float* __restrict__ g,
                                                    float* __restrict__ m, float* __restrict__ v,
                                                    uint16_t* __restrict__ mirror, int64_t n, float lr,
                                                    float b1, float b2, float b1c, float b2c, float eps,
                                                    float wd, const float* __restrict__ partial, int np,
                                                    float clip) {
  __shared__ float s_scale;
  if (partial) {
    if (threadIdx.x == 0) s_scale = clip_scale(partial, np, clip);
    __syncthreads();
  }
  const float scale = partial ? s_scale : 1.0f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float mi = m[i], vi = v[i];
    const float nw = adamw_elem(w[i], g[i] * scale, mi, vi, lr, b1, b2, b1c, b2c, eps, wd);
    m[i] = mi;
    v[i] = vi;
    w[i] = nw;
    if (mirror) mirror[i] = f32_to_bf16(nw);
  }
}

// AdamW over one [S, H] graft projection fused with the refresh of its four
// bf16 mirrors in the packed slice: row-major [S,H], row-major [H,S], and
// the fragment layout of both. One workgroup per 64 x 64 tile (S and H
// multiples of 64, so no fragment block is padded): the f32 state streams
// through registers as 16-byte accesses, the new weights go through LDS
// once, and every mirror is written with 16-byte stores. The master is read
// once instead of once per mirror.
__global__ void __launch_bounds__(256) adamw_pack_kernel(float* __restrict__ w, const float* __restrict__ g,
                                                         float* __restrict__ m, float* __restrict__ v, int S,
                                                         int H, float lr, float b1, float b2, float b1c,
                                                         float b2c, float eps, float wd,
                                                         uint16_t* __restrict__ rm, uint16_t* __restrict__ rmt,
                                                         uint16_t* __restrict__ sh, uint16_t* __restrict__ sht) {
  __shared__ float tile[64][65];
  const int hb = H / 64;
  const int r0 = (blockIdx.x / hb) * 64, c0 = (blockIdx.x % hb) * 64;
  const int t = threadIdx.x;
  {
    const int rr = t >> 4, c4 = (t & 15) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rr + 16 * i;
      const int64_t o = (int64_t)(r0 + r) * H + c0 + c4;
      const f32x4 wi = *reinterpret_cast<const f32x4*>(w + o), gi = *reinterpret_cast<const f32x4*>(g + o);
      f32x4 mi = *reinterpret_cast<const f32x4*>(m + o), vi = *reinterpret_cast<const f32x4*>(v + o);
      f32x4 nw;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float a = mi[e], b = vi[e];
        nw[e] = adamw_elem(wi[e], gi[e], a, b, lr, b1, b2, b1c, b2c, eps, wd);
        mi[e] = a;
        vi[e] = b;
        tile[r][c4 + e] = nw[e];
      }
      *reinterpret_cast<f32x4*>(m + o) = mi;
      *reinterpret_cast<f32x4*>(v + o) = vi;
      *reinterpret_cast<f32x4*>(w + o) = nw;
      u32x2 q;
      q.x = pack_bf16x2(nw[0], nw[1]);
      q.y = pack_bf16x2(nw[2], nw[3]);
      *reinterpret_cast<u32x2*>(rm + o) = q;
    }
  }
  __syncthreads();
  {
    // [H,S] row-major: column c of the tile, 16 consecutive rows per thread
    const int c = t >> 2, rs = (t & 3) * 16;
    uint16_t* dst = rmt + (int64_t)(c0 + c) * S + r0 + rs;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4 q;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        q[e] = pack_bf16x2(tile[rs + 8 * h + 2 * e][c], tile[rs + 8 * h + 2 * e + 1][c]);
      *reinterpret_cast<u32x4*>(dst + 8 * h) = q;
    }
  }
  {
    // fragment layout: (substep s, lane) chunk t of a 32 x 64 block holds
    // row (lane & 31), K = 16 s + 8 (lane >> 5) .. +7
    const int s = t >> 6, lane = t & 63;
    const int rr = lane & 31, kq = 16 * s + 8 * (lane >> 5);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int br = half * 32 + rr;
      u32x4 q, qt;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        q[e] = pack_bf16x2(tile[br][kq + 2 * e], tile[br][kq + 2 * e + 1]);     // B = W [S rows, K = H]
        qt[e] = pack_bf16x2(tile[kq + 2 * e][br], tile[kq + 2 * e + 1][br]);    // B = W^T [H rows, K = S]
      }
      const int64_t blk = (int64_t)(r0 / 32 + half) * hb + c0 / 64;
      const int64_t blkt = (int64_t)(c0 / 32 + half) * (S / 64) + r0 / 64;
      *reinterpret_cast<u32x4*>(sh + blk * kShufBlock + t * 8) = q;
      *reinterpret_cast<u32x4*>(sht + blkt * kShufBlock + t * 8) = qt;
    }
  }
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int grid_n(int64_t n) {
  int64_t b = cdiv(n, 256);
  return (int)(b < 1 ? 1 : b > 16384 ? 16384 : b);
}

}  // namespace glt

using namespace glt;

extern "C" {

size_t glt_adamw_workspace_size(int64_t n) { return (size_t)kClipBlocks * sizeof(float); }

glt_status glt_adamw_step(float* w, float* g, float* m, float* v, uint16_t* mirror, int64_t n, int32_t step,
                          float lr, float beta1, float beta2, float eps, float weight_decay, float clip_norm,
                          void* ws, size_t ws_bytes, void* stream) {
  GLT_CHECK(n >= 0 && step >= 0, GLT_ERR_SHAPE, "glt_adamw_step: n=%lld step=%d", (long long)n, step);
  GLT_CHECK(n == 0 || (w && g && m && v), GLT_ERR_INVALID_ARG, "glt_adamw_step: null pointer");
  if (n == 0) return GLT_OK;
  hipStream_t st = as_stream(stream);
  float* partial = nullptr;
  int np = 0;
  if (clip_norm > 0.f) {
    GLT_CHECK(ws && ws_bytes >= glt_adamw_workspace_size(n), GLT_ERR_WORKSPACE,
              "glt_adamw_step: clip needs %zu workspace bytes", glt_adamw_workspace_size(n));
    partial = static_cast<float*>(ws);
    np = (int)std::min<int64_t>(kClipBlocks, cdiv(n, 256));
    GLT_LAUNCH("clip_sumsq", sumsq_partial_kernel, dim3(np), dim3(256), 0, st, g, n, partial);
    GLT_LAUNCH_CHECK("sumsq_partial");
  }
  // bias corrections as the reference computes them on the host
  // (src/kernels_optimizer_impl.inc:64-65)
  const float b1c = 1.0f / (1.0f - powf(beta1, (float)(step + 1)));
  const float b2c = 1.0f / (1.0f - powf(beta2, (float)(step + 1)));
  GLT_LAUNCH("adamw", adamw_kernel, dim3(grid_n(n)), dim3(256), 0, st, w, g, m, v, mirror, n, lr, beta1, beta2,
                     b1c, b2c, eps, weight_decay, partial, np, clip_norm);
  GLT_LAUNCH_CHECK("adamw");
  return GLT_OK;
}

glt_status glt_adamw_graft_step(const glt_graft_slice* slices, int32_t n_slices, float* const* grads,
                                float* const* m, float* const* v, uint16_t* const* packed_out,
                                int32_t proj_mask, int32_t step, float lr, float beta1, float beta2,
                                float eps, float weight_decay, void* stream) {
  GLT_CHECK(n_slices >= 0 && (n_slices == 0 || (slices && grads && m && v)), GLT_ERR_INVALID_ARG,
            "glt_adamw_graft_step: null pointer");
  hipStream_t st = as_stream(stream);
  const float b1c = 1.0f / (1.0f - powf(beta1, (float)(step + 1)));
  const float b2c = 1.0f / (1.0f - powf(beta2, (float)(step + 1)));
  for (int j = 0; j < n_slices; ++j) {
    const glt_graft_slice& sl = slices[j];
    const int64_t sh = (int64_t)sl.s * sl.h;
    const float* masters[3] = {sl.master_gate, sl.master_up, sl.master_down};
    for (int p = 0; p < 3; ++p) {
      if (!masters[p] || !(proj_mask & (1 << p))) continue;
      float* w = const_cast<float*>(masters[p]);
      float* gp = grads[j] + p * sh;
      float* mp = m[j] + p * sh;
      float* vp = v[j] + p * sh;
      uint16_t* pk = packed_out ? packed_out[j] : nullptr;
      if (pk && sl.s % 64 == 0 && sl.h % 64 == 0 && al16(w) && al16(gp) && al16(mp) && al16(vp) && al16(pk)) {
        const int64_t tiles = sh / 4096;
        GLT_CHECK(tiles < (1ll << 31), GLT_ERR_SHAPE, "glt_adamw_graft_step: %lld tiles", (long long)tiles);
        uint16_t* rm = pk + 2 * p * sh;
        GLT_LAUNCH("adamw_pack", adamw_pack_kernel, dim3((unsigned)tiles), dim3(256), 0, st, w, gp, mp, vp,
                   sl.s, sl.h, lr, beta1, beta2, b1c, b2c, eps, weight_decay, rm, rm + sh,
                   pk + packed_shuf_offset(sl.s, sl.h, 2 * p), pk + packed_shuf_offset(sl.s, sl.h, 2 * p + 1));
        GLT_LAUNCH_CHECK("adamw_pack");
        continue;
      }
      GLT_LAUNCH("adamw", adamw_kernel, dim3(grid_n(sh)), dim3(256), 0, st, w, grads[j] + p * sh,
                         m[j] + p * sh, v[j] + p * sh, (uint16_t*)nullptr, sh, lr, beta1, beta2, b1c, b2c, eps,
                         weight_decay, (const float*)nullptr, 0, 0.f);
      GLT_LAUNCH_CHECK("adamw_graft");
      if (packed_out && packed_out[j]) {
        glt_status s = pack_projection(w, sl.s, sl.h, p, packed_out[j], st);
        if (s != GLT_OK) return s;
      }
    }
  }
  return GLT_OK;
}

}  // extern "C"
