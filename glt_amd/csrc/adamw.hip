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

// (reference adamw_fused_kernel, src/kernels_optimizer_impl.inc:27-51)
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
    const float gi = g[i] * scale;
    float mi = m[i], vi = v[i];
    mi = b1 * mi + (1.0f - b1) * gi;
    vi = b2 * vi + (1.0f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    const float mh = mi * b1c, vh = vi * b2c;
    const float denom = sqrtf(vh) + eps;
    const float wi = w[i];
    const float nw = wi - lr * mh / denom - lr * wd * wi;
    w[i] = nw;
    if (mirror) mirror[i] = f32_to_bf16(nw);
  }
}

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
