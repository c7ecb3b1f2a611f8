// RMSNorm forward/backward and rotate-half RoPE for gfx950.
//
// RMSNorm: one 64-lane wavefront per token row, four rows per 256-thread
// workgroup. A row of D <= 64*8*kMaxChunks bf16 values is read once with
// 16-byte loads and kept in registers between the sum-of-squares reduction
// (wave-level butterfly, no LDS) and the scaled write.
#include <cmath>

#include "common.hpp"

namespace glt {

constexpr int kRowsPerBlock = 4;
constexpr int kMaxChunks = 16;  // 8 bf16 per chunk per lane -> D <= 8192 in registers

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ void unpack8(const u32x4& q, float* f) {
  f[0] = bf16_to_f32((uint16_t)(q.x & 0xFFFF)); f[1] = bf16_to_f32((uint16_t)(q.x >> 16));
  f[2] = bf16_to_f32((uint16_t)(q.y & 0xFFFF)); f[3] = bf16_to_f32((uint16_t)(q.y >> 16));
  f[4] = bf16_to_f32((uint16_t)(q.z & 0xFFFF)); f[5] = bf16_to_f32((uint16_t)(q.z >> 16));
  f[6] = bf16_to_f32((uint16_t)(q.w & 0xFFFF)); f[7] = bf16_to_f32((uint16_t)(q.w >> 16));
}

// Vector path: D % 8 == 0, rows 16-byte aligned, D <= 512*kMaxChunks.
template <int CH>
__global__ void __launch_bounds__(256) rmsnorm_fwd_vec(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ w,
                                                       uint16_t* __restrict__ y, float* __restrict__ var,
                                                       int M, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= M) return;
  const int nch = D >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (int64_t)row * D);
  u32x4 xv[CH];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      xv[i] = __builtin_nontemporal_load(xr + c);
      float f[8];
      unpack8(xv[i], f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
    }
  }
  ss = wave_sum(ss);
  const float v = ss / (float)D;
  const float r = rsqrtf(v + eps);
  if (lane == 0) var[row] = v;
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  u32x4* yr = reinterpret_cast<u32x4*>(y + (int64_t)row * D);
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      float f[8], g[8];
      unpack8(xv[i], f);
      unpack8(wr[c], g);
      u32x4 o;
      o.x = pack_bf16x2(f[0] * r * g[0], f[1] * r * g[1]);
      o.y = pack_bf16x2(f[2] * r * g[2], f[3] * r * g[3]);
      o.z = pack_bf16x2(f[4] * r * g[4], f[5] * r * g[5]);
      o.w = pack_bf16x2(f[6] * r * g[6], f[7] * r * g[7]);
      __builtin_nontemporal_store(o, yr + c);
    }
  }
}

// Scalar path for any D / alignment (two passes over x).
__global__ void __launch_bounds__(256) rmsnorm_fwd_scalar(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          uint16_t* __restrict__ y,
                                                          float* __restrict__ var, int M, int D,
                                                          float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint16_t* xr = x + (int64_t)row * D;
  float ss = 0.f;
  for (int c = lane; c < D; c += 64) {
    const float f = bf16_to_f32(xr[c]);
    ss += f * f;
  }
  ss = wave_sum(ss);
  const float v = ss / (float)D;
  const float r = rsqrtf(v + eps);
  if (lane == 0) var[row] = v;
  for (int c = lane; c < D; c += 64)
    y[(int64_t)row * D + c] = f32_to_bf16(bf16_to_f32(xr[c]) * r * bf16_to_f32(w[c]));
}

// Backward: dx = dy*r*w - x*mean(dy*x*w)*r^3 (reference
// src/kernels_rmsnorm_kernels.inc:86-125), one wavefront per row.
template <int CH>
__global__ void __launch_bounds__(256) rmsnorm_bwd_vec(const float* __restrict__ dy,
                                                       const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ w,
                                                       const float* __restrict__ var,
                                                       float* __restrict__ dx, int M, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= M) return;
  const int nch = D >> 3;
  const float r = rsqrtf(var[row] + eps);
  const float r3 = r * r * r;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (int64_t)row * D);
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  const f32x4* dyr = reinterpret_cast<const f32x4*>(dy + (int64_t)row * D);
  u32x4 xv[CH];
  f32x4 d0[CH], d1[CH];
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      xv[i] = xr[c];
      d0[i] = dyr[2 * c];
      d1[i] = dyr[2 * c + 1];
      float f[8], g[8];
      unpack8(xv[i], f);
      unpack8(wr[c], g);
      acc += d0[i].x * f[0] * g[0] + d0[i].y * f[1] * g[1] + d0[i].z * f[2] * g[2] + d0[i].w * f[3] * g[3];
      acc += d1[i].x * f[4] * g[4] + d1[i].y * f[5] * g[5] + d1[i].z * f[6] * g[6] + d1[i].w * f[7] * g[7];
    }
  }
  acc = wave_sum(acc);
  const float mean = acc / (float)D;
  f32x4* dxr = reinterpret_cast<f32x4*>(dx + (int64_t)row * D);
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      float f[8], g[8];
      unpack8(xv[i], f);
      unpack8(wr[c], g);
      f32x4 o0, o1;
      o0.x = d0[i].x * r * g[0] - f[0] * mean * r3;
      o0.y = d0[i].y * r * g[1] - f[1] * mean * r3;
      o0.z = d0[i].z * r * g[2] - f[2] * mean * r3;
      o0.w = d0[i].w * r * g[3] - f[3] * mean * r3;
      o1.x = d1[i].x * r * g[4] - f[4] * mean * r3;
      o1.y = d1[i].y * r * g[5] - f[5] * mean * r3;
      o1.z = d1[i].z * r * g[6] - f[6] * mean * r3;
      o1.w = d1[i].w * r * g[7] - f[7] * mean * r3;
      dxr[2 * c] = o0;
      dxr[2 * c + 1] = o1;
    }
  }
}

__global__ void __launch_bounds__(256) rmsnorm_bwd_scalar(const float* __restrict__ dy,
                                                          const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const float* __restrict__ var,
                                                          float* __restrict__ dx, int M, int D,
                                                          float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= M) return;
  const float r = rsqrtf(var[row] + eps);
  const float r3 = r * r * r;
  const int64_t o = (int64_t)row * D;
  float acc = 0.f;
  for (int c = lane; c < D; c += 64) acc += dy[o + c] * bf16_to_f32(x[o + c]) * bf16_to_f32(w[c]);
  acc = wave_sum(acc);
  const float mean = acc / (float)D;
  for (int c = lane; c < D; c += 64)
    dx[o + c] = dy[o + c] * r * bf16_to_f32(w[c]) - bf16_to_f32(x[o + c]) * mean * r3;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

#define GLT_CH_DISPATCH(LABEL, CHN, KERNEL, ...)                                    \
  switch (CHN) {                                                                   \
    case 1: GLT_LAUNCH(LABEL, KERNEL<1>, __VA_ARGS__); break;                      \
    case 2: GLT_LAUNCH(LABEL, KERNEL<2>, __VA_ARGS__); break;                      \
    case 4: GLT_LAUNCH(LABEL, KERNEL<4>, __VA_ARGS__); break;                      \
    case 8: GLT_LAUNCH(LABEL, KERNEL<8>, __VA_ARGS__); break;                      \
    default: GLT_LAUNCH(LABEL, KERNEL<16>, __VA_ARGS__); break;                    \
  }

static int chunk_bucket(int D) {
  const int ch = (int)cdiv(D / 8, 64);
  return ch <= 1 ? 1 : ch <= 2 ? 2 : ch <= 4 ? 4 : ch <= 8 ? 8 : 16;
}

// ------------------------------------------------------------------- RoPE
// One workgroup per token (b, t): the 64 (cos, sin) pairs of the position are
// computed once into LDS with the reference's f32 recipe and rounded to bf16,
// then every q and k head of the token is rotated from them. A thread owns
// 8 consecutive rotary pairs (16-byte loads of x1 and x2 halves).
__global__ void __launch_bounds__(256) rope_kernel(uint16_t* __restrict__ q, int nq,
                                                   uint16_t* __restrict__ k, int nk, int T,
                                                   int hd, float theta, int pos_offset, int vec) {
  extern __shared__ float cs[];  // [half] cos then [half] sin
  const int half = hd >> 1;
  const int64_t tok = blockIdx.x;
  const int pos = (int)(tok % T) + pos_offset;
  for (int i = threadIdx.x; i < half; i += blockDim.x) {
    // reference src/rope_impl.inc:14-19: i2 = 2i (f32), inv = 1/theta^(i2/hd),
    // ang = pos*inv, emb = [ang, ang], cos/sin cast to the tensor dtype
    const float e = (float)(2 * i) / (float)hd;
    const float inv = 1.0f / powf(theta, e);
    const float ang = (float)pos * inv;
    cs[i] = bf16_to_f32(f32_to_bf16(cosf(ang)));
    cs[half + i] = bf16_to_f32(f32_to_bf16(sinf(ang)));
  }
  __syncthreads();
  for (int pass = 0; pass < 2; ++pass) {
    uint16_t* t = pass == 0 ? q : k;
    const int nh = pass == 0 ? nq : nk;
    if (!t) continue;
    uint16_t* row = t + tok * (int64_t)nh * hd;
    if (vec) {
      const int groups = half >> 3;  // 8 pairs per thread
      for (int item = threadIdx.x; item < nh * groups; item += blockDim.x) {
        const int h = item / groups, g = item % groups;
        u32x4* p1 = reinterpret_cast<u32x4*>(row + (int64_t)h * hd + 8 * g);
        u32x4* p2 = reinterpret_cast<u32x4*>(row + (int64_t)h * hd + half + 8 * g);
        float a[8], b[8];
        unpack8(*p1, a);
        unpack8(*p2, b);
        float r1[8], r2[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float c = cs[8 * g + j], s = cs[half + 8 * g + j];
          r1[j] = a[j] * c - b[j] * s;
          r2[j] = b[j] * c + a[j] * s;
        }
        u32x4 o1, o2;
        o1.x = pack_bf16x2(r1[0], r1[1]); o1.y = pack_bf16x2(r1[2], r1[3]);
        o1.z = pack_bf16x2(r1[4], r1[5]); o1.w = pack_bf16x2(r1[6], r1[7]);
        o2.x = pack_bf16x2(r2[0], r2[1]); o2.y = pack_bf16x2(r2[2], r2[3]);
        o2.z = pack_bf16x2(r2[4], r2[5]); o2.w = pack_bf16x2(r2[6], r2[7]);
        *p1 = o1;
        *p2 = o2;
      }
    } else {
      for (int item = threadIdx.x; item < nh * half; item += blockDim.x) {
        const int h = item / half, i = item % half;
        uint16_t* p = row + (int64_t)h * hd;
        const float a = bf16_to_f32(p[i]), b = bf16_to_f32(p[half + i]);
        const float c = cs[i], s = cs[half + i];
        p[i] = f32_to_bf16(a * c - b * s);
        p[half + i] = f32_to_bf16(b * c + a * s);
      }
    }
  }
}

}  // namespace glt

using namespace glt;

extern "C" {

glt_status glt_rmsnorm_fwd(const uint16_t* x, const uint16_t* w, uint16_t* y, float* var, int32_t M,
                           int32_t D, float eps, void* stream) {
  GLT_CHECK(M >= 0 && D > 0, GLT_ERR_SHAPE, "glt_rmsnorm_fwd: M=%d D=%d", M, D);
  GLT_CHECK(M == 0 || (x && w && y && var), GLT_ERR_INVALID_ARG, "glt_rmsnorm_fwd: null pointer");
  if (M == 0) return GLT_OK;
  hipStream_t st = as_stream(stream);
  dim3 grid((unsigned)cdiv(M, kRowsPerBlock)), block(256);
  if (D % 8 == 0 && D <= 512 * kMaxChunks && aligned16(x) && aligned16(w) && aligned16(y)) {
    GLT_CH_DISPATCH("rmsnorm_fwd", chunk_bucket(D), rmsnorm_fwd_vec, grid, block, 0, st, x, w, y, var, M, D, eps);
  } else {
    GLT_LAUNCH("rmsnorm_fwd", rmsnorm_fwd_scalar, grid, block, 0, st, x, w, y, var, M, D, eps);
  }
  GLT_LAUNCH_CHECK("rmsnorm_fwd");
  return GLT_OK;
}

glt_status glt_rmsnorm_bwd(const float* dy, const uint16_t* x, const uint16_t* w, const float* var,
                           float* dx, int32_t M, int32_t D, float eps, void* stream) {
  GLT_CHECK(M >= 0 && D > 0, GLT_ERR_SHAPE, "glt_rmsnorm_bwd: M=%d D=%d", M, D);
  GLT_CHECK(M == 0 || (dy && x && w && var && dx), GLT_ERR_INVALID_ARG, "glt_rmsnorm_bwd: null pointer");
  if (M == 0) return GLT_OK;
  hipStream_t st = as_stream(stream);
  dim3 grid((unsigned)cdiv(M, kRowsPerBlock)), block(256);
  if (D % 8 == 0 && D <= 512 * kMaxChunks && aligned16(x) && aligned16(w) && aligned16(dy) &&
      aligned16(dx)) {
    GLT_CH_DISPATCH("rmsnorm_bwd", chunk_bucket(D), rmsnorm_bwd_vec, grid, block, 0, st, dy, x, w, var, dx, M, D, eps);
  } else {
    GLT_LAUNCH("rmsnorm_bwd", rmsnorm_bwd_scalar, grid, block, 0, st, dy, x, w, var, dx, M, D, eps);
  }
  GLT_LAUNCH_CHECK("rmsnorm_bwd");
  return GLT_OK;
}

glt_status glt_rope_fwd(uint16_t* q, int32_t n_q_heads, uint16_t* k, int32_t n_kv_heads, int32_t B,
                        int32_t T, int32_t head_dim, float theta, int32_t pos_offset, void* stream) {
  GLT_CHECK(B >= 0 && T >= 0 && head_dim > 0 && head_dim % 2 == 0, GLT_ERR_SHAPE,
            "glt_rope_fwd: B=%d T=%d head_dim=%d", B, T, head_dim);
  GLT_CHECK(n_q_heads >= 0 && n_kv_heads >= 0, GLT_ERR_SHAPE, "glt_rope_fwd: heads");
  GLT_CHECK(q || n_q_heads == 0, GLT_ERR_INVALID_ARG, "glt_rope_fwd: null q");
  GLT_CHECK(k || n_kv_heads == 0, GLT_ERR_INVALID_ARG, "glt_rope_fwd: null k");
  GLT_CHECK(theta > 0.f, GLT_ERR_INVALID_ARG, "glt_rope_fwd: theta");
  if ((int64_t)B * T == 0) return GLT_OK;
  const int vec = (head_dim % 16 == 0) && (!q || aligned16(q)) && (!k || aligned16(k));
  GLT_LAUNCH("rope", rope_kernel, dim3((unsigned)((int64_t)B * T)), dim3(256), head_dim * sizeof(float),
                     as_stream(stream), n_q_heads ? q : nullptr, n_q_heads, n_kv_heads ? k : nullptr,
                     n_kv_heads, T, head_dim, theta, pos_offset, vec);
  GLT_LAUNCH_CHECK("rope");
  return GLT_OK;
}

}  // extern "C"
