// RMSNorm forward/backward and rotate-half RoPE for gfx950.
//
// RMSNorm: one workgroup per token row, the row spread over its wavefronts
// (4 in the forward, 8 in the backward) so that every lane holds one or two
// 16-byte chunks: the row is read once into registers, each wavefront sums
// its part with a butterfly, the partial sums meet in LDS (added in a fixed
// order, so every wavefront gets the same total), and the scaled row is
// written from the registers. Measured at 16384 x 4096 on the box with the
// inputs out of the caches (a 1 GiB read before every launch), against one
// wavefront per row: forward 51.3 -> 44.7 us, backward 117.3 -> 100.2 us.
// The inputs read long before (x) use the nontemporal policy: right after a
// kernel that leaves the last-level cache full of dirty lines (the optimizer
// step before the next forward) plain loads of x took 50 % longer; dy (just
// written by the dX GEMM) and the outputs (the next GEMM's input) are plain.
#include <atomic>
#include <cmath>

#include "common.hpp"
#include "norm_rope.hpp"

namespace glt {

constexpr int kRowsPerBlock = 4;                 // scalar paths: one wavefront per row
constexpr int kFwdWaves = 4, kBwdWaves = 8;      // vector paths: wavefronts per row

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

// Sum over the workgroup's W wavefronts of a per-wavefront value (lane 0's).
template <int W>
__device__ __forceinline__ float row_sum(float v, float* part) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int k = 0; k < W; ++k) t += part[k];
  return t;
}

// Vector path: D % 8 == 0, rows 16-byte aligned. Lane L of wavefront q owns
// chunks (8 bf16) q*64*NC + L + 64*i, i < NC, of its row.
template <int NC>
__global__ void __launch_bounds__(64 * kFwdWaves) rmsnorm_fwd_vec(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ y, float* __restrict__ var,
                                                                 int M, int D, float eps) {
  __shared__ float part[kFwdWaves];
  const int lane = threadIdx.x & 63, c0 = (threadIdx.x >> 6) * 64 * NC + lane;
  const int64_t row = blockIdx.x;
  const int nch = D >> 3;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * D);
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  // the row and its weight chunks are loaded together, so no load waits
  // behind the row reduction
  u32x4 xv[NC], wv[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i)
    if (c0 + 64 * i < nch) {
      xv[i] = __builtin_nontemporal_load(xr + c0 + 64 * i);
      wv[i] = wr[c0 + 64 * i];
    }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i)
    if (c0 + 64 * i < nch) {
      float f[8];
      unpack8(xv[i], f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
    }
  const float v = row_sum<kFwdWaves>(ss, part) / (float)D;
  const float r = rsqrtf(v + eps);
  if (threadIdx.x == 0) var[row] = v;
  u32x4* yr = reinterpret_cast<u32x4*>(y + row * D);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = c0 + 64 * i;
    if (c < nch) {
      float f[8], g[8];
      unpack8(xv[i], f);
      unpack8(wv[i], g);
      u32x4 o;
      o.x = pack_bf16x2(f[0] * r * g[0], f[1] * r * g[1]);
      o.y = pack_bf16x2(f[2] * r * g[2], f[3] * r * g[3]);
      o.z = pack_bf16x2(f[4] * r * g[4], f[5] * r * g[5]);
      o.w = pack_bf16x2(f[6] * r * g[6], f[7] * r * g[7]);
      yr[c] = o;
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
// src/kernels_rmsnorm_kernels.inc:86-125). The per-chunk arithmetic (8
// elements: x and w as bf16, dy and dx as f32) is shared by both backward
// kernels, so they round alike.
__device__ __forceinline__ float bwd_chunk_dot(const u32x4& xq, const u32x4& wq, const f32x4& d0, const f32x4& d1) {
  float f[8], g[8];
  unpack8(xq, f);
  unpack8(wq, g);
  float acc = 0.f;
  acc += d0.x * f[0] * g[0] + d0.y * f[1] * g[1] + d0.z * f[2] * g[2] + d0.w * f[3] * g[3];
  acc += d1.x * f[4] * g[4] + d1.y * f[5] * g[5] + d1.z * f[6] * g[6] + d1.w * f[7] * g[7];
  return acc;
}
__device__ __forceinline__ void bwd_chunk_out(const u32x4& xq, const u32x4& wq, const f32x4& d0, const f32x4& d1,
                                              float r, float mean, float r3, f32x4& o0, f32x4& o1) {
  float f[8], g[8];
  unpack8(xq, f);
  unpack8(wq, g);
  o0.x = d0.x * r * g[0] - f[0] * mean * r3;
  o0.y = d0.y * r * g[1] - f[1] * mean * r3;
  o0.z = d0.z * r * g[2] - f[2] * mean * r3;
  o0.w = d0.w * r * g[3] - f[3] * mean * r3;
  o1.x = d1.x * r * g[4] - f[4] * mean * r3;
  o1.y = d1.y * r * g[5] - f[5] * mean * r3;
  o1.z = d1.z * r * g[6] - f[6] * mean * r3;
  o1.w = d1.w * r * g[7] - f[7] * mean * r3;
}

// Lane L of wavefront q owns chunks
// q*64*NC + L + 64*i (8 elements: x as bf16, dy and dx as f32).
// dy and dx may be the same buffer (an in-place backward): every store of a
// row follows all loads of that row, so neither pointer is __restrict__.
template <int NC>
__global__ void __launch_bounds__(64 * kBwdWaves) rmsnorm_bwd_vec(const float* dy,
                                                                 const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 const float* __restrict__ var,
                                                                 float* dx, int M, int D, float eps) {
  __shared__ float part[kBwdWaves];
  const int lane = threadIdx.x & 63, c0 = (threadIdx.x >> 6) * 64 * NC + lane;
  const int64_t row = blockIdx.x;
  const int nch = D >> 3;
  const float r = rsqrtf(var[row] + eps);
  const float r3 = r * r * r;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * D);
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  const f32x4* dyr = reinterpret_cast<const f32x4*>(dy + row * D);
  u32x4 xv[NC], wv[NC];
  f32x4 d0[NC], d1[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = c0 + 64 * i;
    if (c < nch) {
      xv[i] = __builtin_nontemporal_load(xr + c);
      wv[i] = wr[c];
      d0[i] = dyr[2 * c];
      d1[i] = dyr[2 * c + 1];
    }
  }
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = c0 + 64 * i;
    if (c < nch) acc += bwd_chunk_dot(xv[i], wv[i], d0[i], d1[i]);
  }
  const float mean = row_sum<kBwdWaves>(acc, part) / (float)D;
  f32x4* dxr = reinterpret_cast<f32x4*>(dx + row * D);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = c0 + 64 * i;
    if (c < nch) {
      f32x4 o0, o1;
      bwd_chunk_out(xv[i], wv[i], d0[i], d1[i], r, mean, r3, o0, o1);
      dxr[2 * c] = o0;
      dxr[2 * c + 1] = o1;
    }
  }
}

// The same backward, one wavefront per row, for a persistent grid that runs
// beside another kernel on the CUs that kernel leaves idle (D/8 <= 512
// chunks: the single-chunk layout of rmsnorm_bwd_vec). Lane L does the work
// of lane L of each of the eight wavefronts of rmsnorm_bwd_vec<1> (chunk
// 64 q + L for q = 0..7), reduces each of those partial sums across the
// wavefront and adds the eight totals in order: the row's mean and dx are
// bit-identical to rmsnorm_bwd_vec<1>'s. The weight row is loaded once.
// Four wavefronts per workgroup (one per SIMD: the row's 24 KB of operands
// stay in registers).
constexpr int kRowsWaves = 4;
__global__ void __launch_bounds__(64 * kRowsWaves) rmsnorm_bwd_rows_kernel(const float* dy, const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ w, const float* __restrict__ var,
                                                        float* dx, int M, int D, float eps) {
  constexpr int Q = kBwdWaves;  // the eight wavefronts of rmsnorm_bwd_vec<1>
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = D >> 3;
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  u32x4 wv[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) wv[q] = 64 * q + lane < nch ? wr[64 * q + lane] : u32x4{0u, 0u, 0u, 0u};
  for (int64_t row = (int64_t)blockIdx.x * kRowsWaves + wave; row < M; row += (int64_t)gridDim.x * kRowsWaves) {
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * D);
    const f32x4* dyr = reinterpret_cast<const f32x4*>(dy + row * D);
    u32x4 xv[Q];
    f32x4 d0[Q], d1[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int c = 64 * q + lane;
      if (c < nch) {
        xv[q] = __builtin_nontemporal_load(xr + c);
        d0[q] = dyr[2 * c];
        d1[q] = dyr[2 * c + 1];
      }
    }
    const float r = rsqrtf(var[row] + eps);
    const float r3 = r * r * r;
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int c = 64 * q + lane;
      float acc = 0.f;
      if (c < nch) acc += bwd_chunk_dot(xv[q], wv[q], d0[q], d1[q]);
      t += wave_sum(acc);
    }
    const float mean = t / (float)D;
    f32x4* dxr = reinterpret_cast<f32x4*>(dx + row * D);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int c = 64 * q + lane;
      if (c < nch) {
        f32x4 o0, o1;
        bwd_chunk_out(xv[q], wv[q], d0[q], d1[q], r, mean, r3, o0, o1);
        dxr[2 * c] = o0;
        dxr[2 * c + 1] = o1;
      }
    }
  }
}



__global__ void __launch_bounds__(256) rmsnorm_bwd_scalar(const float* dy,
                                                          const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const float* __restrict__ var,
                                                          float* dx, int M, int D,
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

// chunks per lane of the vector paths: rows of up to W*64*8 chunks of 8
static int lane_chunks(int D, int waves) {
  const int64_t ch = cdiv(cdiv(D / 8, 64), waves);
  return ch <= 1 ? 1 : ch <= 2 ? 2 : ch <= 4 ? 4 : ch <= 8 ? 8 : 0;
}

// LDS the row kernel asks for (it uses none): more than half of a CU's
// 160 KB, so two of its workgroups never share a CU.
constexpr int kRowsKernelLds = 96 * 1024;

bool rmsnorm_bwd_rows_ok(const float* dy, const uint16_t* x, const uint16_t* w, const float* dx, int M, int D) {
  return M > 0 && D > 0 && D % 8 == 0 && lane_chunks(D, kBwdWaves) == 1 && aligned16(x) && aligned16(w) &&
         aligned16(dy) && aligned16(dx);
}

glt_status rmsnorm_bwd_rows(const float* dy, const uint16_t* x, const uint16_t* w, const float* var, float* dx, int M,
                            int D, float eps, int grid, hipStream_t st) {
  GLT_CHECK(rmsnorm_bwd_rows_ok(dy, x, w, dx, M, D) && grid > 0, GLT_ERR_UNSUPPORTED,
            "rmsnorm_bwd_rows: M=%d D=%d grid=%d", M, D, grid);
  static std::atomic<bool> attr_set[64];
  int dev = 0;
  GLT_TRY_HIP(hipGetDevice(&dev));
  GLT_CHECK(dev >= 0 && dev < 64, GLT_ERR_HIP, "rmsnorm_bwd_rows: device index %d out of range", dev);
  if (!attr_set[dev].load(std::memory_order_acquire)) {
    GLT_TRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(rmsnorm_bwd_rows_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kRowsKernelLds));
    attr_set[dev].store(true, std::memory_order_release);
  }
  GLT_LAUNCH("rmsnorm_bwd_beside", rmsnorm_bwd_rows_kernel, dim3((unsigned)grid), dim3(64 * kRowsWaves), kRowsKernelLds, st,
             dy, x, w, var, dx, M, D, eps);
  GLT_LAUNCH_CHECK("rmsnorm_bwd_rows");
  return GLT_OK;
}

// ------------------------------------------------------------------- RoPE
// One workgroup per token (b, t). A thread owns up to IT items of 8
// consecutive rotary pairs (one 16-byte load from each half of a head) over
// all q and k heads of the token, and issues all of its loads first; then the
// 64 (cos, sin) pairs of the position are computed into LDS with the
// reference's f32 recipe and rounded to bf16 while the loads are in flight,
// and every item is rotated and written back in place. (Measured cold at the
// decoder-layer shape: 32.6 -> 30.1 us against computing the pairs first and
// looping over the items.)
template <int IT>
__global__ void __launch_bounds__(256) rope_vec_kernel(uint16_t* __restrict__ q, int nq, uint16_t* __restrict__ k,
                                                       int nk, int T, int hd, float theta, int pos_offset) {
  extern __shared__ float cs[];  // [half] cos then [half] sin
  const int half = hd >> 1, groups = half >> 3;
  const int64_t tok = blockIdx.x;
  const int pos = (int)(tok % T) + pos_offset;
  const int nitems = (nq + nk) * groups;
  u32x4 a[IT], b[IT];
  u32x4* p1[IT];
  int gi[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int item = threadIdx.x + 256 * it;
    p1[it] = nullptr;
    if (item < nitems) {
      const int h = item / groups, g = item % groups;
      uint16_t* head = h < nq ? q + (tok * nq + h) * (int64_t)hd : k + (tok * nk + (h - nq)) * (int64_t)hd;
      p1[it] = reinterpret_cast<u32x4*>(head + 8 * g);
      gi[it] = g;
      a[it] = p1[it][0];
      b[it] = *reinterpret_cast<const u32x4*>(head + half + 8 * g);
    }
  }
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
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (!p1[it]) continue;
    float x1[8], x2[8];
    unpack8(a[it], x1);
    unpack8(b[it], x2);
    const float* c = cs + 8 * gi[it];
    const float* s = cs + half + 8 * gi[it];
    float r1[8], r2[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      r1[j] = x1[j] * c[j] - x2[j] * s[j];
      r2[j] = x2[j] * c[j] + x1[j] * s[j];
    }
    u32x4 o1, o2;
    o1.x = pack_bf16x2(r1[0], r1[1]); o1.y = pack_bf16x2(r1[2], r1[3]);
    o1.z = pack_bf16x2(r1[4], r1[5]); o1.w = pack_bf16x2(r1[6], r1[7]);
    o2.x = pack_bf16x2(r2[0], r2[1]); o2.y = pack_bf16x2(r2[2], r2[3]);
    o2.z = pack_bf16x2(r2[4], r2[5]); o2.w = pack_bf16x2(r2[6], r2[7]);
    p1[it][0] = o1;
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p1[it]) + half) = o2;
  }
}

// Any head_dim / alignment: the pairs first, then one element pair per
// thread-iteration.
__global__ void __launch_bounds__(256) rope_kernel(uint16_t* __restrict__ q, int nq, uint16_t* __restrict__ k, int nk,
                                                   int T, int hd, float theta, int pos_offset) {
  extern __shared__ float cs[];
  const int half = hd >> 1;
  const int64_t tok = blockIdx.x;
  const int pos = (int)(tok % T) + pos_offset;
  for (int i = threadIdx.x; i < half; i += blockDim.x) {
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

}  // namespace glt

using namespace glt;

extern "C" {

glt_status glt_rmsnorm_fwd(const uint16_t* x, const uint16_t* w, uint16_t* y, float* var, int32_t M,
                           int32_t D, float eps, void* stream) {
  GLT_CHECK(M >= 0 && D > 0, GLT_ERR_SHAPE, "glt_rmsnorm_fwd: M=%d D=%d", M, D);
  GLT_CHECK(M == 0 || (x && w && y && var), GLT_ERR_INVALID_ARG, "glt_rmsnorm_fwd: null pointer");
  if (M == 0) return GLT_OK;
  hipStream_t st = as_stream(stream);
  const int nc = lane_chunks(D, kFwdWaves);
  if (D % 8 == 0 && nc > 0 && aligned16(x) && aligned16(w) && aligned16(y)) {
    const dim3 grid((unsigned)M), block(64 * kFwdWaves);
    switch (nc) {
      case 1: GLT_LAUNCH("rmsnorm_fwd", rmsnorm_fwd_vec<1>, grid, block, 0, st, x, w, y, var, M, D, eps); break;
      case 2: GLT_LAUNCH("rmsnorm_fwd", rmsnorm_fwd_vec<2>, grid, block, 0, st, x, w, y, var, M, D, eps); break;
      case 4: GLT_LAUNCH("rmsnorm_fwd", rmsnorm_fwd_vec<4>, grid, block, 0, st, x, w, y, var, M, D, eps); break;
      default: GLT_LAUNCH("rmsnorm_fwd", rmsnorm_fwd_vec<8>, grid, block, 0, st, x, w, y, var, M, D, eps); break;
    }
  } else {
    GLT_LAUNCH("rmsnorm_fwd", rmsnorm_fwd_scalar, dim3((unsigned)cdiv(M, kRowsPerBlock)), dim3(256), 0, st, x, w, y,
               var, M, D, eps);
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
  const int nc = lane_chunks(D, kBwdWaves);
  if (D % 8 == 0 && nc > 0 && nc <= 4 && aligned16(x) && aligned16(w) && aligned16(dy) && aligned16(dx)) {
    const dim3 grid((unsigned)M), block(64 * kBwdWaves);
    switch (nc) {
      case 1: GLT_LAUNCH("rmsnorm_bwd", rmsnorm_bwd_vec<1>, grid, block, 0, st, dy, x, w, var, dx, M, D, eps); break;
      case 2: GLT_LAUNCH("rmsnorm_bwd", rmsnorm_bwd_vec<2>, grid, block, 0, st, dy, x, w, var, dx, M, D, eps); break;
      default: GLT_LAUNCH("rmsnorm_bwd", rmsnorm_bwd_vec<4>, grid, block, 0, st, dy, x, w, var, dx, M, D, eps); break;
    }
  } else {
    GLT_LAUNCH("rmsnorm_bwd", rmsnorm_bwd_scalar, dim3((unsigned)cdiv(M, kRowsPerBlock)), dim3(256), 0, st, dy, x, w,
               var, dx, M, D, eps);
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
  const int64_t items = (int64_t)(n_q_heads + n_kv_heads) * (head_dim / 16);
  const int it = items <= 256 ? 1 : items <= 512 ? 2 : items <= 1024 ? 4 : 0;
  uint16_t* qq = n_q_heads ? q : nullptr;
  uint16_t* kk = n_kv_heads ? k : nullptr;
  const dim3 grid((unsigned)((int64_t)B * T)), block(256);
  const size_t lds = head_dim * sizeof(float);
  hipStream_t st = as_stream(stream);
  if (vec && it == 1)
    GLT_LAUNCH("rope", rope_vec_kernel<1>, grid, block, lds, st, qq, n_q_heads, kk, n_kv_heads, T, head_dim, theta,
               pos_offset);
  else if (vec && it == 2)
    GLT_LAUNCH("rope", rope_vec_kernel<2>, grid, block, lds, st, qq, n_q_heads, kk, n_kv_heads, T, head_dim, theta,
               pos_offset);
  else if (vec && it == 4)
    GLT_LAUNCH("rope", rope_vec_kernel<4>, grid, block, lds, st, qq, n_q_heads, kk, n_kv_heads, T, head_dim, theta,
               pos_offset);
  else
    GLT_LAUNCH("rope", rope_kernel, grid, block, lds, st, qq, n_q_heads, kk, n_kv_heads, T, head_dim, theta,
               pos_offset);
  GLT_LAUNCH_CHECK("rope");
  return GLT_OK;
}

}  // extern "C"
