// AdamW over graft parameters with the optional global-L2 gradient clip and
// the bf16 mirror refresh fused into the update.
#include <algorithm>
#include <cmath>
#include <mutex>

#include "common.hpp"
#include "layout.hpp"

namespace glt {


constexpr int kClipBlocks = 512;
constexpr int kClipSegsPerLaunch = 32;

// The gradient vectors of one launch of the clip's partial sums: f32 sums of
// g^2 (like the reference reduce_l2_kernel,
// src/kernels_elementwise_impl.inc:141-165), one partial per workgroup.
// Workgroup b covers elements [(b - blk0[j]) * chunk, ...+chunk) of segment
// j, blk0[j] <= b < blk0[j+1], and writes partial[out0 + b]. One clip norm
// may take several launches (any number of segments): they share one chunk
// size and write consecutive ranges of the partials.
struct ClipSegs {
  const float* g[kClipSegsPerLaunch];
  int64_t n[kClipSegsPerLaunch];
  int blk0[kClipSegsPerLaunch + 1];
  int64_t chunk;  // elements per workgroup, a multiple of 1024
  int nseg;
  int out0;
};

__global__ void __launch_bounds__(256) sumsq_partial_kernel(const ClipSegs segs, float* __restrict__ partial) {
  __shared__ float wsum[4];
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < segs.nseg && b >= segs.blk0[j + 1]) ++j;
  const float* g = segs.g[j];
  const int64_t lo = (int64_t)(b - segs.blk0[j]) * segs.chunk;
  const int64_t hi = min(lo + segs.chunk, segs.n[j]);
  float s = 0.f;
  if ((reinterpret_cast<uintptr_t>(g) & 15) == 0) {
    // 16-byte loads, eight in flight per thread before any is summed
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
    const int64_t lo4 = lo / 4, hi4 = hi / 4;  // chunk % 4 == 0: lo4 * 4 == lo
    constexpr int U = 8;
    for (int64_t i0 = lo4 + threadIdx.x; i0 < hi4; i0 += 256 * U) {
      f32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = i0 + 256 * u < hi4 ? g4[i0 + 256 * u] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < U; ++u) s += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
    }
    for (int64_t i = hi4 * 4 + threadIdx.x; i < hi; i += 256) s += g[i] * g[i];
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) s += g[i] * g[i];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[segs.out0 + b] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

// scale = clip/norm if norm > clip else 1, norm = sqrt(sum + 1e-8)
// (reference calc_scale_kernel, src/kernels_elementwise_impl.inc:170-197).
// Every workgroup of an update kernel adds the np partials in the same
// fixed order, so all of them get the same scale without a launch of its own.
__device__ float block_clip_scale(const float* __restrict__ partial, int np, float clip) {
  __shared__ float wsum[4];
  float s = 0.f;
  for (int i = threadIdx.x; i < np; i += 256) s += partial[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
  __syncthreads();
  const float norm = sqrtf(wsum[0] + wsum[1] + wsum[2] + wsum[3] + 1e-8f);
  return norm > clip ? clip / norm : 1.0f;
}

// The partials of one clip norm over the nseg gradient vectors g[j] of n[j]
// elements: ws[0, np), from as many launches as the segments need
// (kClipSegsPerLaunch each). The chunk is the smallest multiple of 1024 whose
// workgroups over all segments number at most kClipBlocks, so each segment
// needs at least one partial: at most kClipBlocks segments. Returns np
// through *np_out.
glt_status launch_clip(const float* const* g, const int64_t* n, int nseg, float* ws, size_t ws_floats, int* np_out,
                       hipStream_t st) {
  GLT_CHECK(nseg <= kClipBlocks, GLT_ERR_UNSUPPORTED,
            "adamw clip: %d gradient segments, at most %d (one partial sum each)", nseg, kClipBlocks);
  int64_t total = 0;
  for (int j = 0; j < nseg; ++j) total += n[j];
  int64_t chunk = std::max<int64_t>(1024, cdiv(cdiv(total, kClipBlocks), 1024) * 1024);
  auto blocks = [&](int64_t c) {
    int64_t nb = 0;
    for (int j = 0; j < nseg; ++j) nb += cdiv(n[j], c);
    return nb;
  };
  while (blocks(chunk) > kClipBlocks) chunk += 1024;
  int np = 0;
  for (int j0 = 0; j0 < nseg; j0 += kClipSegsPerLaunch) {
    ClipSegs segs{};
    segs.chunk = chunk;
    segs.out0 = np;
    int nb = 0;
    for (int j = j0; j < nseg && segs.nseg < kClipSegsPerLaunch; ++j) {
      segs.g[segs.nseg] = g[j];
      segs.n[segs.nseg] = n[j];
      segs.blk0[segs.nseg] = nb;
      nb += (int)cdiv(n[j], chunk);
      ++segs.nseg;
    }
    segs.blk0[segs.nseg] = nb;
    if (nb == 0) continue;  // every segment of this launch is empty
    GLT_CHECK((size_t)(np + nb) <= ws_floats, GLT_ERR_WORKSPACE, "adamw clip: %d partial sums, room for %zu",
              np + nb, ws_floats);
    GLT_LAUNCH("clip_sumsq", sumsq_partial_kernel, dim3(nb), dim3(256), 0, st, segs, ws);
    GLT_LAUNCH_CHECK("sumsq_partial");
    np += nb;
  }
  // every segment empty: np = 0, and the update's scale comes from the
  // norm of an empty sum
  *np_out = np;
  return GLT_OK;
}

// Clip inputs of an update kernel: partial == nullptr means no clip.
struct ClipIn {
  const float* partial;
  int np;
  float clip;
};

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
                                                    float wd, const ClipIn ci) {
  const float scale = ci.partial ? block_clip_scale(ci.partial, ci.np, ci.clip) : 1.0f;
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

// AdamW over [S, H] graft projections fused with the refresh of their four
// bf16 mirrors in the packed slice: row-major [S,H], row-major [H,S], and
// the fragment layout of both. One workgroup per 64 x 64 tile (S and H
// multiples of 64, so no fragment block is padded), the tiles of every
// projection of a step in one launch: the f32 state streams through
// registers as 16-byte accesses, the new weights go through LDS once, and
// every mirror is written with 16-byte stores. The master is read once
// instead of once per mirror. One launch takes up to kMaxPackJobs
// projections; a step over more issues several, which all read the same
// clip partials.
constexpr int kMaxPackJobs = 24;
struct PackJob {
  float* w;
  const float* g;
  float* m;
  float* v;
  uint16_t* rm;   // row-major [S,H]
  uint16_t* rmt;  // row-major [H,S]
  uint16_t* sh;   // fragment layout of [S,H]
  uint16_t* sht;  // fragment layout of [H,S]
  int S, H;
  int tile0;      // first workgroup of this projection
};
struct PackJobs {
  PackJob j[kMaxPackJobs];
  int n;
};

__global__ void __launch_bounds__(256) adamw_pack_kernel(const PackJobs jobs, float lr, float b1, float b2, float b1c,
                                                         float b2c, float eps, float wd, const ClipIn ci) {
  __shared__ float tile[64][65];
  const float scale = ci.partial ? block_clip_scale(ci.partial, ci.np, ci.clip) : 1.0f;
  int jb = 0;
  while (jb + 1 < jobs.n && (int)blockIdx.x >= jobs.j[jb + 1].tile0) ++jb;
  const PackJob& J = jobs.j[jb];
  float* __restrict__ w = J.w;
  const float* __restrict__ g = J.g;
  float* __restrict__ m = J.m;
  float* __restrict__ v = J.v;
  const int S = J.S, H = J.H;
  const int hb = H / 64;
  const int bt = (int)blockIdx.x - J.tile0;
  const int r0 = (bt / hb) * 64, c0 = (bt % hb) * 64;
  const int t = threadIdx.x;
  {
    const int rr = t >> 4, c4 = (t & 15) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rr + 16 * i;
      const int64_t o = (int64_t)(r0 + r) * H + c0 + c4;
      const f32x4 wi = *reinterpret_cast<const f32x4*>(w + o);
      const f32x4 gi = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g + o));
      f32x4 mi = *reinterpret_cast<const f32x4*>(m + o), vi = *reinterpret_cast<const f32x4*>(v + o);
      f32x4 nw;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float a = mi[e], b = vi[e];
        nw[e] = adamw_elem(wi[e], gi[e] * scale, a, b, lr, b1, b2, b1c, b2c, eps, wd);
        mi[e] = a;
        vi[e] = b;
        tile[r][c4 + e] = nw[e];
      }
      // the moments and masters are read again only by the next step's
      // update: written past the caches
      __builtin_nontemporal_store(mi, reinterpret_cast<f32x4*>(m + o));
      __builtin_nontemporal_store(vi, reinterpret_cast<f32x4*>(v + o));
      __builtin_nontemporal_store(nw, reinterpret_cast<f32x4*>(w + o));
      u32x2 q;
      q.x = pack_bf16x2(nw[0], nw[1]);
      q.y = pack_bf16x2(nw[2], nw[3]);
      *reinterpret_cast<u32x2*>(J.rm + o) = q;
    }
  }
  __syncthreads();
  {
    // [H,S] row-major: column c of the tile, 16 consecutive rows per thread
    const int c = t >> 2, rs = (t & 3) * 16;
    uint16_t* dst = J.rmt + (int64_t)(c0 + c) * S + r0 + rs;
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
      *reinterpret_cast<u32x4*>(J.sh + blk * kShufBlock + t * 8) = q;
      *reinterpret_cast<u32x4*>(J.sht + blkt * kShufBlock + t * 8) = qt;
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
  ClipIn ci{nullptr, 0, clip_norm};
  if (clip_norm > 0.f) {
    GLT_CHECK(ws && ws_bytes >= glt_adamw_workspace_size(n), GLT_ERR_WORKSPACE,
              "glt_adamw_step: clip needs %zu workspace bytes", glt_adamw_workspace_size(n));
    const float* gs[1] = {g};
    const int64_t ns[1] = {n};
    glt_status s = launch_clip(gs, ns, 1, static_cast<float*>(ws), ws_bytes / sizeof(float), &ci.np, st);
    if (s != GLT_OK) return s;
    ci.partial = static_cast<const float*>(ws);
  }
  // bias corrections as the reference computes them on the host
  // (src/kernels_optimizer_impl.inc:64-65)
  const float b1c = 1.0f / (1.0f - powf(beta1, (float)(step + 1)));
  const float b2c = 1.0f / (1.0f - powf(beta2, (float)(step + 1)));
  GLT_LAUNCH("adamw", adamw_kernel, dim3(grid_n(n)), dim3(256), 0, st, w, g, m, v, mirror, n, lr, beta1, beta2,
                     b1c, b2c, eps, weight_decay, ci);
  GLT_LAUNCH_CHECK("adamw");
  return GLT_OK;
}

namespace glt {
// The graft step; the clip's partial sums go to clip_ws (clip_ws_floats
// floats, at least kClipBlocks).
static glt_status graft_step(const glt_graft_slice* slices, int32_t n_slices, float* const* grads, float* const* m,
                             float* const* v, uint16_t* const* packed_out, int32_t proj_mask, int32_t step, float lr,
                             float beta1, float beta2, float eps, float weight_decay, float clip_norm,
                             float* clip_ws, size_t clip_ws_floats, hipStream_t st) {
  GLT_CHECK(n_slices >= 0, GLT_ERR_SHAPE, "glt_adamw_graft_step: %d slices", n_slices);
  GLT_CHECK(n_slices == 0 || (slices && grads && m && v), GLT_ERR_INVALID_ARG, "glt_adamw_graft_step: null pointer");
  for (int j = 0; j < n_slices; ++j)
    GLT_CHECK(grads[j] && m[j] && v[j], GLT_ERR_INVALID_ARG, "glt_adamw_graft_step: null state of slice %d", j);
  ClipIn ci{nullptr, 0, clip_norm};
  if (clip_norm > 0.f) {
    // one global L2 norm over every projection this step updates, of every
    // slice (the reference clips all of its L*3 deltas together,
    // grafting.hip:1149-1164; the gradients of projections it does not
    // graft stay zero)
    const float* gs[kClipBlocks];
    int64_t ns[kClipBlocks];
    int nseg = 0;
    for (int j = 0; j < n_slices; ++j) {
      const glt_graft_slice& sl = slices[j];
      const int64_t sh = (int64_t)sl.s * sl.h;
      const float* masters[3] = {sl.master_gate, sl.master_up, sl.master_down};
      for (int p = 0; p < 3; ++p) {
        if (!masters[p] || !(proj_mask & (1 << p))) continue;
        GLT_CHECK(nseg < kClipBlocks, GLT_ERR_UNSUPPORTED,
                  "glt_adamw_graft_step: the clip covers at most %d projections (slice %d)", kClipBlocks, j);
        gs[nseg] = grads[j] + p * sh;
        ns[nseg] = sh;
        ++nseg;
      }
    }
    if (nseg > 0) {
      glt_status s = launch_clip(gs, ns, nseg, clip_ws, clip_ws_floats, &ci.np, st);
      if (s != GLT_OK) return s;
      ci.partial = clip_ws;
    }
  }
  const float b1c = 1.0f / (1.0f - powf(beta1, (float)(step + 1)));
  const float b2c = 1.0f / (1.0f - powf(beta2, (float)(step + 1)));
  // projections with whole 64 x 64 tiles and a packed mirror: fused
  // launches of up to kMaxPackJobs projections; the others one flat update
  // and a repack each
  PackJobs jobs{};
  int tiles = 0;
  auto flush = [&]() -> glt_status {
    if (jobs.n == 0) return GLT_OK;
    GLT_LAUNCH("adamw_pack", adamw_pack_kernel, dim3((unsigned)tiles), dim3(256), 0, st, jobs, lr, beta1, beta2, b1c,
               b2c, eps, weight_decay, ci);
    GLT_LAUNCH_CHECK("adamw_pack");
    jobs.n = 0;
    tiles = 0;
    return GLT_OK;
  };
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
        const int64_t t = sh / 4096;
        GLT_CHECK(t < (1ll << 31), GLT_ERR_SHAPE, "glt_adamw_graft_step: %lld tiles in one projection", (long long)t);
        if (jobs.n == kMaxPackJobs || tiles + t >= (1ll << 31)) {
          glt_status s = flush();
          if (s != GLT_OK) return s;
        }
        uint16_t* rm = pk + 2 * p * sh;
        jobs.j[jobs.n++] = PackJob{w, gp, mp, vp, rm, rm + sh, pk + packed_shuf_offset(sl.s, sl.h, 2 * p),
                                   pk + packed_shuf_offset(sl.s, sl.h, 2 * p + 1), sl.s, sl.h, tiles};
        tiles += (int)t;
        continue;
      }
      GLT_LAUNCH("adamw", adamw_kernel, dim3(grid_n(sh)), dim3(256), 0, st, w, gp, mp, vp, (uint16_t*)nullptr, sh,
                 lr, beta1, beta2, b1c, b2c, eps, weight_decay, ci);
      GLT_LAUNCH_CHECK("adamw_graft");
      if (pk) {
        glt_status s = pack_projection(w, sl.s, sl.h, p, pk, st);
        if (s != GLT_OK) return s;
      }
    }
  }
  return flush();
}
}  // namespace glt

glt_status glt_adamw_graft_step(const glt_graft_slice* slices, int32_t n_slices, float* const* grads,
                                float* const* m, float* const* v, uint16_t* const* packed_out,
                                int32_t proj_mask, int32_t step, float lr, float beta1, float beta2,
                                float eps, float weight_decay, float clip_norm, void* ws, size_t ws_bytes,
                                void* stream) {
  GLT_CHECK(clip_norm <= 0.f || (ws && ws_bytes >= glt_adamw_workspace_size(0)), GLT_ERR_WORKSPACE,
            "glt_adamw_graft_step: clip needs %zu workspace bytes", glt_adamw_workspace_size(0));
  return graft_step(slices, n_slices, grads, m, v, packed_out, proj_mask, step, lr, beta1, beta2, eps, weight_decay,
                    clip_norm, static_cast<float*>(ws), ws_bytes / sizeof(float), as_stream(stream));
}

}  // extern "C"

// ------------------------------------------------- the allocation-free step
// glt_adamw_graft_step_noalloc keeps its clip partials in `scratch`, a
// file-scope device array of kClipBlocks floats (2 KB) that every GPU the
// library runs on holds until the process ends. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol):
// the device address of each GPU's copy is looked up once per device with
// that device current and kept in g_scratch_ptr.
namespace glt {
static __device__ __align__(256) float scratch[kClipBlocks];
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[64] = {};  // per device, guarded by g_scratch_mu

static glt_status scratch_ptr(float** out) {
  int dev = 0;
  GLT_TRY_HIP(hipGetDevice(&dev));
  GLT_CHECK(dev >= 0 && dev < 64, GLT_ERR_HIP, "glt_adamw_graft_step_noalloc: device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    GLT_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    GLT_CHECK(p, GLT_ERR_HIP, "glt_adamw_graft_step_noalloc: no device address for the clip scratch");
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return GLT_OK;
}
}  // namespace glt

extern "C" {

glt_status glt_adamw_graft_step_noalloc(const glt_graft_slice* slices, int32_t n_slices, float* const* grads,
                                        float* const* m, float* const* v, uint16_t* const* packed_out,
                                        int32_t proj_mask, int32_t step, float lr, float beta1, float beta2,
                                        float eps, float weight_decay, float clip_norm, void* stream) {
  float* ws = nullptr;
  if (clip_norm > 0.f) {
    const glt_status s = scratch_ptr(&ws);
    if (s != GLT_OK) return s;
  }
  // every partial the clip reads is written by the same call's sumsq launch,
  // so the scratch needs no clearing
  return graft_step(slices, n_slices, grads, m, v, packed_out, proj_mask, step, lr, beta1, beta2, eps, weight_decay,
                    clip_norm, ws, ws ? (size_t)kClipBlocks : 0, as_stream(stream));
}

}  // extern "C"
