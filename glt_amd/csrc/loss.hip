// Training-step neighbours of the grafted layers:
//   * masked cross-entropy over the shifted logits and its gradient
//     (reference grafting.hip:1027-1050 loss, :1122-1135 grad_logits);
//   * the OOD silence terms: per-token delta energy and the silence
//     gradient blend (src/kernels_elementwise_impl.inc:8-67, :222-275,
//     :458-560);
//   * the warmup + cosine learning-rate schedule (src/config.hpp:122-129).
//
// Masked CE. Row (b, t) of the logits, t < T-1, is scored against token
// ids[b, t+1] and counts when ood[b, t+1] == 0 (domain mask = 1 - ood).
// The reference runs these as separate ATen ops on bf16 tensors, each
// rounding its result to bf16:
//   p   = bf16(exp(x - max) / sum)                    softmax
//   g   = bf16(p - 1) at the label                    index_put_
//   g   = bf16(g * mask), bf16(g * (1/n)), bf16(g * scale)
//   ce  = -bf16(x_label - max - log(sum))             log_softmax + gather
//   loss = sum(ce * mask) * (1/n), n = max(sum(mask), 1)
// The last position of each sequence gets a zero gradient row
// (grad_logits_full). Here one workgroup of 1024 threads takes a row: for
// vocabularies up to 131072 the whole row stays in registers (64 VGPRs of
// packed bf16 per thread), so the logits are read once and the gradient
// written once; larger vocabularies re-read the row for the gradient.
// exp is exp2 of a pre-scaled argument (a few ulp in f32 before the bf16
// rounding); the row sum's order differs from ATen's block reduction.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "common.hpp"

namespace glt {

namespace {

constexpr int kCeThreads = 1024;
constexpr int kCeWaves = kCeThreads / 64;
constexpr int kCeChunks = 16;                                   // 16-byte chunks per thread (resident)
constexpr int kCeResidentV = kCeThreads * kCeChunks * 8;        // 131072
constexpr float kLog2e = 1.4426950408889634f;
// Cache policies of the resident rows' loads, gradient stores and zero rows:
// the nontemporal bit on the stores (a gradient is written once) measured
// 4.5 % faster at 4 x 4096 x 128256 with every third token excluded, on
// the loads 4 % slower.
constexpr int kCeAuxLd = 0, kCeAuxSt = 2, kCeAuxZero = 2;
constexpr uint16_t kBf16NegInf = 0xFF80u;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float rbf(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
// Block-wide max / sum over kCeWaves wavefronts; every thread gets the result.
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kCeWaves; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < kCeWaves; ++i) r += red[i];
  __syncthreads();
  return r;
}
// The same reductions for a workgroup that uses each red array once: no
// barrier after the reads (nothing writes the array again).
__device__ __forceinline__ float block_max_once(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kCeWaves; ++i) r = fmaxf(r, red[i]);
  return r;
}
__device__ __forceinline__ float block_sum_once(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < kCeWaves; ++i) r += red[i];
  return r;
}

// 8 consecutive bf16 of a row starting at element e (e % 8 == 0); lanes of
// the chunk past V read as -inf, which adds nothing to max or sum.
__device__ __forceinline__ u32x4 load_chunk(const uint16_t* x, int e, int V, bool vec) {
  if (vec && e + 8 <= V) return *reinterpret_cast<const u32x4*>(x + e);
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t lo = (e + 2 * q < V) ? x[e + 2 * q] : kBf16NegInf;
    const uint32_t hi = (e + 2 * q + 1 < V) ? x[e + 2 * q + 1] : kBf16NegInf;
    w[q] = lo | (hi << 16);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

struct CeArgs {
  const uint16_t* logits;
  int64_t ld;
  const int32_t* ids;
  const int32_t* ood;
  int B, T, V;
  float scale;
  uint16_t* grad;
  int64_t ld_grad;
  float* ce;        // [B*(T-1)] or null
  float* partial;   // [3][B*(T-1)]: ce*mask, x_label*mask, p_label*mask
  const float* stats;
  // bytes between a thread's resident chunks (kCeThreads * 16), passed at
  // run time so the compiler keeps it in the scalar offset instead of
  // folding each chunk's constant into a separate address register
  uint32_t chunk_stride;
};

// Gradient of one chunk of an unmasked row (8 elements), packed bf16:
// bf16(bf16(bf16(p) * (1/n)) * scale) with the hardware RNE conversion
// (v_cvt_pk_bf16_f32, equal to the bias-and-shift rounding for finite
// values); the label element is patched in afterwards. mask = 1 makes the
// reference's bf16(g * mask) exact, and scale == 1 its last step. p =
// exp(x - m) / s is formed as exp2(x log2(e) - c) with c = m log2(e) +
// log2(s), one fma per element (c is rounded once per row: a few ulp of p,
// the same for the whole row).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
template <bool SCALED>
__device__ __forceinline__ u32x4 grad_chunk(u32x4 c, float cexp, float inv_n, float scale) {
  const uint32_t ws[4] = {c.x, c.y, c.z, c.w};
  uint32_t out[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float p0 = __builtin_amdgcn_exp2f(fmaf(bf_lo(ws[q]), kLog2e, -cexp));
    const float p1 = __builtin_amdgcn_exp2f(fmaf(bf_hi(ws[q]), kLog2e, -cexp));
    const uint32_t pb = cvt2(p0, p1);
    uint32_t gb = cvt2(bf_lo(pb) * inv_n, bf_hi(pb) * inv_n);
    if constexpr (SCALED) gb = cvt2(bf_lo(gb) * scale, bf_hi(gb) * scale);
    out[q] = gb;
  }
  return u32x4{out[0], out[1], out[2], out[3]};
}
// Replaces element j (0..7) of a packed chunk by the bf16 bits b.
__device__ __forceinline__ u32x4 patch_chunk(u32x4 v, int j, uint32_t b) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if ((j >> 1) == q) w[q] = (j & 1) ? ((w[q] & 0xFFFFu) | (b << 16)) : ((w[q] & 0xFFFF0000u) | b);
  return u32x4{w[0], w[1], w[2], w[3]};
}
__device__ __forceinline__ void store_chunk(uint16_t* g, u32x4 v, int e, int V, bool vec) {
  if (vec && e + 8 <= V) {
    *reinterpret_cast<u32x4*>(g + e) = v;
    return;
  }
  const uint32_t out[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (e + 2 * q < V) g[e + 2 * q] = (uint16_t)(out[q] & 0xFFFFu);
    if (e + 2 * q + 1 < V) g[e + 2 * q + 1] = (uint16_t)(out[q] >> 16);
  }
}

// Running max and sum of exp(x - max) over a thread's chunks, each chunk's
// values unpacked once. The running max starts finite and low (kCeLowMax =
// -2^126, not -inf): a first chunk then rescales a zero sum by exp2 of a
// large negative number (0), and -inf logits (the generic path's padding)
// add exp2(-inf) = 0, with no per-chunk test for either.
constexpr float kCeLowMax = -8.5070592e37f;  // -2^126: times log2(e) stays finite
__device__ __forceinline__ void ce_fold(float& mt, float& st, u32x4 v) {
  const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
  float xs[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    xs[2 * q] = bf_lo(ws[q]);
    xs[2 * q + 1] = bf_hi(ws[q]);
  }
  float mc = xs[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mc = fmaxf(mc, xs[e]);
  const float mn = fmaxf(mt, mc);
  const float mn2 = mn * kLog2e;
  float sc = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) sc += __builtin_amdgcn_exp2f(fmaf(xs[e], kLog2e, -mn2));
  st = st * __builtin_amdgcn_exp2f(fmaf(mt, kLog2e, -mn2)) + sc;
  mt = mn;
}

// One scored row's reference terms once its max m (m2 = m log2 e) and sum s
// are known: thread 0 writes ce, and the ce / target-logit / target-
// probability partials; every thread gets the label's gradient element in
// full: bf16(p) - 1, * mask, * (1/n), * scale, each rounded.
struct CeRowTerms {
  float m2, inv_s, inv_n, cexp;  // cexp = m log2(e) + log2(s)
  uint32_t gl;
};
__device__ __forceinline__ CeRowTerms ce_row_terms(const CeArgs& a, int r, bool valid_label, float x_label,
                                                    float mask, float m, float s, float n) {
  CeRowTerms o;
  o.m2 = m * kLog2e;
  o.inv_s = 1.0f / s;
  o.inv_n = 1.0f / n;
  o.cexp = o.m2 + log2f(s);
  if (threadIdx.x == 0) {
    float ce_v = NAN, xl = NAN, pl = NAN;
    if (valid_label) {
      xl = x_label;
      ce_v = -rbf((xl - m) - logf(s));
      pl = rbf(__builtin_amdgcn_exp2f(fmaf(xl, kLog2e, -o.m2)) * o.inv_s);
    }
    if (a.ce) a.ce[r] = ce_v;
    const int R = a.B * (a.T - 1);
    a.partial[r] = ce_v * mask;
    a.partial[R + r] = xl * mask;
    a.partial[2 * R + r] = pl * mask;
  }
  o.gl = 0;
  if (valid_label) {
    float v = rbf(__builtin_amdgcn_exp2f(fmaf(x_label, kLog2e, -o.m2)) * o.inv_s);
    v = rbf(v - 1.0f);
    v = rbf(v * mask);
    v = rbf(v * o.inv_n);
    o.gl = f32_to_bf16(v * a.scale);
  }
  return o;
}

// Generic rows (V past the resident size, or unaligned rows): one workgroup
// per row, the row read twice (max and sum, then the gradient).
__global__ void __launch_bounds__(kCeThreads) masked_ce_kernel(const CeArgs a) {
  __shared__ float red[kCeWaves];
  const int row = blockIdx.x;
  const int b = row / a.T, t = row - b * a.T;
  const int tid = threadIdx.x;
  uint16_t* g = a.grad ? a.grad + (int64_t)row * a.ld_grad : nullptr;
  const bool gvec = a.grad && (a.ld_grad % 8 == 0) && ((reinterpret_cast<uintptr_t>(a.grad) & 15) == 0);
  if (t == a.T - 1) {  // no next token: zero gradient row
    if (g)
      for (int e = tid; e < a.V; e += kCeThreads) g[e] = 0;
    return;
  }
  const int r = b * (a.T - 1) + t;  // shifted-row index
  const uint16_t* x = a.logits + (int64_t)row * a.ld;
  const bool vec = (a.ld % 8 == 0) && ((reinterpret_cast<uintptr_t>(a.logits) & 15) == 0);
  const int label = a.ids[(int64_t)b * a.T + t + 1];
  const bool valid_label = label >= 0 && label < a.V;
  const float x_label = valid_label ? bf16_to_f32(x[label]) : 0.f;
  const float mask = (a.ood && a.ood[(int64_t)b * a.T + t + 1] != 0) ? 0.f : 1.f;
  const int nchunks = (a.V + 7) / 8;
  float mt = kCeLowMax, st = 0.f;
  for (int ci = tid; ci < nchunks; ci += kCeThreads) ce_fold(mt, st, load_chunk(x, ci * 8, a.V, vec));
  const float m = block_max(mt, red);
  const float s = block_sum(st * __builtin_amdgcn_exp2f(fmaf(mt, kLog2e, -m * kLog2e)), red);
  const CeRowTerms w = ce_row_terms(a, r, valid_label, x_label, mask, m, s, a.stats[3]);
  if (!g) return;
  // an excluded row (mask 0) is +0 everywhere but at the label
  const bool masked = mask == 0.f;
  const int lab_chunk = valid_label ? label >> 3 : -1;
  for (int ci = tid; ci < nchunks; ci += kCeThreads) {
    const u32x4 xc = load_chunk(x, ci * 8, a.V, vec);
    u32x4 o = masked ? u32x4{0u, 0u, 0u, 0u}
                     : a.scale == 1.0f ? grad_chunk<false>(xc, w.cexp, w.inv_n, a.scale)
                                       : grad_chunk<true>(xc, w.cexp, w.inv_n, a.scale);
    if (ci == lab_chunk) o = patch_chunk(o, label & 7, w.gl);
    store_chunk(g, o, ci * 8, a.V, gvec);
  }
}

// Resident rows (V <= kCeResidentV, V % 8 == 0, 16-byte aligned rows): one
// workgroup per row, the row in registers (chunk k of thread tid is chunk
// tid + 1024 k of the row, 16 per thread), so the logits are read once and
// the gradient written once. Buffer accesses: one per-lane byte offset, the
// chunk index in the scalar offset of the loads (no per-chunk address
// registers). LD and ST are the cache policies of the row's loads and the
// gradient's stores, Z that of the stores of a zero row (a row without a
// next token, or an excluded one: its gradient is 0 but at the label).
template <int LD, int ST, int Z>
__global__ void __launch_bounds__(kCeThreads) masked_ce_row_kernel(const CeArgs a) {
  __shared__ float red_m[kCeWaves], red_s[kCeWaves];
  __shared__ float xl_sh;
  const int row = blockIdx.x;
  const int b = row / a.T, t = row - b * a.T;
  const int tid = threadIdx.x;
  const uint32_t vo = (uint32_t)tid * 16;
  uint16_t* g = a.grad ? a.grad + (int64_t)row * a.ld_grad : nullptr;
  if (t == a.T - 1) {  // no next token: zero gradient row
    if (g) {
      const __amdgpu_buffer_rsrc_t rg = make_rsrc(g, (uint32_t)a.V * 2);
#pragma unroll
      for (int k = 0; k < kCeChunks; ++k)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rg, vo + k * a.chunk_stride, 0, Z);
    }
    return;
  }
  // The row's loads go first: nothing they address depends on the row's
  // label, mask or token count, whose loads are issued behind them.
  const uint16_t* x = a.logits + (int64_t)row * a.ld;
  const int nchunks = a.V >> 3;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)a.V * 2);
  u32x4 c[kCeChunks];
  // issued in chunk order (the scheduler otherwise moves chunk 0, whose
  // scalar offset is the constant 0, behind the others, and the first fold
  // then waits for nearly the whole row)
#pragma unroll
  for (int k = 0; k < kCeChunks; ++k) {
    c[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, vo, k * a.chunk_stride, LD));
    __builtin_amdgcn_sched_barrier(0);
  }
  const int label = a.ids[(int64_t)b * a.T + t + 1];
  const float mask = (a.ood && a.ood[(int64_t)b * a.T + t + 1] != 0) ? 0.f : 1.f;
  const float n_scored = a.stats[3];
  const bool valid_label = label >= 0 && label < a.V;
  // which of the resident chunks holds the label is the same for every
  // thread (lab_k); one thread holds it
  const int lab_chunk = valid_label ? label >> 3 : -1;
  const int lab_k = valid_label ? lab_chunk / kCeThreads : -1;
  const bool lab_mine = valid_label && lab_chunk % kCeThreads == tid;
  float mt = kCeLowMax, st = 0.f;
#pragma unroll
  for (int k = 0; k < kCeChunks; ++k) {
    // chunks past the row (zeros from beyond the descriptor's extent) are skipped
    if (tid + k * kCeThreads < nchunks) ce_fold(mt, st, c[k]);
    // the gradient pass unpacks the chunk again rather than keeping
    // these values alive (128 more registers)
    asm volatile("" : "+v"(c[k]));
  }
  // the label's logit comes from the resident chunk that holds it, through
  // LDS (published by the max reduction's barrier)
  if (lab_mine) {
    u32x4 lc = c[0];
#pragma unroll
    for (int k = 1; k < kCeChunks; ++k)
      if (k == lab_k) lc = c[k];
    const uint32_t wsel[4] = {lc.x, lc.y, lc.z, lc.w};
    uint32_t wl = wsel[0];
#pragma unroll
    for (int q = 1; q < 4; ++q)
      if (q == ((label & 7) >> 1)) wl = wsel[q];
    xl_sh = (label & 1) ? bf_hi(wl) : bf_lo(wl);
  }
  const float m = block_max_once(mt, red_m);
  const float x_label = valid_label ? xl_sh : 0.f;
  const float s = block_sum_once(st * __builtin_amdgcn_exp2f(fmaf(mt, kLog2e, -m * kLog2e)), red_s);
  const CeRowTerms w = ce_row_terms(a, b * (a.T - 1) + t, valid_label, x_label, mask, m, s, n_scored);
  if (!g) return;
  const __amdgpu_buffer_rsrc_t rg = make_rsrc(g, (uint32_t)a.V * 2);
  // one loop per case (the case is the same for the whole row); an
  // excluded row (mask 0) is +0 everywhere but at the label
  auto stores = [&](auto chunk_of, auto policy) {
#pragma unroll
    for (int k = 0; k < kCeChunks; ++k) {
      u32x4 o = chunk_of(c[k]);
      if (k == lab_k && lab_mine) o = patch_chunk(o, label & 7, w.gl);
      // stores past the row fall outside the descriptor and are dropped.
      // The chunk offset rides in the per-lane offset, not the scalar one:
      // a 16-byte store needs wait states before its data registers are
      // rewritten, and the compiler leaves them out for buffer stores with
      // a register scalar offset (which on gfx950 then store the next
      // chunk's values).
      __builtin_amdgcn_raw_buffer_store_b128(o, rg, vo + k * a.chunk_stride, 0, decltype(policy)::value);
    }
  };
  using zero_policy = std::integral_constant<int, Z>;
  using grad_policy = std::integral_constant<int, ST>;
  if (mask == 0.f) stores([](u32x4) { return u32x4{0u, 0u, 0u, 0u}; }, zero_policy{});
  else if (a.scale == 1.0f)
    stores([&](u32x4 v) { return grad_chunk<false>(v, w.cexp, w.inv_n, a.scale); }, grad_policy{});
  else stores([&](u32x4 v) { return grad_chunk<true>(v, w.cexp, w.inv_n, a.scale); }, grad_policy{});
}

// n = max(sum over scored rows of (1 - ood[b, t+1]), 1) into stats[3].
__global__ void __launch_bounds__(1024) ce_count_kernel(const int32_t* ood, int B, int T, float* stats) {
  __shared__ float red[kCeWaves];
  const int R = T > 1 ? B * (T - 1) : 0;
  float c = 0.f;
  for (int r = threadIdx.x; r < R; r += blockDim.x) {
    const int b = r / (T - 1), t = r - b * (T - 1);
    c += (ood && ood[(int64_t)b * T + t + 1] != 0) ? 0.f : 1.f;
  }
  const float n = block_sum(c, red);
  if (threadIdx.x == 0) stats[3] = n < 1.0f ? 1.0f : n;
}

// loss, target-logit mean, target-probability mean from the row partials.
__global__ void __launch_bounds__(1024) ce_finalize_kernel(const float* partial, int R, float* stats) {
  __shared__ float red[kCeWaves];
  float acc[3] = {0.f, 0.f, 0.f};
  for (int r = threadIdx.x; r < R; r += blockDim.x)
#pragma unroll
    for (int j = 0; j < 3; ++j) acc[j] += partial[(int64_t)j * R + r];
  const float inv_n = 1.0f / stats[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const float v = block_sum(acc[j], red);
    if (threadIdx.x == 0) stats[j] = v * inv_n;
  }
}

// ---------------------------------------------------------------- silence
// One workgroup of 256 per token row of `slice` values (f32 or bf16 at row
// stride ld). Sum of squares in f32.
constexpr int kSilThreads = 256;

template <typename T>
__device__ __forceinline__ float ldv(const T* p, int64_t i) {
  if constexpr (sizeof(T) == 4) return p[i];
  else return bf16_to_f32(p[i]);
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  const float r = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return r;
}

// energy[t] = sqrt(sum d^2 + 1e-8) / sqrt(slice) (compute_energy_kernel)
template <typename T>
__global__ void __launch_bounds__(kSilThreads) energy_kernel(const T* d, int64_t ld, int slice, float* energy) {
  __shared__ float red[4];
  const T* row = d + (int64_t)blockIdx.x * ld;
  float s = 0.f;
  for (int i = threadIdx.x; i < slice; i += kSilThreads) {
    const float v = ldv(row, i);
    s += v * v;
  }
  const float tot = block_sum256(s, red);
  if (threadIdx.x == 0) energy[blockIdx.x] = sqrtf(tot + 1e-8f) * (1.0f / sqrtf((float)slice));
}

// For OOD tokens: dy += lambda / (||d|| sqrt(slice)) * d, ||d|| = sqrt(sum d^2
// + 1e-8) (silence_blend_kernel).
__global__ void __launch_bounds__(kSilThreads) silence_blend_kernel(float* dy, const float* d, const int32_t* ood,
                                                                    int slice, float lambda) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  if (ood[t] == 0) return;
  const float* row = d + (int64_t)t * slice;
  float s = 0.f;
  for (int i = threadIdx.x; i < slice; i += kSilThreads) s += row[i] * row[i];
  const float tot = block_sum256(s, red);
  const float norm = sqrtf(tot + 1e-8f);
  const float scale = lambda / (norm * sqrtf((float)slice));
  float* out = dy + (int64_t)t * slice;
  for (int i = threadIdx.x; i < slice; i += kSilThreads) out[i] += scale * row[i];
}

// Gate and up together (fused_silence_blend_energy_kernel): energies of both
// (written when the pointers are non-null), then for OOD tokens
// dy += lambda / (energy * slice + 1e-8) * d, the reference's
// norm = energy * sqrt(slice), scale = lambda / (norm * sqrt(slice) + 1e-8).
__global__ void __launch_bounds__(kSilThreads) silence_blend_energy_kernel(float* dy_g, const float* d_g, float* dy_u,
                                                                           const float* d_u, float* e_g, float* e_u,
                                                                           const int32_t* ood, int slice,
                                                                           float lambda) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const int64_t off = (int64_t)t * slice;
  float sg = 0.f, su = 0.f;
  for (int i = threadIdx.x; i < slice; i += kSilThreads) {
    sg += d_g[off + i] * d_g[off + i];
    su += d_u[off + i] * d_u[off + i];
  }
  const float tg = block_sum256(sg, red);
  const float tu = block_sum256(su, red);
  const float rs = sqrtf((float)slice);
  const float eg = sqrtf(tg + 1e-8f) * (1.0f / rs);
  const float eu = sqrtf(tu + 1e-8f) * (1.0f / rs);
  if (threadIdx.x == 0) {
    if (e_g) e_g[t] = eg;
    if (e_u) e_u[t] = eu;
  }
  if (ood[t] != 1) return;
  const float scale_g = lambda / (eg * rs * rs + 1e-8f);
  const float scale_u = lambda / (eu * rs * rs + 1e-8f);
  for (int i = threadIdx.x; i < slice; i += kSilThreads) {
    dy_g[off + i] += scale_g * d_g[off + i];
    dy_u[off + i] += scale_u * d_u[off + i];
  }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

}  // namespace glt

using namespace glt;

extern "C" {

size_t glt_masked_ce_workspace_size(int32_t B, int32_t T) {
  if (B <= 0 || T <= 1) return 256;
  return align256((size_t)3 * B * (T - 1) * sizeof(float));
}

glt_status glt_masked_ce(const uint16_t* logits, int64_t ld, const int32_t* ids, const int32_t* ood, int32_t B,
                         int32_t T, int32_t V, float scale, uint16_t* grad, int64_t ld_grad, float* ce_per_token,
                         float* stats, void* workspace, size_t workspace_bytes, void* stream) {
  GLT_CHECK(B >= 0 && T >= 0 && V > 0, GLT_ERR_SHAPE, "glt_masked_ce: B=%d T=%d V=%d", B, T, V);
  GLT_CHECK(ld >= V && (!grad || ld_grad >= V), GLT_ERR_SHAPE, "glt_masked_ce: row strides must be >= V");
  GLT_CHECK(stats, GLT_ERR_INVALID_ARG, "glt_masked_ce: null stats");
  hipStream_t st = as_stream(stream);
  const int R = (T > 1) ? B * (T - 1) : 0;
  if (B > 0 && T > 0) GLT_CHECK(logits && ids, GLT_ERR_INVALID_ARG, "glt_masked_ce: null logits/ids");
  GLT_CHECK(workspace && workspace_bytes >= glt_masked_ce_workspace_size(B, T) &&
                (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
            GLT_ERR_WORKSPACE, "glt_masked_ce: needs %zu workspace bytes, 256-byte aligned",
            glt_masked_ce_workspace_size(B, T));
  // n first (the gradient scales by 1/n), then the rows, then the means.
  // Without scored rows (T <= 1) n is 1 and loss and means are 0; every
  // row is a last position and gets a zero gradient.
  GLT_LAUNCH("ce_count", ce_count_kernel, dim3(1), dim3(1024), 0, st, ood, B, T, stats);
  GLT_LAUNCH_CHECK("ce_count");
  if ((int64_t)B * T > 0) {
    CeArgs a{logits, ld,     ids, ood,   B, T, V, scale, grad, ld_grad, ce_per_token, static_cast<float*>(workspace),
             stats,  kCeThreads * 16};
    const int64_t rows = (int64_t)B * T;
    const bool aligned = V % 8 == 0 && ld % 8 == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0 &&
                         (!grad || (ld_grad % 8 == 0 && (reinterpret_cast<uintptr_t>(grad) & 15) == 0));
    if (V <= kCeResidentV && aligned) {
      GLT_LAUNCH("masked_ce", (masked_ce_row_kernel<kCeAuxLd, kCeAuxSt, kCeAuxZero>), dim3((unsigned)rows), dim3(kCeThreads), 0, st, a);
    } else {
      GLT_LAUNCH("masked_ce", masked_ce_kernel, dim3((unsigned)rows), dim3(kCeThreads), 0, st, a);
    }
    GLT_LAUNCH_CHECK("masked_ce");
  }
  GLT_LAUNCH("ce_finalize", ce_finalize_kernel, dim3(1), dim3(1024), 0, st, static_cast<const float*>(workspace), R,
             stats);
  GLT_LAUNCH_CHECK("ce_finalize");
  return GLT_OK;
}

glt_status glt_silence_energy(const void* delta, int32_t dtype, int64_t ld, int32_t tokens, int32_t slice,
                              float* energy, void* stream) {
  GLT_CHECK(tokens >= 0 && slice > 0 && ld >= slice, GLT_ERR_SHAPE, "glt_silence_energy: tokens=%d slice=%d ld=%lld",
            tokens, slice, (long long)ld);
  GLT_CHECK(dtype == GLT_DTYPE_F32 || dtype == GLT_DTYPE_BF16, GLT_ERR_DTYPE, "glt_silence_energy: dtype %d", dtype);
  if (tokens == 0) return GLT_OK;
  GLT_CHECK(delta && energy, GLT_ERR_INVALID_ARG, "glt_silence_energy: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == GLT_DTYPE_F32) {
    GLT_LAUNCH("silence_energy", energy_kernel<float>, dim3(tokens), dim3(kSilThreads), 0, st,
               static_cast<const float*>(delta), ld, slice, energy);
  } else {
    GLT_LAUNCH("silence_energy", energy_kernel<uint16_t>, dim3(tokens), dim3(kSilThreads), 0, st,
               static_cast<const uint16_t*>(delta), ld, slice, energy);
  }
  GLT_LAUNCH_CHECK("silence_energy");
  return GLT_OK;
}

glt_status glt_silence_blend(float* dy, const float* delta, const int32_t* ood, int32_t tokens, int32_t slice,
                             float lambda, void* stream) {
  GLT_CHECK(tokens >= 0 && slice > 0, GLT_ERR_SHAPE, "glt_silence_blend: tokens=%d slice=%d", tokens, slice);
  if (tokens == 0) return GLT_OK;
  GLT_CHECK(dy && delta && ood, GLT_ERR_INVALID_ARG, "glt_silence_blend: null pointer");
  GLT_LAUNCH("silence_blend", silence_blend_kernel, dim3(tokens), dim3(kSilThreads), 0, as_stream(stream), dy, delta,
             ood, slice, lambda);
  GLT_LAUNCH_CHECK("silence_blend");
  return GLT_OK;
}

glt_status glt_silence_blend_energy(float* dy_gate, const float* delta_gate, float* dy_up, const float* delta_up,
                                    float* energy_gate, float* energy_up, const int32_t* ood, int32_t tokens,
                                    int32_t slice, float lambda, void* stream) {
  GLT_CHECK(tokens >= 0 && slice > 0, GLT_ERR_SHAPE, "glt_silence_blend_energy: tokens=%d slice=%d", tokens, slice);
  if (tokens == 0) return GLT_OK;
  GLT_CHECK(dy_gate && delta_gate && dy_up && delta_up && ood, GLT_ERR_INVALID_ARG,
            "glt_silence_blend_energy: null pointer");
  GLT_LAUNCH("silence_blend_energy", silence_blend_energy_kernel, dim3(tokens), dim3(kSilThreads), 0,
             as_stream(stream), dy_gate, delta_gate, dy_up, delta_up, energy_gate, energy_up, ood, slice, lambda);
  GLT_LAUNCH_CHECK("silence_blend_energy");
  return GLT_OK;
}

float glt_lr_schedule(int32_t step, int32_t total_steps, int32_t warmup_steps, float lr_peak) {
  if (step < warmup_steps) return lr_peak * (step + 1) / warmup_steps;
  const float denominator = (float)(total_steps - warmup_steps);
  const float progress = (float)(step - warmup_steps) / fmaxf(denominator, 1.0f);
  return lr_peak * (1.0f + cosf(M_PI * progress)) * 0.5f;
}

}  // extern "C"
