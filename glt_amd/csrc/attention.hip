// Causal GQA attention forward for gfx950 (the base attention of the
// decoder layer, reference forward_layer src/layer_forward_impl.inc:25-56:
// q/k/v split into heads, k/v repeated to the query heads with
// repeat_interleave, at::scaled_dot_product_attention(q, k, v, {}, 0.0,
// is_causal=true), heads merged back).
//
// Layouts: q [B, T, Hq, 128], k/v [B, T, Hkv, 128], out [B, T, Hq, 128],
// bf16, row-major; query head h reads kv head h / (Hq / Hkv).
//
// One workgroup per (batch, query head, 128-row query block); wavefront w
// owns query rows q0 + 32w .. +31 and walks the key tiles (64 keys) up to its
// causal limit. Both products are computed transposed so that a lane always
// holds ONE query (the MFMA output column):
//   S^T[key][q] = K . Q^T   (A = K fragment from LDS, B = Q fragment in VGPRs)
//   O^T[d][q]  += V^T . P^T (A = V^T fragment from LDS, B = P^T in VGPRs)
// so the online-softmax statistics of a query live in the lane pair
// (l, l^32) and the rescale of O is one multiply per accumulator. The P^T
// operand of a 16-key step takes four of the lane's probabilities and four
// of its partner's (one v_permlane32_swap per register).
//
// LDS per stage: the K tile as [64 keys][128 d] (direct-to-LDS loads, 16-byte
// chunk c of row r at c ^ (r & 15)) and the V^T tile as [128 d][64 keys]
// (V transposed through VGPRs, 8-byte writes; row R stored at R ^ ((R >> 3)
// & 1) and chunk c at c ^ ((R' >> 1) & 7)). Both the fragment reads and the
// transposing writes are free of bank conflicts. Two stages, the next key
// tile is loaded while the current one is consumed.
#include <atomic>
#include "common.hpp"

namespace glt {

namespace {

constexpr int kHd = 128;          // head dimension
constexpr int kQBlock = 128;      // query rows per workgroup
constexpr int kKvTile = 64;       // keys per step
constexpr int kKBytes = kKvTile * kHd * 2;   // 16 KB
constexpr int kStageBytes = 2 * kKBytes;     // K + V^T
constexpr int kAttnLds = 2 * kStageBytes;    // 64 KB
constexpr float kMaskVal = -1.0e30f;         // finite: no inf - inf
constexpr float kSlack = 8.0f;               // running-max slack (log2 units)
constexpr int kKPrefetch = 4;                // K fragments read ahead of their MFMA
constexpr uint32_t kExtentA = 0x7FFFFFF0u;   // buffer extent below kOob

typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));

// two floats to packed bf16, round to nearest even (hardware conversion)
__device__ __forceinline__ uint32_t pack2_rne(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// v_permlane32_swap(a, b) returns r0 = [a of lanes 0-31 | b of lanes 0-31]
// and r1 = [a of lanes 32-63 | b of lanes 32-63] (lanes 0-31 | 32-63).
// For a value held per lane, r0/r1 of swap(x, x) are the values of the two
// lanes of the pair (l, l^32), in every lane.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ uint32_t vt_off(int R, int c, int half) {
  const int pr = R ^ ((R >> 3) & 1);
  return (uint32_t)(pr * 128 + ((c ^ ((pr >> 1) & 7)) << 4) + (half << 3));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t uni_rsrc_a(const void* p, uint32_t n) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(n));
}

__global__ void __launch_bounds__(256, 2)
attn_fwd_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                uint16_t* __restrict__ out, int B, int T, int Hq, int Hkv, float scale_log2, int causal) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Block order: query blocks longest-first; within a rank, (batch, head)
  // with the kv head fastest. Workgroups are dealt round-robin over the 8
  // XCDs, so one XCD's workgroups share kv heads (and their K/V in its L2).
  const int nqb = (T + kQBlock - 1) / kQBlock;
  const int rep = Hq / Hkv, nhb = Hq * B;
  const int id = blockIdx.x;
  const int qb = nqb - 1 - id / nhb;
  const int hb = id % nhb;
  const int g = hb % Hkv, h = g * rep + (hb / Hkv) % rep, b = hb / Hq;
  const int q0 = qb * kQBlock;
  const int wq0 = q0 + 32 * wave;                    // this wavefront's first query
  const int lq = lane & 31, lh = lane >> 5;
  const int myq = wq0 + lq;                          // this lane's query

  // key tiles: the workgroup loads up to its last row's limit, each
  // wavefront computes up to its own
  const int kv_end = causal ? min(T, q0 + kQBlock) : T;
  const int ntiles = (kv_end + kKvTile - 1) / kKvTile;
  const int w_end = causal ? min(T, wq0 + 32) : T;
  const int w_tiles = wq0 < T ? (w_end + kKvTile - 1) / kKvTile : 0;

  const int64_t q_ld = (int64_t)Hq * kHd, kv_ld = (int64_t)Hkv * kHd;

  // ---- Q fragments (B operand of S^T): lane holds query lq, d = 16s + 8lh .. +7
  bf16x8 qf[8];
  {
    const uint16_t* qp = q + ((int64_t)b * T + min(myq, T - 1)) * q_ld + (int64_t)h * kHd + 8 * lh;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const u32x4 x = myq < T ? *reinterpret_cast<const u32x4*>(qp + 16 * s) : u32x4{0, 0, 0, 0};
      qf[s] = __builtin_bit_cast(bf16x8, x);
    }
  }

  // ---- K tile loads: 16 direct-to-LDS loads of 1 KB per tile, four per
  // wavefront; instruction i of wave w fills rows 4(4i+w) .. +3, lane L
  // takes row +L/16 and physical chunk L&15 = logical chunk ^ (row & 15).
  const __amdgpu_buffer_rsrc_t rk = uni_rsrc_a(k, kExtentA);
  uint32_t kvo[4];
  int krow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    krow[i] = 4 * (4 * i + wave) + (lane >> 4);
    const int c = (lane & 15) ^ (krow[i] & 15);
    kvo[i] = (uint32_t)((((int64_t)b * T) * kv_ld + (int64_t)g * kHd + 8 * c) * 2);
  }
  auto load_k = [&](int tile, int stage) {
    char* dst = smem + stage * kStageBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = tile * kKvTile + krow[i];
      const uint32_t off = key < T ? kvo[i] + (uint32_t)((int64_t)key * kv_ld * 2) : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(dst + (4 * i + wave) * 1024), 16, off, 0, 0, 0);
    }
  };
  // ---- V tile: thread t loads keys 4(t & 15) .. +3 of d chunk t >> 4 (8 d)
  // and writes the transposed 8 x 4 block as eight 8-byte rows of V^T.
  const int vkg = tid & 15, vdc = tid >> 4;
  u32x4 vr[4];
  auto load_v = [&](int tile) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = tile * kKvTile + 4 * vkg + e;
      vr[e] = key < T ? *reinterpret_cast<const u32x4*>(v + ((int64_t)b * T + key) * kv_ld + (int64_t)g * kHd + 8 * vdc)
                      : u32x4{0, 0, 0, 0};
    }
  };
  // V^T write offsets of this thread's eight rows (the same every tile)
  uint32_t vto[8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    vto[2 * p] = vt_off(8 * vdc + 2 * p, vkg >> 1, vkg & 1);
    vto[2 * p + 1] = vt_off(8 * vdc + 2 * p + 1, vkg >> 1, vkg & 1);
  }
  auto store_vt = [&](int stage) {
    char* dst = smem + stage * kStageBytes + kKBytes;
    const uint32_t w0[4] = {vr[0].x, vr[1].x, vr[2].x, vr[3].x};
    const uint32_t w1[4] = {vr[0].y, vr[1].y, vr[2].y, vr[3].y};
    const uint32_t w2[4] = {vr[0].z, vr[1].z, vr[2].z, vr[3].z};
    const uint32_t w3[4] = {vr[0].w, vr[1].w, vr[2].w, vr[3].w};
    const uint32_t* wd[4] = {w0, w1, w2, w3};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // d = 8*vdc + 2p (low halves) and +1 (high halves) of keys 4vkg..+3
      const uint32_t* x = wd[p];
      const uint32_t lo01 = (x[0] & 0xFFFFu) | (x[1] << 16), lo23 = (x[2] & 0xFFFFu) | (x[3] << 16);
      const uint32_t hi01 = (x[0] >> 16) | (x[1] & 0xFFFF0000u), hi23 = (x[2] >> 16) | (x[3] & 0xFFFF0000u);
      *reinterpret_cast<u32x2a*>(dst + vto[2 * p]) = u32x2a{lo01, lo23};
      *reinterpret_cast<u32x2a*>(dst + vto[2 * p + 1]) = u32x2a{hi01, hi23};
    }
  };

  // ---- state
  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};
  float m_run = kMaskVal, l_run = 0.f;

  if (ntiles > 0) {
    load_k(0, 0);
    load_v(0);
  }
  for (int t = 0; t < ntiles; ++t) {
    const int st = t & 1;
    // V^T of tile t into its stage; K of tile t has been issued
    store_vt(st);
    // this thread's K loads of tile t and V^T writes are done
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // tile t+1 in flight while tile t is consumed
    if (t + 1 < ntiles) {
      load_k(t + 1, st ^ 1);
      load_v(t + 1);
    }
    if (t < w_tiles) {
      const char* kt = smem + st * kStageBytes;
      const char* vt = kt + kKBytes;
      // S^T blocks: keys 32kb + (8(e>>2) + 4lh + (e&3)), query lq. One
      // accumulation chain per key block (the two alternate, and an MFMA
      // accumulating onto its chain's previous result does not stall); the
      // K fragment of step i + kKPrefetch is read before the MFMA of step i,
      // which keeps the reads' LDS latency off the MFMA chain.
      f32x16 sacc[2] = {f32x16{}, f32x16{}};
      auto kread = [&](int i) {  // step i: key block i & 1, d 16(i >> 1) ..
        const int r = 32 * (i & 1) + lq, c = 2 * (i >> 1) + lh;
        return *reinterpret_cast<const bf16x8*>(kt + r * 256 + ((c ^ (r & 15)) << 4));
      };
      bf16x8 kq[kKPrefetch];
#pragma unroll
      for (int i = 0; i < kKPrefetch; ++i) kq[i] = kread(i);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const bf16x8 kf = kq[i % kKPrefetch];
        if (i + kKPrefetch < 16) kq[i % kKPrefetch] = kread(i + kKPrefetch);
        sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[i >> 1], sacc[i & 1], 0, 0, 0);
      }
      // Mask (only a tile that reaches past this wavefront's first query
      // or past T needs it): key index < lim, with lim the lane's causal /
      // sequence bound relative to this lane's first key of the tile.
      const int key0 = t * kKvTile;
      if (key0 + kKvTile > T || (causal && key0 + kKvTile - 1 > wq0)) {
        const int lim = (causal ? min(T, myq + 1) : T) - (key0 + 4 * lh);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            sacc[kb][e] = (32 * kb + 8 * (e >> 2) + (e & 3)) < lim ? sacc[kb][e] : kMaskVal;
      }
      // tile maximum of the query's 64 scores (lane pair), in exp2 units
      float mt = kMaskVal;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) mt = fmaxf(mt, sacc[kb][e]);
      mt = pair_max(mt) * scale_log2;
      // The running maximum moves only when some lane's grows by more than
      // kSlack: probabilities then stay below 2^kSlack, the same result up
      // to rounding, and O is rescaled on few tiles.
      if (__any(mt > m_run + kSlack)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] *= alpha;
      }
      float psum = 0.f;
      uint32_t pk[2][4][2];  // [kb][group][packed pair]: 4 probabilities of the group
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          float p4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            p4[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][4 * gi + e], scale_log2, -m_run));
            psum += p4[e];
          }
          pk[kb][gi][0] = pack2_rne(p4[0], p4[1]);
          pk[kb][gi][1] = pack2_rne(p4[2], p4[3]);
        }
      l_run += psum;
      // O^T += V^T . P^T over four 16-key steps: step s2 covers keys
      // 16 s2 .. +15 = groups 2(s2&1), 2(s2&1)+1 of block s2>>1. The lane
      // with lh = 0 needs keys +0..7 (its own first four, its partner's
      // next four), lh = 1 keys +8..15: swap(own g0, own g1) gives lanes
      // 0-31 their g0 keys +0..3 (r0) and the partner's +4..7 (r1), lanes
      // 32-63 the partner's g1 keys +0..3 (r0) and their own +4..7 (r1).
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        const int kb = s2 >> 1, g0 = 2 * (s2 & 1), g1 = g0 + 1;
        const auto s0 = __builtin_amdgcn_permlane32_swap(pk[kb][g0][0], pk[kb][g1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(pk[kb][g0][1], pk[kb][g1][1], false, false);
        const bf16x8 pb = __builtin_bit_cast(bf16x8, u32x4{s0[0], s1[0], s0[1], s1[1]});
#pragma unroll
        for (int hb = 0; hb < 4; ++hb) {
          const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vt + vt_off(32 * hb + lq, 2 * s2 + lh, 0));
          o[hb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb, o[hb], 0, 0, 0);
        }
      }
    }
    // no second barrier: stage st is next written after the first barrier
    // of tile t+1, which every wavefront reaches only once done with tile t
  }

  // ---- normalise and store: lane holds d = 32hb + 8(e>>2) + 4lh + (e&3)
  const float l_tot = pair_sum(l_run);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (myq < T) {
    uint16_t* op = out + ((int64_t)b * T + myq) * q_ld + (int64_t)h * kHd + 4 * lh;
#pragma unroll
    for (int hb = 0; hb < 4; ++hb)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const f32x16& a = o[hb];
        const u32x2a d = {pack2_rne(a[4 * gi] * inv, a[4 * gi + 1] * inv), pack2_rne(a[4 * gi + 2] * inv, a[4 * gi + 3] * inv)};
        *reinterpret_cast<u32x2a*>(op + 32 * hb + 8 * gi) = d;
      }
  }
}

}  // namespace

}  // namespace glt

using namespace glt;

extern "C" glt_status glt_attention_fwd(const void* q, const void* k, const void* v, void* out, int32_t B, int32_t T,
                                        int32_t Hq, int32_t Hkv, int32_t head_dim, float scale, int32_t causal,
                                        void* stream) {
  GLT_CHECK(B >= 0 && T >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, GLT_ERR_SHAPE,
            "glt_attention_fwd: B=%d T=%d Hq=%d Hkv=%d (Hq must be a multiple of Hkv)", B, T, Hq, Hkv);
  GLT_CHECK(head_dim == kHd, GLT_ERR_UNSUPPORTED, "glt_attention_fwd: head_dim %d (only %d)", head_dim, kHd);
  if (B == 0 || T == 0) return GLT_OK;
  GLT_CHECK(q && k && v && out, GLT_ERR_INVALID_ARG, "glt_attention_fwd: null pointer");
  GLT_CHECK(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16 == 0, GLT_ERR_ALIGNMENT,
            "glt_attention_fwd: tensors must be 16-byte aligned");
  // K rows are addressed through 31-bit buffer offsets
  GLT_CHECK((int64_t)B * T * Hkv * kHd * 2 < (int64_t)kOob, GLT_ERR_SHAPE, "glt_attention_fwd: K of %lld bytes",
            (long long)B * T * Hkv * kHd * 2);
  // the dynamic-LDS limit is a per-device attribute of the kernel (set
  // once per device; a concurrent first call sets the same value again)
  static std::atomic<bool> attr_set[64];
  int dev = 0;
  GLT_TRY_HIP(hipGetDevice(&dev));
  GLT_CHECK(dev >= 0 && dev < 64, GLT_ERR_HIP, "glt_attention_fwd: device index %d out of range", dev);
  if (!attr_set[dev].load(std::memory_order_acquire)) {
    GLT_TRY_HIP(hipFuncSetAttribute((const void*)attn_fwd_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kAttnLds));
    attr_set[dev].store(true, std::memory_order_release);
  }
  const float scale_log2 = scale * 1.4426950408889634f;
  // 1-D over (query block, batch, head)
  const int64_t nblk = (int64_t)((T + kQBlock - 1) / kQBlock) * Hq * B;
  GLT_CHECK(nblk < INT32_MAX, GLT_ERR_SHAPE, "glt_attention_fwd: %lld workgroups", (long long)nblk);
  dim3 grid((unsigned)nblk, 1, 1);
  GLT_LAUNCH("attention", attn_fwd_kernel, grid, dim3(256), kAttnLds, as_stream(stream),
             static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
             static_cast<uint16_t*>(out), B, T, Hq, Hkv, scale_log2, causal);
  GLT_LAUNCH_CHECK("attention");
  return GLT_OK;
}
