// Causal GQA attention forward for gfx950 (the base attention of the
// decoder layer, reference forward_layer src/layer_forward_impl.inc:25-56:
// q/k/v split into heads, k/v repeated to the query heads with
// repeat_interleave, at::scaled_dot_product_attention(q, k, v, {}, 0.0,
// is_causal=true), heads merged back).
//
// Layouts: q [B, T, Hq, 128], k/v [B, T, Hkv, 128], out [B, T, Hq, 128],
// bf16, row-major; query head h reads kv head h / (Hq / Hkv).
//
// First pass (vt_pack_kernel): V is copied transposed into the caller's
// workspace, vt [B, Hkv, 128, T rounded up to 64] (keys past T zero), so the
// attention kernel loads V^T tiles straight into LDS like K tiles.
//
// Attention (attn_fwd_kernel): one workgroup of eight wavefronts per
// (batch, query head, 256-row query block); wavefront w owns query rows
// q0 + 32w .. +31. Both products are computed transposed so that a lane
// always holds ONE query (the MFMA output column):
//   S^T[key][q] = K . Q^T   (A = K fragment from LDS, B = Q fragment in VGPRs)
//   O^T[d][q]  += V^T . P^T (A = V^T fragment from LDS, B = P^T in VGPRs)
// so the online-softmax statistics of a query live in the lane pair
// (l, l^32) and the rescale of O is one multiply per accumulator. The P^T
// operand of a 16-key step takes four of the lane's probabilities and four
// of its partner's (one v_permlane32_swap per register).
//
// Ping-pong: wavefronts 0-3 (group A) and 4-7 (group B) share the four
// SIMDs, one of each per SIMD, and alternate between an MFMA phase (S^T of
// key tile m and O^T += V^T(m-1) . P^T(m-1): 32 MFMAs) and an arithmetic
// phase (mask, maximum, exponentials and P^T of tile m, plus the group's
// direct-to-LDS loads), one group in each kind of phase at a time, with a
// workgroup barrier between phases. The exponentials of one wavefront thus
// run beside the MFMAs of its SIMD partner instead of between its own.
//
// LDS: three K slots of [64 keys][128 d] (16-byte chunk c of row r at
// c ^ (r & 15)) and two V^T slots of [128 d][64 keys] (row R stored at
// R ^ ((R >> 3) & 1), chunk c at c ^ ((R' >> 1) & 7)), 80 KB; both filled by
// direct-to-LDS loads, both read conflict-free. Group A loads K(m+2) in its
// arithmetic phase m, group B V^T(m+1) in its, each waits for its loads at
// the end of its next MFMA phase.
#include <atomic>

#include "common.hpp"

namespace glt {

namespace {

constexpr int kHd = 128;          // head dimension
constexpr int kQBlock = 256;      // query rows per workgroup (8 wavefronts of 32)
constexpr int kKvTile = 64;       // keys per tile
constexpr int kTileBytes = kKvTile * kHd * 2;    // 16 KB
constexpr int kVtBase = 3 * kTileBytes;          // three K slots, then two V^T slots
constexpr int kAttnLds = 5 * kTileBytes;         // 80 KB
constexpr float kMaskVal = -1.0e30f;         // finite: no inf - inf
constexpr float kSlack = 8.0f;               // running-max slack (log2 units)
constexpr uint32_t kExtentA = 0x7FFFFFF0u;   // buffer extent below kOob

typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// two floats to packed bf16, round to nearest even (hardware conversion)
__device__ __forceinline__ uint32_t pack2_rne(float a, float b) {
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
constexpr bf16x2_t kOnes2 = {(__bf16)1.0f, (__bf16)1.0f};

// v_permlane32_swap(a, b) returns r0 = [a of lanes 0-31 | b of lanes 0-31]
// and r1 = [a of lanes 32-63 | b of lanes 32-63] (lanes 0-31 | 32-63).
// For a value held per lane, r0/r1 of swap(x, x) are the values of the two
// lanes of the pair (l, l^32), in every lane.
// Maxima use the NaN-propagating maximum (v_maximum3_f32): fmaxf would make
// the compiler canonicalise each MFMA result first (one more instruction per
// score pair); no score is NaN.
__device__ __forceinline__ float fmax_nc(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
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

// Phase boundary: this wavefront's LDS writes are done, then s_barrier; no
// memory access or arithmetic is moved across it.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
constexpr int vmcnt_enc(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// V [B, T, Hkv, 128] -> vt [B, Hkv, 128, Tpad] (keys past T zero): one
// workgroup per (64-key tile, batch x kv head). Loads are whole 256-byte
// key rows (lane: key L/16, chunk L&15), stored to LDS with chunk c of key
// r at c ^ ((r >> 2) & 15); thread t then reads keys 4(t&15) .. +3 of d
// chunk t>>4 (conflict-free), transposes the 4 x 8 block in registers and
// stores eight 8-byte pieces of V^T rows (each store instruction covers four
// whole 128-byte rows).
__global__ void __launch_bounds__(256) vt_pack_kernel(const uint16_t* __restrict__ v, uint16_t* __restrict__ vt,
                                                      int T, int Tpad, int Hkv) {
  __shared__ __attribute__((aligned(16))) char tile[kKvTile * kHd * 2];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int t0 = blockIdx.x * kKvTile, bg = blockIdx.y;
  const int b = bg / Hkv, g = bg % Hkv;
  const int64_t kv_ld = (int64_t)Hkv * kHd;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * i + 4 * w + (lane >> 4), c = lane & 15;
    const int key = t0 + r;
    const u32x4 x = key < T ? *reinterpret_cast<const u32x4*>(v + ((int64_t)b * T + key) * kv_ld + (int64_t)g * kHd + 8 * c)
                            : u32x4{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(tile + r * 256 + ((c ^ ((r >> 2) & 15)) << 4)) = x;
  }
  __syncthreads();
  const int kg = tid & 15, dc = tid >> 4;
  uint32_t x[4][4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = 4 * kg + e;
    const u32x4 y = *reinterpret_cast<const u32x4*>(tile + r * 256 + ((dc ^ ((r >> 2) & 15)) << 4));
    x[e][0] = y.x; x[e][1] = y.y; x[e][2] = y.z; x[e][3] = y.w;
  }
  uint16_t* dst = vt + (((int64_t)b * Hkv + g) * kHd + 8 * dc) * Tpad + t0 + 4 * kg;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // d = 8 dc + 2p (low halves of the keys' words) and +1 (high halves)
    const uint32_t lo01 = __builtin_amdgcn_perm(x[1][p], x[0][p], 0x05040100u);
    const uint32_t lo23 = __builtin_amdgcn_perm(x[3][p], x[2][p], 0x05040100u);
    const uint32_t hi01 = __builtin_amdgcn_perm(x[1][p], x[0][p], 0x07060302u);
    const uint32_t hi23 = __builtin_amdgcn_perm(x[3][p], x[2][p], 0x07060302u);
    *reinterpret_cast<u32x2a*>(dst + (int64_t)(2 * p) * Tpad) = u32x2a{lo01, lo23};
    *reinterpret_cast<u32x2a*>(dst + (int64_t)(2 * p + 1) * Tpad) = u32x2a{hi01, hi23};
  }
}

__global__ void __launch_bounds__(512, 1)
attn_fwd_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ vt,
                uint16_t* __restrict__ out, int B, int T, int Tpad, int Hq, int Hkv, float scale_log2, int causal) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wig = wave & 3;         // group (0: A, 1: B), wavefront in group
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
  // key tiles up to the workgroup's last row's limit (every wavefront runs
  // every tile; a tile past a wavefront's causal limit is masked whole)
  const int kv_end = causal ? min(T, q0 + kQBlock) : T;
  const int ntiles = (kv_end + kKvTile - 1) / kKvTile;
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

  const __amdgpu_buffer_rsrc_t rk = uni_rsrc_a(k, kExtentA);
  const __amdgpu_buffer_rsrc_t rv = uni_rsrc_a(vt, kExtentA);
  const uint32_t row_bytes = (uint32_t)(kv_ld * 2);
  const uint32_t kv_base = (uint32_t)(((int64_t)b * T * kv_ld + (int64_t)g * kHd) * 2);
  // ---- K tile (by one group of four wavefronts: group A in its
  // arithmetic phases, K(1) by group B in the prologue): 16 direct-to-LDS
  // loads of 1 KB, four per wavefront; load i of the group's wavefront w
  // fills rows 4(4i+w) .. +3, lane L takes
  // row +L/16 and physical chunk L&15 = logical chunk ^ (row & 15). The
  // per-lane part of each load's offset is fixed; the tile's part rides in
  // the scalar offset (tiles wholly below T) or is added with the key bound
  // check (the last tile).
  uint32_t kof[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * (4 * i + wig) + (lane >> 4);
    kof[i] = kv_base + (uint32_t)(((lane & 15) ^ (row & 15)) * 16) + (uint32_t)row * row_bytes;
  }
  auto load_k = [&](int tile, int slot) {
    char* dst = smem + slot * kTileBytes;
    const uint32_t tile_off = (uint32_t)tile * kKvTile * row_bytes;
    if ((tile + 1) * kKvTile <= T) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(dst + (4 * i + wig) * 1024), 16, kof[i], tile_off, 0,
                                                 0);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = tile * kKvTile + 4 * (4 * i + wig) + (lane >> 4);
        const uint32_t off = key < T ? kof[i] + tile_off : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(dst + (4 * i + wig) * 1024), 16, off, 0, 0, 0);
      }
    }
  };
  // ---- V^T tile (group B) from the transposed copy vt [B, Hkv, 128, Tpad]
  // (keys past T are zero there): 16 direct-to-LDS loads of 1 KB (8 V^T
  // rows of 64 keys), four per wavefront; load n fills stored rows 8n ..
  // +7; lane L takes stored row r = 8n + L/8 and physical chunk L&7, i.e.
  // logical row R = r ^ ((r>>3)&1) and logical chunk (L&7) ^ ((r>>1)&7)
  // (the layout vt_off reads). The tile's part of the offset is scalar.
  uint32_t vof[4];
  {
    const uint32_t vt_base = (uint32_t)(((int64_t)b * Hkv + g) * kHd * Tpad * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 8 * (4 * i + wig) + (lane >> 3);
      const int R = r ^ ((r >> 3) & 1), c = (lane & 7) ^ ((r >> 1) & 7);
      vof[i] = vt_base + (uint32_t)((R * Tpad + 8 * c) * 2);
    }
  }
  auto load_vt = [&](int tile, int slot) {
    char* dst = smem + kVtBase + slot * kTileBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(dst + (4 * i + wig) * 1024), 16, vof[i],
                                               (uint32_t)tile * kKvTile * 2, 0, 0);
  };
  // ---- fragment offsets: K tile (key block kb adds 32 rows = 8 KB; d
  // step s: row lq, chunk 2s + lh) and V^T tile (d block hb adds 32 rows =
  // 4 KB; 16-key step s2: row lq, chunk 2 s2 + lh)
  uint32_t kfa[8], vfa[4];
#pragma unroll
  for (int s = 0; s < 8; ++s) kfa[s] = (uint32_t)(lq * 256 + (((2 * s + lh) ^ (lq & 15)) << 4));
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) vfa[s2] = vt_off(lq, 2 * s2 + lh, 0);

  // ---- state
  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};
  f32x16 sacc[2] = {f32x16{}, f32x16{}};  // S^T of the tile in flight (key blocks 0, 1)
  bf16x8 pb[4];                           // P^T operands of the last softmaxed tile (16-key steps)
#pragma unroll
  for (int i = 0; i < 4; ++i) pb[i] = bf16x8{};
  float m_run = kMaskVal, l_run = 0.f;

  // MFMA phase m: S^T(m) = K(m) . Q^T (K slot m % 3) and O^T += V^T(m-1) .
  // P^T(m-1) (V^T slot (m-1)&1), the two products' MFMAs interleaved.
  auto mfma_phase = [&](int m) {
    const char* kt = smem + (m % 3) * kTileBytes;
    const char* vt = smem + kVtBase + ((m + 1) & 1) * kTileBytes;
    sacc[0] = f32x16{};
    sacc[1] = f32x16{};
    // MFMA pair i: S^T step (key block i & 1, d step i >> 1) and PV step
    // (16-key step i >> 2, d block i & 3); each fragment is read three
    // pairs ahead (a fence per pair keeps the reads from all being hoisted).
    auto kread = [&](int i) { return *reinterpret_cast<const bf16x8*>(kt + (i & 1) * 8192 + kfa[i >> 1]); };
    auto vread = [&](int i) { return *reinterpret_cast<const bf16x8*>(vt + (i & 3) * 4096 + vfa[i >> 2]); };
    bf16x8 kq[3], vq[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      kq[i] = kread(i);
      vq[i] = vread(i);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const bf16x8 kf = kq[i % 3], vf = vq[i % 3];
      if (i + 3 < 16) {
        kq[i % 3] = kread(i + 3);
        vq[i % 3] = vread(i + 3);
      }
      sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[i >> 1], sacc[i & 1], 0, 0, 0);
      o[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[i >> 2], o[i & 3], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Softmax of S^T(m): mask (only a tile that reaches past this
  // wavefront's first query or past T needs it; key index < lim, lim the
  // lane's causal / sequence bound relative to its first key of the tile),
  // maximum, rescale (the running maximum moves only when some lane's grows
  // by more than kSlack: probabilities then stay below 2^kSlack, the same
  // result up to rounding, and O is rescaled on few tiles), probabilities
  // into the P^T operands of the four 16-key steps. A tile masked whole
  // adds exactly nothing (p = 0, no rescale).
  auto softmax = [&](int m) {
    const int key0 = m * kKvTile;
    if (key0 + kKvTile > T || (causal && key0 + kKvTile - 1 > wq0)) {
      const int lim = (causal ? min(T, myq + 1) : T) - (key0 + 4 * lh);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          sacc[kb][e] = (32 * kb + 8 * (e >> 2) + (e & 3)) < lim ? sacc[kb][e] : kMaskVal;
    }
    // two independent chains of three-input maxima, one per key block
    float m2[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      m2[kb] = sacc[kb][0];
#pragma unroll
      for (int e = 1; e < 16; ++e) m2[kb] = fmax_nc(m2[kb], sacc[kb][e]);
    }
    float mt = pair_max(fmax_nc(m2[0], m2[1])) * scale_log2;
    if (__any(mt > m_run + kSlack)) {
      const float m_new = fmax_nc(m_run, mt);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= alpha;
    }
    uint32_t pk[2][4][2];  // [kb][group][packed pair]: 4 probabilities of the group
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        float p4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          p4[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][4 * gi + e], scale_log2, -m_run));
        pk[kb][gi][0] = pack2_rne(p4[0], p4[1]);
        pk[kb][gi][1] = pack2_rne(p4[2], p4[3]);
      }
    // row sum of the rounded probabilities the PV product uses: a dot
    // product with (1, 1) per packed pair, two independent chains, the
    // first continuing the running sum
    float ps[2] = {l_run, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int gi = 0; gi < 4; ++gi)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
          ps[h2] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk[kb][gi][h2]), kOnes2, ps[h2],
                                                   false);
    l_run = ps[0] + ps[1];
    // 16-key step s2 covers keys 16 s2 .. +15 = groups 2(s2&1), 2(s2&1)+1
    // of key block s2>>1. The lane with lh = 0 needs keys +0..7 (its own
    // first four, its partner's next four), lh = 1 keys +8..15: swap(own
    // g0, own g1) gives lanes 0-31 their g0 keys +0..3 (r0) and the
    // partner's +4..7 (r1), lanes 32-63 the partner's g1 keys +0..3 (r0)
    // and their own +4..7 (r1).
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const int kb = s2 >> 1, g0 = 2 * (s2 & 1), g1 = g0 + 1;
      const auto s0 = __builtin_amdgcn_permlane32_swap(pk[kb][g0][0], pk[kb][g1][0], false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap(pk[kb][g0][1], pk[kb][g1][1], false, false);
      pb[s2] = __builtin_bit_cast(bf16x8, u32x4{s0[0], s1[0], s0[1], s1[1]});
    }
  };
  // MFMA phase m of this wavefront. Every MFMA phase runs both products:
  // phase 0's PV step multiplies the zeroed P^T operands with the zeroed
  // V^T slot 1 (adds exactly 0), and phase ntiles' S^T is computed and never
  // used. Then the wavefront waits for its own loads of the arithmetic
  // phase before (the next barrier publishes them).
  auto m_phase = [&](int m) {
    __builtin_amdgcn_s_setprio(1);
    mfma_phase(m);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_enc(0));
  };
  // Arithmetic phase m: group A loads K(m+2) into the slot of K(m-1) (read
  // by both groups' MFMA phase m-1, which ended two barriers before), group
  // B loads V^T(m+1) into the slot of V^T(m-1) (read in MFMA phase m, which
  // ended at the barrier before); then the softmax of S^T(m).
  auto v_phase = [&](int m) {
    if (grp == 0) {
      if (m + 2 < ntiles) load_k(m + 2, (m + 2) % 3);
    } else {
      if (m + 1 < ntiles) load_vt(m + 1, (m + 1) & 1);
    }
    if (m >= 0 && m < ntiles) softmax(m);
  };

  // prologue: K(0) (group A) and K(1) (group B); V^T slot 1 zeroed (the
  // first MFMA phase reads it with zero P^T operands)
  if (grp == 0) load_k(0, 0);
  else if (kKvTile < kv_end) load_k(1, 1);
#pragma unroll
  for (int i = 0; i < 2; ++i)
    *reinterpret_cast<u32x4*>(smem + kVtBase + kTileBytes + (i * 512 + tid) * 16) = u32x4{0u, 0u, 0u, 0u};
  __builtin_amdgcn_s_waitcnt(vmcnt_enc(0));
  phase_barrier();
  // Phases: 2m (group A: MFMA m, group B: arithmetic m-1) and 2m+1 (A:
  // arithmetic m, B: MFMA m), m = 0 .. ntiles; each wavefront of a SIMD
  // pair is in the other kind of phase, so one's exponentials run under
  // the other's MFMAs. Each group runs its own loop; both meet the same
  // barriers.
  if (grp == 0) {
    for (int m = 0; m <= ntiles; ++m) {
      m_phase(m);
      phase_barrier();
      v_phase(m);
      phase_barrier();
    }
  } else {
    for (int m = 0; m <= ntiles; ++m) {
      v_phase(m - 1);
      phase_barrier();
      m_phase(m);
      phase_barrier();
    }
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

extern "C" size_t glt_attention_workspace_size(int32_t B, int32_t T, int32_t Hkv, int32_t head_dim) {
  if (B <= 0 || T <= 0 || Hkv <= 0 || head_dim <= 0) return 256;
  const int64_t Tpad = (T + kKvTile - 1) / kKvTile * kKvTile;
  return (size_t)(((int64_t)B * Hkv * head_dim * Tpad * 2 + 255) / 256 * 256);
}

extern "C" glt_status glt_attention_fwd(const void* q, const void* k, const void* v, void* out, int32_t B, int32_t T,
                                        int32_t Hq, int32_t Hkv, int32_t head_dim, float scale, int32_t causal,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  GLT_CHECK(B >= 0 && T >= 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, GLT_ERR_SHAPE,
            "glt_attention_fwd: B=%d T=%d Hq=%d Hkv=%d (Hq must be a multiple of Hkv)", B, T, Hq, Hkv);
  GLT_CHECK(head_dim == kHd, GLT_ERR_UNSUPPORTED, "glt_attention_fwd: head_dim %d (only %d)", head_dim, kHd);
  if (B == 0 || T == 0) return GLT_OK;
  GLT_CHECK(q && k && v && out, GLT_ERR_INVALID_ARG, "glt_attention_fwd: null pointer");
  GLT_CHECK(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16 == 0, GLT_ERR_ALIGNMENT,
            "glt_attention_fwd: tensors must be 16-byte aligned");
  const size_t need = glt_attention_workspace_size(B, T, Hkv, head_dim);
  GLT_CHECK(workspace && workspace_bytes >= need && (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
            GLT_ERR_WORKSPACE, "glt_attention_fwd: needs %zu workspace bytes, 256-byte aligned", need);
  // K and V^T rows are addressed through 31-bit buffer offsets
  GLT_CHECK((int64_t)B * T * Hkv * kHd * 2 < (int64_t)kOob && need < (size_t)kOob, GLT_ERR_SHAPE,
            "glt_attention_fwd: K of %lld bytes, V^T of %zu", (long long)B * T * Hkv * kHd * 2, need);
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
  const int Tpad = (T + kKvTile - 1) / kKvTile * kKvTile;
  uint16_t* vt = static_cast<uint16_t*>(workspace);
  GLT_LAUNCH("attn_vt", vt_pack_kernel, dim3((unsigned)(Tpad / kKvTile), (unsigned)(B * Hkv)), dim3(256), 0,
             as_stream(stream), static_cast<const uint16_t*>(v), vt, T, Tpad, Hkv);
  GLT_LAUNCH_CHECK("attn_vt");
  // 1-D over (query block, batch, head)
  const int64_t nblk = (int64_t)((T + kQBlock - 1) / kQBlock) * Hq * B;
  GLT_CHECK(nblk < INT32_MAX, GLT_ERR_SHAPE, "glt_attention_fwd: %lld workgroups", (long long)nblk);
  dim3 grid((unsigned)nblk, 1, 1);
  GLT_LAUNCH("attention", attn_fwd_kernel, grid, dim3(512), kAttnLds, as_stream(stream),
             static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), vt, static_cast<uint16_t*>(out), B, T,
             Tpad, Hq, Hkv, scale_log2, causal);
  GLT_LAUNCH_CHECK("attention");
  return GLT_OK;
}
