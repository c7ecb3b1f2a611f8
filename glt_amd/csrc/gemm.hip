// Segment-list GEMM kernels: the gfx950 bf16 MFMA kernel and the strided
// generic kernel (f32 path, unaligned shapes, graft-GEMM probes).
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cmath>

#include "gemm.hpp"
#include "layout.hpp"

namespace glt {

// ---------------------------------------------------------------- epilogue
// GEMM outputs are rounded with the gfx950 conversion instruction: round to
// nearest even, the same result as the reference's bias-and-shift rounding
// (src/kernels_elementwise_impl.inc:570-580) for every finite value. (The
// bit-exact conversion entry points keep the reference's integer form,
// which also fixes what NaN payloads become.)
__device__ __forceinline__ uint16_t bf16_hw(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }
__device__ __forceinline__ uint32_t pack2_hw(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
// sigmoid 1/(1+exp(-g)) from the hardware exp2 and reciprocal (each within
// about 1 ulp in f32) instead of the correctly rounded library sequences,
// which cost some 30 instructions per element in the epilogues; the values
// are rounded to the path dtype right after.
__device__ __forceinline__ float sigmoid_fast(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

template <typename TO>
__device__ __forceinline__ float ld_elem(const void* p, int64_t i) {
  if constexpr (sizeof(TO) == 4) return static_cast<const float*>(p)[i];
  else return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <typename TO>
__device__ __forceinline__ void st_elem(void* p, int64_t i, float v) {
  if constexpr (sizeof(TO) == 4) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = bf16_hw(v);
}
template <typename TO>
__device__ __forceinline__ float round_like(float v) {
  if constexpr (sizeof(TO) == 4) return v;
  else return bf16_to_f32(bf16_hw(v));
}

// a0 = accumulator (gate accumulator in the dual form), a1 = up accumulator.
template <typename TO, int MODE>
__device__ __forceinline__ void epilogue(const GProb& P, int m, int n, float a0, float a1) {
  if (m >= P.M || n >= P.N) return;
  const int64_t o = (int64_t)m * P.ldo + n;
  if constexpr (MODE == EPI_STORE) {
    float v = P.alpha * a0;
    if (P.beta != 0.f) v += P.beta * ld_elem<TO>(P.out0, o);
    st_elem<TO>(P.out0, o, v);
  } else if constexpr (MODE == EPI_RESID) {
    // the layer output is rounded to the path dtype, then added to the
    // residual stream (reference x = x + ffn_out, src/layer_forward_impl.inc:271-275)
    st_elem<TO>(P.out0, o, ld_elem<TO>(P.out0, o) + round_like<TO>(P.alpha * a0));
  } else if constexpr (MODE == EPI_SILU) {
    // gate/up pre-activations leave the accumulator rounded to the path
    // dtype (bf16 in the reference, src/layer_forward_impl.inc:72,122), and
    // silu(g)*u is formed from those values in the reference's f32 order
    // (src/kernels_elementwise_impl.inc:440-446): sg = 1/(1+exp(-g)), (g*sg)*u,
    // with sg from sigmoid_fast.
    const float g = round_like<TO>(a0), u = round_like<TO>(a1);
    const float sg = sigmoid_fast(g);
    st_elem<TO>(P.out0, o, g * sg * u);
    if (P.out1) st_elem<TO>(P.out1, o, g);
    if (P.out2) st_elem<TO>(P.out2, o, u);
  } else {
    // SiLU*up derivative on the dInter accumulator
    // (reference fused_gate_up_bwd_kernel, src/kernels_elementwise_impl.inc:107-117).
    const int64_t oa = (int64_t)m * P.ldaux + n;
    const float g = ld_elem<TO>(P.aux0, oa), u = ld_elem<TO>(P.aux1, oa);
    const float sg = sigmoid_fast(g);
    const float gv = g * sg;
    const float sgrad = sg * (1.0f + g * (1.0f - sg));
    st_elem<TO>(P.out0, o, a0 * u * sgrad);
    st_elem<TO>(P.out1, o, a0 * gv);
  }
}

// Locates problem and tile of tile index t. Within a problem tiles run in
// groups of kGroupM M-tiles, so tiles with neighbouring indices share A and
// B rows in L2.
// (4 measured best of 1, 2, 4, 8, 16 on the step's GEMMs: each XCD's 32
// tiles of a round form a 4 x 8 block.)
constexpr int kGroupM = 4;
__device__ __forceinline__ int locate_tile(const GArgs& args, int t, int& tm, int& tn) {
  int pi = 0;
  while (pi + 1 < args.nprob && t >= args.p[pi + 1].tile_begin) ++pi;
  const GProb& P = args.p[pi];
  t -= P.tile_begin;
  const int per_group = kGroupM * P.tiles_n;
  const int g = t / per_group;
  const int first_m = g * kGroupM;
  const int gm = min(P.tiles_m - first_m, kGroupM);
  const int r = t - g * per_group;
  tm = first_m + r % gm;
  tn = r / gm;
  return pi;
}

__device__ __forceinline__ bool seg_hits(const GSeg& S, const GProb& P, int n0, int bn) {
  return S.K > 0 && max(S.n_lo, n0) < min(min(S.n_hi, P.N), n0 + bn);
}

// =========================================================================
// gfx950 MFMA kernel: bf16 x bf16 -> f32, v_mfma_f32_32x32x16_bf16.
//
// Workgroup tile 256 (M) x 256 B-rows, K in steps of 64, 4 wavefronts in a
// 2x2 arrangement; each wavefront owns 128x128 outputs = 4x4 MFMA 32x32
// tiles (256 fp32 accumulators per lane, in AGPRs). Plain form: the 256
// B-rows are 256 output columns. Dual form: B-rows [0,128) are gate rows and
// [128,256) the up rows of the same 128 output columns.
//
// Persistent: the grid is one workgroup per CU; workgroup b walks tiles
// xb, xb + G, xb + 2G, ... (G = grid size). Workgroups are dealt
// round-robin over the 8 XCDs, so xb = (b & 7) * G/8 + b / 8 gives the 32
// workgroups of one XCD 32 consecutive tiles per round, which share A and B
// rows in that XCD's L2.
//
// Operands. LDS bandwidth is the scarce resource of this tile shape, so only
// A (activations, row-major) goes through LDS: direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds), each wavefront instruction moving 1 KB
// (8 rows x 128 bytes) with lane L landing at base + 16*L, into a ring of
// four 32 KB stages, issued two to three K-steps ahead of use and spread
// two per MFMA phase: the CU's address path moves about 64 bytes per clock,
// and loads issued in a burst stall the issuing wavefronts' MFMAs. B (weights) is read
// from the shuffled layout of layout.hpp straight into registers: per
// K-substep a wavefront's four 32-row fragments are four coalesced 1 KB
// loads, issued one K-step ahead. Rows outside a tile's valid range get an
// out-of-range offset and arrive as zeros. The load side walks the K-steps
// of all of the workgroup's tiles as one stream, so the next tile's first
// steps are in flight while the epilogue of the current one runs. The
// epilogue stores straight from the accumulators: the MFMA takes the B
// fragment as its first operand, which leaves each lane four consecutive
// output columns of one row per accumulator group.
// =========================================================================
constexpr int kBM = 256, kBK = 64;
constexpr int kTileElems = kBM * kBK;                    // one A tile = one LDS stage (32 KB)
constexpr int kAStages = 4;
constexpr uint32_t kExtent = 0x7FFFFFF0u;                // buffer extent below kOob
// cache policy of the epilogue's streams (written or read once here, used
// again only by another kernel): the nontemporal bit
constexpr int kNt = 2;
constexpr int kEpWaveBytes = 8192;                         // epilogue staging per wavefront
constexpr size_t kMfmaLds = (size_t)kAStages * kTileElems * 2 + 4 * kEpWaveBytes;  // 160 KB
constexpr uint32_t kShufStepBytes = kShufBlock * 2;      // one 32 x 64 block of B (4 KB)

// Rows are 64 bf16 = 128 bytes, one cache line each, so every global
// request a tile issues moves a whole line. gfx950 LDS serves a
// 16-byte-per-lane access 16 lanes at a time over 64 banks (256 bytes); a
// 16-lane group reading one logical chunk of 16 consecutive rows touches
// bank group 8*(row&1) + physical chunk, so the physical chunk is the
// logical one XOR (row>>1)&7, which makes the 16 groups distinct.
__device__ __forceinline__ int swz_key(int row) { return (row >> 1) & 7; }

// Buffer descriptor of a wave-uniform base and extent. The compiler loses
// track of their uniformity through the kernel's position bookkeeping and
// would wrap every buffer load in a per-lane loop over descriptor values;
// readfirstlane states it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uni_rsrc(const void* p, uint32_t n) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(n));
}

// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt <= n and leaves
// expcnt / lgkmcnt unconstrained.
constexpr int vmcnt_enc(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Workgroup barrier of the K loop: waits for this wavefront's LDS reads
// (and scalar loads), then s_barrier; the "memory" clobber keeps the
// compiler from moving memory accesses across it. The caller has already
// waited for the direct-to-LDS loads the next reads need. __syncthreads()
// would add a release fence, which the compiler implements by waiting for
// nearly every direct-to-LDS load in flight, draining the prefetch ring at
// each barrier.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Orders one wavefront's LDS accesses across lanes: LDS executes a
// wavefront's instructions in order, so only the compiler must not move
// accesses across this point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One accumulator element moved to a VGPR where it is used. Arithmetic
// cannot read AGPRs; left to itself the compiler copies every accumulator
// to VGPRs as the K loop exits (256 registers at once) and spills. The
// "a" operand keeps the accumulators in AGPRs up to each group's reads.
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

template <typename TO, int MODE, bool DUAL>
__global__ void __launch_bounds__(256, 1) gemm_mfma_kernel(const GArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  constexpr int BN = DUAL ? 128 : 256;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int G = gridDim.x, total = args.total_tiles;
  const int b = blockIdx.x;
  const int first = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;

  auto next_active = [&](const GProb& P, int n0, int s, int send) __attribute__((always_inline)) {
    ++s;
    while (s < send && !seg_hits(args.s[s], P, n0, BN)) ++s;
    return s;
  };

  // ---- K-step stream positions: tile t, its problem pi, origin (m0, n0),
  // segment s (of [seg0, send)), K offset k within the segment's K.
  struct Pos {
    int t, pi, m0, n0, send, s, k, K;
  };
  // Moves q to the first active segment of tile q.t or of a later tile of
  // this workgroup (tiles without one have no K-steps); false past the end.
  auto first_seg = [&](Pos& q) __attribute__((always_inline)) {
    for (; q.t < total; q.t += G) {
      int tm, tn;
      q.pi = locate_tile(args, q.t, tm, tn);
      const GProb& P = args.p[q.pi];
      q.m0 = tm * kBM;
      q.n0 = tn * BN;
      q.send = P.seg0 + P.nseg;
      q.s = next_active(P, q.n0, P.seg0 - 1, q.send);
      if (q.s < q.send) {
        q.k = 0;
        q.K = args.s[q.s].K;
        return true;
      }
    }
    return false;
  };
  // One K-step on, after the caller has added kBK to q.k and found q.k >=
  // q.K: the next active segment of the tile, else the first of a later
  // tile (1), or the end of the stream (2). The common step (same segment)
  // stays in the K loop as one add and a branch not taken; this cold part
  // runs once per segment. Past the end the stream's K is kNoEnd, so it is
  // not entered again, and q.k restarts at 0 (the trailing loads' offsets
  // are kOob, so the scalar offset only has to stay small).
  constexpr int kNoEnd = 1 << 30;
  auto step_cold = [&](Pos& q) __attribute__((always_inline)) {
    q.k = 0;
    if (q.t >= total) {
      q.K = kNoEnd;
      return 2;
    }
    q.s = next_active(args.p[q.pi], q.n0, q.s, q.send);
    if (q.s < q.send) {
      q.K = args.s[q.s].K;
      return 1;
    }
    q.t += G;
    if (first_seg(q)) return 1;
    q.k = 0;
    q.K = kNoEnd;
    return 2;
  };

  // ---- A side: 8 direct-to-LDS loads per wavefront per K-step; load i of
  // wave w fills tile rows 8*g .. 8*g+7 with g = 4*i + w; lane L takes row
  // 8*g + L/8 and physical chunk L&7, i.e. logical chunk (L&7) ^
  // swz_key(row). Past the end of the stream every offset is kOob: trailing
  // loads deliver zeros without touching memory, which keeps the per-step
  // load count (and so the vmcnt arithmetic below) the same in every step.
  Pos pa{first, 0, 0, 0, 0, 0, 0, 0};
  const void* pA = nullptr;
  uint32_t nA = 0, voA[8];
  auto setup_a = [&]() __attribute__((always_inline)) {
    const GSeg& S = args.s[pa.s];
    const GProb& P = args.p[pa.pi];
    pA = S.A;
    nA = pA ? kExtent : 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (4 * i + wave) * 8 + (lane >> 3);
      const int kc = (lane & 7) ^ swz_key(row);
      const int m = pa.m0 + row;
      voA[i] = m < P.M ? (uint32_t)(((int64_t)m * S.lda + S.a_col + kc * 8) * 2) : kOob;
    }
  };
  auto end_a = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) voA[i] = kOob;
  };
  auto adv_a = [&]() __attribute__((always_inline)) {
    pa.k += kBK;
    if (__builtin_expect(pa.k >= pa.K, 0)) {
      if (step_cold(pa) == 1) setup_a();
      else end_a();
    }
  };
  typedef __attribute__((address_space(3))) void lds_void;
  auto load_a = [&](int stage, int i) {
    uint16_t* dst = smem + stage * kTileElems + (4 * i + wave) * 8 * kBK;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(uni_rsrc(pA, nA), (lds_void*)dst, 16, voA[i], (uint32_t)pa.k * 2, 0, 0);
  };

  // ---- B side: fragment j of this wavefront covers B rows
  // n0 + (dual: wn*64 + (j&1)*32, from B1 for j >= 2; plain: wn*128 + j*32)
  // .. +31. Its per-lane offset selects the 32-row block and the lane's
  // 16 bytes in it; the K-step and substep ride in the scalar offset.
  Pos pb{first, 0, 0, 0, 0, 0, 0, 0};
  const void *pB0 = nullptr, *pB1 = nullptr;
  uint32_t nB0 = 0, nB1 = 0, voB[4];
  auto setup_b = [&]() __attribute__((always_inline)) {
    const GSeg& S = args.s[pb.s];
    const GProb& P = args.p[pb.pi];
    pB0 = S.B0;
    pB1 = DUAL ? S.B1 : S.B0;
    nB0 = pB0 ? kExtent : 0;
    nB1 = pB1 ? kExtent : 0;
    const int nlo = S.n_lo, nhi = min(S.n_hi, P.N);
    auto voff = [&](int j, int64_t ld, int r0) {
      const int f0 = pb.n0 + (DUAL ? wn * 64 + (j & 1) * 32 : wn * 128 + j * 32);
      const int n = f0 + (lane & 31);
      return (n >= nlo && n < nhi) ? (uint32_t)((int64_t)((f0 - r0) >> 5) * ld * 64 + lane * 16) : kOob;
    };
    // Separate loops for the two operands: a per-fragment choice between
    // two fields of the argument block makes the compiler copy the block to
    // scratch.
#pragma unroll
    for (int j = 0; j < 2; ++j) voB[j] = voff(j, S.ldb0, S.b0_row0);
#pragma unroll
    for (int j = 2; j < 4; ++j) voB[j] = DUAL ? voff(j, S.ldb1, S.b1_row0) : voff(j, S.ldb0, S.b0_row0);
  };
  auto end_b = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) voB[j] = kOob;
  };
  auto adv_b = [&]() __attribute__((always_inline)) {
    pb.k += kBK;
    if (__builtin_expect(pb.k >= pb.K, 0)) {
      if (step_cold(pb) == 1) setup_b();
      else end_b();
    }
  };
  bf16x8 fb[4][4];  // [substep][fragment]
  auto load_b = [&](int s, int j) {
    const __amdgpu_buffer_rsrc_t r = (DUAL && j >= 2) ? uni_rsrc(pB1, nB1) : uni_rsrc(pB0, nB0);
    const uint32_t so = (uint32_t)(pb.k / kBK) * kShufStepBytes + s * 1024;
    fb[s][j] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voB[j], so, 0));
  };

  // ---- compute side. A K-step is four substeps of 16; the A fragments of
  // the next substep are read from LDS while the 16 MFMAs of the current
  // one run, and each B fragment is reloaded for the next K-step as soon as
  // its four MFMAs have been issued.
  f32x16 acc[4][4];
  const int lr = lane & 31, lkh = lane >> 5;
  int aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) aoff[i] = (wm * 128 + i * 32 + lr) * kBK;
  const int sw = swz_key(lr);  // every fragment row this lane reads is lr mod 32
  bf16x8 fa[2][4];
  auto read_a = [&](int stage, int ks, int slot, int i) {
    const int ch = ((ks * 2 + lkh) ^ sw) << 3;
    fa[slot][i] = *reinterpret_cast<const bf16x8*>(smem + stage * kTileElems + aoff[i] + ch);
  };
  // MFMAs of substep s (A slot fs) in four groups, one per B fragment j:
  // four MFMAs, then the A read i = j of (rst, rks) into slot fs^1, then the
  // reload of fb[s][j]; `extra` adds work per group (the A loads).
  // The B loads are unconditional: the compiler's waits on fb then stay
  // one K-step deep.
  auto phase = [&](int fs, int s, int rst, int rks, auto&& extra) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[s][j], fa[fs][i], acc[i][j], 0, 0, 0);
      read_a(rst, rks, fs ^ 1, j);
      load_b(s, j);
      extra(j);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Pipeline fill: A tiles of K-steps 0..2 into stages 0..2, loads 0-1 of
  // step 3 (the rest follow in step 0), B of step 0.
  if (!first_seg(pa)) {
    pa.k = 0;
    pa.K = kNoEnd;
  }
  pb = pa;
  if (pa.t < total) {
    setup_a();
    setup_b();
  } else {
    end_a();
    end_b();
  }
#pragma unroll 1
  for (int st = 0; st < kAStages - 1; ++st) {
#pragma unroll
    for (int i = 0; i < 8; ++i) load_a(st, i);
    adv_a();
  }
  load_a(kAStages - 1, 0);
  load_a(kAStages - 1, 1);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) load_b(s, j);
  adv_b();
  // A of steps 0 and 1: the last load of step 1 is followed by 8 A loads of
  // step 2, 2 of step 3 and the 16 B loads. With step 1 landed here, the
  // first K-step needs no wait of its own (as the first step after an
  // epilogue).
  __builtin_amdgcn_s_waitcnt(vmcnt_enc(26));
  ring_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i) read_a(0, 0, 0, i);
  int g = 0;  // K-steps consumed so far; step g's A tile sits in stage g % 4

  char* const ep = reinterpret_cast<char*>(smem) + (size_t)kAStages * kTileElems * 2 + wave * kEpWaveBytes;
  // A of the step after the current one is already known to have landed
  // (waited for before the last epilogue, or in the pipeline fill)
  bool prewaited = true;
  for (int ct = first; ct < total; ct += G) {
    int tm, tn;
    const int pi = locate_tile(args, ct, tm, tn);
    const GProb& P = args.p[pi];
    const int m0 = tm * kBM, n0 = tn * BN, send = P.seg0 + P.nseg;
    int T = 0;  // K-steps of this tile over the segments it touches
    for (int s = next_active(P, n0, P.seg0 - 1, send); s < send; s = next_active(P, n0, s, send))
      T += args.s[s].K / kBK;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

    // Per K-step g (A stage st = g % 4):
    //   phases 0-2  MFMAs of substeps 0..2 | A reads of substeps 1..3 |
    //               B loads of substeps 0..2 of step g+1 | A loads 2-7 of
    //               step g+3 into stage (g+3) % 4, free since step g-1
    //   wait for this thread's A loads of step g+1, barrier: step g+1 is in
    //               LDS for everyone and nobody reads stage st any more
    //   phase 3     MFMAs of substep 3 | A loads 0-1 of step g+4 into st |
    //               A reads of substep 0 of step g+1 | B loads of substep 3
    // Every phase issues B, B, A, B, B, A (one B per MFMA group, an A after
    // groups 1 and 3).
    // Step g+1 may belong to the next tile: its substep-0 A fragments and
    // its B fragments stay in registers across the epilogue.
    for (int it = 0; it < T; ++it, ++g) {
      const int st = g & (kAStages - 1), nst = (g + 1) & (kAStages - 1), pst = (g + 3) & (kAStages - 1);
      phase(0, 0, st, 1, [&](int j) {
        if (j & 1) load_a(pst, 2 + (j >> 1));
      });
      phase(1, 1, st, 2, [&](int j) {
        if (j & 1) load_a(pst, 4 + (j >> 1));
      });
      phase(0, 2, st, 3, [&](int j) {
        if (j & 1) load_a(pst, 6 + (j >> 1));
      });
      adv_a();
      // Loads complete in order, so vmcnt <= n guarantees every load that
      // has at least n loads issued after it. The last A load of step g+1
      // was issued at the end of phase 2 of step g-2; after it come 48
      // loads (phase 3 of step g-2, step g-1, phases 0-2 of step g: 6 per
      // phase). Stores in between only raise the count. In the first step
      // of the kernel and right after an epilogue that wait was already
      // done, with no stores outstanding.
      if (__builtin_expect(!prewaited, 1)) __builtin_amdgcn_s_waitcnt(vmcnt_enc(48));
      prewaited = false;
      ring_barrier();
      __builtin_amdgcn_sched_barrier(0);
      phase(1, 3, nst, 0, [&](int j) {
        if (j & 1) load_a(st, j >> 1);
      });
      adv_b();
    }
    // The first step of the next tile needs A of step g+1 (g = steps
    // consumed). Once two steps have run, its last load has 30 loads after
    // it (phase 3 of step g-2 and step g-1), so waiting here, before the
    // epilogue's stores raise the count, is nearly free. (Earlier the first
    // step waits as usual; the stores only make that wait longer.)
    if (g >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_enc(30));
    prewaited = g >= 2;

    // ---- epilogue. The B fragment is the MFMA's first operand, so block
    // acc[i][j] is the transposed 32x32 product: lane l owns output row
    // 32*i + (l & 31) of the wavefront's rows and, in elements 4q..4q+3, the
    // four consecutive columns 32*jc + 8*q + 4*(l >> 5) .. +3 of its columns
    // (jc = j; dual: j & 1, with j < 2 gate and j >= 2 up). Groups of four
    // go to the wavefront's private LDS block as one 8-byte (bf16) or
    // 16-byte (f32) write and come back row-wise, so each global access is
    // 16 bytes per lane over whole 128-byte lines.
    constexpr int ESZ = sizeof(TO);
    const int rbase = m0 + wm * 128;
    const int cbase = n0 + (DUAL ? wn * 64 : wn * 128);
    const int wr = lane & 31, wh = lane >> 5;  // staging-write row and half
    const __amdgpu_buffer_rsrc_t r0 = uni_rsrc(P.out0, kExtent);
    // byte offset of output (row, col), kOob outside [M, N)
    auto ooff = [&](int row, int col, int64_t ld, int esz) {
      return (row < P.M && col < P.N) ? (uint32_t)(((int64_t)row * ld + col) * esz) : kOob;
    };
    if constexpr (ESZ == 2 && MODE != EPI_DGDU) {
      // bf16 outputs. Plain: 32 rows x 128 columns per block (256-byte
      // rows, 16 chunks); dual: 32 x 64 per output (128-byte rows, 8
      // chunks). Chunk c of row r sits at chunk c ^ key(r) and its two
      // 8-byte halves swap for r >= 16: the 32 rows of one 8-byte write
      // then cover all 64 banks once, and so do the 16-byte row reads.
      constexpr int kPitch = DUAL ? 128 : 256;
      auto key = [](int r) { return DUAL ? (r >> 1) & 7 : r & 15; };
      auto put = [&](int c, u32x2 d) {
        *reinterpret_cast<u32x2*>(ep + wr * kPitch + ((c ^ key(wr)) << 4) + ((wh ^ (wr >> 4)) << 3)) = d;
      };
      // reads: DUAL 8 lanes x 8 rows per instruction, plain 16 x 4
      constexpr int kLanesPerRow = kPitch / 16, kRowsPerRead = 64 / kLanesPerRow;
      const int rc = lane % kLanesPerRow, rr0 = lane / kLanesPerRow;
      auto drain = [&](__amdgpu_buffer_rsrc_t r, int i) {
        u32x4 q[32 / kRowsPerRead];
        uint32_t o[32 / kRowsPerRead];
#pragma unroll
        for (int k = 0; k < 32 / kRowsPerRead; ++k) {
          const int row = k * kRowsPerRead + rr0;
          q[k] = *reinterpret_cast<const u32x4*>(ep + row * kPitch + ((rc ^ key(row)) << 4));
          if (k * kRowsPerRead >= 16) q[k] = u32x4{q[k].z, q[k].w, q[k].x, q[k].y};
          o[k] = ooff(rbase + 32 * i + row, cbase + 8 * rc, P.ldo, 2);
        }
        if constexpr (MODE == EPI_RESID) {
          // residual rows are read where they are written: 16 bytes per lane
#pragma unroll
          for (int k = 0; k < 32 / kRowsPerRead; ++k) {
            const u32x4 x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o[k], 0, 0));
            const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ys[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
            uint32_t zs[4];
#pragma unroll
            for (int w = 0; w < 4; ++w)
              zs[w] = pack2_hw(__uint_as_float(xs[w] << 16) + __uint_as_float(ys[w] << 16),
                               __uint_as_float(xs[w] & 0xFFFF0000u) + __uint_as_float(ys[w] & 0xFFFF0000u));
            q[k] = u32x4{zs[0], zs[1], zs[2], zs[3]};
          }
        }
#pragma unroll
        for (int k = 0; k < 32 / kRowsPerRead; ++k) __builtin_amdgcn_raw_buffer_store_b128(q[k], r, o[k], 0, kNt);
      };
      if constexpr (MODE == EPI_STORE || MODE == EPI_RESID) {
        const float alpha = P.alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              float v[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = alpha * acc_read(acc[i][j][4 * q + e]);
              put(4 * j + q, u32x2{pack2_hw(v[0], v[1]), pack2_hw(v[2], v[3])});
            }
          wave_lds_sync();
          drain(r0, i);
          wave_lds_sync();
        }
      } else {
        // gate/up pre-activations leave the accumulator rounded to the path
        // dtype; silu(g)*u is formed from those values. A null out1/out2
        // gets a zero-extent descriptor, whose stores are dropped.
        const __amdgpu_buffer_rsrc_t r1 = uni_rsrc(P.out1, P.out1 ? kExtent : 0u);
        const __amdgpu_buffer_rsrc_t r2 = uni_rsrc(P.out2, P.out2 ? kExtent : 0u);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          u32x2 pg[2][4], pu[2][4];
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              float g[4], u[4], r[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                g[e] = round_like<TO>(acc_read(acc[i][j][4 * q + e]));
                u[e] = round_like<TO>(acc_read(acc[i][j + 2][4 * q + e]));
                r[e] = g[e] * sigmoid_fast(g[e]) * u[e];
              }
              pg[j][q] = u32x2{pack2_hw(g[0], g[1]), pack2_hw(g[2], g[3])};
              pu[j][q] = u32x2{pack2_hw(u[0], u[1]), pack2_hw(u[2], u[3])};
              put(4 * j + q, u32x2{pack2_hw(r[0], r[1]), pack2_hw(r[2], r[3])});
            }
          wave_lds_sync();
          drain(r0, i);
          wave_lds_sync();
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) put(4 * j + q, pg[j][q]);
          wave_lds_sync();
          drain(r1, i);
          wave_lds_sync();
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) put(4 * j + q, pu[j][q]);
          wave_lds_sync();
          drain(r2, i);
          wave_lds_sync();
        }
      }
    } else {
      // f32 staging: each block is done in two halves of 32 rows x 64
      // columns (256-byte rows, 16 chunks of four f32; chunk c of row r at
      // c ^ (r & 15)). A write puts 16 lanes on 16 rows of one chunk, a
      // read 16 lanes on the 16 chunks of one row: conflict-free both ways.
      auto put = [&](int c, const float* v) {
        *reinterpret_cast<f32x4*>(ep + wr * 256 + ((c ^ (wr & 15)) << 4)) = f32x4{v[0], v[1], v[2], v[3]};
      };
      const int rc = lane & 15, rr0 = lane >> 4;  // reads: 16 lanes x 4 rows
      auto stage = [&](int i, int jh, float scale) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = scale * acc_read(acc[i][2 * jh + jj][4 * q + e]);
            put(8 * jj + 2 * q + wh, v);
          }
      };
      auto fetch = [&](int k) {  // row k*4 + rr0 of the staged half, 4 f32
        const int row = 4 * k + rr0;
        return *reinterpret_cast<const f32x4*>(ep + row * 256 + ((rc ^ (row & 15)) << 4));
      };
      if constexpr (MODE == EPI_STORE || MODE == EPI_RESID) {
        const float alpha = P.alpha;
#pragma unroll
        for (int h = 0; h < 8; ++h) {
          const int i = h >> 1, jh = h & 1;
          stage(i, jh, alpha);
          wave_lds_sync();
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            f32x4 v = fetch(k);
            const uint32_t o = ooff(rbase + 32 * i + 4 * k + rr0, cbase + 64 * jh + 4 * rc, P.ldo, ESZ);
            if constexpr (MODE == EPI_RESID)
              v += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r0, o, 0, 0));
            const u32x4 d = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
            __builtin_amdgcn_raw_buffer_store_b128(d, r0, o, 0, 0);
          }
          wave_lds_sync();
        }
      } else {
        static_assert(MODE != EPI_DGDU || ESZ == 2, "the DGDU epilogue reads and writes bf16");
        // SiLU*up derivative (reference fused_gate_up_bwd_kernel,
        // src/kernels_elementwise_impl.inc:107-117) on the f32 dInter
        // values; the saved gate/up pre-activations of a half are loaded
        // one half ahead.
        const __amdgpu_buffer_rsrc_t r1 = uni_rsrc(P.out1, kExtent);
        const __amdgpu_buffer_rsrc_t rG = uni_rsrc(P.aux0, kExtent);
        const __amdgpu_buffer_rsrc_t rU = uni_rsrc(P.aux1, kExtent);
        // Halves h = 2 i + jh; the loop over the four row blocks i stays
        // rolled (only the accumulator block of a half needs a constant
        // index, chosen by a switch), which keeps this epilogue's code a
        // quarter of its unrolled size.
        u32x2 ga[2][8], ua[2][8];
        auto aux = [&](int i, int jh, int slot) {
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const uint32_t o = ooff(rbase + 32 * i + 4 * k + rr0, cbase + 64 * jh + 4 * rc, P.ldaux, 2);
            ga[slot][k] = __builtin_amdgcn_raw_buffer_load_b64(rG, o, 0, kNt);
            ua[slot][k] = __builtin_amdgcn_raw_buffer_load_b64(rU, o, 0, kNt);
          }
        };
        aux(0, 0, 0);
#pragma unroll 1
        for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) {
          if (jh == 0) aux(i, 1, 1);
          else if (i < 3) aux(i + 1, 0, 0);
          switch (i) {
            case 0: stage(0, jh, 1.0f); break;
            case 1: stage(1, jh, 1.0f); break;
            case 2: stage(2, jh, 1.0f); break;
            default: stage(3, jh, 1.0f); break;
          }
          wave_lds_sync();
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const f32x4 a4 = fetch(k);
            const float av[4] = {a4.x, a4.y, a4.z, a4.w};
            const u32x2 gk = ga[jh][k], uk = ua[jh][k];
            const float gv[4] = {__uint_as_float(gk.x << 16), __uint_as_float(gk.x & 0xFFFF0000u),
                                 __uint_as_float(gk.y << 16), __uint_as_float(gk.y & 0xFFFF0000u)};
            const float uv[4] = {__uint_as_float(uk.x << 16), __uint_as_float(uk.x & 0xFFFF0000u),
                                 __uint_as_float(uk.y << 16), __uint_as_float(uk.y & 0xFFFF0000u)};
            float dg[4], du[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float sg = sigmoid_fast(gv[e]);
              const float sgrad = sg * (1.0f + gv[e] * (1.0f - sg));
              dg[e] = av[e] * uv[e] * sgrad;
              du[e] = av[e] * (gv[e] * sg);
            }
            const uint32_t o = ooff(rbase + 32 * i + 4 * k + rr0, cbase + 64 * jh + 4 * rc, P.ldo, 2);
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack2_hw(dg[0], dg[1]), pack2_hw(dg[2], dg[3])}, r0, o, 0, kNt);
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack2_hw(du[0], du[1]), pack2_hw(du[2], du[3])}, r1, o, 0, kNt);
          }
          wave_lds_sync();
        }
        }
      }
    }
  }
  // trailing (zero) loads must land before the workgroup's LDS is released
  __builtin_amdgcn_s_waitcnt(vmcnt_enc(0));
}

// =========================================================================
// Generic strided kernel: 64x64 output tile (dual: 64 gate + 64 up columns),
// K-step 16, operands converted to f32 on load, f32 FMA accumulation.
// =========================================================================
template <int KIND>
__device__ __forceinline__ float ld_kind(const void* p, int64_t i) {
  if constexpr (KIND == LD_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else if constexpr (KIND == LD_F32) return static_cast<const float*>(p)[i];
  else return bf16_to_f32(f32_to_bf16(static_cast<const float*>(p)[i]));
}

template <int LA, int LB, typename TO, int MODE, bool DUAL>
__global__ void __launch_bounds__(256) gemm_generic_kernel(const GArgs args) {
  constexpr int BM = 64, BN = 64, BK = 16, NB = DUAL ? 2 : 1;
  __shared__ float As[BK][BM + 1];
  __shared__ float Bs[NB][BK][BN + 1];
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  int tm, tn;
  const int pi = locate_tile(args, blockIdx.x, tm, tn);
  const GProb& P = args.p[pi];
  const int m0 = tm * BM, n0 = tn * BN;
  float acc[NB][4][4] = {};
  for (int s = P.seg0; s < P.seg0 + P.nseg; ++s) {
    const GSeg& S = args.s[s];
    if (!seg_hits(S, P, n0, BN)) continue;
    const int nhi = min(S.n_hi, P.N);
    for (int k0 = 0; k0 < S.K; k0 += BK) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = tid + 256 * q, r = e >> 4, kk = e & 15;
        const int m = m0 + r, k = k0 + kk;
        As[kk][r] = (m < P.M && k < S.K) ? ld_kind<LA>(S.A, (int64_t)m * S.lda + (int64_t)(S.a_col + k) * S.a_ks) : 0.f;
#pragma unroll
        for (int h = 0; h < NB; ++h) {
          const void* B = h ? S.B1 : S.B0;
          const int64_t ld = h ? S.ldb1 : S.ldb0;
          const int r0 = h ? S.b1_row0 : S.b0_row0;
          const int n = n0 + r;
          Bs[h][kk][r] = (B && n >= S.n_lo && n < nhi && k < S.K)
                             ? ld_kind<LB>(B, (int64_t)(n - r0) * ld + (int64_t)k * S.b_ks)
                             : 0.f;
        }
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < BK; ++kk) {
        float a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = As[kk][tr + 16 * i];
#pragma unroll
        for (int h = 0; h < NB; ++h)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float b = Bs[h][kk][tc + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[h][i][j] = fmaf(a[i], b, acc[h][i][j]);
          }
      }
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      epilogue<TO, MODE>(P, m0 + tr + 16 * i, n0 + tc + 16 * j, acc[0][i][j], DUAL ? acc[NB - 1][i][j] : 0.f);
}

// ------------------------------------------------------------------ host
static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

bool gemm_mfma_eligible(const GemmPlan& plan) {
  if (plan.a_kind != LD_BF16 || plan.b_kind != LD_SHUF) return false;
  for (int i = 0; i < plan.nseg; ++i) {
    const GSeg& s = plan.args.s[i];
    if (s.a_ks != 1 || s.K % kBK != 0 || s.a_col % 8 != 0 || s.lda % 8 != 0 || !al16(s.A)) return false;
    // B fragments start on 32-row blocks of the shuffled operand
    if (s.n_lo % 32 != 0 || s.b0_row0 % 32 != 0 || s.ldb0 % kBK != 0 || s.K > s.ldb0 || !al16(s.B0)) return false;
    if (plan.dual && (s.b1_row0 % 32 != 0 || s.ldb1 % kBK != 0 || s.K > s.ldb1 || !al16(s.B1))) return false;
  }
  for (int p = 0; p < plan.args.nprob; ++p) {
    const GProb& P = plan.args.p[p];
    // the epilogue stores 16-byte column chunks (8 bf16 / 4 f32, so N is a
    // multiple of that) through 31-bit buffer offsets and never reads the
    // output (beta = 0)
    if (P.ldo % 8 || !al16(P.out0) || !al16(P.out1) || !al16(P.out2) || P.beta != 0.f) return false;
    if (P.N % (P.out_f32 ? 4 : 8) || (int64_t)(P.M + kBM) * P.ldo * (P.out_f32 ? 4 : 2) >= (int64_t)kOob)
      return false;
    if (P.mode == EPI_DGDU && (P.ldaux % 8 || !al16(P.aux0) || !al16(P.aux1))) return false;
    // the DGDU epilogue reads aux rows through 31-bit buffer offsets
    if (P.mode == EPI_DGDU && (int64_t)(P.M + kBM) * P.ldaux * 2 >= (int64_t)kOob) return false;
    for (int i = P.seg0; i < P.seg0 + P.nseg; ++i) {
      const GSeg& s = plan.args.s[i];
      // every byte offset a tile forms must fit the 31-bit buffer range
      if ((int64_t)(P.M + kBM) * s.lda * 2 >= (int64_t)kOob) return false;
      if ((int64_t)(s.n_hi - s.b0_row0 + 256) * s.ldb0 * 2 >= (int64_t)kOob) return false;
      if (plan.dual && (int64_t)(s.n_hi - s.b1_row0 + 256) * s.ldb1 * 2 >= (int64_t)kOob) return false;
    }
  }
  return true;
}

// CUs of the current device (the persistent grid size), cached per device.
// The caches are atomics: host threads making their first calls at the same
// time may both query the device (the same value), never race on the slot.
glt_status device_cus(int& cus) {
  static std::atomic<int> cached[64];
  int dev = 0;
  GLT_TRY_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) {
    set_error("gemm: device index %d out of range", dev);
    return GLT_ERR_HIP;
  }
  int c = cached[dev].load(std::memory_order_acquire);
  if (c == 0) {
    GLT_TRY_HIP(hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev));
    cached[dev].store(c, std::memory_order_release);
  }
  cus = c;
  return GLT_OK;
}

template <typename TO, int MODE, bool DUAL>
static glt_status launch_mfma(const GArgs& a, hipStream_t st, const char* label) {
  // the dynamic-LDS limit is a per-device attribute of the kernel (set
  // once per device; a concurrent first call sets the same value again)
  static std::atomic<bool> attr_set[64];
  auto fn = gemm_mfma_kernel<TO, MODE, DUAL>;
  int dev = 0;
  GLT_TRY_HIP(hipGetDevice(&dev));
  GLT_CHECK(dev >= 0 && dev < 64, GLT_ERR_HIP, "gemm: device index %d out of range", dev);
  if (!attr_set[dev].load(std::memory_order_acquire)) {
    GLT_TRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMfmaLds));
    attr_set[dev].store(true, std::memory_order_release);
  }
  int cus = 0;
  const glt_status rc = device_cus(cus);
  if (rc != GLT_OK) return rc;
  // one workgroup per CU (160 KB of LDS admits no second one)
  const int grid = a.total_tiles < cus ? a.total_tiles : cus;
  GLT_LAUNCH(label, fn, dim3(grid), dim3(256), kMfmaLds, st, a);
  GLT_LAUNCH_CHECK("gemm_mfma");
  return GLT_OK;
}

template <int LA, int LB, typename TO, int MODE, bool DUAL>
static glt_status launch_generic(const GArgs& a, hipStream_t st, const char* label) {
  GLT_LAUNCH(label, (gemm_generic_kernel<LA, LB, TO, MODE, DUAL>), dim3(a.total_tiles), dim3(256), 0, st, a);
  GLT_LAUNCH_CHECK("gemm_generic");
  return GLT_OK;
}

int gemm_mfma_tiles(const GemmPlan& plan) {
  const int bn = plan.dual ? 128 : 256;
  int tiles = 0;
  for (int p = 0; p < plan.args.nprob; ++p)
    tiles += (int)(cdiv(plan.args.p[p].M, kBM) * cdiv(plan.args.p[p].N, bn));
  return tiles;
}

// Rows per launch (a multiple of kBM) for which every byte offset the MFMA
// kernel forms from a problem's output, aux and A bases fits its 31-bit
// buffer range; 0 if not even one tile of rows does.
static int64_t mfma_row_block(const GemmPlan& plan) {
  int64_t rows = INT64_MAX;
  auto limit = [&](int64_t ld, int64_t esz) {
    if (ld > 0) rows = std::min(rows, ((int64_t)kOob - 1) / (ld * esz) - kBM);
  };
  for (int p = 0; p < plan.args.nprob; ++p) {
    const GProb& P = plan.args.p[p];
    limit(P.ldo, P.out_f32 ? 4 : 2);
    if (P.mode == EPI_DGDU) limit(P.ldaux, 2);
    for (int i = P.seg0; i < P.seg0 + P.nseg; ++i) limit(plan.args.s[i].lda, 2);
  }
  return rows <= 0 ? 0 : rows / kBM * kBM;
}

// Rows [r0, r0 + rows) of every problem of plan, as a plan of their own
// (output, aux and A bases moved to row r0).
static GemmPlan mfma_rows(const GemmPlan& plan, int64_t r0, int64_t rows) {
  GemmPlan sub = plan;
  for (int p = 0; p < sub.args.nprob; ++p) {
    GProb& P = sub.args.p[p];
    const int64_t m = std::max<int64_t>(0, std::min<int64_t>(rows, (int64_t)P.M - r0));
    if (m > 0) {
      const int64_t eo = P.out_f32 ? 4 : 2;
      auto mv = [&](void* q, int64_t ld, int64_t esz) {
        return q ? static_cast<void*>(static_cast<char*>(q) + r0 * ld * esz) : nullptr;
      };
      P.out0 = mv(P.out0, P.ldo, eo);
      P.out1 = mv(P.out1, P.ldo, eo);
      P.out2 = mv(P.out2, P.ldo, eo);
      P.aux0 = mv(const_cast<void*>(P.aux0), P.ldaux, 2);
      P.aux1 = mv(const_cast<void*>(P.aux1), P.ldaux, 2);
      for (int i = P.seg0; i < P.seg0 + P.nseg; ++i) {
        GSeg& S = sub.args.s[i];
        S.A = S.A ? static_cast<const char*>(S.A) + r0 * S.lda * 2 : nullptr;
      }
    }
    P.M = (int)m;
  }
  return sub;
}

glt_status run_gemm(GemmPlan& plan, hipStream_t st, bool allow_mfma) {
  GArgs& a = plan.args;
  if (a.nprob == 0) return GLT_OK;
  bool mfma = allow_mfma && gemm_mfma_eligible(plan);
  if (allow_mfma && !mfma && plan.a_kind == LD_BF16 && plan.b_kind == LD_SHUF) {
    // Too many rows for 31-bit offsets from the operand bases (e.g. an LM
    // head of 16384 tokens x 128256 logits, 4 GiB of output): the MFMA
    // kernel in row blocks whose offsets fit.
    int64_t max_m = 0;
    for (int p = 0; p < a.nprob; ++p) max_m = std::max<int64_t>(max_m, a.p[p].M);
    const int64_t rows = mfma_row_block(plan);
    if (rows >= kBM && rows < max_m && gemm_mfma_eligible(mfma_rows(plan, 0, rows))) {
      for (int64_t r0 = 0; r0 < max_m; r0 += rows) {
        GemmPlan sub = mfma_rows(plan, r0, rows);
        const glt_status s = run_gemm(sub, st, true);
        if (s != GLT_OK) return s;
      }
      return GLT_OK;
    }
  }
  const int bm = mfma ? kBM : 64;
  const int bn = mfma ? (plan.dual ? 128 : 256) : 64;
  const int mode = a.p[0].mode;
  const int of32 = a.p[0].out_f32;
  int tiles = 0;
  for (int p = 0; p < a.nprob; ++p) {
    GProb& P = a.p[p];
    GLT_CHECK(P.mode == mode && P.out_f32 == of32, GLT_ERR_INVALID_ARG, "run_gemm: mixed epilogues in one launch");
    P.tiles_m = (int)cdiv(P.M, bm);
    P.tiles_n = (int)cdiv(P.N, bn);
    P.tile_begin = tiles;
    tiles += P.tiles_m * P.tiles_n;
  }
  a.total_tiles = tiles;
  if (tiles == 0) return GLT_OK;
  if (mfma) {
    if (mode == EPI_SILU && plan.dual) return launch_mfma<uint16_t, EPI_SILU, true>(a, st, plan.label);
    if (mode == EPI_DGDU && !plan.dual) return launch_mfma<uint16_t, EPI_DGDU, false>(a, st, plan.label);
    if (mode == EPI_STORE && !plan.dual)
      return of32 ? launch_mfma<float, EPI_STORE, false>(a, st, plan.label)
                  : launch_mfma<uint16_t, EPI_STORE, false>(a, st, plan.label);
    if (mode == EPI_RESID && !plan.dual)
      return of32 ? launch_mfma<float, EPI_RESID, false>(a, st, plan.label)
                  : launch_mfma<uint16_t, EPI_RESID, false>(a, st, plan.label);
    set_error("run_gemm: no MFMA kernel for mode %d dual %d", mode, (int)plan.dual);
    return GLT_ERR_UNSUPPORTED;
  }
  const int la = plan.a_kind, lb = plan.b_kind;
  GLT_CHECK(lb != LD_SHUF && la != LD_SHUF, GLT_ERR_UNSUPPORTED,
            "run_gemm(%s): shuffled operand on a shape the MFMA kernel does not take", plan.label);
#define GLT_GEN(LA_, LB_, TO_, MODE_, DUAL_)                                                     \
  if (la == LA_ && lb == LB_ && (sizeof(TO_) == 4) == (of32 != 0) && mode == MODE_ && plan.dual == DUAL_) \
    return launch_generic<LA_, LB_, TO_, MODE_, DUAL_>(a, st, plan.label);
  // f32 path
  GLT_GEN(LD_F32, LD_F32, float, EPI_STORE, false)
  GLT_GEN(LD_F32, LD_F32, float, EPI_RESID, false)
  GLT_GEN(LD_F32, LD_F32, float, EPI_SILU, true)
  GLT_GEN(LD_F32, LD_F32, float, EPI_DGDU, false)
  // bf16 path on shapes the MFMA kernel does not take
  GLT_GEN(LD_BF16, LD_BF16, uint16_t, EPI_STORE, false)
  GLT_GEN(LD_BF16, LD_BF16, uint16_t, EPI_RESID, false)
  GLT_GEN(LD_BF16, LD_BF16, float, EPI_STORE, false)
  GLT_GEN(LD_BF16, LD_BF16, uint16_t, EPI_SILU, true)
  GLT_GEN(LD_BF16, LD_BF16, uint16_t, EPI_DGDU, false)
  // graft-GEMM probes (f32 operands rounded to bf16 on load)
  GLT_GEN(LD_BF16, LD_F32_AS_BF16, float, EPI_STORE, false)
  GLT_GEN(LD_F32_AS_BF16, LD_BF16, float, EPI_STORE, false)
  GLT_GEN(LD_F32_AS_BF16, LD_F32_AS_BF16, float, EPI_STORE, false)
#undef GLT_GEN
  set_error("run_gemm: no generic kernel for kinds (%d,%d) out_f32 %d mode %d dual %d", la, lb, of32, mode,
            (int)plan.dual);
  return GLT_ERR_UNSUPPORTED;
}

}  // namespace glt
