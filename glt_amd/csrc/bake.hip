// shadow_bake: merge graft deltas into bf16 base matrices.
//
// Every output element is bf16_rne(f32(base) + f32(delta)), the same single
// rounding as the reference kernel (src/shadow_bake_impl.inc:46-49), so the
// result is bit-exact. The reference launches one workgroup per graft row
// and, for the down projection, writes the transposed block with a row
// stride of I elements per lane (uncoalesced).
//
// Here one launch covers up to 16 layers (grid.z) and has two kinds
// of workgroup:
//  * stream blocks: each thread owns one 16-byte chunk (8 elements) of an
//    output row, consecutive threads and workgroups walk consecutive chunks
//    of the row-major region, so HBM sees long sequential runs in both the
//    base read and the output write. Gate/up graft rows are contiguous along
//    the output row, so they are added straight from global memory.
//  * tile blocks (down projection only): a 64x64 output tile that a graft
//    block touches. The graft's contiguous axis runs down the output column,
//    so the tile stages it through LDS and adds it in output orientation.
//    Stream blocks skip every chunk of such a tile.
#include <algorithm>

#include "common.hpp"

namespace glt {

constexpr int kTile = 64;
// Layers per launch and slices per bake: the launch argument block carries a
// graft pointer per (layer, slice), 1 KB at 16 x 8. Eight slices cover every
// stack glt_mlp_fwd / glt_mlp_bwd take (at most 8).
constexpr int kMaxLayers = 16;
constexpr int kMaxBakeSlices = 8;

struct BakePlacement {
  int i0, s, h0, h;
};

struct BakeLaunch {
  const uint16_t* src[kMaxLayers];            // base matrix per layer (read)
  uint16_t* dst[kMaxLayers];                  // output per layer (== src in place)
  const void* graft[kMaxLayers][kMaxBakeSlices];  // [S,H] delta of this projection
  BakePlacement pl[kMaxBakeSlices];
  int nslices;
  int trans;                 // 0: gate/up orientation, 1: down (transposed block)
  int src_rows, src_cols;    // base extent; reads outside are zero (appended tail)
  int64_t src_ld, dst_ld;
  int reg_r0, reg_r1, reg_c0, reg_c1;  // output region processed
  int chunks_per_row;        // 8-element chunks per region row
  uint32_t stream_chunks;    // chunks per layer handled by stream blocks
  int tile_bx0, tile_by0, tiles_x, n_tile_blocks;  // tile blocks: bounding box in region tile units
};

template <typename G>
__device__ __forceinline__ float gload(const G* p, int64_t i);
template <> __device__ __forceinline__ float gload<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float gload<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_to_f32(p[i]);
}

// 8 consecutive graft values from a 16-byte aligned address.
__device__ __forceinline__ void gload8(const float* p, float* v) {
  const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + 1);
  v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
  v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
}
__device__ __forceinline__ void unpack8(const u32x4 q, float* v) {
  v[0] = bf16_to_f32((uint16_t)(q.x & 0xFFFF)); v[1] = bf16_to_f32((uint16_t)(q.x >> 16));
  v[2] = bf16_to_f32((uint16_t)(q.y & 0xFFFF)); v[3] = bf16_to_f32((uint16_t)(q.y >> 16));
  v[4] = bf16_to_f32((uint16_t)(q.z & 0xFFFF)); v[5] = bf16_to_f32((uint16_t)(q.z >> 16));
  v[6] = bf16_to_f32((uint16_t)(q.w & 0xFFFF)); v[7] = bf16_to_f32((uint16_t)(q.w >> 16));
}
__device__ __forceinline__ void gload8(const uint16_t* p, float* v) {
  unpack8(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)), v);
}

// Does any slice's block (in output orientation) intersect the tile at
// (tr0, tc0)? Block-uniform.
__device__ __forceinline__ bool tile_hit(const BakeLaunch& a, int tr0, int tc0) {
  const int tr1 = min(tr0 + kTile, a.reg_r1), tc1 = min(tc0 + kTile, a.reg_c1);
  bool any = false;
#pragma unroll
  for (int j = 0; j < kMaxBakeSlices; ++j) {
    if (j >= a.nslices) break;
    const BakePlacement p = a.pl[j];
    const int fr0 = a.trans ? p.h0 : p.i0, fr1 = a.trans ? p.h0 + p.h : p.i0 + p.s;
    const int fc0 = a.trans ? p.i0 : p.h0, fc1 = a.trans ? p.i0 + p.s : p.h0 + p.h;
    any |= (max(tr0, fr0) < min(tr1, fr1)) && (max(tc0, fc0) < min(tc1, fc1));
  }
  return any;
}

// Base chunk (r, c..c+7) as f32; elements outside the base extent or past
// c_end read zero.
__device__ __forceinline__ void load_base8(const BakeLaunch& a, const uint16_t* src, int r, int c, int c_end,
                                           float* v) {
  const bool in_rows = r < a.src_rows;
  const int64_t so = (int64_t)r * a.src_ld + c;
  if (in_rows && c + 8 <= a.src_cols && c + 8 <= c_end && ((reinterpret_cast<uintptr_t>(src + so) & 15) == 0)) {
    unpack8(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + so)), v);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (in_rows && c + j < a.src_cols && c + j < c_end) ? bf16_to_f32(src[so + j]) : 0.f;
  }
}

__device__ __forceinline__ void store8(uint16_t* dst, int64_t dofs, int c, int c_end, const float* v) {
  if (c + 8 <= c_end && ((reinterpret_cast<uintptr_t>(dst + dofs) & 15) == 0)) {
    u32x4 o;
    o.x = pack_bf16x2(v[0], v[1]);
    o.y = pack_bf16x2(v[2], v[3]);
    o.z = pack_bf16x2(v[4], v[5]);
    o.w = pack_bf16x2(v[6], v[7]);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(dst + dofs));
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (c + j < c_end) dst[dofs + j] = f32_to_bf16(v[j]);
  }
}

template <typename G>
__device__ __forceinline__ void bake_stream(const BakeLaunch& a, int L, uint32_t q) {
  if (q >= a.stream_chunks) return;
  const uint32_t cpr = (uint32_t)a.chunks_per_row;
  const uint32_t qr = q / cpr;
  const int r = a.reg_r0 + (int)qr, c = a.reg_c0 + 8 * (int)(q - qr * cpr);
  // chunks are 8-aligned from reg_c0, so a chunk lies in exactly one tile
  if (a.n_tile_blocks && tile_hit(a, a.reg_r0 + ((r - a.reg_r0) & ~(kTile - 1)),
                                  a.reg_c0 + ((c - a.reg_c0) & ~(kTile - 1))))
    return;
  const int c_end = min(c + 8, a.reg_c1);
  float v[8];
  load_base8(a, a.src[L], r, c, c_end, v);
  if (!a.trans) {
    // -0.0 is the additive identity for every f32 (x + -0.0 == x, also for
    // x = -0.0), so elements no slice covers pass the base through bit for
    // bit; a covered element becomes base + delta. The tile blocks sum the
    // same way.
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = -0.0f;
    bool hit = false;
#pragma unroll
    for (int j = 0; j < kMaxBakeSlices; ++j) {
      if (j >= a.nslices) break;
      const BakePlacement p = a.pl[j];
      if (r < p.i0 || r >= p.i0 + p.s) continue;
      const int lo = max(c, p.h0), hi = min(c_end, p.h0 + p.h);
      if (lo >= hi) continue;
      hit = true;
      const G* g = static_cast<const G*>(a.graft[L][j]) + (int64_t)(r - p.i0) * p.h + (c - p.h0);
      if (lo == c && hi == c + 8 && ((reinterpret_cast<uintptr_t>(g) & 15) == 0)) {
        float w[8];
        gload8(g, w);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += w[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (c + e >= lo && c + e < hi) acc[e] += gload(g, e);
      }
    }
    if (hit) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += acc[e];
    }
  }
  store8(a.dst[L], (int64_t)r * a.dst_ld + c, c, c_end, v);
}

template <typename G>
__device__ __forceinline__ void bake_tile(const BakeLaunch& a, int L, int tb, float (*gt)[kTile + 1]) {
  const int tr0 = a.reg_r0 + (a.tile_by0 + tb / a.tiles_x) * kTile;
  const int tc0 = a.reg_c0 + (a.tile_bx0 + tb % a.tiles_x) * kTile;
  if (!tile_hit(a, tr0, tc0)) return;  // stream blocks cover it
  const int tr1 = min(tr0 + kTile, a.reg_r1);
  const int tc1 = min(tc0 + kTile, a.reg_c1);
  const int t = threadIdx.x;
  for (int e = t; e < kTile * kTile; e += 256) gt[e >> 6][e & 63] = -0.0f;
  __syncthreads();
  for (int j = 0; j < a.nslices; ++j) {
    const BakePlacement p = a.pl[j];
    const G* g = static_cast<const G*>(a.graft[L][j]);
    // out(r, c) += G[c - i0, r - h0]; consecutive threads walk r (contiguous in G)
    for (int e = t; e < kTile * kTile; e += 256) {
      const int lc = e >> 6, lr = e & 63, r = tr0 + lr, c = tc0 + lc;
      if (r < tr1 && c < tc1 && c >= p.i0 && c < p.i0 + p.s && r >= p.h0 && r < p.h0 + p.h)
        gt[lr][lc] += gload(g, (int64_t)(c - p.i0) * p.h + (r - p.h0));
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = t + 256 * i;
    const int lr = q >> 3, lc = (q & 7) * 8;
    const int r = tr0 + lr, c = tc0 + lc;
    if (r >= tr1 || c >= tc1) continue;
    float v[8];
    load_base8(a, a.src[L], r, c, tc1, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] += gt[lr][lc + j];
    store8(a.dst[L], (int64_t)r * a.dst_ld + c, c, tc1, v);
  }
}

template <typename G>
__global__ void __launch_bounds__(256) bake_kernel(const BakeLaunch a) {
  __shared__ float gt[kTile][kTile + 1];
  const int L = blockIdx.z;
  if ((int)blockIdx.x < a.n_tile_blocks)
    bake_tile<G>(a, L, blockIdx.x, gt);
  else
    bake_stream<G>(a, L, (uint32_t)(blockIdx.x - a.n_tile_blocks) * 256u + threadIdx.x);
}

// Fills the work split of a launch whose region, slices and orientation are
// set, then launches it over `nlayers` layers.
static glt_status launch_bake(BakeLaunch& a, int nlayers, int graft_dtype, hipStream_t st) {
  if (nlayers == 0 || a.reg_r1 <= a.reg_r0 || a.reg_c1 <= a.reg_c0) return GLT_OK;
  const int rows = a.reg_r1 - a.reg_r0, cols = a.reg_c1 - a.reg_c0;
  a.chunks_per_row = cdiv(cols, 8);
  const int64_t chunks = (int64_t)rows * a.chunks_per_row;
  GLT_CHECK(chunks < (int64_t)UINT32_MAX - 256, GLT_ERR_SHAPE, "shadow_bake: %d x %d region too large", rows,
            cols);
  a.stream_chunks = (uint32_t)chunks;
  a.n_tile_blocks = 0;
  a.tiles_x = 1;
  a.tile_bx0 = a.tile_by0 = 0;
  if (a.trans) {
    // bounding box, in region tile units, of the tiles the slices touch
    int bx0 = INT32_MAX, by0 = INT32_MAX, bx1 = -1, by1 = -1;
    bool whole = false;
    for (int j = 0; j < a.nslices; ++j) {
      const BakePlacement p = a.pl[j];
      const int r0 = std::max(p.h0, a.reg_r0), r1 = std::min(p.h0 + p.h, a.reg_r1);
      const int c0 = std::max(p.i0, a.reg_c0), c1 = std::min(p.i0 + p.s, a.reg_c1);
      if (r0 >= r1 || c0 >= c1) continue;
      by0 = std::min(by0, (r0 - a.reg_r0) / kTile);
      by1 = std::max(by1, (r1 - 1 - a.reg_r0) / kTile);
      bx0 = std::min(bx0, (c0 - a.reg_c0) / kTile);
      bx1 = std::max(bx1, (c1 - 1 - a.reg_c0) / kTile);
      whole |= r0 == a.reg_r0 && r1 == a.reg_r1 && c0 == a.reg_c0 && c1 == a.reg_c1;
    }
    if (bx1 >= 0) {
      a.tile_bx0 = bx0;
      a.tile_by0 = by0;
      a.tiles_x = bx1 - bx0 + 1;
      a.n_tile_blocks = a.tiles_x * (by1 - by0 + 1);
      // one slice covering the whole region: every chunk is in a tile
      if (whole) a.stream_chunks = 0;
    }
  }
  const int64_t blocks = a.n_tile_blocks + cdiv((int64_t)a.stream_chunks, 256);
  dim3 grid((unsigned)blocks, 1, (unsigned)nlayers);
  if (graft_dtype == GLT_DTYPE_F32)
    GLT_LAUNCH("bake", bake_kernel<float>, grid, dim3(256), 0, st, a);
  else
    GLT_LAUNCH("bake", bake_kernel<uint16_t>, grid, dim3(256), 0, st, a);
  GLT_LAUNCH_CHECK("bake");
  return GLT_OK;
}

}  // namespace glt

using namespace glt;

extern "C" glt_status glt_shadow_bake(const glt_bake_desc* d, glt_model_state* state, void* const* gate,
                                      void* const* up, void* const* down, void* const* gate_out,
                                      void* const* up_out, void* const* down_out, void* stream) {
  GLT_CHECK(d && state, GLT_ERR_INVALID_ARG, "glt_shadow_bake: null descriptor/state");
  GLT_CHECK(!state->baked, GLT_ERR_ALREADY_BAKED,
            "glt_shadow_bake: model already baked (a second bake would add the grafts twice)");
  GLT_CHECK(d->mode == GLT_BAKE_IN_PLACE || d->mode == GLT_BAKE_MATERIALIZE, GLT_ERR_INVALID_ARG,
            "glt_shadow_bake: mode %d", d->mode);
  GLT_CHECK(d->graft_dtype == GLT_DTYPE_F32 || d->graft_dtype == GLT_DTYPE_BF16, GLT_ERR_DTYPE,
            "glt_shadow_bake: graft dtype %d", d->graft_dtype);
  GLT_CHECK(d->num_layers >= 0 && d->D > 0 && d->I >= 0 && d->n_slices >= 0 && d->n_slices <= kMaxBakeSlices,
            GLT_ERR_SHAPE, "glt_shadow_bake: bad dims (layers=%d D=%d I=%d slices=%d, max slices %d)",
            d->num_layers, d->D, d->I, d->n_slices, kMaxBakeSlices);
  GLT_CHECK(d->proj_mask >= 0 && d->proj_mask <= GLT_PROJ_MASK_ALL, GLT_ERR_INVALID_ARG,
            "glt_shadow_bake: proj_mask %d", d->proj_mask);
  const bool mat = d->mode == GLT_BAKE_MATERIALIZE;
  const int N = mat ? d->N : d->I;
  GLT_CHECK(N >= d->I, GLT_ERR_SHAPE, "glt_shadow_bake: N=%d < I=%d", N, d->I);
  GLT_CHECK(d->n_slices == 0 || (d->placement && d->graft), GLT_ERR_INVALID_ARG,
            "glt_shadow_bake: null placement/graft");
  for (int j = 0; j < d->n_slices; ++j) {
    const int32_t* p = d->placement + 4 * j;
    GLT_CHECK(p[0] >= 0 && p[1] > 0 && p[2] >= 0 && p[3] > 0 && p[0] + p[1] <= N && p[2] + p[3] <= d->D,
              GLT_ERR_SHAPE, "glt_shadow_bake: slice %d {i0=%d S=%d h0=%d H=%d} outside [%d x %d]", j, p[0],
              p[1], p[2], p[3], N, d->D);
  }
  void* const* bases[3] = {gate, up, down};
  void* const* outs[3] = {gate_out, up_out, down_out};
  const int lo = d->layer_start < 0 ? 0 : d->layer_start;
  const int hi = d->layer_end >= d->num_layers ? d->num_layers - 1 : d->layer_end;
  for (int p = 0; p < 3; ++p) {
    if (!(d->proj_mask & (1 << p))) continue;
    GLT_CHECK(bases[p], GLT_ERR_INVALID_ARG, "glt_shadow_bake: null base array for projection %d", p);
    GLT_CHECK(!mat || outs[p], GLT_ERR_INVALID_ARG, "glt_shadow_bake: null output array for projection %d", p);
    for (int l = lo; l <= hi; ++l) {
      GLT_CHECK(bases[p][l] && (!mat || outs[p][l]), GLT_ERR_INVALID_ARG,
                "glt_shadow_bake: null matrix (projection %d layer %d)", p, l);
      for (int j = 0; j < d->n_slices; ++j)
        GLT_CHECK(d->graft[(int64_t)j * d->num_layers + l], GLT_ERR_INVALID_ARG,
                  "glt_shadow_bake: null graft (slice %d layer %d)", j, l);
    }
  }

  hipStream_t st = as_stream(stream);
  const size_t esz = d->graft_dtype == GLT_DTYPE_F32 ? 4 : 2;
  for (int p = 0; p < 3; ++p) {
    if (!(d->proj_mask & (1 << p))) continue;
    const bool trans = p == GLT_PROJ_DOWN;
    // In place, each slice's block is its own region (one launch per slice so
    // that a tile never adds another slice twice); materialised, all slices
    // go through one pass over the whole output.
    const int passes = mat ? 1 : d->n_slices;
    for (int pass = 0; pass < passes; ++pass) {
      for (int l0 = lo; l0 <= hi; l0 += kMaxLayers) {
        BakeLaunch a = {};
        a.trans = trans;
        a.src_rows = trans ? d->D : d->I;
        a.src_cols = trans ? d->I : d->D;
        a.src_ld = trans ? d->I : d->D;
        a.dst_ld = mat ? (trans ? N : d->D) : a.src_ld;
        const int j0 = mat ? 0 : pass, j1 = mat ? d->n_slices : pass + 1;
        a.nslices = j1 - j0;
        for (int j = j0; j < j1; ++j) {
          const int32_t* q = d->placement + 4 * j;
          a.pl[j - j0] = BakePlacement{q[0], q[1], q[2], q[3]};
        }
        if (mat) {
          a.reg_r0 = 0; a.reg_c0 = 0;
          a.reg_r1 = trans ? d->D : N;
          a.reg_c1 = trans ? N : d->D;
        } else {
          const BakePlacement q = a.pl[0];
          a.reg_r0 = trans ? q.h0 : q.i0;
          a.reg_r1 = trans ? q.h0 + q.h : q.i0 + q.s;
          a.reg_c0 = trans ? q.i0 : q.h0;
          a.reg_c1 = trans ? q.i0 + q.s : q.h0 + q.h;
        }
        int n = 0;
        for (int l = l0; l <= hi && n < kMaxLayers; ++l, ++n) {
          a.src[n] = static_cast<const uint16_t*>(bases[p][l]);
          a.dst[n] = static_cast<uint16_t*>(mat ? outs[p][l] : bases[p][l]);
          for (int j = j0; j < j1; ++j)
            a.graft[n][j - j0] = static_cast<const char*>(d->graft[(int64_t)j * d->num_layers + l]) +
                                 (size_t)p * a.pl[j - j0].s * a.pl[j - j0].h * esz;
        }
        glt_status s = launch_bake(a, n, d->graft_dtype, st);
        if (s != GLT_OK) return s;
      }
    }
  }
  state->baked = 1;
  return GLT_OK;
}
