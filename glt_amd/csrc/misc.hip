// Library info, error text, conversions, synthetic inputs, transposes,
// graft mirror packing and the unfused elementwise probes.
#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "common.hpp"
#include "layout.hpp"

namespace glt {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

glt_status hip_fail(hipError_t e, const char* what) {
  set_error("%s failed: %s", what, hipGetErrorString(e));
  return GLT_ERR_HIP;
}

// ------------------------------------------------------------ f32 -> bf16
__global__ void __launch_bounds__(256) f32_to_bf16_kernel(const float* __restrict__ in,
                                                          uint16_t* __restrict__ out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x * 4;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < n; i += stride) {
    if (i + 4 <= n && ((reinterpret_cast<uintptr_t>(in + i) | reinterpret_cast<uintptr_t>(out + i)) & 7) == 0 &&
        (reinterpret_cast<uintptr_t>(in + i) & 15) == 0) {
      f32x4 v = *reinterpret_cast<const f32x4*>(in + i);
      u32x2 o;
      o.x = pack_bf16x2(v.x, v.y);
      o.y = pack_bf16x2(v.z, v.w);
      *reinterpret_cast<u32x2*>(out + i) = o;
    } else {
      for (int64_t j = i; j < n && j < i + 4; ++j) out[j] = f32_to_bf16(in[j]);
    }
  }
}

static int grid_for(int64_t work_items, int per_block = 256) {
  int64_t b = cdiv(work_items, per_block);
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return static_cast<int>(b);
}

// -------------------------------------------------------- normal generator
// Counter-based: value i of tensor (seed, tensor_id) depends only on i.
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void __launch_bounds__(256) fill_normal_kernel(void* out, int dtype, int64_t n,
                                                          uint64_t key, double mean, double stdev) {
  const int64_t npairs = (n + 1) / 2;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < npairs; p += stride) {
    const uint64_t r1 = splitmix64(key + 2 * (uint64_t)p);
    const uint64_t r2 = splitmix64(key + 2 * (uint64_t)p + 1);
    const double u1 = (double)((r1 >> 11) + 1) * 0x1.0p-53;  // (0, 1]
    const double u2 = (double)(r2 >> 11) * 0x1.0p-53;        // [0, 1)
    const double rad = sqrt(-2.0 * log(u1));
    const double th = 6.283185307179586 * u2;
    const float z0 = (float)(mean + stdev * (rad * cos(th)));
    const float z1 = (float)(mean + stdev * (rad * sin(th)));
    const int64_t i = 2 * p;
    if (dtype == GLT_DTYPE_F32) {
      float* o = static_cast<float*>(out);
      o[i] = z0;
      if (i + 1 < n) o[i + 1] = z1;
    } else {
      uint16_t* o = static_cast<uint16_t*>(out);
      o[i] = f32_to_bf16(z0);
      if (i + 1 < n) o[i + 1] = f32_to_bf16(z1);
    }
  }
}

// ---------------------------------------------------------------- transpose
// dst[c, r] = convert(src[r, c]) for a rows x cols source, through a 64x64
// LDS tile (f32 staging, padded row to avoid bank conflicts).
template <typename Tin, typename Tout>
__device__ __forceinline__ Tout cvt(Tin v);
template <> __device__ __forceinline__ float cvt<float, float>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t cvt<uint16_t, uint16_t>(uint16_t v) { return v; }
template <> __device__ __forceinline__ uint16_t cvt<float, uint16_t>(float v) { return f32_to_bf16(v); }

template <typename Tin, typename Tout>
__global__ void __launch_bounds__(256) transpose_kernel(const Tin* __restrict__ src,
                                                        Tout* __restrict__ dst, int rows,
                                                        int cols, int64_t src_ld) {
  __shared__ Tin tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = r0 + ty + 4 * i, c = c0 + tx;
    if (r < rows && c < cols) tile[ty + 4 * i][tx] = src[(int64_t)r * src_ld + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int c = c0 + ty + 4 * i, r = r0 + tx;  // output row c, output col r
    if (c < cols && r < rows) dst[(int64_t)c * rows + r] = cvt<Tin, Tout>(tile[tx][ty + 4 * i]);
  }
}

// bf16 transposes of whole 64 x 64 tiles, one tile per wavefront, no LDS,
// several independent matrices per launch (job j owns tiles
// [tile0[j], tile0[j+1])). Lane (cb = lane & 7, kb = lane >> 3) owns the
// 8 x 8 sub-block at source rows 8 kb .. +7 and columns 8 cb .. +7: it
// loads the eight 16-byte row pieces (each load instruction covers eight
// whole 128-byte lines), transposes the block in registers with byte
// permutes, and stores eight 16-byte pieces of output rows 8 cb .. +7
// (again eight whole lines per instruction).
struct T16Batch {
  int n;
  int64_t tile0[kMaxT16Jobs + 1];
  const uint16_t* src[kMaxT16Jobs];
  uint16_t* dst[kMaxT16Jobs];
  int rows[kMaxT16Jobs], cols[kMaxT16Jobs];
  int64_t ld[kMaxT16Jobs];
};

__global__ void __launch_bounds__(256) transpose16_kernel(const T16Batch bt) {
  const int lane = threadIdx.x & 63;
  int64_t tile = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tile >= bt.tile0[bt.n]) return;
  int j = 0;
  while (j + 1 < bt.n && tile >= bt.tile0[j + 1]) ++j;
  j = __builtin_amdgcn_readfirstlane(j);
  tile -= bt.tile0[j];
  const uint16_t* __restrict__ src = bt.src[j];
  uint16_t* __restrict__ dst = bt.dst[j];
  const int rows = bt.rows[j], tcols = bt.cols[j] / 64;
  const int64_t src_ld = bt.ld[j];
  const int r0 = (int)(tile / tcols) * 64, c0 = (int)(tile % tcols) * 64;
  const int cb = lane & 7, kb = lane >> 3;
  u32x4 in[8];
#pragma unroll
  for (int r = 0; r < 8; ++r)
    in[r] = *reinterpret_cast<const u32x4*>(src + (int64_t)(r0 + 8 * kb + r) * src_ld + c0 + 8 * cb);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    // output word w of column c = (row 2w, row 2w+1) halves c & 1 of word c / 2
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = __builtin_amdgcn_perm(in[2 * w + 1][c >> 1], in[2 * w][c >> 1], sel);
    *reinterpret_cast<u32x4*>(dst + (int64_t)(c0 + 8 * cb + c) * rows + r0 + 8 * kb) = o;
  }
}

static bool t16_ok(const void* src, const void* dst, int rows, int cols, int64_t src_ld) {
  const bool al = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
  return al && rows % 64 == 0 && cols % 64 == 0 && src_ld % 8 == 0;
}

glt_status transpose_any(const void* src, void* dst, int rows, int cols, int64_t src_ld, int dtype,
                         hipStream_t st);

glt_status transpose16_batch(const T16Job* jobs, int n, hipStream_t st) {
  GLT_CHECK(n >= 0 && n <= kMaxT16Jobs, GLT_ERR_INVALID_ARG, "transpose16_batch: %d jobs", n);
  T16Batch bt{};
  bt.n = n;
  int64_t tiles = 0;
  for (int j = 0; j < n; ++j) {
    const T16Job& J = jobs[j];
    GLT_CHECK(t16_ok(J.src, J.dst, J.rows, J.cols, J.src_ld), GLT_ERR_SHAPE,
              "transpose16_batch: job %d is not whole aligned 64 x 64 tiles", j);
    bt.tile0[j] = tiles;
    bt.src[j] = static_cast<const uint16_t*>(J.src);
    bt.dst[j] = static_cast<uint16_t*>(J.dst);
    bt.rows[j] = J.rows;
    bt.cols[j] = J.cols;
    bt.ld[j] = J.src_ld;
    tiles += (int64_t)(J.rows / 64) * (J.cols / 64);
  }
  bt.tile0[n] = tiles;
  if (tiles == 0) return GLT_OK;
  GLT_CHECK(tiles < (1ll << 33), GLT_ERR_SHAPE, "transpose16_batch: %lld tiles", (long long)tiles);
  GLT_LAUNCH("transpose16", transpose16_kernel, dim3((unsigned)cdiv(tiles, 4)), dim3(256), 0, st, bt);
  GLT_LAUNCH_CHECK("transpose16");
  return GLT_OK;
}

glt_status transpose_batch(const T16Job* jobs, int n, int dtype, hipStream_t st) {
  bool fast = dtype == GLT_DTYPE_BF16;
  for (int j = 0; fast && j < n; ++j) fast = t16_ok(jobs[j].src, jobs[j].dst, jobs[j].rows, jobs[j].cols, jobs[j].src_ld);
  if (fast) return transpose16_batch(jobs, n, st);
  for (int j = 0; j < n; ++j) {
    const glt_status s = transpose_any(jobs[j].src, jobs[j].dst, jobs[j].rows, jobs[j].cols, jobs[j].src_ld, dtype, st);
    if (s != GLT_OK) return s;
  }
  return GLT_OK;
}

template <typename Tin, typename Tout>
static glt_status launch_transpose(const Tin* src, Tout* dst, int rows, int cols, int64_t src_ld,
                                   hipStream_t st) {
  if (rows == 0 || cols == 0) return GLT_OK;
  if constexpr (sizeof(Tin) == 2 && sizeof(Tout) == 2) {
    if (t16_ok(src, dst, rows, cols, src_ld)) {
      const T16Job job{src, dst, rows, cols, src_ld};
      return transpose16_batch(&job, 1, st);
    }
  }
  dim3 grid((unsigned)cdiv(cols, 64), (unsigned)cdiv(rows, 64));
  GLT_LAUNCH("transpose", (transpose_kernel<Tin, Tout>), grid, dim3(256), 0, st, src, dst, rows, cols, src_ld);
  GLT_LAUNCH_CHECK("transpose");
  return GLT_OK;
}

// dst [cols, rows] (contiguous) = transpose of a rows x cols block whose rows
// are src_ld elements apart.
glt_status transpose_any(const void* src, void* dst, int rows, int cols, int64_t src_ld, int dtype,
                         hipStream_t st) {
  if (dtype == GLT_DTYPE_F32)
    return launch_transpose(static_cast<const float*>(src), static_cast<float*>(dst), rows, cols, src_ld, st);
  return launch_transpose(static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), rows, cols, src_ld,
                          st);
}

glt_status transpose_f32_to_bf16(const float* src, uint16_t* dst, int rows, int cols, hipStream_t st) {
  return launch_transpose(src, dst, rows, cols, (int64_t)cols, st);
}

glt_status convert_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t st) {
  if (n == 0) return GLT_OK;
  GLT_LAUNCH("f32_to_bf16", f32_to_bf16_kernel, dim3(grid_for(cdiv(n, 4))), dim3(256), 0, st, in, out, n);
  GLT_LAUNCH_CHECK("f32_to_bf16");
  return GLT_OK;
}

glt_status pack_projection(const float* master, int S, int H, int proj, uint16_t* packed, hipStream_t st) {
  const int64_t sh = (int64_t)S * H;
  uint16_t* rm = packed + 2 * proj * sh;
  glt_status s;
  if ((s = convert_f32_to_bf16(master, rm, sh, st)) != GLT_OK) return s;
  if ((s = transpose_f32_to_bf16(master, rm + sh, S, H, st)) != GLT_OK) return s;
  if ((s = shuffle_b(master, GLT_DTYPE_F32, H, false, S, H, packed + packed_shuf_offset(S, H, 2 * proj), st)) !=
      GLT_OK)
    return s;
  return shuffle_b(master, GLT_DTYPE_F32, H, true, H, S, packed + packed_shuf_offset(S, H, 2 * proj + 1), st);
}

// ------------------------------------------------------ elementwise probes
// silu(g)*u with the reference's f32 operation order
// (reference src/kernels_elementwise_impl.inc:395-401): sg = 1/(1+exp(-g)),
// out = bf16((g*sg)*u).
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint16_t* __restrict__ g,
                                                       const uint16_t* __restrict__ u,
                                                       uint16_t* __restrict__ out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gp = bf16_to_f32(g[i]);
    const float uv = bf16_to_f32(u[i]);
    const float sg = 1.0f / (1.0f + expf(-gp));
    out[i] = f32_to_bf16(gp * sg * uv);
  }
}

// (reference src/kernels_elementwise_impl.inc:107-117)
__global__ void __launch_bounds__(256) gate_up_bwd_kernel(const float* __restrict__ gi,
                                                          const uint16_t* __restrict__ g,
                                                          const uint16_t* __restrict__ u,
                                                          float* __restrict__ dg,
                                                          float* __restrict__ du, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gp = bf16_to_f32(g[i]);
    const float uv = bf16_to_f32(u[i]);
    const float sg = 1.0f / (1.0f + expf(-gp));
    const float gv = gp * sg;
    const float silu_grad = sg * (1.0f + gp * (1.0f - sg));
    const float giv = gi[i];
    dg[i] = giv * uv * silu_grad;
    du[i] = giv * gv;
  }
}

}  // namespace glt

using namespace glt;

extern "C" {

int32_t glt_version(void) { return GLT_ABI_VERSION; }

const char* glt_last_error_string(void) { return g_err; }

glt_status glt_device_info(int32_t device, int32_t* cu_count, int32_t* clock_mhz, int64_t* hbm_bytes) {
  hipDeviceProp_t p;
  GLT_TRY_HIP(hipGetDeviceProperties(&p, device));
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (clock_mhz) *clock_mhz = p.clockRate / 1000;
  if (hbm_bytes) *hbm_bytes = (int64_t)p.totalGlobalMem;
  return GLT_OK;
}

glt_status glt_f32_to_bf16(const float* in, uint16_t* out, int64_t n, void* stream) {
  GLT_CHECK(n >= 0, GLT_ERR_SHAPE, "glt_f32_to_bf16: n < 0");
  GLT_CHECK(n == 0 || (in && out), GLT_ERR_INVALID_ARG, "glt_f32_to_bf16: null pointer");
  return convert_f32_to_bf16(in, out, n, as_stream(stream));
}

glt_status glt_fill_normal(void* out, int32_t dtype, int64_t n, uint64_t seed, uint64_t tensor_id,
                           double mean, double stdev, void* stream) {
  GLT_CHECK(n >= 0, GLT_ERR_SHAPE, "glt_fill_normal: n < 0");
  GLT_CHECK(n == 0 || out, GLT_ERR_INVALID_ARG, "glt_fill_normal: null pointer");
  GLT_CHECK(dtype == GLT_DTYPE_F32 || dtype == GLT_DTYPE_BF16, GLT_ERR_DTYPE, "glt_fill_normal: dtype");
  if (n == 0) return GLT_OK;
  const uint64_t key = splitmix64(seed ^ splitmix64(tensor_id + 0x632BE59BD9B4E019ull));
  GLT_LAUNCH("fill_normal", fill_normal_kernel, dim3(grid_for(cdiv(n, 2))), dim3(256), 0, as_stream(stream),
                     out, dtype, n, key, mean, stdev);
  GLT_LAUNCH_CHECK("fill_normal");
  return GLT_OK;
}

glt_status glt_transpose(const void* src, void* dst, int32_t rows, int32_t cols, int32_t dtype,
                         void* stream) {
  GLT_CHECK(rows >= 0 && cols >= 0, GLT_ERR_SHAPE, "glt_transpose: negative shape");
  GLT_CHECK((rows == 0 || cols == 0) || (src && dst), GLT_ERR_INVALID_ARG, "glt_transpose: null pointer");
  GLT_CHECK(dtype == GLT_DTYPE_F32 || dtype == GLT_DTYPE_BF16, GLT_ERR_DTYPE, "glt_transpose: dtype");
  return transpose_any(src, dst, rows, cols, cols, dtype, as_stream(stream));
}

size_t glt_graft_packed_size(int32_t S, int32_t H) {
  if (S <= 0 || H <= 0) return 0;
  return (size_t)packed_bytes(S, H);
}

glt_status glt_graft_pack(const glt_graft_slice* sl, uint16_t* packed, void* stream) {
  GLT_CHECK(sl && packed, GLT_ERR_INVALID_ARG, "glt_graft_pack: null pointer");
  GLT_CHECK(sl->s > 0 && sl->h > 0, GLT_ERR_SHAPE, "glt_graft_pack: empty slice");
  GLT_CHECK((reinterpret_cast<uintptr_t>(packed) & 255) == 0, GLT_ERR_ALIGNMENT,
            "glt_graft_pack: packed buffer must be 256-byte aligned");
  const float* masters[3] = {sl->master_gate, sl->master_up, sl->master_down};
  hipStream_t st = as_stream(stream);
  for (int p = 0; p < 3; ++p) {
    if (!masters[p]) continue;
    glt_status s = pack_projection(masters[p], sl->s, sl->h, p, packed, st);
    if (s != GLT_OK) return s;
  }
  return GLT_OK;
}

glt_status glt_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n, void* stream) {
  GLT_CHECK(n >= 0, GLT_ERR_SHAPE, "glt_silu_mul: n < 0");
  GLT_CHECK(n == 0 || (g && u && out), GLT_ERR_INVALID_ARG, "glt_silu_mul: null pointer");
  if (n == 0) return GLT_OK;
  GLT_LAUNCH("silu_mul", silu_mul_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), g, u, out, n);
  GLT_LAUNCH_CHECK("silu_mul");
  return GLT_OK;
}

glt_status glt_gate_up_bwd(const float* gi, const uint16_t* g, const uint16_t* u, float* dg, float* du,
                           int64_t n, void* stream) {
  GLT_CHECK(n >= 0, GLT_ERR_SHAPE, "glt_gate_up_bwd: n < 0");
  GLT_CHECK(n == 0 || (gi && g && u && dg && du), GLT_ERR_INVALID_ARG, "glt_gate_up_bwd: null pointer");
  if (n == 0) return GLT_OK;
  GLT_LAUNCH("gate_up_bwd", gate_up_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), gi, g, u, dg,
                     du, n);
  GLT_LAUNCH_CHECK("gate_up_bwd");
  return GLT_OK;
}

}  // extern "C"
