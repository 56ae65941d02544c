// Projections with FP8 block-scaled weights: y = x W^T, W = fp16(w8 * s).
//
// The reference keeps its FP8 checkpoint weights (float8_e4m3fn with one
// fp32 `weight_scale_inv` per 128x128 block) and dequantises each projection
// once to fp16 (v2/src/router_ia/qwen36_dequant.py:35-58, then `.to(float16)`
// at qwen36_cached_loop.py:537-542), then runs fp16 F.linear on fp16
// activations (qwen36_attention_cache.py:232-247, 268-276, 295-301, 318-320).
//
// Here the weights stay FP8 in HBM (half the bytes of the fp16 copy) and
// are dequantised in registers to the very fp16 values the reference
// computes (fp32 product, one rounding to fp16), then multiplied on fp16
// MFMA with fp32 accumulation; the result is rounded to fp16 like
// F.linear's fp16 output.
//
//   dequant_fp8_kernel   W16 = fp16(w8 * s) as a tensor (the reference's
//                        dequantised weight; also feeds a library GEMM for
//                        long prompts)
//   linear_fp8_kernel    one workgroup per (16 or 32 output features,
//                        128-row block of x); 4 waves, 32 rows of x each.
//                        Weight chunks (the tile's rows x 128 K = one scale
//                        block) stream through an 8-deep register ring, are
//                        dequantised into an fp16 B-operand buffer in LDS
//                        (double-buffered), and every wave runs 16x16x32 f16
//                        MFMAs over its rows with x operands loaded one chunk
//                        ahead.  Decode-sized M is bound by the weight stream.
#include <algorithm>

#include "ria_common.h"

namespace ria {

constexpr int kFp8Block = 128;  // scale block edge (qwen36_dequant.py:13)
constexpr int kLinRing = 8;     // weight chunks in flight per workgroup
constexpr int kLinRows = 128;   // rows of x per workgroup (4 waves x 32)

// Two fp8 e4m3 (OCP, float8_e4m3fn) bytes of `w` (low pair or high pair) to fp32.
template <bool HIGH>
__device__ __forceinline__ f32x2 fp8x2_to_f32(uint32_t w) {
  const auto v = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), HIGH);
  return f32x2{v[0], v[1]};
}

// fp16 bits of (fp32(w8) * s): the reference's `weight.float() * scale` rounded by `.to(float16)`.
template <bool HIGH>
__device__ __forceinline__ uint32_t dequant_pair(uint32_t w, float s) {
  const f32x2 f = fp8x2_to_f32<HIGH>(w);
  const _Float16 a = static_cast<_Float16>(mul_rn(f[0], s));
  const _Float16 b = static_cast<_Float16>(mul_rn(f[1], s));
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

// One thread per 16 weight bytes of a row (K a multiple of 16).
template <int OT>
__global__ __launch_bounds__(256) void dequant_fp8_kernel(const uint8_t* __restrict__ w, const float* __restrict__ scale,
                                                          int64_t rows, int k, int scale_cols, void* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte unit
  const int per_row = k / 16;
  if (i >= rows * per_row) return;
  const int64_t r = i / per_row;
  const int c = static_cast<int>(i - r * per_row) * 16;
  const float s = scale[(r / kFp8Block) * scale_cols + c / kFp8Block];
  const u32x4 v = *reinterpret_cast<const u32x4*>(w + r * k + c);
  float x[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x2 f0 = fp8x2_to_f32<false>(v[q]), f1 = fp8x2_to_f32<true>(v[q]);
    x[4 * q] = mul_rn(f0[0], s);
    x[4 * q + 1] = mul_rn(f0[1], s);
    x[4 * q + 2] = mul_rn(f1[0], s);
    x[4 * q + 3] = mul_rn(f1[1], s);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) y[j] = x[4 * q + j];
    store_act4<OT>(out, r * k + c + 4 * q, y);
  }
}

struct LinearArgs {
  const void* x;
  int64_t x_stride;
  const uint8_t* w;     // [N, K] e4m3
  const float* scale;   // [ceil(N / 128), scale_cols]
  int scale_cols;
  void* y;
  int64_t y_stride;
  int m, n, k;
};

// x operand of one 16x16x32 MFMA: 8 consecutive K values of one row as fp16.
template <int XT>
__device__ __forceinline__ u32x4 load_x8(const void* x, int64_t i) {
  if constexpr (XT == RIA_DT_F16) {
    return *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + i);
  } else {
    float f[8];
    load_act8<XT>(x, i, f);  // the reference's activation.to(float16)
    uint32_t p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = Kv16<RIA_DT_F16>::pack2(f[2 * j], f[2 * j + 1]);
    return u32x4{p[0], p[1], p[2], p[3]};
  }
}

template <int XT, int OT, int CT>
__global__ __launch_bounds__(256) void linear_fp8_kernel(LinearArgs a) {
  using F16 = Kv16<RIA_DT_F16>;
  constexpr int kCols = 16 * CT;          // output features per workgroup
  constexpr int kLoaders = kCols * 8;     // threads holding 16 weight bytes of a chunk
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n16 = lane & 15, g4 = lane >> 4;
  const int n0 = blockIdx.x * kCols;
  const int m0 = blockIdx.y * kLinRows;
  const int rows = min(kLinRows, a.m - m0);
  const int chunks = a.k / kFp8Block;
  const int nb = n0 / kFp8Block;  // the tile lies in one scale block of rows

  // fp16 B operands of one chunk: [k-step 4][col tile CT][lane 64] x 16 bytes, double-buffered
  __shared__ u32x4 bop[2][4 * CT * 64];

  // weight bytes of this thread in every chunk: row n0 + wr, bytes 16 wk .. + 15 of the chunk
  const int wr = tid >> 3, wk = tid & 7;
  const bool loader = tid < kLoaders;
  const uint8_t* wrow = a.w + (int64_t)(n0 + (loader ? wr : 0)) * a.k + 16 * wk;
  // where its 16 values land: k-step wk / 2, k groups 2 (wk % 2) and + 1, column tile wr / 16
  const int s_of = wk >> 1, g_of = 2 * (wk & 1), c_of = wr >> 4, lane0 = (wr & 15) + 16 * g_of;

  u32x4 ring[kLinRing];
#pragma unroll
  for (int u = 0; u < kLinRing; ++u)
    if (loader) ring[u] = *reinterpret_cast<const u32x4*>(wrow + (int64_t)min(u, chunks - 1) * kFp8Block);

  // this wave's rows: 32 wave .. + 31 (two row tiles); rows past the end repeat the last one
  const bool has_rows0 = 32 * wave < rows, has_rows1 = 32 * wave + 16 < rows;
  const int r0 = min(32 * wave + n16, rows - 1), r1 = min(32 * wave + 16 + n16, rows - 1);
  const int64_t xo0 = (int64_t)(m0 + r0) * a.x_stride + 8 * g4, xo1 = (int64_t)(m0 + r1) * a.x_stride + 8 * g4;
  u32x4 ax[2][4][2];  // x operands of two chunks: [buffer][k-step][row tile]
  auto load_x = [&](int c, u32x4 (&dst)[4][2]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      dst[s][0] = load_x8<XT>(a.x, xo0 + c * kFp8Block + 32 * s);
      dst[s][1] = load_x8<XT>(a.x, xo1 + c * kFp8Block + 32 * s);
    }
  };
  load_x(0, ax[0]);

  f32x4 acc[2][CT];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // chunks run in groups of kLinRing so the ring index is static (and, the
  // group size being even, so is the parity of c that picks the buffers)
  static_assert(kLinRing % 2 == 0, "buffer parity must follow the ring index");
  for (int c0 = 0; c0 < chunks; c0 += kLinRing) {
#pragma unroll
    for (int u = 0; u < kLinRing; ++u) {
      const int c = c0 + u;
      if (c >= chunks) break;
      const int buf = u & 1;
      // dequantise this thread's 16 bytes into the B operands of chunk c
      if (loader) {
        const float sc = a.scale[nb * a.scale_cols + c];
        const u32x4 v = ring[u];
        const u32x4 lo{dequant_pair<false>(v[0], sc), dequant_pair<true>(v[0], sc), dequant_pair<false>(v[1], sc),
                       dequant_pair<true>(v[1], sc)};
        const u32x4 hi{dequant_pair<false>(v[2], sc), dequant_pair<true>(v[2], sc), dequant_pair<false>(v[3], sc),
                       dequant_pair<true>(v[3], sc)};
        bop[buf][(s_of * CT + c_of) * 64 + lane0] = lo;
        bop[buf][(s_of * CT + c_of) * 64 + lane0 + 16] = hi;
        ring[u] = *reinterpret_cast<const u32x4*>(wrow + (int64_t)min(c + kLinRing, chunks - 1) * kFp8Block);
      }
      if (c + 1 < chunks) load_x(c + 1, ax[(u + 1) & 1]);
      __syncthreads();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        u32x4 b[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) b[ct] = bop[buf][(s * CT + ct) * 64 + lane];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          if (has_rows0) acc[0][ct] = F16::mfma_k32(ax[buf][s][0], b[ct], acc[0][ct]);
          if (has_rows1) acc[1][ct] = F16::mfma_k32(ax[buf][s][1], b[ct], acc[1][ct]);
        }
      }
    }
  }

  // D tile rows 4 g4 + i, column n16; F.linear's fp16 result, stored as OT
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 32 * wave + 16 * rt + 4 * g4 + i;
        if (r < rows)
          store_act<OT>(a.y, (int64_t)(m0 + r) * a.y_stride + n0 + 16 * ct + n16,
                        through_dtype<RIA_DT_F16>(acc[rt][ct][i]));
      }
}

template <int XT, int OT>
static void launch_linear_ct(const LinearArgs& a, int ct, dim3 grid, hipStream_t st) {
  if (ct == 2)
    hipLaunchKernelGGL((linear_fp8_kernel<XT, OT, 2>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((linear_fp8_kernel<XT, OT, 1>), grid, dim3(256), 0, st, a);
}

template <int XT>
static void launch_linear_ot(const LinearArgs& a, int out_dtype, int ct, dim3 grid, hipStream_t st) {
  if (out_dtype == RIA_DT_BF16)
    launch_linear_ct<XT, RIA_DT_BF16>(a, ct, grid, st);
  else if (out_dtype == RIA_DT_F16)
    launch_linear_ct<XT, RIA_DT_F16>(a, ct, grid, st);
  else
    launch_linear_ct<XT, RIA_DT_F32>(a, ct, grid, st);
}

static bool lin_dtype_ok(int dt) { return dt == RIA_DT_BF16 || dt == RIA_DT_F16 || dt == RIA_DT_F32; }

}  // namespace ria

using namespace ria;

extern "C" int ria_dequant_fp8(int64_t rows, int cols, const void* weight, const float* scale_inv, void* out,
                               int out_dtype, void* stream) {
  if (rows < 0 || cols <= 0 || cols % 16) return set_error(RIA_ERR_INVALID, "ria_dequant_fp8: cols must be a positive multiple of 16");
  if (!lin_dtype_ok(out_dtype)) return set_error(RIA_ERR_INVALID, "ria_dequant_fp8: unknown dtype code");
  if (rows == 0) return RIA_OK;
  if (!weight || !scale_inv || !out) return set_error(RIA_ERR_INVALID, "ria_dequant_fp8: null pointer");
  if ((reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(out)) % 16)
    return set_error(RIA_ERR_INVALID, "ria_dequant_fp8: weight and out must be 16-byte aligned");
  const int64_t units = rows * (cols / 16);
  const int64_t blocks = (units + 255) / 256;
  if (blocks > 0x7fffffff) return set_error(RIA_ERR_INVALID, "ria_dequant_fp8: too large");
  const int scale_cols = (cols + kFp8Block - 1) / kFp8Block;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(blocks));
  const uint8_t* w = static_cast<const uint8_t*>(weight);
  if (out_dtype == RIA_DT_F16)
    hipLaunchKernelGGL((dequant_fp8_kernel<RIA_DT_F16>), grid, dim3(256), 0, st, w, scale_inv, rows, cols, scale_cols, out);
  else if (out_dtype == RIA_DT_BF16)
    hipLaunchKernelGGL((dequant_fp8_kernel<RIA_DT_BF16>), grid, dim3(256), 0, st, w, scale_inv, rows, cols, scale_cols, out);
  else
    hipLaunchKernelGGL((dequant_fp8_kernel<RIA_DT_F32>), grid, dim3(256), 0, st, w, scale_inv, rows, cols, scale_cols, out);
  return check_launch("ria_dequant_fp8");
}

extern "C" int ria_linear_fp8(int m, int n, int k, const void* x, int x_dtype, int64_t x_row_stride,
                              const void* weight, const float* scale_inv, void* y, int y_dtype, int64_t y_row_stride,
                              void* stream) {
  if (m < 0 || n <= 0 || k <= 0) return set_error(RIA_ERR_INVALID, "ria_linear_fp8: bad sizes");
  if (n % 16 || k % kFp8Block)
    return set_error(RIA_ERR_INVALID, "ria_linear_fp8: N must be a multiple of 16 and K of 128 (got %d, %d)", n, k);
  if (!lin_dtype_ok(x_dtype) || !lin_dtype_ok(y_dtype)) return set_error(RIA_ERR_INVALID, "ria_linear_fp8: unknown dtype code");
  if (m == 0) return RIA_OK;
  if (!x || !weight || !scale_inv || !y) return set_error(RIA_ERR_INVALID, "ria_linear_fp8: null pointer");
  if (x_row_stride < k || y_row_stride < n) return set_error(RIA_ERR_INVALID, "ria_linear_fp8: row stride too small");
  // x moves in 16-byte (fp16/bf16) or 32-byte (fp32) vectors of 8 elements
  if (reinterpret_cast<uintptr_t>(x) % 16 || x_row_stride % 8 || reinterpret_cast<uintptr_t>(weight) % 16)
    return set_error(RIA_ERR_INVALID, "ria_linear_fp8: x and weight 16-byte aligned, x row stride a multiple of 8");
  LinearArgs a{};
  a.x = x;
  a.x_stride = x_row_stride;
  a.w = static_cast<const uint8_t*>(weight);
  a.scale = scale_inv;
  a.scale_cols = k / kFp8Block;
  a.y = y;
  a.y_stride = y_row_stride;
  a.m = m;
  a.n = n;
  a.k = k;
  // 32 output features per workgroup when that still gives a workgroup per CU, else 16
  const int ct = (n % 32 == 0 && n / 32 >= 256) ? 2 : 1;
  const int64_t mblocks = (m + kLinRows - 1) / kLinRows;
  if (mblocks > 65535) return set_error(RIA_ERR_INVALID, "ria_linear_fp8: too many rows");
  const dim3 grid(static_cast<unsigned>(n / (16 * ct)), static_cast<unsigned>(mblocks));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == RIA_DT_F16)
    launch_linear_ot<RIA_DT_F16>(a, y_dtype, ct, grid, st);
  else if (x_dtype == RIA_DT_BF16)
    launch_linear_ot<RIA_DT_BF16>(a, y_dtype, ct, grid, st);
  else
    launch_linear_ot<RIA_DT_F32>(a, y_dtype, ct, grid, st);
  return check_launch("ria_linear_fp8");
}
