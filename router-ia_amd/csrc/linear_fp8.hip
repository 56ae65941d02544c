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
//                        128-row block of x).  Weight chunks (the tile's rows
//                        x 128 K = one scale block) stream through an 8-deep
//                        register ring in four producer waves, are dequantised
//                        into an fp16 B-operand buffer in LDS (double-
//                        buffered), and four consumer waves (32 rows of x
//                        each) run 16x16x32 f16 MFMAs with x operands loaded
//                        one chunk ahead.  Decode-sized M is bound by the
//                        weight stream.  Used past 16 rows for fp32 x.
//   linear_fp8_ks_kernel past 16 rows with fp16 or bf16 x (the forward loop's
//                        projections): one workgroup per tile of rows x
//                        features over the whole K, split between its waves;
//                        operands loaded row-contiguous into registers and
//                        turned into MFMA operands through each wave's own
//                        LDS region.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "ria_common.h"

namespace ria {

constexpr int kFp8Block = 128;  // scale block edge (qwen36_dequant.py:13)
constexpr int kLinRing = 12;    // weight chunks in flight per workgroup
constexpr int kXAhead = 2;      // chunks of x loaded ahead of the MFMAs
constexpr int kLinRows = 128;   // most rows of x per workgroup (4 consumer waves x 32)

// Two fp8 e4m3 (OCP, float8_e4m3fn) bytes of `w` (low pair or high pair) to fp32.
template <bool HIGH>
__device__ __forceinline__ f32x2 fp8x2_to_f32(uint32_t w) {
  const auto v = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), HIGH);
  return f32x2{v[0], v[1]};
}

// fp16 bits of (fp32(w8) * s): the reference's `weight.float() * scale` rounded by `.to(float16)`.
// (two fp32 products, then one packed round-to-nearest conversion to fp16)
template <bool HIGH>
__device__ __forceinline__ uint32_t dequant_pair(uint32_t w, float s) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const f32x2 f = fp8x2_to_f32<HIGH>(w);
  h2 r;
  r[0] = static_cast<_Float16>(mul_rn(f[0], s));
  r[1] = static_cast<_Float16>(mul_rn(f[1], s));
  return __builtin_bit_cast(uint32_t, r);
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

// Up to kLinGroup projections of the same x in one launch (a layer's input
// projections read the same normed hidden state); column tiles of projection
// j are blockIdx.x = tile0[j] .. tile0[j + 1] - 1.
constexpr int kLinGroup = 4;
constexpr int kLinMaxChunks = 256;  // K <= 32768: the tile's scale row is staged in LDS

struct Fp8Proj {
  const uint8_t* w;     // [n, K] e4m3
  const float* scale;   // [ceil(n / 128), K / 128]
  void* y;              // [m, n], rows y_stride elements apart
  int64_t y_stride;
  int n;
  int y_dtype;          // RIA_DT_*: y holds the fp16 result in this dtype
  int y_add;            // nonzero: y (fp32) += the result, the residual add of a layer output
  int tile0;            // first column tile of this projection
};

struct LinearArgs {
  const void* x;
  int64_t x_stride;
  int m, k, count;
  int mt;               // rows of x per workgroup (streaming kernel): 64 or 128
  const float* norm_w;  // fused input RMSNorm (one-pass kernel, up to 4 rows of fp32 x), or null
  float norm_eps;
  int norm_dtype;       // the normed rows are rounded to this dtype, then to fp16
  Fp8Proj p[kLinGroup];
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

// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>): a loop the
// compiler must unroll, so register arrays indexed by the counter stay in
// registers (a rolled loop would move them to scratch memory).
template <typename F, int... U>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, U...>) {
  (f(std::integral_constant<int, U>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// One producer thread's weight bytes of a chunk: 8 (CT 1), 16 (CT 2) or 32 (CT 4).
template <int CT>
struct WeightSlot {
  u32x4 v[CT / 2];
  __device__ __forceinline__ void load(const uint8_t* p) {
#pragma unroll
    for (int q = 0; q < CT / 2; ++q) v[q] = *reinterpret_cast<const u32x4*>(p + 16 * q);
  }
  __device__ __forceinline__ uint32_t word(int i) const { return v[i >> 2][i & 3]; }
};
template <>
struct WeightSlot<1> {
  u32x2 v;
  __device__ __forceinline__ void load(const uint8_t* p) { v = *reinterpret_cast<const u32x2*>(p); }
  __device__ __forceinline__ uint32_t word(int i) const { return v[i]; }
};

// Producer / consumer waves.  A wave's vector-memory counter retires loads in
// issue order, so a wave that both streamed weights far ahead and loaded x
// for the next chunk would have to wait for every weight load issued before
// that x.  Here waves 4-7 only stream weights (an 8-chunk register ring,
// dequantised into the B buffer) and waves 0-3 only load x and run the MFMAs;
// one LDS-only barrier per chunk hands each B buffer over.
//
// Both loops run whole groups of kLinRing chunks with no exit inside (the
// ring slot u is a compile-time index), then the K % (128 kLinRing) tail:
// an exit inside the ring loop makes the compiler join the ring registers
// at each exit, which waits for every weight load in flight.
template <int XT, int CT>
__global__ __launch_bounds__(512) void linear_fp8_kernel(const LinearArgs a) {
  using F16 = Kv16<RIA_DT_F16>;
  constexpr int kCols = 16 * CT;             // output features per workgroup
  constexpr int kBytes = CT * 8;             // weight bytes per producer thread per chunk
  constexpr int kWords = CT * 2;             // .. as 32-bit words
  using Ring = WeightSlot<CT>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, so role branches are scalar
  const int n16 = lane & 15, g4 = lane >> 4;
  const int bx = blockIdx.x;
  // this workgroup's projection: scalar selects over the group
  const uint8_t* w = a.p[0].w;
  const float* scale = a.p[0].scale;
  void* y = a.p[0].y;
  int64_t y_stride = a.p[0].y_stride;
  int n = a.p[0].n, y_dtype = a.p[0].y_dtype, y_add = a.p[0].y_add, tile0 = 0;
#pragma unroll
  for (int j = 1; j < kLinGroup; ++j)
    if (j < a.count && bx >= a.p[j].tile0) {
      w = a.p[j].w;
      scale = a.p[j].scale;
      y = a.p[j].y;
      y_stride = a.p[j].y_stride;
      n = a.p[j].n;
      y_dtype = a.p[j].y_dtype;
      y_add = a.p[j].y_add;
      tile0 = a.p[j].tile0;
    }
  const int n0 = (bx - tile0) * kCols;
  const int m0 = blockIdx.y * a.mt;
  const int rows = min(a.mt, a.m - m0);
  const int chunks = a.k / kFp8Block;
  const int groups = chunks / kLinRing, tail = chunks - groups * kLinRing;

  // fp16 B operands of one chunk: [k-step 4][col tile CT][lane 64] x 16 bytes, double-buffered
  __shared__ u32x4 bop[2][4 * CT * 64];
  __shared__ float sc_s[kLinMaxChunks];  // scale of each chunk (the tile lies in one block of 128 rows)

  // the ring slot u also picks the B buffer (u % 2) and the x buffer
  // (u % (kXAhead + 1)); both must repeat with each group of kLinRing chunks
  static_assert(kLinRing % 2 == 0 && kLinRing % (kXAhead + 1) == 0, "buffers must follow the ring slot");
  if (wave >= 4) {
    // ---- producers: bytes kBytes * pk .. of row n0 + pr in every chunk
    const int p = tid - 256;
    const int pr = p / (128 / kBytes), pk = p % (128 / kBytes);
    // (features past n, in the last tile of a projection narrower than the
    // tile, repeat row n - 1: their columns are computed and not stored)
    const uint8_t* wrow = w + (int64_t)min(n0 + pr, n - 1) * a.k + kBytes * pk;
    // those values are 16 B (CT 2) or 8 B (CT 1) of K at k-step s, k groups g ..
    const int kofs = kBytes * pk, s_of = kofs >> 5, g_of = (kofs & 31) >> 3;
    const int slot = (s_of * CT + (pr >> 4)) * 64 + (pr & 15) + 16 * g_of;
    // the tile's scale row (threads past the row repeat its last entry): loaded
    // before the weight ring, so the wait for it does not wait for the ring
    const int sp = min(p, chunks - 1);
    const float sc0 = scale[(n0 / kFp8Block) * chunks + sp];
    __builtin_amdgcn_sched_barrier(0);
    Ring ring[kLinRing];
    static_for<kLinRing>([&](auto u) { ring[u].load(wrow + (int64_t)min(int(u), chunks - 1) * kFp8Block); });
    sc_s[sp] = sc0;
    lds_barrier();  // sc_s is written
    auto produce = [&](auto u, int c) {
      const float sc = sc_s[c];
      // the thread's bytes are k groups g_of .. g_of + CT - 1 of k-step s_of: 8 fp16 values each
#pragma unroll
      for (int q = 0; q < kWords / 2; ++q) {
        const uint32_t w0 = ring[u].word(2 * q), w1 = ring[u].word(2 * q + 1);
        bop[u & 1][slot + 16 * q] = u32x4{dequant_pair<false>(w0, sc), dequant_pair<true>(w0, sc),
                                          dequant_pair<false>(w1, sc), dequant_pair<true>(w1, sc)};
      }
    };
    for (int gi = 0; gi < groups; ++gi) {
      static_for<kLinRing>([&](auto u) {
        const int c = gi * kLinRing + u;
        produce(u, c);
        // keep the reload after the dequantisation, so it refills ring[u]'s own registers
        __builtin_amdgcn_sched_barrier(0);
        ring[u].load(wrow + (int64_t)min(c + kLinRing, chunks - 1) * kFp8Block);
        lds_barrier();
      });
    }
    static_for<kLinRing>([&](auto u) {
      if (u < tail) {
        produce(u, groups * kLinRing + u);
        lds_barrier();
      }
    });
    return;
  }

  // ---- consumers: rows 32 wave .. + 31 (two row tiles); rows past the end repeat the last one
  const int r0 = min(32 * wave + n16, rows - 1), r1 = min(32 * wave + 16 + n16, rows - 1);
  const int64_t xo0 = (int64_t)(m0 + r0) * a.x_stride + 8 * g4, xo1 = (int64_t)(m0 + r1) * a.x_stride + 8 * g4;
  // The number of row tiles this wave computes is fixed outside the chunk
  // loop (one loop copy per count), so the loop body has no branch: a branch
  // around the MFMAs would make the compiler wait for the next chunk's x too.
  auto consume = [&](auto tiles) {
    constexpr int NT = decltype(tiles)::value;
    u32x4 ax[kXAhead + 1][4][2];  // x operands of the chunks in flight: [buffer][k-step][row tile]
    auto load_x = [&](int c, u32x4 (&dst)[4][2]) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if constexpr (NT >= 1) dst[s][0] = load_x8<XT>(a.x, xo0 + c * kFp8Block + 32 * s);
        if constexpr (NT >= 2) dst[s][1] = load_x8<XT>(a.x, xo1 + c * kFp8Block + 32 * s);
      }
    };
#pragma unroll
    for (int j = 0; j < kXAhead; ++j) load_x(min(j, chunks - 1), ax[j]);
    f32x4 acc[2][CT];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    lds_barrier();  // the producers' sc_s
    auto step = [&](auto u, int c) {
      load_x(min(c + kXAhead, chunks - 1), ax[(u + kXAhead) % (kXAhead + 1)]);  // past the end: reloads
      lds_barrier();  // B operands of chunk c are in bop[u & 1]
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        u32x4 b[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) b[ct] = bop[u & 1][(s * CT + ct) * 64 + lane];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int rt = 0; rt < NT; ++rt)
            acc[rt][ct] = F16::mfma_k32(ax[u % (kXAhead + 1)][s][rt], b[ct], acc[rt][ct]);
      }
    };
    for (int gi = 0; gi < groups; ++gi) static_for<kLinRing>([&](auto u) { step(u, gi * kLinRing + u); });
    static_for<kLinRing>([&](auto u) {
      if (u < tail) step(u, groups * kLinRing + u);
    });
    // D tile rows 4 g4 + i, column n16; F.linear's fp16 result, stored as
    // y_dtype or (y_add) added to the fp32 y.  The y values an add needs are
    // all loaded before the first store: a store between them would make each
    // load wait for the one before (the compiler cannot tell they never
    // overlap).  Whole tiles (the usual case) store with no per-element
    // branch, which would make the compiler wait for every memory operation
    // before each store.
    auto y_index = [&](int rt, int ct, int i) {
      return (int64_t)(m0 + 32 * wave + 16 * rt + 4 * g4 + i) * y_stride + n0 + 16 * ct + n16;
    };
    auto in_range = [&](int rt, int ct, int i) {
      return 32 * wave + 16 * rt + 4 * g4 + i < rows && n0 + 16 * ct + n16 < n;
    };
    auto finish = [&](auto whole) {
      constexpr bool W = decltype(whole)::value;
      if (y_add) {
        float* yf = static_cast<float*>(y);
        float v[2][CT][4];
#pragma unroll
        for (int rt = 0; rt < NT; ++rt)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[rt][ct][i] = W || in_range(rt, ct, i) ? yf[y_index(rt, ct, i)] : 0.f;
#pragma unroll
        for (int rt = 0; rt < NT; ++rt)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              v[rt][ct][i] = add_rn(v[rt][ct][i], through_dtype<RIA_DT_F16>(acc[rt][ct][i]));
              if (W || in_range(rt, ct, i)) yf[y_index(rt, ct, i)] = v[rt][ct][i];
            }
      } else {
#pragma unroll
        for (int rt = 0; rt < NT; ++rt)
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (W || in_range(rt, ct, i))
                store_act_dt(y, y_index(rt, ct, i), through_dtype<RIA_DT_F16>(acc[rt][ct][i]), y_dtype);
      }
    };
    if (32 * wave + 16 * NT <= rows && n0 + 16 * CT <= n)
      finish(std::true_type{});
    else
      finish(std::false_type{});
  };
  if (32 * wave + 16 < rows)
    consume(std::integral_constant<int, 2>{});
  else if (32 * wave < rows)
    consume(std::integral_constant<int, 1>{});
  else
    consume(std::integral_constant<int, 0>{});  // no rows: only keeps the barriers in step
}

// Decode-sized M (up to 16 rows): one workgroup per 16 output features and
// 16 rows of x, one wave per 512 K.  A wave issues every load it needs at once
// (its x operands, then 16 rows x 512 bytes of weight: 8 loads of 16 bytes a
// lane), so the whole weight matrix is in flight with no ring and no LDS
// handoff; it then dequantises in registers and runs 16 MFMAs (x as the A
// operand, rows = tokens; weights as B, columns = features).  A lane's 16
// weight bytes at K = 64 j + 16 g .. + 15 feed two MFMAs (low 8 bytes to step
// 2 j, high 8 to 2 j + 1, k group g of each); x uses the same K order, so each
// MFMA sums 32 matching products.  The waves' partial sums are added in wave
// order through LDS.
constexpr int kGemvSlice = 512;  // K per wave
constexpr int kGemvRows = 16;    // rows of x per workgroup
constexpr int kGemvMaxWaves = 8; // K <= 4096
constexpr int kGemvStageRows = 4; // x rows staged through LDS

template <int XT, bool NORM>
__global__ __launch_bounds__(64 * kGemvMaxWaves) void gemv_fp8_kernel(const LinearArgs a) {
  static_assert(!NORM || XT == RIA_DT_F32, "the fused norm reads the fp32 residual stream");
  using F16 = Kv16<RIA_DT_F16>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = a.k / kGemvSlice;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int bx = blockIdx.x;
  const uint8_t* w = a.p[0].w;
  const float* scale = a.p[0].scale;
  void* y = a.p[0].y;
  int64_t y_stride = a.p[0].y_stride;
  int y_dtype = a.p[0].y_dtype, y_add = a.p[0].y_add, tile0 = 0;
#pragma unroll
  for (int j = 1; j < kLinGroup; ++j)
    if (j < a.count && bx >= a.p[j].tile0) {
      w = a.p[j].w;
      scale = a.p[j].scale;
      y = a.p[j].y;
      y_stride = a.p[j].y_stride;
      y_dtype = a.p[j].y_dtype;
      y_add = a.p[j].y_add;
      tile0 = a.p[j].tile0;
    }
  const int n0 = (bx - tile0) * 16;
  const int m0 = blockIdx.y * kGemvRows;
  const int rows = min(kGemvRows, a.m - m0);
  const int k0 = wave * kGemvSlice;

  const uint8_t* wp = w + (int64_t)(n0 + c16) * a.k + k0 + 16 * g4;
  const float* sp = scale + (n0 / kFp8Block) * (a.k / kFp8Block) + k0 / kFp8Block;
  // The loads of x go first, so that waiting for them leaves the weight loads
  // in flight.  Up to kGemvStageRows rows, a lane loads 16 bytes of one row
  // (one instruction per row for the wave's 1 KB slice) and the slice goes
  // through the wave's own LDS region into the MFMA layout: far fewer load
  // instructions than the layout's 16 per wave, whose issue time (not their
  // bytes) would otherwise delay the weight stream.  Lanes of rows past the
  // last token repeat its x.
  // LDS (sized at launch): per wave max(staged rows, 1) x 1 KB; the first
  // KB of a wave's region later holds its partial sums
  extern __shared__ u32x4 gemv_lds[];
  const int region = 64 * (rows <= kGemvStageRows ? rows : 1);
  u32x4* own = gemv_lds + wave * region;
  u32x4 ax[8][2];
  u32x4 wv[8];
  float sc[4];
  auto load_w = [&] {
#pragma unroll
    for (int j = 0; j < 8; ++j) wv[j] = *reinterpret_cast<const u32x4*>(wp + 64 * j);
    // the slice's four scales (one per 128 K; the 16 features lie in one block of 128)
#pragma unroll
    for (int b = 0; b < 4; ++b) sc[b] = sp[b];
  };
  // NR rows staged (NR = rows, 1 .. kGemvStageRows; the count is a template
  // constant so the loads are straight-line code), or NR = 0: direct loads
  auto load_operands = [&](auto nr) {
    constexpr int NR = decltype(nr)::value;
    if constexpr (NR > 0) {
      u32x4 xs[NR];
      if constexpr (NORM) {
        // h = rmsnorm(x) (1 + w) over the whole row, rounded to norm_dtype, then
        // to fp16 (qwen36_attention_cache.py:227-233, 291-293): each wave sums
        // the squares of its 512 K, the waves' sums meet in LDS (added in wave
        // order), and every wave normalises its own slice.
        f32x4 xf[NR][2];
        const f32x4* xp = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.x) + k0 + 8 * lane);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          xf[r][0] = xp[(m0 + r) * a.x_stride / 4];
          xf[r][1] = xp[(m0 + r) * a.x_stride / 4 + 1];
        }
        const f32x4* wn = reinterpret_cast<const f32x4*>(a.norm_w + k0 + 8 * lane);
        const f32x4 nw0 = wn[0], nw1 = wn[1];
        load_w();
        __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait
        __shared__ float norm_ss[kGemvMaxWaves][kGemvStageRows];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          float ss = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) ss = add_rn(ss, mul_rn(xf[r][0][i], xf[r][0][i]));
#pragma unroll
          for (int i = 0; i < 4; ++i) ss = add_rn(ss, mul_rn(xf[r][1][i], xf[r][1][i]));
          ss = wave_sum(ss);
          if (lane == 0) norm_ss[wave][r] = ss;
        }
        lds_barrier();
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          float tot = 0.f;
          for (int q = 0; q < waves; ++q) tot += norm_ss[q][r];
          const float rs = rms_scale(tot, a.k, a.norm_eps);
          float hv[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            hv[i] = rmsnorm_elem<RIA_DT_F32>(xf[r][0][i], rs, nw0[i]);
            hv[4 + i] = rmsnorm_elem<RIA_DT_F32>(xf[r][1][i], rs, nw1[i]);
          }
#pragma unroll
          for (int i = 0; i < 8; ++i)
            hv[i] = a.norm_dtype == RIA_DT_BF16 ? through_dtype<RIA_DT_BF16>(hv[i]) : hv[i];
          uint32_t pk[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) pk[j] = F16::pack2(hv[2 * j], hv[2 * j + 1]);
          xs[r] = u32x4{pk[0], pk[1], pk[2], pk[3]};
        }
      } else {
#pragma unroll
        for (int r = 0; r < NR; ++r) xs[r] = load_x8<XT>(a.x, (int64_t)(m0 + r) * a.x_stride + k0 + 8 * lane);
        load_w();
        __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait
      }
#pragma unroll
      for (int r = 0; r < NR; ++r) own[64 * r + lane] = xs[r];
      __builtin_amdgcn_wave_barrier();  // the region is this wave's: LDS keeps its order
      // MFMA rows past the last token repeat its x: D row m depends on A row m
      // alone, and only rows below NR are stored, so they need no zeroing
      const int r = min(c16, NR - 1);
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) ax[j][h] = own[64 * r + 8 * j + 2 * g4 + h];  // K = 64 j + 16 g4 + 8 h
    } else {
      // rows past the last token re-read it (see above: their D rows are not stored)
      const int64_t xo = (int64_t)(m0 + min(c16, rows - 1)) * a.x_stride + k0 + 16 * g4;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ax[j][0] = load_x8<XT>(a.x, xo + 64 * j);
        ax[j][1] = load_x8<XT>(a.x, xo + 64 * j + 8);
      }
      load_w();
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  static_assert(kGemvStageRows == 4, "one case per staged row count");
  switch (rows) {
    case 1: load_operands(std::integral_constant<int, 1>{}); break;
    case 2: load_operands(std::integral_constant<int, 2>{}); break;
    case 3: load_operands(std::integral_constant<int, 3>{}); break;
    case 4: load_operands(std::integral_constant<int, 4>{}); break;
    default:
      if constexpr (!NORM) load_operands(std::integral_constant<int, 0>{});  // the host keeps NORM to 4 rows
      break;
  }

  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float s = sc[j >> 1];
    const u32x4 v = wv[j];
    const u32x4 b0{dequant_pair<false>(v[0], s), dequant_pair<true>(v[0], s), dequant_pair<false>(v[1], s),
                   dequant_pair<true>(v[1], s)};
    const u32x4 b1{dequant_pair<false>(v[2], s), dequant_pair<true>(v[2], s), dequant_pair<false>(v[3], s),
                   dequant_pair<true>(v[3], s)};
    acc[0] = F16::mfma_k32(ax[j][0], b0, acc[0]);
    acc[1] = F16::mfma_k32(ax[j][1], b1, acc[1]);
  }
  f32x4 part;
#pragma unroll
  for (int i = 0; i < 4; ++i) part[i] = acc[0][i] + acc[1][i];

  // (the MFMAs consumed this wave's staged x before its partial sums overwrite it)
  reinterpret_cast<f32x4*>(own)[lane] = part;
  lds_barrier();
  if (wave == 0) {
    f32x4 t = reinterpret_cast<const f32x4*>(gemv_lds)[lane];
    for (int q = 1; q < waves; ++q) {
      const f32x4 u = reinterpret_cast<const f32x4*>(gemv_lds + q * region)[lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] += u[i];
    }
    // D rows (tokens) 4 g4 + i, column (feature) c16; F.linear's fp16 result,
    // stored as y_dtype or added to the fp32 y (every y load before the first store)
    if (y_add) {
      float* yf = static_cast<float*>(y);
      float prev[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        prev[i] = 4 * g4 + i < rows ? yf[(int64_t)(m0 + 4 * g4 + i) * y_stride + n0 + c16] : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) prev[i] = add_rn(prev[i], through_dtype<RIA_DT_F16>(t[i]));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * g4 + i < rows) yf[(int64_t)(m0 + 4 * g4 + i) * y_stride + n0 + c16] = prev[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * g4 + i < rows)
          store_act_dt(y, (int64_t)(m0 + 4 * g4 + i) * y_stride + n0 + c16, through_dtype<RIA_DT_F16>(t[i]), y_dtype);
    }
  }
}

// Past 16 rows with fp16 x, or bf16 x (XB) converted to fp16 as it goes into
// LDS: one workgroup per tile of 16 RT rows x 16 CT
// features over the whole of K, whose NW waves split K between them: wave w
// takes the 64-K chunks w, w + NW, w + 2 NW, ...  Each wave loads its own x
// and weight bytes into registers, D chunks deep, with row-contiguous loads
// (a few cache lines per load), passes each chunk through its own LDS region
// to turn the rows into MFMA operands (no barrier in the loop: every byte the
// workgroup needs is loaded once, by one wave), dequantises each weight once
// and feeds it to RT MFMAs.  The waves' partial tiles meet in LDS at the end
// and are added in wave order.  K order inside a chunk: a lane's 16 weight
// bytes at K = 64 c + 16 g .. + 15 feed two MFMAs (the low 8 bytes the first,
// the high 8 the second, as k group g of each), and its x operands take the
// same K.  CH > 0: every wave has exactly CH chunks (K = 64 NW CH), unrolled;
// CH = 0: any K, in groups of D chunks.
constexpr int kKsChunk = 64;

// Eight bf16 values as eight fp16 values (round to nearest even: exact
// within fp16's normal range), as F.linear's x.to(float16) gives them.
__device__ __forceinline__ u32x4 bf16x8_to_f16x8(u32x4 v) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h2 p;
    p[0] = static_cast<_Float16>(__uint_as_float(v[j] << 16));
    p[1] = static_cast<_Float16>(__uint_as_float(v[j] & 0xffff0000u));
    r[j] = __builtin_bit_cast(uint32_t, p);
  }
  return r;
}

template <int RT, int CT, int NW, int D, int CH, bool XB = false>
__global__ __launch_bounds__(64 * NW) void linear_fp8_ks_kernel(const LinearArgs a) {
  using F16 = Kv16<RIA_DT_F16>;
  static_assert(kFp8Block % (16 * CT) == 0, "a tile's features lie in one scale block");
  static_assert((RT * CT) % NW == 0, "the waves share the tiles of the epilogue evenly");
  constexpr int kTiles = RT * CT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, g4 = lane >> 4;
  const int bx = blockIdx.x;
  const uint8_t* w = a.p[0].w;
  const float* scale = a.p[0].scale;
  void* y = a.p[0].y;
  int64_t y_stride = a.p[0].y_stride;
  int n = a.p[0].n, y_dtype = a.p[0].y_dtype, y_add = a.p[0].y_add, tile0 = 0;
#pragma unroll
  for (int j = 1; j < kLinGroup; ++j)
    if (j < a.count && bx >= a.p[j].tile0) {
      w = a.p[j].w;
      scale = a.p[j].scale;
      y = a.p[j].y;
      y_stride = a.p[j].y_stride;
      n = a.p[j].n;
      y_dtype = a.p[j].y_dtype;
      y_add = a.p[j].y_add;
      tile0 = a.p[j].tile0;
    }
  const int n0 = (bx - tile0) * 16 * CT;
  const int m0 = blockIdx.y * 16 * RT;
  const int chunks = a.k / kKsChunk;
  const int cnt = (chunks - wave + NW - 1) / NW;  // this wave's chunks (0 when K has fewer than NW)
  // Operands come through buffer loads: a per-lane byte offset fixed for the
  // kernel plus the chunk's offset in a scalar register, so a load costs no
  // address arithmetic.  Byte offsets fit 32 bits (checked on the host).
  // Rows past the last token and features past n repeat the last one: their
  // results are computed and never stored.  The loads walk along the rows
  // (x: load j holds rows 8 j .. 8 j + 7, lane l row 8 j + l / 8, 16-byte
  // piece l % 8; weights: load ct holds the 16 rows of column tile ct, lane l
  // row l / 4, piece l % 4), so every load covers whole row segments of a few
  // cache lines, and the wave's own LDS region turns the pieces into MFMA
  // operands (lane (n16, g4): row n16, K pieces 2 g4 and 2 g4 + 1 of x, piece
  // g4 of the weights; the two K orders agree, so each product pairs the
  // right elements).
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(a.x), 0, static_cast<int>(static_cast<uint32_t>(((int64_t)(a.m - 1) * a.x_stride + a.k) * 2)), kBufferWord3);
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w), 0, static_cast<int>(static_cast<uint32_t>((int64_t)n * a.k)), kBufferWord3);
  uint32_t xo[2 * RT], wo[CT];
#pragma unroll
  for (int j = 0; j < 2 * RT; ++j)
    xo[j] = static_cast<uint32_t>((min(m0 + 8 * j + (lane >> 3), a.m - 1) * a.x_stride + 8 * (lane & 7)) * 2);
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
    wo[ct] = static_cast<uint32_t>(min(n0 + 16 * ct + (lane >> 2), n - 1) * a.k + 16 * (lane & 3));
  const float* sp = scale + (int64_t)(n0 / kFp8Block) * (a.k / kFp8Block);
  auto bload = [](__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  };

  struct Stage {
    u32x4 x[RT][2];  // the 2 RT row-contiguous x loads, in order
    u32x4 w[CT];
    float s;
  };
  Stage st[D];
  // chunk i of this wave into s (past the wave's last chunk: the last one again, never used)
  auto load = [&](Stage& s, int i) __attribute__((always_inline)) {
    const int c = wave + NW * min(i, cnt - 1);
    const int ko = c * kKsChunk;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      s.x[rt][0] = bload(xr, xo[2 * rt], 2 * ko);
      s.x[rt][1] = bload(xr, xo[2 * rt + 1], 2 * ko);
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) s.w[ct] = bload(wr, wo[ct], ko);
    s.s = sp[c * kKsChunk / kFp8Block];
  };
  // The wave's LDS region, 16-byte entries.  x: block (row tile rt, piece q)
  // of 16 entries, tile row r at entry r ^ hx(q); weights: block (column tile
  // ct, piece p), tile row r at entry r ^ hw(p).  The
  // XOR patterns make every group of 8 or 16 consecutive lanes hit distinct
  // entries modulo 8 or 16 for the stores (x: 8 lanes per row, 2 rows per 16
  // lanes; weights: 4 lanes per row) and for the operand reads (16 rows of
  // one piece), so neither side has bank conflicts.  The wave writes a chunk
  // and reads it back in its own order (LDS operations of one wave complete
  // in order), so one region per wave is enough.
  auto hx = [](int q) { return q ^ ((q & 1) << 3); };
  auto hw = [](int p) { return (p << 1) | ((p & 1) << 3); };
  constexpr int kLtX = RT * 8 * 16, kLtW = CT * 4 * 16;  // entries
  constexpr int kPartBytes = NW * kTiles * 64 * 16;
  constexpr int kLtBytes = NW * (kLtX + kLtW) * 16;
  __shared__ __attribute__((aligned(16))) unsigned char ks_lds[kPartBytes > kLtBytes ? kPartBytes : kLtBytes];
  u32x4* lt = reinterpret_cast<u32x4*>(ks_lds) + wave * (kLtX + kLtW);
  auto operands = [&](const Stage& s, u32x4 (&xa)[RT][2], u32x4 (&wb)[CT]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2 * RT; ++j) {
      const int r = 8 * j + (lane >> 3), q = lane & 7;  // tile row r % 16 of row tile r / 16
      const u32x4 xv = s.x[j >> 1][j & 1];
      lt[((r >> 4) * 8 + q) * 16 + ((r & 15) ^ hx(q))] = XB ? bf16x8_to_f16x8(xv) : xv;
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int r = lane >> 2, p = lane & 3;
      lt[kLtX + (ct * 4 + p) * 16 + (r ^ hw(p))] = s.w[ct];
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int q = 2 * g4 + h;
        xa[rt][h] = lt[(rt * 8 + q) * 16 + (n16 ^ hx(q))];
      }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) wb[ct] = lt[kLtX + (ct * 4 + g4) * 16 + (n16 ^ hw(g4))];
  };
  f32x4 acc[RT][CT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (cnt > 0) {
    static_for<D - 1>([&](auto u) { load(st[u], u); });
    // chunk i sits in slot i % D; step i refills the slot chunk i - 1 left
    // with chunk i + D - 1.  The scheduling barrier keeps the refill loads
    // ahead of the MFMAs (the scheduler would otherwise sink each load next
    // to its use, which leaves one chunk in flight).
    auto step = [&](auto u, auto i, bool refill) __attribute__((always_inline)) {
      if (refill) load(st[(u + D - 1) % D], i + D - 1);
      __builtin_amdgcn_sched_barrier(0);
      const Stage& s = st[u];
      u32x4 xa[RT][2], wb[CT];
      operands(s, xa, wb);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const u32x4 v = wb[ct];
        const u32x4 b0{dequant_pair<false>(v[0], s.s), dequant_pair<true>(v[0], s.s), dequant_pair<false>(v[1], s.s),
                       dequant_pair<true>(v[1], s.s)};
        const u32x4 b1{dequant_pair<false>(v[2], s.s), dequant_pair<true>(v[2], s.s), dequant_pair<false>(v[3], s.s),
                       dequant_pair<true>(v[3], s.s)};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = F16::mfma_k32(xa[rt][0], b0, acc[rt][ct]);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[rt][ct] = F16::mfma_k32(xa[rt][1], b1, acc[rt][ct]);
      }
    };
    if constexpr (CH > 0) {
      // CH chunks per wave, straight-line code: a loop would join the ring's
      // loads at its head, where the compiler waits for every load in flight
      static_for<CH>([&](auto i) {
        step(std::integral_constant<int, i % D>{}, i, i + D - 1 < CH);
      });
    } else {
      const int groups = cnt / D, tail = cnt - groups * D;
      for (int gi = 0; gi < groups; ++gi) static_for<D>([&](auto u) { step(u, gi * D + u, true); });
      static_for<D>([&](auto u) {
        if (u < tail) step(u, groups * D + u, true);
      });
    }
  }

  // ---- the waves' partial tiles, added in wave order; wave w finishes tiles w, w + NW, ..
  __syncthreads();  // the partial tiles reuse the waves' LDS regions
  auto part = reinterpret_cast<f32x4(*)[kTiles][64]>(ks_lds);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) part[wave][rt * CT + ct][lane] = acc[rt][ct];
  __syncthreads();
  constexpr int TPW = kTiles / NW;
  f32x4 tot[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = wave + NW * j;
    tot[j] = part[0][t][lane];
#pragma unroll
    for (int q = 1; q < NW; ++q) {
      const f32x4 u = part[q][t][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) tot[j][i] += u[i];
    }
  }
  // D tile rows 4 g4 + i, column n16: F.linear's fp16 result, stored as
  // y_dtype or (y_add) added to the fp32 y.  The fp16 values are staged in
  // LDS row by row, then every thread stores whole 4-column pieces of rows
  // (one 8- or 16-byte store instead of four 2- or 4-byte stores to four
  // rows); a y whose rows are not 16-byte aligned takes one value at a time.
  constexpr int kPitch = 16 * CT + 4;  // floats per staged row (conflict-free stores)
  static_assert(16 * RT * kPitch * 4 <= (kPartBytes > kLtBytes ? kPartBytes : kLtBytes), "stage fits the LDS block");
  __syncthreads();  // every wave has read the partial tiles
  float* stg = reinterpret_cast<float*>(ks_lds);
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = wave + NW * j;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      stg[(16 * (t / CT) + 4 * g4 + i) * kPitch + 16 * (t % CT) + n16] = through_dtype<RIA_DT_F16>(tot[j][i]);
  }
  __syncthreads();
  const bool vec = reinterpret_cast<uintptr_t>(y) % 16 == 0 && y_stride % 4 == 0;
  constexpr int kPieces = 16 * RT * 4 * CT;  // 4-column pieces of the tile
#pragma unroll
  for (int pc = tid; pc < kPieces; pc += 64 * NW) {
    const int r = pc / (4 * CT), c = 4 * (pc % (4 * CT));
    const int row = m0 + r, col = n0 + c;
    if (row >= a.m) continue;
    const f32x4 v = *reinterpret_cast<const f32x4*>(stg + r * kPitch + c);
    const int64_t off = (int64_t)row * y_stride + col;
    if (vec && col + 4 <= n) {
      if (y_add) {
        f32x4* yp = reinterpret_cast<f32x4*>(static_cast<float*>(y) + off);
        f32x4 o = *yp;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = add_rn(o[e], v[e]);
        *yp = o;
      } else if (y_dtype == RIA_DT_F32) {
        *reinterpret_cast<f32x4*>(static_cast<float*>(y) + off) = v;
      } else {
        uint32_t w0, w1;
        if (y_dtype == RIA_DT_F16) {
          w0 = f32_to_f16_bits(v[0]) | (uint32_t(f32_to_f16_bits(v[1])) << 16);
          w1 = f32_to_f16_bits(v[2]) | (uint32_t(f32_to_f16_bits(v[3])) << 16);
        } else {
          w0 = f32_to_bf16_bits(v[0]) | (uint32_t(f32_to_bf16_bits(v[1])) << 16);
          w1 = f32_to_bf16_bits(v[2]) | (uint32_t(f32_to_bf16_bits(v[3])) << 16);
        }
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(y) + off) = uint2{w0, w1};
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (col + e >= n) break;
        if (y_add) {
          float* yp = static_cast<float*>(y) + off + e;
          *yp = add_rn(*yp, v[e]);
        } else {
          store_act_dt(y, off + e, v[e], y_dtype);
        }
      }
    }
  }
}

// Tile shapes of the K-split kernels (rows 16 RT, features 16 CT)
struct KsShape {
  int rt, ct;
};
constexpr KsShape kKsShapes[] = {{4, 8}, {4, 4}, {2, 2}};

template <int XT, bool NORM = false>
static void launch_gemv(const LinearArgs& a, dim3 grid, hipStream_t st) {
  const int waves = a.k / kGemvSlice;
  const size_t lds = static_cast<size_t>(waves) * (a.m <= kGemvStageRows ? a.m : 1) * 64 * sizeof(u32x4);
  hipLaunchKernelGGL((gemv_fp8_kernel<XT, NORM>), grid, dim3(64 * waves), lds, st, a);
}

template <int XT>
static void launch_linear(const LinearArgs& a, int ct, dim3 grid, hipStream_t st) {
  if (ct == 4)
    hipLaunchKernelGGL((linear_fp8_kernel<XT, 4>), grid, dim3(512), 0, st, a);
  else if (ct == 2)
    hipLaunchKernelGGL((linear_fp8_kernel<XT, 2>), grid, dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL((linear_fp8_kernel<XT, 1>), grid, dim3(512), 0, st, a);
}

// Every K takes the K-split kernel with four waves,
// straight-line for 8 or 16 chunks per wave (K = 2048, the hidden width, and
// K = 4096, the value width).  The wave count is fixed and every shape runs
// the waves over the same chunks in the same order, so a projection's result
// does not depend on the tile shape chosen for it (grouped and separate
// calls agree bit for bit).
template <int RT, int CT, int D, bool XB>
static void launch_ks_k(const LinearArgs& a, dim3 grid, hipStream_t st) {
  constexpr int NW = 4;
  if (a.k == kKsChunk * NW * 8)
    hipLaunchKernelGGL((linear_fp8_ks_kernel<RT, CT, NW, D, 8, XB>), grid, dim3(64 * NW), 0, st, a);
  else if (a.k == kKsChunk * NW * 16)
    hipLaunchKernelGGL((linear_fp8_ks_kernel<RT, CT, NW, D, 16, XB>), grid, dim3(64 * NW), 0, st, a);
  else
    hipLaunchKernelGGL((linear_fp8_ks_kernel<RT, CT, NW, D, 0, XB>), grid, dim3(64 * NW), 0, st, a);
}

template <bool XB>
static void launch_ks(const LinearArgs& a, KsShape s, dim3 grid, hipStream_t st) {
  if (s.rt == 4 && s.ct == 8)
    launch_ks_k<4, 8, 3, XB>(a, grid, st);
  else if (s.rt == 4 && s.ct == 4)
    launch_ks_k<4, 4, 4, XB>(a, grid, st);
  else
    launch_ks_k<2, 2, 6, XB>(a, grid, st);
}

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
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

// Validates and launches one group of projections of the same x (shared by
// ria_linear_fp8 and ria_linear_fp8_group; `who` names the entry point in errors).
static int linear_group(const char* who, int m, int k, const void* x, int x_dtype, int64_t x_row_stride, int count,
                        const ria_fp8_proj* projs, void* stream, const float* norm_w = nullptr, float norm_eps = 0.f,
                        int norm_dtype = RIA_DT_F16) {
  if (count < 1 || count > kLinGroup) return set_error(RIA_ERR_INVALID, "%s: 1 to %d projections per call", who, kLinGroup);
  if (m < 0 || k <= 0) return set_error(RIA_ERR_INVALID, "%s: bad sizes", who);
  if (k % kFp8Block || k / kFp8Block > kLinMaxChunks)
    return set_error(RIA_ERR_INVALID, "%s: K must be a multiple of 128 up to %d (got %d)", who,
                     kFp8Block * kLinMaxChunks, k);
  if (!lin_dtype_ok(x_dtype)) return set_error(RIA_ERR_INVALID, "%s: unknown dtype code", who);
  if (!projs) return set_error(RIA_ERR_INVALID, "%s: null projection list", who);
  for (int j = 0; j < count; ++j) {
    const ria_fp8_proj& q = projs[j];
    if (q.n <= 0 || q.n % 16)
      return set_error(RIA_ERR_INVALID, "%s: N must be a positive multiple of 16 (projection %d: %d)", who, j, q.n);
    if (q.y_row_stride < q.n) return set_error(RIA_ERR_INVALID, "%s: y row stride too small (projection %d)", who, j);
    if (!lin_dtype_ok(q.y_dtype)) return set_error(RIA_ERR_INVALID, "%s: unknown dtype code (projection %d)", who, j);
    if (q.y_add && q.y_dtype != RIA_DT_F32)
      return set_error(RIA_ERR_INVALID, "%s: y_add needs an fp32 y (projection %d)", who, j);
  }
  if (m == 0) return RIA_OK;
  if (!x) return set_error(RIA_ERR_INVALID, "%s: null x", who);
  if (x_row_stride < k) return set_error(RIA_ERR_INVALID, "%s: x row stride too small", who);
  // x moves in 16-byte (fp16/bf16) or 32-byte (fp32) vectors of 8 elements
  if (reinterpret_cast<uintptr_t>(x) % 16 || x_row_stride % 8)
    return set_error(RIA_ERR_INVALID, "%s: x must be 16-byte aligned with a row stride a multiple of 8", who);
  for (int j = 0; j < count; ++j) {
    const ria_fp8_proj& q = projs[j];
    if (!q.weight || !q.scale_inv || !q.y) return set_error(RIA_ERR_INVALID, "%s: null pointer (projection %d)", who, j);
    if (reinterpret_cast<uintptr_t>(q.weight) % 16)
      return set_error(RIA_ERR_INVALID, "%s: weight must be 16-byte aligned (projection %d)", who, j);
  }
  const bool gemv = m <= kGemvRows && k % kGemvSlice == 0 && k / kGemvSlice <= kGemvMaxWaves;
  if (norm_w) {
    if (!gemv || m > kGemvStageRows)
      return set_error(RIA_ERR_INVALID, "%s: the fused input norm takes up to %d rows and K a multiple of %d up to %d",
                       who, kGemvStageRows, kGemvSlice, kGemvSlice * kGemvMaxWaves);
    if (x_dtype != RIA_DT_F32 || x_row_stride % 4 || reinterpret_cast<uintptr_t>(norm_w) % 16)
      return set_error(RIA_ERR_INVALID, "%s: fused norm: fp32 x with a row stride a multiple of 4, 16-byte aligned "
                       "norm weight", who);
    if (norm_dtype != RIA_DT_BF16 && norm_dtype != RIA_DT_F16)
      return set_error(RIA_ERR_INVALID, "%s: fused norm rounds to bf16 or fp16", who);
  }
  // Streaming kernel: workgroups of mt rows x 16 ct output features.  A
  // workgroup reads its mt rows of x (from L2) and its weights through the
  // CU's L1, whose misses in flight bound the rate, so the shape is the one
  // whose busiest CU moves the fewest bytes: (workgroups per CU) x (x bytes
  // + weight bytes of one workgroup); ties go to more workgroups.
  int ct = 1, mt = kLinRows;
  // K-split kernel (fp16 or bf16 x): the tile shape whose busiest CU moves the
  // fewest bytes, (rounds of workgroups over the CUs) x (x + weight bytes of
  // one tile)
  bool ks = !gemv && (x_dtype == RIA_DT_F16 || x_dtype == RIA_DT_BF16) && (int64_t)m * x_row_stride < (int64_t(1) << 31);
  for (int j = 0; j < count; ++j) ks = ks && (int64_t)projs[j].n * k < (int64_t(1) << 31);
  KsShape ks_shape = kKsShapes[0];
  if (ks) {
    const int cus = device_cus();
    int64_t best = -1;
    for (const KsShape s : kKsShapes) {
      int64_t wgs = 0;
      for (int j = 0; j < count; ++j) wgs += (projs[j].n + 16 * s.ct - 1) / (16 * s.ct);
      wgs *= (m + 16 * s.rt - 1) / (16 * s.rt);
      const int64_t cost = (wgs + cus - 1) / cus * ((int64_t)k * (32 * s.rt + 16 * s.ct));
      if (best < 0 || cost < best) {
        best = cost;
        ks_shape = s;
      }
    }
    ct = ks_shape.ct;
    mt = 16 * ks_shape.rt;
  } else if (!gemv) {
    const int cus = device_cus();
    int64_t best = -1, best_wgs = 0;
    for (const int r : {kLinRows, kLinRows / 2})
      for (const int c : {1, 2, 4}) {
        int64_t wgs = 0;
        for (int j = 0; j < count; ++j) wgs += (projs[j].n + 16 * c - 1) / (16 * c);
        wgs *= (m + r - 1) / r;
        const int64_t per_cu = (wgs + cus - 1) / cus * ((int64_t)std::min(r, m) * k * 2 + (int64_t)16 * c * k);
        if (best < 0 || per_cu < best || (per_cu == best && wgs > best_wgs)) {
          best = per_cu;
          best_wgs = wgs;
          ct = c;
          mt = r;
        }
      }
  }
  LinearArgs a{};
  a.x = x;
  a.x_stride = x_row_stride;
  a.m = m;
  a.k = k;
  a.count = count;
  a.mt = mt;
  a.norm_w = norm_w;
  a.norm_eps = norm_eps;
  a.norm_dtype = norm_dtype;
  int tile = 0;
  for (int j = 0; j < count; ++j) {
    const ria_fp8_proj& q = projs[j];
    a.p[j] = Fp8Proj{static_cast<const uint8_t*>(q.weight), q.scale_inv, q.y, q.y_row_stride, q.n, q.y_dtype, q.y_add,
                     tile};
    tile += (q.n + 16 * ct - 1) / (16 * ct);
  }
  const int64_t mblocks = gemv ? 1 : (m + mt - 1) / mt;
  if (mblocks > 65535) return set_error(RIA_ERR_INVALID, "%s: too many rows", who);
  const dim3 grid(static_cast<unsigned>(tile), static_cast<unsigned>(mblocks));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (norm_w) {
    launch_gemv<RIA_DT_F32, true>(a, grid, st);
  } else if (gemv) {
    if (x_dtype == RIA_DT_F16)
      launch_gemv<RIA_DT_F16>(a, grid, st);
    else if (x_dtype == RIA_DT_BF16)
      launch_gemv<RIA_DT_BF16>(a, grid, st);
    else
      launch_gemv<RIA_DT_F32>(a, grid, st);
  } else if (ks) {
    if (x_dtype == RIA_DT_BF16)
      launch_ks<true>(a, ks_shape, grid, st);
    else
      launch_ks<false>(a, ks_shape, grid, st);
  } else if (x_dtype == RIA_DT_BF16) {
    launch_linear<RIA_DT_BF16>(a, ct, grid, st);
  } else {
    launch_linear<RIA_DT_F32>(a, ct, grid, st);
  }
  return check_launch(who);
}

extern "C" int ria_linear_fp8(int m, int n, int k, const void* x, int x_dtype, int64_t x_row_stride,
                              const void* weight, const float* scale_inv, void* y, int y_dtype, int64_t y_row_stride,
                              void* stream) {
  const ria_fp8_proj p{weight, scale_inv, y, y_row_stride, n, y_dtype, 0};
  return linear_group("ria_linear_fp8", m, k, x, x_dtype, x_row_stride, 1, &p, stream);
}

extern "C" int ria_linear_fp8_group(int m, int k, const void* x, int x_dtype, int64_t x_row_stride, int count,
                                    const ria_fp8_proj* projs, void* stream) {
  return linear_group("ria_linear_fp8_group", m, k, x, x_dtype, x_row_stride, count, projs, stream);
}

extern "C" int ria_linear_fp8_group_normed(int m, int k, const float* x, int64_t x_row_stride,
                                           const float* norm_weight, float eps, int h_dtype, int count,
                                           const ria_fp8_proj* projs, void* stream) {
  if (!norm_weight) return set_error(RIA_ERR_INVALID, "ria_linear_fp8_group_normed: null norm_weight");
  return linear_group("ria_linear_fp8_group_normed", m, k, x, RIA_DT_F32, x_row_stride, count, projs, stream,
                      norm_weight, eps, h_dtype);
}
