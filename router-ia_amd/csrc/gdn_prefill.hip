// Chunked (WY, chunk 64) Gated DeltaNet prefill for gfx950.
//
// Equal to running the reference's one-token step (qwen36_attention_cache.py:
// 176-266) over every token of a sequence in order, which is how the
// reference prefills (qwen36_chat_batch.py:255-258).  Per V head and chunk of
// C = 64 tokens (G = cumulative log-decay inside the chunk, D[i,j] =
// exp(G_i - G_j) for j <= i; q, k l2-normalised, q scaled by 128^-0.5):
//     L   = strict_lower(beta_i (k_i . k_j) D[i,j])
//     T   = (I + L)^-1
//     U   = T (beta v),  W = T (beta exp(G) k)
//     v'  = U - W S
//     o   = (exp(G) q) S + (q k^T o D, j <= i) v'
//     S  <- exp(G_C) S + (exp(G_C - G) k)^T v'
//
// Kernels (one sequence per call; the host walks segments of chunks):
//   prefill_conv_kernel   causal depthwise conv + SiLU over the segment's
//                         tokens (bf16, the reference's rounding), history
//                         from the conv ring for tokens before the prompt;
//                         one more workgroup per chunk computes the gates
//                         (beta, the cumulative decay G and its exponentials)
//                         into the chunk's records.
//   chunk_prep_kernel     phase A, one workgroup per (chunk, V head):
//                         l2norm, K K^T and Q K^T on MFMA, blocked fp32
//                         triangular inverse, U and W on MFMA.
//   chunk_scan_kernel     phase B, one workgroup per (V head, 16 state
//                         columns), sequential over chunks, waves in two
//                         roles (state, read-out); the fp32 state block
//                         stays in LDS.
//   (phase A of the prompt's last chunk also writes the last inputs into the
//   conv ring.)
//
// MFMA precision: products run on bf16 MFMA 16x16x32.  The conv outputs q, k
// and v are bf16 values, exact operands, and enter the products as they are
// (their norms and gates as fp32 factors outside); an fp32 operand is split
// as hi + lo bf16: one product with an exact operand becomes two (x*hi +
// x*lo), two fp32 operands three (hi*hi + hi*lo + lo*hi, ~2^-16 relative).
// The cumulative decay, exponentials and the triangular inverse are fp32.
#include <math.h>
#include <algorithm>
#include <type_traits>

#include "ria_common.h"

namespace ria {

constexpr int kChunk = 64;
constexpr int kDim = kGdnHeadDim;  // 128

// Per (chunk, head) phase-A record, consumed by phase B.  Operands are stored
// in MFMA 16x16x32 operand order, one 16-byte unit per lane, so phase B loads
// them as contiguous 1 KiB wavefront reads.  The q and k operands are the
// conv outputs themselves (bf16, exact), their per-token factors applied by
// phase B outside the products; W and (q k^T) o D are fp32 values stored
// pre-split as bf16 hi + lo:
//   Q   q (bf16)           A operand, [token tile 4][k-step 4][lane]
//   Wn  -W                 A operand, [token tile 4][k-step 4][hi/lo][lane]
//   QK  (q k^T) o D        A operand, [token tile 4][k-step 2][hi/lo][lane]
//   K   k^T (bf16)         A operand, [dk tile 8][k-step 2][lane]
//   U   T (beta v)         C tiles in accumulator order, [token tile 4][dim tile 8][lane] x 4 fp32
//   fq  exp(G_t) / |q_t| / sqrt(128), per token (exp(G) q = fq q)
//   fk  exp(G_C - G_t) / |k_t|, per token (the k of S's update = fk k)
//   gl  exp(G_C)
//   Gt  per token {beta, G, exp(G), exp(G_C - G)} from the conv launch's gate
//       pass, read by phase A
constexpr int kRecQt = 0;
constexpr int kRecWn = kRecQt + 4 * 4 * 64 * 16;
constexpr int kRecQK = kRecWn + 4 * 4 * 2 * 64 * 16;
constexpr int kRecKt = kRecQK + 4 * 2 * 2 * 64 * 16;
constexpr int kRecU = kRecKt + 8 * 2 * 64 * 16;
constexpr int kRecFq = kRecU + 4 * 8 * 64 * 16;
constexpr int kRecFk = kRecFq + 64 * 4;
constexpr int kRecGl = kRecFk + 64 * 4;
constexpr int kRecGate = kRecGl + 256;
constexpr int kRecBytes = kRecGate + 64 * 16;

struct PrefillArgs {
  const void* x;  // [L, conv_dim] projection output (pre-conv), x_dtype
  int64_t x_stride;
  const uint16_t* conv_w;
  uint16_t* conv_ring;  // [4, conv_dim] of this sequence
  int32_t n0;           // conv step of token 0
  int length;           // L
  int tok0;             // first token of the segment
  int seg_tokens;       // tokens in the segment
  int chunk0;           // first chunk of the segment
  int seg_chunks;
  uint16_t* post;  // [seg_tokens, conv_dim] post-conv bf16 bits
  float* state;    // [Hv, 128, 128]
  const float* gate_a;
  const float* gate_b;
  int64_t gate_stride;
  const float* A_log;
  const float* dt_bias;
  char* rec;   // [seg_chunks, Hv, kRecBytes]
  void* out;   // [L, Hv, 128] (or the segment's fp32 read-out before the gated norm)
  int out_tok0;  // token stored at row 0 of out
  int num_k_heads;
  int num_v_heads;
  int conv_dim;
  int x_pairs;  // bf16 x, 4-byte aligned rows: a thread's two channels are one 32-bit load
  int gate_raw;  // gate_a / gate_b are the raw projections (RIA_GATE_RAW), else g and beta
};

// ---------------------------------------------------------------- helpers
// Split 8 fp32 values into bf16 hi and lo operand registers.
__device__ __forceinline__ void split8(const float* v, u32x4& hi, u32x4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t h0 = f32_to_bf16_bits(v[2 * j]), h1 = f32_to_bf16_bits(v[2 * j + 1]);
    const uint16_t l0 = f32_to_bf16_bits(v[2 * j] - bf16_bits_to_f32(h0));
    const uint16_t l1 = f32_to_bf16_bits(v[2 * j + 1] - bf16_bits_to_f32(h1));
    h[j] = h0 | (uint32_t(h1) << 16);
    l[j] = l0 | (uint32_t(l1) << 16);
  }
  hi = u32x4{h[0], h[1], h[2], h[3]};
  lo = u32x4{l[0], l[1], l[2], l[3]};
}

__device__ __forceinline__ u32x4 lds16(const uint16_t* p) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  return u32x4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ void load8(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// ---------------------------------------------------------------- conv
// Two adjacent channels per thread, a tile of 64 tokens per workgroup row.
// With bf16 inputs every load of the tile is issued at once (one 32-bit load
// per token for the two channels), then the arithmetic runs: issued in
// batches, each batch's latency was exposed (187 -> 144 us per 16k-token
// prompt in one process).  Other input dtypes load tokens in batches of 8.
// The launch is VALU-bound (the 16k-token prompt moves 0.54 GB, 67 us at
// 8 TB/s): SiLU takes silu_to_bf16, the same bits as the accurate form at
// about a third of its instructions, and the bf16 tile path addresses rows
// through buffer resources with the row in the scalar offset (146 -> 125 us).
constexpr int kConvTile = 64;
static_assert(kConvTile == kChunk, "a conv tile is a chunk: the gate pass takes one per workgroup");

// Gate pass of chunk blockIdx.y (the conv launch's last workgroup column):
// wave w takes V heads w, w + 4, ..; lane t token t of the chunk.  beta =
// sigmoid(b), g = -exp(A_log) softplus(a + dt_bias) (qwen36_attention_cache.py:
// 243-247), or both given; G = the sequential cumulative sum of g inside the
// chunk (tokens past the prompt add 0); then exp(G_t), exp(G_C - G_t) and
// exp(G_C) for phase A and the scan.  Off phase A's path, where it was a
// chain of transcendental and dependent adds on one wave (about 15% of an
// item) while the other three waited at the barrier.
__device__ __forceinline__ void prefill_gates(const PrefillArgs& a, float* gsh) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cl = blockIdx.y;
  const int t = (a.chunk0 + cl) * kChunk + lane;
  const bool ok = t < a.length;
  float* gw = gsh + wave * kChunk;
  for (int h = wave; h < a.num_v_heads; h += 4) {
    float beta = 0.f, g = 0.f;
    if (ok) {
      const float ga = a.gate_a[(int64_t)t * a.gate_stride + h], gb = a.gate_b[(int64_t)t * a.gate_stride + h];
      if (a.gate_raw) {
        beta = sigmoid_f(gb);
        g = -expf(a.A_log[h]) * softplus_f(ga + a.dt_bias[h]);
      } else {
        beta = gb;
        g = ga;
      }
    }
    gw[lane] = g;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // lane t adds g_0 .. g_t one at a time, the order of a sequential cumsum
    // (the masked terms add +0, which leaves the sum unchanged)
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kChunk; i += 4) {
      const float4 gv = *reinterpret_cast<const float4*>(gw + i);
      acc += i + 0 <= lane ? gv.x : 0.f;
      acc += i + 1 <= lane ? gv.y : 0.f;
      acc += i + 2 <= lane ? gv.z : 0.f;
      acc += i + 3 <= lane ? gv.w : 0.f;
    }
    const float gc = __shfl(acc, kChunk - 1, 64);
    char* rec = a.rec + ((int64_t)cl * a.num_v_heads + h) * kRecBytes;
    reinterpret_cast<float4*>(rec + kRecGate)[lane] = float4{beta, acc, expf(acc), expf(gc - acc)};
    if (lane == 0) *reinterpret_cast<float*>(rec + kRecGl) = expf(gc);
    __builtin_amdgcn_wave_barrier();  // gw is read by every lane before the next head writes it
  }
}

template <int XT>
__global__ __launch_bounds__(256) void prefill_conv_kernel(PrefillArgs a) {
  if (blockIdx.x == gridDim.x - 1) {
    __shared__ __attribute__((aligned(16))) float gsh[4 * kChunk];
    prefill_gates(a, gsh);
    return;
  }
  const int c = 2 * (blockIdx.x * 256 + threadIdx.x);
  if (c >= a.conv_dim) return;
  const int t_begin = a.tok0 + blockIdx.y * kConvTile;
  const int t_end = min(t_begin + kConvTile, a.tok0 + a.seg_tokens);
  const uint4 wv = *reinterpret_cast<const uint4*>(a.conv_w + (int64_t)c * kConvTaps);  // 2 channels x 4 taps
  const float wa[4] = {bf16_bits_to_f32(wv.x & 0xffffu), bf16_bits_to_f32(wv.x >> 16),
                       bf16_bits_to_f32(wv.y & 0xffffu), bf16_bits_to_f32(wv.y >> 16)};
  const float wb[4] = {bf16_bits_to_f32(wv.z & 0xffffu), bf16_bits_to_f32(wv.z >> 16),
                       bf16_bits_to_f32(wv.w & 0xffffu), bf16_bits_to_f32(wv.w >> 16)};
  auto input = [&](int t, float& xa, float& xb) {
    if (t >= 0) {
      xa = bf16_bits_to_f32(f32_to_bf16_bits(load_act<XT>(a.x, (int64_t)t * a.x_stride + c)));
      xb = bf16_bits_to_f32(f32_to_bf16_bits(load_act<XT>(a.x, (int64_t)t * a.x_stride + c + 1)));
    } else {
      const uint32_t r = *reinterpret_cast<const uint32_t*>(a.conv_ring + ((a.n0 + t) & 3) * a.conv_dim + c);
      xa = bf16_bits_to_f32(r & 0xffffu);
      xb = bf16_bits_to_f32(r >> 16);
    }
  };
  float ha[3], hb[3];
  for (int i = 0; i < 3; ++i) input(t_begin - 3 + i, ha[i], hb[i]);
  // conv + SiLU of one token for both channels as packed bf16 (channel c in
  // the low half); shifts the history
  using B16 = Kv16<RIA_DT_BF16>;
  auto step = [&](float xa, float xb) -> uint32_t {
    float acc_a = wa[0] * ha[0], acc_b = wb[0] * hb[0];
    acc_a = fmaf(wa[1], ha[1], acc_a);
    acc_b = fmaf(wb[1], hb[1], acc_b);
    acc_a = fmaf(wa[2], ha[2], acc_a);
    acc_b = fmaf(wb[2], hb[2], acc_b);
    acc_a = fmaf(wa[3], xa, acc_a);
    acc_b = fmaf(wb[3], xb, acc_b);
    const uint32_t r = B16::pack2(acc_a, acc_b);  // the bf16 conv output
    ha[0] = ha[1]; ha[1] = ha[2]; ha[2] = xa;
    hb[0] = hb[1]; hb[1] = hb[2]; hb[2] = xb;
    return B16::pack2(silu_to_bf16(B16::lo_f32(r)), silu_to_bf16(B16::hi_f32(r)));
  };
  if (XT == RIA_DT_BF16 && a.x_pairs) {
    // Every load of the tile at once.  Buffer resources over the tile's rows
    // take the row in the scalar offset, so no per-token address arithmetic
    // (x rows clamped to the segment; x_stride < 2^24 elements).
    const int rows = t_end - t_begin;
    const uint16_t* xt = static_cast<const uint16_t*>(a.x) + (int64_t)t_begin * a.x_stride;
    const auto xs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(xt), 0, rows * (int)a.x_stride * 2,
                                                      kBufferWord3);
    const auto ps = __builtin_amdgcn_make_buffer_rsrc(a.post + (int64_t)(t_begin - a.tok0) * a.conv_dim, 0,
                                                      rows * a.conv_dim * 2, kBufferWord3);
    const int voff = c * 2;
    uint32_t xr[kConvTile];
#pragma unroll
    for (int u = 0; u < kConvTile; ++u)
      xr[u] = __builtin_amdgcn_raw_buffer_load_b32(xs, voff, min(u, rows - 1) * (int)a.x_stride * 2, 0);
#pragma unroll
    for (int u = 0; u < kConvTile; ++u)
      if (u < rows)
        __builtin_amdgcn_raw_buffer_store_b32(step(B16::lo_f32(xr[u]), B16::hi_f32(xr[u])), ps, voff,
                                              u * a.conv_dim * 2, 0);
  } else {
    for (int tb = t_begin; tb < t_end; tb += 8) {
      float xa[8], xb[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (tb + u < t_end) input(tb + u, xa[u], xb[u]);
        else xa[u] = xb[u] = 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (tb + u >= t_end) break;
        *reinterpret_cast<uint32_t*>(a.post + (int64_t)(tb + u - a.tok0) * a.conv_dim + c) = step(xa[u], xb[u]);
      }
    }
  }
}


// Step 3 of phase A for wave W: row tile W of Q K^T (A operand = the wave's
// own q rows) and row tile 3 - W of K K^T (A operand from the k rows in LDS),
// 5 tiles in all; B operands are the k rows of tiles tj.  q and k enter as
// the conv's bf16 values, exact MFMA operands, so each product is one MFMA;
// the epilogue applies the rows' norms (fq_s: |q|^-1 / sqrt(128), fk_s:
// |k|^-1) with the decay mask and writes (q k^T) o D and
// L = strict_lower(beta k k^T o D).
template <int W>
__device__ __forceinline__ void prep_qk_kk_tiles(const uint4 (&rq)[4], const uint16_t* kr, const float* G_s,
                                                 const float* beta_s, const float* fq_s, const float* fk_s,
                                                 float* Lm, float* QKs, int n, int g4) {
  using BF = Kv16<RIA_DT_BF16>;
  constexpr int RQ = W, RK = 3 - W;
  constexpr int NB = (RQ > RK ? RQ : RK) + 1;
  f32x4 aq[RQ + 1], ak[RK + 1];
#pragma unroll
  for (int t = 0; t <= RQ; ++t) aq[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t <= RK; ++t) ak[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int d = 32 * s + 8 * g4;
    const u32x4 qa = u32x4{rq[s].x, rq[s].y, rq[s].z, rq[s].w};
    const u32x4 ka = lds16(kr + (16 * RK + n) * 136 + d);
    u32x4 bk[NB];
#pragma unroll
    for (int tj = 0; tj < NB; ++tj) bk[tj] = lds16(kr + (16 * tj + n) * 136 + d);
#pragma unroll
    for (int tj = 0; tj <= RQ; ++tj) aq[tj] = BF::mfma_k32(qa, bk[tj], aq[tj]);
#pragma unroll
    for (int tj = 0; tj <= RK; ++tj) ak[tj] = BF::mfma_k32(ka, bk[tj], ak[tj]);
  }
#pragma unroll
  for (int tj = 0; tj <= RQ; ++tj)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int i = 16 * RQ + 4 * g4 + i4, j = 16 * tj + n;
      QKs[i * 68 + j] = j <= i ? aq[tj][i4] * (fq_s[i] * fk_s[j]) * expf(G_s[i] - G_s[j]) : 0.f;
    }
#pragma unroll
  for (int tj = 0; tj <= RK; ++tj)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int i = 16 * RK + 4 * g4 + i4, j = 16 * tj + n;
      Lm[i * 68 + j] = j < i ? beta_s[i] * (ak[tj][i4] * (fk_s[i] * fk_s[j])) * expf(G_s[i] - G_s[j]) : 0.f;
    }
}

// ---------------------------------------------------------------- phase A
// LDS: three 17 KB slots and the per-token factors, 52.3 KB in all, so three
// workgroups share a CU and their loads and barriers overlap each other's
// arithmetic (at 75 KB and two per CU phase A took 438 us per 16k tokens).
// What each slot holds over the kernel's steps:
//   S0: k rows [64][136] bf16 (steps 2-3) -> T fp32 [64][68] (4-6)
//       -> -W fp32 [64][132] (7, with S1)
//   S1: k^T bf16 [128][72] (2, into S2) -> L fp32 [64][68] (3-4)
//       -> (T o beta) hi/lo (6U) -> (T o beta e^G |k|^-1) hi/lo (6W)
//   S2: (q k^T) o D fp32 [64][68] (3-4) -> inverse scratch (4) -> v^T bf16
//       [128][68] (6U) -> k^T bf16 [128][68] (6W)
constexpr int kSlot = 17408;
constexpr int kS0 = 0;
constexpr int kS1 = kS0 + kSlot;
constexpr int kS2 = kS1 + kSlot;
constexpr int kKtPitch = 72;  // bf16 per k^T row in S1 (16-byte aligned rows)
constexpr int kRScal = kS2 + kSlot;  // beta, G and the per-token factors
constexpr int kPrepLdsBytes = kRScal + 4 * 64 * 5;
static_assert(128 * kKtPitch * 2 <= 2 * kSlot && 64 * 132 * 4 <= 2 * kSlot, "two-slot arrays");
static_assert(3 * kPrepLdsBytes <= 160 * 1024, "three workgroups per CU");

template <int XT>
__global__ __launch_bounds__(256, 3) void chunk_prep_kernel(PrefillArgs a) {
  // Heads vary fastest, so a round of workgroups reads a few chunks' whole
  // rows rather than pieces of every chunk.  With Hv a multiple of 8, x ->
  // head (Hv / 8) (x % 8) + x / 8 puts consecutive V heads (those sharing a K
  // head) on one XCD (workgroup ids congruent mod 8 share an XCD), so their
  // q and k rows are fetched once per L2.
  const int cl = blockIdx.y;  // chunk within the segment
  const int x = blockIdx.x;
  const int h = a.num_v_heads % 8 == 0 ? (a.num_v_heads / 8) * (x % 8) + x / 8 : x;
  // wave in a scalar register: the per-wave branches and job loops below are
  // then scalar
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g4 = lane >> 4;
  const int t0 = (a.chunk0 + cl) * kChunk;  // absolute first token of the chunk
  const int group = a.num_v_heads / a.num_k_heads;
  const int hk = h / group;
  const int kdim = a.num_k_heads * kDim;

  __shared__ __attribute__((aligned(16))) unsigned char lds[kPrepLdsBytes];
  uint16_t* kr = reinterpret_cast<uint16_t*>(lds + kS0);  // k rows [64][136] (bf16 conv values)
  uint16_t* KtB = reinterpret_cast<uint16_t*>(lds + kS1);  // k^T bf16 [128][kKtPitch]
  float* Lm = reinterpret_cast<float*>(lds + kS1);
  float* QKs = reinterpret_cast<float*>(lds + kS2);
  float* beta_s = reinterpret_cast<float*>(lds + kRScal);
  float* G_s = beta_s + 64;
  float* fq_s = G_s + 64;  // per-token factors: |q|^-1 / sqrt(128)
  float* fk_s = fq_s + 64;  // |k|^-1
  float* fw_s = fk_s + 64;  // beta e^G |k|^-1 (the k side of W)
  float* Xs = reinterpret_cast<float*>(lds + kS2);  // [4][16][17], once (q k^T) o D is in the record
  char* rec = a.rec + ((int64_t)cl * a.num_v_heads + h) * kRecBytes;

  // Step 1: lane (n, g4) of wave w loads token 16w + n, dims 32s + 8g4 .. +8 of
  // q, k and v: the MFMA A-operand order, so no transpose is needed later.
  // The row's gates {beta, G, exp(G), exp(G_C - G)} (the conv launch's gate
  // pass) go out first.
  const int row = 16 * wave + n;
  const int t = t0 + row;
  const bool valid = t < a.length;
  const float4 gt = reinterpret_cast<const float4*>(rec + kRecGate)[row];
  float qv[4][8], kv[4][8];
  uint4 rq[4], rk[4], rv[4];  // the conv outputs (bf16): the MFMA operands and the record's q and k
  {
    const uint16_t* base = a.post + (int64_t)(t - a.tok0) * a.conv_dim;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int d = 32 * s + 8 * g4;
      if (valid) {
        rq[s] = *reinterpret_cast<const uint4*>(base + hk * kDim + d);
        rk[s] = *reinterpret_cast<const uint4*>(base + kdim + hk * kDim + d);
        rv[s] = *reinterpret_cast<const uint4*>(base + 2 * kdim + h * kDim + d);
      } else {
        rq[s] = rk[s] = rv[s] = uint4{0u, 0u, 0u, 0u};
      }
    }
    auto unpack = [](uint4 r, float* o) {
      const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[2 * j] = through_dtype<XT>(bf16_bits_to_f32(w[j] & 0xffffu));
        o[2 * j + 1] = through_dtype<XT>(bf16_bits_to_f32(w[j] >> 16));
      }
    };
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      unpack(rq[s], qv[s]);
      unpack(rk[s], kv[s]);
    }
  }
  if (g4 == 0) {
    beta_s[row] = gt.x;
    G_s[row] = gt.y;
  }
  // Step 2: l2norm of the q and k rows (a row is spread over the 4 lane groups).
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sq += mul_rn(qv[s][j], qv[s][j]);
      sk += mul_rn(kv[s][j], kv[s][j]);
    }
  sq += __shfl_xor(sq, 16, 64);
  sq += __shfl_xor(sq, 32, 64);
  sk += __shfl_xor(sk, 16, 64);
  sk += __shfl_xor(sk, 32, 64);
  const float iq = 1.0f / sqrtf(sq + 1e-6f), ik = 1.0f / sqrtf(sk + 1e-6f);
  // No barrier here: beta_s and G_s are first read in step 3, after the next
  // one, and until then each wave writes only its own rows.
  const float eg = gt.z;   // e^{G_t}
  const float ekl = gt.w;  // e^{G_C - G_t}
  const float bt = gt.x;
  // k rows (bf16) into RA; q (bf16) and the per-token factors straight to
  // the record (A-operand order); k^T (bf16) into RB; the rows' factors for
  // the products' epilogues into LDS.
  {
    u32x4* q_rec = reinterpret_cast<u32x4*>(rec + kRecQt);
    const float fq = mul_rn(iq, 0.08838834764831845f);
    if (g4 == 0) {
      reinterpret_cast<float*>(rec + kRecFq)[row] = mul_rn(fq, eg);
      reinterpret_cast<float*>(rec + kRecFk)[row] = mul_rn(ik, ekl);
      fq_s[row] = fq;
      fk_s[row] = ik;
      fw_s[row] = mul_rn(mul_rn(bt, eg), ik);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int d = 32 * s + 8 * g4;
      *reinterpret_cast<uint4*>(kr + row * 136 + d) = rk[s];
      q_rec[(wave * 4 + s) * 64 + lane] = u32x4{rq[s].x, rq[s].y, rq[s].z, rq[s].w};
      const uint32_t kw[4] = {rk[s].x, rk[s].y, rk[s].z, rk[s].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {  // transposed: KtB[dim][token]
        KtB[(d + 2 * j) * kKtPitch + row] = static_cast<uint16_t>(kw[j] & 0xffffu);
        KtB[(d + 2 * j + 1) * kKtPitch + row] = static_cast<uint16_t>(kw[j] >> 16);
      }
    }
  }
  lds_barrier();
  // k^T operand to the record: lane (n, g4) of job (dk tile dt, k-step s)
  // takes dim 16 dt + n, tokens 32 s + 8 g4 .. + 7.
  {
    u32x4* k_rec = reinterpret_cast<u32x4*>(rec + kRecKt);
    for (int job = wave; job < 16; job += 4) {
      const int dt = job >> 1, s = job & 1;
      k_rec[(dt * 2 + s) * 64 + lane] = lds16(KtB + (16 * dt + n) * kKtPitch + 32 * s + 8 * g4);
    }
  }
  lds_barrier();  // S1, S2 free for L and (q k^T) o D
  // Step 3: Q K^T -> (q k^T) o D and K K^T -> L, 5 tiles per wave.
  if (wave == 0) prep_qk_kk_tiles<0>(rq, kr, G_s, beta_s, fq_s, fk_s, Lm, QKs, n, g4);
  else if (wave == 1) prep_qk_kk_tiles<1>(rq, kr, G_s, beta_s, fq_s, fk_s, Lm, QKs, n, g4);
  else if (wave == 2) prep_qk_kk_tiles<2>(rq, kr, G_s, beta_s, fq_s, fk_s, Lm, QKs, n, g4);
  else prep_qk_kk_tiles<3>(rq, kr, G_s, beta_s, fq_s, fk_s, Lm, QKs, n, g4);
  lds_barrier();  // k rows dead: S0 takes T
  // Step 4: QK operand to the record; T = (I + L)^-1 into S0 (blocked 4x4 of 16x16).
  float* Tm = reinterpret_cast<float*>(lds + kS0);
  {
    u32x4* qk_rec = reinterpret_cast<u32x4*>(rec + kRecQK);
    for (int job = wave; job < 8; job += 4) {
      const int w = job >> 1, s = job & 1;
      float tmp[8];
      load8(QKs + (16 * w + n) * 68 + 32 * s + 8 * g4, tmp);
      if (((32 * s + 8 * g4) >> 4) > w) {  // upper tiles of (q k^T) o D are zero (never written)
#pragma unroll
        for (int j = 0; j < 8; ++j) tmp[j] = 0.f;
      }
      u32x4 hi, lo;
      split8(tmp, hi, lo);
      qk_rec[((w * 2 + s) * 2 + 0) * 64 + lane] = hi;
      qk_rec[((w * 2 + s) * 2 + 1) * 64 + lane] = lo;
    }
  }
  if (n == lane) {  // lanes 0..15: wave w inverts diagonal block w, lane j owns column j
    const int b0 = 16 * wave;
    float col[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sacc = 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) sacc = fmaf(Lm[(b0 + i) * 68 + b0 + m], col[m], sacc);
      col[i] = (i == lane) ? 1.f : (i < lane ? 0.f : -sacc);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Tm[(b0 + i) * 68 + b0 + lane] = col[i];
  }
  lds_barrier();
  // T_ij = -T_ii sum_{m=j}^{i-1} L_im T_mj, block distance by distance, on
  // fp32 MFMA 16x16x4: lane l supplies A (row l % 16, k l / 16) and B
  // (k l / 16, column l % 16) and receives C rows 4 (l / 16) .. + 3 of
  // column l % 16.
  for (int dist = 1; dist < 4; ++dist) {
    const int bi = wave + dist, bj = wave;
    if (bi < 4) {
      float* X = Xs + wave * 16 * 17;
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      for (int bm = bj; bm < bi; ++bm)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          x = __builtin_amdgcn_mfma_f32_16x16x4f32(Lm[(16 * bi + n) * 68 + 16 * bm + 4 * kk + g4],
                                                   Tm[(16 * bm + 4 * kk + g4) * 68 + 16 * bj + n], x, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) X[(4 * g4 + r) * 17 + n] = x[r];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        y = __builtin_amdgcn_mfma_f32_16x16x4f32(Tm[(16 * bi + n) * 68 + 16 * bi + 4 * kk + g4],
                                                 X[(4 * kk + g4) * 17 + n], y, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) Tm[(16 * bi + 4 * g4 + r) * 68 + 16 * bj + n] = -y[r];
    }
    lds_barrier();
  }
  // Steps 5 and 6, once for U and once for W: T with its columns scaled by
  // the tokens' factors, as hi/lo pairs into S1 (T o beta for U, then
  // T o beta e^G |k|^-1 for W), so that v and k enter the products as the
  // conv's bf16 values, transposed as raw bf16 into S2; then the product.
  // Wave w takes column tiles td = w and w + 4 for every token tile; the hi
  // and lo products go to separate accumulators, added at the end.
  uint16_t* Th = reinterpret_cast<uint16_t*>(lds + kS1);  // hi [64][68], lo after
  uint16_t* Bt = reinterpret_cast<uint16_t*>(lds + kS2);  // v^T or k^T [128][68]
  auto stage = [&](const float* fac, const uint4 (&raw)[4]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {  // 8 consecutive columns per thread
      const int e8 = tid + 256 * r;
      const int i = e8 >> 3, j0 = (e8 & 7) * 8;
      float tv[8], fj[8];
      load8(Tm + i * 68 + j0, tv);
      load8(fac + j0, fj);
      const bool upper = (j0 >> 4) > (i >> 4);  // T's upper tiles are zero (never written)
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = (upper ? 0.f : tv[j]) * fj[j];
      u32x4 hi, lo;
      split8(x, hi, lo);
      // rows are 136 bytes apart: 8-byte stores keep every access aligned
      auto st8x2 = [](uint16_t* p, const u32x4& v) {
        reinterpret_cast<uint2*>(p)[0] = uint2{v[0], v[1]};
        reinterpret_cast<uint2*>(p)[1] = uint2{v[2], v[3]};
      };
      st8x2(Th + i * 68 + j0, hi);
      st8x2(Th + 64 * 68 + i * 68 + j0, lo);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t bw[4] = {raw[s].x, raw[s].y, raw[s].z, raw[s].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * s + 8 * g4 + 2 * j;
        Bt[d * 68 + row] = static_cast<uint16_t>(bw[j] & 0xffffu);
        Bt[(d + 1) * 68 + row] = static_cast<uint16_t>(bw[j] >> 16);
      }
    }
  };
  constexpr int kSteps[4] = {1, 1, 2, 2};  // T is lower triangular: k-steps of 32 up to column 16 tt + 15
  using BF = Kv16<RIA_DT_BF16>;
  auto t_times = [&](int tt, f32x4 (&acc)[2]) {
    f32x4 ah_acc[2], al_acc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) ah_acc[q] = al_acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (s >= kSteps[tt]) break;
      const int kofs = 32 * s + 8 * g4;
      const u32x4 ah = lds16(Th + (16 * tt + n) * 68 + kofs), al = lds16(Th + 64 * 68 + (16 * tt + n) * 68 + kofs);
      u32x4 bq[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) bq[q] = lds16(Bt + (16 * (wave + 4 * q) + n) * 68 + kofs);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        ah_acc[q] = BF::mfma_k32(ah, bq[q], ah_acc[q]);
        al_acc[q] = BF::mfma_k32(al, bq[q], al_acc[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) acc[q] = ah_acc[q] + al_acc[q];
  };
  stage(beta_s, rv);  // L and the inverse scratch are dead
  lds_barrier();
  {
    f32x4* u_rec = reinterpret_cast<f32x4*>(rec + kRecU);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 acc[2];
      t_times(tt, acc);
#pragma unroll
      for (int q = 0; q < 2; ++q) u_rec[(tt * 8 + wave + 4 * q) * 64 + lane] = acc[q];
    }
  }
  lds_barrier();  // T o beta and v^T read
  stage(fw_s, rk);
  lds_barrier();
  f32x4 wacc[4][2];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) t_times(tt, wacc[tt]);
  lds_barrier();  // T, its W scaling and k^T read: S0 and S1 take the -W staging
  float* Wst = reinterpret_cast<float*>(lds + kS0);  // -W [64][132]
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) Wst[(16 * tt + 4 * g4 + i4) * 132 + 16 * (wave + 4 * q) + n] = -wacc[tt][q][i4];
  lds_barrier();
  // Step 7: -W operand to the record.
  {
    u32x4* wn_rec = reinterpret_cast<u32x4*>(rec + kRecWn);
    for (int job = wave; job < 16; job += 4) {
      const int w = job >> 2, s = job & 3;
      float tmp[8];
      load8(Wst + (16 * w + n) * 132 + 32 * s + 8 * g4, tmp);
      u32x4 hi, lo;
      split8(tmp, hi, lo);
      wn_rec[((w * 4 + s) * 2 + 0) * 64 + lane] = hi;
      wn_rec[((w * 4 + s) * 2 + 1) * 64 + lane] = lo;
    }
  }
  // The conv ring takes the inputs of the prompt's last min(L, 4) tokens:
  // the workgroups of the last segment's last chunk share the channels (the
  // conv launches, the only readers of its old contents, have finished).
  if (a.tok0 + a.seg_tokens == a.length && cl == a.seg_chunks - 1) {
    const int per = (a.conv_dim + gridDim.x - 1) / gridDim.x;
    const int c_end = min(x * per + per, a.conv_dim);
    for (int t = max(0, a.length - 4); t < a.length; ++t)
      for (int c = x * per + tid; c < c_end; c += 256)
        a.conv_ring[((a.n0 + t) & 3) * a.conv_dim + c] = f32_to_bf16_bits(load_act<XT>(a.x, (int64_t)t * a.x_stride + c));
  }
}

// ---------------------------------------------------------------- phase B
// Record operands of one chunk for each role of the scan's waves.
struct StateOps {  // v' = U - W S, fk v', and S <- e^{G_C} S + k^T (fk v')
  u32x4 wn[4][2], kt[2][2];
  f32x4 u, fk;  // fk of the wave's token tile rows 4 g4 .. 4 g4 + 3
  float gl;
};
struct OutOps {  // o = fq (q S) + ((q k^T) o D) v'
  u32x4 qt[4], qk[2][2];
  f32x4 fq;
};

template <int OT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void chunk_scan_kernel(PrefillArgs a) {
  // The 8 column blocks of a head share an XCD (workgroup ids congruent mod 8
  // run on one XCD; id = 32 * cb + h), so its records are fetched once per L2.
  const int h = blockIdx.x % a.num_v_heads;
  const int cb = blockIdx.x / a.num_v_heads;
  // wave stays in a vector register here, so each record load whose scalar
  // offset derives from it is issued through a one-pass waterfall loop; with
  // wave scalar (no loops) the scan measured 446-453 against 417-423 us per
  // 16k-token layer, bit-identical (the loops pace the 84 KB of loads per
  // chunk that queue in the CU's vector memory path)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g4 = lane >> 4;
  // Two roles, one wave of each per SIMD (waves w and w + 4 share SIMD w):
  // waves 0-3 carry the state (v' of token tile w, then S rows 32 w .. 32 w
  // + 31), waves 4-7 the read-out (q S of token tile w, then its intra-chunk
  // term and the output).  Each chunk is two phases closed by a barrier; per
  // phase a wave runs at most 12 of the chunk's MFMAs on its chain instead
  // of 20, and the other role's wave on its SIMD fills the waits.
  const bool state_role = wave < 4;
  const int w = wave & 3;

  // LDS in 16-byte entries [row group][column n] (column n = state column
  // 16 cb + n): 4 rows of fp32 S, or 8 rows of bf16 S hi / lo or v' hi / lo
  // (v' rows are tokens).  A lane reads the entry [row group][n] of its own
  // column, so each 16-lane quarter of a wave reads 256 contiguous bytes.
  // Measured on gfx950 with a probe kernel: a 16-byte access is free of bank
  // conflicts only when each 16-lane quarter covers 256 contiguous bytes
  // (other spacings cost 4 cycles, a 256-byte pitch 28), an 8-byte store only
  // when each quarter covers 128 contiguous bytes.  Every access here is one
  // of those.
  __shared__ __attribute__((aligned(16))) float S32[kDim / 4][16][4];          // S fp32
  __shared__ __attribute__((aligned(16))) uint16_t STh[kDim / 8][16][8];       // S hi / lo (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t STl[kDim / 8][16][8];
  __shared__ __attribute__((aligned(16))) uint16_t VTh[kChunk / 8][16][8];     // v' hi / lo (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t VTl[kChunk / 8][16][8];
  __shared__ __attribute__((aligned(16))) uint16_t VKh[kChunk / 8][16][8];     // fk v' hi / lo (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t VKl[kChunk / 8][16][8];
  // A lane's four rows of a column (rows 4 g4 .. 4 g4 + 3 of a 16-row tile)
  // are half of an 8-row entry; the other half is in lane +-16 (g4 ^ 1).
  // The pair trades halves (one permlane16 swap per 32-bit word), so the
  // even lane stores the whole hi entry and the odd lane the whole lo entry,
  // each one 16-byte store.
  const bool even = (g4 & 1) == 0;
  auto store_hl = [&](uint16_t (*hp)[16][8], uint16_t (*lp)[16][8], int rg, const f32x4& x) {
    uint32_t h2[2], l2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint16_t a0 = f32_to_bf16_bits(x[2 * j]), a1 = f32_to_bf16_bits(x[2 * j + 1]);
      h2[j] = a0 | (uint32_t(a1) << 16);
      l2[j] = f32_to_bf16_bits(x[2 * j] - bf16_bits_to_f32(a0)) |
              (uint32_t(f32_to_bf16_bits(x[2 * j + 1] - bf16_bits_to_f32(a1))) << 16);
    }
    uint32_t got[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t give = even ? l2[j] : h2[j];
      const auto r = __builtin_amdgcn_permlane16_swap(give, give, false, false);  // {row 2i's, row 2i+1's}
      got[j] = even ? r[1] : r[0];
    }
    const u32x4 e = even ? u32x4{h2[0], h2[1], got[0], got[1]} : u32x4{got[0], got[1], l2[0], l2[1]};
    *reinterpret_cast<u32x4*>(even ? hp[rg][n] : lp[rg][n]) = e;
  };

  float* Sg = a.state + (int64_t)h * kDim * kDim + cb * 16;
  for (int e = tid; e < kDim * 16; e += 512) {
    const int r = e >> 4, c = e & 15;
    const float v = Sg[r * kDim + c];
    S32[r >> 2][c][r & 3] = v;
    const uint16_t hb = f32_to_bf16_bits(v);
    STh[r >> 3][c][r & 7] = hb;
    STl[r >> 3][c][r & 7] = f32_to_bf16_bits(v - bf16_bits_to_f32(hb));
  }
  lds_barrier();

  auto rec_of = [&](int cl) { return a.rec + ((int64_t)cl * a.num_v_heads + h) * kRecBytes; };
  // S hi / lo operands of the k-steps over the 128 state rows
  auto read_s = [&](u32x4 (&sh)[4], u32x4 (&sl)[4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      sh[s] = lds16(STh[4 * s + g4][n]);
      sl[s] = lds16(STl[4 * s + g4][n]);
    }
  };

  // Chunk cl + 2's record is pulled into L2 (one load per 128-byte line,
  // spread over the workgroup) while chunk cl computes, so the operand loads
  // of chunk cl + 1, issued at the same time, find their lines in L2: from
  // HBM a chunk's record arrives in about the time a chunk computes, and the
  // scan waited for it.  A touched value is consumed (an empty asm use) one
  // chunk later, when it has long arrived, so no wait is spent on it.
  // The 8 column-block workgroups of a head share an L2, so each touches
  // every 8th line (its own eighth of the record); the state role's 256
  // threads do the touching.
  constexpr int kRecLines = kRecBytes / 128;
  constexpr int kTouch = (kRecLines + 8 * 256 - 1) / (8 * 256);
  // Record loads go through a buffer resource based at the chunk's record
  // (built in scalar registers per chunk): every load is a loop-invariant
  // 32-bit lane offset plus a constant.  With 64-bit per-lane addresses the
  // loop reused a load's destination registers as address temporaries, and
  // the wait that reuse needs drained the record loads in flight every chunk.
  auto rec_rsrc = [&](int cl) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(rec_of(cl)), 0, kRecBytes, kBufferWord3);
  };
  auto bload16 = [](__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  };
  int touch_off[kTouch];
#pragma unroll
  for (int i = 0; i < kTouch; ++i) touch_off[i] = min(8 * (tid + 256 * i) + cb, kRecLines - 1) * 128;
  auto touch = [&](int cl, uint32_t (&tv)[kTouch]) {
    const auto r = rec_rsrc(cl);
#pragma unroll
    for (int i = 0; i < kTouch; ++i) tv[i] = __builtin_amdgcn_raw_buffer_load_b32(r, touch_off[i], 0, 0);
  };
  auto consume = [](const uint32_t (&tv)[kTouch]) {
#pragma unroll
    for (int i = 0; i < kTouch; ++i) asm volatile("" ::"v"(tv[i]));
  };
  // Chunk cl + 1's operands load while chunk cl computes (unrolled by two).
  // The prefetch is unconditional (the last chunk is simply loaded again):
  // a conditional one splits the loop into paths the compiler's wait
  // analysis merges conservatively, draining the prefetch every chunk.
  const int last = a.seg_chunks - 1;
  auto scan = [&](auto& A, auto& B, auto load_ops, auto process, auto touching) {
    constexpr bool kTouching = decltype(touching)::value;
    uint32_t tX[kTouch], tY[kTouch];
#pragma unroll
    for (int i = 0; i < kTouch; ++i) tY[i] = 0u;
    load_ops(0, A);
    for (int cl = 0; cl < a.seg_chunks; cl += 2) {
      load_ops(min(cl + 1, last), B);
      if constexpr (kTouching) touch(min(cl + 2, last), tX);
      process(cl, A);
      if constexpr (kTouching) consume(tY);
      if (cl + 1 >= a.seg_chunks) break;
      load_ops(min(cl + 2, last), A);
      if constexpr (kTouching) touch(min(cl + 3, last), tY);
      process(cl + 1, B);
      if constexpr (kTouching) consume(tX);
    }
  };

  // Each phase reads all of its LDS operands first, then runs its MFMAs; the
  // three products of a hi/lo pair (hi*hi, hi*lo, lo*hi) go to three
  // accumulators that are added at the end, so the MFMAs of a phase form
  // short independent chains.
  using BF = Kv16<RIA_DT_BF16>;
  if (state_role) {
    const int l16 = 16 * lane;
    auto load_ops = [&](int cl, StateOps& o) {
      const auto r = rec_rsrc(cl);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int p = 0; p < 2; ++p) o.wn[s][p] = bload16(r, l16, kRecWn + ((w * 4 + s) * 2 + p) * 1024);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int tk = 0; tk < 2; ++tk) o.kt[tk][s] = bload16(r, l16, kRecKt + ((2 * w + tk) * 2 + s) * 1024);
      o.u = __builtin_bit_cast(f32x4, bload16(r, l16, kRecU + (w * 8 + cb) * 1024));
      o.fk = __builtin_bit_cast(f32x4, bload16(r, 16 * g4, kRecFk + 64 * w));
      // a vector load: a scalar load here would be waited for by the next
      // lds_barrier (lgkmcnt), exposing its latency
      o.gl = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, 0, kRecGl, 0));
    };
    auto process = [&](int, const StateOps& o) {
      // (i) v' = U - W S for token tile w, and fk v'
      u32x4 sh[4], sl[4];
      read_s(sh, sl);
      __builtin_amdgcn_sched_barrier(0);
      f32x4 vn0 = o.u, vn1 = {0.f, 0.f, 0.f, 0.f}, vn2 = vn1;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        vn0 = BF::mfma_k32(o.wn[s][0], sh[s], vn0);
        vn1 = BF::mfma_k32(o.wn[s][0], sl[s], vn1);
        vn2 = BF::mfma_k32(o.wn[s][1], sh[s], vn2);
      }
      __builtin_amdgcn_sched_barrier(0);
      const f32x4 vn = (vn0 + vn1) + vn2;
      f32x4 vk;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) vk[i4] = mul_rn(vn[i4], o.fk[i4]);
      store_hl(VTh, VTl, 2 * w + (g4 >> 1), vn);
      store_hl(VKh, VKl, 2 * w + (g4 >> 1), vk);
      lds_barrier();
      // (iii) S <- exp(G_C) S + k^T (fk v') for dk tiles 2 w, 2 w + 1
      // (k is exact in bf16: two products per k-step)
      u32x4 kh[2], kl[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        kh[s] = lds16(VKh[4 * s + g4][n]);
        kl[s] = lds16(VKl[4 * s + g4][n]);
      }
      f32x4 sn[2];
#pragma unroll
      for (int tk = 0; tk < 2; ++tk) sn[tk] = *reinterpret_cast<const f32x4*>(S32[(16 * (2 * w + tk) + 4 * g4) >> 2][n]);
      __builtin_amdgcn_sched_barrier(0);
      f32x4 sa[2], sb[2];
#pragma unroll
      for (int tk = 0; tk < 2; ++tk) {
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) sa[tk][i4] = o.gl * sn[tk][i4];
        sb[tk] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int tk = 0; tk < 2; ++tk) {
          sa[tk] = BF::mfma_k32(o.kt[tk][s], kh[s], sa[tk]);
          sb[tk] = BF::mfma_k32(o.kt[tk][s], kl[s], sb[tk]);
        }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tk = 0; tk < 2; ++tk) {
        const int r0 = 16 * (2 * w + tk) + 4 * g4;
        const f32x4 snew = sa[tk] + sb[tk];
        *reinterpret_cast<f32x4*>(S32[r0 >> 2][n]) = snew;
        store_hl(STh, STl, r0 >> 3, snew);
      }
      lds_barrier();
    };
    StateOps A, B;
    scan(A, B, load_ops, process, std::true_type{});
  } else {
    const int l16 = 16 * lane;
    auto load_ops = [&](int cl, OutOps& o) {
      const auto r = rec_rsrc(cl);
#pragma unroll
      for (int s = 0; s < 4; ++s) o.qt[s] = bload16(r, l16, kRecQt + (w * 4 + s) * 1024);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int p = 0; p < 2; ++p) o.qk[s][p] = bload16(r, l16, kRecQK + ((w * 2 + s) * 2 + p) * 1024);
      o.fq = __builtin_bit_cast(f32x4, bload16(r, 16 * g4, kRecFq + 64 * w));
    };
    auto process = [&](int cl, const OutOps& o) {
      const int chunk = a.chunk0 + cl;
      // o_inter = fq (q S): q is exact in bf16, so two products (q S_hi +
      // q S_lo), then fq scales each token row
      u32x4 sh[4], sl[4];
      read_s(sh, sl);
      __builtin_amdgcn_sched_barrier(0);
      f32x4 oq0 = {0.f, 0.f, 0.f, 0.f}, oq1 = oq0;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        oq0 = BF::mfma_k32(o.qt[s], sh[s], oq0);
        oq1 = BF::mfma_k32(o.qt[s], sl[s], oq1);
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x4 oi0, oi1 = {0.f, 0.f, 0.f, 0.f}, oi2 = oi1;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) oi0[i4] = mul_rn(oq0[i4] + oq1[i4], o.fq[i4]);
      lds_barrier();
      // (ii) o = o_inter + ((q k^T) o D) v'   (lower triangular: token tiles <= w)
      u32x4 vh[2], vl[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        vh[s] = lds16(VTh[4 * s + g4][n]);
        vl[s] = lds16(VTl[4 * s + g4][n]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (32 * s <= 16 * w + 15) {
          oi0 = BF::mfma_k32(o.qk[s][0], vh[s], oi0);
          oi1 = BF::mfma_k32(o.qk[s][0], vl[s], oi1);
          oi2 = BF::mfma_k32(o.qk[s][1], vh[s], oi2);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      const f32x4 oi = (oi0 + oi1) + oi2;
      // The chunk's output rows through a buffer resource that ends at the
      // prompt's last token: the hardware drops stores past it, so every lane
      // stores without a branch (branches around the stores leave the
      // compiler unsure how many are in flight, and its wait for the
      // prefetched record then drains every load, the prefetch included).
      constexpr int kEsz = OT == RIA_DT_F32 ? 4 : 2;
      const int t0 = chunk * kChunk;
      const int row = a.num_v_heads * kDim;
      char* obase = static_cast<char*>(a.out) + (int64_t)(t0 - a.out_tok0) * row * kEsz;
      const __amdgpu_buffer_rsrc_t orsrc =
          __builtin_amdgcn_make_buffer_rsrc(obase, 0, min(kChunk, a.length - t0) * row * kEsz, kBufferWord3);
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int off = ((16 * w + 4 * g4 + i4) * row + h * kDim + cb * 16 + n) * kEsz;
        if constexpr (OT == RIA_DT_F32)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(oi[i4]), orsrc, off, 0, 0);
        else if constexpr (OT == RIA_DT_BF16)
          __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(oi[i4]), orsrc, off, 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b16(f32_to_f16_bits(oi[i4]), orsrc, off, 0, 0);
      }
      lds_barrier();
    };
    OutOps A, B;
    scan(A, B, load_ops, process, std::false_type{});
  }
  for (int e = tid; e < kDim * 16; e += 512) {
    const int r = e >> 4, c = e & 15;
    Sg[r * kDim + c] = S32[r >> 2][c][r & 3];
  }
}

static bool valid_dtype(int dt) { return dt == RIA_DT_BF16 || dt == RIA_DT_F16 || dt == RIA_DT_F32; }

// Workspace of one segment: [post-conv activations | phase-A records].  The
// first region holds the bf16 post-conv q|k|v until phase A has read it, then
// (with the gated norm) the segment's fp32 read-out between the scan and the
// norm pass.
int64_t prefill_post_bytes(int num_k_heads, int num_v_heads, int seg_chunks) {
  const int64_t conv_dim = (int64_t)(2 * num_k_heads + num_v_heads) * kDim;
  const int64_t tokens = (int64_t)seg_chunks * kChunk;
  const int64_t bytes = std::max(tokens * conv_dim * 2, tokens * num_v_heads * kDim * 4);
  return (bytes + 255) / 256 * 256;
}

int64_t prefill_segment_bytes(int num_k_heads, int num_v_heads, int seg_tokens) {
  const int chunks = (seg_tokens + kChunk - 1) / kChunk;
  return prefill_post_bytes(num_k_heads, num_v_heads, chunks) + (int64_t)chunks * num_v_heads * kRecBytes;
}

static int dtype_bytes(int dt) { return dt == RIA_DT_F32 ? 4 : 2; }

}  // namespace ria

using namespace ria;

extern "C" int64_t ria_gdn_prefill_workspace_bytes(int num_k_heads, int num_v_heads, int segment_tokens) {
  if (num_k_heads <= 0 || num_v_heads <= 0 || segment_tokens <= 0) return 0;
  return prefill_segment_bytes(num_k_heads, num_v_heads, segment_tokens);
}

extern "C" int ria_gdn_prefill(int length, int num_k_heads, int num_v_heads, const void* mixed_qkv, int x_dtype,
                               int64_t x_row_stride, const void* conv_weight, void* conv_ring, int32_t conv_pos,
                               float* state, const float* gate_a, const float* gate_b, int64_t gate_row_stride,
                               int gate_mode, const float* A_log, const float* dt_bias, void* out, int out_dtype,
                               const void* z, int z_dtype, int64_t z_row_stride, const float* norm_weight,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  if (length < 0) return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: length must be >= 0");
  if (length == 0) return RIA_OK;
  if (num_k_heads <= 0 || num_v_heads <= 0 || num_v_heads % num_k_heads)
    return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: num_v_heads must be a positive multiple of num_k_heads");
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype)) return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: unknown dtype");
  if (!mixed_qkv || !conv_weight || !conv_ring || !state || !gate_a || !gate_b || !out || !workspace)
    return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: null pointer");
  if (gate_mode != RIA_GATE_RAW && gate_mode != RIA_GATE_PRECOMPUTED)
    return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: unknown gate_mode %d", gate_mode);
  if (gate_mode == RIA_GATE_RAW && (!A_log || !dt_bias))
    return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: RIA_GATE_RAW needs A_log and dt_bias");
  if (reinterpret_cast<uintptr_t>(state) % 16 || reinterpret_cast<uintptr_t>(conv_weight) % 8 ||
      reinterpret_cast<uintptr_t>(workspace) % 256)
    return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: state 16-byte, conv_weight 8-byte, workspace 256-byte aligned");
  const int conv_dim = (2 * num_k_heads + num_v_heads) * kDim;
  if (x_row_stride < conv_dim || gate_row_stride < num_v_heads)
    return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: row stride too small");
  if (z && (!norm_weight || !valid_dtype(z_dtype) || z_row_stride < (int64_t)num_v_heads * kDim))
    return set_error(RIA_ERR_INVALID, "ria_gdn_prefill: a gate z needs norm_weight, a dtype code and row stride >= Hv*128");
  // Largest segment (whole chunks) the workspace holds.
  int seg_chunks = (length + kChunk - 1) / kChunk;
  while (seg_chunks > 0 && prefill_segment_bytes(num_k_heads, num_v_heads, seg_chunks * kChunk) > workspace_bytes)
    seg_chunks = seg_chunks > 8 ? seg_chunks / 2 : seg_chunks - 1;
  if (seg_chunks == 0)
    return set_error(RIA_ERR_WORKSPACE, "ria_gdn_prefill: workspace %lld bytes < one chunk (%lld)",
                     (long long)workspace_bytes, (long long)prefill_segment_bytes(num_k_heads, num_v_heads, kChunk));

  PrefillArgs a{};
  a.x = mixed_qkv;
  a.x_stride = x_row_stride;
  a.x_pairs = x_dtype == RIA_DT_BF16 && reinterpret_cast<uintptr_t>(mixed_qkv) % 4 == 0 && x_row_stride % 2 == 0 &&
              x_row_stride < (int64_t(1) << 24);
  a.conv_w = static_cast<const uint16_t*>(conv_weight);
  a.conv_ring = static_cast<uint16_t*>(conv_ring);
  a.n0 = conv_pos;
  a.length = length;
  a.state = state;
  a.gate_a = gate_a;
  a.gate_b = gate_b;
  a.gate_stride = gate_row_stride;
  a.A_log = A_log;
  a.dt_bias = dt_bias;
  a.gate_raw = gate_mode == RIA_GATE_RAW;
  a.out = out;
  a.num_k_heads = num_k_heads;
  a.num_v_heads = num_v_heads;
  a.conv_dim = conv_dim;
  const int64_t post_bytes = prefill_post_bytes(num_k_heads, num_v_heads, seg_chunks);
  a.post = static_cast<uint16_t*>(workspace);
  a.rec = static_cast<char*>(workspace) + post_bytes;
  hipStream_t st = static_cast<hipStream_t>(stream);

  const int total_chunks = (length + kChunk - 1) / kChunk;
  for (int c0 = 0; c0 < total_chunks; c0 += seg_chunks) {
    a.chunk0 = c0;
    a.seg_chunks = min(seg_chunks, total_chunks - c0);
    a.tok0 = c0 * kChunk;
    a.seg_tokens = min(a.seg_chunks * kChunk, length - a.tok0);
    dim3 cgrid((conv_dim / 2 + 255) / 256 + 1, (a.seg_tokens + kConvTile - 1) / kConvTile);  // + the gate pass
    dim3 pgrid(num_v_heads, a.seg_chunks);
    dim3 sgrid(num_v_heads * (kDim / 16));
#define RIA_PREFILL_PHASES(XT_)                                                                          \
  hipLaunchKernelGGL((prefill_conv_kernel<XT_>), cgrid, dim3(256), 0, st, a);                           \
  hipLaunchKernelGGL((chunk_prep_kernel<XT_>), pgrid, dim3(256), 0, st, a)
    if (x_dtype == RIA_DT_BF16) {
      RIA_PREFILL_PHASES(RIA_DT_BF16);
    } else if (x_dtype == RIA_DT_F16) {
      RIA_PREFILL_PHASES(RIA_DT_F16);
    } else {
      RIA_PREFILL_PHASES(RIA_DT_F32);
    }
#undef RIA_PREFILL_PHASES
    if (z) {
      // fp32 read-out of the segment into the (now dead) post-conv region,
      // then the gated RMSNorm over whole heads into out
      PrefillArgs sa = a;
      sa.out = a.post;
      sa.out_tok0 = a.tok0;
      hipLaunchKernelGGL((chunk_scan_kernel<RIA_DT_F32>), sgrid, dim3(512), 0, st, sa);
      int rc = check_launch("ria_gdn_prefill");
      if (rc != RIA_OK) return rc;
      const int64_t head_row = (int64_t)num_v_heads * kDim;
      rc = ria_gated_rmsnorm(a.seg_tokens, num_v_heads, kDim, a.post, RIA_DT_F32, head_row,
                             static_cast<const char*>(z) + (int64_t)a.tok0 * z_row_stride * dtype_bytes(z_dtype),
                             z_dtype, z_row_stride, norm_weight, kNormEps,
                             static_cast<char*>(out) + (int64_t)a.tok0 * head_row * dtype_bytes(out_dtype), out_dtype,
                             head_row, stream);
      if (rc != RIA_OK) return rc;
    } else {
      if (out_dtype == RIA_DT_BF16)
        hipLaunchKernelGGL((chunk_scan_kernel<RIA_DT_BF16>), sgrid, dim3(512), 0, st, a);
      else if (out_dtype == RIA_DT_F16)
        hipLaunchKernelGGL((chunk_scan_kernel<RIA_DT_F16>), sgrid, dim3(512), 0, st, a);
      else
        hipLaunchKernelGGL((chunk_scan_kernel<RIA_DT_F32>), sgrid, dim3(512), 0, st, a);
      int rc = check_launch("ria_gdn_prefill");
      if (rc != RIA_OK) return rc;
    }
  }
  return RIA_OK;
}
