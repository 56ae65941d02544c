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
//                         from the conv ring for tokens before the prompt.
//   chunk_prep_kernel     phase A, one workgroup per (chunk, V head):
//                         l2norm, cumulative decay, K K^T and Q K^T on MFMA,
//                         blocked fp32 triangular inverse, U and W on MFMA.
//   chunk_scan_kernel     phase B, one workgroup per (V head, 16 state
//                         columns), sequential over chunks; the fp32 state
//                         block stays in LDS.
//   conv_ring_tail_kernel writes the last inputs into the conv ring.
//
// MFMA precision: every product runs on bf16 MFMA 16x16x32 with both fp32
// operands split as hi + lo bf16 (hi*hi + hi*lo + lo*hi, ~2^-16 relative);
// the cumulative decay, exponentials and the triangular inverse are fp32.
#include <math.h>

#include "ria_common.h"

namespace ria {

constexpr int kChunk = 64;
constexpr int kDim = kGdnHeadDim;  // 128
constexpr int kPadQ = 132;          // fp32 row stride of q / k / v tiles in LDS
constexpr int kPadT = 68;           // fp32 row stride of the 64x64 matrices in LDS

// Per (chunk, head) phase-A outputs, fp32, in this order inside one record.
constexpr int kRecWn = 0;                         // -W            [64][128]
constexpr int kRecU = kRecWn + kChunk * kDim;     //  U            [64][128]
constexpr int kRecQt = kRecU + kChunk * kDim;     //  exp(G) q     [64][128]
constexpr int kRecKtT = kRecQt + kChunk * kDim;   //  (exp(G_C-G) k)^T [128][64]
constexpr int kRecQK = kRecKtT + kDim * kChunk;   //  (q k^T) o D  [64][64]
constexpr int kRecGl = kRecQK + kChunk * kChunk;  //  exp(G_C)
constexpr int kRecFloats = kRecGl + 64;           // padded to 256 B

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
  float* rec;  // [seg_chunks, Hv, kRecFloats]
  void* out;   // [L, Hv, 128]
  int num_k_heads;
  int num_v_heads;
  int conv_dim;
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

// acc += A B with both operands as hi/lo pairs (the lo*lo term is dropped).
__device__ __forceinline__ f32x4 mfma3(u32x4 ah, u32x4 al, u32x4 bh, u32x4 bl, f32x4 acc) {
  acc = Kv16<RIA_DT_BF16>::mfma_k32(ah, bh, acc);
  acc = Kv16<RIA_DT_BF16>::mfma_k32(ah, bl, acc);
  acc = Kv16<RIA_DT_BF16>::mfma_k32(al, bh, acc);
  return acc;
}

__device__ __forceinline__ void load8(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// ---------------------------------------------------------------- conv
// One thread per channel, a tile of tokens per workgroup row.
constexpr int kConvTile = 64;

template <int XT>
__global__ __launch_bounds__(256) void prefill_conv_kernel(PrefillArgs a) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.conv_dim) return;
  const int t_begin = a.tok0 + blockIdx.y * kConvTile;
  const int t_end = min(t_begin + kConvTile, a.tok0 + a.seg_tokens);
  const uint2 wv = *reinterpret_cast<const uint2*>(a.conv_w + (int64_t)c * kConvTaps);
  const float w0 = bf16_bits_to_f32(wv.x & 0xffffu), w1 = bf16_bits_to_f32(wv.x >> 16);
  const float w2 = bf16_bits_to_f32(wv.y & 0xffffu), w3 = bf16_bits_to_f32(wv.y >> 16);
  auto input = [&](int t) -> float {
    if (t >= 0) return bf16_bits_to_f32(f32_to_bf16_bits(load_act<XT>(a.x, (int64_t)t * a.x_stride + c)));
    return bf16_bits_to_f32(a.conv_ring[((a.n0 + t) & 3) * a.conv_dim + c]);
  };
  float h0 = input(t_begin - 3), h1 = input(t_begin - 2), h2 = input(t_begin - 1);
  for (int t = t_begin; t < t_end; ++t) {
    const float xv = input(t);
    float acc = w0 * h0;
    acc = fmaf(w1, h1, acc);
    acc = fmaf(w2, h2, acc);
    acc = fmaf(w3, xv, acc);
    a.post[(int64_t)(t - a.tok0) * a.conv_dim + c] = f32_to_bf16_bits(silu_f(round_bf16(acc)));
    h0 = h1;
    h1 = h2;
    h2 = xv;
  }
}

// The inputs of the last min(L, 4) tokens go to their ring slots (after every
// conv tile has read the old history).
template <int XT>
__global__ __launch_bounds__(256) void conv_ring_tail_kernel(PrefillArgs a) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.conv_dim) return;
  for (int t = max(0, a.length - 4); t < a.length; ++t)
    a.conv_ring[((a.n0 + t) & 3) * a.conv_dim + c] =
        f32_to_bf16_bits(load_act<XT>(a.x, (int64_t)t * a.x_stride + c));
}

// ---------------------------------------------------------------- phase A
template <int XT, int GM>
__global__ __launch_bounds__(256) void chunk_prep_kernel(PrefillArgs a) {
  const int cl = blockIdx.x;  // chunk within the segment
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g4 = lane >> 4;
  const int chunk = a.chunk0 + cl;
  const int t0 = chunk * kChunk;  // absolute first token
  const int group = a.num_v_heads / a.num_k_heads;
  const int hk = h / group;
  const int kdim = a.num_k_heads * kDim;

  __shared__ __attribute__((aligned(16))) float smem[3 * kChunk * kPadQ + 2 * kChunk * kPadT + 4 * 16 * 17 + 5 * kChunk];
  float* qs = smem;                   // [64][kPadQ] q, then exp(G) q
  float* ks = qs + kChunk * kPadQ;    // [64][kPadQ] k
  float* vs = ks + kChunk * kPadQ;    // [64][kPadQ] v
  float* Lm = vs + kChunk * kPadQ;    // [64][kPadT] L
  float* Tm = Lm + kChunk * kPadT;    // [64][kPadT] T
  float* Xs = Tm + kChunk * kPadT;    // [4][16][17] per-wave scratch
  float* beta_s = Xs + 4 * 16 * 17;   // [64]
  float* G_s = beta_s + kChunk;       // [64]
  float* eg_s = G_s + kChunk;         // [64] exp(G)
  float* ss_s = eg_s + kChunk;        // [128] row sums of squares

  // 1. q, k, v rows (post-conv values as the reference sees them), zeros past L.
  for (int e = tid; e < kChunk * 3 * kDim; e += 256) {
    const int r = e / (3 * kDim), col = e % (3 * kDim);
    const int t = t0 + r;
    float val = 0.f;
    if (t < a.length) {
      int c;
      if (col < kDim) c = hk * kDim + col;
      else if (col < 2 * kDim) c = kdim + hk * kDim + (col - kDim);
      else c = 2 * kdim + h * kDim + (col - 2 * kDim);
      val = through_dtype<XT>(bf16_bits_to_f32(a.post[(int64_t)(t - a.tok0) * a.conv_dim + c]));
    }
    float* dst = col < kDim ? qs : (col < 2 * kDim ? ks : vs);
    dst[r * kPadQ + (col % kDim)] = val;
  }
  // 2. gates
  if (tid < kChunk) {
    const int t = t0 + tid;
    float beta = 0.f, g = 0.f;
    if (t < a.length) {
      const float ga = a.gate_a[(int64_t)t * a.gate_stride + h];
      const float gb = a.gate_b[(int64_t)t * a.gate_stride + h];
      if constexpr (GM == RIA_GATE_RAW) {
        beta = sigmoid_f(gb);
        g = -expf(a.A_log[h]) * softplus_f(ga + a.dt_bias[h]);
      } else {
        beta = gb;
        g = ga;
      }
    }
    beta_s[tid] = beta;
    G_s[tid] = g;
  }
  __syncthreads();
  // 3. cumulative decay (sequential, as torch.cumsum) and row sums of squares
  if (tid == 0) {
    float acc = 0.f;
    for (int i = 0; i < kChunk; ++i) {
      acc += G_s[i];
      G_s[i] = acc;
    }
  }
  {
    // waves 0-1: q rows, waves 2-3: k rows; 32 rows per wave
    float* base = wave < 2 ? qs : ks;
    const int r0 = (wave & 1) * 32;
    for (int r = 0; r < 32; ++r) {
      const float* row = base + (r0 + r) * kPadQ;
      const float s = wave_sum(mul_rn(row[lane], row[lane]) + mul_rn(row[lane + 64], row[lane + 64]));
      if (lane == 0) ss_s[(wave < 2 ? 0 : 64) + r0 + r] = s;
    }
  }
  __syncthreads();
  if (tid < kChunk) eg_s[tid] = expf(G_s[tid]);
  // 4. l2norm (q also scaled by 128^-0.5)
  for (int e = tid; e < 2 * kChunk * kDim; e += 256) {
    const int which = e / (kChunk * kDim), rem = e % (kChunk * kDim);
    const int r = rem / kDim, d = rem % kDim;
    float* p = (which == 0 ? qs : ks) + r * kPadQ + d;
    const float inv = 1.0f / sqrtf(ss_s[which * 64 + r] + 1e-6f);
    float y = mul_rn(*p, inv);
    if (which == 0) y = mul_rn(y, 0.08838834764831845f);
    *p = y;
  }
  __syncthreads();

  float* rec = a.rec + ((int64_t)cl * a.num_v_heads + h) * kRecFloats;

  // 5. K K^T -> L (strict lower, beta_i D_ij) and Q K^T -> (q k^T) o D (j <= i).
  // 10 lower tiles of each; wave w takes tiles (ti, tj) with index % 4 == w.
  for (int job = wave; job < 20; job += 4) {
    const bool is_q = job >= 10;
    int idx = job % 10, ti = 0;
    while (idx > ti) {
      idx -= ti + 1;
      ++ti;
    }
    const int tj = idx;
    const float* A = (is_q ? qs : ks) + (16 * ti + n) * kPadQ;
    const float* B = ks + (16 * tj + n) * kPadQ;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float av[8], bv[8];
      load8(A + 32 * s + 8 * g4, av);
      load8(B + 32 * s + 8 * g4, bv);
      u32x4 ah, al, bh, bl;
      split8(av, ah, al);
      split8(bv, bh, bl);
      acc = mfma3(ah, al, bh, bl, acc);
    }
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int i = 16 * ti + 4 * g4 + i4, j = 16 * tj + n;
      const float dec = j <= i ? expf(G_s[i] - G_s[j]) : 0.f;
      if (is_q) {
        rec[kRecQK + i * kChunk + j] = j <= i ? acc[i4] * dec : 0.f;
      } else {
        Lm[i * kPadT + j] = j < i ? beta_s[i] * acc[i4] * dec : 0.f;
      }
    }
  }
  // Q K^T tiles above the diagonal are zero.
  for (int e = tid; e < kChunk * kChunk; e += 256) {
    const int i = e / kChunk, j = e % kChunk;
    if ((j >> 4) > (i >> 4)) rec[kRecQK + e] = 0.f;
  }
  __syncthreads();

  // 6. T = (I + L)^-1, blocked 4x4 over 16x16 blocks.
  // 6a. diagonal blocks: wave w inverts block w; lane j (< 16) owns column j.
  if (n == lane) {  // lanes 0..15
    const int b0 = 16 * wave;
    float col[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) s = fmaf(Lm[(b0 + i) * kPadT + b0 + m], col[m], s);
      col[i] = (i == lane) ? 1.f : (i < lane ? 0.f : -s);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Tm[(b0 + i) * kPadT + b0 + lane] = col[i];
  }
  __syncthreads();
  // 6b. off-diagonal blocks by distance: T_ij = -T_ii (sum_{m=j}^{i-1} L_im T_mj)
  for (int dist = 1; dist < 4; ++dist) {
    const int bi = wave + dist, bj = wave;
    if (bi < 4) {
      float* X = Xs + wave * 16 * 17;
      // X = sum_m L_im T_mj ; lane computes 4 entries (r = lane/4*... )
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = lane * 4 + q4, r = e >> 4, c = e & 15;
        float s = 0.f;
        for (int bm = bj; bm < bi; ++bm)
#pragma unroll
          for (int m = 0; m < 16; ++m)
            s = fmaf(Lm[(16 * bi + r) * kPadT + 16 * bm + m], Tm[(16 * bm + m) * kPadT + 16 * bj + c], s);
        X[r * 17 + c] = s;
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = lane * 4 + q4, r = e >> 4, c = e & 15;
        float s = 0.f;
#pragma unroll
        for (int m = 0; m < 16; ++m) s = fmaf(Tm[(16 * bi + r) * kPadT + 16 * bi + m], X[m * 17 + c], s);
        Tm[(16 * bi + r) * kPadT + 16 * bj + c] = -s;
      }
    }
    __syncthreads();
  }
  // upper blocks of T are zero (read by the U/W products below)
  for (int e = tid; e < kChunk * kChunk; e += 256) {
    const int i = e / kChunk, j = e % kChunk;
    if ((j >> 4) > (i >> 4)) Tm[i * kPadT + j] = 0.f;
  }
  __syncthreads();

  // 7. U = T (beta v) and W = T (beta exp(G) k): 2 x 32 output tiles of 16x16.
  for (int job = wave; job < 64; job += 4) {
    const bool is_w = job >= 32;
    const int tt = (job & 31) >> 3, td = job & 7;  // token tile, dim tile
    const float* src = is_w ? ks : vs;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int nsteps = (16 * tt + 15) / 32 + 1;  // T is lower triangular
    for (int s = 0; s < nsteps; ++s) {
      float av[8], bv[8];
      load8(Tm + (16 * tt + n) * kPadT + 32 * s + 8 * g4, av);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = 32 * s + 8 * g4 + j;
        const float sc = is_w ? beta_s[t] * eg_s[t] : beta_s[t];
        bv[j] = src[t * kPadQ + 16 * td + n] * sc;
      }
      u32x4 ah, al, bh, bl;
      split8(av, ah, al);
      split8(bv, bh, bl);
      acc = mfma3(ah, al, bh, bl, acc);
    }
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int r = 16 * tt + 4 * g4 + i4, d = 16 * td + n;
      if (is_w) rec[kRecWn + r * kDim + d] = -acc[i4];
      else rec[kRecU + r * kDim + d] = acc[i4];
    }
  }
  // 8. exp(G) q, (exp(G_C - G) k)^T and exp(G_C)
  const float g_last = G_s[kChunk - 1];
  for (int e = tid; e < kChunk * kDim; e += 256) {
    const int r = e / kDim, d = e % kDim;
    rec[kRecQt + e] = qs[r * kPadQ + d] * eg_s[r];
    const int dd = e / kChunk, rr = e % kChunk;  // transposed walk for KtT
    rec[kRecKtT + e] = ks[rr * kPadQ + dd] * expf(g_last - G_s[rr]);
  }
  if (tid == 0) rec[kRecGl] = expf(g_last);
}

// ---------------------------------------------------------------- phase B
template <int OT>
__global__ __launch_bounds__(256) void chunk_scan_kernel(PrefillArgs a) {
  // Workgroup id -> (column block, head) with the 8 column blocks of a head
  // sharing an XCD (ids congruent mod 8 run on one XCD; 32 heads * cb + h).
  const int h = blockIdx.x % a.num_v_heads;
  const int cb = blockIdx.x / a.num_v_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g4 = lane >> 4;

  __shared__ float S32[kDim][17];                                  // state block S[:, cb*16 + c]
  __shared__ __attribute__((aligned(16))) uint16_t STh[16][kDim + 8];  // S^T hi / lo (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t STl[16][kDim + 8];
  __shared__ __attribute__((aligned(16))) uint16_t VTh[16][kChunk + 8];  // v'^T hi / lo (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t VTl[16][kChunk + 8];

  float* Sg = a.state + (int64_t)h * kDim * kDim + cb * 16;
  for (int e = tid; e < kDim * 16; e += 256) {
    const int r = e >> 4, c = e & 15;
    const float v = Sg[r * kDim + c];
    S32[r][c] = v;
    const uint16_t hb = f32_to_bf16_bits(v);
    STh[c][r] = hb;
    STl[c][r] = f32_to_bf16_bits(v - bf16_bits_to_f32(hb));
  }
  __syncthreads();

  for (int cl = 0; cl < a.seg_chunks; ++cl) {
    const int chunk = a.chunk0 + cl;
    const float* rec = a.rec + ((int64_t)cl * a.num_v_heads + h) * kRecFloats;
    // (i) v' = U + Wn S and o_inter = Qt S for token tile `wave`.
    f32x4 vn, oi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) vn[i4] = rec[kRecU + (16 * wave + 4 * g4 + i4) * kDim + cb * 16 + n];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 bh4 = *reinterpret_cast<const uint4*>(&STh[n][32 * s + 8 * g4]);
      const uint4 bl4 = *reinterpret_cast<const uint4*>(&STl[n][32 * s + 8 * g4]);
      const u32x4 bh = {bh4.x, bh4.y, bh4.z, bh4.w}, bl = {bl4.x, bl4.y, bl4.z, bl4.w};
      float av[8];
      u32x4 ah, al;
      load8(rec + kRecWn + (16 * wave + n) * kDim + 32 * s + 8 * g4, av);
      split8(av, ah, al);
      vn = mfma3(ah, al, bh, bl, vn);
      load8(rec + kRecQt + (16 * wave + n) * kDim + 32 * s + 8 * g4, av);
      split8(av, ah, al);
      oi = mfma3(ah, al, bh, bl, oi);
    }
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const uint16_t hb = f32_to_bf16_bits(vn[i4]);
      VTh[n][16 * wave + 4 * g4 + i4] = hb;
      VTl[n][16 * wave + 4 * g4 + i4] = f32_to_bf16_bits(vn[i4] - bf16_bits_to_f32(hb));
    }
    __syncthreads();
    // (ii) o = o_inter + (q k^T o D) v'
    const int nsteps = (16 * wave + 15) / 32 + 1;
    for (int s = 0; s < nsteps; ++s) {
      const uint4 bh4 = *reinterpret_cast<const uint4*>(&VTh[n][32 * s + 8 * g4]);
      const uint4 bl4 = *reinterpret_cast<const uint4*>(&VTl[n][32 * s + 8 * g4]);
      const u32x4 bh = {bh4.x, bh4.y, bh4.z, bh4.w}, bl = {bl4.x, bl4.y, bl4.z, bl4.w};
      float av[8];
      u32x4 ah, al;
      load8(rec + kRecQK + (16 * wave + n) * kChunk + 32 * s + 8 * g4, av);
      split8(av, ah, al);
      oi = mfma3(ah, al, bh, bl, oi);
    }
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int t = chunk * kChunk + 16 * wave + 4 * g4 + i4;
      if (t < a.length) store_act<OT>(a.out, ((int64_t)t * a.num_v_heads + h) * kDim + cb * 16 + n, oi[i4]);
    }
    // (iii) S <- exp(G_C) S + Kt^T v' for dk tiles 2*wave, 2*wave + 1.
    const float gl = rec[kRecGl];
#pragma unroll
    for (int tk = 0; tk < 2; ++tk) {
      const int dt = 2 * wave + tk;
      f32x4 sn;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) sn[i4] = gl * S32[16 * dt + 4 * g4 + i4][n];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint4 bh4 = *reinterpret_cast<const uint4*>(&VTh[n][32 * s + 8 * g4]);
        const uint4 bl4 = *reinterpret_cast<const uint4*>(&VTl[n][32 * s + 8 * g4]);
        const u32x4 bh = {bh4.x, bh4.y, bh4.z, bh4.w}, bl = {bl4.x, bl4.y, bl4.z, bl4.w};
        float av[8];
        u32x4 ah, al;
        load8(rec + kRecKtT + (16 * dt + n) * kChunk + 32 * s + 8 * g4, av);
        split8(av, ah, al);
        sn = mfma3(ah, al, bh, bl, sn);
      }
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int r = 16 * dt + 4 * g4 + i4;
        S32[r][n] = sn[i4];
        const uint16_t hb = f32_to_bf16_bits(sn[i4]);
        STh[n][r] = hb;
        STl[n][r] = f32_to_bf16_bits(sn[i4] - bf16_bits_to_f32(hb));
      }
    }
    __syncthreads();
  }
  for (int e = tid; e < kDim * 16; e += 256) {
    const int r = e >> 4, c = e & 15;
    Sg[r * kDim + c] = S32[r][c];
  }
}

static bool valid_dtype(int dt) { return dt == RIA_DT_BF16 || dt == RIA_DT_F16 || dt == RIA_DT_F32; }

int64_t prefill_segment_bytes(int num_k_heads, int num_v_heads, int seg_tokens) {
  const int64_t conv_dim = (int64_t)(2 * num_k_heads + num_v_heads) * kDim;
  const int64_t chunks = (seg_tokens + kChunk - 1) / kChunk;
  const int64_t post = ((int64_t)chunks * kChunk * conv_dim * 2 + 255) / 256 * 256;
  return post + chunks * num_v_heads * (int64_t)kRecFloats * 4;
}

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
  a.out = out;
  a.num_k_heads = num_k_heads;
  a.num_v_heads = num_v_heads;
  a.conv_dim = conv_dim;
  const int64_t post_bytes = ((int64_t)seg_chunks * kChunk * conv_dim * 2 + 255) / 256 * 256;
  a.post = static_cast<uint16_t*>(workspace);
  a.rec = reinterpret_cast<float*>(static_cast<char*>(workspace) + post_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);

  const int total_chunks = (length + kChunk - 1) / kChunk;
  for (int c0 = 0; c0 < total_chunks; c0 += seg_chunks) {
    a.chunk0 = c0;
    a.seg_chunks = min(seg_chunks, total_chunks - c0);
    a.tok0 = c0 * kChunk;
    a.seg_tokens = min(a.seg_chunks * kChunk, length - a.tok0);
    dim3 cgrid((conv_dim + 255) / 256, (a.seg_tokens + kConvTile - 1) / kConvTile);
    dim3 pgrid(a.seg_chunks, num_v_heads);
    dim3 sgrid(num_v_heads * (kDim / 16));
#define RIA_PREFILL_PHASES(XT_)                                                                          \
  hipLaunchKernelGGL((prefill_conv_kernel<XT_>), cgrid, dim3(256), 0, st, a);                           \
  if (gate_mode == RIA_GATE_RAW)                                                                        \
    hipLaunchKernelGGL((chunk_prep_kernel<XT_, RIA_GATE_RAW>), pgrid, dim3(256), 0, st, a);      \
  else                                                                                                  \
    hipLaunchKernelGGL((chunk_prep_kernel<XT_, RIA_GATE_PRECOMPUTED>), pgrid, dim3(256), 0, st, a)
    if (x_dtype == RIA_DT_BF16) {
      RIA_PREFILL_PHASES(RIA_DT_BF16);
    } else if (x_dtype == RIA_DT_F16) {
      RIA_PREFILL_PHASES(RIA_DT_F16);
    } else {
      RIA_PREFILL_PHASES(RIA_DT_F32);
    }
#undef RIA_PREFILL_PHASES
    if (out_dtype == RIA_DT_BF16)
      hipLaunchKernelGGL((chunk_scan_kernel<RIA_DT_BF16>), sgrid, dim3(256), 0, st, a);
    else if (out_dtype == RIA_DT_F16)
      hipLaunchKernelGGL((chunk_scan_kernel<RIA_DT_F16>), sgrid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((chunk_scan_kernel<RIA_DT_F32>), sgrid, dim3(256), 0, st, a);
    int rc = check_launch("ria_gdn_prefill");
    if (rc != RIA_OK) return rc;
  }
  dim3 rgrid((conv_dim + 255) / 256);
  if (x_dtype == RIA_DT_BF16)
    hipLaunchKernelGGL((conv_ring_tail_kernel<RIA_DT_BF16>), rgrid, dim3(256), 0, st, a);
  else if (x_dtype == RIA_DT_F16)
    hipLaunchKernelGGL((conv_ring_tail_kernel<RIA_DT_F16>), rgrid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((conv_ring_tail_kernel<RIA_DT_F32>), rgrid, dim3(256), 0, st, a);
  return check_launch("ria_gdn_prefill (conv ring)");
}
