// Full-attention decode over a paged bf16 KV cache for gfx950.
//
// Reference semantics (v2/src/router_ia/qwen36_attention_cache.py:285-373):
//   k_rot  = RoPE(k, tokens_seen) on dims [0, 64)           (:306, :154-162)
//   K, V  += k_rot, v  at slot `resident`                    (:334-373)
//   s_t    = q_rot . K_t * 256^-0.5  over every resident token (:312)
//   attn   = softmax(s) V ; out = attn * sigmoid(gate)       (:313-317)
// with query head h reading KV head h / 8 (repeat_interleave, :309-310).
//
// Decode is HBM-bound (2 KiB of KV per token per KV head pair, 8 FLOP/B), so
// the design goal is one streaming pass over K and V:
//   * pages: each (page, KV head) tile is 8 KiB.  K is stored in the MFMA
//     A-operand order [kk 8][g 4][tok 16][8 dims] (dim d -> kk = (d%64)/8,
//     g = d/64), so the eight 16-byte loads of a lane are each part of one
//     contiguous 1 KiB wavefront read; V is stored transposed,
//     [256 dim][16 tok], so the P V operand is a contiguous 512 B read.
//   * scores S^T = K Q^T on MFMA 16x16x32 bf16 (tokens x query heads, the
//     8 query heads of a KV head padded to 16); the output layout leaves each
//     lane with 4 tokens of one head, which is exactly the B operand of the
//     P V product, computed as O^T = V^T P^T on MFMA 16x16x16 bf16.  Softmax
//     statistics and O^T columns therefore live in the same lane and no
//     cross-lane transpose is needed.
//   * precision: K and V are exact 16-bit operands (bf16 or fp16 caches); q
//     and the probabilities P are fp32 values, each carried as a 16-bit pair
//     hi + lo (hi = round(x), lo = round(x - hi)), so every product runs
//     twice on MFMA and the operands keep ~16 (bf16) or ~22 (fp16) mantissa
//     bits.  The kernel is HBM-bound with MFMA to spare; a single bf16 q and
//     P alone would cost ~2^-9 relative error.
//   * split-K: a workgroup (4 waves) owns `split_tokens` tokens of one
//     (sequence, KV head); waves take pages round-robin with an online
//     softmax, merge through LDS and emit (max, sum, unnormalised acc); a
//     combine kernel merges the splits and applies the sigmoid gate.
#include <math.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "ria_common.h"

namespace ria {

constexpr int kMaxGroup = 16;  // query heads per KV head handled by one MFMA tile
constexpr int kTileElems = kPageTokens * kAttnHeadDim;  // 4096 bf16 per (page, KV head)

// Offset of K element (token t, dim d) inside its (page, KV head) tile.
__host__ __device__ __forceinline__ int k_tile_offset(int t, int d) {
  return ((((d & 63) >> 3) * 4 + (d >> 6)) * kPageTokens + t) * 8 + (d & 7);
}

struct AttnArgs {
  const void* q;
  int64_t q_stride;
  const void* gate;
  int64_t gate_stride;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int num_pages;
  const int32_t* page_table;
  int64_t pt_stride;
  const int32_t* seq_slot;
  const int32_t* positions;
  int32_t pos_scalar;
  const int32_t* ctx_lens;
  int32_t ctx_scalar;
  const float* inv_freq;
  int rope_dim;
  const float* q_norm_w;  // q_norm weight [256] f32, or null: q arrives normalised
  float scale;
  int split_tokens;
  int max_splits;
  int balanced;      // 1: stream-K partition of all (sequence, KV head) pages over the grid
  int batch;
  int32_t* ws_units; // balanced: [0] total pages, [1] pages per workgroup, [2 ..] page offset of each unit
  float* ws_stats;   // [parts][group][2]  (max in log2 units, sum)
  float* ws_acc;     // [parts][group][256]
  int num_q_heads;
  int num_kv_heads;
  int group;
  void* out;
  // fused append (ria_attn_decode_append): this token's k and v rows, in q's
  // dtype, go into slot ctx - 1 of each row (k_norm, RoPE at the row's
  // position) before the row attends
  const void* k_new;
  int64_t kn_stride;
  const void* v_new;
  int64_t vn_stride;
  const float* k_norm_w;  // k_norm weight [256] f32, or null
  int exclude_last;       // split-K: stop before each row's last token (the combine adds it)
  int kv_dtype;           // RIA_DT_* of the pages (the fused append rounds k and v to it)
};

struct AppendArgs {
  const void* k;
  int64_t k_stride;
  const void* v;
  int64_t v_stride;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int num_pages;
  const int32_t* page_table;
  int64_t pt_stride;
  const int32_t* seq_slot;
  const int32_t* positions;
  int32_t pos_scalar;
  const int32_t* slots;
  int32_t slot_scalar;
  const float* inv_freq;
  int rope_dim;
  const float* norm_w;  // k_norm weight [256] f32, or null: k arrives normalised
  int num_kv_heads;
  int seq_len;  // prompt append: tokens at positions (and slots) pos_scalar .. pos_scalar + seq_len - 1
  float* k_out; // one-token append: row b's k after k_norm and RoPE in fp32 (before the page rounding)
                // at k_out[(b * Hkv + kvh) * 256 + d], or null
  uint16_t* stage_k;  // prompt append from slot 0: the prompt's k and v also as fp16 tiles in page
  uint16_t* stage_v;  // layout, tile (logical page, KV head) at (page * Hkv + kvh) * 4096, or null
};

// RoPE of element d of a row: (x*cos + rotate_half(x)*sin) on [0, rope_dim),
// pass-through above (qwen36_attention_cache.py:154-162).
__device__ __forceinline__ float rope_elem(float xd, float partner, int d, int rope_dim, float pos,
                                           const float* inv_freq) {
  if (d >= rope_dim) return xd;
  const int half = rope_dim >> 1;
  const float ang = mul_rn(pos, inv_freq[d < half ? d : d - half]);
  const float c = cosf(ang), s = sinf(ang);
  const float rot = d < half ? -partner : partner;
  return add_rn(mul_rn(xd, c), mul_rn(rot, s));
}

// One workgroup per (sequence, KV head): optionally RMSNorm k (k_norm,
// qwen36_attention_cache.py:303-305), rotate it, write k and v into the page.
template <int KT, int VT, int KVT>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendArgs a) {
  const int b = blockIdx.x;
  const int kvh = blockIdx.y;
  const int d = threadIdx.x;
  const int row = a.seq_slot ? a.seq_slot[b] : b;
  const int pos = a.positions ? a.positions[b] : a.pos_scalar;
  const int slot = a.slots ? a.slots[b] : a.slot_scalar;
  __shared__ float k_s[kAttnHeadDim];
  __shared__ float ss_s[4];
  float kv = load_act<KT>(a.k, (int64_t)b * a.k_stride + kvh * kAttnHeadDim + d);
  const float vv = load_act<VT>(a.v, (int64_t)b * a.v_stride + kvh * kAttnHeadDim + d);
  if (a.norm_w) {  // uniform: one sum of squares over the 256 dims
    const float ss = wave_sum(mul_rn(kv, kv));
    if ((d & 63) == 0) ss_s[d >> 6] = ss;
    __syncthreads();
    kv = rmsnorm_elem<KT>(kv, rms_scale(ss_s[0] + ss_s[1] + ss_s[2] + ss_s[3], kAttnHeadDim), a.norm_w[d]);
  }
  k_s[d] = kv;
  __syncthreads();
  if (slot < 0 || slot / kPageTokens >= a.pt_stride) return;
  const int half = a.rope_dim >> 1;
  const float partner = d < a.rope_dim ? k_s[d < half ? d + half : d - half] : 0.f;
  const float kr = rope_elem(kv, partner, d, a.rope_dim, static_cast<float>(pos), a.inv_freq);
  if (a.k_out) a.k_out[((int64_t)b * a.num_kv_heads + kvh) * kAttnHeadDim + d] = kr;
  const int phys = a.page_table[(int64_t)row * a.pt_stride + slot / kPageTokens];
  if (phys < 0 || phys >= a.num_pages) return;  // host guarantees allocation; never write out of the pool
  const int off = slot % kPageTokens;
  const int64_t tile = (int64_t)phys * a.num_kv_heads + kvh;
  a.k_cache[tile * kTileElems + k_tile_offset(off, d)] = Kv16<KVT>::from_f32(kr);
  a.v_cache[(tile * kAttnHeadDim + d) * kPageTokens + off] = Kv16<KVT>::from_f32(vv);
}

// A prompt's append (one sequence, token i at position and slot
// pos_scalar + i), one workgroup per (page, KV head): thread d owns dim d of
// the page's 16 tokens and puts each through kv_append_kernel's arithmetic
// (the same sums of squares, k_norm, RoPE and rounding), so the pages get
// the same bits.  A page the prompt fills leaves as 16-byte stores: K
// through an LDS copy of the tile (each 16-byte piece is 8 dims of one
// token), V^T as each dim's 32-byte row; the first and last pages keep the
// tokens outside the prompt (per-token stores).
template <int KT, int VT, int KVT>
__global__ __launch_bounds__(256) void kv_append_page_kernel(AppendArgs a) {
  const int d = threadIdx.x, lane = d & 63, w = d >> 6;
  const int kvh = blockIdx.y;
  const int pg = a.pos_scalar / kPageTokens + static_cast<int>(blockIdx.x);  // page slot in the row
  const int s0 = pg * kPageTokens;
  const int t_lo = max(a.pos_scalar, s0) - s0, t_hi = min(a.pos_scalar + a.seq_len, s0 + kPageTokens) - s0;
  const int phys = a.page_table[pg];
  __shared__ float k_s[kPageTokens][kAttnHeadDim];
  __shared__ float cos_s[kPageTokens][32], sin_s[kPageTokens][32];  // the page's rotary table (rope_dim <= 64)
  __shared__ float ss_s[kPageTokens][4];
  __shared__ __attribute__((aligned(16))) uint16_t kt_s[kTileElems];
  __shared__ __attribute__((aligned(16))) uint16_t kt16_s[kTileElems];  // the fp16 copy (stage)
  float kv[kPageTokens], vv[kPageTokens];
#pragma unroll
  for (int i = 0; i < kPageTokens; ++i) {
    // prompt row of token i (tokens outside the prompt load row 0 and are zeroed)
    const bool in = i >= t_lo && i < t_hi;
    const int64_t r = in ? s0 + i - a.pos_scalar : 0;
    const float kx = load_act<KT>(a.k, r * a.k_stride + kvh * kAttnHeadDim + d);
    const float vx = load_act<VT>(a.v, r * a.v_stride + kvh * kAttnHeadDim + d);
    kv[i] = in ? kx : 0.f;
    vv[i] = in ? vx : 0.f;
  }
  // checked after the row loads are out, so they do not wait for the entry
  if (phys < 0 || phys >= a.num_pages) return;  // host guarantees allocation; never write out of the pool
  const int64_t tile = (int64_t)phys * a.num_kv_heads + kvh;
  // cos / sin of the page's 16 positions x 32 frequencies, two per thread
  // (rope_elem's angle and functions), instead of 32 on each of wave 0's
  // lanes while the other waves wait
  const bool rope_table = a.rope_dim <= 64;
  if (rope_table) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = 8 * h + (d >> 5), f = d & 31;
      if (2 * f < a.rope_dim) {
        const float ang = mul_rn(static_cast<float>(s0 + i), a.inv_freq[f]);
        cos_s[i][f] = cosf(ang);
        sin_s[i][f] = sinf(ang);
      }
    }
  }
  if (a.norm_w) {  // per token: one sum of squares over the 256 dims, waves in order
    const float wn = a.norm_w[d];
#pragma unroll
    for (int i = 0; i < kPageTokens; ++i) {
      const float ss = wave_sum(mul_rn(kv[i], kv[i]));
      if (lane == 0) ss_s[i][w] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPageTokens; ++i)
      kv[i] = rmsnorm_elem<KT>(kv[i], rms_scale(ss_s[i][0] + ss_s[i][1] + ss_s[i][2] + ss_s[i][3], kAttnHeadDim),
                               wn);
  }
#pragma unroll
  for (int i = 0; i < kPageTokens; ++i) k_s[i][d] = kv[i];
  __syncthreads();
  const int half = a.rope_dim >> 1;
  const int pd = d < half ? d + half : d - half;
#pragma unroll
  for (int i = 0; i < kPageTokens; ++i) {
    const float partner = d < a.rope_dim ? k_s[i][pd] : 0.f;
    float kr;
    if (rope_table) {
      const int f = d < half ? d : d - half;
      kr = d < a.rope_dim ? add_rn(mul_rn(kv[i], cos_s[i][f]), mul_rn(d < half ? -partner : partner, sin_s[i][f]))
                          : kv[i];
    } else {
      kr = rope_elem(kv[i], partner, d, a.rope_dim, static_cast<float>(s0 + i), a.inv_freq);
    }
    kt_s[k_tile_offset(i, d)] = Kv16<KVT>::from_f32(kr);
    if (a.stage_k) kt16_s[k_tile_offset(i, d)] = Kv16<RIA_DT_F16>::from_f32(kr);
  }
  __syncthreads();
  if (a.stage_k) {
    // the whole tile (a prompt from slot 0 starts every page at token 0;
    // tokens past its end hold zeros)
    const int64_t st_tile = (int64_t)pg * a.num_kv_heads + kvh;
    uint4* sk = reinterpret_cast<uint4*>(a.stage_k + st_tile * kTileElems);
    sk[d] = reinterpret_cast<const uint4*>(kt16_s)[d];
    sk[d + 256] = reinterpret_cast<const uint4*>(kt16_s)[d + 256];
    uint32_t pk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      pk[j] = static_cast<uint32_t>(Kv16<RIA_DT_F16>::from_f32(vv[2 * j])) |
              (static_cast<uint32_t>(Kv16<RIA_DT_F16>::from_f32(vv[2 * j + 1])) << 16);
    uint4* sv = reinterpret_cast<uint4*>(a.stage_v + (st_tile * kAttnHeadDim + d) * kPageTokens);
    sv[0] = uint4{pk[0], pk[1], pk[2], pk[3]};
    sv[1] = uint4{pk[4], pk[5], pk[6], pk[7]};
  }
  uint16_t* kt = a.k_cache + tile * kTileElems;
  uint16_t* vt = a.v_cache + (tile * kAttnHeadDim + d) * kPageTokens;
  if (t_lo == 0 && t_hi == kPageTokens) {
    const uint4* src = reinterpret_cast<const uint4*>(kt_s);
    reinterpret_cast<uint4*>(kt)[d] = src[d];
    reinterpret_cast<uint4*>(kt)[d + 256] = src[d + 256];
    uint32_t pk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      pk[j] = static_cast<uint32_t>(Kv16<KVT>::from_f32(vv[2 * j])) |
              (static_cast<uint32_t>(Kv16<KVT>::from_f32(vv[2 * j + 1])) << 16);
    reinterpret_cast<uint4*>(vt)[0] = uint4{pk[0], pk[1], pk[2], pk[3]};
    reinterpret_cast<uint4*>(vt)[1] = uint4{pk[4], pk[5], pk[6], pk[7]};
  } else {
#pragma unroll
    for (int e = d; e < kTileElems / 8; e += 256) {  // piece e: 8 dims of token e % 16
      const int i = e % kPageTokens;
      if (i >= t_lo && i < t_hi) reinterpret_cast<uint4*>(kt)[e] = reinterpret_cast<const uint4*>(kt_s)[e];
    }
#pragma unroll
    for (int i = 0; i < kPageTokens; ++i)
      if (i >= t_lo && i < t_hi) vt[i] = Kv16<KVT>::from_f32(vv[i]);
  }
}

// Scalar (SMEM) load of a wave-uniform index from a buffer this kernel never
// writes (positions, context lengths, rows, page tables): it is counted apart
// from the vector loads, so waiting for it does not wait for K/V in flight.
__device__ __forceinline__ int32_t ld_uniform(const int32_t* p, int64_t i) {
  return ((const __attribute__((address_space(4))) int32_t*)p)[i];
}

// Pages of the context of batch row b (never past the row's page-table entries).
__device__ __forceinline__ int row_ctx(const AttnArgs& a, int b) {
  return min(a.ctx_lens ? a.ctx_lens[b] : a.ctx_scalar, (int)min<int64_t>(a.pt_stride * kPageTokens, 1 << 30));
}

// Balanced partition: unit u = b * Hkv + kvh owns pages [off[u], off[u + 1])
// of one global page stream of `total` pages; workgroup w takes pages
// [w * chunk, (w + 1) * chunk).  Workgroup w's partial for unit u lives at
// index w + u, which is unique because the (w, u) pairs that meet form a
// monotone staircase.
//
// When few units share the grid (units * kPadUnitsRatio <= workgroups), each
// unit's range is padded to whole chunks, so no workgroup straddles two
// units: a straddling workgroup runs the q prologue and the merge twice, and
// at small batches, where every workgroup streams only a few pages, it ends
// last.  The chunk is then sized over workgroups - units, which leaves room
// for the padding (at most one partial chunk per unit).
constexpr int kMaxBalancedUnits = 4096;
constexpr int kMinChunkPages = 4;  // 64 tokens: small batches still spread over the CUs
constexpr int kPadUnitsRatio = 32;

// Inclusive scan of one value per lane over a wave.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(v, off, 64);
    if (lane >= off) v += y;
  }
  return v;
}

// Inclusive block scan of up to 256 per-thread values through LDS; returns
// the exclusive prefix of this thread's value and the block total.
__device__ int block_exclusive_scan(int v, int* scratch, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) scratch[wave] = x;
  lds_barrier();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += scratch[w];
  *total = scratch[0] + scratch[1] + scratch[2] + scratch[3];
  lds_barrier();
  return base + x - v;
}

template <int QT, int KVT, bool BALANCED, bool QNORM>
__global__ __launch_bounds__(256, 2) void attn_splitk_kernel(AttnArgs a) {
  using KV = Kv16<KVT>;
  const int G = a.group;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;   // MFMA column: query head (scores) / dim row (PV)
  const int g4 = lane >> 4;  // lane group

  // LDS: the fp32 rotated query rows share space with the end-of-range merge.
  __shared__ float sm_o[4][8][kAttnHeadDim];  // group <= 8 on this path (checked on the host)
  __shared__ uint4 q_pk[2][8][64];            // bf16 Q operand hi / lo, [part][kk][lane]
  __shared__ float sm_m[4][kMaxGroup];
  __shared__ float sm_l[4][kMaxGroup];
  __shared__ float qn_s[8];                   // per-head RMSNorm scale of q
  float (*q_lds)[kAttnHeadDim] = sm_o[0];
  // Scores are kept in log2 units: s2 = (q . k) * scale * log2(e).
  const float sl2 = a.scale * 1.4426950408889634f;
  // Per-launch constants: the RoPE frequency of this thread's rotary dim and
  // the q_norm weights of its dim and RoPE partner.
  const float ifreq = a.rope_dim == 64 ? a.inv_freq[tid & 31] : 0.f;
  float w_self = 0.f, w_partner = 0.f;
  if constexpr (QNORM) {
    w_self = a.q_norm_w[tid];
    w_partner = a.q_norm_w[tid ^ 32];
  }

  // One (batch row, KV head, token range [tok0, min(context, tok_hi))) -> partial `part`.
  auto process = [&](int b, int kvh, int tok0, int tok_hi, int64_t part) {
    // Every load that depends only on the unit is issued at once: the
    // group's q rows (heads unrolled to the largest group, 8; heads past the
    // group re-read the last one, so no load waits inside a branch for its
    // own conversion), the position, the row, the context and this wave's
    // first page-table entry.  The first page's K/V loads follow, so they are
    // in flight while q is normalised, rotated and packed (at small batches a
    // wave streams only a page or two).
    // (an opaque copy of the thread index keeps the prologue's addresses from
    // being hoisted out of the unit loop and held across the page loop)
    int t = tid;
    asm volatile("" : "+v"(t));
    const bool rope = a.rope_dim == 64;
    float qx[8], qp[8];
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      const int64_t base = (int64_t)b * a.q_stride + (int64_t)(kvh * G + min(h, G - 1)) * kAttnHeadDim;
      qx[h] = load_act<QT>(a.q, base + t);
      qp[h] = QNORM ? 0.f : load_act<QT>(a.q, base + (t ^ 32));
    }
    const int page0 = tok0 / kPageTokens;
    const int64_t pfirst = min<int64_t>(page0 + __builtin_amdgcn_readfirstlane(wave), a.pt_stride - 1);
    int row = b, phys_first;  // phys_first is used only if the wave has a page
    if (a.seq_slot) {         // indirected rows: the table row is known only after this load
      row = ld_uniform(a.seq_slot, b);
      phys_first = ld_uniform(a.page_table + (int64_t)row * a.pt_stride, pfirst);
    } else {
      phys_first = ld_uniform(a.page_table + (int64_t)b * a.pt_stride, pfirst);
    }
    const int posi = a.positions ? ld_uniform(a.positions, b) : a.pos_scalar;
    const int ctx = min(a.ctx_lens ? ld_uniform(a.ctx_lens, b) : a.ctx_scalar,
                        static_cast<int>(min<int64_t>(a.pt_stride * kPageTokens, 1 << 30)));
    const int32_t* pt = a.page_table + (int64_t)row * a.pt_stride;
    // fused append: the row's last token (slot ctx - 1, appended by this
    // step) is left to the combine launch, which computes it from the inputs
    const int tok1 = min(a.exclude_last ? ctx - 1 : ctx, tok_hi);
    const int page_end = (tok1 + kPageTokens - 1) / kPageTokens;

    auto load_tile = [&](int phys, u32x4 (&kr)[8], u32x2 (&vr)[16]) {
      phys = (phys < 0 || phys >= a.num_pages) ? 0 : phys;  // unallocated entries never fault
      const int64_t tile = (int64_t)phys * a.num_kv_heads + kvh;
      const u32x4* kp = reinterpret_cast<const u32x4*>(a.k_cache + tile * kTileElems) + lane;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) kr[kk] = ld_stream(kp + kk * 64);
      const uint16_t* vp = a.v_cache + tile * kTileElems + n * kPageTokens + 4 * g4;
#pragma unroll
      for (int db = 0; db < 16; ++db) vr[db] = ld_stream(reinterpret_cast<const u32x2*>(vp + db * 16 * kPageTokens));
    };

    u32x4 kA[8], kB[8];
    u32x2 vA[16], vB[16];
    int p = page0 + __builtin_amdgcn_readfirstlane(wave);  // wave-uniform: the page loop branches on scalars
    if (p < page_end) load_tile(phys_first, kA, vA);
    lds_barrier();  // the previous range's merge has been read out of sm_o

    // ---- Q: rotate the group's query heads into LDS (one thread per dim).
    float rc = 1.f, rs = 0.f;
    if (rope && t < 64) sincosf(mul_rn(static_cast<float>(posi), ifreq), &rs, &rc);
    if constexpr (QNORM) {
      // q_norm (qwen36_attention_cache.py:302-304) before RoPE: raw rows into
      // the second merge slice (free until this range's merge), one wave per
      // head for the sum of squares, then each thread normalises its dim (and
      // its RoPE partner) and rotates.
      const int tl = t & 63, tw = t >> 6;
      float (*raw)[kAttnHeadDim] = sm_o[1];
#pragma unroll
      for (int h = 0; h < 8; ++h)
        if (h < G) raw[h][t] = qx[h];
      lds_barrier();
      for (int h = tw; h < G; h += 4) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < kAttnHeadDim; j += 64) ss = add_rn(ss, mul_rn(raw[h][j + tl], raw[h][j + tl]));
        ss = wave_sum(ss);
        if (tl == 0) qn_s[h] = rms_scale(ss, kAttnHeadDim);
      }
      lds_barrier();
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        if (h < G) {
          float x = rmsnorm_elem<QT>(qx[h], qn_s[h], w_self);
          if (rope && t < 64) {
            const float partner = rmsnorm_elem<QT>(raw[h][t ^ 32], qn_s[h], w_partner);
            x = add_rn(mul_rn(x, rc), mul_rn(t < 32 ? -partner : partner, rs));
          }
          q_lds[h][t] = x;
        }
      }
    } else {
#pragma unroll
      for (int h = 0; h < 8; ++h) {
        if (h < G) {
          float x = qx[h];
          if (rope && t < 64) x = add_rn(mul_rn(x, rc), mul_rn(t < 32 ? -qp[h] : qp[h], rs));
          q_lds[h][t] = x;
        }
      }
    }
    lds_barrier();
    // Pack the B operand: lane (head n, group g4) holds dims 64*g4 + 8*kk + j,
    // as a bf16 hi part and a bf16 remainder.
    {
      const int kk0 = wave * 2;  // each wave packs two kk blocks
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        uint32_t wh[4], wl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x0 = n < G ? q_lds[n & 7][64 * g4 + 8 * (kk0 + k2) + 2 * j] : 0.f;
          const float x1 = n < G ? q_lds[n & 7][64 * g4 + 8 * (kk0 + k2) + 2 * j + 1] : 0.f;
          const uint16_t h0 = KV::from_f32(x0), h1 = KV::from_f32(x1);
          const uint16_t l0 = KV::from_f32(x0 - KV::to_f32(h0));
          const uint16_t l1 = KV::from_f32(x1 - KV::to_f32(h1));
          wh[j] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
          wl[j] = static_cast<uint32_t>(l0) | (static_cast<uint32_t>(l1) << 16);
        }
        q_pk[0][kk0 + k2][lane] = uint4{wh[0], wh[1], wh[2], wh[3]};
        q_pk[1][kk0 + k2][lane] = uint4{wl[0], wl[1], wl[2], wl[3]};
      }
    }
    lds_barrier();

    f32x4 o[16];
#pragma unroll
    for (int db = 0; db < 16; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    auto compute_page = [&](int p, u32x4 (&kr)[8], u32x2 (&vr)[16]) {
      // Re-read the Q operand from LDS every page (an opaque offset keeps the
      // compiler from hoisting 64 loop-invariant VGPRs out of the page loop).
      int qoff = lane;
      asm volatile("" : "+v"(qoff));
      f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const uint4 qh = q_pk[0][kk][qoff], ql = q_pk[1][kk][qoff];
        sc = KV::mfma_k32(kr[kk], u32x4{qh.x, qh.y, qh.z, qh.w}, sc);
        sc = KV::mfma_k32(kr[kk], u32x4{ql.x, ql.y, ql.z, ql.w}, sc);
      }
      const int t_base = p * kPageTokens + 4 * g4;
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = (t_base + i < tok1) ? sc[i] * sl2 : -INFINITY;
        mx = fmaxf(mx, sc[i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // Lazy rescale: keep the reference max while the page max stays within
      // 2^8 of it, so the accumulator is rescaled only when it has to be.
      const bool grow = mx > m_run + 8.0f;
      if (__any(grow)) {
        const float m_new = grow ? mx : m_run;
        const float alpha = exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 16; ++db) o[db] *= alpha;
        m_run = m_new;
      }
      uint16_t ph[4], plo[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pr = exp2f(sc[i] - m_run);
        l_run += pr;
        ph[i] = KV::from_f32(pr);
        plo[i] = KV::from_f32(pr - KV::to_f32(ph[i]));
      }
      const u32x2 pb = {ph[0] | (uint32_t(ph[1]) << 16), ph[2] | (uint32_t(ph[3]) << 16)};
      const u32x2 pl = {plo[0] | (uint32_t(plo[1]) << 16), plo[2] | (uint32_t(plo[3]) << 16)};
      if ((p + 1) * kPageTokens > tok1) {
        // Tokens past the end of the range carry whatever the page holds;
        // zero their V so 0 * garbage cannot reach the accumulator.
#pragma unroll
        for (int db = 0; db < 16; ++db) {
          uint32_t lo = vr[db].x, hi = vr[db].y;
          if (t_base + 0 >= tok1) lo &= 0xffff0000u;
          if (t_base + 1 >= tok1) lo &= 0x0000ffffu;
          if (t_base + 2 >= tok1) hi &= 0xffff0000u;
          if (t_base + 3 >= tok1) hi &= 0x0000ffffu;
          vr[db] = u32x2{lo, hi};
        }
      }
#pragma unroll
      for (int db = 0; db < 16; ++db) {
        o[db] = KV::mfma_k16(vr[db], pb, o[db]);
        o[db] = KV::mfma_k16(vr[db], pl, o[db]);
      }
    };

    // Pages wave, wave+4, ...: the next page's loads are issued before the
    // current page is consumed (two register buffers, loop unrolled by two),
    // and the page-table entry of the page after it one page earlier still,
    // so issuing a page's loads never waits for the loads in flight.
    if (p < page_end) {
      int phys_next = pt[min(p + 4, page_end - 1)];
      while (true) {
        int pn = p + 4;
        if (pn < page_end) {
          const int ph = phys_next;
          phys_next = pt[min(pn + 4, page_end - 1)];
          load_tile(ph, kB, vB);
        }
        compute_page(p, kA, vA);
        if (pn >= page_end) break;
        p = pn;
        pn = p + 4;
        if (pn < page_end) {
          const int ph = phys_next;
          phys_next = pt[min(pn + 4, page_end - 1)];
          load_tile(ph, kA, vA);
        }
        compute_page(p, kB, vB);
        if (pn >= page_end) break;
        p = pn;
      }
    }
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);

    // ---- merge the four waves through LDS (q_lds is dead: every wave passed the barrier above)
    if (g4 == 0 && n < G) {
      sm_m[wave][n] = m_run;
      sm_l[wave][n] = l_run;
    }
    if (n < G) {
#pragma unroll
      for (int db = 0; db < 16; ++db) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sm_o[wave][n & 7][db * 16 + 4 * g4 + i] = o[db][i];
      }
    }
    lds_barrier();
    // Unrolled over the (at most 8) heads so every head's LDS reads issue at
    // once; heads past the group read unused LDS and store nothing.
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, sm_m[w][h]);
      float acc = 0.f, L = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float wt = (sm_m[w][h] == -INFINITY) ? 0.f : exp2f(sm_m[w][h] - M);
        acc = fmaf(wt, sm_o[w][h][tid], acc);
        L = fmaf(wt, sm_l[w][h], L);
      }
      if (h < G) {
        a.ws_acc[(part * G + h) * kAttnHeadDim + tid] = acc;
        if (tid == 0) {
          a.ws_stats[(part * G + h) * 2 + 0] = M;
          a.ws_stats[(part * G + h) * 2 + 1] = L;
        }
      }
    }
  };

  if constexpr (!BALANCED) {
    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int ctx = row_ctx(a, b);
    const int tok0 = split * a.split_tokens;
    if (tok0 >= ctx) return;
    process(b, kvh, tok0, tok0 + a.split_tokens, ((int64_t)b * a.num_kv_heads + kvh) * a.max_splits + split);
  } else {
    // ---- page offsets of every unit (u = b * Hkv + kvh) in LDS
    __shared__ int off[kMaxBalancedUnits + 1];
    __shared__ int scan_scratch[4];
    const int units = a.batch * a.num_kv_heads;
    const int per = (units + 255) / 256;  // units per thread (<= 16)
    const int nwg = static_cast<int>(gridDim.x);
    const int w = static_cast<int>(blockIdx.x);
    const int ctx_cap = static_cast<int>(min<int64_t>(a.pt_stride * kPageTokens, 1 << 30));
    // pages a unit streams: its resident tokens (with the fused append the
    // row's last token is left to the combine launch)
    const int xl = a.exclude_last ? 1 : 0;
    auto unit_pages = [&](int ctx) { return (max(min(ctx, ctx_cap) - xl, 0) + kPageTokens - 1) / kPageTokens; };
    int total = 0, chunk, first_unit;
    if (units <= 64) {
      // Up to 64 units every wave computes the partition on its own, one
      // unit per lane (wave scans: no block-wide LDS pass and no barrier), so
      // the first K/V loads wait only for the context lengths and the page
      // table.  Every wave writes the same offsets to LDS and reads back only
      // what it wrote itself.
      int pg = 0;
      if (lane < units) pg = unit_pages(a.ctx_lens ? a.ctx_lens[lane / a.num_kv_heads] : a.ctx_scalar);
      int incl = wave_inclusive_scan(pg);
      total = __builtin_amdgcn_readlane(incl, 63);
      const bool padded = units * kPadUnitsRatio <= nwg;
      chunk = max((total + nwg - 1) / nwg, kMinChunkPages);
      if (padded) {
        // the smallest chunk at which every unit, padded to whole chunks,
        // still fits the grid (the bound over workgroups - units always does)
        const int c_fit = max((total + nwg - units - 1) / (nwg - units), kMinChunkPages);
        for (; chunk < c_fit; ++chunk)
          if (__builtin_amdgcn_readlane(wave_inclusive_scan((pg + chunk - 1) / chunk), 63) <= nwg) break;
        pg = (pg + chunk - 1) / chunk * chunk;
        incl = wave_inclusive_scan(pg);
        total = __builtin_amdgcn_readlane(incl, 63);
      }
      const int excl = incl - pg;
      if (lane < units) off[lane] = excl;
      if (lane == 0) off[units] = total;
      __builtin_amdgcn_wave_barrier();
      // first unit containing page w * chunk: the highest lane with off <= it
      const uint64_t at_or_before = __ballot(lane < units && excl <= w * chunk);
      first_unit = 63 - __clzll(at_or_before);
    } else {
      int upages[16];
      if (a.ctx_lens) {  // unconditional loads (clamped unit), masked below
#pragma unroll
        for (int i = 0; i < 16; ++i) upages[i] = a.ctx_lens[min(tid * per + i, units - 1) / a.num_kv_heads];
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) upages[i] = a.ctx_scalar;
      }
      int mine = 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int u = tid * per + i;
        upages[i] = (i < per && u < units) ? unit_pages(upages[i]) : 0;
        mine += upages[i];
      }
      int run = block_exclusive_scan(mine, scan_scratch, &total);
      const bool padded = units * kPadUnitsRatio <= nwg;
      chunk = max((total + (padded ? nwg - units : nwg) - 1) / (padded ? nwg - units : nwg), kMinChunkPages);
      if (padded) {  // each unit rounded up to whole chunks
        mine = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          upages[i] = (upages[i] + chunk - 1) / chunk * chunk;
          mine += upages[i];
        }
        run = block_exclusive_scan(mine, scan_scratch, &total);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int u = tid * per + i;
        if (i < per && u < units) {
          off[u] = run;
          run += upages[i];
        }
      }
      if (tid == (units - 1) / per) off[units] = run;  // the thread that holds the last unit
      lds_barrier();
      // first unit containing page w * chunk: the last u with off[u] <= it
      int lo = 0, hi = units - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= w * chunk) lo = mid; else hi = mid - 1;
      }
      first_unit = lo;
    }
    if (blockIdx.x == 0) {
      // publish the partition for the combine kernel
      for (int u = tid; u <= units; u += 256) a.ws_units[2 + u] = off[u];
      if (tid == 0) {
        a.ws_units[0] = total;
        a.ws_units[1] = chunk;
      }
    }
    const int p0 = w * chunk;
    if (p0 >= total) return;
    const int p1 = min(p0 + chunk, total);
    // (the unit and its page range come from LDS, which the compiler treats
    // as per-lane: readfirstlane makes them scalar, so the unit's own loads
    // in process() are scalar loads)
    for (int u = __builtin_amdgcn_readfirstlane(first_unit); u < units; ++u) {
      const int ou = __builtin_amdgcn_readfirstlane(off[u]);
      if (ou >= p1) break;
      const int a0 = max(ou, p0) - ou, a1 = min(__builtin_amdgcn_readfirstlane(off[u + 1]), p1) - ou;  // unit-local pages
      if (a1 <= a0) continue;
      const int b = u / a.num_kv_heads, kvh = u % a.num_kv_heads;
      process(b, kvh, a0 * kPageTokens, a1 * kPageTokens, (int64_t)w + u);
    }
  }
}

// Fused append, in the combine launch of (row b, query head h): the row's new
// token at slot ctx - 1 (the split-K launch stopped before it).  Two stages:
// new_token_load issues every global load the token needs (so the combine
// issues them before its partials and they arrive together), and
// new_token_finish, called by every thread of the workgroup (it holds
// barriers; threads tid < 256 own dim tid), does the arithmetic.  k goes
// through kv_append_kernel's arithmetic (k_norm, RoPE, rounding to the page
// dtype), so the page gets the same bits as a separate append; q through the
// split-K prologue's (q_norm, RoPE).  new_token_finish returns the token's
// score with head h in log2 units (every thread) and leaves its rounded v in
// v_s; with write_cache the token's k and v go into the page.
struct NewTokenIn {
  float qv, kv, vv;    // dim d of the raw q (head h), k and v (its KV head)
  float qn_w, kn_w;    // q_norm / k_norm weights of dim d (when present)
  float fq, fk;        // inverse frequencies of q's and k's rotation of dim d
  int posi, ctx, phys; // position, context, physical page of slot ctx - 1
};

template <int QT>
__device__ __forceinline__ NewTokenIn new_token_load(const AttnArgs& a, int b, int h, bool write_cache) {
  const int tid = threadIdx.x;
  const bool own = tid < kAttnHeadDim;
  const int d = own ? tid : 0;
  const int kvh = h / a.group;
  NewTokenIn t{};
  t.posi = a.positions ? a.positions[b] : a.pos_scalar;
  t.ctx = row_ctx(a, b);
  t.phys = -1;
  if (own) {
    t.qv = load_act<QT>(a.q, (int64_t)b * a.q_stride + (int64_t)h * kAttnHeadDim + d);
    t.kv = load_act<QT>(a.k_new, (int64_t)b * a.kn_stride + (int64_t)kvh * kAttnHeadDim + d);
    t.vv = load_act<QT>(a.v_new, (int64_t)b * a.vn_stride + (int64_t)kvh * kAttnHeadDim + d);
    if (a.q_norm_w) t.qn_w = a.q_norm_w[d];
    if (a.k_norm_w) t.kn_w = a.k_norm_w[d];
    if (a.rope_dim == 64 && d < 64) t.fq = a.inv_freq[d & 31];
    const int half = a.rope_dim >> 1;
    if (d < a.rope_dim) t.fk = a.inv_freq[d < half ? d : d - half];
    if (write_cache && t.ctx > 0) {
      const int row = a.seq_slot ? a.seq_slot[b] : b;
      t.phys = a.page_table[(int64_t)row * a.pt_stride + (t.ctx - 1) / kPageTokens];
    }
  }
  return t;
}

template <int QT>
__device__ float new_token_finish(const AttnArgs& a, const NewTokenIn& t, int b, int h, bool write_cache,
                                  float* x_s, float* red_s, float* v_s) {
  const int tid = threadIdx.x;
  const bool own = tid < kAttnHeadDim;
  const int d = own ? tid : 0;
  const int w = tid >> 6;
  const int kvh = h / a.group;
  float qv = t.qv, kv = t.kv;
  // Sums of squares in the orders of the kernels whose results this token
  // must reproduce.  k: per wave, then the four waves in order
  // (kv_append_kernel).  q: lane l sums dims l, l + 64, l + 128, l + 192 in
  // that order, then one wave sum (the split-K prologue), so the q this
  // token's score uses is bit for bit the q of the resident tokens' scores.
  // The raw q goes through v_s, which takes the token's v only later.
  if (own) v_s[d] = qv;
  const float sk = wave_sum(mul_rn(kv, kv));
  if ((tid & 63) == 0 && w < 4) red_s[4 + w] = sk;
  __syncthreads();
  if (w == 0) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kAttnHeadDim; j += 64) ss = add_rn(ss, mul_rn(v_s[j + tid], v_s[j + tid]));
    ss = wave_sum(ss);
    if (tid == 0) red_s[0] = ss;
  }
  __syncthreads();
  if (own) {
    if (a.q_norm_w) qv = rmsnorm_elem<QT>(qv, rms_scale(red_s[0], kAttnHeadDim), t.qn_w);
    if (a.k_norm_w)
      kv = rmsnorm_elem<QT>(kv, rms_scale(red_s[4] + red_s[5] + red_s[6] + red_s[7], kAttnHeadDim), t.kn_w);
    x_s[d] = qv;
    x_s[kAttnHeadDim + d] = kv;
  }
  __syncthreads();
  float dot = 0.f;
  if (own) {
    const float pos = static_cast<float>(t.posi);
    float qr = qv;
    if (a.rope_dim == 64 && d < 64) {
      float rs, rc;
      sincosf(mul_rn(pos, t.fq), &rs, &rc);
      const float pq = x_s[d ^ 32];
      qr = add_rn(mul_rn(qv, rc), mul_rn(d < 32 ? -pq : pq, rs));
    }
    // k: rope_elem's arithmetic with its frequency already loaded
    const int half = a.rope_dim >> 1;
    float kr = kv;
    if (d < a.rope_dim) {
      const float pk = x_s[kAttnHeadDim + (d < half ? d + half : d - half)];
      const float ang = mul_rn(pos, t.fk);
      const float c = cosf(ang), sn = sinf(ang);
      kr = add_rn(mul_rn(kv, c), mul_rn(d < half ? -pk : pk, sn));
    }
    const bool f16 = a.kv_dtype == RIA_DT_F16;
    const uint16_t k16 = f16 ? Kv16<RIA_DT_F16>::from_f32(kr) : Kv16<RIA_DT_BF16>::from_f32(kr);
    const uint16_t v16 = f16 ? Kv16<RIA_DT_F16>::from_f32(t.vv) : Kv16<RIA_DT_BF16>::from_f32(t.vv);
    const float kq = f16 ? Kv16<RIA_DT_F16>::to_f32(k16) : Kv16<RIA_DT_BF16>::to_f32(k16);
    v_s[d] = f16 ? Kv16<RIA_DT_F16>::to_f32(v16) : Kv16<RIA_DT_BF16>::to_f32(v16);
    dot = qr * kq;
    // the host allocates the page; never write outside the pool
    if (write_cache && t.ctx > 0 && t.phys >= 0 && t.phys < a.num_pages) {
      const int64_t tile = (int64_t)t.phys * a.num_kv_heads + kvh;
      const int off = (t.ctx - 1) % kPageTokens;
      const_cast<uint16_t*>(a.k_cache)[tile * kTileElems + k_tile_offset(off, d)] = k16;
      const_cast<uint16_t*>(a.v_cache)[(tile * kAttnHeadDim + d) * kPageTokens + off] = v16;
    }
  }
  dot = wave_sum(dot);
  if ((tid & 63) == 0 && w < 4) red_s[8 + w] = dot;
  __syncthreads();
  return (red_s[8] + red_s[9] + red_s[10] + red_s[11]) * (a.scale * 1.4426950408889634f);
}

// Merge the partials of one (sequence, query head) and apply the sigmoid gate.
template <int GT, int OT, bool BALANCED, bool APPEND>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const int b = blockIdx.x / a.num_q_heads;
  const int h = blockIdx.x % a.num_q_heads;
  const int d = threadIdx.x;
  const int kvh = h / a.group;
  const int hi = h % a.group;
  // The partial list's bounds are loaded first, then everything the new
  // token and the gate need, so those loads are in flight beside the
  // partials' instead of after them.
  int64_t first, count;
  const int u = b * a.num_kv_heads + kvh;
  int chunk = 1, o0 = 0, o1 = 0, ctx = 0;
  if constexpr (BALANCED) {
    chunk = a.ws_units[1];
    o0 = a.ws_units[2 + u];
    o1 = a.ws_units[3 + u];
  } else {
    ctx = row_ctx(a, b);
  }
  __builtin_amdgcn_sched_barrier(0);
  NewTokenIn nt{};
  if constexpr (APPEND) nt = new_token_load<GT>(a, b, h, hi == 0);
  const int64_t gi = (int64_t)b * a.gate_stride + (int64_t)h * kAttnHeadDim + d;
  const float g_raw = load_act<GT>(a.gate, gi);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (BALANCED) {
    // partials of unit u come from workgroups off[u] / chunk .. (off[u + 1] - 1) / chunk, at index w + u
    const int w0 = o0 / chunk, w1 = (o1 - 1) / chunk;
    first = (int64_t)w0 + u;
    count = o1 > o0 ? w1 - w0 + 1 : 0;
  } else {
    first = (int64_t)u * a.max_splits;
    count = min((ctx + a.split_tokens - 1) / a.split_tokens, a.max_splits);
  }
  // Partials are read kCombineBatch at a time (independent loads in flight)
  // and added in split order, so the result does not depend on the batching.
  constexpr int kCombineBatch = 16;
  float M = -INFINITY;
  float num = 0.f, den = 0.f;
  auto add = [&](float mv, float acc, float sum) {
    const float wt = mv == -INFINITY ? 0.f : exp2f(mv - M);  // stats are in log2 units
    num = fmaf(wt, acc, num);
    den = fmaf(wt, sum, den);
  };
  int64_t s = 0;
  // Short lists in one pass: every partial's statistics and accumulator are
  // loaded at once (N slots; past the end, the last partial again, ignored),
  // then the max, then the sum in split order (the two-pass result).
  auto one_pass = [&](auto n_slots) {
    constexpr int N = decltype(n_slots)::value;
    float mv[N], acc[N], sum[N];
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int64_t ph = (first + min<int64_t>(j, count - 1)) * a.group + hi;
      mv[j] = a.ws_stats[ph * 2];
      sum[j] = a.ws_stats[ph * 2 + 1];
      acc[j] = a.ws_acc[ph * kAttnHeadDim + d];
    }
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (j < count) M = fmaxf(M, mv[j]);
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (j < count) add(mv[j], acc[j], sum[j]);
  };
  if (count <= kCombineBatch) {
    if (count > 4)
      one_pass(std::integral_constant<int, kCombineBatch>{});
    else if (count > 0)
      one_pass(std::integral_constant<int, 4>{});
    s = count;
  }
  for (; s + kCombineBatch <= count; s += kCombineBatch) {
    float mv[kCombineBatch];
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) mv[j] = a.ws_stats[((first + s + j) * a.group + hi) * 2];
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) M = fmaxf(M, mv[j]);
  }
  for (; s < count; ++s) M = fmaxf(M, a.ws_stats[((first + s) * a.group + hi) * 2]);
  for (s = count <= kCombineBatch ? count : 0; s + kCombineBatch <= count; s += kCombineBatch) {
    float mv[kCombineBatch], acc[kCombineBatch], sum[kCombineBatch];
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) {
      const int64_t ph = (first + s + j) * a.group + hi;
      mv[j] = a.ws_stats[ph * 2];
      sum[j] = a.ws_stats[ph * 2 + 1];
      acc[j] = a.ws_acc[ph * kAttnHeadDim + d];
    }
#pragma unroll
    for (int j = 0; j < kCombineBatch; ++j) add(mv[j], acc[j], sum[j]);
  }
  for (; s < count; ++s) {
    const int64_t ph = (first + s) * a.group + hi;
    add(a.ws_stats[ph * 2], a.ws_acc[ph * kAttnHeadDim + d], a.ws_stats[ph * 2 + 1]);
  }
  if constexpr (APPEND) {  // fold in the row's new token (q, k and v in the gate's dtype)
    __shared__ float x_s[2 * kAttnHeadDim], red_s[12], v_s[kAttnHeadDim];
    const float sn = new_token_finish<GT>(a, nt, b, h, hi == 0, x_s, red_s, v_s);
    const float Mn = fmaxf(M, sn);
    const float r = M == -INFINITY ? 0.f : exp2f(M - Mn), pn = exp2f(sn - Mn);
    num = fmaf(pn, v_s[d], num * r);
    den = fmaf(pn, 1.f, den * r);
  }
  const float attn = num / den;
  const float gv = sigmoid_f(g_raw);
  store_act<OT>(a.out, ((int64_t)b * a.num_q_heads + h) * kAttnHeadDim + d, mul_rn(attn, gv));
}

// attn_combine_kernel for long partial lists (a few units share all the
// workgroups, as at small batches).  Wave p of the STREAMS waves takes
// partials p, p + STREAMS, ... (2, 4 or 8 of them in flight), lane dg its dims
// 4 dg .. 4 dg + 3 (16-byte loads), in one pass with a running max; the
// streams are merged in order through LDS.
template <int GT, int OT, bool BALANCED, int STREAMS, bool APPEND>
__global__ __launch_bounds__(64 * STREAMS) void attn_combine_long_kernel(AttnArgs a) {
  const int b = blockIdx.x / a.num_q_heads;
  const int h = blockIdx.x % a.num_q_heads;
  const int dg = threadIdx.x & 63;
  const int p = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kvh = h / a.group;
  const int hi = h % a.group;
  // The partial list's bounds are loaded first, then everything the new
  // token and the gate need, so those loads are in flight beside the
  // partials' instead of after them.
  int64_t first, count;
  const int u = b * a.num_kv_heads + kvh;
  int chunk = 1, o0 = 0, o1 = 0, ctx = 0;
  if constexpr (BALANCED) {
    chunk = a.ws_units[1];
    o0 = a.ws_units[2 + u];
    o1 = a.ws_units[3 + u];
  } else {
    ctx = row_ctx(a, b);
  }
  __builtin_amdgcn_sched_barrier(0);
  NewTokenIn nt{};
  if constexpr (APPEND) nt = new_token_load<GT>(a, b, h, hi == 0);
  // waves 0-3 finish the head, one output dim per lane
  static_assert(STREAMS >= 4, "the head is finished by four waves");
  const int od = 64 * p + dg;
  float g_raw = 0.f;
  if (p < 4) g_raw = load_act<GT>(a.gate, (int64_t)b * a.gate_stride + (int64_t)h * kAttnHeadDim + od);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (BALANCED) {
    // partials of unit u come from workgroups off[u] / chunk .. (off[u + 1] - 1) / chunk, at index w + u
    const int w0 = o0 / chunk, w1 = (o1 - 1) / chunk;
    first = (int64_t)w0 + u;
    count = o1 > o0 ? w1 - w0 + 1 : 0;
  } else {
    first = (int64_t)u * a.max_splits;
    count = min((ctx + a.split_tokens - 1) / a.split_tokens, a.max_splits);
  }
  const float* stats = a.ws_stats + (first * a.group + hi) * 2;  // partial s: stats[s * group * 2 + {0, 1}]
  const float* accs = a.ws_acc + (first * a.group + hi) * kAttnHeadDim + 4 * dg;
  const int64_t sstep = (int64_t)a.group * 2, astep = (int64_t)a.group * kAttnHeadDim;
  // One pass with a running max (stats are in log2 units): each wave keeps
  // (max, num, den) over its partials, rescaled when a batch raises the max.
  // A batch holds 2, 4 or 8 loads per wave, sized to the list (past the
  // end, the last partial again, ignored).
  float M = -INFINITY, den = 0.f;
  f32x4 num = {0.f, 0.f, 0.f, 0.f};
  auto stream = [&](auto batch) {
    constexpr int kBatch = decltype(batch)::value;
    for (int64_t s0 = p; s0 < count; s0 += STREAMS * kBatch) {
      float mv[kBatch], sum[kBatch];
      f32x4 acc[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int64_t s = s0 + j * STREAMS, sc = min(s, count - 1);
        const bool in = s < count;
        const float v = stats[sc * sstep], w = stats[sc * sstep + 1];
        const f32x4 x = *reinterpret_cast<const f32x4*>(accs + sc * astep);
        mv[j] = in ? v : -INFINITY;
        sum[j] = in ? w : 0.f;
        acc[j] = in ? x : f32x4{0.f, 0.f, 0.f, 0.f};
      }
      float mb = M;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) mb = fmaxf(mb, mv[j]);
      if (mb > M) {  // uniform: every lane of the wave reads the same stats
        const float r = exp2f(M - mb);
        den *= r;
#pragma unroll
        for (int i = 0; i < 4; ++i) num[i] *= r;
        M = mb;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const float wt = mv[j] == -INFINITY ? 0.f : exp2f(mv[j] - M);
#pragma unroll
        for (int i = 0; i < 4; ++i) num[i] = fmaf(wt, acc[j][i], num[i]);
        den = fmaf(wt, sum[j], den);
      }
    }
  };
  if (count <= 2 * STREAMS)
    stream(std::integral_constant<int, 2>{});
  else if (count <= 4 * STREAMS)
    stream(std::integral_constant<int, 4>{});
  else
    stream(std::integral_constant<int, 8>{});
  __shared__ float m_s[STREAMS];
  __shared__ f32x4 num_s[STREAMS][64];
  __shared__ float den_s[STREAMS];
  num_s[p][dg] = num;
  if (dg == 0) {
    m_s[p] = M;
    den_s[p] = den;
  }
  float sn = -INFINITY;  // fused append: the new token's score (log2 units); its v in v_s
  __shared__ float x_s[APPEND ? 2 * kAttnHeadDim : 1], red_s[12], v_s[APPEND ? kAttnHeadDim : 1];
  if constexpr (APPEND) sn = new_token_finish<GT>(a, nt, b, h, hi == 0, x_s, red_s, v_s);
  __syncthreads();
  if (p >= 4) return;
  float Mt = APPEND ? sn : -INFINITY;
#pragma unroll
  for (int q = 0; q < STREAMS; ++q) Mt = fmaxf(Mt, m_s[q]);
  float tn = 0.f, td = 0.f;
#pragma unroll
  for (int q = 0; q < STREAMS; ++q) {
    const float wq = m_s[q] == -INFINITY ? 0.f : exp2f(m_s[q] - Mt);
    tn = fmaf(wq, reinterpret_cast<const float*>(num_s[q])[od], tn);  // stream q's dim od
    td = fmaf(wq, den_s[q], td);
  }
  if constexpr (APPEND) {
    const float pn = exp2f(sn - Mt);
    tn = fmaf(pn, v_s[od], tn);
    td = fmaf(pn, 1.f, td);
  }
  store_act<OT>(a.out, ((int64_t)b * a.num_q_heads + h) * kAttnHeadDim + od, mul_rn(tn / td, sigmoid_f(g_raw)));
}

__global__ __launch_bounds__(256) void kv_gather_kernel(const uint16_t* k_cache, const uint16_t* v_cache,
                                                        int num_pages, const int32_t* page_table,
                                                        int64_t pt_stride, const int32_t* seq_slot,
                                                        int num_kv_heads, int32_t start, int32_t count,
                                                        uint16_t* k_out, uint16_t* v_out) {
  const int t = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int d = threadIdx.x;
  const int row = seq_slot ? seq_slot[b] : b;
  const int tok = start + t;
  const int phys = page_table[(int64_t)row * pt_stride + tok / kPageTokens];
  const int64_t o = (((int64_t)b * num_kv_heads + kvh) * count + t) * kAttnHeadDim + d;
  if (phys < 0 || phys >= num_pages) {
    k_out[o] = 0;
    v_out[o] = 0;
    return;
  }
  const int64_t tile = (int64_t)phys * num_kv_heads + kvh;
  const int off = tok % kPageTokens;
  k_out[o] = k_cache[tile * kTileElems + k_tile_offset(off, d)];
  v_out[o] = v_cache[(tile * kAttnHeadDim + d) * kPageTokens + off];
}

static bool valid_dtype(int dt) { return dt == RIA_DT_BF16 || dt == RIA_DT_F16 || dt == RIA_DT_F32; }

// Pages per split: enough splits for ~1024 busy workgroups (4 per CU), but
// as long as possible (up to 192 pages = 3072 tokens, 48 pages per wave) so
// the per-split prologue, merge and partial write stay small next to the
// KV stream.  Measured on MI355X at B=128, contexts U[1k, 32k], with
// streaming loads: 1024-token splits reach 71% of HBM peak, 2048-token 74%,
// 3072-token 75%, 6144-token 65% (too few workgroups).
int auto_split_tokens(int64_t total_pages) {
  int64_t pps = total_pages / 1024;
  if (pps < 4) pps = 4;
  if (pps > 192) pps = 192;
  pps = (pps + 3) / 4 * 4;
  return static_cast<int>(pps * kPageTokens);
}

static int auto_split_tokens(int batch, int num_kv_heads, int max_ctx) {
  return auto_split_tokens((int64_t)batch * num_kv_heads * ((max_ctx + kPageTokens - 1) / kPageTokens));
}

static int resolve_split(int batch, int num_kv_heads, int max_ctx, int split_tokens) {
  return split_tokens > 0 ? split_tokens : auto_split_tokens(batch, num_kv_heads, max_ctx);
}

// rows > 0: one workgroup per (row, KV head); rows == 0: the prompt append,
// one workgroup per (page the prompt touches, KV head).
static void launch_append(const AppendArgs& a, int rows, int k_dtype, int v_dtype, int kv_dtype, hipStream_t st) {
  const bool seq = rows == 0;
  const int pages = seq ? (a.pos_scalar + a.seq_len - 1) / kPageTokens - a.pos_scalar / kPageTokens + 1 : 0;
  dim3 grid(seq ? pages : rows, a.num_kv_heads);
#define RIA_APPEND_ONE(KT_, VT_, KVT_)                                                        \
  if (seq)                                                                                  \
    hipLaunchKernelGGL((kv_append_page_kernel<KT_, VT_, KVT_>), grid, dim3(256), 0, st, a); \
  else                                                                                      \
    hipLaunchKernelGGL((kv_append_kernel<KT_, VT_, KVT_>), grid, dim3(256), 0, st, a)
#define RIA_APPEND_LAUNCH(KT_, VT_)        \
  if (kv_dtype == RIA_DT_F16) {            \
    RIA_APPEND_ONE(KT_, VT_, RIA_DT_F16);  \
  } else {                                 \
    RIA_APPEND_ONE(KT_, VT_, RIA_DT_BF16); \
  }
#define RIA_APPEND_VT(KT_)                 \
  if (v_dtype == RIA_DT_BF16) {             \
    RIA_APPEND_LAUNCH(KT_, RIA_DT_BF16);    \
  } else if (v_dtype == RIA_DT_F16) {       \
    RIA_APPEND_LAUNCH(KT_, RIA_DT_F16);     \
  } else {                                  \
    RIA_APPEND_LAUNCH(KT_, RIA_DT_F32);     \
  }
  if (k_dtype == RIA_DT_BF16) {
    RIA_APPEND_VT(RIA_DT_BF16)
  } else if (k_dtype == RIA_DT_F16) {
    RIA_APPEND_VT(RIA_DT_F16)
  } else {
    RIA_APPEND_VT(RIA_DT_F32)
  }
#undef RIA_APPEND_VT
#undef RIA_APPEND_LAUNCH
#undef RIA_APPEND_ONE
}

static int check_append_common(const char* who, int num_kv_heads, const void* k, int k_dtype, int64_t k_row_stride,
                               const void* v, int v_dtype, int64_t v_row_stride, const void* k_cache,
                               const void* v_cache, int kv_dtype, const int32_t* page_table, const float* inv_freq,
                               int rope_dim) {
  if (num_kv_heads <= 0) return set_error(RIA_ERR_INVALID, "%s: bad num_kv_heads", who);
  if (!valid_dtype(k_dtype) || !valid_dtype(v_dtype)) return set_error(RIA_ERR_INVALID, "%s: unknown dtype", who);
  if (kv_dtype != RIA_DT_BF16 && kv_dtype != RIA_DT_F16)
    return set_error(RIA_ERR_INVALID, "%s: the KV cache must be bf16 or fp16", who);
  if (!k || !v || !k_cache || !v_cache || !page_table) return set_error(RIA_ERR_INVALID, "%s: null pointer", who);
  if (rope_dim < 0 || rope_dim > 64 || rope_dim % 2)
    return set_error(RIA_ERR_INVALID, "%s: rope_dim must be even and <= 64", who);
  if (rope_dim > 0 && !inv_freq) return set_error(RIA_ERR_INVALID, "%s: inv_freq is null", who);
  if (k_row_stride < (int64_t)num_kv_heads * kAttnHeadDim || v_row_stride < (int64_t)num_kv_heads * kAttnHeadDim)
    return set_error(RIA_ERR_INVALID, "%s: row stride smaller than Hkv*256", who);
  return RIA_OK;
}

}  // namespace ria

using namespace ria;

static int kv_append_impl(const char* who, int batch, int num_kv_heads, const void* k, int k_dtype,
                          int64_t k_row_stride, const void* v, int v_dtype, int64_t v_row_stride, void* k_cache,
                          void* v_cache, int kv_dtype, int num_pages, const int32_t* page_table,
                          int64_t page_table_stride, const int32_t* seq_slot, const int32_t* positions,
                          int32_t position_scalar, const int32_t* slots, int32_t slot_scalar, const float* inv_freq,
                          int rope_dim, const float* k_norm_weight, float* k_rot_out, void* stream) {
  if (batch < 0) return set_error(RIA_ERR_INVALID, "%s: bad batch", who);
  int rc = check_append_common(who, num_kv_heads, k, k_dtype, k_row_stride, v, v_dtype, v_row_stride,
                               k_cache, v_cache, kv_dtype, page_table, inv_freq, rope_dim);
  if (rc != RIA_OK) return rc;
  if (batch == 0) return RIA_OK;
  if (!slots && slot_scalar < 0) return set_error(RIA_ERR_INVALID, "%s: negative slot", who);
  AppendArgs a{};
  a.k = k;
  a.k_stride = k_row_stride;
  a.v = v;
  a.v_stride = v_row_stride;
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.num_pages = num_pages;
  a.page_table = page_table;
  a.pt_stride = page_table_stride;
  a.seq_slot = seq_slot;
  a.positions = positions;
  a.pos_scalar = position_scalar;
  a.slots = slots;
  a.slot_scalar = slot_scalar;
  a.inv_freq = inv_freq;
  a.rope_dim = rope_dim;
  a.norm_w = k_norm_weight;
  a.num_kv_heads = num_kv_heads;
  a.k_out = k_rot_out;
  launch_append(a, batch, k_dtype, v_dtype, kv_dtype, static_cast<hipStream_t>(stream));
  return check_launch(who);
}

extern "C" int ria_kv_append(int batch, int num_kv_heads, const void* k, int k_dtype, int64_t k_row_stride,
                             const void* v, int v_dtype, int64_t v_row_stride, void* k_cache, void* v_cache,
                             int kv_dtype, int num_pages, const int32_t* page_table, int64_t page_table_stride,
                             const int32_t* seq_slot, const int32_t* positions, int32_t position_scalar,
                             const int32_t* slots, int32_t slot_scalar, const float* inv_freq, int rope_dim,
                             const float* k_norm_weight, void* stream) {
  return kv_append_impl("ria_kv_append", batch, num_kv_heads, k, k_dtype, k_row_stride, v, v_dtype, v_row_stride,
                        k_cache, v_cache, kv_dtype, num_pages, page_table, page_table_stride, seq_slot, positions,
                        position_scalar, slots, slot_scalar, inv_freq, rope_dim, k_norm_weight, nullptr, stream);
}

extern "C" int ria_kv_append_out(int batch, int num_kv_heads, const void* k, int k_dtype, int64_t k_row_stride,
                                 const void* v, int v_dtype, int64_t v_row_stride, void* k_cache, void* v_cache,
                                 int kv_dtype, int num_pages, const int32_t* page_table, int64_t page_table_stride,
                                 const int32_t* seq_slot, const int32_t* positions, int32_t position_scalar,
                                 const int32_t* slots, int32_t slot_scalar, const float* inv_freq, int rope_dim,
                                 const float* k_norm_weight, float* k_rot_out, void* stream) {
  if (!k_rot_out) return set_error(RIA_ERR_INVALID, "ria_kv_append_out: null k_rot_out");
  return kv_append_impl("ria_kv_append_out", batch, num_kv_heads, k, k_dtype, k_row_stride, v, v_dtype,
                        v_row_stride, k_cache, v_cache, kv_dtype, num_pages, page_table, page_table_stride, seq_slot,
                        positions, position_scalar, slots, slot_scalar, inv_freq, rope_dim, k_norm_weight, k_rot_out,
                        stream);
}

namespace ria {
// ria_kv_append_seq, optionally also writing the prompt's k and v as fp16 tiles (start_pos 0 only).
int kv_append_seq_impl(int length, int num_kv_heads, const void* k, int k_dtype, int64_t k_row_stride,
                       const void* v, int v_dtype, int64_t v_row_stride, void* k_cache, void* v_cache, int kv_dtype,
                       int num_pages, const int32_t* page_table_row, int64_t page_capacity, int32_t start_pos,
                       const float* inv_freq, int rope_dim, const float* k_norm_weight, uint16_t* stage_k,
                       uint16_t* stage_v, void* stream);
}  // namespace ria

extern "C" int ria_kv_append_seq(int length, int num_kv_heads, const void* k, int k_dtype, int64_t k_row_stride,
                                 const void* v, int v_dtype, int64_t v_row_stride, void* k_cache, void* v_cache,
                                 int kv_dtype, int num_pages, const int32_t* page_table_row, int64_t page_capacity,
                                 int32_t start_pos, const float* inv_freq, int rope_dim,
                                 const float* k_norm_weight, void* stream) {
  return kv_append_seq_impl(length, num_kv_heads, k, k_dtype, k_row_stride, v, v_dtype, v_row_stride, k_cache,
                            v_cache, kv_dtype, num_pages, page_table_row, page_capacity, start_pos, inv_freq,
                            rope_dim, k_norm_weight, nullptr, nullptr, stream);
}

int ria::kv_append_seq_impl(int length, int num_kv_heads, const void* k, int k_dtype, int64_t k_row_stride,
                            const void* v, int v_dtype, int64_t v_row_stride, void* k_cache, void* v_cache,
                            int kv_dtype, int num_pages, const int32_t* page_table_row, int64_t page_capacity,
                            int32_t start_pos, const float* inv_freq, int rope_dim, const float* k_norm_weight,
                            uint16_t* stage_k, uint16_t* stage_v, void* stream) {
  if (length < 0 || start_pos < 0) return set_error(RIA_ERR_INVALID, "ria_kv_append_seq: negative length or start");
  if (stage_k && (start_pos != 0 || !stage_v || (reinterpret_cast<uintptr_t>(stage_k) |
                                                  reinterpret_cast<uintptr_t>(stage_v)) % 16))
    return set_error(RIA_ERR_INVALID, "ria_kv_append_seq: an fp16 stage needs start 0 and 16-byte aligned k and v");
  int rc = check_append_common("ria_kv_append_seq", num_kv_heads, k, k_dtype, k_row_stride, v, v_dtype,
                               v_row_stride, k_cache, v_cache, kv_dtype, page_table_row, inv_freq, rope_dim);
  if (rc != RIA_OK) return rc;
  if (length == 0) return RIA_OK;
  if (reinterpret_cast<uintptr_t>(k_cache) % 16 || reinterpret_cast<uintptr_t>(v_cache) % 16)
    return set_error(RIA_ERR_INVALID, "ria_kv_append_seq: the KV caches must be 16-byte aligned");
  if ((int64_t)start_pos + length > page_capacity * kPageTokens)
    return set_error(RIA_ERR_INVALID, "ria_kv_append_seq: %d + %d tokens exceed the row's %lld pages", start_pos,
                     length, (long long)page_capacity);
  AppendArgs a{};
  a.k = k;
  a.k_stride = k_row_stride;
  a.v = v;
  a.v_stride = v_row_stride;
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.num_pages = num_pages;
  a.page_table = page_table_row;
  a.pt_stride = page_capacity;
  a.pos_scalar = start_pos;
  a.inv_freq = inv_freq;
  a.rope_dim = rope_dim;
  a.norm_w = k_norm_weight;
  a.num_kv_heads = num_kv_heads;
  a.seq_len = length;
  a.stage_k = stage_k;
  a.stage_v = stage_v;
  launch_append(a, 0, k_dtype, v_dtype, kv_dtype, static_cast<hipStream_t>(stream));
  return check_launch("ria_kv_append_seq");
}

extern "C" int ria_attn_decode_split_tokens(int num_kv_heads, const int32_t* ctx_lens_host, int batch) {
  if (!ctx_lens_host || batch <= 0 || num_kv_heads <= 0) return 4 * kPageTokens;
  int64_t pages = 0;
  for (int b = 0; b < batch; ++b) pages += (ctx_lens_host[b] + kPageTokens - 1) / kPageTokens;
  return auto_split_tokens(pages * num_kv_heads);
}

// Workgroups of a balanced launch: two per CU (the kernel's occupancy).
static int balanced_workgroups() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return 2 * cus;
}

static bool use_balanced(int batch, int num_kv_heads, int split_tokens) {
  return split_tokens == 0 && (int64_t)batch * num_kv_heads <= kMaxBalancedUnits;
}

// Workspace: [unit table (balanced only), padded to 64 floats][stats][acc].
static int64_t decode_parts(int batch, int num_kv_heads, int max_ctx, int split_tokens, int64_t* unit_ints) {
  if (use_balanced(batch, num_kv_heads, split_tokens)) {
    const int64_t units = (int64_t)batch * num_kv_heads;
    *unit_ints = (units + 3 + 63) / 64 * 64;
    return balanced_workgroups() + units;
  }
  *unit_ints = 0;
  const int st = resolve_split(batch, num_kv_heads, max_ctx, split_tokens);
  return (int64_t)batch * num_kv_heads * ((max_ctx + st - 1) / st);
}

extern "C" int64_t ria_attn_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int max_ctx,
                                                   int split_tokens) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || max_ctx <= 0) return 0;
  int64_t unit_ints = 0;
  const int64_t parts = decode_parts(batch, num_kv_heads, max_ctx, split_tokens, &unit_ints);
  const int64_t group = num_q_heads / num_kv_heads;
  const int64_t stats = parts * group * 2;
  const int64_t stats_aligned = (stats + 63) / 64 * 64;
  return (unit_ints + stats_aligned + parts * group * kAttnHeadDim) * (int64_t)sizeof(float);
}

// The fused append's inputs (ria_attn_decode_append), or none.
struct AppendIn {
  const void* k;
  int64_t k_stride;
  const void* v;
  int64_t v_stride;
  const float* k_norm_w;
};

static int attn_decode_impl(int batch, int num_q_heads, int num_kv_heads, const void* q, int q_dtype,
                            int64_t q_row_stride, const void* gate, int gate_dtype, int64_t gate_row_stride,
                            const void* k_cache, const void* v_cache, int kv_dtype, int num_pages,
                            const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                            const int32_t* positions, int32_t position_scalar, const int32_t* ctx_lens,
                            int32_t ctx_scalar, int max_ctx, const float* inv_freq, int rope_dim,
                            const float* q_norm_weight, float scale, int split_tokens, void* workspace,
                            int64_t workspace_bytes, void* out, int out_dtype, int phase, const AppendIn* app,
                            void* stream) {
  if (phase < RIA_ATTN_SPLITK || phase > RIA_ATTN_BOTH)
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: unknown phase %d", phase);
  if (app) {
    if (!app->k || !app->v) return set_error(RIA_ERR_INVALID, "ria_attn_decode_append: null k or v");
    if (gate_dtype != q_dtype)
      return set_error(RIA_ERR_INVALID, "ria_attn_decode_append: q, gate, k and v must share one dtype");
    if (app->k_stride < (int64_t)num_kv_heads * kAttnHeadDim || app->v_stride < (int64_t)num_kv_heads * kAttnHeadDim)
      return set_error(RIA_ERR_INVALID, "ria_attn_decode_append: k/v row stride smaller than Hkv*256");
  }
  if (batch < 0) return set_error(RIA_ERR_INVALID, "ria_attn_decode: batch must be >= 0");
  if (batch == 0) return RIA_OK;
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: num_q_heads must be a multiple of num_kv_heads");
  const int group = num_q_heads / num_kv_heads;
  if (group > 8) return set_error(RIA_ERR_INVALID, "ria_attn_decode: at most 8 query heads per KV head (got %d)", group);
  if (!valid_dtype(q_dtype) || !valid_dtype(gate_dtype) || !valid_dtype(out_dtype))
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: unknown dtype code");
  if (kv_dtype != RIA_DT_BF16 && kv_dtype != RIA_DT_F16)
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: the KV cache must be bf16 or fp16");
  if (!q || !gate || !k_cache || !v_cache || !page_table || !out || !workspace)
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: null pointer");
  if (rope_dim != 0 && rope_dim != 64) return set_error(RIA_ERR_INVALID, "ria_attn_decode: rope_dim must be 0 or 64");
  if (rope_dim > 0 && !inv_freq) return set_error(RIA_ERR_INVALID, "ria_attn_decode: inv_freq is null");
  if (max_ctx <= 0) return set_error(RIA_ERR_INVALID, "ria_attn_decode: max_ctx must be > 0");
  if (!ctx_lens && (ctx_scalar <= 0 || ctx_scalar > max_ctx))
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: ctx_scalar must be in [1, max_ctx]");
  if (split_tokens < 0 || split_tokens % 64)
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: split_tokens must be 0 or a multiple of 64");
  if (q_row_stride < (int64_t)num_q_heads * kAttnHeadDim || gate_row_stride < (int64_t)num_q_heads * kAttnHeadDim)
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: row stride smaller than Hq*256");
  if (reinterpret_cast<uintptr_t>(k_cache) % 16 || reinterpret_cast<uintptr_t>(v_cache) % 16)
    return set_error(RIA_ERR_INVALID, "ria_attn_decode: KV caches must be 16-byte aligned");
  const int64_t need = ria_attn_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, max_ctx, split_tokens);
  if (workspace_bytes < need)
    return set_error(RIA_ERR_WORKSPACE, "ria_attn_decode: workspace %lld bytes < required %lld",
                     (long long)workspace_bytes, (long long)need);

  AttnArgs a{};
  a.q = q;
  a.q_stride = q_row_stride;
  a.gate = gate;
  a.gate_stride = gate_row_stride;
  a.k_cache = static_cast<const uint16_t*>(k_cache);
  a.v_cache = static_cast<const uint16_t*>(v_cache);
  a.num_pages = num_pages;
  a.page_table = page_table;
  a.pt_stride = page_table_stride;
  a.seq_slot = seq_slot;
  a.positions = positions;
  a.pos_scalar = position_scalar;
  a.ctx_lens = ctx_lens;
  a.ctx_scalar = ctx_scalar;
  a.inv_freq = inv_freq;
  a.rope_dim = rope_dim;
  a.q_norm_w = q_norm_weight;
  a.scale = scale;
  const bool balanced = use_balanced(batch, num_kv_heads, split_tokens);
  int64_t unit_ints = 0;
  const int64_t parts = decode_parts(batch, num_kv_heads, max_ctx, split_tokens, &unit_ints);
  a.balanced = balanced ? 1 : 0;
  a.batch = batch;
  a.split_tokens = balanced ? 0 : resolve_split(batch, num_kv_heads, max_ctx, split_tokens);
  a.max_splits = balanced ? 0 : (max_ctx + a.split_tokens - 1) / a.split_tokens;
  const int64_t stats = parts * group * 2;
  a.ws_units = static_cast<int32_t*>(workspace);
  a.ws_stats = static_cast<float*>(workspace) + unit_ints;
  a.ws_acc = a.ws_stats + (stats + 63) / 64 * 64;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  a.out = out;
  a.kv_dtype = kv_dtype;
  if (app) {
    a.k_new = app->k;
    a.kn_stride = app->k_stride;
    a.v_new = app->v;
    a.vn_stride = app->v_stride;
    a.k_norm_w = app->k_norm_w;
    a.exclude_last = 1;
  }
  if (a.max_splits > 65535 || batch > 65535) return set_error(RIA_ERR_INVALID, "ria_attn_decode: grid too large");

  hipStream_t st = static_cast<hipStream_t>(stream);
  if (phase & RIA_ATTN_SPLITK) {
  // A balanced launch needs no more workgroups than the largest possible page
  // stream fills at the minimum chunk (a small batch leaves the rest idle).
  const int64_t max_stream = (int64_t)batch * num_kv_heads * ((max_ctx + kPageTokens - 1) / kPageTokens);
  const int bal_wgs = static_cast<int>(std::min<int64_t>(
      balanced_workgroups(), (max_stream + kMinChunkPages - 1) / kMinChunkPages + (int64_t)batch * num_kv_heads));
  dim3 grid = balanced ? dim3(bal_wgs) : dim3(a.max_splits, num_kv_heads, batch);
#define RIA_SPLITK_KV(QT_, BAL_, QN_)                                                                  \
  if (kv_dtype == RIA_DT_F16)                                                                          \
    hipLaunchKernelGGL((attn_splitk_kernel<QT_, RIA_DT_F16, BAL_, QN_>), grid, dim3(256), 0, st, a);   \
  else                                                                                                 \
    hipLaunchKernelGGL((attn_splitk_kernel<QT_, RIA_DT_BF16, BAL_, QN_>), grid, dim3(256), 0, st, a)
#define RIA_SPLITK_QN(QT_, BAL_)            \
  if (q_norm_weight) {                      \
    RIA_SPLITK_KV(QT_, BAL_, true);         \
  } else {                                  \
    RIA_SPLITK_KV(QT_, BAL_, false);        \
  }
#define RIA_SPLITK_LAUNCH(QT_)       \
  if (balanced) {                    \
    RIA_SPLITK_QN(QT_, true)         \
  } else {                           \
    RIA_SPLITK_QN(QT_, false)        \
  }
  if (q_dtype == RIA_DT_BF16) {
    RIA_SPLITK_LAUNCH(RIA_DT_BF16);
  } else if (q_dtype == RIA_DT_F16) {
    RIA_SPLITK_LAUNCH(RIA_DT_F16);
  } else {
    RIA_SPLITK_LAUNCH(RIA_DT_F32);
  }
#undef RIA_SPLITK_LAUNCH
#undef RIA_SPLITK_QN
#undef RIA_SPLITK_KV
  int rc = check_launch("ria_attn_decode (split-K)");
  if (rc != RIA_OK) return rc;
  }
  if (!(phase & RIA_ATTN_COMBINE)) return RIA_OK;

  dim3 cgrid(batch * num_q_heads);
  // a few (sequence, KV head) units share all the splits: long partial lists, merged by 16 waves
  const bool long_lists = (int64_t)batch * num_kv_heads <= 32;
#define RIA_COMB_AP(GT_, OT_, AP_)                                                                             \
  if (balanced && long_lists)                                                                                  \
    hipLaunchKernelGGL((attn_combine_long_kernel<GT_, OT_, true, 16, AP_>), cgrid, dim3(1024), 0, st, a);      \
  else if (balanced)                                                                                           \
    hipLaunchKernelGGL((attn_combine_kernel<GT_, OT_, true, AP_>), cgrid, dim3(256), 0, st, a);                \
  else if (long_lists)                                                                                         \
    hipLaunchKernelGGL((attn_combine_long_kernel<GT_, OT_, false, 16, AP_>), cgrid, dim3(1024), 0, st, a);     \
  else                                                                                                         \
    hipLaunchKernelGGL((attn_combine_kernel<GT_, OT_, false, AP_>), cgrid, dim3(256), 0, st, a)
#define RIA_COMB_LAUNCH(GT_, OT_)       \
  if (app) {                            \
    RIA_COMB_AP(GT_, OT_, true);        \
  } else {                              \
    RIA_COMB_AP(GT_, OT_, false);       \
  }
#define RIA_COMB_OT(GT_)                     \
  if (out_dtype == RIA_DT_BF16) {            \
    RIA_COMB_LAUNCH(GT_, RIA_DT_BF16);       \
  } else if (out_dtype == RIA_DT_F16) {      \
    RIA_COMB_LAUNCH(GT_, RIA_DT_F16);        \
  } else {                                   \
    RIA_COMB_LAUNCH(GT_, RIA_DT_F32);        \
  }
  if (gate_dtype == RIA_DT_BF16) {
    RIA_COMB_OT(RIA_DT_BF16)
  } else if (gate_dtype == RIA_DT_F16) {
    RIA_COMB_OT(RIA_DT_F16)
  } else {
    RIA_COMB_OT(RIA_DT_F32)
  }
#undef RIA_COMB_OT
#undef RIA_COMB_LAUNCH
#undef RIA_COMB_AP
  return check_launch("ria_attn_decode (combine)");
}

extern "C" int ria_attn_decode_phase(int batch, int num_q_heads, int num_kv_heads, const void* q, int q_dtype,
                                     int64_t q_row_stride, const void* gate, int gate_dtype, int64_t gate_row_stride,
                                     const void* k_cache, const void* v_cache, int kv_dtype, int num_pages,
                                     const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                                     const int32_t* positions, int32_t position_scalar, const int32_t* ctx_lens,
                                     int32_t ctx_scalar, int max_ctx, const float* inv_freq, int rope_dim,
                                     const float* q_norm_weight, float scale, int split_tokens, void* workspace,
                                     int64_t workspace_bytes, void* out, int out_dtype, int phase, void* stream) {
  return attn_decode_impl(batch, num_q_heads, num_kv_heads, q, q_dtype, q_row_stride, gate, gate_dtype,
                          gate_row_stride, k_cache, v_cache, kv_dtype, num_pages, page_table, page_table_stride,
                          seq_slot, positions, position_scalar, ctx_lens, ctx_scalar, max_ctx, inv_freq, rope_dim,
                          q_norm_weight, scale, split_tokens, workspace, workspace_bytes, out, out_dtype, phase,
                          nullptr, stream);
}

extern "C" int ria_attn_decode_append(int batch, int num_q_heads, int num_kv_heads, const void* q, int q_dtype,
                                      int64_t q_row_stride, const void* gate, int gate_dtype, int64_t gate_row_stride,
                                      const void* k, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                      const float* k_norm_weight, void* k_cache, void* v_cache, int kv_dtype,
                                      int num_pages, const int32_t* page_table, int64_t page_table_stride,
                                      const int32_t* seq_slot, const int32_t* positions, int32_t position_scalar,
                                      const int32_t* ctx_lens, int32_t ctx_scalar, int max_ctx, const float* inv_freq,
                                      int rope_dim, const float* q_norm_weight, float scale, int split_tokens,
                                      void* workspace, int64_t workspace_bytes, void* out, int out_dtype, int phase,
                                      void* stream) {
  const AppendIn app{k, k_row_stride, v, v_row_stride, k_norm_weight};
  return attn_decode_impl(batch, num_q_heads, num_kv_heads, q, q_dtype, q_row_stride, gate, gate_dtype,
                          gate_row_stride, k_cache, v_cache, kv_dtype, num_pages, page_table, page_table_stride,
                          seq_slot, positions, position_scalar, ctx_lens, ctx_scalar, max_ctx, inv_freq, rope_dim,
                          q_norm_weight, scale, split_tokens, workspace, workspace_bytes, out, out_dtype, phase, &app,
                          stream);
}

// ---- ria_attn_decode_append without a caller workspace
// The split-K partials of ria_attn_decode_append_noalloc live in this
// library-owned array instead of a caller workspace, for callers that cannot
// allocate.  16 MiB holds the balanced schedule's unit table and partials
// (8 KiB per partial at 8 query heads per KV head, #workgroups + #units
// partials) for up to about 1,500 (sequence, KV head) units, i.e. 750
// sequences of the model's 2 KV heads.  Each GPU the library runs on holds
// its own copy until the process ends.  Nothing in it has to start at zero:
// every partial and partition entry the combine launch reads is written by
// the same call's split-K launch, and a call always runs both phases.  All
// calls on one GPU share the array, so calls that overlap on one GPU
// (concurrent streams) race.
constexpr int64_t kScratchBytes = int64_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The array's device address, looked up once per device with that device
// current (the array's name is only a host-side stand-in).
constexpr int kMaxScratchDevices = 64;
static void* g_scratch_addr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

static int scratch_address(void** addr, const char* who) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return set_error(RIA_ERR_LAUNCH, "%s: no current HIP device below index %d", who, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(RIA_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                       hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return RIA_OK;
}

extern "C" int ria_attn_decode_append_noalloc(int batch, int num_q_heads, int num_kv_heads, const void* q,
                                              int q_dtype, int64_t q_row_stride, const void* gate, int gate_dtype,
                                              int64_t gate_row_stride, const void* k, int64_t k_row_stride,
                                              const void* v, int64_t v_row_stride, const float* k_norm_weight,
                                              void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                                              const int32_t* page_table, int64_t page_table_stride,
                                              const int32_t* seq_slot, const int32_t* positions,
                                              int32_t position_scalar, const int32_t* ctx_lens, int32_t ctx_scalar,
                                              int max_ctx, const float* inv_freq, int rope_dim,
                                              const float* q_norm_weight, float scale, int split_tokens, void* out,
                                              int out_dtype, int phase, void* stream) {
  static const char* who = "ria_attn_decode_append_noalloc";
  // Both phases in one call: a SPLITK call's partials would sit in the shared
  // array until its COMBINE call, open to any call in between.
  if (phase != RIA_ATTN_BOTH)
    return set_error(RIA_ERR_INVALID, "%s: only phase RIA_ATTN_BOTH (got %d): the partials do not outlive the call",
                     who, phase);
  void* ws = nullptr;
  if (batch > 0) {
    const int64_t need = ria_attn_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, max_ctx, split_tokens);
    if (need > kScratchBytes)
      return set_error(RIA_ERR_WORKSPACE,
                       "%s: these sizes need %lld bytes of partials, more than the library's %lld-byte scratch "
                       "array; call ria_attn_decode_append with a workspace",
                       who, (long long)need, (long long)kScratchBytes);
    const int rc = scratch_address(&ws, who);
    if (rc != RIA_OK) return rc;
  }
  const AppendIn app{k, k_row_stride, v, v_row_stride, k_norm_weight};
  return attn_decode_impl(batch, num_q_heads, num_kv_heads, q, q_dtype, q_row_stride, gate, gate_dtype,
                          gate_row_stride, k_cache, v_cache, kv_dtype, num_pages, page_table, page_table_stride,
                          seq_slot, positions, position_scalar, ctx_lens, ctx_scalar, max_ctx, inv_freq, rope_dim,
                          q_norm_weight, scale, split_tokens, ws, kScratchBytes, out, out_dtype, phase, &app,
                          stream);
}

extern "C" int ria_attn_decode(int batch, int num_q_heads, int num_kv_heads, const void* q, int q_dtype,
                               int64_t q_row_stride, const void* gate, int gate_dtype, int64_t gate_row_stride,
                               const void* k_cache, const void* v_cache, int kv_dtype, int num_pages,
                               const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                               const int32_t* positions, int32_t position_scalar, const int32_t* ctx_lens,
                               int32_t ctx_scalar, int max_ctx, const float* inv_freq, int rope_dim,
                               const float* q_norm_weight, float scale, int split_tokens, void* workspace,
                               int64_t workspace_bytes, void* out, int out_dtype, void* stream) {
  return ria_attn_decode_phase(batch, num_q_heads, num_kv_heads, q, q_dtype, q_row_stride, gate, gate_dtype,
                               gate_row_stride, k_cache, v_cache, kv_dtype, num_pages, page_table, page_table_stride,
                               seq_slot, positions, position_scalar, ctx_lens, ctx_scalar, max_ctx, inv_freq,
                               rope_dim, q_norm_weight, scale, split_tokens, workspace, workspace_bytes, out,
                               out_dtype, RIA_ATTN_BOTH, stream);
}

extern "C" int ria_kv_gather(int batch, int num_kv_heads, const void* k_cache, const void* v_cache, int num_pages,
                             const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                             int32_t start, int32_t count, void* k_out, void* v_out, void* stream) {
  if (batch < 0 || num_kv_heads <= 0 || start < 0 || count < 0)
    return set_error(RIA_ERR_INVALID, "ria_kv_gather: bad sizes");
  if (batch == 0 || count == 0) return RIA_OK;
  if (!k_cache || !v_cache || !page_table || !k_out || !v_out) return set_error(RIA_ERR_INVALID, "ria_kv_gather: null pointer");
  if (batch > 65535 || num_kv_heads > 65535) return set_error(RIA_ERR_INVALID, "ria_kv_gather: grid too large");
  dim3 grid(count, num_kv_heads, batch);
  hipLaunchKernelGGL(kv_gather_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(k_cache), static_cast<const uint16_t*>(v_cache), num_pages,
                     page_table, page_table_stride, seq_slot, num_kv_heads, start, count,
                     static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out));
  return check_launch("ria_kv_gather");
}
