// Causal GQA full-attention prefill over the paged KV cache, for gfx950.
//
// Equal to `length` decode steps of the reference (qwen36_attention_cache.py:
// 306-317) run one token at a time, which is how the reference prefills
// (qwen36_chat_batch.py:255-258): token t of the prompt, at absolute position
// start + t, is RoPE-rotated, appended, and attends to every resident token
// 0 .. start + t; the output is softmax(q K^T * scale) V * sigmoid(gate).
//
// Two launches: the prompt's k (rotated) and v go into the pages first (the
// append kernel in sequence mode), then one workgroup per (16-token query
// block, KV head) streams the keys 0 .. last query of the block in blocks of
// 32 keys (two pages).
//   * 8 waves, one query head each (GQA group <= 8), two waves per SIMD: one
//     wave's softmax (VALU, transcendental) overlaps the other's MFMAs, and
//     every key block fetched serves 16 tokens x 8 heads;
//   * key blocks travel HBM/L2 -> LDS by direct-to-LDS loads into a 4-slot
//     ring, in pairs two blocks ahead of the one being computed, with no
//     registers in flight and one barrier per pair;
//   * scores S^T = K Q^T on 16x16x32 MFMA (16 keys x 16 tokens per tile): the
//     K tile is already in A-operand order (8 dims of one token are 16
//     contiguous bytes); the two score tiles of a block take their rows from
//     the block's tokens in an order that leaves lane group g with exactly 8
//     consecutive tokens of one page, whose V^T column is then one 16-byte
//     operand of O^T = V^T P^T (16x16x32, k = those 32 keys);
//   * with a bf16 cache the rotated q and the probabilities are carried as
//     bf16 hi + lo pairs (near-fp32 operands on MFMA); with an fp16 cache the
//     fp16 hi part alone (11 significant bits); the online softmax is kept in log2
//     units (q is pre-scaled) with a lazy rescale (only when a block max
//     exceeds the running max by 2^8); row statistics combine across lane
//     groups with permlane swaps;
//   * the gated result leaves through LDS so the output stores are coalesced;
//   * query blocks are scheduled from the last (most keys) to the first.
#include <math.h>

#include "ria_common.h"

namespace ria {

constexpr int kTile = kPageTokens * kAttnHeadDim;  // elements per (page, KV head) tile
constexpr int kTileVec = kTile * 2 / 16;           // 16-byte vectors per tile (512)
// Ring slot layout (16-byte vectors): K page 0 at 0, K page 1 at kSlotK1 (64
// bytes further than back-to-back, so the rows of the two pages that one
// 16-lane read pass touches fall on different banks), V^T pages 0 and 1 at
// kSlotV + 512 m, each stored as [token half][dim][8 tokens].
constexpr int kSlotK1 = kTileVec + 4;
constexpr int kSlotV = kSlotK1 + kTileVec;
constexpr int kSlotVec = kSlotV + 2 * kTileVec;
constexpr int kRingSlots = 4;
constexpr int kPrefillWaves = 8;                   // one query head per wave
constexpr int kPrefillThreads = 64 * kPrefillWaves;
constexpr int kStagePitch = kAttnHeadDim + 4;      // floats per staged output row
constexpr int kPrefillLds = kPrefillWaves * 16 * kStagePitch * 4;  // output stage; the ring (128 KiB) aliases it
static_assert(kRingSlots * kSlotVec * 16 <= kPrefillLds, "ring must fit in the LDS block");

struct PrefillAttnArgs {
  const void* q;
  int64_t q_stride;
  const void* gate;
  int64_t gate_stride;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int num_pages;
  int64_t pt_len;  // entries in the sequence's page-table row
  int start;   // tokens resident before the prompt
  int length;  // prompt tokens
  const float* inv_freq;
  int rope_dim;
  const float* q_norm_w;  // q_norm weight [256] f32, or null: q arrives normalised
  float scale;
  int num_q_heads;
  int num_kv_heads;
  int group;
  void* out;
  int staged;  // keys from an fp16 stage with tile (page p, KV head) at p * Hkv + kvh, not the page table
};

// Key held by row r (0..15) of score tile m (0, 1) of a 32-key block, as
// (page of the block, token): lane group g = r / 4 of both tiles together
// holds tokens 8 (g % 2) .. 8 (g % 2) + 7 of page g / 2, tile m the half
// 8 (g % 2) + 4 m .. + 3.
__device__ __forceinline__ int tile_row_page(int r) { return r >> 3; }
__device__ __forceinline__ int tile_row_token(int m, int r) { return 8 * ((r >> 2) & 1) + 4 * m + (r & 3); }

// max of three scores (never NaN: finite products, or -inf where masked) in
// one instruction; fmaxf would first quiet each MFMA result for IEEE NaN rules
__device__ __forceinline__ float max3_f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

__device__ __forceinline__ float swap_max(float x, bool rows16) {
  const auto s = rows16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                        : __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

__device__ __forceinline__ float swap_sum(float x, bool rows16) {
  const auto s = rows16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                        : __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

template <int AT, int KVT>
__global__ __launch_bounds__(kPrefillThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_prefill_kernel(
    PrefillAttnArgs a, const int32_t* __restrict__ pt) {
  using KV = Kv16<KVT>;
  // bf16 operands carry q and the probabilities as hi + lo pairs; fp16 ones
  // keep 11 significant bits in the hi part alone, which is enough here
  constexpr bool kSplit = KVT == RIA_DT_BF16;
  const int nqb = (a.length + 15) / 16;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x) / a.num_kv_heads;  // heaviest blocks first
  const int kvh = static_cast<int>(blockIdx.x) % a.num_kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15;   // MFMA column (token 16 qb + n) / row (key or dim)
  const int g4 = lane >> 4;  // lane group: k slice of the operands, row group of the results

  __shared__ __attribute__((aligned(16))) unsigned char smem[kPrefillLds];
  u32x4* ring = reinterpret_cast<u32x4*>(smem);
  float* stage = reinterpret_cast<float*>(smem);

  const bool head_ok = wave < a.group;
  const int head = kvh * a.group + wave;
  const int t_row = 16 * qb + n;
  const bool row_ok = head_ok && t_row < a.length;
  const int qpos = a.start + t_row;
  const int ctx_total = a.start + a.length;   // keys that exist
  const int qlim = min(qpos, ctx_total - 1);  // last key this column sees

  // ---- q operands: column n, dims 32 kd + 8 g4 + j, RoPE'd, scaled by
  //      scale * log2(e) (scores come out in log2 units), as hi + lo pairs
  u32x4 qh[8], ql[8];
  // SEP: fp16 values converted one at a time, so hipcc folds the multiply
  // that produced each (q times its scale) into the conversion
  // (v_fma_mixlo_f16, one rounding); the probabilities, which no multiply
  // produces, take the paired conversion.
  auto pack = [&](const float (&x)[8], u32x4& hi, u32x4& lo, auto sep) {
    uint32_t h4[4], l4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (decltype(sep)::value && KVT == RIA_DT_F16)
        h4[j] = uint32_t(f32_to_f16_bits(x[2 * j])) | (uint32_t(f32_to_f16_bits(x[2 * j + 1])) << 16);
      else
        h4[j] = KV::pack2(x[2 * j], x[2 * j + 1]);
      l4[j] = KV::pack2(x[2 * j] - KV::lo_f32(h4[j]), x[2 * j + 1] - KV::hi_f32(h4[j]));
    }
    hi = u32x4{h4[0], h4[1], h4[2], h4[3]};
    lo = u32x4{l4[0], l4[1], l4[2], l4[3]};
  };
  const float sl2 = a.scale * 1.4426950408889634f;
  {
    const int64_t base = (int64_t)t_row * a.q_stride + (int64_t)head * kAttnHeadDim + 8 * g4;
    auto load_q8 = [&](int kd, float (&y)[8]) {
      if (row_ok) {
        load_act8<AT>(a.q, base + 32 * kd, y);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = 0.f;
      }
    };
    // q_norm (qwen36_attention_cache.py:302-304) before RoPE: a first pass
    // for the row's sum of squares, whose four 64-dim slices sit in lanes
    // n, n + 16, n + 32, n + 48; the second pass normalises as it loads.
    float qs = 1.f;
    if (a.q_norm_w) {
      float ss = 0.f;
#pragma unroll
      for (int kd = 0; kd < 8; ++kd) {
        float y[8];
        load_q8(kd, y);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = add_rn(ss, mul_rn(y[j], y[j]));
      }
      qs = rms_scale(swap_sum(swap_sum(ss, true), false), kAttnHeadDim);
    }
    auto load_qn = [&](int kd, float (&y)[8]) {
      load_q8(kd, y);
      if (a.q_norm_w) {
        const f32x4* wp = reinterpret_cast<const f32x4*>(a.q_norm_w + 32 * kd + 8 * g4);
        const f32x4 w0 = wp[0], w1 = wp[1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          y[j] = rmsnorm_elem<AT>(y[j], qs, w0[j]);
          y[4 + j] = rmsnorm_elem<AT>(y[4 + j], qs, w1[j]);
        }
      }
    };
    // dims [0, 64) are kd 0, 1; rotate_half pairs dim 8 g4 + j with 32 + 8 g4 + j
    float x[2][8];
#pragma unroll
    for (int kd = 0; kd < 2; ++kd) load_qn(kd, x[kd]);
    if (a.rope_dim == 64) {
      const float pos = static_cast<float>(qpos);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float ang = mul_rn(pos, a.inv_freq[8 * g4 + j]);
        const float cs = cosf(ang), sn = sinf(ang);
        const float x1 = x[0][j], x2 = x[1][j];
        x[0][j] = add_rn(mul_rn(x1, cs), mul_rn(-x2, sn));
        x[1][j] = add_rn(mul_rn(x2, cs), mul_rn(x1, sn));
      }
    }
#pragma unroll
    for (int kd = 0; kd < 2; ++kd) {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[kd][j] *= sl2;
      pack(x[kd], qh[kd], ql[kd], std::true_type{});
    }
#pragma unroll
    for (int kd = 2; kd < 8; ++kd) {
      float y[8];
      load_qn(kd, y);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] *= sl2;
      pack(y, qh[kd], ql[kd], std::true_type{});
    }
  }

  const int q_last = a.start + min(16 * qb + 15, a.length - 1);  // last query position of the block
  const int npages = q_last / kPageTokens + 1;                   // <= pt_len (checked on the host)
  const int nblk = (npages + 1) / 2;
  const int kmax = min(q_last, ctx_total - 1);  // last key any column of the block uses
  const int q_first = a.start + 16 * qb;         // first query position of the block

  // Direct-to-LDS copy of key block b (K and V tiles of pages 2b, 2b+1) into
  // ring slot b % 4: 4 loads of 16 bytes per thread; a page past the block's
  // range reads page 0 and is masked out.
  auto slot_of = [&](int b) { return ring + (b % kRingSlots) * kSlotVec; };
  auto issue = [&](int b) {
    u32x4* slot = slot_of(b);
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
      const int p = 2 * b + pg;
      int phys = p < npages ? (a.staged ? p : pt[p]) : 0;
      phys = (phys < 0 || phys >= a.num_pages) ? 0 : phys;  // unallocated entries never fault
      const int64_t tile = (int64_t)phys * a.num_kv_heads + kvh;
      const u32x4* kp = reinterpret_cast<const u32x4*>(a.k_cache + tile * kTile);
      const u32x4* vp = reinterpret_cast<const u32x4*>(a.v_cache + tile * kTile);
      const int v = wave * 64;  // this wave's 64 vectors of each tile; lane l lands at +l
      __builtin_amdgcn_global_load_lds(kp + v + lane, slot + pg * kSlotK1 + v, 16, 0, 0);
      // V^T position (half, dim) = v + lane holds tile vector 2 dim + half
      const int vdim = (wave & 3) * 64 + lane, vhalf = wave >> 2;
      __builtin_amdgcn_global_load_lds(vp + 2 * vdim + vhalf, slot + kSlotV + pg * kTileVec + v, 16, 0, 0);
    }
  };

  // O^T tiles: dims 16 dt + 4 g4 + i, column n; o[16] is the product with an
  // all-ones V^T tile, every row the sum of the column's probabilities as
  // the MFMAs weighted V with them (the softmax's normaliser, no VALU adds
  // and no cross-lane sum)
  f32x4 o[17];
#pragma unroll
  for (int dt = 0; dt < 17; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  constexpr uint32_t kOne2 = KVT == RIA_DT_F16 ? 0x3C003C00u : 0x3F803F80u;  // two 16-bit 1.0

  // K operand rows of this lane (row n of both score tiles): vector offset of
  // token tile_row_token(m, n) of page tile_row_page(n); dims 32 kd + 8 g4 ..
  // + 7 are dim group q8 = 4 kd + g4 at vector ((q8 % 8) * 4 + q8 / 8) * 16.
  const int k_row0 = tile_row_page(n) * kSlotK1 + tile_row_token(0, n);
  const int k_row1 = tile_row_page(n) * kSlotK1 + tile_row_token(1, n);
  // V^T operand of this lane for dim tile dt: dim 16 dt + n, tokens
  // 8 (g4 % 2) .. + 7 of page g4 / 2 (one 16-byte vector).
  const int v_vec = kSlotV + (g4 >> 1) * kTileVec + (g4 & 1) * 256 + n;
  // key of result row i of score tile m in this lane: 32 b + 8 g4 + 4 m + i

  // Each phase first issues all of its LDS operand reads, then its MFMAs
  // (scheduling barriers keep the compiler from re-serialising them); the
  // V^T reads of a block go out before its softmax so they land meanwhile.
  //
  // ---- scores of block b: two 16-key tiles; q_hi and q_lo products in separate
  //      accumulators so no MFMA waits on the one just before it
  auto qk = [&](int b, f32x4 (&sc)[2]) {
    const u32x4* slot = slot_of(b);
    u32x4 kop[8][2];
#pragma unroll
    for (int kd = 0; kd < 8; ++kd) {
      const int q8 = 4 * kd + g4;
      const int goff = ((q8 & 7) * 4 + (q8 >> 3)) * kPageTokens;
      kop[kd][0] = slot[k_row0 + goff];
      kop[kd][1] = slot[k_row1 + goff];
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kd = 0; kd < 8; ++kd) {
      acc[0] = KV::mfma_k32(kop[kd][0], qh[kd], acc[0]);
      acc[1] = KV::mfma_k32(kop[kd][1], qh[kd], acc[1]);
      if (kSplit) {
        acc[2] = KV::mfma_k32(kop[kd][0], ql[kd], acc[2]);
        acc[3] = KV::mfma_k32(kop[kd][1], ql[kd], acc[3]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    sc[0] = kSplit ? acc[0] + acc[2] : acc[0];
    sc[1] = kSplit ? acc[1] + acc[3] : acc[1];
  };

  auto load_v = [&](int b, u32x4 (&vop)[17]) {
    const u32x4* slot = slot_of(b);
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) vop[dt] = slot[v_vec + 16 * dt];
  };

  // ---- online softmax of block b (log2 units), then O^T += V^T P^T over its 32 keys
  auto softmax_pv = [&](int b, const f32x4 (&sc)[2]) {
    u32x4 vop[17];
    load_v(b, vop);
    vop[16] = u32x4{kOne2, kOne2, kOne2, kOne2};
    __builtin_amdgcn_sched_barrier(0);
    float s[8];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[4 * m + i] = sc[m][i];
    if (32 * b + 31 > q_first) {
      // blocks reaching past the block's first query need the causal mask
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (32 * b + 8 * g4 + 4 * m + i > qlim) s[4 * m + i] = -INFINITY;
    }
    // The probabilities against the running max go out at once; only a
    // block with a score more than 2^8 above it (every column's first block
    // among them) needs the column max (permlane swaps), the rescale and the
    // probabilities again.  m_run is the same in the four lanes of a column,
    // so a lane's own max decides as the column max would.
    const float mloc = max3_f(max3_f(s[0], s[1], s[2]), max3_f(s[3], s[4], s[5]), max3_f(s[6], s[7], s[7]));
    float pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pr[j] = __builtin_amdgcn_exp2f(s[j] - m_run);
      asm volatile("" : "+v"(pr[j]));  // computed here, beside the vote, not sunk past the branch
    }
    if (__any(mloc > m_run + 8.0f)) {
      const float mx = swap_max(swap_max(mloc, true), false);
      // m_run is finite from the first block on (key 0 is visible to every
      // column), so masked scores give exp2(-inf) = 0
      const bool grow = mx > m_run + 8.0f;
      const float m_new = grow ? mx : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first block, where o and l are 0
#pragma unroll
      for (int dt = 0; dt < 17; ++dt) o[dt] *= alpha;
      m_run = m_new;
#pragma unroll
      for (int j = 0; j < 8; ++j) pr[j] = __builtin_amdgcn_exp2f(s[j] - m_run);
    }
    u32x4 ph, pl;
    pack(pr, ph, pl, std::false_type{});
    __builtin_amdgcn_sched_barrier(0);
    // all hi products, then all lo products: 17 MFMAs between dependent ones
#pragma unroll
    for (int dt = 0; dt < 17; ++dt) o[dt] = KV::mfma_k32(vop[dt], ph, o[dt]);
    if (kSplit) {
#pragma unroll
      for (int dt = 0; dt < 17; ++dt) o[dt] = KV::mfma_k32(vop[dt], pl, o[dt]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Key blocks arrive in pairs, two blocks ahead.  At an even block every
  // copy this thread has in flight (the pair b, b + 1, issued two iterations
  // earlier) is waited for, then the barrier makes every thread's copies
  // landed and every wave done with blocks b - 2 and b - 1, whose slots take
  // the next pair.  An odd block's pair has already landed, so odd blocks
  // pass no barrier and the waves drift apart by up to a block (the two
  // waves of a SIMD then rarely reach the softmax at once).  The wait is for
  // all copies, not a count of them: it relies on no ordering among the
  // direct-to-LDS copies, only on each being written to LDS when the counter
  // no longer holds it; pairing gives each copy two iterations to land.
  f32x4 sc[2];
  issue(0);
  if (nblk > 1) issue(1);
  for (int b = 0; b < nblk; ++b) {
    if ((b & 1) == 0) {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (b + 2 < nblk) issue(b + 2);
      if (b + 3 < nblk) issue(b + 3);
    }
    u32x4* slot = slot_of(b);
    if (32 * b + 31 > kmax) {
      // last block: zero V of keys past the last one used, so that
      // 0-probability keys cannot bring NaN/Inf from unwritten slots
#pragma unroll
      for (int j2 = 0; j2 < 2; ++j2) {
        const int vi = j2 * kPrefillThreads + tid;  // vector of the block's two V^T tiles
        const int m = vi / kTileVec;                 // page of the block
        const int half = (vi % kTileVec) >> 8;       // token half: tokens 8 half .. + 7 of one dim
        const int k0 = 32 * b + 16 * m + 8 * half;
        u32x4 w = slot[kSlotV + vi];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint32_t x = w[j];
          if (k0 + 2 * j > kmax) x &= 0xffff0000u;
          if (k0 + 2 * j + 1 > kmax) x &= 0x0000ffffu;
          w[j] = x;
        }
        slot[kSlotV + vi] = w;
      }
      lds_barrier();
    }

    qk(b, sc);
    softmax_pv(b, sc);
  }

  // ---- normalise, stage (the ring is dead once every wave has left the loop), gate, store
  lds_barrier();
  const float l_tot = o[16][0];
  const float inv = 1.0f / l_tot;  // every valid query sees at least itself
  float* st = stage + (wave * 16 + n) * kStagePitch;
#pragma unroll
  for (int dt = 0; dt < 16; ++dt)
    *reinterpret_cast<f32x4*>(st + 16 * dt + 4 * g4) = o[dt] * inv;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (!head_ok) return;
  for (int r = 0; r < 16; ++r) {
    const int t = 16 * qb + r;
    if (t >= a.length) break;
    const int d = 4 * lane;
    // one 16-byte read of the staged row (element reads would hit 4-way bank conflicts)
    const f32x4 row = *reinterpret_cast<const f32x4*>(stage + (wave * 16 + r) * kStagePitch + d);
    float g[4], y[4];
    load_act4<AT>(a.gate, (int64_t)t * a.gate_stride + (int64_t)head * kAttnHeadDim + d, g);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      y[i] = AT == RIA_DT_BF16 ? gate_mul_to_bf16(row[i], g[i]) : mul_rn(row[i], sigmoid_f(g[i]));
    store_act4<AT>(a.out, ((int64_t)t * a.num_q_heads + head) * kAttnHeadDim + d, y);
  }
}

template <int AT>
static void launch_prefill(const PrefillAttnArgs& a, const int32_t* pt, int kv_dtype, dim3 grid, hipStream_t st) {
  if (kv_dtype == RIA_DT_F16)
    hipLaunchKernelGGL((attn_prefill_kernel<AT, RIA_DT_F16>), grid, dim3(kPrefillThreads), 0, st, a, pt);
  else
    hipLaunchKernelGGL((attn_prefill_kernel<AT, RIA_DT_BF16>), grid, dim3(kPrefillThreads), 0, st, a, pt);
}

}  // namespace ria

using namespace ria;



namespace ria {
int kv_append_seq_impl(int length, int num_kv_heads, const void* k, int k_dtype, int64_t k_row_stride,
                       const void* v, int v_dtype, int64_t v_row_stride, void* k_cache, void* v_cache, int kv_dtype,
                       int num_pages, const int32_t* page_table_row, int64_t page_capacity, int32_t start_pos,
                       const float* inv_freq, int rope_dim, const float* k_norm_weight, uint16_t* stage_k,
                       uint16_t* stage_v, void* stream);

static int64_t stage_half_bytes(int length, int num_kv_heads) {
  return (int64_t)((length + kPageTokens - 1) / kPageTokens) * num_kv_heads * kTile * 2;
}

static int prefill_impl(int length, int num_q_heads, int num_kv_heads, const void* q, int64_t q_row_stride,
                        const void* k, int64_t k_row_stride, const void* v, int64_t v_row_stride, const void* gate,
                        int64_t gate_row_stride, int act_dtype, void* k_cache, void* v_cache, int kv_dtype,
                        int num_pages, const int32_t* page_table_row, int64_t page_capacity, int32_t start_pos,
                        const float* inv_freq, int rope_dim, const float* q_norm_weight, const float* k_norm_weight,
                        float scale, void* stage, int64_t stage_bytes, void* out, int phase, void* stream) {
  if (phase < RIA_PREFILL_APPEND || phase > RIA_PREFILL_BOTH)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: phase must be 1 (append), 2 (attention) or 3 (both)");
  if (length < 0 || start_pos < 0) return set_error(RIA_ERR_INVALID, "ria_attn_prefill: negative length or start");
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: num_q_heads must be a multiple of num_kv_heads");
  const int group = num_q_heads / num_kv_heads;
  if (group > 8) return set_error(RIA_ERR_INVALID, "ria_attn_prefill: at most 8 query heads per KV head");
  if (act_dtype != RIA_DT_BF16 && act_dtype != RIA_DT_F16 && act_dtype != RIA_DT_F32)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: unknown dtype code");
  if (kv_dtype != RIA_DT_BF16 && kv_dtype != RIA_DT_F16)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: the KV cache must be bf16 or fp16");
  if (!q || !k || !v || !gate || !k_cache || !v_cache || !page_table_row || !out)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: null pointer");
  if (rope_dim != 0 && rope_dim != 64) return set_error(RIA_ERR_INVALID, "ria_attn_prefill: rope_dim must be 0 or 64");
  if (rope_dim && !inv_freq) return set_error(RIA_ERR_INVALID, "ria_attn_prefill: inv_freq is null");
  if (reinterpret_cast<uintptr_t>(q_norm_weight) % 16)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: q_norm_weight must be 16-byte aligned");
  if ((int64_t)start_pos + length > page_capacity * kPageTokens)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: %d + %d tokens exceed the row's %lld pages", start_pos,
                     length, (long long)page_capacity);
  if (q_row_stride < (int64_t)num_q_heads * kAttnHeadDim || gate_row_stride < (int64_t)num_q_heads * kAttnHeadDim)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: row stride smaller than Hq*256");
  // q, gate and out move in 16-byte vectors
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(out)) % 16 ||
      q_row_stride % 8 || gate_row_stride % 8)
    return set_error(RIA_ERR_INVALID, "ria_attn_prefill: q, gate and out must be 16-byte aligned, row strides multiples of 8");
  if (length == 0) return RIA_OK;
  const int64_t blocks = (int64_t)((length + 15) / 16) * num_kv_heads;
  if (blocks > 0x7fffffff) return set_error(RIA_ERR_INVALID, "ria_attn_prefill: grid too large");
  // a prompt from slot 0 with a stage: its keys also go to fp16 tiles, which the attention reads
  const bool staged = stage && start_pos == 0;
  uint16_t* stage_k = nullptr;
  uint16_t* stage_v = nullptr;
  if (staged) {
    const int64_t half = stage_half_bytes(length, num_kv_heads);
    if (stage_bytes < 2 * half)
      return set_error(RIA_ERR_WORKSPACE, "ria_attn_prefill: stage %lld bytes < required %lld",
                       (long long)stage_bytes, (long long)(2 * half));
    if (reinterpret_cast<uintptr_t>(stage) % 16) return set_error(RIA_ERR_INVALID, "ria_attn_prefill: stage must be 16-byte aligned");
    stage_k = static_cast<uint16_t*>(stage);
    stage_v = stage_k + half / 2;
  }
  if (phase & RIA_PREFILL_APPEND) {
    int rc = kv_append_seq_impl(length, num_kv_heads, k, act_dtype, k_row_stride, v, act_dtype, v_row_stride,
                                k_cache, v_cache, kv_dtype, num_pages, page_table_row, page_capacity, start_pos,
                                inv_freq, rope_dim, k_norm_weight, stage_k, stage_v, stream);
    if (rc != RIA_OK) return rc;
  }
  if (!(phase & RIA_PREFILL_ATTEND)) return RIA_OK;
  PrefillAttnArgs a{};
  a.q = q;
  a.q_stride = q_row_stride;
  a.gate = gate;
  a.gate_stride = gate_row_stride;
  a.k_cache = static_cast<const uint16_t*>(k_cache);
  a.v_cache = static_cast<const uint16_t*>(v_cache);
  a.num_pages = num_pages;
  a.pt_len = page_capacity;
  a.start = start_pos;
  a.length = length;
  a.inv_freq = inv_freq;
  a.rope_dim = rope_dim;
  a.q_norm_w = q_norm_weight;
  a.scale = scale;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  a.out = out;
  int key_dtype = kv_dtype;
  if (staged) {  // the prompt's own fp16 tiles, logical page p at tile p
    a.k_cache = stage_k;
    a.v_cache = stage_v;
    a.num_pages = (length + kPageTokens - 1) / kPageTokens;
    a.staged = 1;
    key_dtype = RIA_DT_F16;
  }
  dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (act_dtype == RIA_DT_BF16)
    launch_prefill<RIA_DT_BF16>(a, page_table_row, key_dtype, grid, st);
  else if (act_dtype == RIA_DT_F16)
    launch_prefill<RIA_DT_F16>(a, page_table_row, key_dtype, grid, st);
  else
    launch_prefill<RIA_DT_F32>(a, page_table_row, key_dtype, grid, st);
  return check_launch("ria_attn_prefill");
}
}  // namespace ria

extern "C" int ria_attn_prefill_phase(int length, int num_q_heads, int num_kv_heads, const void* q,
                                      int64_t q_row_stride, const void* k, int64_t k_row_stride, const void* v,
                                      int64_t v_row_stride, const void* gate, int64_t gate_row_stride, int act_dtype,
                                      void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                                      const int32_t* page_table_row, int64_t page_capacity, int32_t start_pos,
                                      const float* inv_freq, int rope_dim, const float* q_norm_weight,
                                      const float* k_norm_weight, float scale, void* out, int phase,
                                      void* stream) {
  return prefill_impl(length, num_q_heads, num_kv_heads, q, q_row_stride, k, k_row_stride, v, v_row_stride, gate,
                      gate_row_stride, act_dtype, k_cache, v_cache, kv_dtype, num_pages, page_table_row,
                      page_capacity, start_pos, inv_freq, rope_dim, q_norm_weight, k_norm_weight, scale, nullptr, 0,
                      out, phase, stream);
}

extern "C" int64_t ria_attn_prefill_stage_bytes(int length, int num_kv_heads) {
  if (length <= 0 || num_kv_heads <= 0) return 0;
  return 2 * stage_half_bytes(length, num_kv_heads);
}

extern "C" int ria_attn_prefill_staged(int length, int num_q_heads, int num_kv_heads, const void* q,
                                       int64_t q_row_stride, const void* k, int64_t k_row_stride, const void* v,
                                       int64_t v_row_stride, const void* gate, int64_t gate_row_stride,
                                       int act_dtype, void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                                       const int32_t* page_table_row, int64_t page_capacity, int32_t start_pos,
                                       const float* inv_freq, int rope_dim, const float* q_norm_weight,
                                       const float* k_norm_weight, float scale, void* stage, int64_t stage_bytes,
                                       void* out, int phase, void* stream) {
  if (!stage) return set_error(RIA_ERR_INVALID, "ria_attn_prefill_staged: null stage");
  return prefill_impl(length, num_q_heads, num_kv_heads, q, q_row_stride, k, k_row_stride, v, v_row_stride, gate,
                      gate_row_stride, act_dtype, k_cache, v_cache, kv_dtype, num_pages, page_table_row,
                      page_capacity, start_pos, inv_freq, rope_dim, q_norm_weight, k_norm_weight, scale, stage,
                      stage_bytes, out, phase, stream);
}

extern "C" int ria_attn_prefill(int length, int num_q_heads, int num_kv_heads, const void* q, int64_t q_row_stride,
                                const void* k, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                const void* gate, int64_t gate_row_stride, int act_dtype, void* k_cache,
                                void* v_cache, int kv_dtype, int num_pages, const int32_t* page_table_row,
                                int64_t page_capacity, int32_t start_pos, const float* inv_freq, int rope_dim,
                                const float* q_norm_weight, const float* k_norm_weight, float scale, void* out,
                                void* stream) {
  return ria_attn_prefill_phase(length, num_q_heads, num_kv_heads, q, q_row_stride, k, k_row_stride, v, v_row_stride,
                                gate, gate_row_stride, act_dtype, k_cache, v_cache, kv_dtype, num_pages,
                                page_table_row, page_capacity, start_pos, inv_freq, rope_dim, q_norm_weight,
                                k_norm_weight, scale, out, RIA_PREFILL_BOTH, stream);
}
