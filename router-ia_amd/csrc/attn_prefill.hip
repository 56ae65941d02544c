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
//   * the 4 waves own two query heads each (GQA group <= 8): a wave's 32
//     columns are (head, token) pairs, so one 32x32x16 MFMA covers 32 keys x
//     32 queries and every key block fetched serves 16 tokens x 8 heads;
//   * key blocks travel HBM/L2 -> LDS by direct-to-LDS loads into a 3-slot
//     ring, two blocks ahead of the one being computed, with no registers
//     in flight;
//   * scores S^T = K Q^T: the K tile is already in A-operand order (8 dims
//     of one token are 16 contiguous bytes); the rows of a 32-key block take
//     the tokens of each page in the order 0-3, 8-11, 4-7, 12-15, which makes
//     a lane's 16 score rows exactly the 8 + 8 consecutive tokens whose V^T
//     columns it reads as one 16-byte operand for O^T = V^T P^T;
//   * the rotated q and the probabilities are carried as 16-bit hi + lo
//     pairs (near-fp32 operands on MFMA); the online softmax is kept in log2
//     units with a lazy rescale (only when a block max exceeds the running
//     max by 2^8); row statistics combine across the two lane halves with
//     permlane32 swaps;
//   * the gated result leaves through LDS so the output stores are coalesced;
//   * query blocks are scheduled from the last (most keys) to the first.
#include <math.h>

#include "ria_common.h"

namespace ria {

constexpr int kTile = kPageTokens * kAttnHeadDim;  // elements per (page, KV head) tile
constexpr int kTileVec = kTile * 2 / 16;           // 16-byte vectors per tile (512)
constexpr int kSlotVec = 4 * kTileVec;             // ring slot: K page 0, K page 1, V page 0, V page 1
constexpr int kRingSlots = 3;
constexpr int kStagePitch = kAttnHeadDim + 4;      // floats per staged output row
constexpr int kPrefillLds = 4 * 32 * kStagePitch * 4;  // output stage; the ring (96 KiB) aliases it
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
  float scale;
  int num_q_heads;
  int num_kv_heads;
  int group;
  void* out;
};

// Token of a page held by row i (0..15) of a key block: groups of four in the
// order 0-3, 8-11, 4-7, 12-15.
__device__ __forceinline__ int block_row_token(int i) { return 4 * (((i >> 2) & 1) * 2 + (i >> 3)) + (i & 3); }

__device__ __forceinline__ float swap32_max(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

__device__ __forceinline__ float swap32_sum(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

template <int AT, int KVT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_prefill_kernel(
    PrefillAttnArgs a, const int32_t* __restrict__ pt) {
  using KV = Kv16<KVT>;
  const int nqb = (a.length + 15) / 16;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x) / a.num_kv_heads;  // heaviest blocks first
  const int kvh = static_cast<int>(blockIdx.x) % a.num_kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31;  // MFMA column: (head 2 wave + c/16, token c%16); PV: dim row
  const int h = lane >> 5;  // k half of the MFMA operands

  __shared__ __attribute__((aligned(16))) unsigned char smem[kPrefillLds];
  u32x4* ring = reinterpret_cast<u32x4*>(smem);
  float* stage = reinterpret_cast<float*>(smem);

  const int hh = c >> 4;
  const bool head_ok = 2 * wave + hh < a.group;
  const int head = kvh * a.group + 2 * wave + hh;
  const int t_row = 16 * qb + (c & 15);
  const bool row_ok = head_ok && t_row < a.length;
  const int qpos = a.start + t_row;
  const int ctx_total = a.start + a.length;  // keys that exist
  const int qlim = min(qpos, ctx_total - 1);  // last key this column sees

  // ---- q operands: column c, dims 16 kd + 8 h + j, RoPE'd, as hi + lo pairs
  u32x4 qh[16], ql[16];
  auto pack = [&](const float (&x)[8], u32x4& hi, u32x4& lo) {
    uint32_t h4[4], l4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t a0 = KV::from_f32(x[2 * j]), a1 = KV::from_f32(x[2 * j + 1]);
      const uint16_t b0 = KV::from_f32(x[2 * j] - KV::to_f32(a0));
      const uint16_t b1 = KV::from_f32(x[2 * j + 1] - KV::to_f32(a1));
      h4[j] = a0 | (uint32_t(a1) << 16);
      l4[j] = b0 | (uint32_t(b1) << 16);
    }
    hi = u32x4{h4[0], h4[1], h4[2], h4[3]};
    lo = u32x4{l4[0], l4[1], l4[2], l4[3]};
  };
  {
    const int64_t base = (int64_t)t_row * a.q_stride + (int64_t)head * kAttnHeadDim + 8 * h;
    // dims [0, 64): kd 0..3; rotate_half pairs kd with kd ^ 2 at the same j
    float x[4][8];
#pragma unroll
    for (int kd = 0; kd < 4; ++kd) {
      if (row_ok) {
        load_act8<AT>(a.q, base + 16 * kd, x[kd]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[kd][j] = 0.f;
      }
    }
    if (a.rope_dim == 64) {
      const float pos = static_cast<float>(qpos);
#pragma unroll
      for (int kd = 0; kd < 2; ++kd) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float ang = mul_rn(pos, a.inv_freq[16 * kd + 8 * h + j]);
          const float cs = cosf(ang), sn = sinf(ang);
          const float x1 = x[kd][j], x2 = x[kd + 2][j];
          x[kd][j] = add_rn(mul_rn(x1, cs), mul_rn(-x2, sn));
          x[kd + 2][j] = add_rn(mul_rn(x2, cs), mul_rn(x1, sn));
        }
      }
    }
#pragma unroll
    for (int kd = 0; kd < 4; ++kd) pack(x[kd], qh[kd], ql[kd]);
#pragma unroll
    for (int kd = 4; kd < 16; ++kd) {
      float y[8];
      if (row_ok) {
        load_act8<AT>(a.q, base + 16 * kd, y);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = 0.f;
      }
      pack(y, qh[kd], ql[kd]);
    }
  }

  const int q_last = a.start + min(16 * qb + 15, a.length - 1);  // last query position of the block
  const int npages = q_last / kPageTokens + 1;                   // <= pt_len (checked on the host)
  const int nblk = (npages + 1) / 2;
  const int kmax = min(q_last, ctx_total - 1);  // last key any column of the block uses

  // Direct-to-LDS copy of key block b (K and V tiles of pages 2b, 2b+1) into
  // ring slot b % 3: 8 loads of 16 bytes per thread, always 8 so that the
  // wait counts below hold; a page past the block's range reads page 0 and
  // is masked out.
  auto issue = [&](int b) {
    u32x4* slot = ring + (b % kRingSlots) * kSlotVec;
#pragma unroll
    for (int pg = 0; pg < 2; ++pg) {
      const int p = 2 * b + pg;
      int phys = p < npages ? pt[p] : 0;
      phys = (phys < 0 || phys >= a.num_pages) ? 0 : phys;  // unallocated entries never fault
      const int64_t tile = (int64_t)phys * a.num_kv_heads + kvh;
      const u32x4* kp = reinterpret_cast<const u32x4*>(a.k_cache + tile * kTile);
      const u32x4* vp = reinterpret_cast<const u32x4*>(a.v_cache + tile * kTile);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int v = i * 256 + wave * 64;  // this wave's 64 vectors; lane l lands at +l
        __builtin_amdgcn_global_load_lds(kp + v + lane, slot + pg * kTileVec + v, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vp + v + lane, slot + (2 + pg) * kTileVec + v, 16, 0, 0);
      }
    }
  };

  const float sl2 = a.scale * 1.4426950408889634f;  // scores in log2 units
  f32x16 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // K operand of lane (c, h) for dim block kd: key row c -> page c / 16,
  // token block_row_token(c % 16); dims 16 kd + 8 h .. + 7 -> vector
  // ((g % 8) * 4 + g / 8) * 16 + token of the K tile, g = 2 kd + h.
  const int k_row_vec = (c >> 4) * kTileVec + block_row_token(c & 15);

  issue(0);
  if (nblk > 1) issue(1);
  for (int b = 0; b < nblk; ++b) {
    // this thread's copies of block b have landed; after the barrier every
    // thread's have, and every wave is done with slot (b + 2) % 3
    if (b + 1 < nblk)
      asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (b + 2 < nblk) issue(b + 2);
    u32x4* slot = ring + (b % kRingSlots) * kSlotVec;
    if (32 * b + 31 > kmax) {
      // last block: zero V of keys past the last one used, so that
      // 0-probability keys cannot bring NaN/Inf from unwritten slots
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int vi = i * 256 + tid;            // vector of the block's two V tiles
        const int m = vi / kTileVec;             // page of the block
        const int tok0 = 8 * (vi & 1);           // tokens tok0 .. tok0 + 7 of one dim
        const int k0 = 32 * b + 16 * m + tok0;
        u32x4 w = slot[2 * kTileVec + vi];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint32_t x = w[j];
          if (k0 + 2 * j > kmax) x &= 0xffff0000u;
          if (k0 + 2 * j + 1 > kmax) x &= 0x0000ffffu;
          w[j] = x;
        }
        slot[2 * kTileVec + vi] = w;
      }
      lds_barrier();
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) asm volatile("" : "+a"(o[dt]));

    f32x16 sh, sl;
#pragma unroll
    for (int r = 0; r < 16; ++r) sh[r] = sl[r] = 0.f;
    auto k_operand = [&](int kd) {
      const int g = 2 * kd + h;
      return slot[k_row_vec + ((g & 7) * 4 + (g >> 3)) * kPageTokens];
    };
    u32x4 kb[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) kb[0][i] = k_operand(i);
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      if (grp + 1 < 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) kb[(grp + 1) & 1][i] = k_operand(4 * (grp + 1) + i);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sh = KV::mfma32(kb[grp & 1][i], qh[4 * grp + i], sh);
        sl = KV::mfma32(kb[grp & 1][i], ql[4 * grp + i], sl);
      }
    }
    // keep four LDS reads in flight ahead of the MFMAs that consume them
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      if (grp + 1 < 4) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    }
    // row r of this lane holds key 32 b + 16 (r / 8) + 8 h + r % 8
    const int key0 = 32 * b + 8 * h;
    float s[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kpos = key0 + 16 * (r >> 3) + (r & 7);
      s[r] = kpos <= qlim ? (sh[r] + sl[r]) * sl2 : -INFINITY;
      mx = fmaxf(mx, s[r]);
    }
    mx = swap32_max(mx);
    const bool grow = mx > m_run + 8.0f;
    if (__any(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        // through VGPRs here only; the accumulators otherwise stay in AGPRs
        f32x16 t = o[dt];
        asm volatile("" : "+v"(t));
        t *= alpha;
        o[dt] = t;
        asm volatile("" : "+a"(o[dt]));
      }
      m_run = m_new;
    }
    u32x4 ph[2], pl[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      float pr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sv = s[8 * m + j];
        pr[j] = sv == -INFINITY ? 0.f : exp2f(sv - m_run);
        l_run += pr[j];
      }
      pack(pr, ph[m], pl[m]);
    }
    // V^T operand of lane (c, h), dim block dt, page m: dim 32 dt + c,
    // tokens 8 h .. 8 h + 7 (16 contiguous bytes of the V tile)
    auto v_operand = [&](int dt, int m) { return slot[(2 + m) * kTileVec + (32 * dt + c) * 2 + h]; };
    u32x4 vb[2][2];
    vb[0][0] = v_operand(0, 0);
    vb[0][1] = v_operand(0, 1);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      if (dt + 1 < 8) {
        vb[(dt + 1) & 1][0] = v_operand(dt + 1, 0);
        vb[(dt + 1) & 1][1] = v_operand(dt + 1, 1);
      }
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        o[dt] = KV::mfma32(vb[dt & 1][m], ph[m], o[dt]);
        o[dt] = KV::mfma32(vb[dt & 1][m], pl[m], o[dt]);
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      if (dt + 1 < 8) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
    // keep the accumulators resident in AGPRs across iterations (the rare
    // rescale above then copies them out and back only when it runs)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) asm volatile("" : "+a"(o[dt]));
  }

  // ---- normalise, stage (the ring is dead once every wave has left the loop), gate, store
  lds_barrier();
  const float l_tot = swap32_sum(l_run);
  const float inv = 1.0f / l_tot;  // every valid query sees at least itself
  float* st = stage + (wave * 32 + c) * kStagePitch;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
      // rows 8 a4 + 4 h + i of MFMA tile dt are dims 32 dt + 8 a4 + 4 h + i
      const f32x4 v = {o[dt][4 * a4] * inv, o[dt][4 * a4 + 1] * inv, o[dt][4 * a4 + 2] * inv,
                       o[dt][4 * a4 + 3] * inv};
      *reinterpret_cast<f32x4*>(st + 32 * dt + 8 * a4 + 4 * h) = v;
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  for (int col = 0; col < 32; ++col) {
    const int t = 16 * qb + (col & 15);
    const int hw = 2 * wave + (col >> 4);
    if (t >= a.length || hw >= a.group) continue;
    const int hd = kvh * a.group + hw;
    const int d = 4 * lane;
    const float* row = stage + (wave * 32 + col) * kStagePitch + d;
    float g[4], y[4];
    load_act4<AT>(a.gate, (int64_t)t * a.gate_stride + (int64_t)hd * kAttnHeadDim + d, g);
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = mul_rn(row[i], sigmoid_f(g[i]));
    store_act4<AT>(a.out, ((int64_t)t * a.num_q_heads + hd) * kAttnHeadDim + d, y);
  }
}

template <int AT>
static void launch_prefill(const PrefillAttnArgs& a, const int32_t* pt, int kv_dtype, dim3 grid, hipStream_t st) {
  if (kv_dtype == RIA_DT_F16)
    hipLaunchKernelGGL((attn_prefill_kernel<AT, RIA_DT_F16>), grid, dim3(256), 0, st, a, pt);
  else
    hipLaunchKernelGGL((attn_prefill_kernel<AT, RIA_DT_BF16>), grid, dim3(256), 0, st, a, pt);
}

}  // namespace ria

using namespace ria;

extern "C" int ria_kv_append_seq(int length, int num_kv_heads, const void* k, int k_dtype, int64_t k_row_stride,
                                 const void* v, int v_dtype, int64_t v_row_stride, void* k_cache, void* v_cache,
                                 int kv_dtype, int num_pages, const int32_t* page_table_row, int64_t page_capacity,
                                 int32_t start_pos, const float* inv_freq, int rope_dim, void* stream);

extern "C" int ria_attn_prefill(int length, int num_q_heads, int num_kv_heads, const void* q, int64_t q_row_stride,
                                const void* k, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                const void* gate, int64_t gate_row_stride, int act_dtype, void* k_cache,
                                void* v_cache, int kv_dtype, int num_pages, const int32_t* page_table_row,
                                int64_t page_capacity, int32_t start_pos, const float* inv_freq, int rope_dim,
                                float scale, void* out, void* stream) {
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
  int rc = ria_kv_append_seq(length, num_kv_heads, k, act_dtype, k_row_stride, v, act_dtype, v_row_stride, k_cache,
                             v_cache, kv_dtype, num_pages, page_table_row, page_capacity, start_pos, inv_freq,
                             rope_dim, stream);
  if (rc != RIA_OK) return rc;
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
  a.scale = scale;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  a.out = out;
  dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (act_dtype == RIA_DT_BF16)
    launch_prefill<RIA_DT_BF16>(a, page_table_row, kv_dtype, grid, st);
  else if (act_dtype == RIA_DT_F16)
    launch_prefill<RIA_DT_F16>(a, page_table_row, kv_dtype, grid, st);
  else
    launch_prefill<RIA_DT_F32>(a, page_table_row, kv_dtype, grid, st);
  return check_launch("ria_attn_prefill");
}
