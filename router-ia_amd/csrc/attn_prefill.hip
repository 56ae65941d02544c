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
// block, KV head) streams the keys 0 .. last query of the block.
//   * the workgroup's 4 waves own two query heads each (GQA group <= 8), so
//     every (page, KV head) tile is fetched from HBM/L2 once per workgroup and
//     serves 16 tokens x 8 heads; tiles are staged in a 2-slot LDS ring, the
//     next page travels in registers while the current one is computed;
//   * scores S^T = K Q^T and O^T = V^T P^T run on MFMA in the operand orders
//     of the decode kernel (K tile in A-operand order, V transposed), with the
//     rotated q and the probabilities carried as 16-bit hi + lo pairs and the
//     online softmax kept in log2 units with a lazy rescale;
//   * the gated result leaves through LDS so the output stores are coalesced;
//   * query blocks are scheduled from the last (most keys) to the first.
#include <math.h>

#include "ria_common.h"

namespace ria {

constexpr int kTile = kPageTokens * kAttnHeadDim;  // elements per (page, KV head) tile
constexpr int kTileVec = kTile * 2 / 16;           // u32x4 per tile (512)

struct PrefillAttnArgs {
  const void* q;
  int64_t q_stride;
  const void* gate;
  int64_t gate_stride;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int num_pages;
  const int32_t* pt;  // this sequence's page table row
  int64_t pt_len;
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

template <int AT, int KVT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_prefill_kernel(
    PrefillAttnArgs a) {
  using KV = Kv16<KVT>;
  const int nqb = (a.length + 15) / 16;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x) / a.num_kv_heads;  // heaviest blocks first
  const int kvh = static_cast<int>(blockIdx.x) % a.num_kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g4 = lane >> 4;

  __shared__ u32x4 ring[2][2 * kTileVec];           // 2 slots x (K tile, V tile): 32 KiB
  __shared__ float stage[4][16][kAttnHeadDim + 4];  // per-wave output rows: 65 KiB

  const int nrb = max(0, min(2, a.group - 2 * wave));  // query heads of this wave (0..2)

  // ---- q operands: token 16 qb + n of heads (kvh * G + 2 wave + rb),
  //      dims 64 g4 + 8 kk + j (the B operand matching the K tile's A operand)
  const int t_row = 16 * qb + n;
  const bool row_valid = t_row < a.length;
  const float qpos = static_cast<float>(a.start + t_row);
  u32x4 qh[2][8], ql[2][8];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int head = kvh * a.group + 2 * wave + rb;
    const bool ok = row_valid && rb < nrb;
    const int64_t base = (int64_t)t_row * a.q_stride + (int64_t)head * kAttnHeadDim + 64 * g4;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = ok ? load_act<AT>(a.q, base + 8 * kk + j) : 0.f;
      if (g4 == 0 && a.rope_dim == 64) {
        // rotate_half pairs dim e with e +- 32 inside [0, 64): dims 8 kk + j
        // pair with 8 (kk ^ 4) + j, both held by this lane.
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int e = 8 * kk + j;
          const float partner = ok ? load_act<AT>(a.q, base + 8 * (kk ^ 4) + j) : 0.f;
          const float ang = mul_rn(qpos, a.inv_freq[e & 31]);
          const float c = cosf(ang), s = sinf(ang);
          x[j] = add_rn(mul_rn(x[j], c), mul_rn(e < 32 ? -partner : partner, s));
        }
      }
      uint32_t h4[4], l4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t a0 = KV::from_f32(x[2 * j]), a1 = KV::from_f32(x[2 * j + 1]);
        const uint16_t b0 = KV::from_f32(x[2 * j] - KV::to_f32(a0));
        const uint16_t b1 = KV::from_f32(x[2 * j + 1] - KV::to_f32(a1));
        h4[j] = a0 | (uint32_t(a1) << 16);
        l4[j] = b0 | (uint32_t(b1) << 16);
      }
      qh[rb][kk] = u32x4{h4[0], h4[1], h4[2], h4[3]};
      ql[rb][kk] = u32x4{l4[0], l4[1], l4[2], l4[3]};
    }
  }

  const float sl2 = a.scale * 1.4426950408889634f;  // scores in log2 units
  f32x4 o[2][16];
  float m_run[2], l_run[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int db = 0; db < 16; ++db) o[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int ctx_total = a.start + a.length;                      // keys that exist
  const int q_last = a.start + min(16 * qb + 15, a.length - 1);  // last query position of the block
  const int npages = q_last / kPageTokens + 1;                   // <= pt_len (checked on the host)
  const int qp = a.start + t_row;                                // query position of column n

  // Each thread moves 4 of the tile pair's 1024 16-byte vectors: two of K, two of V.
  auto fetch = [&](int p, u32x4(&r)[4]) {
    int phys = a.pt[p];
    phys = (phys < 0 || phys >= a.num_pages) ? 0 : phys;  // unallocated entries never fault
    const int64_t tile = (int64_t)phys * a.num_kv_heads + kvh;
    const u32x4* kp = reinterpret_cast<const u32x4*>(a.k_cache + tile * kTile);
    const u32x4* vp = reinterpret_cast<const u32x4*>(a.v_cache + tile * kTile);
    r[0] = kp[tid];
    r[1] = kp[tid + 256];
    r[2] = vp[tid];
    r[3] = vp[tid + 256];
  };
  auto stash = [&](int slot, const u32x4(&r)[4]) {
    ring[slot][tid] = r[0];
    ring[slot][tid + 256] = r[1];
    ring[slot][kTileVec + tid] = r[2];
    ring[slot][kTileVec + tid + 256] = r[3];
  };

  auto compute_page = [&](int p, int slot) {
    const int key0 = p * kPageTokens + 4 * g4;
    u32x4 kr[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) kr[kk] = ring[slot][kk * 64 + lane];
    f32x4 sc[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      sc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (rb < nrb) {
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          sc[rb] = KV::mfma_k32(kr[kk], qh[rb][kk], sc[rb]);
          sc[rb] = KV::mfma_k32(kr[kk], ql[rb][kk], sc[rb]);
        }
      }
    }
    const uint16_t* vt = reinterpret_cast<const uint16_t*>(&ring[slot][kTileVec]) + n * kPageTokens + 4 * g4;
    u32x2 vr[16];
#pragma unroll
    for (int db = 0; db < 16; ++db) vr[db] = *reinterpret_cast<const u32x2*>(vt + db * 16 * kPageTokens);
    if ((p + 1) * kPageTokens > ctx_total) {
      // keys past the end of the sequence: zero V so 0 * garbage stays 0
#pragma unroll
      for (int db = 0; db < 16; ++db) {
        uint32_t lo = vr[db].x, hi = vr[db].y;
        if (key0 + 0 >= ctx_total) lo &= 0xffff0000u;
        if (key0 + 1 >= ctx_total) lo &= 0x0000ffffu;
        if (key0 + 2 >= ctx_total) hi &= 0xffff0000u;
        if (key0 + 3 >= ctx_total) hi &= 0x0000ffffu;
        vr[db] = u32x2{lo, hi};
      }
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if (rb >= nrb) break;
      float s4[4];
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kpos = key0 + i;
        s4[i] = (kpos <= qp && kpos < ctx_total) ? sc[rb][i] * sl2 : -INFINITY;
        mx = fmaxf(mx, s4[i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // Lazy rescale: keep the reference max while the page max stays
      // within 2^8 of it.
      const bool grow = mx > m_run[rb] + 8.0f;
      if (__any(grow)) {
        const float m_new = grow ? mx : m_run[rb];
        const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run[rb] - m_new);
        l_run[rb] *= alpha;
#pragma unroll
        for (int db = 0; db < 16; ++db) o[rb][db] *= alpha;
        m_run[rb] = m_new;
      }
      uint16_t ph[4], pl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pr = (s4[i] == -INFINITY) ? 0.f : exp2f(s4[i] - m_run[rb]);
        l_run[rb] += pr;
        ph[i] = KV::from_f32(pr);
        pl[i] = KV::from_f32(pr - KV::to_f32(ph[i]));
      }
      const u32x2 pb = {ph[0] | (uint32_t(ph[1]) << 16), ph[2] | (uint32_t(ph[3]) << 16)};
      const u32x2 pbl = {pl[0] | (uint32_t(pl[1]) << 16), pl[2] | (uint32_t(pl[3]) << 16)};
#pragma unroll
      for (int db = 0; db < 16; ++db) {
        o[rb][db] = KV::mfma_k16(vr[db], pb, o[rb][db]);
        o[rb][db] = KV::mfma_k16(vr[db], pbl, o[rb][db]);
      }
    }
  };

  {
    u32x4 nxt[4];
    fetch(0, nxt);
    stash(0, nxt);
    if (npages > 1) fetch(1, nxt);
    for (int p = 0; p < npages; ++p) {
      // every wave is done with slot (p+1)&1 (page p-1) and sees page p in slot p&1
      lds_barrier();
      if (p + 1 < npages) {
        stash((p + 1) & 1, nxt);
        if (p + 2 < npages) fetch(p + 2, nxt);
      }
      compute_page(p, p & 1);
    }
  }

  // ---- normalise, gate, store through this wave's stage rows
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    if (rb >= nrb) break;
    float l = l_run[rb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = 1.0f / l;  // every query sees at least itself
#pragma unroll
    for (int db = 0; db < 16; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) stage[wave][n][db * 16 + 4 * g4 + i] = o[rb][db][i] * inv;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const int head = kvh * a.group + 2 * wave + rb;
    for (int r = 0; r < 16; ++r) {
      const int t = 16 * qb + r;
      if (t >= a.length) break;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane * 4 + c;
        const float gv =
            sigmoid_f(load_act<AT>(a.gate, (int64_t)t * a.gate_stride + (int64_t)head * kAttnHeadDim + d));
        store_act<AT>(a.out, ((int64_t)t * a.num_q_heads + head) * kAttnHeadDim + d, mul_rn(stage[wave][r][d], gv));
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
}

template <int AT>
static void launch_prefill(const PrefillAttnArgs& a, int kv_dtype, dim3 grid, hipStream_t st) {
  if (kv_dtype == RIA_DT_F16)
    hipLaunchKernelGGL((attn_prefill_kernel<AT, RIA_DT_F16>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((attn_prefill_kernel<AT, RIA_DT_BF16>), grid, dim3(256), 0, st, a);
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
  a.pt = page_table_row;
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
    launch_prefill<RIA_DT_BF16>(a, kv_dtype, grid, st);
  else if (act_dtype == RIA_DT_F16)
    launch_prefill<RIA_DT_F16>(a, kv_dtype, grid, st);
  else
    launch_prefill<RIA_DT_F32>(a, kv_dtype, grid, st);
  return check_launch("ria_attn_prefill");
}
