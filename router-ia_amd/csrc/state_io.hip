// Save and restore the attention state of one sequence: its DeltaNet states,
// conv ring and KV pages, as one contiguous device payload.
//
// The reference keeps a sequence's state as per-layer tensors inside its
// AttentionState (v2/src/router_ia/qwen36_attention_cache.py:27-92) and has no
// way to store or reload it.  Here a sequence row of the batched pools is
// copied out into a snapshot that can be restored into any row with enough
// KV pages, of the same engine or another one, after which decoding continues
// exactly as it would have in the original row.
//
// Payload (every section starts on a 256-byte boundary):
//   DeltaNet states  f32  [L_lin, Hv, 128, 128]
//   conv rings       bf16 [L_lin, 4, conv_dim]          (token t in slot t mod 4)
//   K tiles          kv   [L_full, pages, Hkv, 16 x 256] (the cache's tile order)
//   V tiles          kv   [L_full, pages, Hkv, 256 x 16]
// with pages = ceil(tokens / 16) in the row's logical page order.  KV keeps
// the cache's tile layout, so both directions are streaming copies of whole
// 8 KiB tiles; token slots past `tokens` in the last page are saved as zeros,
// so a snapshot's bytes depend only on the sequence's state.
#include <algorithm>

#include "ria_common.h"

namespace ria {

constexpr int kTileBytes = kPageTokens * kAttnHeadDim * 2;  // one (page, KV head) tile of 16-bit elements
constexpr int kTileChunks = kTileBytes / 16;                // 16-byte units per tile

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

struct SeqLayout {
  int64_t lin_block, conv_block;  // bytes per layer
  int64_t off_lin, off_conv, off_k, off_v, total;
  int pages;
};

static SeqLayout seq_layout(int num_linear_layers, int num_v_heads, int conv_dim, int num_full_layers,
                            int num_kv_heads, int tokens) {
  SeqLayout l{};
  l.pages = (tokens + kPageTokens - 1) / kPageTokens;
  l.lin_block = (int64_t)num_v_heads * kGdnHeadDim * kGdnHeadDim * 4;
  l.conv_block = (int64_t)kConvRing * conv_dim * 2;
  const int64_t kv = (int64_t)num_full_layers * l.pages * num_kv_heads * kTileBytes;
  l.off_lin = 0;
  l.off_conv = align256(l.off_lin + num_linear_layers * l.lin_block);
  l.off_k = align256(l.off_conv + num_linear_layers * l.conv_block);
  l.off_v = align256(l.off_k + kv);
  l.total = align256(l.off_v + kv);
  return l;
}

// Copy `layers` blocks of `block` bytes (a multiple of 16): block l goes from
// src + l * src_stride to dst + l * dst_stride.  Grid: (workgroups per block,
// layers); each thread moves 16-byte units with streaming loads and stores.
__global__ __launch_bounds__(256) void dense_copy_kernel(const char* __restrict__ src, int64_t src_stride,
                                                         char* __restrict__ dst, int64_t dst_stride,
                                                         int64_t block) {
  const int64_t units = block / 16;
  const u32x4* s = reinterpret_cast<const u32x4*>(src + blockIdx.y * src_stride);
  u32x4* d = reinterpret_cast<u32x4*>(dst + blockIdx.y * dst_stride);
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256)
    __builtin_nontemporal_store(ld_stream(s + u), d + u);
}

// One workgroup per (page j of the row, KV head, layer x {K, V}).  SAVE
// copies the cache tile of physical page page_table[j] to the payload (slots
// past `tokens` as zeros); restore copies it back.  Pages outside the pool
// save as zeros and are skipped on restore, so no access leaves the pool.
template <bool SAVE>
__global__ __launch_bounds__(256) void tile_copy_kernel(uint16_t* k_cache, uint16_t* v_cache, int num_pages,
                                                        int num_kv_heads, int64_t layer_elems,
                                                        const int32_t* __restrict__ pt_row, int pages, int tokens,
                                                        char* payload_k, char* payload_v) {
  const int j = blockIdx.x;
  const int kvh = blockIdx.y;
  const int layer = blockIdx.z >> 1;
  const bool is_v = blockIdx.z & 1;
  const int phys = pt_row[j];
  const bool ok = phys >= 0 && phys < num_pages;
  const int64_t page = ok ? phys : 0;
  uint16_t* cache = (is_v ? v_cache : k_cache) + layer * layer_elems + (page * num_kv_heads + kvh) * (kTileBytes / 2);
  u32x4* tile = reinterpret_cast<u32x4*>(cache);
  u32x4* blob = reinterpret_cast<u32x4*>((is_v ? payload_v : payload_k) +
                                         (((int64_t)layer * pages + j) * num_kv_heads + kvh) * kTileBytes);
  const int valid = min(kPageTokens, tokens - j * kPageTokens);  // >= 1 for every page of the row
  for (int c = threadIdx.x; c < kTileChunks; c += 256) {
    if constexpr (SAVE) {
      u32x4 x = ok ? ld_stream(tile + c) : u32x4{0u, 0u, 0u, 0u};
      if (valid < kPageTokens) {
        if (!is_v) {
          // K tile [8][4][16 tokens][8 dims]: chunk c holds 8 dims of token c % 16
          if (c % kPageTokens >= valid) x = u32x4{0u, 0u, 0u, 0u};
        } else {
          // V tile [256 dims][16 tokens]: chunk c holds tokens 8 (c % 2) .. + 7 of one dim
          const int t0 = 8 * (c & 1);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t lo = t0 + 2 * w < valid ? 0xffffu : 0u;
            const uint32_t hi = t0 + 2 * w + 1 < valid ? 0xffff0000u : 0u;
            x[w] &= lo | hi;
          }
        }
      }
      __builtin_nontemporal_store(x, blob + c);
    } else {
      if (ok) __builtin_nontemporal_store(ld_stream(blob + c), tile + c);
    }
  }
}

}  // namespace ria

using namespace ria;

extern "C" int64_t ria_seq_state_bytes(int num_linear_layers, int num_v_heads, int conv_dim, int num_full_layers,
                                       int num_kv_heads, int tokens) {
  if (num_linear_layers < 0 || num_v_heads <= 0 || conv_dim <= 0 || num_full_layers < 0 || num_kv_heads <= 0 ||
      tokens < 0)
    return 0;
  return seq_layout(num_linear_layers, num_v_heads, conv_dim, num_full_layers, num_kv_heads, tokens).total;
}

static int seq_state_io(bool save, int row, int pool_rows, int num_linear_layers, int num_v_heads, float* states,
                        void* conv_rings, int conv_dim, int num_full_layers, int num_kv_heads, int num_pages,
                        void* k_cache, void* v_cache, const int32_t* page_table, int64_t page_table_stride,
                        int tokens, void* payload, int64_t payload_bytes, void* stream) {
  const char* who = save ? "ria_seq_state_save" : "ria_seq_state_restore";
  if (pool_rows <= 0 || row < 0 || row >= pool_rows) return set_error(RIA_ERR_INVALID, "%s: row out of the pool", who);
  if (num_linear_layers < 0 || num_full_layers < 0 || num_v_heads <= 0 || num_kv_heads <= 0 || conv_dim <= 0 ||
      conv_dim % 8 || tokens < 0 || num_pages < 0)
    return set_error(RIA_ERR_INVALID, "%s: bad sizes", who);
  const SeqLayout l = seq_layout(num_linear_layers, num_v_heads, conv_dim, num_full_layers, num_kv_heads, tokens);
  if (!payload || payload_bytes < l.total)
    return set_error(RIA_ERR_WORKSPACE, "%s: payload %lld bytes < required %lld", who, (long long)payload_bytes,
                     (long long)l.total);
  if (num_linear_layers > 0 && (!states || !conv_rings)) return set_error(RIA_ERR_INVALID, "%s: null state pool", who);
  if (num_full_layers > 0 && l.pages > 0 && (!k_cache || !v_cache || !page_table))
    return set_error(RIA_ERR_INVALID, "%s: null KV pool", who);
  if (l.pages > page_table_stride)
    return set_error(RIA_ERR_INVALID, "%s: %d tokens exceed the row's %lld pages", who, tokens,
                     (long long)page_table_stride);
  if ((reinterpret_cast<uintptr_t>(payload) | reinterpret_cast<uintptr_t>(states) |
       reinterpret_cast<uintptr_t>(conv_rings) | reinterpret_cast<uintptr_t>(k_cache) |
       reinterpret_cast<uintptr_t>(v_cache)) % 16)
    return set_error(RIA_ERR_INVALID, "%s: pools and payload must be 16-byte aligned", who);
  if (num_full_layers > 65535 / 2 || num_kv_heads > 65535 || num_linear_layers > 65535)
    return set_error(RIA_ERR_INVALID, "%s: too many layers or heads", who);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* blob = static_cast<char*>(payload);
  if (num_linear_layers > 0) {
    // pools are [L, pool_rows, block]; the payload packs [L, block]
    char* s_pool = reinterpret_cast<char*>(states) + (int64_t)row * l.lin_block;
    char* c_pool = static_cast<char*>(conv_rings) + (int64_t)row * l.conv_block;
    const int64_t s_stride = (int64_t)pool_rows * l.lin_block, c_stride = (int64_t)pool_rows * l.conv_block;
    const dim3 sg(static_cast<unsigned>(std::min<int64_t>(64, (l.lin_block / 16 + 255) / 256)), num_linear_layers);
    const dim3 cg(static_cast<unsigned>(std::min<int64_t>(64, (l.conv_block / 16 + 255) / 256)), num_linear_layers);
    if (save) {
      hipLaunchKernelGGL(dense_copy_kernel, sg, dim3(256), 0, st, s_pool, s_stride, blob + l.off_lin, l.lin_block,
                         l.lin_block);
      hipLaunchKernelGGL(dense_copy_kernel, cg, dim3(256), 0, st, c_pool, c_stride, blob + l.off_conv, l.conv_block,
                         l.conv_block);
    } else {
      hipLaunchKernelGGL(dense_copy_kernel, sg, dim3(256), 0, st, blob + l.off_lin, l.lin_block, s_pool, s_stride,
                         l.lin_block);
      hipLaunchKernelGGL(dense_copy_kernel, cg, dim3(256), 0, st, blob + l.off_conv, l.conv_block, c_pool, c_stride,
                         l.conv_block);
    }
  }
  if (num_full_layers > 0 && l.pages > 0) {
    const int64_t layer_elems = (int64_t)num_pages * num_kv_heads * (kTileBytes / 2);
    const dim3 grid(l.pages, num_kv_heads, 2 * num_full_layers);
    const int32_t* pt_row = page_table + (int64_t)row * page_table_stride;
    if (save)
      hipLaunchKernelGGL((tile_copy_kernel<true>), grid, dim3(256), 0, st, static_cast<uint16_t*>(k_cache),
                         static_cast<uint16_t*>(v_cache), num_pages, num_kv_heads, layer_elems, pt_row, l.pages,
                         tokens, blob + l.off_k, blob + l.off_v);
    else
      hipLaunchKernelGGL((tile_copy_kernel<false>), grid, dim3(256), 0, st, static_cast<uint16_t*>(k_cache),
                         static_cast<uint16_t*>(v_cache), num_pages, num_kv_heads, layer_elems, pt_row, l.pages,
                         tokens, blob + l.off_k, blob + l.off_v);
  }
  return check_launch(who);
}

extern "C" int ria_seq_state_save(int row, int pool_rows, int num_linear_layers, int num_v_heads,
                                  const float* linear_states, const void* conv_rings, int conv_dim,
                                  int num_full_layers, int num_kv_heads, int num_pages, const void* k_cache,
                                  const void* v_cache, const int32_t* page_table, int64_t page_table_stride,
                                  int tokens, void* payload, int64_t payload_bytes, void* stream) {
  return seq_state_io(true, row, pool_rows, num_linear_layers, num_v_heads, const_cast<float*>(linear_states),
                      const_cast<void*>(conv_rings), conv_dim, num_full_layers, num_kv_heads, num_pages,
                      const_cast<void*>(k_cache), const_cast<void*>(v_cache), page_table, page_table_stride, tokens,
                      payload, payload_bytes, stream);
}

extern "C" int ria_seq_state_restore(int row, int pool_rows, int num_linear_layers, int num_v_heads,
                                     float* linear_states, void* conv_rings, int conv_dim, int num_full_layers,
                                     int num_kv_heads, int num_pages, void* k_cache, void* v_cache,
                                     const int32_t* page_table, int64_t page_table_stride, int tokens,
                                     const void* payload, int64_t payload_bytes, void* stream) {
  return seq_state_io(false, row, pool_rows, num_linear_layers, num_v_heads, linear_states, conv_rings, conv_dim,
                      num_full_layers, num_kv_heads, num_pages, k_cache, v_cache, page_table, page_table_stride,
                      tokens, const_cast<void*>(payload), payload_bytes, stream);
}
