/*
 * ria_hybrid_attn.h - C ABI of the MI355X (gfx950) hybrid-attention hot path.
 *
 * The library replaces the per-token arithmetic of router-ia's stateful
 * attention cache (v2/src/router_ia/qwen36_attention_cache.py) for B
 * sequences at once: the Gated DeltaNet conv + delta-rule recurrence, the
 * partial-RoPE KV append and the sigmoid-gated GQA decode attention, plus
 * chunked prefill forms of both.  The reference has no FFI for this path; the
 * ABI style (opaque status ints, a last-error string, library path taken
 * from an environment variable on the Python side) follows its native
 * memory pool, native_memory/router_memory.h:11-94.
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are device pointers on the current HIP device.
 *   - `stream` is a hipStream_t (NULL = default stream).  Calls are
 *     asynchronous, never synchronise and never allocate.
 *   - Return RIA_OK (0) on success, otherwise a RIA_ERR_* code; the message
 *     is available from ria_last_error() on the calling thread.
 *   - Activation dtype codes: RIA_DT_BF16, RIA_DT_F16, RIA_DT_F32.
 *   - `seq_slot` maps batch row b to a row of the state / page-table pools;
 *     NULL means row b.  Per-row position arrays may be NULL, in which case
 *     the accompanying *_scalar value is used for every row.
 *   - Sizes are fixed by the model family: DeltaNet head dim 128 (dk == dv),
 *     conv kernel 4, full-attention head dim 256, KV pages of 16 tokens.
 *   - Norm weights are f32 device arrays (convert a bf16 checkpoint weight
 *     once; the reference widens it to fp32 before use).  A NULL norm weight
 *     on a fused entry point means its input arrives already normalised.
 *     Fused norms use the model's eps, 1e-6.
 *
 * Memory layouts
 *   DeltaNet recurrent state  f32  [pool, Hv, 128 (dk, i), 128 (dv, j)]
 *                              (the reference layout, :256-265)
 *   DeltaNet conv ring        bf16 [pool, 4 (slot), conv_dim]; the input of
 *                              step n lives in slot n mod 4.  The reference
 *                              keeps the same four inputs as a shifting
 *                              window [1, conv_dim, 4] (:207-209), which
 *                              ria_gdn_decode_ex / ria_conv1d_window_step
 *                              also take (RIA_CONV_WINDOW).
 *   conv weight               bf16 [conv_dim, 4] (== [conv_dim, 1, 4])
 *   K cache (one layer)       kv_dtype [num_pages, Hkv, 8, 4, 16 (token), 8]: the
 *                              (page, head) tile in MFMA operand order; key
 *                              element (token t, dim d) sits at
 *                              [.., (d % 64) / 8, d / 64, t, d % 8]
 *   V cache (one layer)       kv_dtype [num_pages, Hkv, 256 (dim), 16 (token)]
 *                              kv_dtype is RIA_DT_BF16 or RIA_DT_F16: bf16
 *                              for bf16 activations, fp16 when the
 *                              projections run in fp16 (fp16 keeps the
 *                              reference's fp16 values exactly).
 *   page table                i32  [pool, page_table_stride]; logical token
 *                              t of a sequence lives in physical slot
 *                              page_table[row][t / 16] * 16 + t % 16.  The
 *                              stride is the row's page capacity: kernels
 *                              never read entries at or past it, and treat
 *                              entries outside [0, num_pages) as absent.
 */
#ifndef RIA_HYBRID_ATTN_H
#define RIA_HYBRID_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RIA_ABI_VERSION 5

enum ria_dtype { RIA_DT_BF16 = 0, RIA_DT_F16 = 1, RIA_DT_F32 = 2 };

enum ria_status {
  RIA_OK = 0,
  RIA_ERR_INVALID = 1,   /* bad argument (shape, dtype, null pointer) */
  RIA_ERR_LAUNCH = 2,    /* HIP launch or runtime error */
  RIA_ERR_WORKSPACE = 3  /* caller workspace too small */
};

enum ria_prefill_phase { RIA_PREFILL_APPEND = 1, RIA_PREFILL_ATTEND = 2, RIA_PREFILL_BOTH = 3 };

enum ria_gate_mode {
  /* gate_a holds g (log decay), gate_b holds beta; A_log/dt_bias unused. */
  RIA_GATE_PRECOMPUTED = 0,
  /* gate_a = a_raw, gate_b = b_raw; beta = sigmoid(b),
   * g = -exp(A_log) * softplus(a + dt_bias)   (qwen36_attention_cache.py:242-250) */
  RIA_GATE_RAW = 1
};

/* ABI version of the loaded library (RIA_ABI_VERSION). */
int ria_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ria_last_error(void);

/*
 * The device a measurement ran on (from hipGetDeviceProperties), recorded
 * beside the figures that are quoted against its published peaks.  No
 * counterpart in the reference (it has no device path).
 */
typedef struct ria_device_record {
  char name[256];
  char arch[256];          /* gcnArchName, e.g. gfx950:sramecc+:xnack- */
  int compute_units;
  int clock_khz;           /* peak shader clock */
  int memory_clock_khz;    /* peak memory clock */
  int memory_bus_bits;
  int64_t memory_bytes;
  int l2_bytes;
  int lds_bytes_per_cu;
  int wavefront_size;
} ria_device_record;

int ria_device_info(int device, ria_device_record* out);

/*
 * Gated DeltaNet decode: one token for each of `batch` sequences, one layer.
 * Replaces qwen36_attention_cache.py:235-266 (_causal_conv1d_step, q/k/v
 * split with the 2:1 QK->V head sharing, gating, l2norm, delta-rule update of
 * the recurrent state and read-out from the updated state).
 *
 * mixed_qkv  [batch, conv_dim] of x_dtype, row stride x_row_stride elements.
 *            fuse_conv=1: projection output before the conv (the conv, SiLU,
 *            conv-ring update run here, in bf16 like the reference's bf16
 *            conv weight); fuse_conv=0: already-convolved q|k|v.
 * conv_weight, conv_ring      used only when fuse_conv=1.
 * conv_pos   [batch] step index n of this token (ring slot n mod 4), or NULL
 *            to use conv_pos_scalar for every row.
 * state      recurrent state pool, updated in place.
 * gate_a/b   [batch, Hv] f32 with row stride gate_row_stride (see gate_mode).
 * out        [batch, Hv, 128] of out_dtype: read-out o = S_new^T q, or with
 *            z given the gated RMSNorm of it (qwen36_attention_cache.py:268-271,
 *            qwen36_gated_norm_probe.py:19-36):
 *            out = norm_weight * o / sqrt(mean(o^2) + 1e-6) * SiLU(z) per head.
 * z          NULL, or the gate [batch, Hv, 128] of z_dtype with row stride
 *            z_row_stride (even, z 4-byte aligned); norm_weight [128] f32.
 * conv_dim = 2 * num_k_heads * 128 + num_v_heads * 128.
 */
int ria_gdn_decode(int batch, int num_k_heads, int num_v_heads,
                   const void* mixed_qkv, int x_dtype, int64_t x_row_stride, int fuse_conv,
                   const void* conv_weight, void* conv_ring,
                   const int32_t* conv_pos, int32_t conv_pos_scalar,
                   float* state, const int32_t* seq_slot,
                   const float* gate_a, const float* gate_b, int64_t gate_row_stride,
                   int gate_mode, const float* A_log, const float* dt_bias,
                   void* out, int out_dtype,
                   const void* z, int z_dtype, int64_t z_row_stride, const float* norm_weight,
                   void* stream);

/*
 * Depthwise causal conv1d step alone (kernel 4, SiLU), for `batch` rows of
 * `channels` channels.  Replaces qwen36_attention_cache.py:176-221
 * (_causal_conv1d_step): out = SiLU(sum_j w[c,j] * hist[c, j]) over the three
 * previous inputs and the current one, computed in bf16 and cast to
 * out_dtype; the current input is written to ring slot conv_pos mod 4.
 */
int ria_conv1d_step(int batch, int channels,
                    const void* x, int x_dtype, int64_t x_row_stride,
                    const void* conv_weight, void* conv_ring, const int32_t* seq_slot,
                    const int32_t* conv_pos, int32_t conv_pos_scalar,
                    void* out, int out_dtype, void* stream);

/*
 * ria_conv1d_step on the reference's own conv state: window_in [batch,
 * channels, 4] bf16 holds each row's last four inputs, oldest first
 * (qwen36_attention_cache.py:202-209); window_out receives the shifted window
 * (inputs 2..4 and the current one), which may be window_in itself (in
 * place).  Replaces _causal_conv1d_step (:176-221) with its state tensor
 * layout unchanged.  Windows and conv_weight 8-byte aligned.
 */
int ria_conv1d_window_step(int batch, int channels,
                           const void* x, int x_dtype, int64_t x_row_stride,
                           const void* conv_weight, const void* window_in, void* window_out,
                           void* out, int out_dtype, void* stream);

/* Where the conv state of a ria_gdn_decode_ex call lives. */
enum ria_conv_layout {
  RIA_CONV_NONE = 0,   /* no conv: x already holds the convolved q|k|v */
  RIA_CONV_RING = 1,   /* conv_ring / conv_pos, as in ria_gdn_decode with fuse_conv = 1 */
  RIA_CONV_WINDOW = 2  /* the reference's window [pool, conv_dim, 4], oldest first (:202-209) */
};

/* How q and k arrive in a ria_gdn_decode_ex call. */
enum ria_qk_mode {
  /* x holds the raw q|k of num_k_heads QK heads; l2norm and q * 128^-0.5 run
   * here, and QK head h / (Hv / Hk) serves V head h (:237-254). */
  RIA_QK_RAW = 0,
  /* x (RIA_CONV_NONE only) holds per V head the caller's l2-normalised q
   * (already scaled by 128^-0.5) and k: [Hv*128 q | Hv*128 k | Hv*128 v]
   * (the reference's q, k after :252-254). */
  RIA_QK_NORMALIZED = 1
};

/*
 * One ria_gdn_decode_ex call.  Fields not named here are as in
 * ria_gdn_decode.
 *   conv_layout      see ria_conv_layout.  RIA_CONV_WINDOW reads each row's
 *                    window from conv_window_in and writes the shifted window
 *                    to conv_window_out, which must not overlap it (other
 *                    workgroups read the q/k channels a workgroup shifts).
 *   state_in/out     f32 [pool, Hv, 128, 128]: S is read from state_in and
 *                    S_new written to state_out, the same buffer (in place)
 *                    or a disjoint one (the reference stores a new state
 *                    tensor each step, :261-265).
 *   qk_mode          see ria_qk_mode.
 *   pool_rows        with seq_slot: the rows of the state pools (and of the
 *                    conv window pools) that the slots index; required when
 *                    state_out is not state_in or the layout is
 *                    RIA_CONV_WINDOW, so that the pools can be checked for
 *                    overlap.  Without seq_slot the pools are `batch` rows and
 *                    this field is ignored.  Every slot must be below it.
 */
typedef struct ria_gdn_decode_desc {
  int batch;
  int num_k_heads;
  int num_v_heads;
  const void* x;
  int x_dtype;
  int64_t x_row_stride;
  int conv_layout;
  const void* conv_weight;
  void* conv_ring;
  const int32_t* conv_pos;
  int32_t conv_pos_scalar;
  const void* conv_window_in;
  void* conv_window_out;
  const float* state_in;
  float* state_out;
  const int32_t* seq_slot;
  const float* gate_a;
  const float* gate_b;
  int64_t gate_row_stride;
  int gate_mode;
  const float* A_log;
  const float* dt_bias;
  int qk_mode;
  void* out;
  int out_dtype;
  const void* z;
  int z_dtype;
  int64_t z_row_stride;
  const float* norm_weight;
  int64_t pool_rows;
} ria_gdn_decode_desc;

/*
 * ria_gdn_decode with the state layouts of the reference's AttentionState:
 * a new state tensor per step and the conv window (the drop-in
 * qwen36_attention_cache keeps its dicts as the reference's tensors, :27-32,
 * :202-209, :256-265), and q/k normalised by the caller when the module's
 * _l2norm is replaced (:252-254).  Replaces qwen36_attention_cache.py:235-271.
 */
int ria_gdn_decode_ex(const ria_gdn_decode_desc* desc, void* stream);

/*
 * Row-wise l2 normalisation x * rsqrt(sum(x^2) + eps) in fp32 over rows of
 * `dim` elements.  Replaces qwen36_attention_cache.py:169-173 (_l2norm).
 */
int ria_l2norm(int64_t rows, int dim, const void* x, int x_dtype, float eps,
               float* out, void* stream);

/*
 * RMSNorm with the (1 + w) affine of the model's input, q and k norms:
 * y = x / sqrt(mean(x^2) + eps) * (1 + weight) in fp32, cast back to x_dtype,
 * stored as out_dtype.  Rows are (token, head) pairs: head h of token t holds
 * `dim` elements at x + t * x_token_stride + h * dim.  Replaces
 * qwen36_op_probe.py:55-67 (`rmsnorm`, called at qwen36_attention_cache.py:227
 * and :302-305).  out may alias x when both have one dtype and one stride.
 */
int ria_rmsnorm(int64_t tokens, int heads, int dim,
                const void* x, int x_dtype, int64_t x_token_stride,
                const float* weight, float eps,
                void* out, int out_dtype, int64_t out_token_stride, void* stream);

/*
 * Gated RMSNorm: n = x / sqrt(mean(x^2) + eps) cast to x_dtype, then
 * y = weight * n * SiLU(z) in fp32, cast to x_dtype, stored as out_dtype;
 * rows as in ria_rmsnorm.  Replaces qwen36_gated_norm_probe.py:19-36
 * (`gated_rmsnorm`, called at qwen36_attention_cache.py:268-271).
 */
int ria_gated_rmsnorm(int64_t tokens, int heads, int dim,
                      const void* x, int x_dtype, int64_t x_token_stride,
                      const void* z, int z_dtype, int64_t z_token_stride,
                      const float* weight, float eps,
                      void* out, int out_dtype, int64_t out_token_stride, void* stream);

/*
 * RoPE tables for one position: cos/sin of position * inv_freq duplicated
 * over both halves, `rope_dim` fp32 values each.  inv_freq holds rope_dim/2
 * fp32 frequencies.  Replaces qwen36_attention_cache.py:137-146 (_rope).
 */
int ria_rope_table(int32_t position, const float* inv_freq, int rope_dim,
                   float* cos_out, float* sin_out, void* stream);

/*
 * Partial half-split (NeoX) rotary embedding on rows of `head_dim` fp32
 * values: dims [0, rope_dim) rotate, the rest pass through.  One position
 * for all rows.  Replaces qwen36_attention_cache.py:149-162 (_apply_rope).
 */
int ria_rope_apply(int64_t rows, int head_dim, int rope_dim, const float* x,
                   float* out, const float* inv_freq, int32_t position, void* stream);

/*
 * Append one token per sequence into a layer's paged bf16 KV cache, with
 * partial RoPE applied to k.  Replaces qwen36_attention_cache.py:306-308
 * (_apply_rope on k + _append_full_kv's torch.cat).  Capacity limits are host
 * policy and are checked by the caller before this call.
 *
 * k, v       [batch, Hkv, 256] of k_dtype / v_dtype (row stride in elements).
 * positions  RoPE position of the token (tokens_seen), per row or scalar.
 * slots      logical index of the token in its sequence (tokens resident
 *            before the append), per row or scalar.
 * k_norm_weight  NULL, or the k_norm weight [256] f32: k is RMSNorm'd with
 *            (1 + w) and cast back to k_dtype before RoPE (:303-305).
 */
int ria_kv_append(int batch, int num_kv_heads,
                  const void* k, int k_dtype, int64_t k_row_stride,
                  const void* v, int v_dtype, int64_t v_row_stride,
                  void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                  const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                  const int32_t* positions, int32_t position_scalar,
                  const int32_t* slots, int32_t slot_scalar,
                  const float* inv_freq, int rope_dim, const float* k_norm_weight, void* stream);

/*
 * ria_kv_append that also returns each row's key as the reference stores it:
 * k after k_norm and RoPE in fp32, before its rounding to the page dtype, in
 * k_rot_out [batch, Hkv, 256] fp32 (the fp32 k_token the reference appends
 * to full_keys, qwen36_attention_cache.py:303-307, 365-372).  The drop-in's
 * dicts read their keys back from it exactly; the pages are those of
 * ria_kv_append, bit for bit.
 */
int ria_kv_append_out(int batch, int num_kv_heads,
                      const void* k, int k_dtype, int64_t k_row_stride,
                      const void* v, int v_dtype, int64_t v_row_stride,
                      void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                      const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                      const int32_t* positions, int32_t position_scalar,
                      const int32_t* slots, int32_t slot_scalar,
                      const float* inv_freq, int rope_dim, const float* k_norm_weight,
                      float* k_rot_out, void* stream);

/*
 * Append `length` consecutive tokens of ONE sequence (a prompt) into its
 * pages: token i goes to logical slot start_pos + i with RoPE position
 * start_pos + i.  Equal to `length` ria_kv_append calls, bit for bit, i.e.
 * the reference's per-token prefill of :306-308 and :365-372
 * (qwen36_chat_batch.py:255-258 drives one decode step per prompt token).
 * One workgroup per (page, KV head); slots of the first and last pages
 * outside the prompt keep their contents.
 *
 * k, v            [length, Hkv, 256] of k_dtype / v_dtype.
 * k_cache/v_cache 16-byte aligned (whole pages are written with 16-byte
 *                 stores).
 * page_table_row  this sequence's page-table row, page_capacity entries;
 *                 start_pos + length must fit in page_capacity * 16.
 * k_norm_weight   as in ria_kv_append.
 */
int ria_kv_append_seq(int length, int num_kv_heads,
                      const void* k, int k_dtype, int64_t k_row_stride,
                      const void* v, int v_dtype, int64_t v_row_stride,
                      void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                      const int32_t* page_table_row, int64_t page_capacity,
                      int32_t start_pos, const float* inv_freq, int rope_dim,
                      const float* k_norm_weight, void* stream);

/*
 * Causal GQA attention prefill of `length` prompt tokens of one sequence,
 * one layer: appends the prompt's k (RoPE) and v to the pages exactly as
 * ria_kv_append_seq, then token i (position start_pos + i) attends to keys
 * 0 .. start_pos + i, and out = softmax(q_rot K^T * scale) V * sigmoid(gate).
 * Equal to `length` ria_kv_append + ria_attn_decode steps, the reference's
 * token-by-token prefill of qwen36_attention_cache.py:306-317.
 *
 * q, gate   [length, Hq, 256] (row strides in elements); k, v [length, Hkv, 256].
 *           q, k, v, gate and out share act_dtype.
 * out       [length, Hq, 256] of act_dtype, contiguous.
 * Hq / Hkv <= 8; rope_dim is 0 or 64.  q, gate and out 16-byte aligned, row
 * strides multiples of 8 elements.
 * q_norm_weight, k_norm_weight  NULL, or the q_norm / k_norm weights [256]
 *           f32 (16-byte aligned): q and k are RMSNorm'd with (1 + w) and cast
 *           back to act_dtype before RoPE (:302-305).
 */
int ria_attn_prefill(int length, int num_q_heads, int num_kv_heads,
                     const void* q, int64_t q_row_stride,
                     const void* k, int64_t k_row_stride,
                     const void* v, int64_t v_row_stride,
                     const void* gate, int64_t gate_row_stride, int act_dtype,
                     void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                     const int32_t* page_table_row, int64_t page_capacity, int32_t start_pos,
                     const float* inv_freq, int rope_dim,
                     const float* q_norm_weight, const float* k_norm_weight, float scale,
                     void* out, void* stream);

/*
 * ria_attn_prefill split in its two launches: RIA_PREFILL_APPEND writes the
 * prompt's k/v into the pages, RIA_PREFILL_ATTEND computes the attention over
 * pages already holding them, RIA_PREFILL_BOTH does both (== ria_attn_prefill).
 * Lets a caller time or overlap the phases; the arguments are those of
 * ria_attn_prefill (k, v unused by RIA_PREFILL_ATTEND, q, gate, out unused by
 * RIA_PREFILL_APPEND, but all are validated).
 * Also requires q, gate and out 16-byte aligned with row strides that are
 * multiples of 8 elements (ria_attn_prefill has the same requirement).
 */
int ria_attn_prefill_phase(int length, int num_q_heads, int num_kv_heads,
                           const void* q, int64_t q_row_stride,
                           const void* k, int64_t k_row_stride,
                           const void* v, int64_t v_row_stride,
                           const void* gate, int64_t gate_row_stride, int act_dtype,
                           void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                           const int32_t* page_table_row, int64_t page_capacity, int32_t start_pos,
                           const float* inv_freq, int rope_dim,
                           const float* q_norm_weight, const float* k_norm_weight, float scale,
                           void* out, int phase, void* stream);

/*
 * Bytes of the fp16 stage ria_attn_prefill_staged takes for a prompt of
 * `length` tokens: the prompt's k and v as fp16 tiles in page layout.
 */
int64_t ria_attn_prefill_stage_bytes(int length, int num_kv_heads);

/*
 * ria_attn_prefill_phase with an fp16 stage (`stage`, stage_bytes >=
 * ria_attn_prefill_stage_bytes, 16-byte aligned).  For a prompt that starts
 * the sequence (start_pos 0) the append launch also writes the prompt's
 * rotated k and its v as fp16 tiles into the stage (the pages get exactly
 * what ria_attn_prefill_phase writes), and the attention launch reads its
 * keys and values from the stage: fp16 operands carry 11 significant bits
 * alone, so q and the probabilities need no bf16 hi + lo pair and the MFMA
 * work halves, and the keys are nearer the reference's fp32 ones than the
 * bf16 pages.  Both phases take the same stage.  With start_pos > 0 the call
 * is ria_attn_prefill_phase (the resident keys are only in the pages).  No
 * counterpart in the reference beyond :306-317 (its prefill is token by
 * token).
 */
int ria_attn_prefill_staged(int length, int num_q_heads, int num_kv_heads,
                            const void* q, int64_t q_row_stride,
                            const void* k, int64_t k_row_stride,
                            const void* v, int64_t v_row_stride,
                            const void* gate, int64_t gate_row_stride, int act_dtype,
                            void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                            const int32_t* page_table_row, int64_t page_capacity, int32_t start_pos,
                            const float* inv_freq, int rope_dim,
                            const float* q_norm_weight, const float* k_norm_weight, float scale,
                            void* stage, int64_t stage_bytes,
                            void* out, int phase, void* stream);

/*
 * Split size ria_attn_decode would choose for these context lengths (a host
 * array of `batch` tokens-attended counts): long splits, down to one page
 * per wave when the batch holds too few pages to occupy the GPU.  Passing
 * the result as split_tokens lets callers size the workspace once for a
 * batch they know.  split_tokens = 0 applies the same rule to max_ctx for
 * every row.
 */
int ria_attn_decode_split_tokens(int num_kv_heads, const int32_t* ctx_lens_host, int batch);

/*
 * Workspace bytes ria_attn_decode needs for these sizes (split_tokens = 0
 * selects the automatic split size, as in ria_attn_decode).
 */
int64_t ria_attn_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads,
                                        int max_ctx, int split_tokens);

/*
 * Split-K GQA decode attention over a paged bf16 KV cache with partial RoPE
 * on q and a sigmoid output gate.  Replaces qwen36_attention_cache.py:306,
 * 309-317: q is rotated at `positions`, scores = q K^T * scale over the
 * ctx_lens tokens of each sequence (the just-appended token included), fp32
 * softmax, P V, then attn * sigmoid(gate) elementwise per (head, dim).
 * Query head h reads KV head h / (num_q_heads / num_kv_heads); at most 8
 * query heads per KV head; rope_dim is 0 or 64.
 *
 * q, gate    [batch, Hq, 256] of q_dtype / gate_dtype (row stride in elements).
 * ctx_lens   tokens attended per row (or scalar); max_ctx bounds them.
 * split_tokens  tokens per split (multiple of 64) or 0 for automatic.
 * workspace  caller buffer of ria_attn_decode_workspace_bytes() bytes.
 * q_norm_weight  NULL, or the q_norm weight [256] f32: q is RMSNorm'd with
 *            (1 + w) and cast back to q_dtype before RoPE (:302-304).
 * out        [batch, Hq, 256] of out_dtype.
 */
int ria_attn_decode(int batch, int num_q_heads, int num_kv_heads,
                    const void* q, int q_dtype, int64_t q_row_stride,
                    const void* gate, int gate_dtype, int64_t gate_row_stride,
                    const void* k_cache, const void* v_cache, int kv_dtype, int num_pages,
                    const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                    const int32_t* positions, int32_t position_scalar,
                    const int32_t* ctx_lens, int32_t ctx_scalar, int max_ctx,
                    const float* inv_freq, int rope_dim, const float* q_norm_weight,
                    float scale, int split_tokens,
                    void* workspace, int64_t workspace_bytes,
                    void* out, int out_dtype, void* stream);

/*
 * ria_attn_decode in two launches that can be timed apart: RIA_ATTN_SPLITK
 * writes the per-split partials into the workspace, RIA_ATTN_COMBINE merges
 * them and applies the gate (it must follow a SPLITK call with the same
 * arguments on the same stream); RIA_ATTN_BOTH is ria_attn_decode.
 */
enum ria_attn_phase { RIA_ATTN_SPLITK = 1, RIA_ATTN_COMBINE = 2, RIA_ATTN_BOTH = 3 };

int ria_attn_decode_phase(int batch, int num_q_heads, int num_kv_heads,
                          const void* q, int q_dtype, int64_t q_row_stride,
                          const void* gate, int gate_dtype, int64_t gate_row_stride,
                          const void* k_cache, const void* v_cache, int kv_dtype, int num_pages,
                          const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                          const int32_t* positions, int32_t position_scalar,
                          const int32_t* ctx_lens, int32_t ctx_scalar, int max_ctx,
                          const float* inv_freq, int rope_dim, const float* q_norm_weight,
                          float scale, int split_tokens,
                          void* workspace, int64_t workspace_bytes,
                          void* out, int out_dtype, int phase, void* stream);

/*
 * ria_kv_append followed by ria_attn_decode_phase, with no launch of its own:
 * replaces qwen36_attention_cache.py:302-317 (k_norm and RoPE of the new k,
 * _append_full_kv at :327-373, then the decode attention over the grown
 * context).  Each row's new token goes into slot ctx_lens[b] - 1 (its
 * position is positions[b]).  The split-K phase leaves that token out; the
 * combine phase computes it from k and v with the arithmetic of
 * ria_kv_append (the page gets the same bits), writes it into the page and
 * folds its score and value into the row's softmax.  q, gate, k and v share
 * one dtype; k and v are [batch, Hkv, 256]; k_norm_weight as in
 * ria_kv_append.  The page of slot ctx_lens[b] - 1 must be allocated.  Both
 * phases take the same arguments (phase as in ria_attn_decode_phase).
 */
int ria_attn_decode_append(int batch, int num_q_heads, int num_kv_heads,
                           const void* q, int q_dtype, int64_t q_row_stride,
                           const void* gate, int gate_dtype, int64_t gate_row_stride,
                           const void* k, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                           const float* k_norm_weight,
                           void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                           const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                           const int32_t* positions, int32_t position_scalar,
                           const int32_t* ctx_lens, int32_t ctx_scalar, int max_ctx,
                           const float* inv_freq, int rope_dim, const float* q_norm_weight,
                           float scale, int split_tokens,
                           void* workspace, int64_t workspace_bytes,
                           void* out, int out_dtype, int phase, void* stream);

/*
 * ria_attn_decode_append with no workspace argument and no allocation: the
 * split-K partials go into a 16 MiB array the library holds on each GPU it
 * runs on (a file-scope device array, resolved once per device).  No
 * counterpart in the reference: this entry point is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  Arguments are those of
 * ria_attn_decode_append without workspace / workspace_bytes; sizes whose
 * partials (ria_attn_decode_workspace_bytes) exceed 16 MiB return
 * RIA_ERR_WORKSPACE before any launch (the balanced schedule fits up to about
 * 1,500 (sequence, KV head) units).  `phase` must be RIA_ATTN_BOTH (anything
 * else returns RIA_ERR_INVALID): the partials never outlive the call.  Every
 * call on one GPU shares the array: calls that overlap on one GPU (concurrent
 * streams) race.
 */
int ria_attn_decode_append_noalloc(int batch, int num_q_heads, int num_kv_heads,
                                   const void* q, int q_dtype, int64_t q_row_stride,
                                   const void* gate, int gate_dtype, int64_t gate_row_stride,
                                   const void* k, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                   const float* k_norm_weight,
                                   void* k_cache, void* v_cache, int kv_dtype, int num_pages,
                                   const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                                   const int32_t* positions, int32_t position_scalar,
                                   const int32_t* ctx_lens, int32_t ctx_scalar, int max_ctx,
                                   const float* inv_freq, int rope_dim, const float* q_norm_weight,
                                   float scale, int split_tokens,
                                   void* out, int out_dtype, int phase, void* stream);

/*
 * Workspace bytes ria_gdn_prefill needs to process `segment_tokens` tokens
 * per pass (it walks longer prompts in segments of whole 64-token chunks).
 */
int64_t ria_gdn_prefill_workspace_bytes(int num_k_heads, int num_v_heads, int segment_tokens);

/*
 * Chunked (WY form, chunk 64) Gated DeltaNet prefill of `length` tokens of
 * one sequence, one layer.  Equal to `length` calls of ria_gdn_decode with
 * fuse_conv=1, which is the reference's token-by-token prefill
 * (qwen36_chat_batch.py:255-258 -> qwen36_attention_cache.py:176-266); the
 * chunk algebra is the one transformers' torch_chunk_gated_delta_rule
 * evaluates for the reference's HF path (qwen36_linear_attention_hf.py:91-100).
 *
 * mixed_qkv  [length, conv_dim] projection outputs before the conv.
 * conv_ring  bf16 [4, conv_dim] of this sequence; conv_pos = step of token 0.
 * state      f32 [Hv, 128, 128] of this sequence, updated in place.
 * gate_a/b   [length, Hv] f32 per token (gate_mode as in ria_gdn_decode).
 * out        [length, Hv, 128] of out_dtype: the read-out, or with z given
 *            its gated RMSNorm as in ria_gdn_decode.
 * z          NULL, or the gate [length, Hv, 128] of z_dtype (row stride
 *            z_row_stride); norm_weight [128] f32.
 * workspace  >= ria_gdn_prefill_workspace_bytes(.., 64) bytes, 256-byte
 *            aligned; larger workspaces take longer segments.
 */
int ria_gdn_prefill(int length, int num_k_heads, int num_v_heads,
                    const void* mixed_qkv, int x_dtype, int64_t x_row_stride,
                    const void* conv_weight, void* conv_ring, int32_t conv_pos,
                    float* state,
                    const float* gate_a, const float* gate_b, int64_t gate_row_stride,
                    int gate_mode, const float* A_log, const float* dt_bias,
                    void* out, int out_dtype,
                    const void* z, int z_dtype, int64_t z_row_stride, const float* norm_weight,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Copy tokens [start, start + count) of each sequence out of the paged cache
 * into logical order: k_out, v_out [batch, Hkv, count, 256] in the cache's
 * 16-bit element type (bf16 or fp16; the copy is bit-exact).  The
 * inverse of the append's slot mapping; used to materialise the reference's
 * contiguous full_keys / full_values view (qwen36_attention_cache.py:365-372).
 */
int ria_kv_gather(int batch, int num_kv_heads,
                  const void* k_cache, const void* v_cache, int num_pages,
                  const int32_t* page_table, int64_t page_table_stride, const int32_t* seq_slot,
                  int32_t start, int32_t count, void* k_out, void* v_out, void* stream);

/*
 * Projections with FP8 block-scaled weights.  The reference's checkpoint
 * weights are float8_e4m3fn [N, K] with one fp32 `weight_scale_inv` per
 * 128x128 block ([ceil(N/128), ceil(K/128)]); it dequantises them once to
 * fp16(w * s) (qwen36_dequant.py:35-58, qwen36_cached_loop.py:537-542) and
 * runs fp16 F.linear (qwen36_attention_cache.py:232-247, 268-276, 295-301,
 * 318-320).
 *
 * ria_dequant_fp8: out[r][c] = float(w[r][c]) * s[r/128][c/128], rounded once
 * to out_dtype (RIA_DT_F16 gives the reference's fp16 weight).  cols a
 * multiple of 16; weight and out 16-byte aligned.
 *
 * ria_linear_fp8: y = fp16(x) W^T with W = fp16(w * s) dequantised in
 * registers (the weight stays FP8 in memory), fp32 accumulation, the result
 * rounded to fp16 (F.linear's fp16 output) and stored as y_dtype.  x [m, k]
 * of x_dtype (converted to fp16 like `.to(float16)`), y [m, n].  n a multiple
 * of 16, k of 128; x and weight 16-byte aligned, x row stride a multiple of 8.
 * Built for decode-sized m (one weight pass per 128 rows of x); k up to 32768.
 *
 * ria_linear_fp8_group: 1 to 4 such projections of the same x in one launch,
 * each with its own n, weight, scales, y and y dtype.  It replaces
 * the reference's run of F.linear calls on one normed hidden state: DeltaNet
 * in_proj_qkv / in_proj_z / in_proj_a / in_proj_b (qwen36_attention_cache.py:
 * 232-247, 268) and attention q_proj / k_proj / v_proj (:295-301); results
 * equal separate ria_linear_fp8 calls.  With y_add, y += the fp16 result in
 * fp32 (the residual add `x0.float() + F.linear(...).float()` of :281, :324).
 */
typedef struct ria_fp8_proj {
  const void* weight;      /* [n, k] float8_e4m3fn */
  const float* scale_inv;  /* [ceil(n / 128), k / 128] */
  void* y;                 /* [m, n], rows y_row_stride elements apart */
  int64_t y_row_stride;
  int n;
  int y_dtype;             /* RIA_DT_*: the fp16 result stored in this dtype */
  int y_add;               /* nonzero: y (RIA_DT_F32) += the result instead (a residual add) */
} ria_fp8_proj;

int ria_dequant_fp8(int64_t rows, int cols, const void* weight, const float* scale_inv,
                    void* out, int out_dtype, void* stream);

int ria_linear_fp8(int m, int n, int k, const void* x, int x_dtype, int64_t x_row_stride,
                   const void* weight, const float* scale_inv,
                   void* y, int y_dtype, int64_t y_row_stride, void* stream);

int ria_linear_fp8_group(int m, int k, const void* x, int x_dtype, int64_t x_row_stride,
                         int count, const ria_fp8_proj* projs, void* stream);

/*
 * ria_linear_fp8_group_normed: ria_linear_fp8_group on h = the layer's input
 * RMSNorm of the fp32 residual stream x, in the same launch:
 * h = (x * rsqrt(mean(x^2) + eps)) * (1 + norm_weight) in fp32, rounded to
 * h_dtype (RIA_DT_BF16 for a DeltaNet layer, RIA_DT_F16 for attention) and then
 * to fp16 (qwen36_attention_cache.py:227-233, 291-293).  Decode sizes only:
 * m <= 4, k a multiple of 512 up to 4096; norm_weight fp32 [k], 16-byte
 * aligned; x row stride a multiple of 4.
 */
int ria_linear_fp8_group_normed(int m, int k, const float* x, int64_t x_row_stride,
                                const float* norm_weight, float eps, int h_dtype, int count,
                                const ria_fp8_proj* projs, void* stream);

/*
 * Sequence snapshots: one row's DeltaNet states, conv ring and KV pages as a
 * contiguous device payload, to be restored into any row (of this pool or
 * another with the same shapes) that has pages for `tokens` tokens; decoding
 * then continues exactly as in the original row.  The reference keeps this
 * state in AttentionState's per-layer tensors (qwen36_attention_cache.py:27-92)
 * and cannot save or reload it.
 *
 * Payload sections, each starting on a 256-byte boundary:
 *   DeltaNet states f32  [L_lin, Hv, 128, 128]
 *   conv rings      bf16 [L_lin, 4, conv_dim]           (token t in slot t mod 4)
 *   K tiles         kv   [L_full, pages, Hkv, K tile]   (the cache's tile order)
 *   V tiles         kv   [L_full, pages, Hkv, V tile]
 * with pages = ceil(tokens / 16) in logical page order; token slots past
 * `tokens` are saved as zeros.  Pools are the batched layouts: states
 * [L_lin, pool_rows, Hv, 128, 128], conv rings [L_lin, pool_rows, 4, conv_dim],
 * K/V caches [L_full, num_pages, Hkv, tile] with page_table [pool_rows,
 * page_table_stride].  The position (tokens) travels with the payload on the
 * host side.  Pools and payload 16-byte aligned.
 */
int64_t ria_seq_state_bytes(int num_linear_layers, int num_v_heads, int conv_dim, int num_full_layers,
                            int num_kv_heads, int tokens);

int ria_seq_state_save(int row, int pool_rows, int num_linear_layers, int num_v_heads,
                       const float* linear_states, const void* conv_rings, int conv_dim,
                       int num_full_layers, int num_kv_heads, int num_pages,
                       const void* k_cache, const void* v_cache,
                       const int32_t* page_table, int64_t page_table_stride, int tokens,
                       void* payload, int64_t payload_bytes, void* stream);

int ria_seq_state_restore(int row, int pool_rows, int num_linear_layers, int num_v_heads,
                          float* linear_states, void* conv_rings, int conv_dim,
                          int num_full_layers, int num_kv_heads, int num_pages,
                          void* k_cache, void* v_cache,
                          const int32_t* page_table, int64_t page_table_stride, int tokens,
                          const void* payload, int64_t payload_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RIA_HYBRID_ATTN_H */
