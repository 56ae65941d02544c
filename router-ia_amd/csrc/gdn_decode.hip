// Gated DeltaNet decode for gfx950: causal conv step + gating + l2norm +
// delta-rule update + read-out, one token per sequence, fused in one pass
// over the fp32 recurrent state.
//
// Math (v2/src/router_ia/qwen36_attention_cache.py:176-266, per V head h):
//   hist   = the three previous conv inputs and the current one
//   x_c    = SiLU(sum_j w[c,j] hist[c,j])            (bf16, :207-221)
//   q, k   = l2norm(x_q), l2norm(x_k) for QK head h / (Hv/Hk); q *= 128^-0.5
//   beta, decay = sigmoid(b), exp(-exp(A_log) softplus(a + dt_bias))
//   S'     = decay * S
//   r_j    = sum_i S'[i,j] k_i
//   d_j    = (v_j - r_j) beta
//   S_new  = S' + k_i d_j
//   o_j    = sum_i S_new[i,j] q_i = sum_i S'[i,j] q_i + d_j (k . q)
//
// With a gate z the read-out leaves through the gated RMSNorm
// (qwen36_attention_cache.py:268-271, qwen36_gated_norm_probe.py:19-36):
//   out_j  = w_j * o_j / sqrt(mean(o^2) + 1e-6) * SiLU(z_j)
// which needs the whole head's o in one workgroup (COLS = 128).
//
// Work decomposition: one 256-thread workgroup per (sequence, V head, column
// block of COLS state columns).  Columns of S are independent in this
// update, so small batches split a head over several workgroups.  Each
// thread owns RPT rows x 4 adjacent columns of the tile in registers; a
// wavefront covers whole 512-byte rows, so the state is read and written
// exactly once with full-row coalescing.  The two column reductions over i
// (r_j and the S' q part of o_j) share a single shuffle + LDS pass.
#include <algorithm>

#include "ria_common.h"

namespace ria {

struct GdnDecodeArgs {
  const void* x;
  int64_t x_stride;
  const uint16_t* conv_w;  // [conv_dim, 4] bf16
  uint16_t* conv_ring;     // [pool, 4, conv_dim] bf16 (ring layout)
  const int32_t* conv_pos;
  int32_t conv_pos_scalar;
  // window layout (the reference's [1, conv_dim, 4], oldest input first):
  // the window is read from win_in and the shifted one written to win_out
  int conv_window;
  const uint16_t* win_in;  // [pool, conv_dim, 4] bf16
  uint16_t* win_out;
  const float* state_in;  // [pool, Hv, 128, 128]
  float* state_out;       // == state_in for the in-place update
  const int32_t* seq_slot;
  // q and k arrive l2-normalised (q also scaled by 128^-0.5) per V head:
  // x = [Hv*128 q | Hv*128 k | Hv*128 v]; only without the fused conv
  int qk_prenorm;
  const float* gate_a;
  const float* gate_b;
  int64_t gate_stride;
  const float* A_log;
  const float* dt_bias;
  void* out;  // [batch, Hv, 128]
  const void* z;         // gated-norm gate [batch, Hv, 128] (row stride z_stride), or null
  int64_t z_stride;
  int z_dtype;
  const float* norm_w;   // gated-norm weight [128] f32
  int num_k_heads;
  int num_v_heads;
  int conv_dim;
  int ncb;  // column blocks per head
};

// One channel's conv inputs, loaded ahead of the state tiles: the projection
// output and the three previous inputs (bf16 bits) of the conv history.
struct ConvIn {
  uint32_t x;    // the projection output as stored (dtype XT)
  uint32_t h01;  // history inputs n-3 | n-2 << 16
  uint32_t h2;   // history input n-1
  uint2 w;       // the four bf16 taps
};

// Loads channel c's conv inputs for batch row b (pool row `row`, step n).
// Only loads: the conv and the history write come in conv_finish, after the
// caller has issued its state loads (a store to the history here would keep
// the compiler from issuing the state loads until this channel's loads have
// returned, since it cannot tell the two buffers apart).  The layout is a
// template parameter for the same reason: a run-time branch around loads
// makes the compiler wait for them at the join.
template <int XT, int CONV>
__device__ __forceinline__ ConvIn conv_load(const GdnDecodeArgs& a, int b, int row, int n, int c) {
  ConvIn ci{};
  ci.x = load_act_bits<XT>(a.x, (int64_t)b * a.x_stride + c);
  if constexpr (CONV == RIA_CONV_WINDOW) {
    // the window holds inputs n-4 .. n-1, oldest first; the conv reads slots 1..3
    const uint2 hv = *reinterpret_cast<const uint2*>(a.win_in + ((int64_t)row * a.conv_dim + c) * kConvTaps);
    ci.h01 = (hv.x >> 16) | (hv.y << 16);
    ci.h2 = hv.y >> 16;
  } else if constexpr (CONV == RIA_CONV_RING) {
    const uint16_t* ring = a.conv_ring + (int64_t)row * kConvRing * a.conv_dim;
    ci.h01 = uint32_t(ring[((n - 3) & 3) * a.conv_dim + c]) | (uint32_t(ring[((n - 2) & 3) * a.conv_dim + c]) << 16);
    ci.h2 = ring[((n - 1) & 3) * a.conv_dim + c];
  }
  if constexpr (CONV != RIA_CONV_NONE) ci.w = *reinterpret_cast<const uint2*>(a.conv_w + (int64_t)c * kConvTaps);
  return ci;
}

// Post-conv value of channel c, as the reference sees it after
// `_causal_conv1d_step` returns (bf16 conv, cast back to the input dtype,
// :200-221).  With `write` the conv state takes the current input: ring slot
// n mod 4 in the ring layout, or the shifted window (the last three inputs
// and this one, oldest first, :207-209) in the window layout.  FAST_SILU
// takes silu_to_bf16 (the same bits); the fused recurrence kernels keep
// silu_f, whose register plan measured 0.2% faster there.
template <int XT, int CONV, bool FAST_SILU = false>
__device__ __forceinline__ float conv_finish(const GdnDecodeArgs& a, const ConvIn& ci, int row, int n, int c,
                                             bool write) {
  const float xv = act_from_bits<XT>(ci.x);
  if constexpr (CONV == RIA_CONV_NONE) {
    return xv;
  } else {
    const uint16_t xb = f32_to_bf16_bits(xv);  // mixed_qkv.to(conv_dtype)
    if (write) {
      if constexpr (CONV == RIA_CONV_WINDOW)
        *reinterpret_cast<uint2*>(a.win_out + ((int64_t)row * a.conv_dim + c) * kConvTaps) =
            uint2{ci.h01, ci.h2 | (uint32_t(xb) << 16)};
      else
        a.conv_ring[(int64_t)row * kConvRing * a.conv_dim + (n & 3) * a.conv_dim + c] = xb;
    }
    const float w0 = bf16_bits_to_f32(ci.w.x & 0xffffu), w1 = bf16_bits_to_f32(ci.w.x >> 16);
    const float w2 = bf16_bits_to_f32(ci.w.y & 0xffffu), w3 = bf16_bits_to_f32(ci.w.y >> 16);
    float acc = w0 * bf16_bits_to_f32(ci.h01 & 0xffffu);
    acc = fmaf(w1, bf16_bits_to_f32(ci.h01 >> 16), acc);
    acc = fmaf(w2, bf16_bits_to_f32(ci.h2), acc);
    acc = fmaf(w3, bf16_bits_to_f32(xb), acc);
    const float y = round_bf16(FAST_SILU ? silu_to_bf16(round_bf16(acc)) : silu_f(round_bf16(acc)));
    return through_dtype<XT>(y);
  }
}

// EXT: the extended call (ria_gdn_decode_ex) with a separate output state or
// caller-normalised q/k; without it those run-time choices compile away, so
// the batched in-place path keeps its address and select work minimal.
// VG: only the waves holding v columns load their conv inputs (for 128-column
// blocks, whole waves); without it every wave loads one (a repeat past COLS).
// The repeats cost issue slots when several rounds of workgroups stream the
// state, and save a branch when one round runs at once.
template <int COLS, int XT, int OT, int CONV, int GM, bool NORM, bool EXT, bool VG>
__global__ __launch_bounds__(256) void gdn_decode_kernel(GdnDecodeArgs a) {
  constexpr bool FUSE = CONV != RIA_CONV_NONE;
  static_assert(!NORM || COLS == kGdnHeadDim, "the gated norm needs whole heads");
  constexpr int TPR = COLS / 4;         // threads per state row
  constexpr int RG = 256 / TPR;         // row groups in the workgroup
  constexpr int RPT = kGdnHeadDim / RG; // rows held per thread
  constexpr int NW = 4;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int cb = blockIdx.x % a.ncb;
  const int bh = blockIdx.x / a.ncb;
  const int h = bh % a.num_v_heads;
  const int b = bh / a.num_v_heads;
  const int row = a.seq_slot ? a.seq_slot[b] : b;
  const int col0 = cb * COLS;
  const int group = a.num_v_heads / a.num_k_heads;
  // the QK head serving V head h, and the q (and k) section width of x
  const bool prenorm = EXT && a.qk_prenorm;
  const int hk = prenorm ? h : h / group;
  const int kdim = (prenorm ? a.num_v_heads : a.num_k_heads) * kGdnHeadDim;
  const int n = a.conv_pos ? a.conv_pos[b] : a.conv_pos_scalar;

  const int cg = tid % TPR;
  const int rg = tid / TPR;
  const int jl = 4 * cg;  // column within the block

  __shared__ float q_s[kGdnHeadDim];
  __shared__ float k_s[kGdnHeadDim];
  __shared__ float v_s[COLS];
  __shared__ float red_s[NW][2][COLS];
  __shared__ float scal_s[8];
  __shared__ float zg_s[NORM ? COLS : 1];  // gated norm: SiLU input z and weight w per column
  __shared__ float wg_s[NORM ? COLS : 1];

  // Conv / projection inputs first, then the state tiles, so both are in
  // flight together; the conv itself and its history write follow.
  const bool qk_writer = FUSE && (h % group == 0) && cb == 0;
  const int qk_c = tid < 128 ? hk * kGdnHeadDim + tid : kdim + hk * kGdnHeadDim + (tid - 128);
  const int v_c = 2 * kdim + h * kGdnHeadDim + col0 + tid % COLS;
  const ConvIn qk_in = conv_load<XT, CONV>(a, b, row, n, qk_c);
  ConvIn v_in{};
  if (!VG || __builtin_amdgcn_readfirstlane(wave) * 64 < COLS) v_in = conv_load<XT, CONV>(a, b, row, n, v_c);
  // The gated norm's z (as the raw 32-bit word holding it; every thread loads
  // one, threads past COLS a repeat, so no branch makes the wait early) and w.
  ActWord z_word{};
  float w_raw = 0.f;
  if constexpr (NORM) {
    const int tc = tid % COLS;
    z_word = load_act_word(a.z, (int64_t)b * a.z_stride + h * kGdnHeadDim + tc, a.z_dtype);
    w_raw = a.norm_w[tc];
  }

  __builtin_amdgcn_sched_barrier(0);  // the inputs above are issued first: they are needed first
  const int64_t tile = ((int64_t)row * a.num_v_heads + h) * (kGdnHeadDim * kGdnHeadDim);
  const float* S = a.state_in + tile;
  f32x4 s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    s[r] = ld_stream(reinterpret_cast<const f32x4*>(S + (rg + RG * r) * kGdnHeadDim + col0 + jl));
  }
  // every load above is issued before any of their results is used (the
  // scheduler would otherwise start the conv early and wait for its inputs
  // in the middle of the state loads)
  __builtin_amdgcn_sched_barrier(0);
  const float qk_raw = conv_finish<XT, CONV>(a, qk_in, row, n, qk_c, qk_writer);
  const float v_raw = conv_finish<XT, CONV>(a, v_in, row, n, v_c, FUSE && tid < COLS);

  // Gating (every thread computes the same two scalars).
  const float ga = a.gate_a[(int64_t)b * a.gate_stride + h];
  const float gb = a.gate_b[(int64_t)b * a.gate_stride + h];
  float beta, g;
  if constexpr (GM == RIA_GATE_RAW) {
    beta = sigmoid_f(gb);
    g = -expf(a.A_log[h]) * softplus_f(ga + a.dt_bias[h]);
  } else {
    beta = gb;
    g = ga;
  }
  const float decay = expf(g);

  // l2norm of q (waves 0-1) and k (waves 2-3); then q *= 128^-0.5.
  const float ss = wave_sum(mul_rn(qk_raw, qk_raw));
  if (lane == 0) scal_s[wave] = ss;
  if (tid < COLS) v_s[tid] = v_raw;
  if constexpr (NORM) {
    if (tid < COLS) {
      zg_s[tid] = act_from_word(z_word, a.z_dtype);
      wg_s[tid] = w_raw;
    }
  }
  __syncthreads();
  float qk_n = qk_raw;
  if (!prenorm) {
    const float inv = 1.0f / sqrtf((tid < 128 ? scal_s[0] + scal_s[1] : scal_s[2] + scal_s[3]) + 1e-6f);
    qk_n = mul_rn(qk_raw, inv);
    if (tid < 128) qk_n = mul_rn(qk_n, 0.08838834764831845f);
  }
  if (tid < 128) {
    q_s[tid] = qk_n;
  } else {
    k_s[tid - 128] = qk_n;
  }
  __syncthreads();
  if (wave == 0) {
    const float kq = wave_sum(fmaf(k_s[lane], q_s[lane], k_s[lane + 64] * q_s[lane + 64]));
    if (lane == 0) scal_s[4] = kq;
  }

  // Decay, then partial column sums of S' k and S' q over this thread's rows.
  float rj[4] = {0.f, 0.f, 0.f, 0.f};
  float oj[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + RG * r;
    const float ki = k_s[i];
    const float qi = q_s[i];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s[r][c] = mul_rn(s[r][c], decay);
      rj[c] = fmaf(s[r][c], ki, rj[c]);
      oj[c] = fmaf(s[r][c], qi, oj[c]);
    }
  }
#pragma unroll
  for (int off = TPR; off < 64; off <<= 1) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      rj[c] += __shfl_xor(rj[c], off, 64);
      oj[c] += __shfl_xor(oj[c], off, 64);
    }
  }
  if (lane < TPR) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      red_s[wave][0][jl + c] = rj[c];
      red_s[wave][1][jl + c] = oj[c];
    }
  }
  __syncthreads();

  const float kq = scal_s[4];
  float dj[4], oo[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float rt = 0.f, ot = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      rt += red_s[w][0][jl + c];
      ot += red_s[w][1][jl + c];
    }
    dj[c] = mul_rn(v_s[jl + c] - rt, beta);
    oo[c] = fmaf(dj[c], kq, ot);
  }

  // Rank-1 update, written to state_out (in place when it is state_in).
  float* So = EXT ? a.state_out + tile : const_cast<float*>(S);
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + RG * r;
    const float ki = k_s[i];
#pragma unroll
    for (int c = 0; c < 4; ++c) s[r][c] = add_rn(s[r][c], mul_rn(ki, dj[c]));
    st_stream(reinterpret_cast<f32x4*>(So + i * kGdnHeadDim + col0 + jl), s[r]);
  }

  if constexpr (NORM) {
    // rows group 0 is lanes 0..31 of wave 0 and holds the head's 128 outputs
    if (rg == 0) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) ss = add_rn(ss, mul_rn(oo[c], oo[c]));
      const float r = rms_scale(half_wave_sum(ss), kGdnHeadDim);
#pragma unroll
      for (int c = 0; c < 4; ++c) oo[c] = gated_norm_elem<RIA_DT_F32>(oo[c], r, wg_s[jl + c], zg_s[jl + c]);
    }
  }
  if (rg == 0) {
    const int64_t o = ((int64_t)b * a.num_v_heads + h) * kGdnHeadDim + col0 + jl;
#pragma unroll
    for (int c = 0; c < 4; ++c) store_act<OT>(a.out, o + c, oo[c]);
  }
}

// Standalone conv step (one thread per channel).
template <int XT, int OT, int CONV>
__global__ __launch_bounds__(256) void conv1d_step_kernel(GdnDecodeArgs a) {
  const int b = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.conv_dim) return;
  const int row = a.seq_slot ? a.seq_slot[b] : b;
  const int n = a.conv_pos ? a.conv_pos[b] : a.conv_pos_scalar;
  // The reference returns the bf16 conv result cast to the input dtype; the
  // caller-selected output dtype is applied on top of that.
  const float y = conv_finish<XT, CONV, true>(a, conv_load<XT, CONV>(a, b, row, n, c), row, n, c, true);
  store_act<OT>(a.out, (int64_t)b * a.conv_dim + c, y);
}

// Kernel variant flags chosen on the host (see gdn_decode_kernel).
struct GdnVariant {
  bool ext;
  bool vg;
};

template <int COLS, int XT, int OT, int CONV, bool NORM, bool EXT, bool VG>
static void launch_gdn_inst(const GdnDecodeArgs& a, int gate_mode, int blocks, hipStream_t st) {
  if (gate_mode == RIA_GATE_RAW)
    hipLaunchKernelGGL((gdn_decode_kernel<COLS, XT, OT, CONV, RIA_GATE_RAW, NORM, EXT, VG>), dim3(blocks), dim3(256),
                       0, st, a);
  else
    hipLaunchKernelGGL((gdn_decode_kernel<COLS, XT, OT, CONV, RIA_GATE_PRECOMPUTED, NORM, EXT, VG>), dim3(blocks),
                       dim3(256), 0, st, a);
}

template <int COLS, int XT, int OT, int CONV, bool NORM>
static void launch_gdn_gm(const GdnDecodeArgs& a, int gate_mode, GdnVariant v, int blocks, hipStream_t st) {
  if (v.ext)
    launch_gdn_inst<COLS, XT, OT, CONV, NORM, true, false>(a, gate_mode, blocks, st);
  else if (COLS == kGdnHeadDim && v.vg)
    launch_gdn_inst<COLS, XT, OT, CONV, NORM, false, COLS == kGdnHeadDim>(a, gate_mode, blocks, st);
  else
    launch_gdn_inst<COLS, XT, OT, CONV, NORM, false, false>(a, gate_mode, blocks, st);
}

template <int COLS, int XT, int OT, int CONV>
static void launch_gdn_norm(const GdnDecodeArgs& a, int gate_mode, GdnVariant v, int blocks, hipStream_t st) {
  if constexpr (COLS == kGdnHeadDim) {
    if (a.z) {
      launch_gdn_gm<COLS, XT, OT, CONV, true>(a, gate_mode, v, blocks, st);
      return;
    }
  }
  launch_gdn_gm<COLS, XT, OT, CONV, false>(a, gate_mode, v, blocks, st);
}

template <int COLS, int XT, int OT>
static void launch_gdn_fuse(const GdnDecodeArgs& a, int conv, int gate_mode, GdnVariant v, int blocks,
                            hipStream_t st) {
  if (conv == RIA_CONV_RING)
    launch_gdn_norm<COLS, XT, OT, RIA_CONV_RING>(a, gate_mode, v, blocks, st);
  else if (conv == RIA_CONV_WINDOW)
    launch_gdn_norm<COLS, XT, OT, RIA_CONV_WINDOW>(a, gate_mode, v, blocks, st);
  else
    launch_gdn_norm<COLS, XT, OT, RIA_CONV_NONE>(a, gate_mode, v, blocks, st);
}

template <int COLS, int XT>
static void launch_gdn_ot(const GdnDecodeArgs& a, int ot, int conv, int gate_mode, GdnVariant v, int blocks,
                          hipStream_t st) {
  if (ot == RIA_DT_BF16)
    launch_gdn_fuse<COLS, XT, RIA_DT_BF16>(a, conv, gate_mode, v, blocks, st);
  else if (ot == RIA_DT_F16)
    launch_gdn_fuse<COLS, XT, RIA_DT_F16>(a, conv, gate_mode, v, blocks, st);
  else
    launch_gdn_fuse<COLS, XT, RIA_DT_F32>(a, conv, gate_mode, v, blocks, st);
}

template <int COLS>
static void launch_gdn_xt(const GdnDecodeArgs& a, int xt, int ot, int conv, int gate_mode, GdnVariant v,
                          int blocks, hipStream_t st) {
  if (xt == RIA_DT_BF16)
    launch_gdn_ot<COLS, RIA_DT_BF16>(a, ot, conv, gate_mode, v, blocks, st);
  else if (xt == RIA_DT_F16)
    launch_gdn_ot<COLS, RIA_DT_F16>(a, ot, conv, gate_mode, v, blocks, st);
  else
    launch_gdn_ot<COLS, RIA_DT_F32>(a, ot, conv, gate_mode, v, blocks, st);
}

static bool valid_dtype(int dt) { return dt == RIA_DT_BF16 || dt == RIA_DT_F16 || dt == RIA_DT_F32; }

// Validates a decode description and launches it (shared by ria_gdn_decode
// and ria_gdn_decode_ex).
static int gdn_decode_launch(const ria_gdn_decode_desc& d, void* stream, const char* who) {
  if (d.batch < 0) return set_error(RIA_ERR_INVALID, "%s: batch must be >= 0", who);
  if (d.batch == 0) return RIA_OK;
  const int num_k_heads = d.num_k_heads, num_v_heads = d.num_v_heads;
  if (num_k_heads <= 0 || num_v_heads <= 0 || num_v_heads % num_k_heads != 0)
    return set_error(RIA_ERR_INVALID, "%s: num_v_heads (%d) must be a positive multiple of num_k_heads (%d)", who,
                     num_v_heads, num_k_heads);
  if (!valid_dtype(d.x_dtype) || !valid_dtype(d.out_dtype)) return set_error(RIA_ERR_INVALID, "%s: unknown dtype code", who);
  if (!d.x || !d.state_in || !d.state_out || !d.gate_a || !d.gate_b || !d.out)
    return set_error(RIA_ERR_INVALID, "%s: null tensor pointer", who);
  if (d.conv_layout != RIA_CONV_NONE && d.conv_layout != RIA_CONV_RING && d.conv_layout != RIA_CONV_WINDOW)
    return set_error(RIA_ERR_INVALID, "%s: unknown conv_layout %d", who, d.conv_layout);
  const bool fuse = d.conv_layout != RIA_CONV_NONE;
  if (fuse && !d.conv_weight) return set_error(RIA_ERR_INVALID, "%s: the fused conv needs conv_weight", who);
  if (d.conv_layout == RIA_CONV_RING && !d.conv_ring)
    return set_error(RIA_ERR_INVALID, "%s: RIA_CONV_RING needs conv_ring", who);
  if (d.qk_mode != RIA_QK_RAW && d.qk_mode != RIA_QK_NORMALIZED)
    return set_error(RIA_ERR_INVALID, "%s: unknown qk_mode %d", who, d.qk_mode);
  if (d.qk_mode == RIA_QK_NORMALIZED && fuse)
    return set_error(RIA_ERR_INVALID, "%s: RIA_QK_NORMALIZED takes convolved inputs (conv_layout RIA_CONV_NONE)", who);
  if (d.gate_mode == RIA_GATE_RAW && (!d.A_log || !d.dt_bias))
    return set_error(RIA_ERR_INVALID, "%s: RIA_GATE_RAW needs A_log and dt_bias", who);
  if (d.gate_mode != RIA_GATE_RAW && d.gate_mode != RIA_GATE_PRECOMPUTED)
    return set_error(RIA_ERR_INVALID, "%s: unknown gate_mode %d", who, d.gate_mode);
  if (reinterpret_cast<uintptr_t>(d.state_in) % 16 || reinterpret_cast<uintptr_t>(d.state_out) % 16 ||
      (fuse && reinterpret_cast<uintptr_t>(d.conv_weight) % 8 != 0))
    return set_error(RIA_ERR_INVALID, "%s: states must be 16-byte and conv_weight 8-byte aligned", who);
  const int conv_dim = (2 * num_k_heads + num_v_heads) * kGdnHeadDim;
  const int64_t x_width =
      d.qk_mode == RIA_QK_NORMALIZED ? (int64_t)3 * num_v_heads * kGdnHeadDim : (int64_t)conv_dim;
  if (d.x_row_stride < x_width) return set_error(RIA_ERR_INVALID, "%s: x_row_stride < %lld", who, (long long)x_width);
  if (d.gate_row_stride < num_v_heads) return set_error(RIA_ERR_INVALID, "%s: gate_row_stride < Hv", who);
  if (d.z && (!d.norm_weight || !valid_dtype(d.z_dtype) || d.z_row_stride < (int64_t)num_v_heads * kGdnHeadDim))
    return set_error(RIA_ERR_INVALID, "%s: a gate z needs norm_weight, a dtype code and row stride >= Hv*128", who);
  if (d.z && (reinterpret_cast<uintptr_t>(d.z) % 4 || d.z_row_stride % 2))
    return set_error(RIA_ERR_INVALID, "%s: z must be 4-byte aligned with an even row stride", who);
  // The state tiles of one launch are read and written by one workgroup each,
  // so in place is safe; a partial overlap would let a workgroup read a tile
  // another one has already written.  With seq_slot the pools are the
  // caller's pool_rows rows (every slot below it), otherwise `batch` rows.
  const bool disjoint_state = d.state_in != d.state_out;
  if (d.seq_slot && (disjoint_state || d.conv_layout == RIA_CONV_WINDOW) && d.pool_rows <= 0)
    return set_error(RIA_ERR_INVALID, "%s: with seq_slot, pool_rows (the pools' rows) is required for a separate "
                     "state_out or the window layout", who);
  const int64_t pool_rows = d.seq_slot ? d.pool_rows : d.batch;
  if (disjoint_state) {
    const int64_t pool_bytes = pool_rows * num_v_heads * kGdnHeadDim * kGdnHeadDim * 4;
    const char* i0 = reinterpret_cast<const char*>(d.state_in);
    const char* o0 = reinterpret_cast<const char*>(d.state_out);
    if (i0 < o0 + pool_bytes && o0 < i0 + pool_bytes)
      return set_error(RIA_ERR_INVALID, "%s: state_out overlaps state_in without being it", who);
  }
  if (d.conv_layout == RIA_CONV_WINDOW) {
    if (!d.conv_window_in || !d.conv_window_out)
      return set_error(RIA_ERR_INVALID, "%s: RIA_CONV_WINDOW needs conv_window_in and conv_window_out", who);
    if (reinterpret_cast<uintptr_t>(d.conv_window_in) % 8 || reinterpret_cast<uintptr_t>(d.conv_window_out) % 8)
      return set_error(RIA_ERR_INVALID, "%s: conv windows must be 8-byte aligned", who);
    // other workgroups read the channels a workgroup shifts: out must not overlap in
    const int64_t wbytes = pool_rows * conv_dim * kConvTaps * 2;
    const char* i0 = static_cast<const char*>(d.conv_window_in);
    const char* o0 = static_cast<const char*>(d.conv_window_out);
    if (i0 < o0 + wbytes && o0 < i0 + wbytes)
      return set_error(RIA_ERR_INVALID, "%s: conv_window_out must not overlap conv_window_in", who);
  }

  GdnDecodeArgs a{};
  a.x = d.x;
  a.x_stride = d.x_row_stride;
  a.conv_w = static_cast<const uint16_t*>(d.conv_weight);
  a.conv_ring = static_cast<uint16_t*>(d.conv_ring);
  a.conv_pos = d.conv_pos;
  a.conv_pos_scalar = d.conv_pos_scalar;
  a.conv_window = d.conv_layout == RIA_CONV_WINDOW ? 1 : 0;
  a.win_in = static_cast<const uint16_t*>(d.conv_window_in);
  a.win_out = static_cast<uint16_t*>(d.conv_window_out);
  a.state_in = d.state_in;
  a.state_out = d.state_out;
  a.seq_slot = d.seq_slot;
  a.qk_prenorm = d.qk_mode == RIA_QK_NORMALIZED ? 1 : 0;
  a.gate_a = d.gate_a;
  a.gate_b = d.gate_b;
  a.gate_stride = d.gate_row_stride;
  a.A_log = d.A_log;
  a.dt_bias = d.dt_bias;
  a.out = d.out;
  a.z = d.z;
  a.z_stride = d.z_row_stride;
  a.z_dtype = d.z_dtype;
  a.norm_w = d.norm_weight;
  a.num_k_heads = num_k_heads;
  a.num_v_heads = num_v_heads;
  a.conv_dim = conv_dim;

  // Column blocking: enough workgroups to cover 256 CUs several times over;
  // the gated norm needs whole heads.  From 1024 tiles on, 64-column blocks
  // (8 state vectors per thread) stream slightly faster than whole heads
  // (measured on MI355X in one process: 47.96 against 50.33 us at 2048
  // tiles, 93.7 against 94.2 us at 4096, even at 1024).
  const int64_t tiles = (int64_t)d.batch * num_v_heads;
  int cols = 128;
  if (!d.z) cols = tiles < 256 ? 32 : 64;
  a.ncb = kGdnHeadDim / cols;
  const int64_t blocks64 = tiles * a.ncb;
  if (blocks64 > 0x7fffffff) return set_error(RIA_ERR_INVALID, "%s: grid too large", who);
  const int blocks = static_cast<int>(blocks64);
  GdnVariant v{};
  v.ext = d.state_out != d.state_in || d.qk_mode == RIA_QK_NORMALIZED;
  // guarded v loads once the grid takes more than about 1.6 occupancy rounds
  // (5 workgroups of 128 columns per CU on MI355X's 256 CUs): measured on
  // MI355X, 94.2 against 99.0 us at 4096 tiles, 27.4 against 25.3 us at 1024
  v.vg = blocks >= 2048;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (cols == 128)
    launch_gdn_xt<128>(a, d.x_dtype, d.out_dtype, d.conv_layout, d.gate_mode, v, blocks, st);
  else if (cols == 64)
    launch_gdn_xt<64>(a, d.x_dtype, d.out_dtype, d.conv_layout, d.gate_mode, v, blocks, st);
  else
    launch_gdn_xt<32>(a, d.x_dtype, d.out_dtype, d.conv_layout, d.gate_mode, v, blocks, st);
  return check_launch(who);
}

// Standalone conv step over `channels` channels for `batch` rows, in the ring
// or the window layout (shared by ria_conv1d_step and ria_conv1d_window_step).
static int conv_step_launch(const GdnDecodeArgs& a, int batch, int channels, int x_dtype, int out_dtype,
                            hipStream_t st) {
  dim3 grid((channels + 255) / 256, batch);
#define RIA_CONV_LAUNCH(XT_, OT_)                                                                            \
  if (a.conv_window)                                                                                        \
    hipLaunchKernelGGL((conv1d_step_kernel<XT_, OT_, RIA_CONV_WINDOW>), grid, dim3(256), 0, st, a);        \
  else                                                                                                      \
    hipLaunchKernelGGL((conv1d_step_kernel<XT_, OT_, RIA_CONV_RING>), grid, dim3(256), 0, st, a)
#define RIA_CONV_OT(XT_)                                          \
  if (out_dtype == RIA_DT_BF16) RIA_CONV_LAUNCH(XT_, RIA_DT_BF16); \
  else if (out_dtype == RIA_DT_F16) RIA_CONV_LAUNCH(XT_, RIA_DT_F16); \
  else RIA_CONV_LAUNCH(XT_, RIA_DT_F32);
  if (x_dtype == RIA_DT_BF16) {
    RIA_CONV_OT(RIA_DT_BF16)
  } else if (x_dtype == RIA_DT_F16) {
    RIA_CONV_OT(RIA_DT_F16)
  } else {
    RIA_CONV_OT(RIA_DT_F32)
  }
#undef RIA_CONV_OT
#undef RIA_CONV_LAUNCH
  return RIA_OK;
}

}  // namespace ria

using namespace ria;

extern "C" int ria_gdn_decode(int batch, int num_k_heads, int num_v_heads, const void* mixed_qkv, int x_dtype,
                              int64_t x_row_stride, int fuse_conv, const void* conv_weight, void* conv_ring,
                              const int32_t* conv_pos, int32_t conv_pos_scalar, float* state,
                              const int32_t* seq_slot, const float* gate_a, const float* gate_b,
                              int64_t gate_row_stride, int gate_mode, const float* A_log, const float* dt_bias,
                              void* out, int out_dtype, const void* z, int z_dtype, int64_t z_row_stride,
                              const float* norm_weight, void* stream) {
  ria_gdn_decode_desc d{};
  d.batch = batch;
  d.num_k_heads = num_k_heads;
  d.num_v_heads = num_v_heads;
  d.x = mixed_qkv;
  d.x_dtype = x_dtype;
  d.x_row_stride = x_row_stride;
  d.conv_layout = fuse_conv ? RIA_CONV_RING : RIA_CONV_NONE;
  d.conv_weight = conv_weight;
  d.conv_ring = conv_ring;
  d.conv_pos = conv_pos;
  d.conv_pos_scalar = conv_pos_scalar;
  d.state_in = state;
  d.state_out = state;
  d.seq_slot = seq_slot;
  d.gate_a = gate_a;
  d.gate_b = gate_b;
  d.gate_row_stride = gate_row_stride;
  d.gate_mode = gate_mode;
  d.A_log = A_log;
  d.dt_bias = dt_bias;
  d.qk_mode = RIA_QK_RAW;
  d.out = out;
  d.out_dtype = out_dtype;
  d.z = z;
  d.z_dtype = z_dtype;
  d.z_row_stride = z_row_stride;
  d.norm_weight = norm_weight;
  return gdn_decode_launch(d, stream, "ria_gdn_decode");
}

extern "C" int ria_gdn_decode_ex(const ria_gdn_decode_desc* desc, void* stream) {
  if (!desc) return set_error(RIA_ERR_INVALID, "ria_gdn_decode_ex: null description");
  return gdn_decode_launch(*desc, stream, "ria_gdn_decode_ex");
}

extern "C" int ria_conv1d_step(int batch, int channels, const void* x, int x_dtype, int64_t x_row_stride,
                               const void* conv_weight, void* conv_ring, const int32_t* seq_slot,
                               const int32_t* conv_pos, int32_t conv_pos_scalar, void* out, int out_dtype,
                               void* stream) {
  if (batch < 0 || channels <= 0) return set_error(RIA_ERR_INVALID, "ria_conv1d_step: bad batch/channels");
  if (batch == 0) return RIA_OK;
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype))
    return set_error(RIA_ERR_INVALID, "ria_conv1d_step: unknown dtype code");
  if (!x || !conv_weight || !conv_ring || !out) return set_error(RIA_ERR_INVALID, "ria_conv1d_step: null pointer");
  if (reinterpret_cast<uintptr_t>(conv_weight) % 8 != 0)
    return set_error(RIA_ERR_INVALID, "ria_conv1d_step: conv_weight must be 8-byte aligned");
  if (x_row_stride < channels) return set_error(RIA_ERR_INVALID, "ria_conv1d_step: x_row_stride < channels");
  GdnDecodeArgs a{};
  a.x = x;
  a.x_stride = x_row_stride;
  a.conv_w = static_cast<const uint16_t*>(conv_weight);
  a.conv_ring = static_cast<uint16_t*>(conv_ring);
  a.conv_pos = conv_pos;
  a.conv_pos_scalar = conv_pos_scalar;
  a.seq_slot = seq_slot;
  a.out = out;
  a.conv_dim = channels;
  conv_step_launch(a, batch, channels, x_dtype, out_dtype, static_cast<hipStream_t>(stream));
  return check_launch("ria_conv1d_step");
}

extern "C" int ria_conv1d_window_step(int batch, int channels, const void* x, int x_dtype, int64_t x_row_stride,
                                      const void* conv_weight, const void* window_in, void* window_out, void* out,
                                      int out_dtype, void* stream) {
  if (batch < 0 || channels <= 0) return set_error(RIA_ERR_INVALID, "ria_conv1d_window_step: bad batch/channels");
  if (batch == 0) return RIA_OK;
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype))
    return set_error(RIA_ERR_INVALID, "ria_conv1d_window_step: unknown dtype code");
  if (!x || !conv_weight || !window_in || !window_out || !out)
    return set_error(RIA_ERR_INVALID, "ria_conv1d_window_step: null pointer");
  if (reinterpret_cast<uintptr_t>(conv_weight) % 8 || reinterpret_cast<uintptr_t>(window_in) % 8 ||
      reinterpret_cast<uintptr_t>(window_out) % 8)
    return set_error(RIA_ERR_INVALID, "ria_conv1d_window_step: conv_weight and windows must be 8-byte aligned");
  if (x_row_stride < channels) return set_error(RIA_ERR_INVALID, "ria_conv1d_window_step: x_row_stride < channels");
  // one thread per channel reads its window and writes the shifted one: in place is safe here
  GdnDecodeArgs a{};
  a.x = x;
  a.x_stride = x_row_stride;
  a.conv_w = static_cast<const uint16_t*>(conv_weight);
  a.conv_window = 1;
  a.win_in = static_cast<const uint16_t*>(window_in);
  a.win_out = static_cast<uint16_t*>(window_out);
  a.out = out;
  a.conv_dim = channels;
  conv_step_launch(a, batch, channels, x_dtype, out_dtype, static_cast<hipStream_t>(stream));
  return check_launch("ria_conv1d_window_step");
}
