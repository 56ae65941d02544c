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
#include "ria_common.h"

namespace ria {

struct GdnDecodeArgs {
  const void* x;
  int64_t x_stride;
  const uint16_t* conv_w;  // [conv_dim, 4] bf16
  uint16_t* conv_ring;     // [pool, 4, conv_dim] bf16
  const int32_t* conv_pos;
  int32_t conv_pos_scalar;
  float* state;  // [pool, Hv, 128, 128]
  const int32_t* seq_slot;
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

// Post-conv value of channel c for batch row b, as the reference sees it
// after `_causal_conv1d_step` returns (cast back to the input dtype).  When
// `write` is set the current input is stored into ring slot n mod 4.
template <int XT, bool FUSE>
__device__ __forceinline__ float conv_channel(const GdnDecodeArgs& a, int b, int row, int n, int c,
                                              bool write) {
  const float xv = load_act<XT>(a.x, (int64_t)b * a.x_stride + c);
  if constexpr (!FUSE) {
    return xv;
  } else {
    const uint16_t xb = f32_to_bf16_bits(xv);  // mixed_qkv.to(conv_dtype)
    uint16_t* ring = a.conv_ring + (int64_t)row * kConvRing * a.conv_dim;
    const float h0 = bf16_bits_to_f32(ring[((n - 3) & 3) * a.conv_dim + c]);
    const float h1 = bf16_bits_to_f32(ring[((n - 2) & 3) * a.conv_dim + c]);
    const float h2 = bf16_bits_to_f32(ring[((n - 1) & 3) * a.conv_dim + c]);
    const uint2 wv = *reinterpret_cast<const uint2*>(a.conv_w + (int64_t)c * kConvTaps);
    const float w0 = bf16_bits_to_f32(wv.x & 0xffffu), w1 = bf16_bits_to_f32(wv.x >> 16);
    const float w2 = bf16_bits_to_f32(wv.y & 0xffffu), w3 = bf16_bits_to_f32(wv.y >> 16);
    float acc = w0 * h0;
    acc = fmaf(w1, h1, acc);
    acc = fmaf(w2, h2, acc);
    acc = fmaf(w3, bf16_bits_to_f32(xb), acc);
    const float y = round_bf16(silu_f(round_bf16(acc)));
    if (write) ring[(n & 3) * a.conv_dim + c] = xb;
    return through_dtype<XT>(y);
  }
}

template <int COLS, int XT, int OT, bool FUSE, int GM, bool NORM>
__global__ __launch_bounds__(256) void gdn_decode_kernel(GdnDecodeArgs a) {
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
  const int hk = h / group;
  const int kdim = a.num_k_heads * kGdnHeadDim;
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

  // Conv / projection inputs first, so their latency overlaps the state loads.
  const bool qk_writer = FUSE && (h % group == 0) && cb == 0;
  const int qk_c = tid < 128 ? hk * kGdnHeadDim + tid : kdim + hk * kGdnHeadDim + (tid - 128);
  float qk_raw = conv_channel<XT, FUSE>(a, b, row, n, qk_c, qk_writer);
  float v_raw = 0.f;
  if (tid < COLS) v_raw = conv_channel<XT, FUSE>(a, b, row, n, 2 * kdim + h * kGdnHeadDim + col0 + tid, FUSE);
  // The gated norm's z (as the raw 32-bit word holding it; every thread loads
  // one, threads past COLS a repeat, so no branch makes the wait early) and w.
  ActWord z_word{};
  float w_raw = 0.f;
  if constexpr (NORM) {
    const int tc = tid % COLS;
    z_word = load_act_word(a.z, (int64_t)b * a.z_stride + h * kGdnHeadDim + tc, a.z_dtype);
    w_raw = a.norm_w[tc];
  }

  float* S = a.state + ((int64_t)row * a.num_v_heads + h) * (kGdnHeadDim * kGdnHeadDim);
  f32x4 s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    s[r] = ld_stream(reinterpret_cast<const f32x4*>(S + (rg + RG * r) * kGdnHeadDim + col0 + jl));
  }


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
  const float inv = 1.0f / sqrtf((tid < 128 ? scal_s[0] + scal_s[1] : scal_s[2] + scal_s[3]) + 1e-6f);
  float qk_n = mul_rn(qk_raw, inv);
  if (tid < 128) {
    qk_n = mul_rn(qk_n, 0.08838834764831845f);
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

  // Rank-1 update, written back in place.
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg + RG * r;
    const float ki = k_s[i];
#pragma unroll
    for (int c = 0; c < 4; ++c) s[r][c] = add_rn(s[r][c], mul_rn(ki, dj[c]));
    st_stream(reinterpret_cast<f32x4*>(S + i * kGdnHeadDim + col0 + jl), s[r]);
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
template <int XT, int OT>
__global__ __launch_bounds__(256) void conv1d_step_kernel(GdnDecodeArgs a) {
  const int b = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.conv_dim) return;
  const int row = a.seq_slot ? a.seq_slot[b] : b;
  const int n = a.conv_pos ? a.conv_pos[b] : a.conv_pos_scalar;
  // The reference returns the bf16 conv result cast to the input dtype; the
  // caller-selected output dtype is applied on top of that.
  const float y = conv_channel<XT, true>(a, b, row, n, c, true);
  store_act<OT>(a.out, (int64_t)b * a.conv_dim + c, y);
}

template <int COLS, int XT, int OT, bool FUSE, bool NORM>
static void launch_gdn_gm(const GdnDecodeArgs& a, int gate_mode, int blocks, hipStream_t st) {
  if (gate_mode == RIA_GATE_RAW)
    hipLaunchKernelGGL((gdn_decode_kernel<COLS, XT, OT, FUSE, RIA_GATE_RAW, NORM>), dim3(blocks), dim3(256), 0, st,
                       a);
  else
    hipLaunchKernelGGL((gdn_decode_kernel<COLS, XT, OT, FUSE, RIA_GATE_PRECOMPUTED, NORM>), dim3(blocks), dim3(256),
                       0, st, a);
}

template <int COLS, int XT, int OT, bool FUSE>
static void launch_gdn_norm(const GdnDecodeArgs& a, int gate_mode, int blocks, hipStream_t st) {
  if constexpr (COLS == kGdnHeadDim) {
    if (a.z) {
      launch_gdn_gm<COLS, XT, OT, FUSE, true>(a, gate_mode, blocks, st);
      return;
    }
  }
  launch_gdn_gm<COLS, XT, OT, FUSE, false>(a, gate_mode, blocks, st);
}

template <int COLS, int XT, int OT>
static void launch_gdn_fuse(const GdnDecodeArgs& a, bool fuse, int gate_mode, int blocks, hipStream_t st) {
  if (fuse)
    launch_gdn_norm<COLS, XT, OT, true>(a, gate_mode, blocks, st);
  else
    launch_gdn_norm<COLS, XT, OT, false>(a, gate_mode, blocks, st);
}

template <int COLS, int XT>
static void launch_gdn_ot(const GdnDecodeArgs& a, int ot, bool fuse, int gate_mode, int blocks, hipStream_t st) {
  if (ot == RIA_DT_BF16)
    launch_gdn_fuse<COLS, XT, RIA_DT_BF16>(a, fuse, gate_mode, blocks, st);
  else if (ot == RIA_DT_F16)
    launch_gdn_fuse<COLS, XT, RIA_DT_F16>(a, fuse, gate_mode, blocks, st);
  else
    launch_gdn_fuse<COLS, XT, RIA_DT_F32>(a, fuse, gate_mode, blocks, st);
}

template <int COLS>
static void launch_gdn_xt(const GdnDecodeArgs& a, int xt, int ot, bool fuse, int gate_mode, int blocks,
                          hipStream_t st) {
  if (xt == RIA_DT_BF16)
    launch_gdn_ot<COLS, RIA_DT_BF16>(a, ot, fuse, gate_mode, blocks, st);
  else if (xt == RIA_DT_F16)
    launch_gdn_ot<COLS, RIA_DT_F16>(a, ot, fuse, gate_mode, blocks, st);
  else
    launch_gdn_ot<COLS, RIA_DT_F32>(a, ot, fuse, gate_mode, blocks, st);
}

static bool valid_dtype(int dt) { return dt == RIA_DT_BF16 || dt == RIA_DT_F16 || dt == RIA_DT_F32; }

}  // namespace ria

using namespace ria;

extern "C" int ria_gdn_decode(int batch, int num_k_heads, int num_v_heads, const void* mixed_qkv, int x_dtype,
                              int64_t x_row_stride, int fuse_conv, const void* conv_weight, void* conv_ring,
                              const int32_t* conv_pos, int32_t conv_pos_scalar, float* state,
                              const int32_t* seq_slot, const float* gate_a, const float* gate_b,
                              int64_t gate_row_stride, int gate_mode, const float* A_log, const float* dt_bias,
                              void* out, int out_dtype, const void* z, int z_dtype, int64_t z_row_stride,
                              const float* norm_weight, void* stream) {
  if (batch < 0) return set_error(RIA_ERR_INVALID, "ria_gdn_decode: batch must be >= 0");
  if (batch == 0) return RIA_OK;
  if (num_k_heads <= 0 || num_v_heads <= 0 || num_v_heads % num_k_heads != 0)
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: num_v_heads (%d) must be a positive multiple of num_k_heads (%d)",
                     num_v_heads, num_k_heads);
  if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype))
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: unknown dtype code");
  if (!mixed_qkv || !state || !gate_a || !gate_b || !out)
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: null tensor pointer");
  if (fuse_conv && (!conv_weight || !conv_ring))
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: fuse_conv needs conv_weight and conv_ring");
  if (gate_mode == RIA_GATE_RAW && (!A_log || !dt_bias))
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: RIA_GATE_RAW needs A_log and dt_bias");
  if (gate_mode != RIA_GATE_RAW && gate_mode != RIA_GATE_PRECOMPUTED)
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: unknown gate_mode %d", gate_mode);
  if (reinterpret_cast<uintptr_t>(state) % 16 != 0 || (fuse_conv && reinterpret_cast<uintptr_t>(conv_weight) % 8 != 0))
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: state must be 16-byte and conv_weight 8-byte aligned");
  const int conv_dim = (2 * num_k_heads + num_v_heads) * kGdnHeadDim;
  if (x_row_stride < conv_dim) return set_error(RIA_ERR_INVALID, "ria_gdn_decode: x_row_stride < conv_dim");
  if (gate_row_stride < num_v_heads) return set_error(RIA_ERR_INVALID, "ria_gdn_decode: gate_row_stride < Hv");
  if (z && (!norm_weight || !valid_dtype(z_dtype) || z_row_stride < (int64_t)num_v_heads * kGdnHeadDim))
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: a gate z needs norm_weight, a dtype code and row stride >= Hv*128");
  if (z && (reinterpret_cast<uintptr_t>(z) % 4 || z_row_stride % 2))
    return set_error(RIA_ERR_INVALID, "ria_gdn_decode: z must be 4-byte aligned with an even row stride");

  GdnDecodeArgs a{};
  a.x = mixed_qkv;
  a.x_stride = x_row_stride;
  a.conv_w = static_cast<const uint16_t*>(conv_weight);
  a.conv_ring = static_cast<uint16_t*>(conv_ring);
  a.conv_pos = conv_pos;
  a.conv_pos_scalar = conv_pos_scalar;
  a.state = state;
  a.seq_slot = seq_slot;
  a.gate_a = gate_a;
  a.gate_b = gate_b;
  a.gate_stride = gate_row_stride;
  a.A_log = A_log;
  a.dt_bias = dt_bias;
  a.out = out;
  a.z = z;
  a.z_stride = z_row_stride;
  a.z_dtype = z_dtype;
  a.norm_w = norm_weight;
  a.num_k_heads = num_k_heads;
  a.num_v_heads = num_v_heads;
  a.conv_dim = conv_dim;

  // Column blocking: enough workgroups to cover 256 CUs several times over;
  // the gated norm needs whole heads.
  const int64_t tiles = (int64_t)batch * num_v_heads;
  int cols = 128;
  if (!z) {
    if (tiles < 256) cols = 32;
    else if (tiles < 1024) cols = 64;
  }
  a.ncb = kGdnHeadDim / cols;
  const int64_t blocks64 = tiles * a.ncb;
  if (blocks64 > 0x7fffffff) return set_error(RIA_ERR_INVALID, "ria_gdn_decode: grid too large");
  const int blocks = static_cast<int>(blocks64);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool fuse = fuse_conv != 0;
  if (cols == 128)
    launch_gdn_xt<128>(a, x_dtype, out_dtype, fuse, gate_mode, blocks, st);
  else if (cols == 64)
    launch_gdn_xt<64>(a, x_dtype, out_dtype, fuse, gate_mode, blocks, st);
  else
    launch_gdn_xt<32>(a, x_dtype, out_dtype, fuse, gate_mode, blocks, st);
  return check_launch("ria_gdn_decode");
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
  dim3 grid((channels + 255) / 256, batch);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RIA_CONV_LAUNCH(XT_, OT_) hipLaunchKernelGGL((conv1d_step_kernel<XT_, OT_>), grid, dim3(256), 0, st, a)
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
  return check_launch("ria_conv1d_step");
}
