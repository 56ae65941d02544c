// Small elementwise entry points behind the module-level helpers of the
// attention cache: _rope, _apply_rope and _l2norm
// (v2/src/router_ia/qwen36_attention_cache.py:137-173), and the two RMSNorm
// forms around it: the (1 + w) RMSNorm of the layer input and of q / k
// (qwen36_op_probe.py:55-67, used at qwen36_attention_cache.py:227,302-305)
// and the gated RMSNorm of the DeltaNet read-out (qwen36_gated_norm_probe.py:19-36,
// used at qwen36_attention_cache.py:268-271).
#include <math.h>

#include "ria_common.h"

namespace ria {

__global__ void rope_table_kernel(int32_t position, const float* inv_freq, int rope_dim, float* cos_out,
                                  float* sin_out) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= rope_dim) return;
  const int half = rope_dim >> 1;
  // angles = float(position) * inv_freq ; emb = cat(angles, angles)
  const float ang = mul_rn(static_cast<float>(position), inv_freq[d < half ? d : d - half]);
  cos_out[d] = cosf(ang);
  sin_out[d] = sinf(ang);
}

// One workgroup per row; rows of up to 1024 elements held in LDS.
__global__ __launch_bounds__(256) void rope_apply_kernel(int head_dim, int rope_dim, const float* x, float* out,
                                                         const float* inv_freq, int32_t position) {
  __shared__ float row_s[1024];
  const int64_t r = blockIdx.x;
  const float* xr = x + r * head_dim;
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) row_s[d] = xr[d];
  __syncthreads();
  const int half = rope_dim >> 1;
  const float pos = static_cast<float>(position);
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
    float y = row_s[d];
    if (d < rope_dim) {
      const float ang = mul_rn(pos, inv_freq[d < half ? d : d - half]);
      const float c = cosf(ang), s = sinf(ang);
      const float rot = d < half ? -row_s[d + half] : row_s[d - half];
      y = add_rn(mul_rn(row_s[d], c), mul_rn(rot, s));
    }
    out[r * head_dim + d] = y;
  }
}

// One wavefront per row: x * (1 / sqrt(sum(x*x) + eps)).
template <int XT>
__global__ __launch_bounds__(256) void l2norm_kernel(int64_t rows, int dim, const void* x, float eps, float* out) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  float ss = 0.f;
  for (int d = lane; d < dim; d += 64) {
    const float v = load_act<XT>(x, r * dim + d);
    ss += mul_rn(v, v);
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss + eps);
  for (int d = lane; d < dim; d += 64) out[r * dim + d] = mul_rn(load_act<XT>(x, r * dim + d), inv);
}

struct NormArgs {
  const void* x;
  int64_t x_stride;  // elements between tokens
  const void* z;     // gated form only
  int64_t z_stride;
  int z_dtype;
  const float* weight;
  float eps;
  void* out;
  int64_t out_stride;
  int64_t rows;  // tokens * heads
  int heads;
  int dim;
};

// One wavefront per (token, head) row of `dim` elements; head h of a token
// starts at element h * dim of the token's row.  Each lane reads its own
// elements in both passes, so `out` may alias `x` when both have one dtype
// and one stride.
template <int XT, int OT, bool GATED>
__global__ __launch_bounds__(256) void rmsnorm_kernel(NormArgs a) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= a.rows) return;
  const int64_t t = r / a.heads;
  const int64_t hoff = (r - t * a.heads) * a.dim;
  const int64_t xo = t * a.x_stride + hoff;
  float ss = 0.f;
  for (int d = lane; d < a.dim; d += 64) {
    const float v = load_act<XT>(a.x, xo + d);
    ss = add_rn(ss, mul_rn(v, v));
  }
  const float rs = rms_scale(wave_sum(ss), a.dim, a.eps);
  const int64_t oo = t * a.out_stride + hoff;
  const int64_t zo = t * a.z_stride + hoff;
  for (int d = lane; d < a.dim; d += 64) {
    const float v = load_act<XT>(a.x, xo + d);
    float y;
    if constexpr (GATED)
      y = gated_norm_elem<XT>(v, rs, a.weight[d], load_act_dt(a.z, zo + d, a.z_dtype));
    else
      y = rmsnorm_elem<XT>(v, rs, a.weight[d]);
    store_act<OT>(a.out, oo + d, y);
  }
}

// Vector form for rows whose elements can move four at a time (dim, strides
// and head offsets multiples of 4, bases aligned to 4 elements): a group of
// RL lanes owns each row, every lane loads and stores 4 contiguous elements
// per access, and the group reduces its sum of squares with xor shuffles.
template <int XT, int OT, bool GATED, int RL, int NCH>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(NormArgs a) {
  constexpr int kRowsPerWave = 64 / RL;
  const int lane = threadIdx.x & 63;
  const int64_t r = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kRowsPerWave + lane / RL;
  const int li = lane % RL;
  const bool ok = r < a.rows;  // rows past the end still take part in the shuffles
  const int64_t t = ok ? r / a.heads : 0;
  const int64_t hoff = ok ? (r - t * a.heads) * a.dim : 0;
  const int64_t xo = t * a.x_stride + hoff;
  const int64_t oo = t * a.out_stride + hoff;
  const int64_t zo = t * a.z_stride + hoff;
  // z: the gate's 4 values at c (gated), loaded by the caller
  auto finish = [&](int c, const float (&v)[4], float rs, f32x4 w, const float (&z)[4]) {
    float y[4];
    if constexpr (GATED) {
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] = gated_norm_elem<XT>(v[j], rs, w[j], z[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] = rmsnorm_elem<XT>(v[j], rs, w[j]);
    }
    store_act4<OT>(a.out, oo + c, y);
  };
  float ss = 0.f;
  if constexpr (NCH > 0) {
    // dim == 4 RL NCH: the lane's NCH chunks are loaded at once and kept in
    // registers for the second pass (the squares are summed in the same order
    // as the loop below, so both give the same bits)
    float v[NCH][4], z[NCH][4] = {};
    f32x4 w[NCH];  // the weights and the gate too, so their loads overlap the reduction
    if (ok) {
#pragma unroll
      for (int q = 0; q < NCH; ++q) load_act4<XT>(a.x, xo + 4 * li + 4 * RL * q, v[q]);
#pragma unroll
      for (int q = 0; q < NCH; ++q) w[q] = *reinterpret_cast<const f32x4*>(a.weight + 4 * li + 4 * RL * q);
      if constexpr (GATED) {
#pragma unroll
        for (int q = 0; q < NCH; ++q) load_act4_dt(a.z, zo + 4 * li + 4 * RL * q, a.z_dtype, z[q]);
      }
#pragma unroll
      for (int q = 0; q < NCH; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) ss = add_rn(ss, mul_rn(v[q][j], v[q][j]));
    }
#pragma unroll
    for (int off = RL / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (!ok) return;
    const float rs = rms_scale(ss, a.dim, a.eps);
#pragma unroll
    for (int q = 0; q < NCH; ++q) finish(4 * li + 4 * RL * q, v[q], rs, w[q], z[q]);
  } else {
    if (ok) {
      for (int c = 4 * li; c < a.dim; c += 4 * RL) {
        float v[4];
        load_act4<XT>(a.x, xo + c, v);
#pragma unroll
        for (int j = 0; j < 4; ++j) ss = add_rn(ss, mul_rn(v[j], v[j]));
      }
    }
#pragma unroll
    for (int off = RL / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    if (!ok) return;
    const float rs = rms_scale(ss, a.dim, a.eps);
    for (int c = 4 * li; c < a.dim; c += 4 * RL) {
      float v[4], z[4] = {};
      load_act4<XT>(a.x, xo + c, v);
      if constexpr (GATED) load_act4_dt(a.z, zo + c, a.z_dtype, z);
      finish(c, v, rs, *reinterpret_cast<const f32x4*>(a.weight + c), z);
    }
  }
}

template <int XT, int OT, bool GATED>
static void launch_norm_rl(const NormArgs& a, bool vec, hipStream_t st) {
  if (!vec) {  // one row per wavefront, four per workgroup
    hipLaunchKernelGGL((rmsnorm_kernel<XT, OT, GATED>), dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, st, a);
    return;
  }
  // lanes per row: one 4-element chunk per lane for dims up to 256
  const int rl = a.dim >= 256 ? 64 : (a.dim >= 128 ? 32 : 16);
  const int64_t rows_per_block = 4 * (64 / rl);
  const dim3 grid((unsigned)((a.rows + rows_per_block - 1) / rows_per_block));
  // chunks of 4 per lane: held in registers when the row is 1, 2, 4 or 8 of them
  const int nch = a.dim % (4 * rl) == 0 ? a.dim / (4 * rl) : 0;
#define RIA_NORM_VEC(RL_, NCH_) hipLaunchKernelGGL((rmsnorm_vec_kernel<XT, OT, GATED, RL_, NCH_>), grid, dim3(256), 0, st, a)
  if (rl == 64) {
    if (nch == 8)
      RIA_NORM_VEC(64, 8);
    else if (nch == 4)
      RIA_NORM_VEC(64, 4);
    else if (nch == 2)
      RIA_NORM_VEC(64, 2);
    else if (nch == 1)
      RIA_NORM_VEC(64, 1);
    else
      RIA_NORM_VEC(64, 0);
  } else if (rl == 32) {
    if (nch == 1)
      RIA_NORM_VEC(32, 1);
    else
      RIA_NORM_VEC(32, 0);
  } else {
    RIA_NORM_VEC(16, 0);
  }
#undef RIA_NORM_VEC
}

template <int XT, bool GATED>
static void launch_norm_ot(const NormArgs& a, int out_dtype, bool vec, hipStream_t st) {
  if (out_dtype == RIA_DT_BF16)
    launch_norm_rl<XT, RIA_DT_BF16, GATED>(a, vec, st);
  else if (out_dtype == RIA_DT_F16)
    launch_norm_rl<XT, RIA_DT_F16, GATED>(a, vec, st);
  else
    launch_norm_rl<XT, RIA_DT_F32, GATED>(a, vec, st);
}

static int dt_bytes(int dt) { return dt == RIA_DT_F32 ? 4 : 2; }

// Whether every row of this launch can move in aligned 4-element vectors.
static bool norm_vectorizable(const NormArgs& a, int x_dtype, int out_dtype, bool gated) {
  auto aligned = [](const void* p, int dt, int64_t stride) {
    return reinterpret_cast<uintptr_t>(p) % (4 * dt_bytes(dt)) == 0 && stride % 4 == 0;
  };
  return a.dim % 4 == 0 && reinterpret_cast<uintptr_t>(a.weight) % 16 == 0 && aligned(a.x, x_dtype, a.x_stride) &&
         aligned(a.out, out_dtype, a.out_stride) && (!gated || aligned(a.z, a.z_dtype, a.z_stride));
}

static bool norm_dtype_ok(int dt) { return dt == RIA_DT_BF16 || dt == RIA_DT_F16 || dt == RIA_DT_F32; }

template <bool GATED>
static int launch_norm(const char* who, int64_t tokens, int heads, int dim, const void* x, int x_dtype,
                       int64_t x_stride, const void* z, int z_dtype, int64_t z_stride, const float* weight, float eps,
                       void* out, int out_dtype, int64_t out_stride, void* stream) {
  if (tokens < 0 || heads <= 0 || dim <= 0) return set_error(RIA_ERR_INVALID, "%s: bad sizes", who);
  if (!norm_dtype_ok(x_dtype) || !norm_dtype_ok(out_dtype) || (GATED && !norm_dtype_ok(z_dtype)))
    return set_error(RIA_ERR_INVALID, "%s: unknown dtype code", who);
  const int64_t row = (int64_t)heads * dim;
  if (x_stride < row || out_stride < row || (GATED && z_stride < row))
    return set_error(RIA_ERR_INVALID, "%s: token stride smaller than heads * dim", who);
  if (!(eps >= 0.f)) return set_error(RIA_ERR_INVALID, "%s: eps must be >= 0", who);
  if (tokens == 0) return RIA_OK;
  if (!x || !weight || !out || (GATED && !z)) return set_error(RIA_ERR_INVALID, "%s: null pointer", who);
  const int64_t rows = tokens * heads;
  if ((rows + 3) / 4 > 0x7fffffff) return set_error(RIA_ERR_INVALID, "%s: too many rows", who);
  NormArgs a{};
  a.x = x;
  a.x_stride = x_stride;
  a.z = z;
  a.z_stride = z_stride;
  a.z_dtype = z_dtype;
  a.weight = weight;
  a.eps = eps;
  a.out = out;
  a.out_stride = out_stride;
  a.rows = rows;
  a.heads = heads;
  a.dim = dim;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = norm_vectorizable(a, x_dtype, out_dtype, GATED);
  if (x_dtype == RIA_DT_BF16)
    launch_norm_ot<RIA_DT_BF16, GATED>(a, out_dtype, vec, st);
  else if (x_dtype == RIA_DT_F16)
    launch_norm_ot<RIA_DT_F16, GATED>(a, out_dtype, vec, st);
  else
    launch_norm_ot<RIA_DT_F32, GATED>(a, out_dtype, vec, st);
  return check_launch(who);
}

}  // namespace ria

using namespace ria;

extern "C" int ria_rmsnorm(int64_t tokens, int heads, int dim, const void* x, int x_dtype, int64_t x_token_stride,
                           const float* weight, float eps, void* out, int out_dtype, int64_t out_token_stride,
                           void* stream) {
  return launch_norm<false>("ria_rmsnorm", tokens, heads, dim, x, x_dtype, x_token_stride, nullptr, RIA_DT_F32, 0,
                            weight, eps, out, out_dtype, out_token_stride, stream);
}

extern "C" int ria_gated_rmsnorm(int64_t tokens, int heads, int dim, const void* x, int x_dtype,
                                 int64_t x_token_stride, const void* z, int z_dtype, int64_t z_token_stride,
                                 const float* weight, float eps, void* out, int out_dtype, int64_t out_token_stride,
                                 void* stream) {
  return launch_norm<true>("ria_gated_rmsnorm", tokens, heads, dim, x, x_dtype, x_token_stride, z, z_dtype,
                           z_token_stride, weight, eps, out, out_dtype, out_token_stride, stream);
}

extern "C" int ria_rope_table(int32_t position, const float* inv_freq, int rope_dim, float* cos_out,
                              float* sin_out, void* stream) {
  if (rope_dim <= 0 || rope_dim % 2) return set_error(RIA_ERR_INVALID, "ria_rope_table: rope_dim must be positive and even");
  if (!inv_freq || !cos_out || !sin_out) return set_error(RIA_ERR_INVALID, "ria_rope_table: null pointer");
  hipLaunchKernelGGL(rope_table_kernel, dim3((rope_dim + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), position, inv_freq, rope_dim, cos_out, sin_out);
  return check_launch("ria_rope_table");
}

extern "C" int ria_rope_apply(int64_t rows, int head_dim, int rope_dim, const float* x, float* out,
                              const float* inv_freq, int32_t position, void* stream) {
  if (rows < 0 || head_dim <= 0 || head_dim > 1024) return set_error(RIA_ERR_INVALID, "ria_rope_apply: head_dim must be in [1, 1024]");
  if (rope_dim < 0 || rope_dim % 2 || rope_dim > head_dim)
    return set_error(RIA_ERR_INVALID, "ria_rope_apply: rope_dim must be even and <= head_dim");
  if (rows == 0) return RIA_OK;
  if (!x || !out || (rope_dim > 0 && !inv_freq)) return set_error(RIA_ERR_INVALID, "ria_rope_apply: null pointer");
  if (rows > 0x7fffffff) return set_error(RIA_ERR_INVALID, "ria_rope_apply: too many rows");
  hipLaunchKernelGGL(rope_apply_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), head_dim, rope_dim, x, out, inv_freq, position);
  return check_launch("ria_rope_apply");
}

extern "C" int ria_l2norm(int64_t rows, int dim, const void* x, int x_dtype, float eps, float* out, void* stream) {
  if (rows < 0 || dim <= 0) return set_error(RIA_ERR_INVALID, "ria_l2norm: bad sizes");
  if (rows == 0) return RIA_OK;
  if (!x || !out) return set_error(RIA_ERR_INVALID, "ria_l2norm: null pointer");
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffff) return set_error(RIA_ERR_INVALID, "ria_l2norm: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(blocks));
  if (x_dtype == RIA_DT_BF16)
    hipLaunchKernelGGL((l2norm_kernel<RIA_DT_BF16>), grid, dim3(256), 0, st, rows, dim, x, eps, out);
  else if (x_dtype == RIA_DT_F16)
    hipLaunchKernelGGL((l2norm_kernel<RIA_DT_F16>), grid, dim3(256), 0, st, rows, dim, x, eps, out);
  else if (x_dtype == RIA_DT_F32)
    hipLaunchKernelGGL((l2norm_kernel<RIA_DT_F32>), grid, dim3(256), 0, st, rows, dim, x, eps, out);
  else
    return set_error(RIA_ERR_INVALID, "ria_l2norm: unknown dtype code");
  return check_launch("ria_l2norm");
}
