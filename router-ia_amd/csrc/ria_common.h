// Shared device helpers for the gfx950 hybrid-attention kernels.
//
// Numeric conventions follow the PyTorch ops the reference path uses
// (v2/src/router_ia/qwen36_attention_cache.py): bf16 <-> fp32 conversion is
// round-to-nearest-even on the bit pattern (c10::BFloat16), fp16 uses the
// hardware RNE conversion, and elementwise products/sums that torch evaluates
// as separate kernels are written with non-contracting intrinsics so the
// compiler cannot fuse them into an FMA with a different rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ria_hybrid_attn.h"

namespace ria {

// Head geometry fixed by the model family (v2/src/router_ia/qwen36_40layer_loop.py:36-50).
constexpr int kGdnHeadDim = 128;   // DeltaNet dk == dv
constexpr int kConvTaps = 4;       // LINEAR_CONV_KERNEL
constexpr int kConvRing = 4;       // ring slots per channel (slot = step mod 4)
constexpr int kAttnHeadDim = 256;  // FULL_HEAD_DIM
constexpr int kPageTokens = 16;    // tokens per KV page

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16, as c10::BFloat16 rounds finite values.
// gfx950 converts in hardware (v_cvt_pk_bf16_f32, two values per instruction).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, b);
  return static_cast<float>(h);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

// Load element `i` of an activation tensor with dtype code DT and widen to fp32.
template <int DT>
__device__ __forceinline__ float load_act(const void* p, int64_t i) {
  if constexpr (DT == RIA_DT_BF16) {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else if constexpr (DT == RIA_DT_F16) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return static_cast<const float*>(p)[i];
  }
}

// load_act split in two: the raw element (16 or 32 bits) now, its fp32
// value later, so that a caller can issue more loads before any widening
// makes the compiler wait for this one.
template <int DT>
__device__ __forceinline__ uint32_t load_act_bits(const void* p, int64_t i) {
  if constexpr (DT == RIA_DT_F32) {
    return static_cast<const uint32_t*>(p)[i];
  } else {
    return static_cast<const uint16_t*>(p)[i];
  }
}

template <int DT>
__device__ __forceinline__ float act_from_bits(uint32_t b) {
  if constexpr (DT == RIA_DT_BF16) {
    return bf16_bits_to_f32(static_cast<uint16_t>(b));
  } else if constexpr (DT == RIA_DT_F16) {
    return f16_bits_to_f32(static_cast<uint16_t>(b));
  } else {
    return __uint_as_float(b);
  }
}

// load_act with the dtype code known only at run time (side inputs such as
// the gated norm's z, where a template parameter would multiply instances).
__device__ __forceinline__ float load_act_dt(const void* p, int64_t i, int dt) {
  if (dt == RIA_DT_BF16) return load_act<RIA_DT_BF16>(p, i);
  if (dt == RIA_DT_F16) return load_act<RIA_DT_F16>(p, i);
  return load_act<RIA_DT_F32>(p, i);
}

// Element i of a tensor with a run-time dtype code, loaded without branches
// (a branch around a load makes the compiler wait for it at the join): the
// aligned 32-bit word holding the element is loaded, and act_from_word picks
// the element out later, so that the wait for the load can come late too.
// A 16-bit tensor must start on a 4-byte boundary with an even row stride.
struct ActWord {
  uint32_t w;
  bool high;  // 16-bit element in the upper half
};

__device__ __forceinline__ ActWord load_act_word(const void* p, int64_t i, int dt) {
  const int64_t byte = dt == RIA_DT_F32 ? i * 4 : i * 2;
  return ActWord{*reinterpret_cast<const uint32_t*>(static_cast<const char*>(p) + (byte & ~int64_t(3))),
                 (byte & 2) != 0};
}

__device__ __forceinline__ float act_from_word(ActWord a, int dt) {
  const uint16_t h = static_cast<uint16_t>(a.high ? (a.w >> 16) : (a.w & 0xffffu));
  const float narrow = dt == RIA_DT_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
  return dt == RIA_DT_F32 ? __uint_as_float(a.w) : narrow;
}

template <int DT>
__device__ __forceinline__ void store_act(void* p, int64_t i, float v) {
  if constexpr (DT == RIA_DT_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  } else if constexpr (DT == RIA_DT_F16) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

// store_act with the dtype as a run-time value.
__device__ __forceinline__ void store_act_dt(void* p, int64_t i, float v, int dt) {
  if (dt == RIA_DT_BF16)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  else if (dt == RIA_DT_F16)
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  else
    static_cast<float*>(p)[i] = v;
}

// Eight consecutive activation elements starting at element i (i a multiple
// of 8, base pointer 16-byte aligned), widened to fp32.
template <int DT>
__device__ __forceinline__ void load_act8(const void* p, int64_t i, float (&x)[8]) {
  if constexpr (DT == RIA_DT_F32) {
    const f32x4* v = reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
    const f32x4 a = v[0], b = v[1];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = a[j];
      x[4 + j] = b[j];
    }
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t lo = static_cast<uint16_t>(w[j] & 0xffffu), hi = static_cast<uint16_t>(w[j] >> 16);
      if constexpr (DT == RIA_DT_BF16) {
        x[2 * j] = bf16_bits_to_f32(lo);
        x[2 * j + 1] = bf16_bits_to_f32(hi);
      } else {
        x[2 * j] = f16_bits_to_f32(lo);
        x[2 * j + 1] = f16_bits_to_f32(hi);
      }
    }
  }
}

// Four consecutive elements at i (a multiple of 4, base 16-byte aligned).
template <int DT>
__device__ __forceinline__ void load_act4(const void* p, int64_t i, float (&x)[4]) {
  if constexpr (DT == RIA_DT_F32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = a[j];
  } else {
    const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint16_t lo = static_cast<uint16_t>(w[j] & 0xffffu), hi = static_cast<uint16_t>(w[j] >> 16);
      if constexpr (DT == RIA_DT_BF16) {
        x[2 * j] = bf16_bits_to_f32(lo);
        x[2 * j + 1] = bf16_bits_to_f32(hi);
      } else {
        x[2 * j] = f16_bits_to_f32(lo);
        x[2 * j + 1] = f16_bits_to_f32(hi);
      }
    }
  }
}

// load_act4 with the dtype code known only at run time.
__device__ __forceinline__ void load_act4_dt(const void* p, int64_t i, int dt, float (&x)[4]) {
  if (dt == RIA_DT_BF16)
    load_act4<RIA_DT_BF16>(p, i, x);
  else if (dt == RIA_DT_F16)
    load_act4<RIA_DT_F16>(p, i, x);
  else
    load_act4<RIA_DT_F32>(p, i, x);
}

template <int DT>
__device__ __forceinline__ void store_act4(void* p, int64_t i, const float (&x)[4]) {
  if constexpr (DT == RIA_DT_F32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i) = f32x4{x[0], x[1], x[2], x[3]};
  } else {
    uint32_t w[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint16_t lo = DT == RIA_DT_BF16 ? f32_to_bf16_bits(x[2 * j]) : f32_to_f16_bits(x[2 * j]);
      const uint16_t hi = DT == RIA_DT_BF16 ? f32_to_bf16_bits(x[2 * j + 1]) : f32_to_f16_bits(x[2 * j + 1]);
      w[j] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    }
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p) + i) = u32x2{w[0], w[1]};
  }
}

// Value of an fp32 number after a round trip through dtype DT (torch `.to(dt)`).
template <int DT>
__device__ __forceinline__ float through_dtype(float v) {
  if constexpr (DT == RIA_DT_BF16) {
    return round_bf16(v);
  } else if constexpr (DT == RIA_DT_F16) {
    return f16_bits_to_f32(f32_to_f16_bits(v));
  } else {
    return v;
  }
}

// A rounded product / sum that is never fused with a neighbouring add or
// multiply into an FMA.  hipcc contracts by default (-ffp-contract=fast-
// honor-pragmas) and HIP's __fmul_rn / __fadd_rn are plain `*` / `+`, so the
// pragma is what keeps torch's separate roundings: it clears the contract
// flag on these operations, which survives inlining.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// torch.sigmoid / F.softplus(beta=1, threshold=20) / F.silu on fp32.
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// A float that rounds to the same bf16 as silu_f(x), for a bf16 value x (a
// post-conv activation), at a fraction of the accurate form's VALU cost.  For
// x > -16 the hardware exp2 and reciprocal put y within 14 fp32 ulps of
// silu_f(x) (measured over every bf16 input; most of it from rounding
// -x log2(e) before exp2, which grows with |x|: 3 ulps for -2 <= x < 0).
// Where y lies more than kSiluTieGuard ulps from a bf16 rounding midpoint
// (low 16 bits 0x8000) both round to the same bf16; lanes nearer a midpoint,
// about 1 in 1600, and x <= -16 or NaN take the accurate form.  Checked over
// all 65536 bf16 inputs.
constexpr uint32_t kSiluTieGuard = 20;
__device__ __forceinline__ float silu_to_bf16(float x) {
  const float y = x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504f));
  const uint32_t lo = (__float_as_uint(y) & 0xffffu) - (0x8000u - kSiluTieGuard);
  if (lo <= 2 * kSiluTieGuard || !(x > -16.0f)) return silu_f(x);
  return y;
}

// x sigmoid(g) as a float that rounds to the same bf16 as mul_rn(x,
// sigmoid_f(g)), for a bf16 gate g and any fp32 x.  For g > -16 the
// hardware exp2 and reciprocal put the sigmoid within 12 fp32 ulps of
// sigmoid_f(g) (measured over every bf16 gate), so the two products lie
// within 25 ulps of each other; where the product lies more than
// kGateTieGuard ulps from a bf16 rounding midpoint both round to the same
// bf16, and lanes nearer one, g <= -16 or NaN take the accurate form.
constexpr uint32_t kGateTieGuard = 32;
__device__ __forceinline__ float gate_mul_to_bf16(float x, float g) {
  const float y = mul_rn(x, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504f)));
  const uint32_t lo = (__float_as_uint(y) & 0xffffu) - (0x8000u - kGateTieGuard);
  if (lo <= 2 * kGateTieGuard || !(g > -16.0f)) return mul_rn(x, sigmoid_f(g));
  return y;
}

// RMSNorm pieces shared by the standalone and the fused forms.  eps is the
// model's 1e-6 (qwen36_op_probe.py:32, qwen36_gated_norm_probe.py:16).
constexpr float kNormEps = 1e-6f;

// 1 / sqrt(mean(x^2) + eps) from the row's sum of squares over n elements.
__device__ __forceinline__ float rms_scale(float sum_sq, int n, float eps = kNormEps) {
  return 1.0f / sqrtf(add_rn(__fdiv_rn(sum_sq, static_cast<float>(n)), eps));
}

// Qwen RMSNorm element (qwen36_op_probe.py:55-67): (x r)(1 + w) in fp32, cast
// back to the input dtype XT.
template <int XT>
__device__ __forceinline__ float rmsnorm_elem(float x, float r, float w) {
  return through_dtype<XT>(mul_rn(mul_rn(x, r), add_rn(1.0f, w)));
}

// Gated RMSNorm element (qwen36_gated_norm_probe.py:19-36): the normalised
// value is cast to the input dtype XT, scaled by w, gated by SiLU(z) in fp32,
// and the product cast to XT again.
template <int XT>
__device__ __forceinline__ float gated_norm_elem(float x, float r, float w, float z) {
  return through_dtype<XT>(mul_rn(mul_rn(w, through_dtype<XT>(mul_rn(x, r))), silu_f(z)));
}

// 16-bit KV element formats: conversion and the two MFMA shapes the decode
// kernel uses (16x16x32 with 8 operands per lane, 16x16x16 with 4).
template <int KVT>
struct Kv16;

template <>
struct Kv16<RIA_DT_BF16> {
  static __device__ __forceinline__ uint16_t from_f32(float f) { return f32_to_bf16_bits(f); }
  static __device__ __forceinline__ float to_f32(uint16_t b) { return bf16_bits_to_f32(b); }
  // two values rounded to nearest-even in one instruction: a in the low half
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  }
  static __device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  static __device__ __forceinline__ f32x4 mfma_k32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma_k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                     0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
};

template <>
struct Kv16<RIA_DT_F16> {
  static __device__ __forceinline__ uint16_t from_f32(float f) { return f32_to_f16_bits(f); }
  static __device__ __forceinline__ float to_f32(uint16_t b) { return f16_bits_to_f32(b); }
  // two values rounded to nearest-even in one instruction: a in the low half
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  }
  static __device__ __forceinline__ float lo_f32(uint32_t w) { return f16_bits_to_f32(static_cast<uint16_t>(w)); }
  static __device__ __forceinline__ float hi_f32(uint32_t w) { return f16_bits_to_f32(static_cast<uint16_t>(w >> 16)); }
  static __device__ __forceinline__ f32x4 mfma_k32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  }
  static __device__ __forceinline__ f32x4 mfma_k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  }
};

// Streaming loads/stores (non-temporal hint): data touched once per kernel.
// On MI355X they lift a pure read stream from ~6.1 to ~6.8 TB/s.
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ u32x2 ld_stream(const u32x2* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ f32x4 ld_stream(const f32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream(f32x4* p, f32x4 v) { __builtin_nontemporal_store(v, p); }

// Workgroup barrier for LDS traffic only: it waits for this wave's LDS (and
// scalar) operations but not for outstanding global loads or stores, which
// __syncthreads() would also drain (exposing prefetches and store latency).
// Word 3 of a raw buffer resource on gfx9-family parts: data format 32 bits
// (a zero format makes every load return zero), no swizzle, no index stride.
// Accesses past the resource's byte range are dropped (stores) or read zero.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over each half of the wavefront (lanes 0..31 and 32..63 separately),
// by ds_swizzle in xor mode: the lane pattern is an immediate, so no lane
// address registers stay live (pattern = and_mask 0x1f | xor_mask << 10).
__device__ __forceinline__ float half_wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (1 << 10)));
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (2 << 10)));
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (4 << 10)));
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (8 << 10)));
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (16 << 10)));
  return v;
}

}  // namespace ria

// Host-side error plumbing shared by every entry point (defined in abi.hip).
namespace ria {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
}  // namespace ria
