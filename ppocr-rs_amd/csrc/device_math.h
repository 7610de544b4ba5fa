// Device-side scalar numerics shared by the kernels.
//
// The formulas are the reference CPU path's (src/cpu/kernels/mod.rs:2376-2403):
// GELU uses the Abramowitz-Stegun 7.1.26 erf approximation, written out from
// that published method.  Epilogues run these once per output element, so
// the exponential is the hardware exp2 (v_exp_f32) on x*log2(e) and the
// reciprocals are v_rcp_f32: each is within a few ulp of the correctly
// rounded value, far inside the 1e-3 output tolerance, and several times
// cheaper than the IEEE-exact library forms.
#pragma once

#include <hip/hip_runtime.h>

#include "kernels.h"

namespace ppocr {

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Raw buffer access: vector memory instructions through a buffer resource,
// with a 32-bit lane offset and a wave-uniform offset in a scalar register
// (no 64-bit address per access), range-checked by the hardware: loads past
// the resource's size return zero and stores there are dropped.
typedef int int32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2v __attribute__((ext_vector_type(2)));

// Raw buffer resource over `bytes` bytes at `base` (stride 0, 32-bit
// format): the descriptor of the gfx9 family.
__device__ __forceinline__ int32x4_t buffer_resource(const void* base, unsigned bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  int32x4_t r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xFFFFu));
  r.z = __builtin_amdgcn_readfirstlane((int)bytes);
  r.w = 0x00020000;
  return r;
}
__device__ f32x2v llvm_raw_buffer_load_v2f32(int32x4_t rsrc, int voffset, int soffset,
                                             int aux) __asm("llvm.amdgcn.raw.buffer.load.v2f32");
__device__ void llvm_raw_buffer_store_v2f32(f32x2v v, int32x4_t rsrc, int voffset, int soffset,
                                            int aux) __asm("llvm.amdgcn.raw.buffer.store.v2f32");

// Merges two partial softmax reductions (max m, sum of exp(x - m), last index
// of the max) into (m, s, i).  Empty partials (s == 0, m = -inf) contribute
// nothing; equal maxima keep the larger index.
__device__ __forceinline__ void lse_merge(float& m, float& s, int& i, float om, float os, int oi) {
  const float nm = fmaxf(m, om);
  const float a = s == 0.0f ? 0.0f : s * fast_exp(m - nm);
  const float b = os == 0.0f ? 0.0f : os * fast_exp(om - nm);
  i = om > m ? oi : (om < m ? i : max(i, oi));
  m = nm;
  s = a + b;
}

// GELU(v) = v/2 (1 + erf(v / sqrt 2)) with the A-S 7.1.26 erf: for
// x = |v| / sqrt 2, t = 1 / (1 + p x) and E = poly(t) exp(-x^2),
// erf(v / sqrt 2) = sign(v) (1 - E).  With h = v/2, h sign(v) = |h|, so
// GELU(v) = h + |h| (1 - E): one fused multiply-add and an add in place of
// the sign select and three products.  The 1/sqrt 2 scaling is folded into
// the constants (p / sqrt 2 in the t denominator; the exp2 argument
// x^2 log2(e) is y^2 with y = |v| sqrt(log2(e) / 2)).  Fourteen vector
// operations per element, two of them transcendental, one of them the
// clamp: at v = +inf, E is 0 and |h| infinite, so the product's factor is
// clamped to the largest finite float, -|h| E is 0 rather than NaN, and the
// result is +inf, as v/2 (1 + erf) gives (at -inf both forms give NaN).
__device__ __forceinline__ float gelu_as(float v) {
  const float a = fabsf(v);
  const float t = fast_rcp(fmaf(a, 0.3275911f * 0.70710678118654752f, 1.0f));
  const float poly = t * (0.2548296f + t * (-0.28449672f + t * (1.4214138f + t * (-1.4531521f + t * 1.0614054f))));
  const float y = a * 0.84932180028801904f;
  const float e = poly * __builtin_amdgcn_exp2f(-(y * y));
  const float h = 0.5f * v, ha = fabsf(h);
  return h + fmaf(-fminf(ha, 3.40282347e38f), e, ha);
}

__device__ __forceinline__ float act_apply(int act, float v) {
  switch (act) {
    case ACT_RELU: return fmaxf(v, 0.0f);
    case ACT_GELU: return gelu_as(v);
    case ACT_SILU: return v * fast_rcp(1.0f + fast_exp(-v));
    case ACT_HSIG6: return fminf(fmaxf(fmaf(v, 1.0f / 6.0f, 0.5f), 0.0f), 1.0f);
    case ACT_HSIG5: return fminf(fmaxf(fmaf(v, 0.2f, 0.5f), 0.0f), 1.0f);
    case ACT_HSWISH: return v * fminf(fmaxf(v * (1.0f / 6.0f) + 0.5f, 0.0f), 1.0f);
    case ACT_SIGMOID: return fast_rcp(1.0f + fast_exp(-v));
    default: return v;
  }
}

// x * y rounded to fp32 on its own.  Device code is compiled with FMA
// contraction allowed; the pragma keeps this product out of any fused
// multiply-add with a later sum (the reference rounds it first).
__device__ __forceinline__ float mul_rn(float x, float y) {
#pragma clang fp contract(off)
  return x * y;
}

// x + x*g with the reference's two roundings (src/cpu/kernels/mod.rs:790-795).
__device__ __forceinline__ float residual_mul(float x, float g) {
#pragma clang fp contract(off)
  return x * g + x;
}

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// ---- activation storage: fp32 or bf16 (round-to-nearest-even on store).
typedef __bf16 bf16;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// lo and hi rounded to bf16 and packed as (hi << 16) | lo: one
// v_cvt_pk_bf16_f32, which rounds to nearest even (denormals kept) and
// keeps a NaN a NaN, so non-finite values still reach the output checks.
// (Its results equal the integer form (u + 0x7FFF + ((u >> 16) & 1)) >> 16,
// with NaN mapped to a quiet NaN, on all 2^32 inputs.)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return pack_bf16x2(f, 0.0f) & 0xFFFFu; }

// Four bf16 values packed low half first in a and b, as floats.
__device__ __forceinline__ float4 unpack_bf16x4(uint32_t a, uint32_t b) {
  return make_float4(__uint_as_float(a << 16), __uint_as_float(a & 0xFFFF0000u), __uint_as_float(b << 16),
                     __uint_as_float(b & 0xFFFF0000u));
}

// v rounded to the storage type T (what st4 stores and ld4 reads back).
template <typename T>
__device__ __forceinline__ float4 round4(float4 v);
template <>
__device__ __forceinline__ float4 round4<float>(float4 v) {
  return v;
}
template <>
__device__ __forceinline__ float4 round4<bf16>(float4 v) {
  const uint32_t a = pack_bf16x2(v.x, v.y), b = pack_bf16x2(v.z, v.w);
  return make_float4(__uint_as_float(a << 16), __uint_as_float(a & 0xFFFF0000u), __uint_as_float(b << 16),
                     __uint_as_float(b & 0xFFFF0000u));
}

// Four consecutive values (16 B as fp32, 8 B as bf16).
template <typename T>
__device__ __forceinline__ float4 ld4(const T* p);
template <>
__device__ __forceinline__ float4 ld4<float>(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
template <>
__device__ __forceinline__ float4 ld4<bf16>(const bf16* p) {
  uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(bf16_bits_to_f32(u.x & 0xFFFFu), bf16_bits_to_f32(u.x >> 16), bf16_bits_to_f32(u.y & 0xFFFFu),
                     bf16_bits_to_f32(u.y >> 16));
}

template <typename T>
__device__ __forceinline__ void st4(T* p, float4 v);
template <>
__device__ __forceinline__ void st4<float>(float* p, float4 v) {
  *reinterpret_cast<float4*>(p) = v;
}
template <>
__device__ __forceinline__ void st4<bf16>(bf16* p, float4 v) {
  uint2 u;
  u.x = pack_bf16x2(v.x, v.y);
  u.y = pack_bf16x2(v.z, v.w);
  *reinterpret_cast<uint2*>(p) = u;
}

template <typename T>
__device__ __forceinline__ float ld1(const T* p);
template <>
__device__ __forceinline__ float ld1<float>(const float* p) {
  return *p;
}
template <>
__device__ __forceinline__ float ld1<bf16>(const bf16* p) {
  return bf16_bits_to_f32(*reinterpret_cast<const unsigned short*>(p));
}

template <typename T>
__device__ __forceinline__ void st1(T* p, float v);
template <>
__device__ __forceinline__ void st1<float>(float* p, float v) {
  *p = v;
}
template <>
__device__ __forceinline__ void st1<bf16>(bf16* p, float v) {
  *reinterpret_cast<unsigned short*>(p) = (unsigned short)f32_to_bf16_bits(v);
}

__device__ __forceinline__ float4 f4_mul(float4 a, float4 b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}

}  // namespace ppocr
