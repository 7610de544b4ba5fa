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

__device__ __forceinline__ float erf_as(float value) {
  float sign = value < 0.0f ? -1.0f : 1.0f;
  float x = fabsf(value);
  float t = fast_rcp(fmaf(x, 0.3275911f, 1.0f));
  float poly = t * (0.2548296f + t * (-0.28449672f + t * (1.4214138f + t * (-1.4531521f + t * 1.0614054f))));
  return sign * (1.0f - poly * fast_exp(-x * x));
}

__device__ __forceinline__ float act_apply(int act, float v) {
  switch (act) {
    case ACT_RELU: return fmaxf(v, 0.0f);
    case ACT_GELU: return 0.5f * v * (1.0f + erf_as(v * 0.70710678118654752f));
    case ACT_SILU: return v * fast_rcp(1.0f + fast_exp(-v));
    case ACT_HSIG6: return fminf(fmaxf(fmaf(v, 1.0f / 6.0f, 0.5f), 0.0f), 1.0f);
    case ACT_HSIG5: return fminf(fmaxf(fmaf(v, 0.2f, 0.5f), 0.0f), 1.0f);
    case ACT_HSWISH: return v * fminf(fmaxf(v * (1.0f / 6.0f) + 0.5f, 0.0f), 1.0f);
    case ACT_SIGMOID: return fast_rcp(1.0f + fast_exp(-v));
    default: return v;
  }
}

// x + x*g with the reference's two roundings (src/cpu/kernels/mod.rs:790-795).
__device__ __forceinline__ float residual_mul(float x, float g) { return __fadd_rn(__fmul_rn(x, g), x); }

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

}  // namespace ppocr
