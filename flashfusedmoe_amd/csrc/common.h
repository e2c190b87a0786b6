// Shared device helpers for the ffmoe HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

#include <string>

#include "../../include/ffmoe.h"

namespace ffmoe {

typedef uint16_t bf16_t;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Records `msg` as this thread's last error and returns 1.
int set_error(const std::string& msg);
// Clears the last error and returns 0.
int clear_error();
// Checks hipGetLastError() after a launch; returns 0 or records the failure.
int check_launch(const char* what);

// The gate-gradient product dgate [E, D] = gl^T x on the MFMA GEMM pipeline
// (gemm.hip), for expert counts beyond the fused dot2 kernel's: K split over
// the tokens, fp32 partials (gate_grad_mfma_split(N, D, E) slabs of E*D
// floats in `workspace`) reduced in a fixed order.
int gate_grad_mfma_split(int64_t N, int D, int E);
int gate_grad_mfma(const void* gl, const void* x, int64_t N, int D, int E, void* workspace, int64_t ws_bytes,
                   void* dgate, void* stream);

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 -> bf16, the rounding torch uses for
// .to(torch.bfloat16) (NaN stays a quiet NaN).  gfx950 does it in hardware
// (v_cvt_pk_bf16_f32, two values per instruction); a branchy software
// version costs ~12 instructions with exec-mask changes per value.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Unpack 8 bf16 held in a uint4 (16 bytes) to fp32.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Logistic sigmoid from the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32: about 1 ulp each in fp32, far below the bf16 rounding every GLU
// result goes through).  Saturates cleanly: 1/(1 + inf) = 0.
__device__ __forceinline__ float fast_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// GLU activations in fp32 (the reference computes them in fp32 from bf16
// operands, activations.py:27-142).  tanh is taken as 2*sigmoid(2z) - 1
// (activations.py:21-24).  The activation is a template argument so that
// hot loops carry no per-element branch; with_act() dispatches a runtime
// activation id once.
template <int ACT>
__device__ __forceinline__ float glu_fwd_t(float g, float u) {
  if constexpr (ACT == FFMOE_ACT_SWIGLU) {
    return g * fast_sigmoid(g) * u;
  } else if constexpr (ACT == FFMOE_ACT_GEGLU) {
    const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    const float th = 2.0f * fast_sigmoid(2.0f * inner) - 1.0f;
    return 0.5f * g * (1.0f + th) * u;
  } else if constexpr (ACT == FFMOE_ACT_GEGLU_ERF) {
    return 0.5f * g * (1.0f + erff(g * 0.7071067811865476f)) * u;
  } else {
    const float r = g > 0.0f ? g : 0.0f;
    return r * r * u;
  }
}

// d(act)/d(gate), d(act)/d(up) scaled by the upstream grad `ga`.
template <int ACT>
__device__ __forceinline__ void glu_bwd_t(float ga, float g, float u, float* gg, float* gu) {
  if constexpr (ACT == FFMOE_ACT_SWIGLU) {
    const float s = fast_sigmoid(g);
    *gu = ga * g * s;
    *gg = ga * u * (s * (1.0f + g * (1.0f - s)));
  } else if constexpr (ACT == FFMOE_ACT_GEGLU) {
    const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    const float th = 2.0f * fast_sigmoid(2.0f * inner) - 1.0f;
    const float gelu = 0.5f * g * (1.0f + th);
    const float dinner = 0.7978845608028654f * (1.0f + 3.0f * 0.044715f * g * g);
    const float dgelu = 0.5f * (1.0f + th) + 0.5f * g * (1.0f - th * th) * dinner;
    *gu = ga * gelu;
    *gg = ga * u * dgelu;
  } else if constexpr (ACT == FFMOE_ACT_GEGLU_ERF) {
    // d/dg [g * Phi(g)] = Phi(g) + g * phi(g)
    const float cdf = 0.5f * (1.0f + erff(g * 0.7071067811865476f));
    const float pdf = 0.3989422804014327f * __expf(-0.5f * g * g);
    *gu = ga * g * cdf;
    *gg = ga * u * (cdf + g * pdf);
  } else {
    const float r = g > 0.0f ? g : 0.0f;
    *gu = ga * r * r;
    *gg = ga * u * 2.0f * r;
  }
}

// Calls f(std::integral_constant<int, ACT>) for a runtime activation id.
template <class F>
__device__ __forceinline__ void with_act(int act, F&& f) {
  if (act == FFMOE_ACT_SWIGLU)
    f(std::integral_constant<int, FFMOE_ACT_SWIGLU>{});
  else if (act == FFMOE_ACT_GEGLU)
    f(std::integral_constant<int, FFMOE_ACT_GEGLU>{});
  else if (act == FFMOE_ACT_GEGLU_ERF)
    f(std::integral_constant<int, FFMOE_ACT_GEGLU_ERF>{});
  else
    f(std::integral_constant<int, FFMOE_ACT_RELU2>{});
}

__device__ __forceinline__ float glu_fwd(int act, float g, float u) {
  float r = 0.0f;
  with_act(act, [&](auto a) { r = glu_fwd_t<decltype(a)::value>(g, u); });
  return r;
}

__device__ __forceinline__ void glu_bwd(int act, float ga, float g, float u, float* gg, float* gu) {
  with_act(act, [&](auto a) { glu_bwd_t<decltype(a)::value>(ga, g, u, gg, gu); });
}

}  // namespace ffmoe
