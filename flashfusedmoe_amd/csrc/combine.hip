// Bandwidth-bound kernels of the fused MoE layer: the weighted top-k combine
// (and its unweighted backward twin, the dX reduce), the routing backward,
// the standalone GLU kernels and the padded-layout row scatter.
#include <string>

#include "common.h"

namespace ffmoe {

__device__ __forceinline__ int src_row(int row) {
  return row >= 0 ? row : (row == FFMOE_ROW_ALIAS0 ? 0 : -1);
}

// out[n, 8v:8v+8] = sum_s w_s * rows[src(row_of[n*k+s]), 8v:8v+8], fp32 in
// slot order (moe_ops.py:156-203), then bf16; optional bf16 addend added after
// rounding (fused_moe.py:590).
__global__ __launch_bounds__(256) void combine_kernel(const bf16_t* __restrict__ rows,
                                                      const int32_t* __restrict__ row_of,
                                                      const float* __restrict__ topk_w,
                                                      const bf16_t* __restrict__ addend, int64_t N,
                                                      int D, int k, bf16_t* __restrict__ out) {
  const int nvec = D / 8;
  const int64_t total = N * nvec;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = u / nvec;
    const int v = static_cast<int>(u % nvec);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < k; ++s) {
      const int r = src_row(row_of[n * k + s]);
      if (r < 0) continue;
      const float w = topk_w != nullptr ? round_bf16(topk_w[n * k + s]) : 1.0f;
      float f[8];
      unpack8(reinterpret_cast<const uint4*>(rows + static_cast<int64_t>(r) * D)[v], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += w * f[i];
    }
    if (addend != nullptr) {
      float a[8];
      unpack8(reinterpret_cast<const uint4*>(addend + n * D)[v], a);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = round_bf16(acc[i]) + a[i];
    }
    reinterpret_cast<uint4*>(out + n * D)[v] = pack8(acc);
  }
}

// Routing backward, one wave per token n:
//   g_w[s] = <down[src_s], go[n]> (fp32)                 fused_moe.py:527-535
//   wgo[row_s] = bf16(go[n] * bf16(w_s)) for owned rows   moe_ops.py:248-288
//   g_tl = softmax / sigmoid top-k backward               fused_moe.py:573-584
//   gl[n,:] = scatter(g_tl) + d z_loss/dl + d aux/dl       :587-588, :1178-1194
template <int KMAX>
__global__ __launch_bounds__(256) void route_bwd_kernel(
    const bf16_t* __restrict__ go, const bf16_t* __restrict__ down,
    const int32_t* __restrict__ row_of, const int64_t* __restrict__ topk_idx,
    const float* __restrict__ topk_w, const bf16_t* __restrict__ logits,
    const float* __restrict__ lse, const int32_t* __restrict__ counts,
    const float* __restrict__ g_aux, const float* __restrict__ g_z, float aux_coeff, float z_coeff,
    int64_t N, int D, int E, int k, int gating, int capacity_mode, bf16_t* __restrict__ wgo,
    bf16_t* __restrict__ gl, float* __restrict__ grad_w) {
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (n >= N) return;
  const int nvec = D / 8;
  const uint4* gor = reinterpret_cast<const uint4*>(go + n * D);
  float gw[KMAX];
  float wsum = 0.0f;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    gw[s] = 0.0f;
    if (s >= k) continue;
    const int row = row_of[n * k + s];
    const int r = src_row(row);
    const float w = topk_w[n * k + s];
    wsum += w;
    const float wb = round_bf16(w);
    float dot = 0.0f;
    for (int v = lane; v < nvec; v += 64) {
      float g[8];
      unpack8(gor[v], g);
      if (r >= 0) {
        float d[8];
        unpack8(reinterpret_cast<const uint4*>(down + static_cast<int64_t>(r) * D)[v], d);
#pragma unroll
        for (int i = 0; i < 8; ++i) dot += d[i] * g[i];
      }
      if (row >= 0) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = g[i] * wb;
        reinterpret_cast<uint4*>(wgo + static_cast<int64_t>(row) * D)[v] = pack8(o);
      }
    }
    gw[s] = wave_sum(dot);
  }
  if (capacity_mode && !(wsum > 0.0f)) {
#pragma unroll
    for (int s = 0; s < KMAX; ++s) gw[s] = 0.0f;
  }
  // top-k backward (identical in every lane)
  float gtl[KMAX];
  int ids[KMAX];
  if (gating == FFMOE_GATING_SOFTMAX) {
    float sg = 0.0f;
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
      if (s < k) sg += gw[s] * topk_w[n * k + s];
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
      if (s < k) gtl[s] = topk_w[n * k + s] * (gw[s] - sg);
  } else {
    float tsum = 0.0f, gdw = 0.0f;
    float ts[KMAX];
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
      if (s < k) {
        const float l = bf16_to_f32(logits[n * E + topk_idx[n * k + s]]);
        ts[s] = 1.0f / (1.0f + expf(-l));
        tsum += ts[s];
        gdw += gw[s] * topk_w[n * k + s];
      }
    }
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
      if (s < k) gtl[s] = (gw[s] - gdw) / (tsum + 1e-6f) * ts[s] * (1.0f - ts[s]);
  }
#pragma unroll
  for (int s = 0; s < KMAX; ++s)
    if (s < k) ids[s] = static_cast<int>(topk_idx[n * k + s]);
  if (grad_w != nullptr && lane < k) {
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
      if (s == lane) grad_w[n * k + s] = gw[s];
  }
  const float zc = (g_z != nullptr) ? (*g_z) * z_coeff * 2.0f * lse[n] / static_cast<float>(N) : 0.0f;
  const float ac = (g_aux != nullptr && gating == FFMOE_GATING_SIGMOID)
                       ? (*g_aux) * aux_coeff * static_cast<float>(E) / static_cast<float>(N)
                       : 0.0f;
  for (int e = lane; e < E; e += 64) {
    float g = 0.0f;
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
      if (s < k && ids[s] == e) g += gtl[s];
    if (zc != 0.0f || ac != 0.0f) {
      const float l = bf16_to_f32(logits[n * E + e]);
      if (zc != 0.0f) g += zc * expf(l - lse[n]);
      if (ac != 0.0f) {
        const float sg = 1.0f / (1.0f + expf(-l));
        g += ac * (static_cast<float>(counts[e]) / static_cast<float>(N)) * sg * (1.0f - sg);
      }
    }
    gl[n * E + e] = f32_to_bf16(g);
  }
}

__global__ __launch_bounds__(256) void glu_fwd_kernel(const bf16_t* __restrict__ up, int64_t M,
                                                      int H, int act, bf16_t* __restrict__ out) {
  const int hv = H / 8;
  const int64_t total = M * hv;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t m = u / hv;
    const int v = static_cast<int>(u % hv);
    float g[8], x[8], o[8];
    unpack8(reinterpret_cast<const uint4*>(up + m * 2 * H)[v], g);
    unpack8(reinterpret_cast<const uint4*>(up + m * 2 * H + H)[v], x);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = glu_fwd(act, g[i], x[i]);
    reinterpret_cast<uint4*>(out + m * H)[v] = pack8(o);
  }
}

__global__ __launch_bounds__(256) void glu_bwd_kernel(const bf16_t* __restrict__ ga,
                                                      const bf16_t* __restrict__ up, int64_t M,
                                                      int H, int act, bf16_t* __restrict__ gup) {
  const int hv = H / 8;
  const int64_t total = M * hv;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t m = u / hv;
    const int v = static_cast<int>(u % hv);
    float a[8], g[8], x[8], og[8], ou[8];
    unpack8(reinterpret_cast<const uint4*>(ga + m * H)[v], a);
    unpack8(reinterpret_cast<const uint4*>(up + m * 2 * H)[v], g);
    unpack8(reinterpret_cast<const uint4*>(up + m * 2 * H + H)[v], x);
#pragma unroll
    for (int i = 0; i < 8; ++i) glu_bwd(act, a[i], g[i], x[i], &og[i], &ou[i]);
    reinterpret_cast<uint4*>(gup + m * 2 * H)[v] = pack8(og);
    reinterpret_cast<uint4*>(gup + m * 2 * H + H)[v] = pack8(ou);
  }
}

__global__ __launch_bounds__(256) void scatter_rows_kernel(const bf16_t* __restrict__ src,
                                                           const int64_t* __restrict__ dst_row,
                                                           const float* __restrict__ w,
                                                           int64_t n_entries, int k, int D,
                                                           int64_t dst_rows,
                                                           bf16_t* __restrict__ dst) {
  const int nvec = D / 8;
  const int64_t total = n_entries * nvec;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t j = u / nvec;
    const int v = static_cast<int>(u % nvec);
    const int64_t r = dst_row[j];
    if (r < 0 || r >= dst_rows) continue;
    uint4 val = reinterpret_cast<const uint4*>(src + (j / k) * D)[v];
    if (w != nullptr) {
      float f[8];
      unpack8(val, f);
      const float wb = round_bf16(w[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] *= wb;
      val = pack8(f);
    }
    reinterpret_cast<uint4*>(dst + r * D)[v] = val;
  }
}

static inline unsigned grid_for(int64_t units) {
  int64_t b = (units + 255) / 256;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return static_cast<unsigned>(b);
}

}  // namespace ffmoe

using namespace ffmoe;

extern "C" int ffmoe_combine(const void* rows, const int32_t* row_of, const float* topk_w,
                             const void* addend, int64_t N, int D, int k, void* out, void* stream) {
  if (N <= 0 || D <= 0 || D % 8 != 0) return set_error("ffmoe_combine: D must be a positive multiple of 8");
  if (k < 1 || k > FFMOE_MAX_TOPK) return set_error("ffmoe_combine: bad k");
  hipLaunchKernelGGL(combine_kernel, dim3(grid_for(N * (D / 8))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const bf16_t*>(rows), row_of,
                     topk_w, static_cast<const bf16_t*>(addend), N, D, k, static_cast<bf16_t*>(out));
  if (check_launch("combine_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_route_bwd(const void* go, const void* down, const int32_t* row_of,
                               const int64_t* topk_idx, const float* topk_w, const void* logits,
                               const float* lse, const int32_t* counts, const float* g_aux,
                               const float* g_z, float aux_coeff, float z_coeff, int64_t N, int D,
                               int E, int k, int gating, int capacity_mode, void* wgo,
                               void* grad_logits, float* grad_w, void* stream) {
  if (N <= 0 || D <= 0 || D % 8 != 0) return set_error("ffmoe_route_bwd: D must be a positive multiple of 8");
  if (k < 1 || k > FFMOE_MAX_TOPK || E < 1 || E > FFMOE_MAX_EXPERTS)
    return set_error("ffmoe_route_bwd: bad k/E");
  if ((g_z != nullptr || gating == FFMOE_GATING_SIGMOID || g_aux != nullptr) && logits == nullptr)
    return set_error("ffmoe_route_bwd: logits required");
  if (g_z != nullptr && lse == nullptr) return set_error("ffmoe_route_bwd: lse required");
  if (g_aux != nullptr && counts == nullptr) return set_error("ffmoe_route_bwd: counts required");
  const dim3 grid(static_cast<unsigned>((N + 3) / 4));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define FFMOE_RB(KM)                                                                            \
  hipLaunchKernelGGL(route_bwd_kernel<KM>, grid, dim3(256), 0, st,                              \
                     static_cast<const bf16_t*>(go), static_cast<const bf16_t*>(down), row_of,  \
                     topk_idx, topk_w, static_cast<const bf16_t*>(logits), lse, counts, g_aux,  \
                     g_z, aux_coeff, z_coeff, N, D, E, k, gating, capacity_mode,                \
                     static_cast<bf16_t*>(wgo), static_cast<bf16_t*>(grad_logits), grad_w)
  if (k <= 2)
    FFMOE_RB(2);
  else if (k <= 4)
    FFMOE_RB(4);
  else if (k <= 8)
    FFMOE_RB(8);
  else
    FFMOE_RB(16);
#undef FFMOE_RB
  if (check_launch("route_bwd_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_glu_fwd(const void* up, int64_t M, int H, int activation, void* act,
                             void* stream) {
  if (M < 0 || H <= 0 || H % 8 != 0) return set_error("ffmoe_glu_fwd: H must be a positive multiple of 8");
  if (activation < 0 || activation > 2) return set_error("ffmoe_glu_fwd: unknown activation");
  if (M == 0) return clear_error();
  hipLaunchKernelGGL(glu_fwd_kernel, dim3(grid_for(M * (H / 8))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const bf16_t*>(up), M, H,
                     activation, static_cast<bf16_t*>(act));
  if (check_launch("glu_fwd_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_glu_bwd(const void* grad_act, const void* up, int64_t M, int H, int activation,
                             void* grad_up, void* stream) {
  if (M < 0 || H <= 0 || H % 8 != 0) return set_error("ffmoe_glu_bwd: H must be a positive multiple of 8");
  if (activation < 0 || activation > 2) return set_error("ffmoe_glu_bwd: unknown activation");
  if (M == 0) return clear_error();
  hipLaunchKernelGGL(glu_bwd_kernel, dim3(grid_for(M * (H / 8))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const bf16_t*>(grad_act),
                     static_cast<const bf16_t*>(up), M, H, activation, static_cast<bf16_t*>(grad_up));
  if (check_launch("glu_bwd_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_scatter_rows(const void* src, const int64_t* dst_row, const float* w,
                                  int64_t n_entries, int k, int D, int64_t dst_rows, void* dst,
                                  void* stream) {
  if (n_entries < 0 || k < 1 || D <= 0 || D % 8 != 0)
    return set_error("ffmoe_scatter_rows: D must be a positive multiple of 8");
  if (n_entries == 0) return clear_error();
  hipLaunchKernelGGL(scatter_rows_kernel, dim3(grid_for(n_entries * (D / 8))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const bf16_t*>(src), dst_row, w,
                     n_entries, k, D, dst_rows, static_cast<bf16_t*>(dst));
  if (check_launch("scatter_rows_kernel")) return 1;
  return clear_error();
}
