// Bandwidth-bound kernels of the fused MoE layer: the weighted top-k combine
// (and its unweighted backward twin, the dX reduce), the routing backward,
// the standalone GLU kernels and the padded-layout row scatter.
#include <mutex>
#include <string>

#include "common.h"

namespace ffmoe {

__device__ __forceinline__ int src_row(int row) {
  return row >= 0 ? row : (row == FFMOE_ROW_ALIAS0 ? 0 : -1);
}

// Gathers of k rows per token.  A thread owns U 16-byte vectors of one token
// (v0 + j * nvec/U, j < U): it reads the token's k row indices once, then
// issues every slot's loads before the first add, so k*U loads are in flight
// per thread instead of one dependent pair per slot.
template <int KMAX, int U>
__device__ __forceinline__ void gather_rows(const bf16_t* __restrict__ rows,
                                            const int32_t* __restrict__ row_of, int64_t n, int k,
                                            int nvec, int v0, int nq, int* r, uint4 (*val)[U]) {
#pragma unroll
  for (int s = 0; s < KMAX; ++s) r[s] = s < k ? src_row(row_of[n * k + s]) : -1;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
#pragma unroll
    for (int j = 0; j < U; ++j) {
      val[s][j] = make_uint4(0, 0, 0, 0);
      if (r[s] >= 0)
        val[s][j] = reinterpret_cast<const uint4*>(rows + static_cast<int64_t>(r[s]) * (nvec * 8))[v0 + j * nq];
    }
  }
}

// out[n, 8v:8v+8] = sum_s w_s * rows[src(row_of[n*k+s]), 8v:8v+8], fp32 in
// slot order (moe_ops.py:156-203), then bf16; optional bf16 addend added after
// rounding (fused_moe.py:590).
template <int KMAX, int U>
__global__ __launch_bounds__(256) void combine_kernel(const bf16_t* __restrict__ rows,
                                                      const int32_t* __restrict__ row_of,
                                                      const float* __restrict__ topk_w,
                                                      const bf16_t* __restrict__ addend, int64_t N,
                                                      int D, int k, bf16_t* __restrict__ out) {
  const int nvec = D / 8;
  const int nq = nvec / U;
  const int64_t total = N * nq;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = u / nq;
    const int v0 = static_cast<int>(u % nq);
    int r[KMAX];
    uint4 val[KMAX][U];
    float w[KMAX];
#pragma unroll
    for (int s = 0; s < KMAX; ++s)
      w[s] = (s < k && topk_w != nullptr) ? round_bf16(topk_w[n * k + s]) : 1.0f;
    gather_rows<KMAX, U>(rows, row_of, n, k, nvec, v0, nq, r, val);
    uint4 av[U];
    if (addend != nullptr) {
#pragma unroll
      for (int j = 0; j < U; ++j) av[j] = reinterpret_cast<const uint4*>(addend + n * D)[v0 + j * nq];
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KMAX; ++s) {
        if (r[s] < 0) continue;
        float f[8];
        unpack8(val[s][j], f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += w[s] * f[i];
      }
      if (addend != nullptr) {
        float a[8];
        unpack8(av[j], a);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = round_bf16(acc[i]) + a[i];
      }
      reinterpret_cast<uint4*>(out + n * D)[v0 + j * nq] = pack8(acc);
    }
  }
}

// dX reduce with the gate-gradient term fused (E <= FFMOE_MAX_FUSED_GATE_E):
//   out[n] = bf16(bf16(sum_s ghb[src(row_of[n*k+s])]) + bf16(gl[n,:] . gate))
// The sum over slots is fp32 in slot order (moe_ops.py:156-241 with unit
// weights, fused_moe.py:556-561); the gl . gate product is fp32 over experts
// in index order, two experts per v_dot2c_f32_bf16 (each bf16 product is
// exact in fp32), rounded to bf16 as the reference's bf16 `gl @ gate` GEMM
// output is (fused_moe.py:590).  The slot rows are gathered with all their
// loads in flight, the gate rows (L2-resident) four expert pairs at a time.
template <int KMAX>
__global__ __launch_bounds__(256) void dx_reduce_kernel(const bf16_t* __restrict__ rows,
                                                        const int32_t* __restrict__ row_of,
                                                        const bf16_t* __restrict__ gl,
                                                        const bf16_t* __restrict__ gate, int64_t N,
                                                        int D, int E, int k,
                                                        bf16_t* __restrict__ out) {
  constexpr int PB = 4;  // expert pairs per batch of loads
  const int nvec = D / 8;
  const int64_t total = N * nvec;
  const int EP = E / 2;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = u / nvec;
    const int v = static_cast<int>(u % nvec);
    int r[KMAX];
    uint4 val[KMAX][1];
    gather_rows<KMAX, 1>(rows, row_of, n, k, nvec, v, 0, r, val);
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int p0 = 0; p0 < EP; p0 += PB) {
      uint32_t gp[PB];
      uint4 g0[PB], g1[PB];
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        const int pr = p0 + q;
        const bool ok = pr < EP;
        // with an even E, pair pr of gl row n is 4-byte aligned
        const bf16_t* gpp = gl + n * E + 2 * pr;
        gp[q] = !ok ? 0u
                    : (E & 1) ? (static_cast<uint32_t>(gpp[0]) | (static_cast<uint32_t>(gpp[1]) << 16))
                              : *reinterpret_cast<const uint32_t*>(gpp);
        g0[q] = ok ? reinterpret_cast<const uint4*>(gate + static_cast<int64_t>(2 * pr) * D)[v]
                   : make_uint4(0, 0, 0, 0);
        g1[q] = ok ? reinterpret_cast<const uint4*>(gate + static_cast<int64_t>(2 * pr + 1) * D)[v]
                   : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        if (p0 + q >= EP) break;
        const bf16x2_t gv = __builtin_bit_cast(bf16x2_t, gp[q]);
        const uint32_t w0[4] = {g0[q].x, g0[q].y, g0[q].z, g0[q].w};
        const uint32_t w1[4] = {g1[q].x, g1[q].y, g1[q].z, g1[q].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // columns 2j, 2j+1 of experts 2pr (low half) and 2pr+1 (high half)
          const uint32_t lo = (w0[j] & 0xffffu) | (w1[j] << 16);
          const uint32_t hi = (w0[j] >> 16) | (w1[j] & 0xffff0000u);
          a[2 * j] = __builtin_amdgcn_fdot2_f32_bf16(gv, __builtin_bit_cast(bf16x2_t, lo), a[2 * j], false);
          a[2 * j + 1] =
              __builtin_amdgcn_fdot2_f32_bf16(gv, __builtin_bit_cast(bf16x2_t, hi), a[2 * j + 1], false);
        }
      }
    }
    if (E & 1) {  // the last expert of an odd count
      const float g = bf16_to_f32(gl[n * E + E - 1]);
      float w[8];
      unpack8(reinterpret_cast<const uint4*>(gate + static_cast<int64_t>(E - 1) * D)[v], w);
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] += g * w[i];
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
      if (r[s] < 0) continue;
      float f[8];
      unpack8(val[s][0], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += f[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = round_bf16(acc[i]) + round_bf16(a[i]);
    reinterpret_cast<uint4*>(out + n * D)[v] = pack8(acc);
  }
}

// Gate weight gradient dgate[E, D] = gl^T x (fused_moe.py:591), E <=
// FFMOE_MAX_FUSED_GATE_E.  Pass 1: a block takes a kGateCols-column slice of
// kGateChunk tokens.  Thread (row group rg, vector cv) owns 8 columns and the
// tokens rg, rg + 16, ...: its x loads are all issued at once (the block's
// 32 KiB x tile is in flight together, two blocks per CU), its gl loads per
// batch of 8 experts.  Per batch the 16 row groups are added in row-group order
// through LDS into one fp32 partial per block.  Pass 2 sums the partials in
// a fixed order and rounds to bf16.  x is read once; deterministic.
constexpr int kGateChunk = 128;
constexpr int kGateCols = 128;
constexpr int kGateGroups = 256 / (kGateCols / 8);  // row groups per block
constexpr int kGateTok = kGateChunk / kGateGroups;  // tokens per thread

// GL8: E is a multiple of 8 (each batch of 8 experts of a gl row is one
// aligned 16-byte load and the product runs on bf16 dot2 over token pairs).
template <bool GL8>
__global__ __launch_bounds__(256) void gate_grad_partial_kernel(const bf16_t* __restrict__ gl,
                                                                const bf16_t* __restrict__ x,
                                                                int64_t N, int D, int E,
                                                                float* __restrict__ part) {
  static_assert(kGateTok % 2 == 0, "token pairs");
  __shared__ float4 s_red[kGateGroups][8][kGateCols / 4];
  const int tid = threadIdx.x;
  const int rg = tid / (kGateCols / 8), cv = tid % (kGateCols / 8);
  const int cbase = blockIdx.x * kGateCols;
  const int col = cbase + cv * 8;
  const int64_t chunk = blockIdx.y;
  const int64_t n0 = chunk * kGateChunk;
  const int nt = static_cast<int>(min<int64_t>(kGateChunk, N - n0));
  const bool col_ok = col < D;  // D % 8 == 0: a vector is wholly in or out
  uint4 xv[kGateTok];
#pragma unroll
  for (int j = 0; j < kGateTok; ++j) {
    const int t = rg + j * kGateGroups;
    xv[j] = (col_ok && t < nt) ? *reinterpret_cast<const uint4*>(x + (n0 + t) * D + col)
                               : make_uint4(0, 0, 0, 0);
  }
  for (int eb = 0; eb < E; eb += 8) {
    float acc[8][8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[q][i] = 0.0f;
    if constexpr (GL8) {
      uint4 gp[kGateTok];
#pragma unroll
      for (int j = 0; j < kGateTok; ++j) {
        const int t = rg + j * kGateGroups;
        gp[j] = t < nt ? *reinterpret_cast<const uint4*>(gl + (n0 + t) * E + eb) : make_uint4(0, 0, 0, 0);
      }
      // two tokens per v_dot2c_f32_bf16: (gl[t][e], gl[t'][e]) . (x[t][c], x[t'][c]),
      // each bf16 product exact in fp32; tokens past the chunk hold zeros
#pragma unroll
      for (int j = 0; j < kGateTok; j += 2) {
        const uint32_t x0[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
        const uint32_t x1[4] = {xv[j + 1].x, xv[j + 1].y, xv[j + 1].z, xv[j + 1].w};
        const uint32_t g0[4] = {gp[j].x, gp[j].y, gp[j].z, gp[j].w};
        const uint32_t g1[4] = {gp[j + 1].x, gp[j + 1].y, gp[j + 1].z, gp[j + 1].w};
        bf16x2_t xp[8], gq[8];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          xp[2 * w] = __builtin_bit_cast(bf16x2_t, (x0[w] & 0xffffu) | (x1[w] << 16));
          xp[2 * w + 1] = __builtin_bit_cast(bf16x2_t, (x0[w] >> 16) | (x1[w] & 0xffff0000u));
          gq[2 * w] = __builtin_bit_cast(bf16x2_t, (g0[w] & 0xffffu) | (g1[w] << 16));
          gq[2 * w + 1] = __builtin_bit_cast(bf16x2_t, (g0[w] >> 16) | (g1[w] & 0xffff0000u));
        }
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[q][i] = __builtin_amdgcn_fdot2_f32_bf16(gq[q], xp[i], acc[q][i], false);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kGateTok; ++j) {
        const int t = rg + j * kGateGroups;
        float g[8], xf[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          g[q] = (t < nt && eb + q < E) ? bf16_to_f32(gl[(n0 + t) * E + eb + q]) : 0.0f;
        unpack8(xv[j], xf);
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[q][i] += g[q] * xf[i];
      }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      s_red[rg][q][cv * 2] = make_float4(acc[q][0], acc[q][1], acc[q][2], acc[q][3]);
      s_red[rg][q][cv * 2 + 1] = make_float4(acc[q][4], acc[q][5], acc[q][6], acc[q][7]);
    }
    __syncthreads();
    {  // 8 experts x 128 columns, 4 per thread; row groups added in order
      const int q = tid / (kGateCols / 4), c4 = tid % (kGateCols / 4);
      float4 r = s_red[0][q][c4];
#pragma unroll
      for (int w = 1; w < kGateGroups; ++w) {
        const float4 v = s_red[w][q][c4];
        r.x += v.x;
        r.y += v.y;
        r.z += v.z;
        r.w += v.w;
      }
      if (eb + q < E && cbase + c4 * 4 < D)
        *reinterpret_cast<float4*>(part + (chunk * E + eb + q) * static_cast<int64_t>(D) + cbase + c4 * 4) = r;
    }
    __syncthreads();
  }
}

// Pass 2: 16 output quads (4 consecutive outputs) per block, 16 threads per
// quad; thread j sums parts j, j + 16, ... in order (all its loads in
// flight), then the 16 sums are added in j order.
constexpr int kGateFinalLoads = 8;

__global__ __launch_bounds__(256) void gate_grad_final_kernel(const float* __restrict__ part,
                                                              int64_t nparts, int D, int E,
                                                              bf16_t* __restrict__ out) {
  __shared__ float4 s[16][16];
  const int tid = threadIdx.x;
  const int oq = tid >> 4, j = tid & 15;
  const int64_t total = static_cast<int64_t>(E) * D;  // a multiple of 8
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 16 + oq) * 4;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i < total) {
    for (int64_t c0 = j; c0 < nparts; c0 += 16 * kGateFinalLoads) {
      float4 v[kGateFinalLoads];
#pragma unroll
      for (int u = 0; u < kGateFinalLoads; ++u) {
        const int64_t c = c0 + 16 * u;
        v[u] = c < nparts ? *reinterpret_cast<const float4*>(part + c * total + i) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < kGateFinalLoads; ++u) {
        if (c0 + 16 * u >= nparts) break;
        acc.x += v[u].x;
        acc.y += v[u].y;
        acc.z += v[u].z;
        acc.w += v[u].w;
      }
    }
  }
  s[oq][j] = acc;
  __syncthreads();
  if (j == 0 && i < total) {
    float4 r = s[oq][0];
    for (int q = 1; q < 16; ++q) {
      r.x += s[oq][q].x;
      r.y += s[oq][q].y;
      r.z += s[oq][q].z;
      r.w += s[oq][q].w;
    }
    *reinterpret_cast<uint2*>(out + i) = make_uint2(pack_bf16x2(r.x, r.y), pack_bf16x2(r.z, r.w));
  }
}

// The aux loss's routing when its gradient flows through the routing weights:
// the reference's slow routing path (any of expert_bias, pre_softmax,
// scoring_factor, n_group) computes the aux-loss weights with differentiable
// torch ops (fused_moe.py:144-200, :1165-1189), softmax gating only.
struct AuxRoute {
  int through_weights;     // 1: add d aux / d logits through the weights
  const int64_t* idx;      // the aux routing's top-k [N,k] (null: the dispatch routing)
  const int32_t* counts;   // its per-expert counts (null: `counts`)
  int pre_softmax;         // weights were renormalised softmax probabilities
  float scoring;           // > 0: weights were scaled by scoring / top_k
};

// Routing backward, one wave per token n:
//   g_w[s] = <down[src_s], go[n]> (fp32)                 fused_moe.py:527-535
//   wgo[row_s] = T(go[n] * T(w_s)) for owned rows         moe_ops.py:248-288
//   g_tl = softmax / sigmoid top-k backward               fused_moe.py:573-584
//   gl[n,:] = scatter(g_tl) + d z_loss/dl + d aux/dl       :587-588, :1178-1194
// T is the compute dtype: bf16 (16-byte vectors, bf16 logits) or fp32 /
// fp64 (element-wise, fp32 logits: the reference's top-k and losses read
// logits.float()); products and the top-k backward are fp32 either way, as
// the reference's Triton kernels and fp32 routing tensors are.
template <typename T> struct LogitOf { using type = float; };
template <> struct LogitOf<bf16_t> { using type = bf16_t; };
__device__ __forceinline__ float to_f32(bf16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(double v) { return static_cast<float>(v); }
template <typename T> __device__ __forceinline__ T from_f32(float f) { return static_cast<T>(f); }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float f) { return f32_to_bf16(f); }

template <int KMAX, typename T = bf16_t>
__global__ __launch_bounds__(256) void route_bwd_kernel(
    const T* __restrict__ go, const T* __restrict__ down,
    const int32_t* __restrict__ row_of, const int64_t* __restrict__ topk_idx,
    const float* __restrict__ topk_w, const typename LogitOf<T>::type* __restrict__ logits,
    const float* __restrict__ lse, const int32_t* __restrict__ counts,
    const float* __restrict__ g_aux, const float* __restrict__ g_z, float aux_coeff, float z_coeff,
    int64_t N, int D, int E, int k, int gating, int capacity_mode, AuxRoute ar,
    T* __restrict__ wgo, T* __restrict__ gl, float* __restrict__ grad_w) {
  constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (n >= N) return;
  // every slot's row index and weight first; then, per chunk of VC vectors
  // per lane, the go vectors and every slot's down vectors are all in flight
  // before the first product (per slot, the lane still adds its vectors in
  // increasing order)
  constexpr int VC = KMAX <= 4 ? 2 : 1;
  int rowv[KMAX], rsrc[KMAX];
  float wb[KMAX], dot[KMAX], gw[KMAX];
  float wsum = 0.0f;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    rowv[s] = -1;
    rsrc[s] = -1;
    wb[s] = 0.0f;
    dot[s] = 0.0f;
    if (s < k) {
      rowv[s] = row_of[n * k + s];
      rsrc[s] = src_row(rowv[s]);
      const float w = topk_w[n * k + s];
      wsum += w;
      wb[s] = kBf16 ? round_bf16(w) : w;  // topk_w.to(dtype), then fp32 in the kernel
    }
  }
  if constexpr (!kBf16) {
    for (int d = lane; d < D; d += 64) {
      const float g = to_f32(go[n * D + d]);
#pragma unroll
      for (int s = 0; s < KMAX; ++s) {
        if (rsrc[s] >= 0) dot[s] += to_f32(down[static_cast<int64_t>(rsrc[s]) * D + d]) * g;
        if (rowv[s] >= 0) wgo[static_cast<int64_t>(rowv[s]) * D + d] = static_cast<T>(g * wb[s]);
      }
    }
  } else {
  const int nvec = D / 8;
  const uint4* gor = reinterpret_cast<const uint4*>(go + n * D);
  for (int v0 = lane; v0 < nvec; v0 += 64 * VC) {
    uint4 gv[VC], dv[KMAX][VC];
#pragma unroll
    for (int j = 0; j < VC; ++j) {
      const int v = v0 + 64 * j;
      gv[j] = v < nvec ? gor[v] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int s = 0; s < KMAX; ++s)
        dv[s][j] = (rsrc[s] >= 0 && v < nvec)
                       ? reinterpret_cast<const uint4*>(down + static_cast<int64_t>(rsrc[s]) * D)[v]
                       : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < VC; ++j) {
      const int v = v0 + 64 * j;
      if (v >= nvec) continue;
      float g[8];
      unpack8(gv[j], g);
#pragma unroll
      for (int s = 0; s < KMAX; ++s) {
        if (rsrc[s] >= 0) {
          float d[8];
          unpack8(dv[s][j], d);
#pragma unroll
          for (int i = 0; i < 8; ++i) dot[s] += d[i] * g[i];
        }
        if (rowv[s] >= 0) {
          float o[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = g[i] * wb[s];
          reinterpret_cast<uint4*>(wgo + static_cast<int64_t>(rowv[s]) * D)[v] = pack8(o);
        }
      }
    }
  }
  }
#pragma unroll
  for (int s = 0; s < KMAX; ++s) gw[s] = s < k ? wave_sum(dot[s]) : 0.0f;
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
        const float l = to_f32(logits[n * E + topk_idx[n * k + s]]);
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
  // aux loss through the routing weights: d aux / d w[s] = g * c * E * f_e / N
  // with f_e = counts[e] / N, back through the weight formula
  float aux_sel[KMAX];  // contribution to gl at aux_ids[s] (softmax over selected)
  int aux_ids[KMAX];
  float aux_dp[KMAX];   // pre-softmax: d aux / d p at aux_ids[s]
  float aux_t = 0.0f;   // pre-softmax: sum_s p_s dp_s
  const bool aux_w = ar.through_weights && g_aux != nullptr && gating == FFMOE_GATING_SOFTMAX;
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    aux_sel[s] = 0.0f;
    aux_dp[s] = 0.0f;
    aux_ids[s] = -1;
  }
  if (aux_w) {
    const int64_t* ai = ar.idx != nullptr ? ar.idx : topk_idx;
    const int32_t* ac = ar.counts != nullptr ? ar.counts : counts;
    const float A = (*g_aux) * aux_coeff * static_cast<float>(E) / static_cast<float>(N);
    const float a = ar.scoring > 0.0f ? ar.scoring / static_cast<float>(k) : 1.0f;
    float ga[KMAX], l[KMAX];
    float mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
      ga[s] = 0.0f;
      l[s] = 0.0f;
      if (s < k) {
        aux_ids[s] = static_cast<int>(ai[n * k + s]);
        ga[s] = A * (static_cast<float>(ac[aux_ids[s]]) / static_cast<float>(N));
        l[s] = to_f32(logits[n * E + aux_ids[s]]);
        mx = fmaxf(mx, l[s]);
      }
    }
    if (!ar.pre_softmax) {  // w = a * softmax(selected logits)
      float ws[KMAX], z = 0.0f, sg = 0.0f;
#pragma unroll
      for (int s = 0; s < KMAX; ++s) {
        ws[s] = s < k ? expf(l[s] - mx) : 0.0f;
        z += ws[s];
      }
#pragma unroll
      for (int s = 0; s < KMAX; ++s) {
        ws[s] /= z;
        sg += ws[s] * a * ga[s];
      }
#pragma unroll
      for (int s = 0; s < KMAX; ++s)
        if (s < k) aux_sel[s] = ws[s] * (a * ga[s] - sg);
    } else {  // w = a * p_sel / (sum p_sel + 1e-6), p = softmax over all experts
      float p[KMAX], S = 0.0f, gp = 0.0f;
#pragma unroll
      for (int s = 0; s < KMAX; ++s) {
        p[s] = s < k ? expf(l[s] - lse[n]) : 0.0f;
        S += p[s];
        gp += ga[s] * p[s];
      }
      const float d = S + 1e-6f;
#pragma unroll
      for (int s = 0; s < KMAX; ++s) {
        if (s < k) {
          aux_dp[s] = a * (ga[s] / d - gp / (d * d));
          aux_t += p[s] * aux_dp[s];
        }
      }
    }
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
    if (aux_w) {
      if (!ar.pre_softmax) {
#pragma unroll
        for (int s = 0; s < KMAX; ++s)
          if (s < k && aux_ids[s] == e) g += aux_sel[s];
      } else {
        float dp = 0.0f;
#pragma unroll
        for (int s = 0; s < KMAX; ++s)
          if (s < k && aux_ids[s] == e) dp += aux_dp[s];
        g += expf(to_f32(logits[n * E + e]) - lse[n]) * (dp - aux_t);
      }
    }
    if (zc != 0.0f || ac != 0.0f) {
      const float l = to_f32(logits[n * E + e]);
      if (zc != 0.0f) g += zc * expf(l - lse[n]);
      if (ac != 0.0f) {
        const float sg = 1.0f / (1.0f + expf(-l));
        g += ac * (static_cast<float>(counts[e]) / static_cast<float>(N)) * sg * (1.0f - sg);
      }
    }
    gl[n * E + e] = from_f32<T>(g);
  }
}

template <int ACT>
__global__ __launch_bounds__(256) void glu_fwd_kernel(const bf16_t* __restrict__ up, int64_t M,
                                                      int H, bf16_t* __restrict__ out) {
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
    for (int i = 0; i < 8; ++i) o[i] = glu_fwd_t<ACT>(g[i], x[i]);
    reinterpret_cast<uint4*>(out + m * H)[v] = pack8(o);
  }
}

template <int ACT>
__global__ __launch_bounds__(256) void glu_bwd_kernel(const bf16_t* __restrict__ ga,
                                                      const bf16_t* __restrict__ up, int64_t M,
                                                      int H, bf16_t* __restrict__ gup) {
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
    for (int i = 0; i < 8; ++i) glu_bwd_t<ACT>(a[i], g[i], x[i], &og[i], &ou[i]);
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

// The reference's padded routing scatter (moe_ops.py:43-106): sorted
// position p names entry j = sorted_order[p] of expert e = flat_ids[j] with
// rank p - starts[e]; an entry of rank < mt gets e2b[j] = e*mt + rank and
// its token's row x[j / k] is copied to out[e2b[j]].  Entries of rank >= mt
// are skipped (their e2b keeps the caller's zero).  Indices outside their
// tensors are skipped too, so malformed routing cannot address memory
// outside the buffers.  One 16-byte vector per thread, grid-stride.
__global__ __launch_bounds__(256) void routing_scatter_kernel(
    const int64_t* __restrict__ sorted_order, const int64_t* __restrict__ flat_ids,
    const int64_t* __restrict__ starts, const bf16_t* __restrict__ x, int64_t n_sorted, int64_t NK,
    int D, int E, int64_t mt, int k, bf16_t* __restrict__ out, int64_t* __restrict__ e2b) {
  const int nvec = D / 8;
  const int64_t total = n_sorted * nvec;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t p = u / nvec;
    const int v = static_cast<int>(u % nvec);
    const int64_t j = sorted_order[p];
    if (j < 0 || j >= NK) continue;
    const int64_t e = flat_ids[j];
    if (e < 0 || e >= E) continue;
    const int64_t rank = p - starts[e];
    if (rank < 0 || rank >= mt) continue;
    const int64_t pos = e * mt + rank;
    if (v == 0) e2b[j] = pos;
    reinterpret_cast<uint4*>(out + pos * D)[v] = reinterpret_cast<const uint4*>(x + (j / k) * D)[v];
  }
}

}  // namespace ffmoe

using namespace ffmoe;

extern "C" int ffmoe_routing_scatter_padded(const int64_t* sorted_order, const int64_t* flat_ids,
                                            const int64_t* starts, const void* x, int64_t N, int D,
                                            int E, int64_t mt, int k, int64_t n_sorted, void* out,
                                            int64_t* e2b, void* stream) {
  if (N < 0 || D <= 0 || D % 8 != 0)
    return set_error("ffmoe_routing_scatter_padded: D must be a positive multiple of 8");
  if (E < 1 || k < 1 || mt < 0 || n_sorted < 0 || n_sorted > N * k)
    return set_error("ffmoe_routing_scatter_padded: bad E, k, max_tokens or num_sorted");
  if (n_sorted == 0) return clear_error();
  hipLaunchKernelGGL(routing_scatter_kernel, dim3(grid_for(n_sorted * (D / 8))), dim3(256), 0,
                     static_cast<hipStream_t>(stream), sorted_order, flat_ids, starts,
                     static_cast<const bf16_t*>(x), n_sorted, N * k, D, E, mt, k,
                     static_cast<bf16_t*>(out), e2b);
  if (check_launch("routing_scatter_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_t_routing_scatter_padded(int dtype, const int64_t* sorted_order, const int64_t* flat_ids,
                                              const int64_t* starts, const void* x, int64_t N, int D, int E,
                                              int64_t mt, int k, int64_t n_sorted, void* out, int64_t* e2b,
                                              void* stream) {
  // a row copy: rows of D fp32 / fp64 elements are moved as 2D / 4D bf16-sized units
  const int units = dtype == FFMOE_DTYPE_F32 ? 2 : dtype == FFMOE_DTYPE_F64 ? 4 : 0;
  if (units == 0) return set_error("ffmoe_t_routing_scatter_padded: dtype must be FFMOE_DTYPE_F32 or FFMOE_DTYPE_F64");
  if (D <= 0 || D % 8 != 0 || static_cast<int64_t>(D) * units > 0x7fffffff)
    return set_error("ffmoe_t_routing_scatter_padded: D must be a positive multiple of 8");
  return ffmoe_routing_scatter_padded(sorted_order, flat_ids, starts, x, N, D * units, E, mt, k, n_sorted, out,
                                      e2b, stream);
}

extern "C" int ffmoe_combine(const void* rows, const int32_t* row_of, const float* topk_w,
                             const void* addend, int64_t N, int D, int k, void* out, void* stream) {
  if (N <= 0 || D <= 0 || D % 8 != 0) return set_error("ffmoe_combine: D must be a positive multiple of 8");
  if (k < 1 || k > FFMOE_MAX_TOPK) return set_error("ffmoe_combine: bad k");
  const int nvec = D / 8;
  const bool two = nvec % 2 == 0 && k <= 8;  // two vectors per thread
  const unsigned grid = grid_for(N * (two ? nvec / 2 : nvec));
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto rb = static_cast<const bf16_t*>(rows);
  auto ab = static_cast<const bf16_t*>(addend);
  auto ob = static_cast<bf16_t*>(out);
#define FFMOE_CB(KM, U) \
  hipLaunchKernelGGL((combine_kernel<KM, U>), dim3(grid), dim3(256), 0, st, rb, row_of, topk_w, ab, N, D, k, ob)
  if (two) {
    if (k <= 2) FFMOE_CB(2, 2);
    else if (k <= 4) FFMOE_CB(4, 2);
    else FFMOE_CB(8, 2);
  } else {
    if (k <= 2) FFMOE_CB(2, 1);
    else if (k <= 4) FFMOE_CB(4, 1);
    else if (k <= 8) FFMOE_CB(8, 1);
    else FFMOE_CB(16, 1);
  }
#undef FFMOE_CB
  if (check_launch("combine_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_dx_reduce(const void* ghb, const int32_t* row_of, const void* gl,
                               const void* gate, int64_t N, int D, int E, int k, void* out,
                               void* stream) {
  if (N <= 0 || D <= 0 || D % 8 != 0) return set_error("ffmoe_dx_reduce: D must be a positive multiple of 8");
  if (k < 1 || k > FFMOE_MAX_TOPK) return set_error("ffmoe_dx_reduce: bad k");
  if (E < 1 || E > FFMOE_MAX_FUSED_GATE_E) return set_error("ffmoe_dx_reduce: E out of range");
  const dim3 grid(grid_for(N * (D / 8)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto rb = static_cast<const bf16_t*>(ghb);
  auto gb = static_cast<const bf16_t*>(gl);
  auto wb = static_cast<const bf16_t*>(gate);
  auto ob = static_cast<bf16_t*>(out);
#define FFMOE_DX(KM) \
  hipLaunchKernelGGL((dx_reduce_kernel<KM>), grid, dim3(256), 0, st, rb, row_of, gb, wb, N, D, E, k, ob)
  if (k <= 2) FFMOE_DX(2);
  else if (k <= 4) FFMOE_DX(4);
  else if (k <= 8) FFMOE_DX(8);
  else FFMOE_DX(16);
#undef FFMOE_DX
  if (check_launch("dx_reduce_kernel")) return 1;
  return clear_error();
}

extern "C" int64_t ffmoe_gate_grad_workspace_bytes(int64_t N, int D, int E) {
  if (N <= 0 || D <= 0 || E <= 0) return 0;
  if (E > FFMOE_MAX_FUSED_GATE_E) {  // MFMA path: one fp32 [E, D] slab per K split
    const int S = gate_grad_mfma_split(N, D, E);
    return S > 1 ? static_cast<int64_t>(S) * E * D * 4 : 0;
  }
  return ((N + kGateChunk - 1) / kGateChunk) * static_cast<int64_t>(E) * D * 4;
}

static int gate_grad_check(const char* name, int64_t N, int D, int E) {
  if (N <= 0 || D <= 0 || D % 8 != 0) return set_error(std::string(name) + ": D must be a positive multiple of 8");
  if (E < 1 || E > FFMOE_MAX_EXPERTS) return set_error(std::string(name) + ": E out of range");
  if (E > FFMOE_MAX_FUSED_GATE_E && (E % 8 != 0 || N > 0x7fffffff))
    return set_error(std::string(name) + ": above 32 experts E must be a multiple of 8");
  if ((N + kGateChunk - 1) / kGateChunk > 65535)
    return set_error(std::string(name) + ": N too large (at most 8388480 tokens)");
  return 0;
}

// Both passes of the gate-weight gradient with the fp32 partials in
// `workspace` (ffmoe_gate_grad_workspace_bytes(N, D, E) bytes, every byte
// written by pass 1 before pass 2 reads it: nothing needs clearing).
static int gate_grad_launch(const void* gl, const void* x, int64_t N, int D, int E, void* workspace,
                            void* dgate, void* stream) {
  if (E > FFMOE_MAX_FUSED_GATE_E)
    return gate_grad_mfma(gl, x, N, D, E, workspace, ffmoe_gate_grad_workspace_bytes(N, D, E), dgate, stream);
  const int64_t nchunk = (N + kGateChunk - 1) / kGateChunk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const dim3 grid(static_cast<unsigned>((D + kGateCols - 1) / kGateCols), static_cast<unsigned>(nchunk));
  if (E % 8 == 0)
    hipLaunchKernelGGL(gate_grad_partial_kernel<true>, grid, dim3(256), 0, st, static_cast<const bf16_t*>(gl),
                       static_cast<const bf16_t*>(x), N, D, E, part);
  else
    hipLaunchKernelGGL(gate_grad_partial_kernel<false>, grid, dim3(256), 0, st, static_cast<const bf16_t*>(gl),
                       static_cast<const bf16_t*>(x), N, D, E, part);
  if (check_launch("gate_grad_partial_kernel")) return 1;
  const int64_t total = static_cast<int64_t>(E) * D;
  hipLaunchKernelGGL(gate_grad_final_kernel, dim3(static_cast<unsigned>((total / 4 + 15) / 16)),
                     dim3(256), 0, st, part, nchunk, D, E, static_cast<bf16_t*>(dgate));
  if (check_launch("gate_grad_final_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_gate_grad(const void* gl, const void* x, int64_t N, int D, int E,
                               void* workspace, void* dgate, void* stream) {
  if (gate_grad_check("ffmoe_gate_grad", N, D, E)) return 1;
  return gate_grad_launch(gl, x, N, D, E, workspace, dgate, stream);
}

// Scratch of the allocation-free variant: the fp32 partials live in this
// file-scope device array instead of a caller's workspace.  Each device the
// library runs on holds its own copy until the process ends; its address on
// a device comes from hipGetSymbolAddress (the array's name in host code is
// only a stand-in), looked up once per device on the first call there.
constexpr int64_t kGateGradScratchBytes = 32ll << 20;
static __device__ __align__(256) float scratch[kGateGradScratchBytes / 4];

static void* g_scratch_ptr[64];
static std::mutex g_scratch_mu;

static void* scratch_ptr(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

extern "C" int64_t ffmoe_gate_grad_noalloc_max_bytes(void) { return kGateGradScratchBytes; }

extern "C" int ffmoe_gate_grad_noalloc(const void* gl, const void* x, int64_t N, int D, int E,
                                       void* dgate, void* stream) {
  if (gate_grad_check("ffmoe_gate_grad_noalloc", N, D, E)) return 1;
  const int64_t need = ffmoe_gate_grad_workspace_bytes(N, D, E);
  if (need > kGateGradScratchBytes)
    return set_error("ffmoe_gate_grad_noalloc: needs " + std::to_string(need) +
                     " bytes of scratch (ceil(N/128)*E*D*4); the allocation-free variant holds at most " +
                     std::to_string(kGateGradScratchBytes) + " (use ffmoe_gate_grad with a workspace)");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error("ffmoe_gate_grad_noalloc: cannot query the current device");
  void* ptr = scratch_ptr(dev);
  if (ptr == nullptr) return set_error("ffmoe_gate_grad_noalloc: hipGetSymbolAddress failed for the scratch array");
  return gate_grad_launch(gl, x, N, D, E, ptr, dgate, stream);
}

static int route_bwd_impl(const void* go, const void* down, const int32_t* row_of,
                          const int64_t* topk_idx, const float* topk_w, const void* logits,
                          const float* lse, const int32_t* counts, const float* g_aux,
                          const float* g_z, float aux_coeff, float z_coeff, int64_t N, int D, int E,
                          int k, int gating, int capacity_mode, AuxRoute ar, void* wgo,
                          void* grad_logits, float* grad_w, void* stream) {
  if (N <= 0 || D <= 0 || D % 8 != 0) return set_error("ffmoe_route_bwd: D must be a positive multiple of 8");
  if (k < 1 || k > FFMOE_MAX_TOPK || E < 1 || E > FFMOE_MAX_EXPERTS)
    return set_error("ffmoe_route_bwd: bad k/E");
  if ((g_z != nullptr || gating == FFMOE_GATING_SIGMOID || g_aux != nullptr) && logits == nullptr)
    return set_error("ffmoe_route_bwd: logits required");
  if ((g_z != nullptr || (ar.through_weights && ar.pre_softmax)) && lse == nullptr)
    return set_error("ffmoe_route_bwd: lse required");
  if (g_aux != nullptr && counts == nullptr) return set_error("ffmoe_route_bwd: counts required");
  const dim3 grid(static_cast<unsigned>((N + 3) / 4));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define FFMOE_RB(KM)                                                                            \
  hipLaunchKernelGGL(route_bwd_kernel<KM>, grid, dim3(256), 0, st,                              \
                     static_cast<const bf16_t*>(go), static_cast<const bf16_t*>(down), row_of,  \
                     topk_idx, topk_w, static_cast<const bf16_t*>(logits), lse, counts, g_aux,  \
                     g_z, aux_coeff, z_coeff, N, D, E, k, gating, capacity_mode, ar,            \
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

namespace ffmoe {

template <typename T>
static void route_bwd_t_k(int k, dim3 grid, hipStream_t st, const void* go, const void* down,
                          const int32_t* row_of, const int64_t* topk_idx, const float* topk_w,
                          const float* logits, const float* lse, const int32_t* counts, const float* g_aux,
                          const float* g_z, float aux_coeff, float z_coeff, int64_t N, int D, int E,
                          int gating, int capacity_mode, const AuxRoute& ar, void* wgo, void* gl,
                          float* grad_w) {
#define FFMOE_RBT(KM)                                                                                 \
  hipLaunchKernelGGL((route_bwd_kernel<KM, T>), grid, dim3(256), 0, st, static_cast<const T*>(go),    \
                     static_cast<const T*>(down), row_of, topk_idx, topk_w, logits, lse, counts, g_aux, \
                     g_z, aux_coeff, z_coeff, N, D, E, k, gating, capacity_mode, ar,                   \
                     static_cast<T*>(wgo), static_cast<T*>(gl), grad_w)
  if (k <= 2)
    FFMOE_RBT(2);
  else if (k <= 4)
    FFMOE_RBT(4);
  else if (k <= 8)
    FFMOE_RBT(8);
  else
    FFMOE_RBT(16);
#undef FFMOE_RBT
}

int route_bwd_t_launch(int dtype, const void* go, const void* down, const int32_t* row_of,
                       const int64_t* topk_idx, const float* topk_w, const float* logits, const float* lse,
                       const int32_t* counts, const float* g_aux, const float* g_z, float aux_coeff,
                       float z_coeff, int64_t N, int D, int E, int k, int gating, int capacity_mode,
                       int aux_through, const int64_t* aux_idx, const int32_t* aux_counts, int pre_softmax,
                       float scoring, void* wgo, void* gl, float* grad_w, hipStream_t st) {
  if (g_aux != nullptr && counts == nullptr) return set_error("ffmoe_t_route_bwd: counts required");
  const AuxRoute ar{aux_through, aux_idx, aux_counts, pre_softmax, scoring};
  const dim3 grid(static_cast<unsigned>((N + 3) / 4));
  if (dtype == FFMOE_DTYPE_F32)
    route_bwd_t_k<float>(k, grid, st, go, down, row_of, topk_idx, topk_w, logits, lse, counts, g_aux, g_z,
                         aux_coeff, z_coeff, N, D, E, gating, capacity_mode, ar, wgo, gl, grad_w);
  else
    route_bwd_t_k<double>(k, grid, st, go, down, row_of, topk_idx, topk_w, logits, lse, counts, g_aux, g_z,
                          aux_coeff, z_coeff, N, D, E, gating, capacity_mode, ar, wgo, gl, grad_w);
  if (check_launch("route_bwd_kernel")) return 1;
  return clear_error();
}

}  // namespace ffmoe

extern "C" int ffmoe_route_bwd(const void* go, const void* down, const int32_t* row_of,
                               const int64_t* topk_idx, const float* topk_w, const void* logits,
                               const float* lse, const int32_t* counts, const float* g_aux,
                               const float* g_z, float aux_coeff, float z_coeff, int64_t N, int D,
                               int E, int k, int gating, int capacity_mode, void* wgo,
                               void* grad_logits, float* grad_w, void* stream) {
  const AuxRoute ar{0, nullptr, nullptr, 0, 0.0f};
  return route_bwd_impl(go, down, row_of, topk_idx, topk_w, logits, lse, counts, g_aux, g_z,
                        aux_coeff, z_coeff, N, D, E, k, gating, capacity_mode, ar, wgo,
                        grad_logits, grad_w, stream);
}

extern "C" int ffmoe_route_bwd_ex(const void* go, const void* down, const int32_t* row_of,
                                  const int64_t* topk_idx, const float* topk_w, const void* logits,
                                  const float* lse, const int32_t* counts, const float* g_aux,
                                  const float* g_z, float aux_coeff, float z_coeff, int64_t N,
                                  int D, int E, int k, int gating, int capacity_mode,
                                  int aux_through_weights, const int64_t* aux_topk_idx,
                                  const int32_t* aux_counts, int pre_softmax,
                                  float scoring_factor, void* wgo, void* grad_logits,
                                  float* grad_w, void* stream) {
  const AuxRoute ar{aux_through_weights, aux_topk_idx, aux_counts, pre_softmax, scoring_factor};
  return route_bwd_impl(go, down, row_of, topk_idx, topk_w, logits, lse, counts, g_aux, g_z,
                        aux_coeff, z_coeff, N, D, E, k, gating, capacity_mode, ar, wgo,
                        grad_logits, grad_w, stream);
}

extern "C" int ffmoe_glu_fwd(const void* up, int64_t M, int H, int activation, void* act,
                             void* stream) {
  if (M < 0 || H <= 0 || H % 8 != 0) return set_error("ffmoe_glu_fwd: H must be a positive multiple of 8");
  if (activation < 0 || activation > FFMOE_ACT_GEGLU_ERF) return set_error("ffmoe_glu_fwd: unknown activation");
  if (M == 0) return clear_error();
  const dim3 grid(grid_for(M * (H / 8)));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bf16_t* u = static_cast<const bf16_t*>(up);
  bf16_t* o = static_cast<bf16_t*>(act);
  switch (activation) {
    case FFMOE_ACT_SWIGLU: hipLaunchKernelGGL(glu_fwd_kernel<FFMOE_ACT_SWIGLU>, grid, dim3(256), 0, st, u, M, H, o); break;
    case FFMOE_ACT_GEGLU: hipLaunchKernelGGL(glu_fwd_kernel<FFMOE_ACT_GEGLU>, grid, dim3(256), 0, st, u, M, H, o); break;
    case FFMOE_ACT_RELU2: hipLaunchKernelGGL(glu_fwd_kernel<FFMOE_ACT_RELU2>, grid, dim3(256), 0, st, u, M, H, o); break;
    default: hipLaunchKernelGGL(glu_fwd_kernel<FFMOE_ACT_GEGLU_ERF>, grid, dim3(256), 0, st, u, M, H, o); break;
  }
  if (check_launch("glu_fwd_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_glu_bwd(const void* grad_act, const void* up, int64_t M, int H, int activation,
                             void* grad_up, void* stream) {
  if (M < 0 || H <= 0 || H % 8 != 0) return set_error("ffmoe_glu_bwd: H must be a positive multiple of 8");
  if (activation < 0 || activation > FFMOE_ACT_GEGLU_ERF) return set_error("ffmoe_glu_bwd: unknown activation");
  if (M == 0) return clear_error();
  const dim3 grid(grid_for(M * (H / 8)));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bf16_t* ga = static_cast<const bf16_t*>(grad_act);
  const bf16_t* u = static_cast<const bf16_t*>(up);
  bf16_t* o = static_cast<bf16_t*>(grad_up);
  switch (activation) {
    case FFMOE_ACT_SWIGLU: hipLaunchKernelGGL(glu_bwd_kernel<FFMOE_ACT_SWIGLU>, grid, dim3(256), 0, st, ga, u, M, H, o); break;
    case FFMOE_ACT_GEGLU: hipLaunchKernelGGL(glu_bwd_kernel<FFMOE_ACT_GEGLU>, grid, dim3(256), 0, st, ga, u, M, H, o); break;
    case FFMOE_ACT_RELU2: hipLaunchKernelGGL(glu_bwd_kernel<FFMOE_ACT_RELU2>, grid, dim3(256), 0, st, ga, u, M, H, o); break;
    default: hipLaunchKernelGGL(glu_bwd_kernel<FFMOE_ACT_GEGLU_ERF>, grid, dim3(256), 0, st, ga, u, M, H, o); break;
  }
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
