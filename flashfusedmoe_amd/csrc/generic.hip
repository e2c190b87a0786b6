// fp32 / fp64 compute path of the fused MoE layer.
//
// The reference computes in the input dtype when autocast is off
// (fused_moe.py:93-97, :318-327): its GEMMs are torch.bmm in that dtype and
// its Triton kernels (GLU, gather-reduce, weighted scatter, top-k) load their
// operands, compute in fp32 and store in that dtype (activations.py:58-74,
// moe_ops.py:190-203, :283-288, fused_topk.py:52).  This file holds the
// kernels of that path: a grouped / dense GEMM with fp32 (or fp64)
// accumulation, the routed GLU in fp32 (the shared expert's in the compute
// dtype, as its torch ops run, nn.py:31-40), the top-k combine and the
// routing-weight gradient with weighted scatter.  Routing itself (top-k,
// weights, statistics, permutation) reuses the bf16 path's kernels on fp32
// logits and row bytes.
//
// The GEMM is LDS-tiled on the vector ALUs (64x64 output tiles, 16-deep K
// slices, 4x4 outputs per thread): it is a generality path, sized for
// correctness at the reference's fp32 / fp64 test and C1 shapes, not the
// MFMA pipeline of the bf16 path.
#include "common.h"

namespace ffmoe {

namespace {

constexpr int kTB = 64;   // tile rows / columns
constexpr int kTK = 16;   // K slice
constexpr int kTThreads = 256;

template <typename T> struct AccOf { using type = float; };
template <> struct AccOf<double> { using type = double; };

// A(m, k) = A[m * sam + k * sak], B(k, n) = B[k * sbk + n * sbn],
// C(m, n) = C[m * ldc + n].  Modes:
//  0 dense: group g = blockIdx.z, operands offset by g * {a,b,c}_gs;
//  1 grouped rows: row tiles of BM = kTB per group from tile_offsets, the
//    group's rows offsets[e] .. offsets[e+1] of A and C, B offset by e * b_gs;
//  2 grouped K: group e = blockIdx.z reduces over rows offsets[e] ..
//    offsets[e+1] (the K index), C offset by e * c_gs.
struct GemmT {
  const void* A;
  const void* B;
  void* C;
  int64_t sam, sak, sbk, sbn, ldc;
  int64_t a_gs, b_gs, c_gs;
  int M, N, K;
  const int32_t* offsets;
  const int32_t* tile_offsets;
  int E;
  int n_tiles;
};

template <typename T, typename TO, int MODE>
__global__ __launch_bounds__(kTThreads) void gemm_t_kernel(GemmT p) {
  using TA = typename AccOf<T>::type;
  __shared__ T As[kTK][kTB + 1];
  __shared__ T Bs[kTK][kTB + 1];
  const int tid = threadIdx.x;
  const int tx = tid % 16, ty = tid / 16;
  const T* A = static_cast<const T*>(p.A);
  const T* B = static_cast<const T*>(p.B);
  TO* C = static_cast<TO*>(p.C);
  int nt = static_cast<int>(blockIdx.x % p.n_tiles);
  int mt = static_cast<int>(blockIdx.x / p.n_tiles);
  int64_t row0 = 0, row_end = p.M;  // output rows [row0, row_end) of this tile's group
  int64_t k_begin = 0, k_end = p.K;
  if constexpr (MODE == 0) {
    const int64_t g = blockIdx.z;
    A += g * p.a_gs;
    B += g * p.b_gs;
    C += g * p.c_gs;
    row0 = static_cast<int64_t>(mt) * kTB;
  } else if constexpr (MODE == 1) {
    if (mt >= p.tile_offsets[p.E]) return;
    int lo = 0, hi = p.E - 1;  // last e with tile_offsets[e] <= mt
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.tile_offsets[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    B += static_cast<int64_t>(lo) * p.b_gs;
    row0 = p.offsets[lo] + static_cast<int64_t>(mt - p.tile_offsets[lo]) * kTB;
    row_end = p.offsets[lo + 1];
  } else {
    const int e = blockIdx.z;
    C += static_cast<int64_t>(e) * p.c_gs;
    row0 = static_cast<int64_t>(mt) * kTB;
    k_begin = p.offsets[e];
    k_end = p.offsets[e + 1];
  }
  const int64_t n0 = static_cast<int64_t>(nt) * kTB;
  if (row0 >= row_end) return;
  TA acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = TA(0);
  // load maps: consecutive threads walk the operand's contiguous dimension
  const bool a_kc = p.sak == 1;
  const bool b_nc = p.sbn == 1;
  for (int64_t k0 = k_begin; k0 < k_end; k0 += kTK) {
#pragma unroll
    for (int i = 0; i < kTB * kTK / kTThreads; ++i) {
      const int q = i * kTThreads + tid;
      const int m = a_kc ? q / kTK : q % kTB;
      const int kk = a_kc ? q % kTK : q / kTB;
      const int64_t gm = row0 + m, gk = k0 + kk;
      As[kk][m] = (gm < row_end && gk < k_end) ? A[gm * p.sam + gk * p.sak] : T(0);
      const int n = b_nc ? q % kTB : q / kTK;
      const int kb = b_nc ? q / kTB : q % kTK;
      const int64_t gn = n0 + n, gkb = k0 + kb;
      Bs[kb][n] = (gn < p.N && gkb < k_end) ? B[gkb * p.sbk + gn * p.sbn] : T(0);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kTK; ++kk) {
      TA a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = static_cast<TA>(As[kk][ty + 16 * i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = static_cast<TA>(Bs[kk][tx + 16 * j]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t gm = row0 + ty + 16 * i;
    if (gm >= row_end) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + tx + 16 * j;
      if (gn < p.N) C[gm * p.ldc + gn] = static_cast<TO>(acc[i][j]);
    }
  }
}

template <typename T, typename TO, int MODE>
int launch_gemm_t(const GemmT& p, int64_t m_tiles, int groups, hipStream_t st, const char* name) {
  const int64_t blocks = m_tiles * p.n_tiles;
  if (blocks <= 0 || groups <= 0) return clear_error();
  if (blocks > 0x7fffffff || groups > 65535) return set_error(std::string(name) + ": problem too large");
  hipLaunchKernelGGL((gemm_t_kernel<T, TO, MODE>), dim3(static_cast<unsigned>(blocks), 1, groups),
                     dim3(kTThreads), 0, st, p);
  return check_launch(name) ? 1 : clear_error();
}

template <typename T>
int gemm_t_dispatch(int mode, int out_f32, const GemmT& p, int64_t m_tiles, int groups, hipStream_t st,
                    const char* name) {
  if (out_f32 && !std::is_same<T, float>::value) {
    if (mode != 0) return set_error(std::string(name) + ": an fp32 output is for dense products only");
    return launch_gemm_t<T, float, 0>(p, m_tiles, groups, st, name);
  }
  if (mode == 0) return launch_gemm_t<T, T, 0>(p, m_tiles, groups, st, name);
  if (mode == 1) return launch_gemm_t<T, T, 1>(p, m_tiles, groups, st, name);
  return launch_gemm_t<T, T, 2>(p, m_tiles, groups, st, name);
}

int gemm_t(int dtype, int mode, int out_f32, const GemmT& p, int64_t m_tiles, int groups, hipStream_t st,
           const char* name) {
  if (dtype == FFMOE_DTYPE_F32) return gemm_t_dispatch<float>(mode, out_f32, p, m_tiles, groups, st, name);
  if (dtype == FFMOE_DTYPE_F64) return gemm_t_dispatch<double>(mode, out_f32, p, m_tiles, groups, st, name);
  return set_error(std::string(name) + ": dtype must be FFMOE_DTYPE_F32 or FFMOE_DTYPE_F64");
}

// ---------------------------------------------------------------------------
// GLU.  TC = float: the routed experts' Triton kernels (fp32 math from the
// stored operands, activations.py:58-74, :108-142, tanh form of GeGLU);
// TC = T: the shared expert's torch ops in the compute dtype (nn.py:33-38,
// exact erf GELU).

__device__ __forceinline__ double glu_fwd_d(int act, double g, double u) {
  if (act == FFMOE_ACT_SWIGLU) return g / (1.0 + exp(-g)) * u;
  if (act == FFMOE_ACT_GEGLU) {
    const double inner = 0.7978845608028654 * (g + 0.044715 * g * g * g);
    return 0.5 * g * (1.0 + tanh(inner)) * u;
  }
  if (act == FFMOE_ACT_GEGLU_ERF) return 0.5 * g * (1.0 + erf(g * 0.7071067811865476)) * u;
  const double r = g > 0.0 ? g : 0.0;
  return r * r * u;
}

__device__ __forceinline__ void glu_bwd_d(int act, double ga, double g, double u, double* gg, double* gu) {
  if (act == FFMOE_ACT_SWIGLU) {
    const double s = 1.0 / (1.0 + exp(-g));
    *gu = ga * g * s;
    *gg = ga * u * (s * (1.0 + g * (1.0 - s)));
  } else if (act == FFMOE_ACT_GEGLU) {
    const double inner = 0.7978845608028654 * (g + 0.044715 * g * g * g);
    const double th = tanh(inner);
    const double dinner = 0.7978845608028654 * (1.0 + 3.0 * 0.044715 * g * g);
    *gu = ga * 0.5 * g * (1.0 + th);
    *gg = ga * u * (0.5 * (1.0 + th) + 0.5 * g * (1.0 - th * th) * dinner);
  } else if (act == FFMOE_ACT_GEGLU_ERF) {
    const double cdf = 0.5 * (1.0 + erf(g * 0.7071067811865476));
    const double pdf = 0.3989422804014327 * exp(-0.5 * g * g);
    *gu = ga * g * cdf;
    *gg = ga * u * (cdf + g * pdf);
  } else {
    const double r = g > 0.0 ? g : 0.0;
    *gu = ga * r * r;
    *gg = ga * u * 2.0 * r;
  }
}

template <typename TC> struct Glu;
template <> struct Glu<float> {
  static __device__ float fwd(int act, float g, float u) { return glu_fwd(act, g, u); }
  static __device__ void bwd(int act, float ga, float g, float u, float* gg, float* gu) {
    glu_bwd(act, ga, g, u, gg, gu);
  }
};
template <> struct Glu<double> {
  static __device__ double fwd(int act, double g, double u) { return glu_fwd_d(act, g, u); }
  static __device__ void bwd(int act, double ga, double g, double u, double* gg, double* gu) {
    glu_bwd_d(act, ga, g, u, gg, gu);
  }
};

template <typename T, typename TC>
__global__ __launch_bounds__(256) void glu_fwd_t_kernel(const T* __restrict__ up, int64_t M, int H, int act,
                                                        T* __restrict__ out) {
  const int64_t total = M * H;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t m = u / H;
    const int j = static_cast<int>(u % H);
    const TC g = static_cast<TC>(up[m * 2 * H + j]);
    const TC x = static_cast<TC>(up[m * 2 * H + H + j]);
    out[u] = static_cast<T>(Glu<TC>::fwd(act, g, x));
  }
}

template <typename T, typename TC>
__global__ __launch_bounds__(256) void glu_bwd_t_kernel(const T* __restrict__ ga, const T* __restrict__ up,
                                                        int64_t M, int H, int act, T* __restrict__ gup) {
  const int64_t total = M * H;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t m = u / H;
    const int j = static_cast<int>(u % H);
    TC gg, gu;
    Glu<TC>::bwd(act, static_cast<TC>(ga[u]), static_cast<TC>(up[m * 2 * H + j]),
                 static_cast<TC>(up[m * 2 * H + H + j]), &gg, &gu);
    gup[m * 2 * H + j] = static_cast<T>(gg);
    gup[m * 2 * H + H + j] = static_cast<T>(gu);
  }
}

unsigned grid_for(int64_t total) {
  const int64_t b = (total + 255) / 256;
  return static_cast<unsigned>(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

// ---------------------------------------------------------------------------
// Combine: out[n, d] = T(sum_s w_s * rows[src_s, d]) in fp32 slot order
// (moe_ops.py:190-203; the weights are topk_w.to(dtype), exact for fp32 and
// fp64), then T(out + addend) when an addend is given (fused_moe.py:590).
// No weights: the unweighted dX gather (moe_ops.py gather-reduce with the
// keep mask: a dropped entry contributes nothing).

__device__ __forceinline__ int src_of(int row) {
  return row >= 0 ? row : (row == FFMOE_ROW_ALIAS0 ? 0 : -1);
}

template <typename T>
__global__ __launch_bounds__(256) void combine_t_kernel(const T* __restrict__ rows, const int32_t* __restrict__ row_of,
                                                        const float* __restrict__ topk_w, const T* __restrict__ addend,
                                                        int64_t N, int D, int k, T* __restrict__ out) {
  const int64_t total = N * D;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = u / D;
    const int d = static_cast<int>(u % D);
    float acc = 0.0f;
    for (int s = 0; s < k; ++s) {
      const int r = src_of(row_of[n * k + s]);
      if (r < 0) continue;
      const float v = static_cast<float>(rows[static_cast<int64_t>(r) * D + d]);
      acc += (topk_w != nullptr ? topk_w[n * k + s] : 1.0f) * v;
    }
    T o = static_cast<T>(acc);
    if (addend != nullptr) o = o + addend[u];
    out[u] = o;
  }
}

// Padded weighted scatter for the kernel-level boundary (moe_ops.py:248-288):
// dst[dst_row[j]] = T(fp32(src[j / k]) * w[j]) (w NULL: a copy).
template <typename T>
__global__ __launch_bounds__(256) void scatter_rows_t_kernel(const T* __restrict__ src, const int64_t* __restrict__ dst_row,
                                                             const float* __restrict__ w, int64_t n_entries, int k,
                                                             int D, int64_t dst_rows, T* __restrict__ dst) {
  const int64_t total = n_entries * D;
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; u < total;
       u += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t j = u / D;
    const int d = static_cast<int>(u % D);
    const int64_t r = dst_row[j];
    if (r < 0 || r >= dst_rows) continue;
    const T v = src[(j / k) * D + d];
    dst[r * D + d] = w != nullptr ? static_cast<T>(static_cast<float>(v) * w[j]) : v;
  }
}

}  // namespace

// Routing-weight gradient and weighted scatter of the fp32 / fp64 path, with
// the top-k backward of the routing path shared with the bf16 kernel.
int route_bwd_t_launch(int dtype, const void* go, const void* down, const int32_t* row_of,
                       const int64_t* topk_idx, const float* topk_w, const float* logits, const float* lse,
                       const int32_t* counts, const float* g_aux, const float* g_z, float aux_coeff,
                       float z_coeff, int64_t N, int D, int E, int k, int gating, int capacity_mode,
                       int aux_through, const int64_t* aux_idx, const int32_t* aux_counts, int pre_softmax,
                       float scoring, void* wgo, void* gl, float* grad_w, hipStream_t st);

}  // namespace ffmoe

using namespace ffmoe;

static int check_dtype(int dtype, const char* name) {
  if (dtype != FFMOE_DTYPE_F32 && dtype != FFMOE_DTYPE_F64)
    return set_error(std::string(name) + ": dtype must be FFMOE_DTYPE_F32 or FFMOE_DTYPE_F64");
  return 0;
}

extern "C" int ffmoe_t_gemm_dense(int dtype, int trans_a, int trans_b, const void* a, const void* b, void* c,
                                  int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc, int out_f32,
                                  void* stream) {
  if (check_dtype(dtype, "ffmoe_t_gemm_dense")) return 1;
  if (M < 0 || N < 0 || K < 0 || a == nullptr || b == nullptr || c == nullptr)
    return set_error("ffmoe_t_gemm_dense: bad arguments");
  if (M == 0 || N == 0) return clear_error();
  GemmT p{};
  p.A = a;
  p.B = b;
  p.C = c;
  // op(A)(m, k), op(B)(k, n) of row-major A and B
  p.sam = trans_a ? 1 : lda;
  p.sak = trans_a ? lda : 1;
  p.sbk = trans_b ? 1 : ldb;
  p.sbn = trans_b ? ldb : 1;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  p.n_tiles = (N + kTB - 1) / kTB;
  return gemm_t(dtype, 0, out_f32, p, (M + kTB - 1) / kTB, 1, static_cast<hipStream_t>(stream),
                "ffmoe_t_gemm_dense");
}

extern "C" int ffmoe_t_gemm_rows(int dtype, const void* a, const void* b, const int32_t* offsets,
                                 const int32_t* tile_offsets, int E, int64_t max_rows, int K, int N, int b_kn,
                                 void* c, void* stream) {
  if (check_dtype(dtype, "ffmoe_t_gemm_rows")) return 1;
  if (E < 1 || K <= 0 || N <= 0 || max_rows < 0 || a == nullptr || b == nullptr || c == nullptr ||
      offsets == nullptr || tile_offsets == nullptr)
    return set_error("ffmoe_t_gemm_rows: bad arguments");
  if (max_rows == 0) return clear_error();
  GemmT p{};
  p.A = a;
  p.B = b;
  p.C = c;
  p.sam = K;
  p.sak = 1;
  // b_kn = 0: B[e] is [N, K] (x w^T); 1: B[e] is [K, N] (x w)
  p.sbk = b_kn ? N : 1;
  p.sbn = b_kn ? 1 : K;
  p.b_gs = static_cast<int64_t>(N) * K;
  p.ldc = N;
  p.M = 0;
  p.N = N;
  p.K = K;
  p.offsets = offsets;
  p.tile_offsets = tile_offsets;
  p.E = E;
  p.n_tiles = (N + kTB - 1) / kTB;
  const int64_t m_tiles = (max_rows + kTB - 1) / kTB + E;  // upper bound of the device-side row tiles
  return gemm_t(dtype, 1, 0, p, m_tiles, 1, static_cast<hipStream_t>(stream), "ffmoe_t_gemm_rows");
}

extern "C" int ffmoe_t_gemm_wgrad(int dtype, const void* a, const void* b, const int32_t* offsets, int E, int M,
                                  int Nc, void* c, void* stream) {
  if (check_dtype(dtype, "ffmoe_t_gemm_wgrad")) return 1;
  if (E < 1 || E > 65535 || M <= 0 || Nc <= 0 || a == nullptr || b == nullptr || c == nullptr ||
      offsets == nullptr)
    return set_error("ffmoe_t_gemm_wgrad: bad arguments");
  GemmT p{};
  p.A = a;
  p.B = b;
  p.C = c;
  p.sam = 1;
  p.sak = M;
  p.sbk = Nc;
  p.sbn = 1;
  p.c_gs = static_cast<int64_t>(M) * Nc;
  p.ldc = Nc;
  p.M = M;
  p.N = Nc;
  p.K = 0;
  p.offsets = offsets;
  p.E = E;
  p.n_tiles = (Nc + kTB - 1) / kTB;
  return gemm_t(dtype, 2, 0, p, (M + kTB - 1) / kTB, E, static_cast<hipStream_t>(stream), "ffmoe_t_gemm_wgrad");
}

extern "C" int ffmoe_t_glu_fwd(int dtype, const void* up, int64_t M, int H, int activation, int compute_in_dtype,
                               void* out, void* stream) {
  if (check_dtype(dtype, "ffmoe_t_glu_fwd")) return 1;
  if (M < 0 || H <= 0 || activation < 0 || activation > FFMOE_ACT_GEGLU_ERF)
    return set_error("ffmoe_t_glu_fwd: bad arguments");
  if (M == 0) return clear_error();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(M * H));
  if (dtype == FFMOE_DTYPE_F32)
    hipLaunchKernelGGL((glu_fwd_t_kernel<float, float>), grid, dim3(256), 0, st, static_cast<const float*>(up), M, H,
                       activation, static_cast<float*>(out));
  else if (compute_in_dtype)
    hipLaunchKernelGGL((glu_fwd_t_kernel<double, double>), grid, dim3(256), 0, st, static_cast<const double*>(up), M,
                       H, activation, static_cast<double*>(out));
  else
    hipLaunchKernelGGL((glu_fwd_t_kernel<double, float>), grid, dim3(256), 0, st, static_cast<const double*>(up), M,
                       H, activation, static_cast<double*>(out));
  return check_launch("glu_fwd_t_kernel") ? 1 : clear_error();
}

extern "C" int ffmoe_t_glu_bwd(int dtype, const void* grad_act, const void* up, int64_t M, int H, int activation,
                               int compute_in_dtype, void* grad_up, void* stream) {
  if (check_dtype(dtype, "ffmoe_t_glu_bwd")) return 1;
  if (M < 0 || H <= 0 || activation < 0 || activation > FFMOE_ACT_GEGLU_ERF)
    return set_error("ffmoe_t_glu_bwd: bad arguments");
  if (M == 0) return clear_error();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(M * H));
  if (dtype == FFMOE_DTYPE_F32)
    hipLaunchKernelGGL((glu_bwd_t_kernel<float, float>), grid, dim3(256), 0, st, static_cast<const float*>(grad_act),
                       static_cast<const float*>(up), M, H, activation, static_cast<float*>(grad_up));
  else if (compute_in_dtype)
    hipLaunchKernelGGL((glu_bwd_t_kernel<double, double>), grid, dim3(256), 0, st,
                       static_cast<const double*>(grad_act), static_cast<const double*>(up), M, H, activation,
                       static_cast<double*>(grad_up));
  else
    hipLaunchKernelGGL((glu_bwd_t_kernel<double, float>), grid, dim3(256), 0, st,
                       static_cast<const double*>(grad_act), static_cast<const double*>(up), M, H, activation,
                       static_cast<double*>(grad_up));
  return check_launch("glu_bwd_t_kernel") ? 1 : clear_error();
}

extern "C" int ffmoe_t_combine(int dtype, const void* rows, const int32_t* row_of, const float* topk_w,
                               const void* addend, int64_t N, int D, int k, void* out, void* stream) {
  if (check_dtype(dtype, "ffmoe_t_combine")) return 1;
  if (N < 0 || D <= 0 || k < 1 || k > FFMOE_MAX_TOPK || rows == nullptr || row_of == nullptr || out == nullptr)
    return set_error("ffmoe_t_combine: bad arguments");
  if (N == 0) return clear_error();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(N * D));
  if (dtype == FFMOE_DTYPE_F32)
    hipLaunchKernelGGL(combine_t_kernel<float>, grid, dim3(256), 0, st, static_cast<const float*>(rows), row_of,
                       topk_w, static_cast<const float*>(addend), N, D, k, static_cast<float*>(out));
  else
    hipLaunchKernelGGL(combine_t_kernel<double>, grid, dim3(256), 0, st, static_cast<const double*>(rows), row_of,
                       topk_w, static_cast<const double*>(addend), N, D, k, static_cast<double*>(out));
  return check_launch("combine_t_kernel") ? 1 : clear_error();
}

extern "C" int ffmoe_t_route_bwd(int dtype, const void* grad_out, const void* down, const int32_t* row_of,
                                 const int64_t* topk_idx, const float* topk_w, const float* logits,
                                 const float* lse, const int32_t* counts, const float* g_aux, const float* g_z,
                                 float aux_coeff, float z_coeff, int64_t N, int D, int E, int k, int gating,
                                 int capacity_mode, int aux_through_weights, const int64_t* aux_idx,
                                 const int32_t* aux_counts, int pre_softmax, float scoring_factor, void* wgo,
                                 void* grad_logits, float* grad_topk_w, void* stream) {
  if (check_dtype(dtype, "ffmoe_t_route_bwd")) return 1;
  if (N <= 0 || D <= 0 || E < 1 || E > FFMOE_MAX_EXPERTS || k < 1 || k > E || k > FFMOE_MAX_TOPK)
    return set_error("ffmoe_t_route_bwd: bad shape");
  if (grad_out == nullptr || down == nullptr || row_of == nullptr || topk_idx == nullptr || topk_w == nullptr ||
      wgo == nullptr || grad_logits == nullptr)
    return set_error("ffmoe_t_route_bwd: null argument");
  if ((g_z != nullptr || pre_softmax || gating == FFMOE_GATING_SIGMOID || aux_through_weights) && logits == nullptr)
    return set_error("ffmoe_t_route_bwd: logits needed");
  if ((g_z != nullptr || pre_softmax) && lse == nullptr) return set_error("ffmoe_t_route_bwd: lse needed");
  return route_bwd_t_launch(dtype, grad_out, down, row_of, topk_idx, topk_w, logits, lse, counts, g_aux, g_z,
                            aux_coeff, z_coeff, N, D, E, k, gating, capacity_mode, aux_through_weights, aux_idx,
                            aux_counts, pre_softmax, scoring_factor, wgo, grad_logits, grad_topk_w,
                            static_cast<hipStream_t>(stream));
}

extern "C" int ffmoe_t_scatter_rows(int dtype, const void* src, const int64_t* dst_row, const float* w,
                                    int64_t n_entries, int k, int D, int64_t dst_rows, void* dst, void* stream) {
  if (check_dtype(dtype, "ffmoe_t_scatter_rows")) return 1;
  if (n_entries < 0 || k < 1 || D <= 0 || dst_rows < 0 || src == nullptr || dst_row == nullptr || dst == nullptr)
    return set_error("ffmoe_t_scatter_rows: bad arguments");
  if (n_entries == 0) return clear_error();
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n_entries * D));
  if (dtype == FFMOE_DTYPE_F32)
    hipLaunchKernelGGL(scatter_rows_t_kernel<float>, grid, dim3(256), 0, st, static_cast<const float*>(src), dst_row,
                       w, n_entries, k, D, dst_rows, static_cast<float*>(dst));
  else
    hipLaunchKernelGGL(scatter_rows_t_kernel<double>, grid, dim3(256), 0, st, static_cast<const double*>(src),
                       dst_row, w, n_entries, k, D, dst_rows, static_cast<double*>(dst));
  return check_launch("scatter_rows_t_kernel") ? 1 : clear_error();
}
