// Expert grouped GEMMs on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16), bf16 in,
// fp32 accumulate, bf16 out, with the GLU forward / backward fused into the
// epilogues.
//
// Row groups (experts) live on the device: offsets[E+1] gives each expert's
// compact row range and tile_offsets[E+1] its first BM-row tile, so no host
// synchronisation is needed and padding rows are never computed.
//
// Operand layouts (row-major in HBM):
//   K-contiguous  (x_sorted, act, wgo, gup as A; w_up / w_down rows as B of
//                  the forward GEMMs) -> LDS tile [R][BK], 16-byte chunks
//                  XOR-swizzled by row; MFMA fragments are one 16-byte read.
//   MN-contiguous (w_down, w_up as B of the dgrad GEMMs; both operands of
//                  the wgrad GEMMs) -> LDS tile [BK][R + pad]; fragments are
//                  read with ds_read_b64_tr_b16 (gfx950 LDS transpose read).
#include <string>

#include "common.h"

namespace ffmoe {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;      // 4 waves, 2 x 2, each 64 x 64
constexpr int MN_PAD = 16;         // elements of padding per MN-tile row
constexpr int KC_ELEMS = 128 * BK;             // K-contiguous tile
constexpr int MN_ELEMS = BK * (128 + MN_PAD);  // MN-contiguous tile

enum Epi { EPI_STORE = 0, EPI_GLU_FWD = 1, EPI_GLU_BWD = 2 };

static int g_use_tr = 1;  // LDS transpose reads for MN-contiguous operands

struct GemmArgs {
  const bf16_t* A;
  const bf16_t* B;
  bf16_t* C;
  int64_t lda, ldb, ldc;
  int64_t b_stride;  // elements between experts' B matrices
  int64_t c_stride;  // elements between experts' C matrices (wgrad)
  const int32_t* offsets;
  const int32_t* tile_offsets;
  int E;
  int M;  // wgrad: rows of C; grouped-rows mode: unused
  int N;  // output columns (GLU forward: H, i.e. activation columns)
  int K;  // reduction length (grouped-rows mode)
  int n_tiles;
  int m_tiles;  // wgrad: tiles along M
  int64_t total_tiles;
  // epilogue extras
  const bf16_t* up;  // GLU backward: pre-activation [rows, 2H]
  bf16_t* C2;        // GLU forward: pre-activation out [rows, 2H] (optional)
  int H;
  int act;
};

__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nblocks) {
  // Blocks are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous run of tiles so neighbouring tiles share its L2.
  const int64_t per = (nblocks + 7) / 8;
  return (bid & 7) * per + (bid >> 3);
}

// K-contiguous tile: element (r, k) at r*BK + ((k/8) ^ (r&7))*8 + k%8.
__device__ __forceinline__ int kc_off(int r, int chunk) { return r * BK + ((chunk ^ (r & 7)) << 3); }

__device__ __forceinline__ bf16x8_t lds_frag_kc(const bf16_t* t, int r, int chunk) {
  return *reinterpret_cast<const bf16x8_t*>(t + kc_off(r, chunk));
}

typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

// MN-contiguous tile [BK][128 + MN_PAD]: fragment for column `c0 + lane%32`
// and k = ks*16 + (lane/32)*8 .. +8 of a 32x32x16 MFMA operand.
template <bool TR>
__device__ __forceinline__ bf16x8_t lds_frag_mn(const bf16_t* t, int c0, int ks, int lane) {
  constexpr int LD = 128 + MN_PAD;
  if constexpr (TR) {
    // ds_read_b64_tr_b16: within each 16-lane group, lane i supplies the
    // address of row (i/4), columns (i%4)*4..+4 of a 4 x 16 block and receives
    // column i of it (4 consecutive rows).
    const int g = lane >> 4, i = lane & 15;
    const int kb = ks * 16 + (g >> 1) * 8 + (i >> 2);
    const int col = c0 + (g & 1) * 16 + (i & 3) * 4;
    const bf16_t* p0 = t + kb * LD + col;
    const bf16_t* p1 = p0 + 4 * LD;
    const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(p0));
    const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)(p1));
    return bf16x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  } else {
    const int col = c0 + (lane & 31);
    const int kb = ks * 16 + (lane >> 5) * 8;
    bf16x8_t v;
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = __builtin_bit_cast(__bf16, t[(kb + q) * LD + col]);
    return v;
  }
}

// Local B-tile row -> global B row for the GLU forward: rows [0,64) are gate
// rows a0.., rows [64,128) the matching up rows H + a0..
__device__ __forceinline__ int glu_brow(int r, int a0, int H, bool* ok) {
  const int a = a0 + (r & 63);
  *ok = a < H;
  return (r < 64) ? a : H + a;
}

// Column base of accumulator tile tn of wave column wn within the block tile.
template <int EPI>
__device__ __forceinline__ int tile_col(int wn, int tn) {
  if constexpr (EPI == EPI_GLU_FWD) return tn * 64 + wn * 32;  // gate / up pairs
  else return wn * 64 + tn * 32;
}

// MODE 0: grouped rows (A rows = expert rows, B per expert).
// MODE 1: grouped K (wgrad): reduction over an expert's rows.
template <bool A_KC, bool B_KC, int MODE, int EPI, bool TR>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) bf16_t smem[2 * ((A_KC ? KC_ELEMS : MN_ELEMS) +
                                                           (B_KC ? KC_ELEMS : MN_ELEMS))];
  constexpr int A_ELEMS = A_KC ? KC_ELEMS : MN_ELEMS;
  constexpr int B_ELEMS = B_KC ? KC_ELEMS : MN_ELEMS;
  constexpr int LDMN = 128 + MN_PAD;

  const int64_t tile = xcd_remap(blockIdx.x, gridDim.x);
  if (tile >= p.total_tiles) return;

  // ---- tile decode ----
  int e, m0, n0;
  int row_begin = 0, row_end = 0;  // MODE 0: A rows; MODE 1: K range
  if constexpr (MODE == 0) {
    const int mt = static_cast<int>(tile / p.n_tiles);
    n0 = static_cast<int>(tile % p.n_tiles) * BN;
    if (mt >= p.tile_offsets[p.E]) return;
    int lo = 0, hi = p.E - 1;  // last e with tile_offsets[e] <= mt
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.tile_offsets[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    e = lo;
    row_begin = p.offsets[e] + (mt - p.tile_offsets[e]) * BM;
    row_end = p.offsets[e + 1];
    m0 = 0;
  } else {
    const int64_t per_e = static_cast<int64_t>(p.m_tiles) * p.n_tiles;
    e = static_cast<int>(tile / per_e);
    const int64_t r = tile % per_e;
    m0 = static_cast<int>(r / p.n_tiles) * BM;
    n0 = static_cast<int>(r % p.n_tiles) * BN;
    row_begin = p.offsets[e];
    row_end = p.offsets[e + 1];
  }
  const int K = (MODE == 0) ? p.K : (row_end - row_begin);
  const bf16_t* Be = (MODE == 0) ? p.B + static_cast<int64_t>(e) * p.b_stride : p.B;
  const int a0 = (EPI == EPI_GLU_FWD) ? n0 / 2 : 0;  // activation column base

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // buffer b: A tile at smem + b*(A_ELEMS+B_ELEMS), B tile right after it
  auto a_tile = [&](int b) { return smem + b * (A_ELEMS + B_ELEMS); };
  auto b_tile = [&](int b) { return smem + b * (A_ELEMS + B_ELEMS) + A_ELEMS; };

  uint4 ra[4], rb[4];

  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i;
      uint4 v = make_uint4(0, 0, 0, 0);
      if constexpr (A_KC) {  // MODE 0 only: tile [128 rows][BK]
        const int r = c >> 3, kc = c & 7;
        const int grow = row_begin + r;
        const int kk = k0 + kc * 8;
        if (grow < row_end && kk < K) v = *reinterpret_cast<const uint4*>(p.A + grow * p.lda + kk);
      } else {  // MODE 1: tile [BK][128 cols of M]
        const int kr = c >> 4, rc = c & 15;
        const int grow = row_begin + k0 + kr;
        const int m = m0 + rc * 8;
        if (grow < row_end && m < p.M) v = *reinterpret_cast<const uint4*>(p.A + grow * p.lda + m);
      }
      ra[i] = v;
    }
  };
  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i;
      uint4 v = make_uint4(0, 0, 0, 0);
      if constexpr (B_KC) {  // MODE 0 NT: B [N rows][K]
        const int r = c >> 3, kc = c & 7;
        const int kk = k0 + kc * 8;
        bool ok;
        int brow;
        if constexpr (EPI == EPI_GLU_FWD) {
          brow = glu_brow(r, a0, p.H, &ok);
        } else {
          brow = n0 + r;
          ok = brow < p.N;
        }
        if (ok && kk < K) v = *reinterpret_cast<const uint4*>(Be + static_cast<int64_t>(brow) * p.ldb + kk);
      } else if constexpr (MODE == 0) {  // NN: B [K rows][N]
        const int kr = c >> 4, rc = c & 15;
        const int kk = k0 + kr;
        const int n = n0 + rc * 8;
        if (kk < K && n < p.N) v = *reinterpret_cast<const uint4*>(Be + static_cast<int64_t>(kk) * p.ldb + n);
      } else {  // wgrad: B [rows][N]
        const int kr = c >> 4, rc = c & 15;
        const int grow = row_begin + k0 + kr;
        const int n = n0 + rc * 8;
        if (grow < row_end && n < p.N) v = *reinterpret_cast<const uint4*>(Be + grow * p.ldb + n);
      }
      rb[i] = v;
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i;
      if constexpr (A_KC) {
        *reinterpret_cast<uint4*>(a_tile(buf) + kc_off(c >> 3, c & 7)) = ra[i];
      } else {
        *reinterpret_cast<uint4*>(a_tile(buf) + (c >> 4) * LDMN + (c & 15) * 8) = ra[i];
      }
      if constexpr (B_KC) {
        *reinterpret_cast<uint4*>(b_tile(buf) + kc_off(c >> 3, c & 7)) = rb[i];
      } else {
        *reinterpret_cast<uint4*>(b_tile(buf) + (c >> 4) * LDMN + (c & 15) * 8) = rb[i];
      }
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = (K + BK - 1) / BK;
  if (nk > 0) {
    load_a(0);
    load_b(0);
    store_tiles(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) {
        load_a((kt + 1) * BK);
        load_b((kt + 1) * BK);
      }
      const bf16_t* at = a_tile(cur);
      const bf16_t* bt = b_tile(cur);
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8_t af[2], bfr[2];
#pragma unroll
        for (int tm = 0; tm < 2; ++tm) {
          const int r0 = wm * 64 + tm * 32;
          if constexpr (A_KC) af[tm] = lds_frag_kc(at, r0 + (lane & 31), ks * 2 + (lane >> 5));
          else af[tm] = lds_frag_mn<TR>(at, r0, ks, lane);
        }
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
          const int c0 = tile_col<EPI>(wn, tn);
          if constexpr (B_KC) bfr[tn] = lds_frag_kc(bt, c0 + (lane & 31), ks * 2 + (lane >> 5));
          else bfr[tn] = lds_frag_mn<TR>(bt, c0, ks, lane);
        }
#pragma unroll
        for (int tm = 0; tm < 2; ++tm)
#pragma unroll
          for (int tn = 0; tn < 2; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[tm], bfr[tn], acc[tm][tn], 0, 0, 0);
      }
      if (kt + 1 < nk) store_tiles(cur ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue ----
  // 32x32 accumulator layout: acc[r] of lane l is row (r/4)*8 + (l/32)*4 + r%4,
  // column l%32 of the 32x32 tile.
  const int lc = lane & 31;
#pragma unroll
  for (int tm = 0; tm < 2; ++tm) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int lr = wm * 64 + tm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if constexpr (MODE == 0) {
        const int grow = row_begin + lr;
        if (grow >= row_end) continue;
        if constexpr (EPI == EPI_GLU_FWD) {
          const int a = a0 + wn * 32 + lc;
          if (a >= p.H) continue;
          const bf16_t gh = f32_to_bf16(acc[tm][0][r]);
          const bf16_t uh = f32_to_bf16(acc[tm][1][r]);
          if (p.C2 != nullptr) {
            p.C2[grow * (2 * static_cast<int64_t>(p.H)) + a] = gh;
            p.C2[grow * (2 * static_cast<int64_t>(p.H)) + p.H + a] = uh;
          }
          p.C[grow * p.ldc + a] = f32_to_bf16(glu_fwd(p.act, bf16_to_f32(gh), bf16_to_f32(uh)));
        } else {
#pragma unroll
          for (int tn = 0; tn < 2; ++tn) {
            const int col = n0 + tile_col<EPI>(wn, tn) + lc;
            if (col >= p.N) continue;
            if constexpr (EPI == EPI_GLU_BWD) {
              const float ga = round_bf16(acc[tm][tn][r]);
              const int64_t ub = grow * (2 * static_cast<int64_t>(p.H));
              const float g = bf16_to_f32(p.up[ub + col]);
              const float u = bf16_to_f32(p.up[ub + p.H + col]);
              float gg, gu;
              glu_bwd(p.act, ga, g, u, &gg, &gu);
              p.C[ub + col] = f32_to_bf16(gg);
              p.C[ub + p.H + col] = f32_to_bf16(gu);
            } else {
              p.C[grow * p.ldc + col] = f32_to_bf16(acc[tm][tn][r]);
            }
          }
        }
      } else {
        const int m = m0 + lr;
        if (m >= p.M) continue;
        bf16_t* Ce = p.C + static_cast<int64_t>(e) * p.c_stride;
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
          const int col = n0 + tile_col<EPI>(wn, tn) + lc;
          if (col < p.N) Ce[static_cast<int64_t>(m) * p.ldc + col] = f32_to_bf16(acc[tm][tn][r]);
        }
      }
    }
  }
}

template <bool A_KC, bool B_KC, int MODE, int EPI>
static int launch(const GemmArgs& a, hipStream_t st, const char* name) {
  if (a.total_tiles <= 0) return clear_error();
  const int64_t grid = (a.total_tiles + 7) / 8 * 8;
  if (grid > 0x7fffffff) return set_error(std::string(name) + ": problem too large");
  if (g_use_tr)
    hipLaunchKernelGGL((gemm_kernel<A_KC, B_KC, MODE, EPI, true>), dim3(static_cast<unsigned>(grid)),
                       dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_kernel<A_KC, B_KC, MODE, EPI, false>), dim3(static_cast<unsigned>(grid)),
                       dim3(kThreads), 0, st, a);
  if (check_launch(name)) return 1;
  return clear_error();
}

static GemmArgs base_args(const int32_t* offsets, const int32_t* tile_offsets, int E) {
  GemmArgs a{};
  a.offsets = offsets;
  a.tile_offsets = tile_offsets;
  a.E = E;
  return a;
}

static int64_t row_tiles_bound(int64_t max_rows, int E) { return (max_rows + BM - 1) / BM + E; }

}  // namespace ffmoe

using namespace ffmoe;

extern "C" int ffmoe_gemm_tile_rows(void) { return BM; }

extern "C" int ffmoe_set_lds_transpose(int enable) {
  const int prev = g_use_tr;
  g_use_tr = enable ? 1 : 0;
  return prev;
}

extern "C" int ffmoe_gemm_up_glu(const void* x_sorted, const void* w_up, const int32_t* offsets,
                                 const int32_t* tile_offsets, int E, int64_t max_rows, int D, int H,
                                 int activation, void* up_out, void* act_out, void* stream) {
  if (E < 1 || E > FFMOE_MAX_EXPERTS || D <= 0 || D % 8 != 0 || H <= 0 || H % 8 != 0 || max_rows < 0)
    return set_error("ffmoe_gemm_up_glu: D and H must be positive multiples of 8");
  if (activation < 0 || activation > 2) return set_error("ffmoe_gemm_up_glu: unknown activation");
  GemmArgs a = base_args(offsets, tile_offsets, E);
  a.A = static_cast<const bf16_t*>(x_sorted);
  a.B = static_cast<const bf16_t*>(w_up);
  a.C = static_cast<bf16_t*>(act_out);
  a.C2 = static_cast<bf16_t*>(up_out);
  a.lda = D;
  a.ldb = D;
  a.ldc = H;
  a.b_stride = static_cast<int64_t>(2) * H * D;
  a.N = H;
  a.K = D;
  a.H = H;
  a.act = activation;
  a.n_tiles = (H + 63) / 64;
  a.total_tiles = row_tiles_bound(max_rows, E) * a.n_tiles;
  return launch<true, true, 0, EPI_GLU_FWD>(a, static_cast<hipStream_t>(stream), "gemm_up_glu");
}

extern "C" int ffmoe_gemm_down(const void* act, const void* w_down, const int32_t* offsets,
                               const int32_t* tile_offsets, int E, int64_t max_rows, int H, int D,
                               void* down_out, void* stream) {
  if (E < 1 || E > FFMOE_MAX_EXPERTS || D <= 0 || D % 8 != 0 || H <= 0 || H % 8 != 0 || max_rows < 0)
    return set_error("ffmoe_gemm_down: D and H must be positive multiples of 8");
  GemmArgs a = base_args(offsets, tile_offsets, E);
  a.A = static_cast<const bf16_t*>(act);
  a.B = static_cast<const bf16_t*>(w_down);
  a.C = static_cast<bf16_t*>(down_out);
  a.lda = H;
  a.ldb = H;
  a.ldc = D;
  a.b_stride = static_cast<int64_t>(D) * H;
  a.N = D;
  a.K = H;
  a.n_tiles = (D + BN - 1) / BN;
  a.total_tiles = row_tiles_bound(max_rows, E) * a.n_tiles;
  return launch<true, true, 0, EPI_STORE>(a, static_cast<hipStream_t>(stream), "gemm_down");
}

extern "C" int ffmoe_gemm_dgrad_glu(const void* wgo, const void* w_down, const void* up,
                                    const int32_t* offsets, const int32_t* tile_offsets, int E,
                                    int64_t max_rows, int D, int H, int activation, void* gup_out,
                                    void* stream) {
  if (E < 1 || E > FFMOE_MAX_EXPERTS || D <= 0 || D % 8 != 0 || H <= 0 || H % 8 != 0 || max_rows < 0)
    return set_error("ffmoe_gemm_dgrad_glu: D and H must be positive multiples of 8");
  if (activation < 0 || activation > 2) return set_error("ffmoe_gemm_dgrad_glu: unknown activation");
  GemmArgs a = base_args(offsets, tile_offsets, E);
  a.A = static_cast<const bf16_t*>(wgo);
  a.B = static_cast<const bf16_t*>(w_down);
  a.C = static_cast<bf16_t*>(gup_out);
  a.up = static_cast<const bf16_t*>(up);
  a.lda = D;
  a.ldb = H;
  a.ldc = 2 * static_cast<int64_t>(H);
  a.b_stride = static_cast<int64_t>(D) * H;
  a.N = H;
  a.K = D;
  a.H = H;
  a.act = activation;
  a.n_tiles = (H + BN - 1) / BN;
  a.total_tiles = row_tiles_bound(max_rows, E) * a.n_tiles;
  return launch<true, false, 0, EPI_GLU_BWD>(a, static_cast<hipStream_t>(stream), "gemm_dgrad_glu");
}

extern "C" int ffmoe_gemm_dgrad(const void* gup, const void* w_up, const int32_t* offsets,
                                const int32_t* tile_offsets, int E, int64_t max_rows, int H, int D,
                                void* ghb_out, void* stream) {
  if (E < 1 || E > FFMOE_MAX_EXPERTS || D <= 0 || D % 8 != 0 || H <= 0 || H % 8 != 0 || max_rows < 0)
    return set_error("ffmoe_gemm_dgrad: D and H must be positive multiples of 8");
  GemmArgs a = base_args(offsets, tile_offsets, E);
  a.A = static_cast<const bf16_t*>(gup);
  a.B = static_cast<const bf16_t*>(w_up);
  a.C = static_cast<bf16_t*>(ghb_out);
  a.lda = 2 * static_cast<int64_t>(H);
  a.ldb = D;
  a.ldc = D;
  a.b_stride = static_cast<int64_t>(2) * H * D;
  a.N = D;
  a.K = 2 * H;
  a.n_tiles = (D + BN - 1) / BN;
  a.total_tiles = row_tiles_bound(max_rows, E) * a.n_tiles;
  return launch<true, false, 0, EPI_STORE>(a, static_cast<hipStream_t>(stream), "gemm_dgrad");
}

extern "C" int ffmoe_gemm_wgrad(const void* a_, const void* b_, const int32_t* offsets, int E, int M,
                                int Nc, void* c_out, void* stream) {
  if (E < 1 || M <= 0 || M % 8 != 0 || Nc <= 0 || Nc % 8 != 0)
    return set_error("ffmoe_gemm_wgrad: M and Nc must be positive multiples of 8");
  GemmArgs a = base_args(offsets, nullptr, E);
  a.A = static_cast<const bf16_t*>(a_);
  a.B = static_cast<const bf16_t*>(b_);
  a.C = static_cast<bf16_t*>(c_out);
  a.lda = M;
  a.ldb = Nc;
  a.ldc = Nc;
  a.c_stride = static_cast<int64_t>(M) * Nc;
  a.M = M;
  a.N = Nc;
  a.m_tiles = (M + BM - 1) / BM;
  a.n_tiles = (Nc + BN - 1) / BN;
  a.total_tiles = static_cast<int64_t>(E) * a.m_tiles * a.n_tiles;
  return launch<false, false, 1, EPI_STORE>(a, static_cast<hipStream_t>(stream), "gemm_wgrad");
}
