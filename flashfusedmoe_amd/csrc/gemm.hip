// Expert grouped GEMMs on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16), bf16 in,
// fp32 accumulate, bf16 out, with the GLU forward / backward fused into the
// epilogues.
//
// Row groups (experts) live on the device: offsets[E+1] gives each expert's
// compact row range and tile_offsets[E+1] its first BM-row tile, so no host
// synchronisation is needed and padding rows are never computed.
//
// Block = 4 waves in a 2 x 2 grid; a BM x BN block tile gives each wave a
// (BM/2) x (BN/2) tile of 32x32 MFMA tiles (128 x 128 at BM = BN = 256: 256
// fp32 accumulators per lane, held in AGPRs, one wave per SIMD).  The MFMA
// operands are passed (B, A) so each lane accumulates 4 consecutive output
// COLUMNS of one row, and the epilogue writes 8-byte packed bf16 stores.
//
// Operand layouts (row-major in HBM):
//   K-contiguous  (x_sorted, act, wgo, gup as A; w_up / w_down rows as B of
//                  the forward GEMMs) -> LDS tile [R][BK], 16-byte chunks
//                  XOR-swizzled by row; MFMA fragments are one 16-byte read.
//   MN-contiguous (w_down, w_up as B of the dgrad GEMMs; both operands of
//                  the wgrad GEMMs) -> LDS tile [BK][R + pad]; fragments are
//                  read with ds_read_b64_tr_b16 (gfx950 LDS transpose read).
// Two LDS stages; the next stage's global loads are issued before the current
// stage's MFMAs and land in LDS after them (one barrier per BK step).
#include <string>
#include <type_traits>

#include "common.h"

namespace ffmoe {

constexpr int BK = 64;
constexpr int kThreads = 256;
constexpr int MN_PAD = 16;  // elements of padding per MN-contiguous LDS row

enum Epi { EPI_STORE = 0, EPI_GLU_FWD = 1, EPI_GLU_BWD = 2 };

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// buffer-instruction cache policy: sc1, device scope (coherent across XCDs)
constexpr int kDeviceScope = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// The same from values the caller knows to be block-uniform, taken from lane
// 0 so the descriptor is in scalar registers even where the compiler cannot
// prove them uniform (a descriptor in vector registers turns every buffer
// instruction into a loop over the distinct values).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_u(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xffffffffu)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint32_t n = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(bytes)));
  return make_rsrc(reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo), n);
}

// buffer-instruction cache policy: non-temporal (streaming)
constexpr int kNonTemporal = 2;
// an offset past every descriptor's range: the access is dropped (stores)
// or returns zeros (loads)
constexpr uint32_t kOutOfRange = 0xFFFFFFF0u;

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
  int M;  // wgrad: rows of C
  int N;  // output columns (GLU forward: H, the activation columns)
  int K;  // reduction length (grouped-rows mode)
  int n_tiles;
  int m_tiles;  // grouped-rows: upper bound of row tiles; wgrad: tiles along M
  int64_t total_tiles;
  const bf16_t* up;  // GLU backward: pre-activation [rows, 2H]
  bf16_t* C2;        // GLU forward: pre-activation out [rows, 2H] (optional)
  int H;
  int act;
  float* part;  // persistent kernel: fp32 partial tiles, one slot per block
  int* flags;   // persistent kernel: one flag per block + an error word
  int pub_off;  // cut tiles: publication of counter `key` is flags[pub_off + key]
  int err_idx;  // cut tiles: the error word is flags[err_idx]
  int lpt;      // wgrad: test the routing skew and balance the tiles over the XCDs
  int64_t split_rows;  // split-K: rows of one fp32 partial slab
  // An optional dense row group after the routed experts (the shared expert
  // of MoELayer): its own operands and outputs, x_rows rows, activation
  // x_act.  Grouped rows: rows [0, x_rows) of xA against xB; grouped K: the
  // (E+1)-th group, K = x_rows rows of xA and xB, output xC.
  const bf16_t* xA;
  const bf16_t* xB;
  bf16_t* xC;
  bf16_t* xC2;
  const bf16_t* xUp;
  int x_rows;
  int x_act;
  // grouped K only: x_split = 2 cuts the dense group's K into two groups of
  // x_chunk and x_rows - x_chunk rows whose tiles are finished as cut tiles
  // (counter flags[kPairKey + tile], fp32 partial in slot `tile`)
  int x_split;
  int x_chunk;
  // fused up+down launch: claim counter, exit counter, per-row-tile counts
  int* fused;
};

// Grouped K: groups of the extra dense group (two when its K is split).
__host__ __device__ __forceinline__ int extra_groups(const GemmArgs& p) {
  return p.x_rows > 0 ? (p.x_split > 1 ? 2 : 1) : 0;
}

// Grouped K: rows (K) of group i (the routed experts, then the dense group's).
__device__ __forceinline__ int group_rows(const GemmArgs& p, int i) {
  if (i < p.E) return p.offsets[i + 1] - p.offsets[i];
  if (p.x_split < 2) return p.x_rows;
  return i == p.E ? p.x_chunk : p.x_rows - p.x_chunk;
}

// Row tiles of the extra dense group.
template <int BM>
__device__ __forceinline__ int extra_tiles(const GemmArgs& p) {
  return p.x_rows > 0 ? (p.x_rows + BM - 1) / BM : 0;
}

__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t nblocks) {
  // Blocks are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous run of tiles so neighbouring tiles share its L2.
  const int64_t per = (nblocks + 7) / 8;
  return (bid & 7) * per + (bid >> 3);
}

// Within an XCD's run, visit tiles in groups of kGroupM row tiles x all
// column tiles, so the A rows and B columns in flight both stay few.
constexpr int kGroupM = 4;
__device__ __forceinline__ void grouped_order(int64_t t, int m_tiles, int n_tiles, int* mt,
                                              int* nt) {
  const int64_t per_group = static_cast<int64_t>(kGroupM) * n_tiles;
  const int64_t g = t / per_group;
  const int first = static_cast<int>(g * kGroupM);
  const int gm = min(m_tiles - first, kGroupM);
  const int r = static_cast<int>(t - g * per_group);
  *mt = first + r % gm;
  *nt = r / gm;
}

// K-contiguous tile [R][BK]: element (r, k) at r*BK + ((k/8) ^ (r&7))*8 + k%8.
__device__ __forceinline__ int kc_off(int r, int chunk) { return r * BK + ((chunk ^ (r & 7)) << 3); }

__device__ __forceinline__ bf16x8_t lds_frag_kc(const bf16_t* t, int r, int chunk) {
  return *reinterpret_cast<const bf16x8_t*>(t + kc_off(r, chunk));
}

typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

// MN-contiguous tile [BK][LD]: operand fragment for column c0 + lane%32 and
// k = ks*16 + (lane/32)*8 .. +8 of a 32x32x16 MFMA.
template <bool TR, int LD>
__device__ __forceinline__ bf16x8_t lds_frag_mn(const bf16_t* t, int c0, int ks, int lane) {
  if constexpr (TR) {
    // ds_read_b64_tr_b16: in each 16-lane group, lane i supplies the address
    // of row i/4, columns (i%4)*4..+4 of a 4 x 16 block and receives column i
    // of it (4 consecutive rows).
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

__device__ __forceinline__ uint2 pack4(float a, float b, float c, float d) {
  return make_uint2(pack_bf16x2(a, b), pack_bf16x2(c, d));
}

__device__ __forceinline__ void unpack4(uint2 v, float* f) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xffff0000u);
}

// Chunk swizzle of k-row k of an MN-contiguous stage tile of R columns:
// 16-byte chunk c sits at chunk c ^ mn_swz<R>(k).  Rows of 128 columns or
// more: (k & 3) << 2 (four rows cover distinct bank slots); rows of 64
// (128 bytes, so rows k and k + 2 share banks): ((k >> 1) & 1) << 2.  Both
// are the same for rows k and k + 4.
template <int R>
__device__ __forceinline__ constexpr int mn_swz(int k) {
  return R >= 128 ? (k & 3) << 2 : ((k >> 1) & 1) << 2;
}

// Transpose-read fragment from a swizzled MN-contiguous stage tile [32][R]
// (chunk swizzle mn_swz<R>).
//
// The two ds_read_b64_tr_b16 are issued as inline assembly: after a
// direct-to-LDS buffer load the compiler conservatively puts a vmcnt(0) wait
// in front of the transpose-read builtin (it cannot tell which LDS bytes the
// DMA writes), which would make every K step wait for the stage it has just
// started loading.  The stage the reads target is covered by the K loop's
// own vmcnt wait and barrier.  The compiler does not track the asm reads'
// completion: callers wait with lds_frags_ready() before using the result.
template <int R>
__device__ __forceinline__ bf16x8_t lds_frag_mn_sw(const bf16_t* t, int c0, int ks, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int kb = ks * 16 + (g >> 1) * 8 + (i >> 2);
  const int col = c0 + (g & 1) * 16 + (i & 3) * 4;
  const int sw = mn_swz<R>(kb);  // same for rows kb and kb + 4
  const int off = (((col >> 3) ^ sw) << 3) + (col & 7);
  const uint32_t a0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(t + kb * R + off));
  typedef unsigned int u32x2v_t __attribute__((ext_vector_type(2)));
  u32x2v_t lo, hi;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %2\n\t"
      "ds_read_b64_tr_b16 %1, %2 offset:%3"
      : "=&v"(lo), "=&v"(hi)
      : "v"(a0), "i"(4 * R * 2));
  const bf16x4_t l = __builtin_bit_cast(bf16x4_t, lo), h = __builtin_bit_cast(bf16x4_t, hi);
  return bf16x8_t{l[0], l[1], l[2], l[3], h[0], h[1], h[2], h[3]};
}

// ds_read_b128 as inline assembly, for K loops whose other fragment reads
// are asm transpose reads: if the compiler tracked some LDS reads and not
// others, its own lgkmcnt waits would count the untracked ones too and
// stall on them.
__device__ __forceinline__ bf16x8_t lds_read_b128_asm(const bf16_t* p) {
  typedef unsigned int u32x4v_t __attribute__((ext_vector_type(4)));
  u32x4v_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p))));
  return __builtin_bit_cast(bf16x8_t, v);
}

// Waits until every LDS read this wave issued has returned (the asm
// transpose reads above are not tracked by the compiler) and orders the
// MFMAs that consume `fa` / `fb` after the wait.  Placed where only those
// fragments' reads are outstanding, so it costs nothing in steady state.
template <int NA, int NB>
__device__ __forceinline__ void lds_frags_ready(bf16x8_t (&fa)[NA], bf16x8_t (&fb)[NB]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < NA; ++i) asm volatile("" : "+v"(fa[i]));
#pragma unroll
  for (int i = 0; i < NB; ++i) asm volatile("" : "+v"(fb[i]));
}

// GLU backward epilogue, split in two so the pre-activation loads can be in
// flight while the accumulators are staged: item i of a thread covers row
// row_base + idx / (BN/8) and columns n0 + (idx % (BN/8))*8 .. +8 of the
// tile, idx = i * kThreads + tid.  All loads are issued before any store (a
// vector-memory wait would also drain earlier stores).
template <int ROWS, int BN, int NT = kThreads>
constexpr int glu_bwd_items() { return ROWS * (BN / 8) / NT; }

template <int ROWS, int BN, int NT = kThreads>
__device__ __forceinline__ void glu_bwd_prefetch(const GemmArgs& p, int row_base, int row_end, int n0,
                                                 uint4* pg, uint4* pu) {
  constexpr int CH = BN / 8;
  constexpr int IT = glu_bwd_items<ROWS, BN, NT>();
  static_assert((ROWS * CH) % NT == 0, "whole items");
  const int tid = threadIdx.x;
  const int64_t H = p.H;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int idx = it * NT + tid;
    const int64_t row = static_cast<int64_t>(row_base) + idx / CH;
    const int col = n0 + (idx % CH) * 8;
    pg[it] = make_uint4(0, 0, 0, 0);
    pu[it] = make_uint4(0, 0, 0, 0);
    if (row < row_end && col < p.N) {
      pg[it] = *reinterpret_cast<const uint4*>(p.up + row * 2 * H + col);
      pu[it] = *reinterpret_cast<const uint4*>(p.up + row * 2 * H + H + col);
    }
  }
}

template <int ROWS, int BN, int LDC, int NT = kThreads>
__device__ __forceinline__ void glu_bwd_store(const GemmArgs& p, const bf16_t* Cs, int row_base, int row_end,
                                              int n0, const uint4* pg, const uint4* pu) {
  constexpr int CH = BN / 8;
  constexpr int IT = glu_bwd_items<ROWS, BN, NT>();
  constexpr int BT = IT < 4 ? IT : 4;  // items per batch: a batch's LDS reads go out together
  static_assert(IT % BT == 0, "whole batches");
  const int tid = threadIdx.x;
  const int64_t H = p.H;
  // rows past the group fall outside the descriptor's range (dropped)
  const int rows = max(0, min(row_end - row_base, ROWS));
  const __amdgpu_buffer_rsrc_t rc = make_rsrc_u(p.C + static_cast<int64_t>(row_base) * 2 * H,
                                                static_cast<uint32_t>(rows * 2 * H * 2));
  with_act(p.act, [&](auto actc) {
    constexpr int ACT = decltype(actc)::value;
#pragma unroll
    for (int b = 0; b < IT; b += BT) {
      uint4 gav[BT];
#pragma unroll
      for (int i = 0; i < BT; ++i) {
        const int idx = (b + i) * NT + tid;
        gav[i] = *reinterpret_cast<const uint4*>(Cs + (idx / CH) * LDC + (idx % CH) * 8);
      }
#pragma unroll
      for (int i = 0; i < BT; ++i) {
        const int idx = (b + i) * NT + tid;
        const int ml = idx / CH, col = n0 + (idx % CH) * 8;
        float ga[8], g[8], u[8], gg[8], gu[8];
        unpack8(gav[i], ga);
        unpack8(pg[b + i], g);
        unpack8(pu[b + i], u);
#pragma unroll
        for (int k = 0; k < 8; ++k) glu_bwd_t<ACT>(ga[k], g[k], u[k], &gg[k], &gu[k]);
        const uint32_t off = col < p.N ? static_cast<uint32_t>((ml * 2 * H + col) * 2) : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, pack8(gg)), rc, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, pack8(gu)), rc,
                                               col < p.N ? off + static_cast<uint32_t>(H * 2) : kOutOfRange, 0, 0);
      }
    }
  });
}

// Stores ROWS rows of a bf16 C tile staged in LDS (row stride LDC) with the
// block's NT threads, 16 bytes each: plain store, GLU forward (tile columns
// [0, BN/2) gate, [BN/2, BN) up: writes act and, if requested, the
// pre-activation) or GLU backward (reads the pre-activation, writes its
// gradient).  Rows are row_base + i (grouped rows, valid below row_end) or
// m_base + i (wgrad, valid below M).
template <int ROWS, int BN, int LDC, int MODE, int EPI, bool CO_C = false, int NT = kThreads>
__device__ __forceinline__ void store_c_tile(const GemmArgs& p, const bf16_t* Cs, int e, int m_base,
                                             int row_base, int row_end, int n0, int a0) {
  const int tid = threadIdx.x;
  // Every store is a buffer store through a block-uniform descriptor over
  // the tile's valid rows (rows past them are dropped by its range, columns
  // past N by an out-of-range offset), so the loops have no branches and
  // each batch's LDS reads go out before its first store.
  if constexpr (EPI == EPI_GLU_FWD) {
    constexpr int CH = BN / 16;  // 8-column chunks per half row
    constexpr int IT = ROWS * CH / NT;
    static_assert((ROWS * CH) % NT == 0, "whole items");
    constexpr int BT = IT < 4 ? IT : 4;
    static_assert(IT % BT == 0, "whole batches");
    const int64_t H = p.H;
    const int rows = max(0, min(row_end - row_base, ROWS));
    // CO_C: the activation rows are read by other blocks of the same launch
    // (the fused up+down GEMM): device-scope stores (written through to the
    // level every XCD reads)
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc_u(p.C + static_cast<int64_t>(row_base) * p.ldc, static_cast<uint32_t>(rows * p.ldc * 2));
    const bool pre = p.C2 != nullptr;
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc_u(pre ? p.C2 + static_cast<int64_t>(row_base) * 2 * H : p.C,
                    pre ? static_cast<uint32_t>(rows * 2 * H * 2) : 0u);
    with_act(p.act, [&](auto actc) {
      constexpr int ACT = decltype(actc)::value;
#pragma unroll 1
      for (int b = 0; b < IT; b += BT) {
        uint4 gv[BT], uv[BT];
#pragma unroll
        for (int i = 0; i < BT; ++i) {
          const int idx = (b + i) * NT + tid;
          const bf16_t* src = Cs + (idx / CH) * LDC + (idx % CH) * 8;
          gv[i] = *reinterpret_cast<const uint4*>(src);
          uv[i] = *reinterpret_cast<const uint4*>(src + BN / 2);
        }
#pragma unroll
        for (int i = 0; i < BT; ++i) {
          const int idx = (b + i) * NT + tid;
          const int ml = idx / CH, a = a0 + (idx % CH) * 8;
          const bool ok = a < p.H;
          float g[8], u[8], o[8];
          unpack8(gv[i], g);
          unpack8(uv[i], u);
#pragma unroll
          for (int k = 0; k < 8; ++k) o[k] = glu_fwd_t<ACT>(g[k], u[k]);
          if (pre) {
            const uint32_t po = ok ? static_cast<uint32_t>((ml * 2 * H + a) * 2) : kOutOfRange;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, gv[i]), rp, po, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, uv[i]), rp,
                                                   ok ? po + static_cast<uint32_t>(H * 2) : kOutOfRange, 0, 0);
          }
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4_t, pack8(o)), rc,
              ok ? static_cast<uint32_t>((ml * p.ldc + a) * 2) : kOutOfRange, 0, CO_C ? kDeviceScope : 0);
        }
      }
    });
  } else if constexpr (EPI == EPI_GLU_BWD) {
    uint4 pg[glu_bwd_items<ROWS, BN, NT>()], pu[glu_bwd_items<ROWS, BN, NT>()];
    glu_bwd_prefetch<ROWS, BN, NT>(p, row_base, row_end, n0, pg, pu);
    glu_bwd_store<ROWS, BN, LDC, NT>(p, Cs, row_base, row_end, n0, pg, pu);
  } else {
    constexpr int CH = BN / 8;
    constexpr int IT = ROWS * CH / NT;
    static_assert((ROWS * CH) % NT == 0, "whole items");
    constexpr int BT = IT < 8 ? IT : 8;
    static_assert(IT % BT == 0, "whole batches");
    const bf16_t* Cb = (MODE == 1) ? p.C + static_cast<int64_t>(e) * p.c_stride + static_cast<int64_t>(m_base) * p.ldc
                                   : p.C + static_cast<int64_t>(row_base) * p.ldc;
    const int rows = (MODE == 1) ? max(0, min(p.M - m_base, ROWS)) : max(0, min(row_end - row_base, ROWS));
    const __amdgpu_buffer_rsrc_t rc = make_rsrc_u(Cb, static_cast<uint32_t>(rows * p.ldc * 2));
#pragma unroll 1
    for (int b = 0; b < IT; b += BT) {
      uint4 v[BT];
#pragma unroll
      for (int i = 0; i < BT; ++i) {
        const int idx = (b + i) * NT + tid;
        v[i] = *reinterpret_cast<const uint4*>(Cs + (idx / CH) * LDC + (idx % CH) * 8);
      }
#pragma unroll
      for (int i = 0; i < BT; ++i) {
        const int idx = (b + i) * NT + tid;
        const int ml = idx / CH, col = n0 + (idx % CH) * 8;
        // weight gradients (MODE 1) are not read again by the step:
        // streaming stores keep them from evicting the operand rows the
        // other tiles still read (measured: C5 wgrads -4 to -6%, C2 -2%)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(u32x4_t, v[i]), rc,
            col < p.N ? static_cast<uint32_t>((ml * p.ldc + col) * 2) : kOutOfRange, 0,
            MODE == 1 ? kNonTemporal : 0);
      }
    }
  }
}

// Register-staged kernel (fallback for K not a multiple of the direct-to-LDS
// K step, and the element-wise LDS read variant used to cross-check the
// transpose reads).
// MODE 0: grouped rows (A rows = expert rows, B per expert).
// MODE 1: grouped K (wgrad): reduction over an expert's rows.
template <int BM, int BN, bool A_KC, bool B_KC, int MODE, int EPI, bool TR>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmArgs p) {
  constexpr int WM = BM / 2, WN = BN / 2;   // per-wave tile
  constexpr int TM = WM / 32, TN = WN / 32;  // 32x32 MFMA tiles per wave
  constexpr int LDA = BM + MN_PAD, LDB = BN + MN_PAD;
  constexpr int A_ELEMS = A_KC ? BM * BK : BK * LDA;
  constexpr int B_ELEMS = B_KC ? BN * BK : BK * LDB;
  constexpr int STAGE = A_ELEMS + B_ELEMS;
  constexpr int LDC = BN + 8;  // C tile row stride in LDS (elements)
  constexpr int SMEM = (2 * STAGE > BM * LDC) ? 2 * STAGE : BM * LDC;
  constexpr int A_LOADS = BM / 32;  // 16-byte chunks per thread per stage
  constexpr int B_LOADS = BN / 32;
  static_assert(EPI != EPI_GLU_FWD || (TN % 2 == 0), "GLU forward pairs gate/up tiles");
  __shared__ __attribute__((aligned(16))) bf16_t smem[SMEM];

  const int64_t tile = xcd_remap(blockIdx.x, gridDim.x);
  if (tile >= p.total_tiles) return;

  // ---- tile decode ----
  int e, m0 = 0, n0;
  int row_begin = 0, row_end = 0;  // MODE 0: A rows; MODE 1: K range
  if constexpr (MODE == 0) {
    int mt, nt;
    grouped_order(tile, p.m_tiles, p.n_tiles, &mt, &nt);
    n0 = nt * BN;
    if (mt >= p.tile_offsets[p.E]) return;
    int lo = 0, hi = p.E - 1;  // last e with tile_offsets[e] <= mt
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.tile_offsets[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    e = lo;
    row_begin = p.offsets[e] + (mt - p.tile_offsets[e]) * BM;
    row_end = p.offsets[e + 1];
  } else {
    const int64_t per_e = static_cast<int64_t>(p.m_tiles) * p.n_tiles;
    e = static_cast<int>(tile / per_e);
    int mt, nt;
    grouped_order(tile - static_cast<int64_t>(e) * per_e, p.m_tiles, p.n_tiles, &mt, &nt);
    m0 = mt * BM;
    n0 = nt * BN;
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

  auto a_tile = [&](int b) { return smem + b * STAGE; };
  auto b_tile = [&](int b) { return smem + b * STAGE + A_ELEMS; };
  // column base (within the block tile) of accumulator tile tn of this wave
  auto tile_col = [&](int tn) {
    if constexpr (EPI == EPI_GLU_FWD)
      return (tn < TN / 2) ? wn * (WN / 2) + tn * 32 : BN / 2 + wn * (WN / 2) + (tn - TN / 2) * 32;
    else
      return wn * WN + tn * 32;
  };

  uint4 ra[A_LOADS], rb[B_LOADS];

  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int c = tid + kThreads * i;
      uint4 v = make_uint4(0, 0, 0, 0);
      if constexpr (A_KC) {  // MODE 0: tile [BM rows][BK]
        const int r = c >> 3, kc = c & 7;
        const int grow = row_begin + r;
        const int kk = k0 + kc * 8;
        if (grow < row_end && kk < K) v = *reinterpret_cast<const uint4*>(p.A + grow * p.lda + kk);
      } else {  // MODE 1: tile [BK][BM columns of M]
        const int kr = c / (BM / 8), rc = c % (BM / 8);
        const int grow = row_begin + k0 + kr;
        const int m = m0 + rc * 8;
        if (grow < row_end && m < p.M) v = *reinterpret_cast<const uint4*>(p.A + grow * p.lda + m);
      }
      ra[i] = v;
    }
  };
  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int c = tid + kThreads * i;
      uint4 v = make_uint4(0, 0, 0, 0);
      if constexpr (B_KC) {  // MODE 0 NT: B [N rows][K]
        const int r = c >> 3, kc = c & 7;
        const int kk = k0 + kc * 8;
        bool ok;
        int brow;
        if constexpr (EPI == EPI_GLU_FWD) {
          // rows [0, BN/2): gate rows a0.., rows [BN/2, BN): up rows H + a0..
          const int a = a0 + (r % (BN / 2));
          ok = a < p.H;
          brow = (r < BN / 2) ? a : p.H + a;
        } else {
          brow = n0 + r;
          ok = brow < p.N;
        }
        if (ok && kk < K) v = *reinterpret_cast<const uint4*>(Be + static_cast<int64_t>(brow) * p.ldb + kk);
      } else if constexpr (MODE == 0) {  // NN: B [K rows][N]
        const int kr = c / (BN / 8), rc = c % (BN / 8);
        const int kk = k0 + kr;
        const int n = n0 + rc * 8;
        if (kk < K && n < p.N) v = *reinterpret_cast<const uint4*>(Be + static_cast<int64_t>(kk) * p.ldb + n);
      } else {  // wgrad: B [rows][N]
        const int kr = c / (BN / 8), rc = c % (BN / 8);
        const int grow = row_begin + k0 + kr;
        const int n = n0 + rc * 8;
        if (grow < row_end && n < p.N) v = *reinterpret_cast<const uint4*>(Be + grow * p.ldb + n);
      }
      rb[i] = v;
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int c = tid + kThreads * i;
      if constexpr (A_KC)
        *reinterpret_cast<uint4*>(a_tile(buf) + kc_off(c >> 3, c & 7)) = ra[i];
      else
        *reinterpret_cast<uint4*>(a_tile(buf) + (c / (BM / 8)) * LDA + (c % (BM / 8)) * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int c = tid + kThreads * i;
      if constexpr (B_KC)
        *reinterpret_cast<uint4*>(b_tile(buf) + kc_off(c >> 3, c & 7)) = rb[i];
      else
        *reinterpret_cast<uint4*>(b_tile(buf) + (c / (BN / 8)) * LDB + (c % (BN / 8)) * 8) = rb[i];
    }
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
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
        bf16x8_t af[TM], bfr[TN];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
          const int r0 = wm * WM + tm * 32;
          if constexpr (A_KC) af[tm] = lds_frag_kc(at, r0 + (lane & 31), ks * 2 + (lane >> 5));
          else af[tm] = lds_frag_mn<TR, LDA>(at, r0, ks, lane);
        }
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const int c0 = tile_col(tn);
          if constexpr (B_KC) bfr[tn] = lds_frag_kc(bt, c0 + (lane & 31), ks * 2 + (lane >> 5));
          else bfr[tn] = lds_frag_mn<TR, LDB>(bt, c0, ks, lane);
        }
        // (B, A) operand order: lane l accumulates row l%32 of the tile and
        // columns 8*(r/4) + 4*(l/32) + r%4.
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[tn], af[tm], acc[tm][tn], 0, 0, 0);
      }
      if (kt + 1 < nk) store_tiles(cur ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue ----
  // 1) every lane writes its accumulators, rounded to bf16, into a C tile in
  //    LDS (the pipeline buffers are free after the loop's last barrier);
  //    lane l holds row l%32 and columns 8*(r/4) + 4*(l/32) + r%4 of each
  //    32x32 tile: 4 consecutive columns -> one 8-byte LDS write.
  // 2) the block reads the tile back in 16-byte row chunks and applies the
  //    epilogue op with coalesced 16-byte global loads and stores.
  bf16_t* Cs = smem;
  {
    const int lr = lane & 31;
    const int lq = (lane >> 5) * 4;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int ml = wm * WM + tm * 32 + lr;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int nl = tile_col(tn) + lq;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          *reinterpret_cast<uint2*>(Cs + ml * LDC + nl + q * 8) =
              pack4(acc[tm][tn][4 * q], acc[tm][tn][4 * q + 1], acc[tm][tn][4 * q + 2],
                    acc[tm][tn][4 * q + 3]);
        }
      }
    }
  }
  __syncthreads();
  store_c_tile<BM, BN, LDC, MODE, EPI>(p, Cs, e, m0, row_begin, row_end, n0, a0);
}

// ---------------------------------------------------------------------------
// Direct-to-LDS pipeline (the main path): BK = 64, a ring of two or three
// LDS stages filled by buffer_load_dwordx4 ... lds (each wave instruction writes 1 KiB of
// consecutive LDS; per-lane source addresses implement the swizzle;
// out-of-range rows read as zero through the buffer descriptor's bounds).
// Every row segment a stage loads is a whole 128-byte line (64 bf16 of a
// K-contiguous row, or 256+ bf16 of an MN-contiguous k-row): half-line
// segments halve what the L2 delivers to a CU.
//   K-contiguous stage tile [R][64]: 16-byte chunk c of row r stored at
//     chunk c ^ ((r >> 1) & 7): the 16 rows one ds_read_b128 cycle serves hit
//     16 distinct 16-byte bank slots (64 banks x 4 bytes).
//   MN-contiguous stage tile [64][R]: chunk c of k-row k stored at
//     c ^ mn_swz<R>(k): the 2 x 4 rows x 32 bytes of one transpose-read
//     cycle hit distinct bank slots.
// Each 64-K stage is four MFMA k-steps of 16; operand fragments are
// double-buffered in registers.  Before the last k-step of stage kt: wait for
// stage kt+1's loads, one s_barrier, refill stage kt's buffer with stage
// kt+NS, read stage kt+1's first fragments, then run the last k-step.
constexpr int DL_BK = 64;
// Stages of the LDS ring: three where they fit in the 160 KiB of LDS (tiles
// of at most 384 rows + columns), else two.
template <int BM, int BN>
constexpr int dl_stages() { return (BM + BN) <= 384 ? 3 : 2; }
// LDS elements of a tile: the stage ring, or the C staging tile (rows of
// BN + 8) the epilogue reuses it for, whichever is larger.
template <int BM, int BN>
constexpr int dl_smem_elems() {
  return dl_stages<BM, BN>() * (BM + BN) * 64 > BM * (BN + 8) ? dl_stages<BM, BN>() * (BM + BN) * 64
                                                               : BM * (BN + 8);
}

__device__ __forceinline__ void wait_vmcnt_le(int n) {
  // s_waitcnt with only the vector-memory count constrained (expcnt and
  // lgkmcnt at their maxima); n is one of a few small constants
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
    case 16: __builtin_amdgcn_s_waitcnt(0x4F70); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
}

// Parts a stage's direct-to-LDS loads are issued in (see gemm_dl_tile).
// Measured at C2 (in-step µs, 1 / 2 / 4 parts): three-stage 256x128 tiles
// gain from 4 (down 99 / 99 / 96.5, dgrad+GLU 156 / 154 / 149); two-stage
// 256x256 tiles from 2 (dgrad 161 / 155 / 173, wgrad 143 / 135 / 152),
// except the up GEMM with its GLU epilogue (180 / 187 / 191).  With eight
// waves (four loads per thread per operand and stage) two parts for all
// (up GEMM 162 / 155 µs with 1 / 2).
template <int BM, int BN, int EPI, int NT = kThreads>
constexpr int issue_parts() {
  if (NT == 512) return 2;
  return dl_stages<BM, BN>() >= 3 ? 4 : (EPI == EPI_GLU_FWD ? 1 : 2);
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Which part of a tile's K range a block computes.  ROLE_FULL: all of it,
// then the epilogue.  ROLE_CUT: one of the two K ranges of a tile cut
// between two blocks.  Both count themselves in on the tile's counter; the
// first to arrive publishes its fp32 partial (and which slot holds it) and
// is done, the second waits for that publication (its writer is already
// running, so no co-residency is needed), adds the partial (two terms: the
// same bits in either order) and runs the epilogue.
// ROLE_SPLIT: one of several K ranges of a tile whose fp32 partials a
// separate reduction kernel adds up (split-K dense GEMMs): the block writes
// its accumulators to fp32 slab `slot` ([rows, N] row-major) and is done.
enum Role { ROLE_FULL = 0, ROLE_CUT = 1, ROLE_SPLIT = 2 };

struct TileCoord {
  int e, m0, n0, row_begin, row_end;
  bool valid;
  bool extra;  // a tile of the extra dense group
  int xt;      // grouped K, extra group: the tile's index in its group
};

// Row-group tables are read through the constant address space: they do not
// change during a launch, so the loads are scalar (s_load) even after the
// kernel's own stores, where the compiler could not otherwise prove that.
typedef __attribute__((address_space(4))) const int32_t const_i32_t;
__device__ __forceinline__ int ld_const(const int32_t* p, int i) {
  return ((const const_i32_t*)p)[i];
}

// Grouped-rows tile of row tile mt and column tile nt.
template <int BM, int BN>
__device__ __forceinline__ TileCoord decode_rows_mn(const GemmArgs& p, int mt, int nt) {
  TileCoord c{};
  c.n0 = nt * BN;
  const int R = ld_const(p.tile_offsets, p.E);
  c.valid = mt < R + extra_tiles<BM>(p);
  if (!c.valid) return c;
  if (mt >= R) {  // the extra dense group's row tiles follow the routed ones
    c.extra = true;
    c.e = 0;
    c.row_begin = (mt - R) * BM;
    c.row_end = p.x_rows;
    return c;
  }
  int lo = 0, hi = p.E - 1;  // last e with tile_offsets[e] <= mt
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ld_const(p.tile_offsets, mid) <= mt) lo = mid; else hi = mid - 1;
  }
  c.e = lo;
  c.row_begin = ld_const(p.offsets, lo) + (mt - ld_const(p.tile_offsets, lo)) * BM;
  c.row_end = ld_const(p.offsets, lo + 1);
  return c;
}

// Grouped-rows tile t of a grid of m_count row tiles x n_tiles column tiles.
template <int BM, int BN>
__device__ __forceinline__ TileCoord decode_rows_tile(const GemmArgs& p, int64_t t, int m_count) {
  int mt, nt;
  grouped_order(t, m_count, p.n_tiles, &mt, &nt);
  return decode_rows_mn<BM, BN>(p, mt, nt);
}

// Grouped-K (wgrad) tile t: expert-major, then grouped over M x N tiles.
template <int BM, int BN>
__device__ __forceinline__ TileCoord decode_k_tile(const GemmArgs& p, int64_t t) {
  TileCoord c{};
  const int64_t per_e = static_cast<int64_t>(p.m_tiles) * p.n_tiles;
  c.e = static_cast<int>(t / per_e);
  int mt, nt;
  grouped_order(t - static_cast<int64_t>(c.e) * per_e, p.m_tiles, p.n_tiles, &mt, &nt);
  c.m0 = mt * BM;
  c.n0 = nt * BN;
  c.valid = true;
  if (c.e >= p.E) {  // the extra dense group: all of its rows, or one of two K halves
    const int half = c.e - p.E;
    c.extra = true;
    c.xt = static_cast<int>(t - static_cast<int64_t>(c.e) * per_e);
    c.e = 0;
    c.row_begin = half == 0 ? 0 : p.x_chunk;
    c.row_end = (half == 0 && p.x_split > 1) ? p.x_chunk : p.x_rows;
    return c;
  }
  c.row_begin = ld_const(p.offsets, c.e);
  c.row_end = ld_const(p.offsets, c.e + 1);
  return c;
}

constexpr int kSpinLimit = 1 << 22;  // flag polls before a wait gives up

// One tile (K steps [k0, k1); k1 < 0: to the end of K).  The body is a
// __device__ function (the buffer-descriptor type exists only in the device
// pass); the kernels below loop over tiles with it.
// CO (fused up+down launch): kCoLoadA = the A rows were written by other
// blocks of this launch (device-scope loads), kCoStoreC = the C rows are
// read by other blocks of this launch (device-scope stores; the caller
// counts them complete through the next tile's signal).  XS: the LDS buffer is the caller's (xsm), so that one
// kernel can run tiles of two shapes out of one allocation.
constexpr int kCoLoadA = 1, kCoStoreC = 2;
// signal (fused up+down launch): a counter thread 0 adds signal_add to once every
// thread has waited for all its earlier vector-memory operations (vmcnt 0)
// and a block barrier has followed, i.e. once the previous tile's stores are
// complete; with two stages that is the first K step's wait.
template <int BM, int BN, bool A_KC, bool B_KC, int MODE, int EPI, int CO = 0, bool XS = false,
          int NT = kThreads>
__device__ __forceinline__ void gemm_dl_tile(const GemmArgs& pa, const TileCoord& tc, int k0, int k1,
                                             int role, int slot, int key, bf16_t* xsm = nullptr,
                                             int* signal = nullptr, int signal_add = 1) {
  // a tile of the extra dense group reads and writes its own tensors
  GemmArgs p = pa;
  if (__builtin_amdgcn_readfirstlane(tc.extra ? 1 : 0)) {  // block-uniform: keeps p's pointers scalar
    p.A = pa.xA;
    p.B = pa.xB;
    p.C = pa.xC;
    p.C2 = pa.xC2;
    p.up = pa.xUp;
    p.act = pa.x_act;
    p.b_stride = 0;
    p.c_stride = 0;
  }
  // NT / 64 waves in a 2 x (NT / 128) grid over the tile
  static_assert(NT == 256 || NT == 512, "four or eight waves");
  constexpr int WGN = NT / 128;
  constexpr int WM = BM / 2, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_EL = BM * DL_BK, B_EL = BN * DL_BK;  // elements per stage tile
  constexpr int STAGE = A_EL + B_EL;
  constexpr int LA = BM * DL_BK / 8 / NT;  // 16-byte loads per thread per stage
  constexpr int LB = BN * DL_BK / 8 / NT;
  constexpr int LDC = BN + 8;                // C staging row stride
  constexpr int NS = dl_stages<BM, BN>();
  constexpr int SMEM = dl_smem_elems<BM, BN>();
  static_assert(SMEM == ((NS * STAGE > BM * LDC) ? NS * STAGE : BM * LDC), "LDS size");
  static_assert(SMEM * 2 <= 160 * 1024, "LDS budget");
  constexpr int NF = TM * TN * 4;            // fp32 partial: float4s per thread
  static_assert(EPI != EPI_GLU_FWD || (TN % 2 == 0), "GLU forward pairs gate/up tiles");
  __shared__ __attribute__((aligned(1024))) bf16_t smem_own[XS ? 1 : SMEM];
  bf16_t* const smem = XS ? xsm : smem_own;

  // tile coordinates are block-uniform; readfirstlane keeps them (and the
  // buffer descriptors built from them) in scalar registers even where the
  // compiler cannot prove the loads they came from uniform
  const int e = __builtin_amdgcn_readfirstlane(tc.e);
  const int m0 = __builtin_amdgcn_readfirstlane(tc.m0);
  const int n0 = __builtin_amdgcn_readfirstlane(tc.n0);
  const int row_begin = __builtin_amdgcn_readfirstlane(tc.row_begin);
  const int row_end = __builtin_amdgcn_readfirstlane(tc.row_end);
  const int K = (MODE == 0) ? p.K : (row_end - row_begin);
  const int a0 = (EPI == EPI_GLU_FWD) ? n0 / 2 : 0;

  // per-thread addressing is recomputed for every tile: hoisted out of a
  // persistent block's tile loop it would occupy registers the whole time
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wm = wave >> (WGN / 2), wn = wave & (WGN - 1);

  // buffer descriptors: reads outside [base, base + bytes) return zero
  __amdgpu_buffer_rsrc_t ra, rb;
  if constexpr (MODE == 0) {
    const int rows = min(row_end - row_begin, BM);
    ra = make_rsrc(p.A + static_cast<int64_t>(row_begin) * p.lda,
                   static_cast<uint32_t>(rows * p.lda * 2));
    const bf16_t* Be = p.B + static_cast<int64_t>(e) * p.b_stride;
    const int64_t brows = B_KC ? ((EPI == EPI_GLU_FWD) ? 2 * static_cast<int64_t>(p.H) : p.N) : p.K;
    rb = make_rsrc(Be, static_cast<uint32_t>(brows * p.ldb * 2));
  } else {
    const int64_t rows = row_end - row_begin;
    ra = make_rsrc(p.A + static_cast<int64_t>(row_begin) * p.lda, static_cast<uint32_t>(rows * p.lda * 2));
    rb = make_rsrc(p.B + static_cast<int64_t>(row_begin) * p.ldb, static_cast<uint32_t>(rows * p.ldb * 2));
  }

  // per-thread byte offsets of its stage-0 chunks (the k step adds a stride)
  uint32_t offa[LA], offb[LB];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int pos = i * NT + tid;
    if constexpr (A_KC) {
      const int r = pos >> 3, c = (pos & 7) ^ ((r >> 1) & 7);
      offa[i] = static_cast<uint32_t>((r * p.lda + c * 8) * 2);
    } else {
      const int k = pos / (BM / 8), c = (pos % (BM / 8)) ^ mn_swz<BM>(k);
      offa[i] = static_cast<uint32_t>((k * p.lda + m0 + c * 8) * 2);
    }
  }
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    const int pos = i * NT + tid;
    if constexpr (B_KC) {
      const int r = pos >> 3, c = (pos & 7) ^ ((r >> 1) & 7);
      int brow;
      if constexpr (EPI == EPI_GLU_FWD) {
        const int a = a0 + (r % (BN / 2));
        brow = (r < BN / 2) ? a : p.H + a;
      } else {
        brow = n0 + r;
      }
      offb[i] = static_cast<uint32_t>((static_cast<int64_t>(brow) * p.ldb + c * 8) * 2);
    } else {
      const int k = pos / (BN / 8), c = (pos % (BN / 8)) ^ mn_swz<BN>(k);
      offb[i] = static_cast<uint32_t>((k * p.ldb + n0 + c * 8) * 2);
    }
  }
  // byte advance of one K step
  const uint32_t stepa = A_KC ? DL_BK * 2 : static_cast<uint32_t>(DL_BK * p.lda * 2);
  const uint32_t stepb = B_KC ? DL_BK * 2 : static_cast<uint32_t>(DL_BK * p.ldb * 2);

  if (k1 < 0) k1 = (K + DL_BK - 1) / DL_BK;
  // Loads of K step `kstep` into stage buffer `buf`.  Steps past k1 are still
  // issued, with an out-of-range offset (the buffer returns zeros and moves no
  // memory), so every step has the same number of loads in flight.
  // A stage's loads go out in IP parts: part 0 with the last k-step of the
  // stage before (right after the barrier that frees the buffer), parts
  // 1..IP-1 with the next k-steps, so the LDS writes of a stage arrive spread
  // over the step instead of in one burst.
  constexpr int IP = issue_parts<BM, BN, EPI, NT>();
  static_assert(LA % IP == 0 && LB % IP == 0 && IP <= 4, "issue parts");
  constexpr int PA = LA / IP, PB = LB / IP;
  auto issue_part = [&](int kstep, int buf, int part) {
    bf16_t* at = smem + buf * STAGE;
    bf16_t* bt = at + A_EL;
    const bool live = kstep < k1;
#pragma unroll
    for (int i = part * PA; i < (part + 1) * PA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (lds_void_t*)(at + (i * NT + wave * 64) * 8), 16,
          live ? offa[i] + kstep * stepa : 0xFFFFFFF0u, 0, 0, (CO & kCoLoadA) ? kDeviceScope : 0);
#pragma unroll
    for (int i = part * PB; i < (part + 1) * PB; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (lds_void_t*)(bt + (i * NT + wave * 64) * 8), 16,
          live ? offb[i] + kstep * stepb : 0xFFFFFFF0u, 0, 0, 0);
  };
  auto issue = [&](int kstep, int buf) {
#pragma unroll
    for (int q = 0; q < IP; ++q) issue_part(kstep, buf, q);
  };

  auto tile_col = [&](int tn) {
    if constexpr (EPI == EPI_GLU_FWD)
      return (tn < TN / 2) ? wn * (WN / 2) + tn * 32 : BN / 2 + wn * (WN / 2) + (tn - TN / 2) * 32;
    else
      return wn * WN + tn * 32;
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  static_assert(DL_BK == 64, "four MFMA k-steps per stage");
  // MFMA operand fragments of one k-step (16 of K), double-buffered in
  // registers (sets F0 / F1): the reads of one set overlap the MFMAs of the
  // other.  k-step 0 of stage kt+1 is read right after the barrier that
  // publishes it, during k-step 3 of stage kt.
  bf16x8_t fa0[TM], fb0[TN], fa1[TM], fb1[TN];
  // every fragment read is asm (ds_read_b128 / ds_read_b64_tr_b16) and
  // lds_frags_ready() does the waiting, one lgkmcnt(0) per fragment set:
  // with a transpose-read operand the compiler's own waits would count the
  // untracked asm reads; with two K-contiguous operands its per-fragment
  // waits were measured slower (C2 up+down 258-260 against 254-255 us)
  auto read_kc = [&](const bf16_t* ptr) { return lds_read_b128_asm(ptr); };
  auto read_ks = [&](int buf, int ks, bf16x8_t (&fa)[TM], bf16x8_t (&fb)[TN]) {
    const bf16_t* at = smem + buf * STAGE;
    const bf16_t* bt = at + A_EL;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int r0 = wm * WM + tm * 32;
      if constexpr (A_KC) {
        const int r = r0 + (lane & 31);
        const int c = (ks * 2 + (lane >> 5)) ^ ((r >> 1) & 7);
        fa[tm] = read_kc(at + r * DL_BK + c * 8);
      } else {
        fa[tm] = lds_frag_mn_sw<BM>(at, r0, ks, lane);
      }
    }
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int c0 = tile_col(tn);
      if constexpr (B_KC) {
        const int r = c0 + (lane & 31);
        const int c = (ks * 2 + (lane >> 5)) ^ ((r >> 1) & 7);
        fb[tn] = read_kc(bt + r * DL_BK + c * 8);
      } else {
        fb[tn] = lds_frag_mn_sw<BN>(bt, c0, ks, lane);
      }
    }
  };
  auto mfma_ks = [&](const bf16x8_t (&fa)[TM], const bf16x8_t (&fb)[TN]) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[tn], fa[tm], acc[tm][tn], 0, 0, 0);
  };
  // LDS fragment reads per k-step (a transpose-read fragment takes two)
  constexpr int NR = (A_KC ? TM : 2 * TM) + (B_KC ? TN : 2 * TN);
  constexpr int NM = TM * TN;  // MFMAs per k-step
  constexpr int kLoads = LA + LB;  // loads per thread per stage
  static_assert(kLoads < 64, "vmcnt range");
  static_assert((NS - 1) * kLoads < 64, "vmcnt range");
  // prologue: stage 0 landed (stages 1..NS-2 and part 0 of stage NS-1 may
  // be in flight), LDS count free
  constexpr int kPart = kLoads / IP;  // loads per thread per issue part
  constexpr int kPro = (NS - 2) * kLoads + kPart;
  constexpr int kWaitStage0 = (kPro & 15) | ((kPro >> 4) << 14) | 0x70 | 0xF00;
  // in the loop: the next stage landed (the NS-2 after it may be in flight)
  // and this wave's LDS reads retired
  constexpr int kIn = (NS - 2) * kLoads;
  constexpr int kWaitNext = (kIn & 15) | ((kIn >> 4) << 14) | 0x70;

  // Scheduling of one k-step region: pair each LDS read and each stage load
  // with an MFMA, so one wave per SIMD issues them in the MFMAs' shadow.
  auto interleave = [&](int nvmem) {
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);      // MFMA
      if (i < nvmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
      if (i < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // DS read
    }
  };

  // GLU backward: the pre-activation values of the tile are loaded during
  // the last stage's k-steps (their latency hides under its MFMAs).  Buffer
  // loads (rows past the group read zeros), so every thread issues exactly
  // 2 * PIT of them, after the last stage load: the wait before the epilogue
  // can then leave them in flight (vector-memory loads complete in order).
  constexpr int PIT = (EPI == EPI_GLU_BWD) ? glu_bwd_items<BM, BN, NT>() : 1;
  uint4 pre_g[PIT], pre_u[PIT];
  auto prefetch_up = [&]() {
    if constexpr (EPI == EPI_GLU_BWD) {
      constexpr int CH = BN / 8;
      const int64_t H2 = 2 * static_cast<int64_t>(p.H);
      const int rows = max(0, min(row_end - row_begin, BM));
      const __amdgpu_buffer_rsrc_t ru =
          make_rsrc_u(p.up + static_cast<int64_t>(row_begin) * H2, static_cast<uint32_t>(rows * H2 * 2));
#pragma unroll
      for (int it = 0; it < PIT; ++it) {
        const int idx = it * NT + tid;
        const uint32_t off = static_cast<uint32_t>(((idx / CH) * H2 + n0 + (idx % CH) * 8) * 2);
        pre_g[it] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ru, off, 0, 0));
        pre_u[it] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ru, off + p.H * 2, 0, 0));
      }
      asm volatile("" ::: "memory");
    }
  };
  const int nks = k1 - k0;
  if (nks > 0) {
#pragma unroll
    for (int s = 0; s + 1 < NS; ++s) issue(k0 + s, s);
    issue_part(k0 + NS - 1, NS - 1, 0);
    // the stage whose parts 1..IP-1 go out with the next k-steps
    int pend_step = k0 + NS - 1, pend_buf = NS - 1;
    // k-step j (0, 1, 2) of a stage issues part j + 1 of the pending stage
    auto issue_pending = [&](int j) {
      if constexpr (IP > 1) {
        if (j + 1 < IP) issue_part(pend_step, pend_buf, j + 1);
      }
    };
    constexpr int kSub0 = IP > 1 ? kPart : 0, kSub1 = IP > 2 ? kPart : 0, kSub2 = IP > 3 ? kPart : 0;
    __builtin_amdgcn_s_waitcnt(kWaitStage0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_ks(0, 0, fa0, fb0);
    // wait for a fragment set (asm reads) before its MFMAs
    auto ready = [&](bf16x8_t (&fa)[TM], bf16x8_t (&fb)[TN]) { lds_frags_ready(fa, fb); };
    int cur = 0;  // ring buffer of the stage being computed
    for (int i = 0; i + 1 < nks; ++i) {
      ready(fa0, fb0);
      read_ks(cur, 1, fa1, fb1);
      mfma_ks(fa0, fb0);
      issue_pending(0);
      interleave(kSub0);
      ready(fa1, fb1);
      read_ks(cur, 2, fa0, fb0);
      mfma_ks(fa1, fb1);
      issue_pending(1);
      interleave(kSub1);
      ready(fa0, fb0);
      read_ks(cur, 3, fa1, fb1);
      mfma_ks(fa0, fb0);
      issue_pending(2);
      interleave(kSub2);
      ready(fa1, fb1);
      // publish the next stage; every wave's reads of this one have retired
      __builtin_amdgcn_s_waitcnt(kWaitNext);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if constexpr (kIn == 0) {
        if (i == 0 && signal != nullptr && tid == 0)
          __hip_atomic_fetch_add(signal, signal_add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // refill this stage's buffer NS steps ahead (part 0 now, the rest with
      // the next k-steps), read k-step 0 of the next stage, run k-step 3 of
      // this one
      pend_step = k0 + i + NS;
      pend_buf = cur;
      issue_part(pend_step, pend_buf, 0);
      const int nxt = cur + 1 == NS ? 0 : cur + 1;
      read_ks(nxt, 0, fa0, fb0);
      mfma_ks(fa1, fb1);
      interleave(kPart);
      cur = nxt;
    }
    prefetch_up();
    ready(fa0, fb0);
    read_ks(cur, 1, fa1, fb1);
    mfma_ks(fa0, fb0);
    ready(fa1, fb1);
    read_ks(cur, 2, fa0, fb0);
    mfma_ks(fa1, fb1);
    ready(fa0, fb0);
    read_ks(cur, 3, fa1, fb1);
    mfma_ks(fa0, fb0);
    ready(fa1, fb1);
    mfma_ks(fa1, fb1);
  } else {
    prefetch_up();
  }
  if constexpr (EPI == EPI_GLU_BWD) {
    // the stage loads (and their LDS writes) done; the 2 * PIT pre-activation
    // loads issued after them may still be in flight
    constexpr int kUp = 2 * PIT;
    static_assert(kUp < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((kUp & 15) | ((kUp >> 4) << 14) | 0x70 | 0xF00);
  } else {
    wait_vmcnt_le(0);
  }
  __syncthreads();
  if (signal != nullptr && (kIn != 0 || nks < 2) && tid == 0)
    __hip_atomic_fetch_add(signal, signal_add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  if (role == ROLE_SPLIT) {
    // row r of the tile holds output row row_begin + r (grouped rows) or
    // m0 + r (grouped K); slab rows are output rows
    float* slab = p.part + static_cast<int64_t>(slot) * p.split_rows * p.N;
    const int rlim = (MODE == 0) ? row_end : p.M;
    const int rbase = (MODE == 0) ? row_begin : m0;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = rbase + wm * WM + tm * 32 + (lane & 31);
          const int col = n0 + tile_col(tn) + 8 * q + 4 * (lane >> 5);
          if (row < rlim && col < p.N)
            *reinterpret_cast<float4*>(slab + static_cast<int64_t>(row) * p.N + col) =
                make_float4(acc[tm][tn][4 * q], acc[tm][tn][4 * q + 1], acc[tm][tn][4 * q + 2],
                            acc[tm][tn][4 * q + 3]);
        }
    return;
  }

  // cut tile: counter flags[key], publication flags[G + key] (= slot + 1)
  int partner = 0;
  if (role == ROLE_CUT) {
    int* s_word = reinterpret_cast<int*>(smem);
    if (tid == 0)
      *s_word = __hip_atomic_fetch_add(p.flags + key, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const bool first = *s_word == 0;
    __syncthreads();
    if (first) {
      // publish the fp32 partial: coalesced 16-byte stores in register
      // order.  They are device-scope stores (sc1: written through to the
      // level all XCDs share, as relaxed agent-scope atomic stores are), so
      // completing them (vmcnt 0) is all that must precede the publication;
      // no L2 write-back is needed.  Buffer stores take each store's offset
      // from a scalar constant, so no address registers are kept per store.
      const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.part + static_cast<int64_t>(slot) * NF * NT * 4,
                                                  NF * NT * 16);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4_t v = {acc[tm][tn][4 * q], acc[tm][tn][4 * q + 1], acc[tm][tn][4 * q + 2],
                               acc[tm][tn][4 * q + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), rp, tid * 16,
                                                   ((tm * TN + tn) * 4 + q) * NT * 16, kDeviceScope);
          }
          __builtin_amdgcn_sched_barrier(0);  // one 32x32 tile of accumulator reads at a time
        }
      wait_vmcnt_le(0);
      __syncthreads();
      if (tid == 0)
        __hip_atomic_store(p.flags + p.pub_off + key, slot + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    // second arrival: wait for the publication (bounded: its writer is past
    // the counter, i.e. running), then clear both words for the next launch
    if (tid == 0) {
      int src = 0, polls = 0;
      while ((src = __hip_atomic_load(p.flags + p.pub_off + key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0 &&
             ++polls < kSpinLimit)
        __builtin_amdgcn_s_sleep(8);
      if (src != 0) {
        __hip_atomic_store(p.flags + key, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.flags + p.pub_off + key, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        // Never expected.  The tile is finished without the partner's
        // partial and the error word is set; both flag words are left as
        // they are (the partner may still publish), so the workspace stays
        // unusable until ffmoe_gemm_check() reports the error and clears it.
        __hip_atomic_store(p.flags + p.err_idx, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      *s_word = src - 1;  // -1: no partial to add
    }
    __syncthreads();  // the partial is read below with device-scope loads
    partner = __builtin_amdgcn_readfirstlane(*s_word);  // block-uniform: a scalar descriptor below
    __syncthreads();
  }

  // epilogue: every wave stages its bf16 accumulators in the LDS C tile (one
  // 32x32 MFMA tile at a time; the scheduling barriers keep the compiler from
  // hoisting all accumulator reads, which would spill), then the block stores
  // the whole tile
  // (the second block of a cut tile adds the first's fp32 partial here, so
  // the accumulators are only ever written by the MFMAs)
  bf16_t* Cs = smem;
  const int lr = lane & 31;
  const int lq = (lane >> 5) * 4;
  const __amdgpu_buffer_rsrc_t rpart =
      make_rsrc(p.part + static_cast<int64_t>(partner < 0 ? 0 : partner) * NF * NT * 4,
                NF * NT * 16);
  auto stage = [&](auto add) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int ml = wm * WM + tm * 32 + lr;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int nl = tile_col(tn) + lq;
        if constexpr (decltype(add)::value) {
          f32x4_t pv[4];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            pv[q] = __builtin_bit_cast(
                f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                             rpart, tid * 16, ((tm * TN + tn) * 4 + q) * NT * 16, kDeviceScope));
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<uint2*>(Cs + ml * LDC + nl + q * 8) =
                pack4(acc[tm][tn][4 * q] + pv[q][0], acc[tm][tn][4 * q + 1] + pv[q][1],
                      acc[tm][tn][4 * q + 2] + pv[q][2], acc[tm][tn][4 * q + 3] + pv[q][3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<uint2*>(Cs + ml * LDC + nl + q * 8) =
                pack4(acc[tm][tn][4 * q], acc[tm][tn][4 * q + 1], acc[tm][tn][4 * q + 2],
                      acc[tm][tn][4 * q + 3]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  if (role == ROLE_CUT && partner >= 0) stage(std::true_type{});
  else stage(std::false_type{});
  __syncthreads();
  if constexpr (EPI == EPI_GLU_BWD)
    glu_bwd_store<BM, BN, LDC, NT>(p, Cs, row_begin, row_end, n0, pre_g, pre_u);
  else
    store_c_tile<BM, BN, LDC, MODE, EPI, (CO & kCoStoreC) != 0, NT>(p, Cs, e, m0, row_begin, row_end, n0, a0);
  __syncthreads();  // the C tile is read before a next tile's loads refill the LDS
}

constexpr int kLptMaxE = 1024;  // experts the skew-balanced wgrad order handles
// Flag words of the split dense-group wgrad tiles in the persistent GEMMs'
// workspace: counters [kPairKey, kPairKey + kPairMax), publications
// kPairPubOff words further on.  The persistent GEMMs' own words take
// [0, 2G] (G = CUs), so this needs 2G < kPairKey.
constexpr int kPairKey = 1024;
constexpr int kPairPubOff = 512;
constexpr int kPairMax = 512;

// Body of the one-block-per-tile kernels.
template <int BM, int BN, bool A_KC, bool B_KC, int MODE, int EPI, int NT = kThreads>
__device__ __forceinline__ void gemm_dl_body(const GemmArgs& p) {
  TileCoord tc;
  if constexpr (MODE == 0) {
    // Blocks are dispatched round-robin over the 8 XCDs (XCD x runs blocks
    // x, x + 8, ...).  The grid covers an upper bound of row tiles; the R
    // real ones (known on the device) are split evenly, each XCD taking a
    // contiguous run, so no XCD runs a round more than the others.
    const int R = ld_const(p.tile_offsets, p.E) + extra_tiles<BM>(p);
    const int64_t T = static_cast<int64_t>(R) * p.n_tiles;
    const int64_t per = (T + 7) / 8;
    const int64_t idx = blockIdx.x >> 3;
    const int64_t tile = (blockIdx.x & 7) * per + idx;
    if (idx >= per || tile >= T) return;
    tc = decode_rows_tile<BM, BN>(p, tile, R);
  } else {
    // Off the skewed path each XCD takes a contiguous run of tiles (block
    // x + 8 s runs on XCD x), so neighbouring tiles share its L2.
    const int64_t per = (p.total_tiles + 7) / 8;
    const int64_t idx = blockIdx.x >> 3;
    const int64_t tile = (blockIdx.x & 7) * per + idx;
    const bool in_run = idx < per && tile < p.total_tiles;
    if (in_run) tc = decode_k_tile<BM, BN>(p, tile);
    bool skewed = false;
    if (p.lpt) {
      // An expert's tiles all take K = its row count, so when one expert
      // holds at least 1.5x the mean row count, the XCD holding its tiles
      // sets the launch time.  Every wave reads the counts and takes the
      // same decision (one ballot), so the test needs no block barrier.
      // Loads go out four per lane at a time (clamped in range) before any
      // is waited for.
      // the extra dense group (if any) is group E (and E + 1: its second K half)
      const int NG = p.E + extra_groups(p);
      const int64_t total3 = 3 * (static_cast<int64_t>(p.offsets[p.E] - p.offsets[0]) + (p.x_rows > 0 ? p.x_rows : 0));
      bool heavy = false;
      for (int i0 = threadIdx.x & 63; i0 < NG; i0 += 256) {
        int cnt[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) cnt[u] = group_rows(p, min(i0 + 64 * u, NG - 1));
#pragma unroll
        for (int u = 0; u < 4; ++u)
          heavy |= i0 + 64 * u < NG && 2 * static_cast<int64_t>(cnt[u]) * NG >= total3;
      }
      skewed = __ballot(heavy && total3 > 0) != 0;
    }
    if (skewed) {
      // Every XCD takes a contiguous slice of ceil(per_e / 8) tiles of every
      // group, and the groups are visited heaviest first (ties: lower
      // index first), so the long tiles start at once and the short ones
      // fill in behind them.
      __shared__ int s_cnt[kLptMaxE + 2];
      __shared__ int s_sel;
      const int NG = p.E + extra_groups(p);
      const int per_e = p.m_tiles * p.n_tiles;
      const int c = (per_e + 7) / 8;
      const int sl = static_cast<int>(blockIdx.x >> 3);
      const int r = sl / c;                                           // rank of the group
      const int sub = static_cast<int>(blockIdx.x & 7) * c + sl % c;  // its tile
      if (r >= NG || sub >= per_e) return;
      for (int i = threadIdx.x; i < NG; i += NT) s_cnt[i] = group_rows(p, i);
      __syncthreads();
      for (int i = threadIdx.x; i < NG; i += NT) {
        const int ci = s_cnt[i];
        int rank = 0;
        for (int j = 0; j < NG; ++j) {
          const int cj = s_cnt[j];
          rank += (cj > ci) || (cj == ci && j < i);
        }
        if (rank == r) s_sel = i;
      }
      __syncthreads();
      tc = decode_k_tile<BM, BN>(p, static_cast<int64_t>(s_sel) * per_e + sub);
    } else if (!in_run) {
      return;
    }
  }
  if (!tc.valid) return;
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only needs the launch stub
  if (MODE == 1 && tc.extra && p.x_split > 1)  // one K half of a split dense-group tile
    gemm_dl_tile<BM, BN, A_KC, B_KC, MODE, EPI, 0, false, NT>(p, tc, 0, -1, ROLE_CUT, tc.xt, kPairKey + tc.xt);
  else
    gemm_dl_tile<BM, BN, A_KC, B_KC, MODE, EPI, 0, false, NT>(p, tc, 0, -1, ROLE_FULL, 0, 0);
#endif
}

// One block per tile.
template <int BM, int BN, bool A_KC, bool B_KC, int MODE, int EPI>
__global__ __launch_bounds__(kThreads, 1) void gemm_dl_kernel(GemmArgs p) {
  gemm_dl_body<BM, BN, A_KC, B_KC, MODE, EPI>(p);
}

// The same with eight waves (two per SIMD, a 2 x 4 grid of wave tiles, at
// most 256 registers a lane): while one wave of a SIMD waits on its loads
// or LDS reads the other issues MFMAs (256 x 256 up GEMM: K step 3.17 k ->
// 2.57 k cycles).
template <int BM, int BN, bool A_KC, bool B_KC, int MODE, int EPI>
__global__ __launch_bounds__(512, 1) void gemm_dl8_kernel(GemmArgs p) {
  gemm_dl_body<BM, BN, A_KC, B_KC, MODE, EPI, 512>(p);
}

// Grouped rows with eight waves, the last hx tiles of each XCD's run (of
// ceil(T / 8) tiles, T known on the device) cut into two row halves
// (BM/2 x BN), so each XCD's last round is made of shorter items; the grid
// covers the host's upper bound of tiles plus hx items per XCD.
template <int BM, int BN, bool A_KC, bool B_KC, int EPI>
__global__ __launch_bounds__(512, 1) void gemm_dl8h_kernel(GemmArgs p, int hx) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only needs the launch stub
  // one LDS array for both tile shapes (with two, the compiler scopes the
  // direct-to-LDS loads by variable and waits on all of them)
  constexpr int S1 = dl_smem_elems<BM, BN>(), S2 = dl_smem_elems<BM / 2, BN>();
  __shared__ __attribute__((aligned(1024))) bf16_t sm[S1 > S2 ? S1 : S2];
  const int R = ld_const(p.tile_offsets, p.E) + extra_tiles<BM>(p);
  const int64_t T = static_cast<int64_t>(R) * p.n_tiles;
  const int64_t per = (T + 7) / 8;
  const int64_t h = min(static_cast<int64_t>(hx), per);
  const int64_t idx = blockIdx.x >> 3;
  const int64_t base = static_cast<int64_t>(blockIdx.x & 7) * per;
  if (idx < per - h) {
    if (base + idx >= T) return;
    const TileCoord tc = decode_rows_tile<BM, BN>(p, base + idx, R);
    if (!tc.valid) return;
    gemm_dl_tile<BM, BN, A_KC, B_KC, 0, EPI, 0, true, 512>(p, tc, 0, -1, ROLE_FULL, 0, 0, sm);
  } else if (idx < per + h) {
    const int64_t v = idx - (per - h);
    const int64_t tile = base + (per - h) + v / 2;
    if (tile >= T) return;
    TileCoord tc = decode_rows_tile<BM, BN>(p, tile, R);
    tc.row_begin += static_cast<int>(v & 1) * (BM / 2);
    if (!tc.valid || tc.row_begin >= tc.row_end) return;  // an empty second half
    gemm_dl_tile<BM / 2, BN, A_KC, B_KC, 0, EPI, 0, true, 512>(p, tc, 0, -1, ROLE_FULL, 0, 0, sm);
  }
#endif
}


// Fused up+down launch: the up GEMM with its GLU epilogue and the down GEMM
// in one persistent grid (G blocks, a multiple of 8), so the down tiles of
// finished row tiles fill the up GEMM's last, partial round.  Words of
// p.fused (zero on entry; the last block out zeroes them again):
//   [0, 8)                   up-tile claim counters of the 8 XCD slots
//   kFusedDown               down-tile claim counter
//   kFusedExit               blocks that have left
//   kFusedHalf               half-tile claim counter (see below)
//   [kFusedRow0, + R)        finished up tiles of each row tile, in halves
// Up tiles, in grouped order, are cut into chunks of S = G / 8; chunk c
// belongs to slot c % 8, so in round k each XCD runs one chunk and the
// chunks start in tile order.  A block claims up tiles from its own slot
// (blockIdx % 8: the XCD it is dispatched to), then from any slot that still
// has some, and only then claims down tiles (row-major, the order the row
// tiles finish in).  A down tile waits until all up tiles of its row tile
// are counted; by then every up tile has been claimed by a running block and
// up tiles wait for nothing, so the wait ends without any co-residency
// guarantee (it is bounded all the same: a timeout sets the error word).
// Staggered start: every block would otherwise reach its up-tile epilogue
// (192 KiB of stores at 256 x 256) at the same moment as all the others, and
// the stores of all CUs at once run at the XCDs' write bandwidth.  So the
// odd blocks of each slot (blockIdx / 8 odd) begin with half of one of the
// slots' first NH tiles (256 x 128: 64 gate and 64 up columns, claimed from
// one counter) and take their next tiles half a tile's time after the even
// blocks; claims of whole tiles start at each slot's tile NH.  Row counts
// are kept in halves (a whole tile adds 2, a half 1; a row tile is complete
// at 2 * NU).  At the other end, the last G/4 down tiles are cut into row
// halves.  Measured at C2 with the odd blocks held back instead: per up
// tile the store phase 14k -> 9.4k cycles, its next tile's first stage
// 11k -> 7k.
// Each claim for the next tile is issued before the current tile, so its
// latency hides under the tile (it is the oldest vector-memory operation of
// the tile's waves, which only makes the tile's counted waits stricter).  The act rows cross blocks (and XCDs):
// up tiles store them with device-scope stores completed before the row
// count moves, down tiles load them with device-scope loads.
constexpr int kFusedDown = 8, kFusedExit = 9, kFusedHalf = 10, kFusedRow0 = 16;
constexpr int kFusedWords = 16384;
constexpr int64_t kFusedBytes = kFusedWords * 4;

template <int BM>
__global__ __launch_bounds__(kThreads, 1) void gemm_updown_kernel(GemmArgs pu, GemmArgs pd) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only needs the launch stub
  constexpr int BNU = 256, BND = 128;
  constexpr int SU = dl_smem_elems<BM, BNU>(), SD = dl_smem_elems<BM, BND>();
  // One LDS variable: with a second one the compiler scopes the
  // direct-to-LDS loads by variable and then waits for all of them (vmcnt 0)
  // before LDS reads in the K loops.  The claim words follow the tiles' area.
  constexpr int SMAX = SU > SD ? SU : SD;
  __shared__ __attribute__((aligned(1024))) bf16_t sm[SMAX + 8];
  int* const s_word = reinterpret_cast<int*>(sm + SMAX);
  int* const fl = pu.fused;
  const int tid = threadIdx.x;
  const int R = ld_const(pu.tile_offsets, pu.E) + extra_tiles<BM>(pu);
  const int NU = pu.n_tiles, ND = pd.n_tiles;
  const int64_t TU = static_cast<int64_t>(R) * NU, TD = static_cast<int64_t>(R) * ND;
  const int S = static_cast<int>(gridDim.x >> 3);
  // up tile of claim j of slot x (>= TU once the slot is empty)
  auto up_tile = [&](int j, int x) { return (static_cast<int64_t>(j / S) * 8 + x) * S + j % S; };
  auto fetch_add = [&](int w) { return __hip_atomic_fetch_add(fl + w, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  // The claim of the next tile: one atomic add, from lane 0 of wave 0 (the
  // other waves run the instruction with no lane on), returning into that
  // lane with no wait.  It is written in assembly because compiled code
  // waits for the value where a one-lane branch rejoins; thread 0 reads it
  // only after a vmcnt(0) wait at the end of the tile.
  auto claim_ahead = [&](int w) {
    int v;
    uint64_t save;
    const int lanes = __builtin_amdgcn_readfirstlane(threadIdx.x < 64 ? 1 : 0);
    asm volatile(
        "s_mov_b64 %1, exec\n\t"
        "s_mov_b32 exec_lo, %4\n\t"
        "s_mov_b32 exec_hi, 0\n\t"
        "global_atomic_add %0, %2, %3, off sc0\n\t"
        "s_mov_b64 exec, %1"
        : "=&v"(v), "=&s"(save)
        : "v"(fl + w), "v"(1), "s"(lanes)
        : "memory");
    return v;
  };
  // one claim, broadcast to the block
  auto claim = [&](int w) {
    if (tid == 0) s_word[0] = fetch_add(w);
    __syncthreads();
    const int v = s_word[0];
    __syncthreads();
    return v;
  };
  const int home = static_cast<int>(blockIdx.x & 7);
  int x = home;
  int prev_row = -1;  // row tile of this block's last up tile, not yet counted
  int prev_w = 0;     // its weight in the row count: 2 (whole tile) or 1 (half)
  // Each slot's first NH tiles are done as halves: half item hh (of HT, one
  // counter) is half hh >> 3 & 1 of tile (hh >> 4) of slot hh & 7.
  const int NH = (S / 2) / 2;
  const int HT = 16 * NH;
  auto half_tile = [&](int hh) {
    const int64_t t = up_tile(hh >> 4, hh & 7);
    if (t >= TU) return;
    int mt, nt;
    grouped_order(t, R, NU, &mt, &nt);
    const TileCoord tc = decode_rows_mn<BM, BNU / 2>(pu, mt, 2 * nt + ((hh >> 3) & 1));
    gemm_dl_tile<BM, BNU / 2, true, true, 0, EPI_GLU_FWD, kCoStoreC, true>(
        pu, tc, 0, -1, ROLE_FULL, 0, 0, sm, prev_row >= 0 ? fl + kFusedRow0 + prev_row : nullptr, prev_w);
    prev_row = mt;
    prev_w = 1;
  };
  if ((blockIdx.x >> 3) & 1) {
    const int hh = claim(kFusedHalf);
    if (hh < HT) half_tile(hh);
  }
  int j = claim(x) + NH;
  for (;;) {
    const int64_t t = up_tile(j, x);
    if (t >= TU) {
      // this slot is empty: move to the next one (from the home slot on)
      // that is not
      if (tid < 64) {
        const int c = tid < 8 ? __hip_atomic_load(fl + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
        const uint32_t m = static_cast<uint32_t>(__ballot(tid < 8 && up_tile(c + NH, tid) < TU)) & 0xFFu;
        if (tid == 0) {
          const uint32_t rot = ((m >> (home + 1)) | (m << (7 - home))) & 0xFFu;  // bit i: slot home + 1 + i
          s_word[1] = rot ? (home + 1 + __builtin_ctz(rot)) & 7 : -1;
        }
      }
      __syncthreads();
      const int ns = s_word[1];
      __syncthreads();
      if (ns < 0) break;
      x = ns;
      j = claim(x) + NH;
      continue;
    }
    const int nj = claim_ahead(x);  // NH is added once the value is in (after the tile)
    int mt, nt;
    grouped_order(t, R, NU, &mt, &nt);
    const TileCoord tc = decode_rows_mn<BM, BNU>(pu, mt, nt);
    // counts the previous up tile of this block done once its act stores
    // are (during the K loop); it waits for all vector-memory operations
    // (the claim's too) before its epilogue
    gemm_dl_tile<BM, BNU, true, true, 0, EPI_GLU_FWD, kCoStoreC, true>(
        pu, tc, 0, -1, ROLE_FULL, 0, 0, sm, prev_row >= 0 ? fl + kFusedRow0 + prev_row : nullptr, prev_w);
    prev_row = mt;
    prev_w = 2;
    if (tid == 0) s_word[0] = nj;
    __syncthreads();
    j = s_word[0] + NH;
    __syncthreads();
  }
  // no half item is left unclaimed once a block takes down tiles (which wait
  // for their row tiles), so every wait is for blocks already running
  for (int hh = claim(kFusedHalf); hh < HT; hh = claim(kFusedHalf)) half_tile(hh);
  // the last up tile's act stores
  wait_vmcnt_le(0);
  __syncthreads();
  if (prev_row >= 0 && tid == 0)
    __hip_atomic_fetch_add(fl + kFusedRow0 + prev_row, prev_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the last NSD = G/4 down tiles are cut into row halves (128 x BND), which
  // fill the launch's last round with shorter items (C2: 240.5-241.3 ->
  // 235.6-236.1 us; G/8 the same, G/2 and more slower); claimed after each
  // tile (a claim issued ahead would be read on paths the build's assembly
  // check cannot tell apart)
  const int64_t NSD = min(TD / 4, static_cast<int64_t>(gridDim.x / 4));
  // waits until row tile r's up tiles are all counted
  auto wait_row = [&](int r) {
    if (tid == 0) {
      int polls = 0;
      while (__hip_atomic_load(fl + kFusedRow0 + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < 2 * NU) {
        if (++polls >= kSpinLimit) {  // never expected: the tile is computed from whatever act holds
          __hip_atomic_store(pu.flags + pu.err_idx, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    __syncthreads();
  };
  int d = claim(kFusedDown);
  while (d < TD - NSD) {
    const int r = static_cast<int>(d / ND), c = static_cast<int>(d - static_cast<int64_t>(r) * ND);
    wait_row(r);
    const int nd = claim_ahead(kFusedDown);  // after the wait's loads, which it would join
    const TileCoord tc = decode_rows_mn<BM, BND>(pd, r, c);
    gemm_dl_tile<BM, BND, true, true, 0, EPI_STORE, kCoLoadA, true>(pd, tc, 0, -1, ROLE_FULL, 0, 0, sm);
    if (tid == 0) s_word[0] = nd;  // the tile waited for all vector-memory operations before its epilogue
    __syncthreads();
    d = s_word[0];
    __syncthreads();
  }
  while (d < TD + NSD) {
    const int64_t v = d - (TD - NSD), fd = TD - NSD + v / 2;
    const int r = static_cast<int>(fd / ND), c = static_cast<int>(fd - static_cast<int64_t>(r) * ND);
    wait_row(r);
    TileCoord tc = decode_rows_mn<BM, BND>(pd, r, c);
    tc.row_begin += static_cast<int>(v & 1) * (BM / 2);
    if (tc.row_begin < tc.row_end)
      gemm_dl_tile<BM / 2, BND, true, true, 0, EPI_STORE, kCoLoadA, true>(pd, tc, 0, -1, ROLE_FULL, 0, 0, sm);
    d = claim(kFusedDown);
  }
  // the last block out has seen every block finish all its tiles: it clears
  // the words for the next launch
  if (tid == 0) s_word[1] = fetch_add(kFusedExit);
  __syncthreads();
  if (s_word[1] == static_cast<int>(gridDim.x) - 1)
    for (int i = tid; i < kFusedRow0 + R; i += kThreads)
      __hip_atomic_store(fl + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#endif
}

// Fused dgrad + up-side wgrad launch: ghb = gup · w_up[e] (grouped rows,
// BMD x 256 tiles) and dW_up[e] = gupᵀ · x_sorted (grouped K, 256 x 256
// tiles) read the same gup and are independent, so one persistent grid
// runs both tile lists as one: the dgrad tiles (the longer ones: K = 2H)
// first, then the wgrad tiles, groups heaviest first (ties: lower index
// first).  The list is cut into chunks of G/8 tiles; chunk c belongs to XCD
// slot c mod 8; a block claims from its own slot (an atomic counter per
// slot in p.fused's words [0, 8)), then from any slot that still has tiles.
// No tile waits for another (a wgrad tile of a dense group cut along K
// waits only for its partner half, which is already running), and no
// stream-K partials are needed.  Cutting C2's 268 dgrad tiles into K halves
// as well (so the list's items were of similar length) was slower: 316
// against 297 us, the halves' fp32 partials cost more than the shorter tail.
// Claims are made after each tile: issued ahead of it, the claim's return
// register lived across the tile, and under this kernel's register pressure
// the compiler spilled it before the value had arrived.
// The list's last NSP wgrad tiles (G/4 of them, at most a quarter of the
// wgrad tiles) are cut into column halves (256 x 128), so the last round is
// filled by shorter items: at C2 (268 dgrad tiles of ~200k cycles, 512
// wgrad tiles of ~113k on 256 CUs) a greedy list schedule puts the busiest
// CU 24% above the mean with whole tiles and 11% above it with the last 64
// wgrad tiles halved.
template <int BMD, int NT = kThreads>
__global__ __launch_bounds__(NT, 1) void gemm_dw_kernel(GemmArgs pd, GemmArgs pw) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only needs the launch stub
  constexpr int BW = 256;
  constexpr int SD = dl_smem_elems<BMD, 256>(), SW = dl_smem_elems<BW, BW>(), SH = dl_smem_elems<BW, BW / 2>();
  constexpr int SMAX = SD > SW ? (SD > SH ? SD : SH) : (SW > SH ? SW : SH);
  constexpr int kOrd = kLptMaxE + 2;
  // one LDS variable (see gemm_updown_kernel): the tiles' area, then the
  // claim words and the wgrad groups' row counts and order
  __shared__ __attribute__((aligned(1024))) bf16_t sm[SMAX + 2 * (8 + 2 * kOrd)];
  int* const s_word = reinterpret_cast<int*>(sm + SMAX);
  int* const s_cnt = s_word + 8;
  int* const s_ord = s_cnt + kOrd;
  int* const fl = pd.fused;
  const int tid = threadIdx.x;
  const int Rd = ld_const(pd.tile_offsets, pd.E) + extra_tiles<BMD>(pd);
  const int64_t TD = static_cast<int64_t>(Rd) * pd.n_tiles;
  const int NG = pw.E + extra_groups(pw);
  const int per_e = pw.m_tiles * pw.n_tiles;
  const int64_t NGT = static_cast<int64_t>(NG) * per_e;  // whole wgrad tiles
  const int64_t NSP = min(NGT / 4, static_cast<int64_t>(gridDim.x / 4));  // the last ones, halved
  const int64_t TT = TD + NGT + NSP;
  const int S = static_cast<int>(gridDim.x >> 3);
  for (int i = tid; i < NG; i += NT) s_cnt[i] = group_rows(pw, i);
  __syncthreads();
  for (int i = tid; i < NG; i += NT) {
    const int ci = s_cnt[i];
    int rank = 0;
    for (int j = 0; j < NG; ++j) {
      const int cj = s_cnt[j];
      rank += (cj > ci) || (cj == ci && j < i);
    }
    s_ord[rank] = i;
  }
  __syncthreads();
  auto list_tile = [&](int j, int x) { return (static_cast<int64_t>(j / S) * 8 + x) * S + j % S; };
  auto claim = [&](int w) {
    if (tid == 0) s_word[0] = __hip_atomic_fetch_add(fl + w, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int v = s_word[0];
    __syncthreads();
    return v;
  };
  const int home = static_cast<int>(blockIdx.x & 7);
  int x = home;
  int j = claim(x);
  for (;;) {
    const int64_t g = list_tile(j, x);
    if (g >= TT) {
      if (tid < 64) {
        const int c = tid < 8 ? __hip_atomic_load(fl + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
        const uint32_t m = static_cast<uint32_t>(__ballot(tid < 8 && list_tile(c, tid) < TT)) & 0xFFu;
        if (tid == 0) {
          const uint32_t rot = ((m >> (home + 1)) | (m << (7 - home))) & 0xFFu;  // bit i: slot home + 1 + i
          s_word[1] = rot ? (home + 1 + __builtin_ctz(rot)) & 7 : -1;
        }
      }
      __syncthreads();
      const int ns = s_word[1];
      __syncthreads();
      if (ns < 0) break;
      x = ns;
      j = claim(x);
      continue;
    }
    if (g < TD) {
      const TileCoord tc = decode_rows_tile<BMD, 256>(pd, g, Rd);
      gemm_dl_tile<BMD, 256, true, false, 0, EPI_STORE, 0, true, NT>(pd, tc, 0, -1, ROLE_FULL, 0, 0, sm);
    } else {
      // wgrad item: whole tile u, or (past NGT - NSP) half (v & 1) of tile
      // NGT - NSP + v / 2
      const int64_t u0 = g - TD, v = u0 - (NGT - NSP);
      const int64_t u = v < 0 ? u0 : NGT - NSP + v / 2;
      const int r = static_cast<int>(u / per_e);
      TileCoord tc =
          decode_k_tile<BW, BW>(pw, static_cast<int64_t>(s_ord[r]) * per_e + (u - static_cast<int64_t>(r) * per_e));
      if (tc.extra && pw.x_split > 1) {  // one K half of a split dense-group tile (whole in N)
        if (v < 0 || (v & 1) == 0)
          gemm_dl_tile<BW, BW, false, false, 1, EPI_STORE, 0, true, NT>(pw, tc, 0, -1, ROLE_CUT, tc.xt,
                                                                     kPairKey + tc.xt, sm);
      } else if (v < 0) {
        gemm_dl_tile<BW, BW, false, false, 1, EPI_STORE, 0, true, NT>(pw, tc, 0, -1, ROLE_FULL, 0, 0, sm);
      } else {
        tc.n0 += static_cast<int>(v & 1) * (BW / 2);
        gemm_dl_tile<BW, BW / 2, false, false, 1, EPI_STORE, 0, true, NT>(pw, tc, 0, -1, ROLE_FULL, 0, 0, sm);
      }
    }
    j = claim(x);
  }
  // the last block out has seen every block finish all its tiles: it clears
  // the claim words for the next launch
  if (tid == 0) s_word[1] = __hip_atomic_fetch_add(fl + kFusedExit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_word[1] == static_cast<int>(gridDim.x) - 1 && tid < kFusedRow0)
    __hip_atomic_store(fl + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#endif
}

// Persistent grouped-rows GEMM, one block per CU.  The R x n_tiles tiles
// (R = tile_offsets[E], read on the device) are split into whole-tile rounds
// of G tiles, one per block, and a stream-K tail: the last T - (T/G - 1)*G
// tiles' K steps are cut into G equal contiguous ranges, so every block gets
// the same work and block epilogues fall at different times.  A tile cut
// between two blocks is finished by whichever of them gets there second
// (ROLE_CUT); a block only ever waits for one that is already running, so
// the launch needs no co-residency guarantee.
template <int BM, int BN, bool A_KC, bool B_KC, int EPI>
__device__ __forceinline__ void gemm_sk_body(const GemmArgs& p) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only needs the launch stub
  const int G = gridDim.x;
  const int v = (G % 8 == 0) ? static_cast<int>(xcd_remap(blockIdx.x, G)) : static_cast<int>(blockIdx.x);
  const int R = ld_const(p.tile_offsets, p.E) + extra_tiles<BM>(p);
  const int64_t T = static_cast<int64_t>(R) * p.n_tiles;
  const int nk = p.K / DL_BK;
  if (T == 0 || nk == 0) return;
  // whole-tile rounds (all tiles when there are at most G of them)
  const int64_t rounds = T <= G ? 1 : T / G - 1;
  const int64_t base = T <= G ? T : rounds * G;
  const int64_t iters = (T - base) * nk;
  const int64_t S = (iters + G - 1) / G;
  int64_t r = 0;                 // next whole-tile round
  // The stream-K range [g, gend) is walked from its end: every block then
  // starts its range at K step 0 of a tile at the same moment, so the blocks
  // sharing A rows or B columns read the same K slices together (L2 hits);
  // walked forwards, each block would start at its own K offset.
  const int64_t g = v * S;
  int64_t gcur = g + S < iters ? g + S : iters;
  // one call site for every work item keeps a single copy of the tile code
  for (;;) {
    int64_t t;
    int k0 = 0, k1 = nk, role = ROLE_FULL, key = v;
    if (r < rounds) {
      t = r * G + v;
      ++r;
      if (t >= base) continue;
    } else if (gcur > g) {
      const int64_t ts = (gcur - 1) / nk;
      const int64_t tstart = ts * nk;
      k0 = static_cast<int>((g > tstart ? g : tstart) - tstart);
      k1 = static_cast<int>(gcur - tstart);
      if (k0 > 0) {
        role = ROLE_CUT;  // the range's first tile; block v - 1 holds [0, k0)
        key = v - 1;
      } else if (k1 < nk) {
        role = ROLE_CUT;  // the range's last tile; block v + 1 holds [k1, nk)
      }
      t = base + ts;
      gcur = tstart + k0;
    } else {
      break;
    }
    const TileCoord tc = decode_rows_tile<BM, BN>(p, t, R);
    // a block may publish for both of its cut tiles (the start of one, then
    // the end of another) before either partner reads: one slot for each
    gemm_dl_tile<BM, BN, A_KC, B_KC, 0, EPI>(p, tc, k0, k1, role, 2 * v + (k0 == 0 ? 1 : 0), key);
  }
#endif
}

template <int BM, int BN, bool A_KC, bool B_KC, int EPI>
__global__ __launch_bounds__(kThreads, 1) void gemm_sk_kernel(GemmArgs p) {
  gemm_sk_body<BM, BN, A_KC, B_KC, EPI>(p);
}

// Split-K dense GEMM (one row group): block b computes split b % S of tile
// b / S over its contiguous share of the K steps (grouped rows) or of the
// rows (grouped K) and writes an fp32 partial slab; split_reduce_kernel adds
// the S slabs in split order (deterministic) and rounds to bf16 once.
// Dense GEMM of one row group (no offset tables): grouped rows, C [M, N] =
// A [M, K] B (MODE 0), or grouped K over all K rows, C [M, N] = A^T B
// (MODE 1).  With S == 1 each block computes a whole tile and stores bf16;
// with S > 1 block b computes split b % S of tile b / S over its contiguous
// share of the K steps and writes an fp32 partial slab, and
// split_reduce_kernel adds the S slabs in split order (deterministic) and
// rounds to bf16 once.
template <int BM, int BN, bool A_KC, bool B_KC, int MODE>
__global__ __launch_bounds__(kThreads, 1) void gemm_dense_kernel(GemmArgs p, int S) {
  const int64_t t = blockIdx.x / S;
  const int s = static_cast<int>(blockIdx.x % S);
  if (t >= p.total_tiles) return;
  TileCoord tc{};
  int mt, nt;
  grouped_order(t, p.m_tiles, p.n_tiles, &mt, &nt);
  tc.e = 0;
  tc.n0 = nt * BN;
  tc.valid = true;
  int k0 = 0, k1 = -1;
  if constexpr (MODE == 0) {
    tc.row_begin = mt * BM;
    tc.row_end = p.M;
    const int nk = p.K / DL_BK;
    k0 = static_cast<int>(static_cast<int64_t>(nk) * s / S);
    k1 = static_cast<int>(static_cast<int64_t>(nk) * (s + 1) / S);
  } else {
    tc.m0 = mt * BM;
    // the K rows split into S chunks of whole 64-row steps
    const int nk = (p.K + DL_BK - 1) / DL_BK;
    tc.row_begin = static_cast<int>(static_cast<int64_t>(nk) * s / S) * DL_BK;
    tc.row_end = min(static_cast<int>(static_cast<int64_t>(nk) * (s + 1) / S) * DL_BK, p.K);
  }
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass only needs the launch stub
  gemm_dl_tile<BM, BN, A_KC, B_KC, MODE, EPI_STORE>(p, tc, k0, k1, S > 1 ? ROLE_SPLIT : ROLE_FULL, s, 0);
#endif
}

// out[i] = bf16(sum_{s < S} part[s][i]) in split order; 4 outputs per thread.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part, int S, int64_t n,
                                                           bf16_t* __restrict__ out) {
  for (int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x * 4) {
    float4 a = *reinterpret_cast<const float4*>(part + i);
    for (int s = 1; s < S; ++s) {
      const float4 b = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(s) * n + i);
      a.x += b.x;
      a.y += b.y;
      a.z += b.z;
      a.w += b.w;
    }
    *reinterpret_cast<uint2*>(out + i) = make_uint2(pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w));
  }
}

template <int BM, int BN, bool A_KC, bool B_KC, int MODE, int EPI>
static int launch(const GemmArgs& a, hipStream_t st, const char* name) {
  if (a.total_tiles <= 0) return clear_error();
  // the direct-to-LDS pipeline needs whole K steps (grouped-rows mode) and the
  // transpose-read path; everything else takes the register-staged kernel
  const bool dl = g_use_tr && (MODE == 1 || a.K % DL_BK == 0);
  if (a.x_rows > 0 && !dl)
    return set_error(std::string(name) + ": a dense extra group needs K a multiple of 64 and the transpose-read path");
  const int groups = a.E + (a.x_rows > 0 ? (a.x_split > 1 ? 2 : 1) : 0);
  const int64_t grid = (dl && a.lpt) ? static_cast<int64_t>(groups) * 8 * ((a.m_tiles * a.n_tiles + 7) / 8)
                                     : (a.total_tiles + 7) / 8 * 8;
  if (grid > 0x7fffffff) return set_error(std::string(name) + ": problem too large");
  if constexpr (BM == 256 && BN == 256) {
    if (dl) {  // eight waves: measured 3-9% faster for every 256 x 256 GEMM here
      hipLaunchKernelGGL((gemm_dl8_kernel<BM, BN, A_KC, B_KC, MODE, EPI>),
                         dim3(static_cast<unsigned>(grid)), dim3(512), 0, st, a);
      if (check_launch(name)) return 1;
      return clear_error();
    }
  }
  if (dl)
    hipLaunchKernelGGL((gemm_dl_kernel<BM, BN, A_KC, B_KC, MODE, EPI>),
                       dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st, a);
  else if (g_use_tr)
    hipLaunchKernelGGL((gemm_kernel<BM, BN, A_KC, B_KC, MODE, EPI, true>),
                       dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_kernel<BM, BN, A_KC, B_KC, MODE, EPI, false>),
                       dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st, a);
  if (check_launch(name)) return 1;
  return clear_error();
}

// Persistent blocks per device: one per CU.
constexpr int kMaxSkBlocks = 1023;
constexpr int kSkMinK = 4096;
constexpr int kSkMaxRounds = 8;
constexpr int64_t kSkFlagBytes = 8192;  // int32 counters [G], publications [G], error word; zero on entry
constexpr int64_t kSkSlotBytes = 256 * 256 * 4;  // fp32 partial of the largest tile

static int sk_blocks() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = cus < kMaxSkBlocks ? cus : kMaxSkBlocks;
  }
  return cached[dev];
}

// min_k: the persistent schedule is used from this K on.  It moves an fp32
// partial (BM x BN x 4 bytes, written and read once) for every cut tile, so
// it pays where the partial is small against the tile's operand bytes; below
// min_k the GEMM runs one block per tile.
template <int BM, int BN, bool B_KC, int EPI>
static int launch_sk(GemmArgs a, void* ws, int min_k, hipStream_t st, const char* name) {
  if (a.total_tiles <= 0) return clear_error();
  if (ws == nullptr || a.K % DL_BK != 0 || a.K < min_k || !g_use_tr)
    return launch<BM, BN, true, B_KC, 0, EPI>(a, st, name);
  const int G = sk_blocks();
  if (G <= 0) return set_error(std::string(name) + ": cannot query the CU count");
  // at 8 or more rounds of tiles (the host's upper bound) the last round's
  // quantisation is small and the cut tiles' partials cost more than they
  // save: one block per tile (C5: dgrad 4.11 -> 3.75 ms, dgrad+GLU 2.25 ->
  // 2.16 ms; C4: dgrad 1.49 -> 1.44 ms, dgrad+GLU 1.00 -> 0.95 ms)
  if (a.total_tiles >= static_cast<int64_t>(kSkMaxRounds) * G) return launch<BM, BN, true, B_KC, 0, EPI>(a, st, name);
  a.flags = static_cast<int*>(ws);
  a.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kSkFlagBytes);
  a.pub_off = G;
  a.err_idx = 2 * G;
  hipLaunchKernelGGL((gemm_sk_kernel<BM, BN, true, B_KC, EPI>), dim3(G), dim3(kThreads), 0, st, a);
  if (check_launch(name)) return 1;
  return clear_error();
}

// Grouped-rows launch with the row-tile height the caller's tile_offsets were
// computed for.
template <int BN, bool B_KC, int EPI>
static int launch_rows(const GemmArgs& a, int tile_rows, void* ws, int min_k, hipStream_t st,
                       const char* name) {
  if (tile_rows == 256) return launch_sk<256, BN, B_KC, EPI>(a, ws, min_k, st, name);
  return launch_sk<128, BN, B_KC, EPI>(a, ws, min_k, st, name);
}

static GemmArgs rows_args(const int32_t* offsets, const int32_t* tile_offsets, int E,
                          int64_t max_rows, int tile_rows, int n_tiles) {
  GemmArgs a{};
  a.offsets = offsets;
  a.tile_offsets = tile_offsets;
  a.E = E;
  a.n_tiles = n_tiles;
  a.m_tiles = static_cast<int>((max_rows + tile_rows - 1) / tile_rows + E);
  a.total_tiles = static_cast<int64_t>(a.m_tiles) * n_tiles;
  return a;
}

// Adds the extra dense group to grouped-rows arguments (its row tiles after
// the routed ones).
static int apply_shared(GemmArgs& a, const ffmoe_dense_group* g, int tile_rows, const char* name) {
  if (g == nullptr || g->rows <= 0) return 0;
  if (g->a == nullptr || g->b == nullptr || g->c == nullptr || g->rows > 0x7fffffff ||
      g->activation < 0 || g->activation > FFMOE_ACT_GEGLU_ERF)
    return set_error(std::string(name) + ": bad dense extra group");
  a.xA = static_cast<const bf16_t*>(g->a);
  a.xB = static_cast<const bf16_t*>(g->b);
  a.xC = static_cast<bf16_t*>(g->c);
  a.xC2 = static_cast<bf16_t*>(g->c2);
  a.xUp = static_cast<const bf16_t*>(g->up);
  a.x_rows = static_cast<int>(g->rows);
  a.x_act = g->activation;
  a.m_tiles += static_cast<int>((g->rows + tile_rows - 1) / tile_rows);
  a.total_tiles = static_cast<int64_t>(a.m_tiles) * a.n_tiles;
  return 0;
}

static int check_rows(const char* name, int E, int64_t max_rows, int D, int H, int tile_rows) {
  if (E < 1 || E > FFMOE_MAX_EXPERTS || D <= 0 || D % 8 != 0 || H <= 0 || H % 8 != 0 || max_rows < 0)
    return set_error(std::string(name) + ": D and H must be positive multiples of 8");
  if (tile_rows != 128 && tile_rows != 256)
    return set_error(std::string(name) + ": tile_rows must be 128 or 256");
  return 0;
}

}  // namespace ffmoe

using namespace ffmoe;

extern "C" int ffmoe_gemm_tile_rows(int64_t max_rows, int E) {
  // 256-row tiles once experts average at least 384 rows; 128 below, where a
  // half-empty 256-row tail tile would waste more than the bigger tile saves.
  return (E > 0 && max_rows / E >= 384) ? 256 : 128;
}

// Workspace: the persistent GEMMs' flag words, their fp32 partial slots (two
// per block), then the fused up+down launch's words.
static int64_t fused_words_offset(int G) { return kSkFlagBytes + 2 * static_cast<int64_t>(G) * kSkSlotBytes; }

extern "C" int64_t ffmoe_gemm_workspace_bytes(void) {
  const int G = sk_blocks();
  return G > 0 ? fused_words_offset(G) + kFusedBytes : -1;
}

extern "C" int ffmoe_gemm_check(void* sk_workspace, void* stream) {
  if (sk_workspace == nullptr) return clear_error();
  const int G = sk_blocks();
  if (G <= 0) return set_error("ffmoe_gemm_check: cannot query the CU count");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int err = 0;
  const char* base = static_cast<const char*>(sk_workspace);
  if (hipMemcpyAsync(&err, base + 2 * static_cast<int64_t>(G) * 4, sizeof(int), hipMemcpyDeviceToHost, st) !=
          hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return set_error("ffmoe_gemm_check: cannot read the workspace's error word");
  if (err == 0) return clear_error();
  // every block of the failed launch has finished (the stream is idle), so
  // clearing the flag words here cannot race a late publication
  if (hipMemsetAsync(sk_workspace, 0, kSkFlagBytes, st) != hipSuccess ||
      hipMemsetAsync(static_cast<char*>(sk_workspace) + fused_words_offset(G), 0, kFusedBytes, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return set_error("ffmoe_gemm_check: cannot clear the workspace");
  return set_error(
      "ffmoe_gemm_check: a stream-K partner wait timed out in an earlier grouped GEMM on this workspace; "
      "that GEMM's output is wrong (the workspace has been cleared)");
}

extern "C" int ffmoe_set_lds_transpose(int enable) {
  const int prev = g_use_tr;
  g_use_tr = enable ? 1 : 0;
  return prev;
}

extern "C" int ffmoe_gemm_up_glu_shared(const void* x_sorted, const void* w_up, const int32_t* offsets,
                                        const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                                        int D, int H, int activation, void* up_out, void* act_out,
                                        const ffmoe_dense_group* shared, void* sk_workspace, void* stream) {
  if (check_rows("ffmoe_gemm_up_glu", E, max_rows, D, H, tile_rows)) return 1;
  if (activation < 0 || activation > FFMOE_ACT_GEGLU_ERF) return set_error("ffmoe_gemm_up_glu: unknown activation");
  constexpr int BN = 256;
  GemmArgs a = rows_args(offsets, tile_offsets, E, max_rows, tile_rows, (H + BN / 2 - 1) / (BN / 2));
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
  if (apply_shared(a, shared, tile_rows, "ffmoe_gemm_up_glu")) return 1;
  // 256 x 256 tiles, K = D: stream-K only for long K (its cut-tile partials
  // cost more than the whole-tile tail round at D = 1024, measured)
  return launch_rows<BN, true, EPI_GLU_FWD>(a, tile_rows, sk_workspace, kSkMinK,
                                            static_cast<hipStream_t>(stream), "gemm_up_glu");
}

extern "C" int ffmoe_gemm_up_glu(const void* x_sorted, const void* w_up, const int32_t* offsets,
                                 const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                                 int D, int H, int activation, void* up_out, void* act_out,
                                 void* sk_workspace, void* stream) {
  return ffmoe_gemm_up_glu_shared(x_sorted, w_up, offsets, tile_offsets, tile_rows, E, max_rows, D, H,
                                  activation, up_out, act_out, nullptr, sk_workspace, stream);
}

extern "C" int ffmoe_gemm_down_shared(const void* act, const void* w_down, const int32_t* offsets,
                                      const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                                      int H, int D, void* down_out, const ffmoe_dense_group* shared,
                                      void* sk_workspace, void* stream) {
  if (check_rows("ffmoe_gemm_down", E, max_rows, D, H, tile_rows)) return 1;
  constexpr int BN = 128;  // 256 x 128 tiles: a three-stage LDS ring fits
  GemmArgs a = rows_args(offsets, tile_offsets, E, max_rows, tile_rows, (D + BN - 1) / BN);
  a.A = static_cast<const bf16_t*>(act);
  a.B = static_cast<const bf16_t*>(w_down);
  a.C = static_cast<bf16_t*>(down_out);
  a.lda = H;
  a.ldb = H;
  a.ldc = D;
  a.b_stride = static_cast<int64_t>(D) * H;
  a.N = D;
  a.K = H;
  if (apply_shared(a, shared, tile_rows, "ffmoe_gemm_down")) return 1;
  return launch_rows<BN, true, EPI_STORE>(a, tile_rows, sk_workspace, 0, static_cast<hipStream_t>(stream),
                                          "gemm_down");
}

extern "C" int ffmoe_gemm_down(const void* act, const void* w_down, const int32_t* offsets,
                               const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                               int H, int D, void* down_out, void* sk_workspace, void* stream) {
  return ffmoe_gemm_down_shared(act, w_down, offsets, tile_offsets, tile_rows, E, max_rows, H, D, down_out,
                                nullptr, sk_workspace, stream);
}

// The up GEMM + GLU and the down GEMM in one persistent launch where that
// schedule applies (256-row tiles, K of both a multiple of 64, the up GEMM's
// K below the stream-K threshold, a workspace), else the two launches.
extern "C" int ffmoe_gemm_up_down_shared(const void* x_sorted, const void* w_up, const void* w_down,
                                         const int32_t* offsets, const int32_t* tile_offsets, int tile_rows,
                                         int E, int64_t max_rows, int D, int H, int activation, void* up_out,
                                         void* act_out, void* down_out, const ffmoe_dense_group* shared_up,
                                         const ffmoe_dense_group* shared_down, void* sk_workspace,
                                         void* stream) {
  if (check_rows("ffmoe_gemm_up_down", E, max_rows, D, H, tile_rows)) return 1;
  if (activation < 0 || activation > FFMOE_ACT_GEGLU_ERF) return set_error("ffmoe_gemm_up_down: unknown activation");
  const bool su = shared_up != nullptr && shared_up->rows > 0, sd = shared_down != nullptr && shared_down->rows > 0;
  if (su != sd || (su && (shared_up->rows != shared_down->rows || shared_down->a != shared_up->c)))
    return set_error("ffmoe_gemm_up_down: the dense group's down GEMM must read its up GEMM's activation rows");
  const int G = sk_blocks() / 8 * 8;
  const int64_t row_tiles = (max_rows + tile_rows - 1) / tile_rows + E + (su ? (shared_up->rows + tile_rows - 1) / tile_rows : 0);
  const bool fused = sk_workspace != nullptr && g_use_tr && tile_rows == 256 && D % DL_BK == 0 && H % DL_BK == 0 &&
                     D < kSkMinK && G >= 8 && row_tiles <= kFusedWords - kFusedRow0;
  if (!fused) {
    if (ffmoe_gemm_up_glu_shared(x_sorted, w_up, offsets, tile_offsets, tile_rows, E, max_rows, D, H, activation,
                                 up_out, act_out, shared_up, sk_workspace, stream))
      return 1;
    return ffmoe_gemm_down_shared(act_out, w_down, offsets, tile_offsets, tile_rows, E, max_rows, H, D, down_out,
                                  shared_down, sk_workspace, stream);
  }
  constexpr int BNU = 256, BND = 128;
  GemmArgs u = rows_args(offsets, tile_offsets, E, max_rows, tile_rows, (H + BNU / 2 - 1) / (BNU / 2));
  u.A = static_cast<const bf16_t*>(x_sorted);
  u.B = static_cast<const bf16_t*>(w_up);
  u.C = static_cast<bf16_t*>(act_out);
  u.C2 = static_cast<bf16_t*>(up_out);
  u.lda = D;
  u.ldb = D;
  u.ldc = H;
  u.b_stride = static_cast<int64_t>(2) * H * D;
  u.N = H;
  u.K = D;
  u.H = H;
  u.act = activation;
  if (apply_shared(u, shared_up, tile_rows, "ffmoe_gemm_up_down")) return 1;
  GemmArgs d = rows_args(offsets, tile_offsets, E, max_rows, tile_rows, (D + BND - 1) / BND);
  d.A = static_cast<const bf16_t*>(act_out);
  d.B = static_cast<const bf16_t*>(w_down);
  d.C = static_cast<bf16_t*>(down_out);
  d.lda = H;
  d.ldb = H;
  d.ldc = D;
  d.b_stride = static_cast<int64_t>(D) * H;
  d.N = D;
  d.K = H;
  if (apply_shared(d, shared_down, tile_rows, "ffmoe_gemm_up_down")) return 1;
  u.flags = static_cast<int*>(sk_workspace);
  u.err_idx = 2 * sk_blocks();
  u.fused = reinterpret_cast<int*>(static_cast<char*>(sk_workspace) + fused_words_offset(sk_blocks()));
  hipLaunchKernelGGL(gemm_updown_kernel<256>, dim3(G), dim3(kThreads), 0, static_cast<hipStream_t>(stream), u, d);
  if (check_launch("gemm_up_down")) return 1;
  return clear_error();
}

extern "C" int ffmoe_gemm_dgrad_glu_shared(const void* wgo, const void* w_down, const void* up,
                                           const int32_t* offsets, const int32_t* tile_offsets,
                                           int tile_rows, int E, int64_t max_rows, int D, int H,
                                           int activation, void* gup_out, const ffmoe_dense_group* shared,
                                           void* sk_workspace, void* stream) {
  if (check_rows("ffmoe_gemm_dgrad_glu", E, max_rows, D, H, tile_rows)) return 1;
  if (activation < 0 || activation > FFMOE_ACT_GEGLU_ERF) return set_error("ffmoe_gemm_dgrad_glu: unknown activation");
  // 256-row tiles: 256 x 128 tiles, a three-stage LDS ring and eight waves,
  // so one wave of a SIMD runs MFMAs while the other waits on loads (C2:
  // 120 -> 117.5 us against 256 x 64 tiles two blocks per CU; C4: 0.956 ->
  // 0.923 ms against four waves); 128-row tiles: the 128 x 128 launches
  const bool eight = tile_rows == 256 && g_use_tr && D % DL_BK == 0;
  constexpr int BN = 128;
  GemmArgs a = rows_args(offsets, tile_offsets, E, max_rows, tile_rows, (H + BN - 1) / BN);
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
  if (shared != nullptr && shared->rows > 0 && shared->up == nullptr)
    return set_error("ffmoe_gemm_dgrad_glu: the dense extra group needs its pre-activation");
  if (apply_shared(a, shared, tile_rows, "ffmoe_gemm_dgrad_glu")) return 1;
  if (eight) {
    if (a.total_tiles <= 0) return clear_error();
    // the last G/32 tiles of each XCD's run in row halves (C2: 126.4 ->
    // 119.8 us; 4 a run: 122.9, 16: 119.8)
    const int hx = sk_blocks() / 32 > 1 ? sk_blocks() / 32 : 1;
    const int64_t grid = ((a.total_tiles + 7) / 8 + hx) * 8;
    if (grid > 0x7fffffff) return set_error("ffmoe_gemm_dgrad_glu: problem too large");
    hipLaunchKernelGGL((gemm_dl8h_kernel<256, BN, true, false, EPI_GLU_BWD>), dim3(static_cast<unsigned>(grid)),
                       dim3(512), 0, static_cast<hipStream_t>(stream), a, hx);
    if (check_launch("gemm_dgrad_glu")) return 1;
    return clear_error();
  }
  return launch_rows<128, false, EPI_GLU_BWD>(a, tile_rows, sk_workspace, 0, static_cast<hipStream_t>(stream),
                                              "gemm_dgrad_glu");
}

extern "C" int ffmoe_gemm_dgrad_glu(const void* wgo, const void* w_down, const void* up,
                                    const int32_t* offsets, const int32_t* tile_offsets,
                                    int tile_rows, int E, int64_t max_rows, int D, int H,
                                    int activation, void* gup_out, void* sk_workspace, void* stream) {
  return ffmoe_gemm_dgrad_glu_shared(wgo, w_down, up, offsets, tile_offsets, tile_rows, E, max_rows, D, H,
                                     activation, gup_out, nullptr, sk_workspace, stream);
}

// dgrad arguments: ghb [rows, D] = gup [rows, 2H] · w_up[e] [2H, D], 256-column tiles.
static int dgrad_args(GemmArgs& a, const void* gup, const void* w_up, const int32_t* offsets,
                      const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows, int H, int D,
                      void* ghb_out, const ffmoe_dense_group* shared) {
  if (check_rows("ffmoe_gemm_dgrad", E, max_rows, D, H, tile_rows)) return 1;
  constexpr int BN = 256;
  a = rows_args(offsets, tile_offsets, E, max_rows, tile_rows, (D + BN - 1) / BN);
  a.A = static_cast<const bf16_t*>(gup);
  a.B = static_cast<const bf16_t*>(w_up);
  a.C = static_cast<bf16_t*>(ghb_out);
  a.lda = 2 * static_cast<int64_t>(H);
  a.ldb = D;
  a.ldc = D;
  a.b_stride = static_cast<int64_t>(2) * H * D;
  a.N = D;
  a.K = 2 * H;
  return apply_shared(a, shared, tile_rows, "ffmoe_gemm_dgrad");
}

extern "C" int ffmoe_gemm_dgrad_shared(const void* gup, const void* w_up, const int32_t* offsets,
                                       const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                                       int H, int D, void* ghb_out, const ffmoe_dense_group* shared,
                                       void* sk_workspace, void* stream) {
  GemmArgs a;
  if (dgrad_args(a, gup, w_up, offsets, tile_offsets, tile_rows, E, max_rows, H, D, ghb_out, shared)) return 1;
  // 256 x 256 tiles (two stages) under the stream-K schedule
  return launch_rows<256, false, EPI_STORE>(a, tile_rows, sk_workspace, 0, static_cast<hipStream_t>(stream),
                                            "gemm_dgrad");
}

extern "C" int ffmoe_gemm_dgrad(const void* gup, const void* w_up, const int32_t* offsets,
                                const int32_t* tile_offsets, int tile_rows, int E, int64_t max_rows,
                                int H, int D, void* ghb_out, void* sk_workspace, void* stream) {
  return ffmoe_gemm_dgrad_shared(gup, w_up, offsets, tile_offsets, tile_rows, E, max_rows, H, D, ghb_out,
                                 nullptr, sk_workspace, stream);
}

// Dense GEMM launch: tiles of BM x BN, the K split S chosen so the grid
// covers the CUs about once (at most 8 splits, at least 2 K steps each).
template <int BM, int BN, bool A_KC, bool B_KC, int MODE>
static int launch_dense(GemmArgs a, void* ws, int64_t ws_bytes, int split, hipStream_t st, const char* name) {
  a.E = 1;
  a.b_stride = 0;
  a.c_stride = 0;
  a.m_tiles = static_cast<int>((a.M + BM - 1) / BM);
  a.n_tiles = (a.N + BN - 1) / BN;
  a.total_tiles = static_cast<int64_t>(a.m_tiles) * a.n_tiles;
  if (a.total_tiles <= 0 || a.K <= 0) return set_error(std::string(name) + ": empty problem");
  if (!g_use_tr || (MODE == 0 && a.K % DL_BK != 0))
    return set_error(std::string(name) + ": K must be a multiple of 64");
  const int S = split;
  a.split_rows = a.M;
  if (S > 1) {
    const int64_t need = static_cast<int64_t>(S) * a.M * a.N * 4;
    if (ws == nullptr || ws_bytes < need) return set_error(std::string(name) + ": workspace too small");
    a.part = static_cast<float*>(ws);
  }
  const int64_t grid = a.total_tiles * S;
  if (grid > 0x7fffffff) return set_error(std::string(name) + ": problem too large");
  hipLaunchKernelGGL((gemm_dense_kernel<BM, BN, A_KC, B_KC, MODE>), dim3(static_cast<unsigned>(grid)),
                     dim3(kThreads), 0, st, a, S);
  if (check_launch(name)) return 1;
  if (S > 1) {
    bf16_t* out = a.C;
    const int64_t n = static_cast<int64_t>(a.M) * a.N;
    int64_t blocks = (n / 4 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(split_reduce_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, a.part, S,
                       n, out);
    if (check_launch(name)) return 1;
  }
  return clear_error();
}

// K split for a dense GEMM of `tiles` output tiles and `nk` 64-deep K steps.
static int dense_split(int64_t tiles, int64_t nk) {
  const int G = sk_blocks() > 0 ? sk_blocks() : 256;
  int64_t S = (G + tiles - 1) / tiles;
  if (S > 8) S = 8;
  if (S > nk / 2) S = nk / 2;
  return S < 1 ? 1 : static_cast<int>(S);
}

static int gate_logits_split(int64_t N, int D, int E) {
  return dense_split(((N + 255) / 256) * ((E + 127) / 128), D / DL_BK);
}

namespace ffmoe {
int gate_grad_mfma_split(int64_t N, int D, int E) {
  return dense_split(((E + 255) / 256) * static_cast<int64_t>((D + 255) / 256), (N + DL_BK - 1) / DL_BK);
}
}  // namespace ffmoe

extern "C" int64_t ffmoe_gate_logits_workspace_bytes(int64_t N, int D, int E) {
  if (N <= 0 || D <= 0 || E <= 0) return 0;
  const int S = gate_logits_split(N, D, E);
  return S > 1 ? static_cast<int64_t>(S) * N * E * 4 : 0;
}

extern "C" int ffmoe_gate_logits(const void* x, const void* gate, int64_t N, int D, int E, void* logits,
                                 void* workspace, void* stream) {
  if (N <= 0 || N > 0x7fffffff || D <= 0 || D % DL_BK != 0 || E < 1 || E > FFMOE_MAX_EXPERTS || E % 8 != 0)
    return set_error("ffmoe_gate_logits: needs D a multiple of 64 and E a multiple of 8 (at most 256)");
  GemmArgs a{};
  a.A = static_cast<const bf16_t*>(x);
  a.B = static_cast<const bf16_t*>(gate);
  a.C = static_cast<bf16_t*>(logits);
  a.lda = D;
  a.ldb = D;
  a.ldc = E;
  a.M = static_cast<int>(N);
  a.N = E;
  a.K = D;
  const int S = gate_logits_split(N, D, E);
  return launch_dense<256, 128, true, true, 0>(a, workspace, ffmoe_gate_logits_workspace_bytes(N, D, E), S,
                                               static_cast<hipStream_t>(stream), "ffmoe_gate_logits");
}

extern "C" int ffmoe_gate_dx(const void* gl, const void* gate, int64_t N, int D, int E, void* out,
                             void* stream) {
  if (N <= 0 || N > 0x7fffffff || D <= 0 || D % 8 != 0 || E < 1 || E > FFMOE_MAX_EXPERTS || E % DL_BK != 0)
    return set_error("ffmoe_gate_dx: needs D a multiple of 8 and E a multiple of 64 (at most 256)");
  GemmArgs a{};
  a.A = static_cast<const bf16_t*>(gl);
  a.B = static_cast<const bf16_t*>(gate);
  a.C = static_cast<bf16_t*>(out);
  a.lda = E;
  a.ldb = D;
  a.ldc = D;
  a.M = static_cast<int>(N);
  a.N = D;
  a.K = E;
  return launch_dense<256, 256, true, false, 0>(a, nullptr, 0, 1, static_cast<hipStream_t>(stream),
                                                "ffmoe_gate_dx");
}

// dgate [E, D] = gl^T x over all N token rows (the gate-gradient product
// for expert counts beyond the fused kernel's), split along the tokens.
int ffmoe::gate_grad_mfma(const void* gl, const void* x, int64_t N, int D, int E, void* workspace,
                          int64_t ws_bytes, void* dgate, void* stream) {
  GemmArgs a{};
  a.A = static_cast<const bf16_t*>(gl);
  a.B = static_cast<const bf16_t*>(x);
  a.C = static_cast<bf16_t*>(dgate);
  a.lda = E;
  a.ldb = D;
  a.ldc = D;
  a.M = E;
  a.N = D;
  a.K = static_cast<int>(N);
  return launch_dense<256, 256, false, false, 1>(a, workspace, ws_bytes, gate_grad_mfma_split(N, D, E),
                                                 static_cast<hipStream_t>(stream), "ffmoe_gate_grad");
}

#ifndef FFMOE_WGRAD_LPT_MIN_E
#define FFMOE_WGRAD_LPT_MIN_E 2
#endif
static int wgrad_lpt(int E) { return E >= FFMOE_WGRAD_LPT_MIN_E && E <= kLptMaxE; }

// wgrad arguments: c[e] [M, Nc] = a[rows of e, M]^T · b[rows of e, Nc], 256 x 256 tiles.
static int wgrad_args(GemmArgs& a, const void* a_, const void* b_, const int32_t* offsets, int E, int M, int Nc,
                      void* c_out, const ffmoe_dense_group* shared, void* sk_workspace) {
  if (E < 1 || M <= 0 || M % 8 != 0 || Nc <= 0 || Nc % 8 != 0)
    return set_error("ffmoe_gemm_wgrad: M and Nc must be positive multiples of 8");
  constexpr int BM = 256, BN = 256;
  a = GemmArgs{};
  a.offsets = offsets;
  a.E = E;
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
  a.lpt = wgrad_lpt(E);
  if (shared != nullptr && shared->rows > 0) {
    // the dense group is group E: K = its rows of a and b, output c [M, Nc]
    if (shared->a == nullptr || shared->b == nullptr || shared->c == nullptr || shared->rows > 0x7fffffff)
      return set_error("ffmoe_gemm_wgrad: bad dense extra group");
    a.xA = static_cast<const bf16_t*>(shared->a);
    a.xB = static_cast<const bf16_t*>(shared->b);
    a.xC = static_cast<bf16_t*>(shared->c);
    a.x_rows = static_cast<int>(shared->rows);
    // A dense group's tiles take K = all of its rows, where a routed
    // expert's take K = its share; from kPairMinRows rows on its K is cut in
    // two halves (two groups, each tile finished by whichever half arrives
    // second, through the persistent GEMMs' workspace), so its tiles are no
    // longer the launch's long pole.  Each cut tile moves a 256 KiB fp32
    // partial, small against the >= 2 MiB of operands a half reads.
    constexpr int kPairMinRows = 4096;
    const int P = a.m_tiles * a.n_tiles;
    const int G = sk_blocks();
    int groups = 1;
    if (sk_workspace != nullptr && a.x_rows >= kPairMinRows && G > 0 && 2 * G < kPairKey && P <= kPairMax &&
        P <= 2 * G) {
      groups = 2;
      a.x_split = 2;
      a.x_chunk = ((a.x_rows + 1) / 2 + 63) / 64 * 64;
      a.flags = static_cast<int*>(sk_workspace);
      a.part = reinterpret_cast<float*>(static_cast<char*>(sk_workspace) + kSkFlagBytes);
      a.pub_off = kPairPubOff;
      a.err_idx = 2 * G;
    }
    a.total_tiles += static_cast<int64_t>(groups) * P;
    a.lpt = E + groups <= kLptMaxE;
  }
  return 0;
}

extern "C" int ffmoe_gemm_wgrad_shared(const void* a_, const void* b_, const int32_t* offsets, int E, int M,
                                       int Nc, void* c_out, const ffmoe_dense_group* shared, void* sk_workspace,
                                       void* stream) {
  GemmArgs a;
  if (wgrad_args(a, a_, b_, offsets, E, M, Nc, c_out, shared, sk_workspace)) return 1;
  return launch<256, 256, false, false, 1, EPI_STORE>(a, static_cast<hipStream_t>(stream), "gemm_wgrad");
}

constexpr int kDwEightMaxRows = 512;  // mean rows per expert up to which the fused launch runs eight waves

// The up-side weight gradient and dgrad in one persistent launch where that
// schedule applies (a workspace, the transpose-read path, 2H a multiple of
// 64, 128- or 256-row tiles), else the two launches, wgrad first.
extern "C" int ffmoe_gemm_dgrad_wgrad_shared(const void* gup, const void* w_up, const void* x_sorted,
                                             const int32_t* offsets, const int32_t* tile_offsets, int tile_rows,
                                             int E, int64_t max_rows, int H, int D, void* ghb_out, void* dwu_out,
                                             const ffmoe_dense_group* shared_dgrad,
                                             const ffmoe_dense_group* shared_wgrad, void* sk_workspace,
                                             void* stream) {
  GemmArgs d, w;
  if (dgrad_args(d, gup, w_up, offsets, tile_offsets, tile_rows, E, max_rows, H, D, ghb_out, shared_dgrad))
    return 1;
  if (wgrad_args(w, gup, x_sorted, offsets, E, 2 * H, D, dwu_out, shared_wgrad, sk_workspace)) return 1;
  const int G = sk_blocks() / 8 * 8;
  const int NG = E + extra_groups(w);
  const bool fused = sk_workspace != nullptr && g_use_tr && (2 * H) % DL_BK == 0 && G >= 8 &&
                     NG <= kLptMaxE + 2 && (tile_rows == 256 || tile_rows == 128);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!fused) {
    if (launch<256, 256, false, false, 1, EPI_STORE>(w, st, "gemm_wgrad")) return 1;
    return launch_rows<256, false, EPI_STORE>(d, tile_rows, sk_workspace, 0, st, "gemm_dgrad");
  }
  d.fused = reinterpret_cast<int*>(static_cast<char*>(sk_workspace) + fused_words_offset(sk_blocks()));
  // few rows per expert (short wgrad tiles: K steps of at most 8 on
  // average): eight waves, which keep more operand loads in flight (C5);
  // else four (at C2, 2048 rows per expert, eight were slower: 274 -> 281 us)
  const bool eight = max_rows <= static_cast<int64_t>(kDwEightMaxRows) * E;
  if (tile_rows == 256) {
    if (eight)
      hipLaunchKernelGGL((gemm_dw_kernel<256, 512>), dim3(G), dim3(512), 0, st, d, w);
    else
      hipLaunchKernelGGL(gemm_dw_kernel<256>, dim3(G), dim3(kThreads), 0, st, d, w);
  } else {
    if (eight)
      hipLaunchKernelGGL((gemm_dw_kernel<128, 512>), dim3(G), dim3(512), 0, st, d, w);
    else
      hipLaunchKernelGGL(gemm_dw_kernel<128>, dim3(G), dim3(kThreads), 0, st, d, w);
  }
  if (check_launch("gemm_dgrad_wgrad")) return 1;
  return clear_error();
}

extern "C" int ffmoe_gemm_wgrad(const void* a_, const void* b_, const int32_t* offsets, int E, int M,
                                int Nc, void* c_out, void* stream) {
  return ffmoe_gemm_wgrad_shared(a_, b_, offsets, E, M, Nc, c_out, nullptr, nullptr, stream);
}
