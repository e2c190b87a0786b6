// Routing forward: gate GEMM (MFMA) + scoring + top-k + per-block statistics,
// the global prefix scan, and the stable permutation into expert-sorted rows.
//
// Determinism: every count and rank comes from ordered scans (no atomics), so
// the permutation equals the reference's stable argsort (fused_moe.py:345)
// bit for bit, and every fp32 reduction has a fixed order.
#include <algorithm>
#include <string>
#include <type_traits>

#include "common.h"

#ifndef FFMOE_ROUTE_PART
#define FFMOE_ROUTE_PART 0
#endif

namespace ffmoe {

// Tokens per route block: one wave of 16 (one MFMA row tile).  Small blocks
// spread the latency-bound gate GEMM and top-k over every CU (measured at
// C2: 13 us with 16-token blocks, 15 us with 32, 23 us with 64).
constexpr int kRouteTokens = 16;
constexpr int kRouteThreads = 64;

struct RouteWs {
  int32_t* hist;    // [nblk][E] per-block counts, replaced by block bases
  float* psum;      // [nblk][E] sum of routing weights per expert
  float* ssum;      // [nblk][E] sum of sigmoid(logit) per expert
  float* zpart;     // [nblk] sum of lse^2
};

static inline int64_t route_blocks(int64_t N) { return (N + kRouteTokens - 1) / kRouteTokens; }

static inline RouteWs route_ws(void* ws, int64_t N, int E) {
  const int64_t nb = route_blocks(N);
  char* p = static_cast<char*>(ws);
  RouteWs w;
  w.hist = reinterpret_cast<int32_t*>(p);
  p += nb * E * 4;
  w.psum = reinterpret_cast<float*>(p);
  p += nb * E * 4;
  w.ssum = reinterpret_cast<float*>(p);
  p += nb * E * 4;
  w.zpart = reinterpret_cast<float*>(p);
  return w;
}

// Routing options beyond the fast path (fused_moe.py:116-251).
struct RouteOpts {
  const float* bias;      // expert_bias [E] (selection only), or null
  int bias_round;         // 1: logits + bias rounded to bf16 (a bf16 bias on bf16 logits)
  int pre_softmax;        // softmax over all experts before selection
  float scoring;          // > 0: weights scaled by scoring / top_k
  int n_group;            // > 0: group-limited selection over n_group groups
  int topk_group;         //   keeping the best topk_group groups
  const bf16_t* noise;    // input jitter: logits from bf16(x * noise), or null
};

// Top-k insertion: keeps the KMAX best in (value desc, index asc) order, which
// is the reference's k-round argmax with tie_break_left=True
// (fused_topk.py:63-70).  An element displaced from slot s still precedes an
// equal-valued element in slot s+1 (its index is lower), so the comparison
// is the full lexicographic one, not value alone.
template <int KMAX>
struct TopK {
  float v[KMAX];
  int i[KMAX];
  __device__ void init() {
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
      v[s] = 0.0f;
      i[s] = -1;
    }
  }
  __device__ void push(float val, int idx, int k) {
#pragma unroll
    for (int s = 0; s < KMAX; ++s) {
      if (s < k) {
        const bool take = (i[s] < 0) || (val > v[s]) || (val == v[s] && idx < i[s]);
        if (take) {
          const float tv = v[s];
          const int ti = i[s];
          v[s] = val;
          i[s] = idx;
          val = tv;
          idx = ti;
          if (idx < 0) break;
        }
      }
    }
  }
};

// Logits source of the route kernel: the fused MFMA gate GEMM (bf16), bf16
// logits from memory, or fp32 logits from memory (the fp32 / fp64 compute
// path: the reference's top-k and losses read logits.float(),
// fused_topk.py:52, fused_moe.py:1191).
enum LogitSrc { kGateGemm = 0, kLogitsBf16 = 1, kLogitsF32 = 2 };
__device__ __forceinline__ float logit_f32(bf16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ float logit_f32(float v) { return v; }

template <int ET, int KMAX, int SRC>
__global__ __launch_bounds__(kRouteThreads) void route_fwd_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ gate,
    const void* __restrict__ logits_in_v, RouteOpts o, int64_t N, int D,
    int E, int k, int gating, int need_ssum, bf16_t* __restrict__ logits_out,
    int64_t* __restrict__ topk_idx, float* __restrict__ topk_w, float* __restrict__ lse_out,
    int32_t* __restrict__ rank_local, RouteWs ws) {
  constexpr bool FROM_LOGITS = SRC != kGateGemm;
  using LT = typename std::conditional<SRC == kLogitsF32, float, bf16_t>::type;
  constexpr int LV = 16 / sizeof(LT);  // logits per 16-byte load
  const LT* __restrict__ logits_in = static_cast<const LT*>(logits_in_v);
  constexpr int EP = ET * 16;        // padded expert count
  constexpr int LS = EP + 4 / sizeof(LT);  // LDS row stride (elements): rows 4 bytes apart from 16-byte alignment
  extern __shared__ float smem[];
  LT* L = reinterpret_cast<LT*>(smem);       // [64][LS] logits
  int* sel_i = reinterpret_cast<int*>(smem + kRouteTokens * LS * sizeof(LT) / 4);  // [64*k]
  float* sel_w = reinterpret_cast<float*>(sel_i + kRouteTokens * k);  // [64*k]
  float* zl = sel_w + kRouteTokens * k;              // [64]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t blk = blockIdx.x;
  const int64_t tok_base = blk * kRouteTokens;
  const int ntok = static_cast<int>(min<int64_t>(kRouteTokens, N - tok_base));

  if constexpr (FROM_LOGITS) {
    if (E % LV == 0) {
      // 16-byte loads, all of a thread's in flight before the first LDS
      // write (logits rows are 16-byte aligned when E % LV == 0; the LDS
      // rows, padded by 4 bytes, take them as four 4-byte writes)
      constexpr int NV = kRouteTokens * EP / LV;
      constexpr int PER = (NV + kRouteThreads - 1) / kRouteThreads;
      uint4 v[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int p = i * kRouteThreads + tid;
        const int t = p / (EP / LV), e = (p % (EP / LV)) * LV;
        v[i] = make_uint4(0, 0, 0, 0);
        if (p < NV && t < ntok && e < E)
          v[i] = *reinterpret_cast<const uint4*>(logits_in + (tok_base + t) * E + e);
      }
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int p = i * kRouteThreads + tid;
        const int t = p / (EP / LV), e = (p % (EP / LV)) * LV;
        if (p < NV) {
          uint32_t* d = reinterpret_cast<uint32_t*>(L + t * LS + e);
          d[0] = v[i].x;
          d[1] = v[i].y;
          d[2] = v[i].z;
          d[3] = v[i].w;
        }
      }
    } else {
      for (int p = tid; p < kRouteTokens * EP; p += kRouteThreads) {
        const int t = p / EP, e = p % EP;
        LT v = 0;
        if (t < ntok && e < E) v = logits_in[(tok_base + t) * E + e];
        L[t * LS + e] = v;
      }
    }
  } else if constexpr (SRC == kGateGemm) {
    // Wave `wave` computes logits of tokens [16*wave, 16*wave+16) against all
    // experts with v_mfma_f32_16x16x32_bf16: A = x rows (K-contiguous),
    // B = gate rows (K-contiguous).  Lane l holds row l%16, k-block l/16.
    f32x4_t acc[ET];
#pragma unroll
    for (int t = 0; t < ET; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int row = 16 * wave + (lane & 15);
    const bool row_ok = row < ntok;
    const bf16_t* xr = x + (tok_base + (row_ok ? row : 0)) * static_cast<int64_t>(D);
    const int kq = (lane >> 4) * 8;
    // batches of U k-steps: all of a batch's x loads (and, for few experts,
    // gate loads) are in flight together instead of one latency per k-step
    constexpr int U = 8;
    for (int k0 = 0; k0 < D; k0 += 32 * U) {
      uint4 av[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kk = k0 + 32 * u + kq;
        av[u] = make_uint4(0, 0, 0, 0);
        if (row_ok && kk < D) av[u] = *reinterpret_cast<const uint4*>(xr + kk);
      }
      if (o.noise != nullptr) {  // input jitter: bf16(x * noise), as the reference's bf16 product
        const bf16_t* nr = o.noise + (tok_base + (row_ok ? row : 0)) * static_cast<int64_t>(D);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int kk = k0 + 32 * u + kq;
          if (row_ok && kk < D) {
            float a[8], b[8];
            unpack8(av[u], a);
            unpack8(*reinterpret_cast<const uint4*>(nr + kk), b);
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] *= b[i];
            av[u] = pack8(a);
          }
        }
      }
      if constexpr (ET <= 2) {
        uint4 bv[U][ET];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int t = 0; t < ET; ++t) {
            const int e = 16 * t + (lane & 15);
            const int kk = k0 + 32 * u + kq;
            bv[u][t] = make_uint4(0, 0, 0, 0);
            if (e < E && kk < D) bv[u][t] = *reinterpret_cast<const uint4*>(gate + static_cast<int64_t>(e) * D + kk);
          }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int t = 0; t < ET; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[u]),
                                                            __builtin_bit_cast(bf16x8_t, bv[u][t]),
                                                            acc[t], 0, 0, 0);
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int t = 0; t < ET; ++t) {
            const int e = 16 * t + (lane & 15);
            const int kk = k0 + 32 * u + kq;
            uint4 bv = make_uint4(0, 0, 0, 0);
            if (e < E && kk < D) bv = *reinterpret_cast<const uint4*>(gate + static_cast<int64_t>(e) * D + kk);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[u]),
                                                            __builtin_bit_cast(bf16x8_t, bv), acc[t],
                                                            0, 0, 0);
          }
      }
    }
    // Output layout: lane l holds expert 16t + l%16 for tokens 4*(l/16) + r.
#pragma unroll
    for (int t = 0; t < ET; ++t) {
      const int e = 16 * t + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tl = 16 * wave + 4 * (lane >> 4) + r;
        const bf16_t h = f32_to_bf16(acc[t][r]);
        L[tl * LS + e] = static_cast<LT>(h);
        if (logits_out != nullptr && tl < ntok && e < E)
          logits_out[(tok_base + tl) * E + e] = h;
      }
    }
  }
  __syncthreads();

  // Scores, top-k, weights, logsumexp: four lanes per token (lane 4t + j of
  // token t takes experts j, j + 4, ... in order).  The lanes' partial
  // logsumexps, pre-softmax sums and top-k lists are combined by a butterfly
  // over the four lanes (xor 1, then xor 2): each step adds the same two
  // operands on both partners, so all four lanes end with identical values,
  // and the top-k order (value desc, index asc) is total, so the merged list
  // is the single-pass list.  Lane j == 0 then writes the token's results.
  {
    constexpr int LPT = kRouteThreads / kRouteTokens;
    static_assert(LPT == 4, "four lanes per token");
    const int t = tid / LPT, jl = tid % LPT;
    const bool tok_ok = t < ntok;
    const LT* lr = L + t * LS;
    float lse = 0.0f;
    // logsumexp of the logits (z-loss and the pre-softmax probabilities)
    float m = -INFINITY, s = 0.0f;
    if (tok_ok) {
#pragma unroll 8
      for (int e = jl; e < E; e += LPT) {
        const float l = logit_f32(lr[e]);
        if (l > m) {
          s = s * expf(m - l) + 1.0f;
          m = l;
        } else {
          s += expf(l - m);
        }
      }
    }
#pragma unroll
    for (int off = 1; off < LPT; off <<= 1) {
      const float m2 = __shfl_xor(m, off, kWave), s2 = __shfl_xor(s, off, kWave);
      const float mn = fmaxf(m, m2);
      const float a1 = m == -INFINITY ? 0.0f : s * expf(m - mn);
      const float a2 = m2 == -INFINITY ? 0.0f : s2 * expf(m2 - mn);
      s = a1 + a2;
      m = mn;
    }
    if (tok_ok) lse = m + logf(s);
    float psum = 0.0f;  // pre-softmax: sum of exp(l - max)
    if (o.pre_softmax) {
      if (tok_ok)
        for (int e = jl; e < E; e += LPT) psum += expf(logit_f32(lr[e]) - m);
#pragma unroll
      for (int off = 1; off < LPT; off <<= 1) psum += __shfl_xor(psum, off, kWave);
    }
    // selection score of expert e (fused_moe.py:144-200)
    auto score = [&](int e) {
      const float l = logit_f32(lr[e]);
      float sc;
      if (gating == FFMOE_GATING_SOFTMAX)
        sc = o.pre_softmax ? expf(l - m) / psum : l;
      else
        sc = 1.0f / (1.0f + expf(-l));
      if (o.bias != nullptr) sc = o.bias_round ? round_bf16(sc + o.bias[e]) : sc + o.bias[e];
      return sc;
    };
    TopK<KMAX> tk;
    tk.init();
    if (o.n_group > 0) {
      if (tok_ok && jl == 0) {
        // group-limited top-k (fused_moe.py:203-251): groups ranked by the sum
        // of their best top_k/topk_group scores (or their best score), the
        // best topk_group groups kept, top_k taken among their experts
        const int epg = E / o.n_group;
        const int per = k / o.topk_group;
        // bf16 selection scores (softmax logits, unbiased or with a bf16 bias)
        // are summed in fp32 and rounded to bf16, as torch sums a bf16 tensor
        const bool bf16_scores = SRC != kLogitsF32 && gating == FFMOE_GATING_SOFTMAX && !o.pre_softmax &&
                                 (o.bias == nullptr || o.bias_round);
        TopK<FFMOE_MAX_TOPK> tg;
        tg.init();
        for (int g = 0; g < o.n_group; ++g) {
          float gs;
          if (per > 1 && per <= epg) {
            TopK<FFMOE_MAX_TOPK> tm;
            tm.init();
            for (int j = 0; j < epg; ++j) tm.push(score(g * epg + j), j, per);
            gs = 0.0f;
#pragma unroll
            for (int q = 0; q < FFMOE_MAX_TOPK; ++q)
              if (q < per) gs += tm.v[q];
            if (bf16_scores) gs = round_bf16(gs);
          } else {
            gs = -INFINITY;
            for (int j = 0; j < epg; ++j) gs = fmaxf(gs, score(g * epg + j));
          }
          tg.push(gs, g, o.topk_group);
        }
        uint32_t keep[FFMOE_MAX_EXPERTS / 32] = {0};
#pragma unroll
        for (int q = 0; q < FFMOE_MAX_TOPK; ++q)
          if (q < o.topk_group) keep[tg.i[q] >> 5] |= 1u << (tg.i[q] & 31);
        for (int e = 0; e < E; ++e) {
          const int g = e / epg;
          if (keep[g >> 5] >> (g & 31) & 1u) tk.push(score(e), e, k);
        }
      }
    } else {
      if (tok_ok) {
#pragma unroll 4
        for (int e = jl; e < E; e += LPT) tk.push(score(e), e, k);
      }
#pragma unroll
      for (int off = 1; off < LPT; off <<= 1) {
        float pv[KMAX];
        int pi[KMAX];
#pragma unroll
        for (int q = 0; q < KMAX; ++q) {
          pv[q] = __shfl_xor(tk.v[q], off, kWave);
          pi[q] = __shfl_xor(tk.i[q], off, kWave);
        }
#pragma unroll
        for (int q = 0; q < KMAX; ++q)
          if (q < k && pi[q] >= 0) tk.push(pv[q], pi[q], k);
      }
    }
    if (tok_ok && jl == 0) {
      float w[KMAX];
      float wsum = 0.0f;
      if (gating == FFMOE_GATING_SOFTMAX && !o.pre_softmax) {
        float mx = -INFINITY;
#pragma unroll
        for (int q = 0; q < KMAX; ++q)
          if (q < k) mx = fmaxf(mx, logit_f32(lr[tk.i[q]]));
#pragma unroll
        for (int q = 0; q < KMAX; ++q) {
          if (q < k) {
            w[q] = expf(logit_f32(lr[tk.i[q]]) - mx);
            wsum += w[q];
          }
        }
#pragma unroll
        for (int q = 0; q < KMAX; ++q)
          if (q < k) w[q] = w[q] / wsum;
      } else {
        // sigmoid scores, or pre-softmax probabilities, renormalised with +1e-6
#pragma unroll
        for (int q = 0; q < KMAX; ++q) {
          if (q < k) {
            const float l = logit_f32(lr[tk.i[q]]);
            w[q] = (gating == FFMOE_GATING_SOFTMAX) ? expf(l - m) / psum : 1.0f / (1.0f + expf(-l));
            wsum += w[q];
          }
        }
        wsum += 1e-6f;
#pragma unroll
        for (int q = 0; q < KMAX; ++q)
          if (q < k) w[q] = w[q] / wsum;
      }
      if (o.scoring > 0.0f) {
        const float f = o.scoring / static_cast<float>(k);
#pragma unroll
        for (int q = 0; q < KMAX; ++q)
          if (q < k) w[q] = w[q] * f;
      }
      const int64_t n = tok_base + t;
#pragma unroll
      for (int q = 0; q < KMAX; ++q) {
        if (q < k) {
          topk_idx[n * k + q] = tk.i[q];
          topk_w[n * k + q] = w[q];
          sel_i[t * k + q] = tk.i[q];
          sel_w[t * k + q] = w[q];
        }
      }
      if (lse_out != nullptr) lse_out[n] = lse;
    }
    if (jl == 0) zl[t] = tok_ok ? lse * lse : 0.0f;
  }
  __syncthreads();

  // Block-local stable ranks (ascending j), counts, weight sums and sigmoid
  // sums, all in a fixed order.  With at most 16 experts and one entry per
  // lane, one ballot per expert gives every entry its rank (the set lanes
  // below it) and lane e the mask of expert e's entries, whose weights it
  // adds in ascending j.  Otherwise thread q owns experts q, q + 64, ... and
  // makes one pass over the block's entries for all of them.
  const int nent = ntok * k;
  auto block_sums = [&](int e, int cnt, float ps) {
    ws.hist[blk * E + e] = cnt;
    ws.psum[blk * E + e] = ps;
    if (need_ssum) {
      float ss = 0.0f;
      for (int t = 0; t < ntok; ++t) ss += 1.0f / (1.0f + expf(-logit_f32(L[t * LS + e])));
      ws.ssum[blk * E + e] = ss;
    }
  };
  if (ET == 1 && nent <= kRouteThreads) {
    const int j = tid;
    const int ej = j < nent ? sel_i[j] : -1;
    uint64_t mine = 0;
    for (int e = 0; e < E; ++e) {
      const uint64_t m = __ballot(ej == e);
      if (ej == e) rank_local[tok_base * k + j] = __popcll(m & ((1ull << j) - 1));
      if (tid == e) mine = m;
    }
    if (tid < E) {
      float ps = 0.0f;
      for (uint64_t m = mine; m != 0; m &= m - 1) ps += sel_w[__builtin_ctzll(m)];
      block_sums(tid, __popcll(mine), ps);
    }
  } else {
    constexpr int EPT = (ET * 16 + kRouteThreads - 1) / kRouteThreads;
    int cnt[EPT];
    float ps[EPT];
#pragma unroll
    for (int v = 0; v < EPT; ++v) {
      cnt[v] = 0;
      ps[v] = 0.0f;
    }
#pragma unroll 4
    for (int j = 0; j < nent; ++j) {
      const int ej = sel_i[j];
      const float wj = sel_w[j];
#pragma unroll
      for (int v = 0; v < EPT; ++v) {
        if (ej == tid + v * kRouteThreads) {
          rank_local[tok_base * k + j] = cnt[v]++;
          ps[v] += wj;
        }
      }
    }
#pragma unroll
    for (int v = 0; v < EPT; ++v) {
      const int e = tid + v * kRouteThreads;
      if (e < E) block_sums(e, cnt[v], ps[v]);
    }
  }
  if (tid == 0) {
    float z = 0.0f;
    for (int t = 0; t < kRouteTokens; ++t) z += zl[t];
    ws.zpart[blk] = z;
  }
}

// Single block: per-expert prefix over route blocks (block bases replace the
// histogram in place), counts, row offsets, GEMM tile offsets, losses and
// routing metrics.  A thread owns EV adjacent experts (EV = 4 when E % 4 ==
// 0: 16-byte loads) and a contiguous run of route blocks; consecutive
// threads take consecutive expert groups of the same run, so the loads of a
// wave are coalesced.  Each thread keeps kScanBatch loads of each array in
// flight (the histogram comes from other XCDs' writes, so every load is a
// long trip), the chunk sums are scanned across the runs in LDS (log2 G
// steps), then a second pass writes the bases.  Every sum is a fixed tree or
// sequence (deterministic).
#if FFMOE_ROUTE_PART == 0
constexpr int kScanThreads = 1024;
constexpr int kScanBatch = 8;

template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, kWave));
  return v;
}

template <int EV, typename T>
__device__ __forceinline__ void load_ev(const T* p, bool in, T* out) {
  if constexpr (EV == 4) {
    using V = typename std::conditional<std::is_same<T, int>::value, int4, float4>::type;
    const V v = in ? *reinterpret_cast<const V*>(p) : V{0, 0, 0, 0};
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  } else {
    out[0] = in ? *p : T(0);
  }
}

template <int EV, typename T>
__device__ __forceinline__ void store_lds_ev(T* p, const T* v) {
  if constexpr (EV == 4) {
    using V = typename std::conditional<std::is_same<T, int>::value, int4, float4>::type;
    *reinterpret_cast<V*>(p) = V{v[0], v[1], v[2], v[3]};
  } else {
    p[0] = v[0];
  }
}

template <int EV>
__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(
    int64_t N, int64_t nblk, int E, int k, int mt, int bm, float aux_coeff, float z_coeff,
    int gating, RouteWs ws, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ tile_offsets, float* __restrict__ stats, int32_t* __restrict__ istats,
    float* __restrict__ aux_out, float* __restrict__ z_out) {
  constexpr int kWaves = kScanThreads / kWave;
  constexpr int kEW = FFMOE_MAX_EXPERTS / kWave;  // waves that hold one expert per lane
  __shared__ __attribute__((aligned(16))) int s_i[kScanThreads * EV];
  __shared__ __attribute__((aligned(16))) float s_f[kScanThreads * EV];
  __shared__ int s_rw[kEW], s_tw[kEW];
  __shared__ int s_cnt[FFMOE_MAX_EXPERTS];
  __shared__ float s_p[FFMOE_MAX_EXPERTS];
  __shared__ float s_zw[kWaves];
  __shared__ float s_fpw[kEW];
  __shared__ long long s_totw[kEW];
  __shared__ int s_dw[kEW], s_mxw[kEW], s_mnw[kEW];
  const int tid = threadIdx.x;
  const int EQ = E / EV;  // expert groups
  // runs of route blocks per group (threads per group): at least a batch of
  // blocks per run, so the LDS scan over runs stays short
  const int64_t g_cap = (nblk + kScanBatch - 1) / kScanBatch;
  const int G = static_cast<int>(min<int64_t>(kScanThreads / EQ, g_cap > 0 ? g_cap : 1));
  const int eq = tid % EQ, g = tid / EQ;
  const bool active = g < G;
  const int64_t chunk = (nblk + G - 1) / G;
  const int64_t b0 = active ? min<int64_t>(nblk, g * chunk) : 0;
  const int64_t b1 = active ? min<int64_t>(nblk, b0 + chunk) : 0;
  const float* fsrc = (gating == FFMOE_GATING_SOFTMAX) ? ws.psum : ws.ssum;
  const int64_t col = static_cast<int64_t>(eq) * EV;

  // the first batch of counts stays in registers for the second pass (one
  // expert per thread; with four, the registers go to more loads in flight)
  constexpr bool kKeep = EV == 1;
  int run[EV];
  float ps[EV];
  int first[kScanBatch][EV];
#pragma unroll
  for (int v = 0; v < EV; ++v) {
    run[v] = 0;
    ps[v] = 0.0f;
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) first[j][v] = 0;
  }
  for (int64_t b = b0; b < b1; b += kScanBatch) {
    int c[kScanBatch][EV];
    float p[kScanBatch][EV];
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) {
      const bool in = b + j < b1;
      load_ev<EV>(ws.hist + (b + j) * E + col, in, c[j]);
      load_ev<EV>(fsrc + (b + j) * E + col, in, p[j]);
    }
#pragma unroll
    for (int j = 0; j < kScanBatch; ++j) {
#pragma unroll
      for (int v = 0; v < EV; ++v) {
        run[v] += c[j][v];
        ps[v] += p[j][v];  // in block order; the padding adds +0
        if (kKeep && b == b0) first[j][v] = c[j][v];
      }
    }
  }
  // z: strided partial sums, reduced below by a fixed tree
  float z = 0.0f;
  for (int64_t b = tid; b < nblk; b += kScanThreads) z += ws.zpart[b];

  // inclusive scan of each expert's chunk sums over the runs (Hillis-Steele;
  // run g of group eq is thread g * EQ + eq)
  int incl[EV];
  float ptot[EV];
#pragma unroll
  for (int v = 0; v < EV; ++v) {
    incl[v] = run[v];
    ptot[v] = ps[v];
  }
  store_lds_ev<EV>(s_i + tid * EV, incl);
  store_lds_ev<EV>(s_f + tid * EV, ptot);
  __syncthreads();
  for (int off = 1; off < G; off <<= 1) {
    int ai[EV];
    float af[EV];
    const bool has = active && g >= off;
    load_ev<EV>(s_i + (has ? tid - off * EQ : tid) * EV, has, ai);
    load_ev<EV>(s_f + (has ? tid - off * EQ : tid) * EV, has, af);
    __syncthreads();
#pragma unroll
    for (int v = 0; v < EV; ++v) {
      incl[v] += ai[v];
      ptot[v] += af[v];
    }
    store_lds_ev<EV>(s_i + tid * EV, incl);
    store_lds_ev<EV>(s_f + tid * EV, ptot);
    __syncthreads();
  }
  if (active) {
    int base[EV];
#pragma unroll
    for (int v = 0; v < EV; ++v) base[v] = incl[v] - run[v];
    for (int64_t b = b0; b < b1; b += kScanBatch) {
      int c[kScanBatch][EV];
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j) {
        if (kKeep && b == b0) {
#pragma unroll
          for (int v = 0; v < EV; ++v) c[j][v] = first[j][v];
        } else {
          load_ev<EV>(ws.hist + (b + j) * E + col, b + j < b1, c[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j) {
        if (b + j < b1) {
          int32_t* dst = ws.hist + (b + j) * E + col;
          if constexpr (EV == 4) {
            *reinterpret_cast<int4*>(dst) = make_int4(base[0], base[1], base[2], base[3]);
          } else {
            dst[0] = base[0];
          }
#pragma unroll
          for (int v = 0; v < EV; ++v) base[v] += c[j][v];
        }
      }
    }
    if (g == G - 1) {  // incl is each expert's total
#pragma unroll
      for (int v = 0; v < EV; ++v) {
        const int e = eq * EV + v;
        s_cnt[e] = incl[v];
        s_p[e] = ptot[v];
        counts[e] = incl[v];
      }
    }
  }
  __syncthreads();

  // per expert (thread q < E): rows, tiles, the aux term; exclusive scans of
  // rows and tiles over the experts
  int cnt = 0, rows = 0, tiles = 0;
  float fp = 0.0f;
  if (tid < E) {
    cnt = s_cnt[tid];
    rows = min(cnt, mt);
    tiles = (rows + bm - 1) / bm;
    fp = (static_cast<float>(cnt) / static_cast<float>(N)) * (s_p[tid] / static_cast<float>(N));
  }
  // inclusive scans of rows and tiles within each expert wave (shuffles);
  // the waves' totals are added below through LDS
  const int wave = tid / kWave, lane = tid % kWave;
  int r_in = rows, t_in = tiles;
  if (wave < kEW) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int ar = __shfl_up(r_in, off, kWave), at = __shfl_up(t_in, off, kWave);
      if (lane >= off) {
        r_in += ar;
        t_in += at;
      }
    }
    if (lane == kWave - 1) {
      s_rw[wave] = r_in;
      s_tw[wave] = t_in;
    }
  }

  // fixed-tree reductions: z over all threads, the rest over the experts
  const auto add_f = [](float x, float y) { return x + y; };
  const float zw = wave_reduce(z, add_f);
  if (lane == 0) s_zw[wave] = zw;
  if (wave < kEW) {
    const bool ex = tid < E;
    const float fpw = wave_reduce(fp, add_f);
    const long long tw = wave_reduce(static_cast<long long>(cnt),
                                     [](long long x, long long y) { return x + y; });
    const int dw = wave_reduce(cnt - rows, [](int x, int y) { return x + y; });
    const int mxw = wave_reduce(cnt, [](int x, int y) { return max(x, y); });
    const int mnw = wave_reduce(ex ? cnt : 0x7fffffff, [](int x, int y) { return min(x, y); });
    if (lane == 0) {
      s_fpw[wave] = fpw;
      s_totw[wave] = tw;
      s_dw[wave] = dw;
      s_mxw[wave] = mxw;
      s_mnw[wave] = mnw;
    }
  }
  __syncthreads();
  if (tid < E) {
    for (int w = 0; w < wave; ++w) {
      r_in += s_rw[w];
      t_in += s_tw[w];
    }
    offsets[tid] = r_in - rows;
    tile_offsets[tid] = t_in - tiles;
    if (tid == E - 1) {
      offsets[E] = r_in;
      tile_offsets[E] = t_in;
    }
  }
  if (tid == 0) {
    float zt = 0.0f, fpt = 0.0f;
    for (int q = 0; q < kWaves; ++q) zt += s_zw[q];
    long long tot = 0;
    int mx = 0, mn = 0x7fffffff, dropped = 0;
    for (int q = 0; q < kEW; ++q) {
      fpt += s_fpw[q];
      tot += s_totw[q];
      dropped += s_dw[q];
      mx = max(mx, s_mxw[q]);
      mn = min(mn, s_mnw[q]);
    }
    stats[FFMOE_STAT_AUX] = aux_coeff * static_cast<float>(E) * fpt;
    stats[FFMOE_STAT_Z] = z_coeff * (zt / static_cast<float>(N));
    if (aux_out != nullptr) *aux_out = stats[FFMOE_STAT_AUX];
    if (z_out != nullptr) *z_out = stats[FFMOE_STAT_Z];
    const float mean = static_cast<float>(tot) / static_cast<float>(E);
    stats[FFMOE_STAT_IMBALANCE] = static_cast<float>(mx) / (mean + 1e-6f);
    stats[FFMOE_STAT_DROP_FRAC] = static_cast<float>(dropped) / static_cast<float>(N * k);
    istats[FFMOE_ISTAT_MAX] = mx;
    istats[FFMOE_ISTAT_MIN] = mn;
    istats[FFMOE_ISTAT_DROPPED] = dropped;
    istats[3] = 0;
  }
}

constexpr int kPermTokens = 8;  // tokens per permute block

// Resolves each entry's row (block base + block-local rank), renormalises the
// kept weights in capacity mode, and copies each token row (nvec 16-byte
// vectors: any element type) once from HBM to each of its k destination rows.
__global__ __launch_bounds__(256) void permute_kernel(
    const uint4* __restrict__ x, const int64_t* __restrict__ topk_idx, float* __restrict__ topk_w,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ rank_local, const int32_t* __restrict__ base, int64_t N, int nvec,
    int E, int k, int mt, int capacity_mode, uint4* __restrict__ xs, int32_t* __restrict__ row_of) {
  __shared__ int s_row[kPermTokens * FFMOE_MAX_TOPK];
  const int tid = threadIdx.x;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kPermTokens;
  const int ntok = static_cast<int>(min<int64_t>(kPermTokens, N - t0));
  const int nent = ntok * k;
  for (int q = tid; q < nent; q += blockDim.x) {
    const int64_t j = t0 * k + q;
    const int64_t n = j / k;
    const int e = static_cast<int>(topk_idx[j]);
    const int rank = base[(n / kRouteTokens) * E + e] + rank_local[j];
    int row;
    if (rank < mt) {
      row = offsets[e] + rank;
    } else if (capacity_mode) {
      row = FFMOE_ROW_DROPPED;
    } else {
      row = counts[0] > 0 ? FFMOE_ROW_ALIAS0 : FFMOE_ROW_DROPPED;
    }
    s_row[q] = row;
    row_of[j] = row;
  }
  __syncthreads();
  if (capacity_mode && tid < ntok) {
    // fused_moe.py:371-375: w*keep / (sum + (1 - has_any))
    const int64_t n = t0 + tid;
    float s = 0.0f;
    for (int q = 0; q < k; ++q) {
      const float w = s_row[tid * k + q] >= 0 ? topk_w[n * k + q] : 0.0f;
      s += w;
    }
    const float den = s + (s > 0.0f ? 0.0f : 1.0f);
    for (int q = 0; q < k; ++q) {
      const float w = s_row[tid * k + q] >= 0 ? topk_w[n * k + q] : 0.0f;
      topk_w[n * k + q] = w / den;
    }
  }
  for (int p = tid; p < ntok * nvec; p += blockDim.x) {
    const int t = p / nvec, v = p % nvec;
    const uint4 val = x[(t0 + t) * static_cast<int64_t>(nvec) + v];
    for (int q = 0; q < k; ++q) {
      const int row = s_row[t * k + q];
      if (row >= 0) xs[static_cast<int64_t>(row) * nvec + v] = val;
    }
  }
}

#endif  // FFMOE_ROUTE_PART == 0

template <int ET, int KMAX, int SRC>
static void launch_route(dim3 grid, size_t shm, hipStream_t st, const bf16_t* x, const bf16_t* gate,
                         const void* li, const RouteOpts& o, int64_t N, int D, int E, int k,
                         int gating, int need_ssum, bf16_t* lo, int64_t* ti, float* tw, float* lse,
                         int32_t* rl, RouteWs ws) {
  hipLaunchKernelGGL((route_fwd_kernel<ET, KMAX, SRC>), grid, dim3(kRouteThreads), shm, st, x, gate,
                     li, o, N, D, E, k, gating, need_ssum, lo, ti, tw, lse, rl, ws);
}

template <int ET, int KMAX>
static void launch_route_fl(int src, dim3 grid, size_t shm, hipStream_t st, const bf16_t* x,
                            const bf16_t* gate, const void* li, const RouteOpts& o, int64_t N,
                            int D, int E, int k, int gating, int need_ssum, bf16_t* lo, int64_t* ti,
                            float* tw, float* lse, int32_t* rl, RouteWs ws) {
  if (src == kLogitsBf16)
    launch_route<ET, KMAX, kLogitsBf16>(grid, shm, st, x, gate, li, o, N, D, E, k, gating, need_ssum,
                                        lo, ti, tw, lse, rl, ws);
  else if (src == kLogitsF32)
    launch_route<ET, KMAX, kLogitsF32>(grid, shm, st, x, gate, li, o, N, D, E, k, gating, need_ssum,
                                       lo, ti, tw, lse, rl, ws);
  else
    launch_route<ET, KMAX, kGateGemm>(grid, shm, st, x, gate, li, o, N, D, E, k, gating, need_ssum,
                                      lo, ti, tw, lse, rl, ws);
}

template <int ET>
void launch_route_k(int k, int fl, dim3 grid, size_t shm, hipStream_t st, const bf16_t* x,
                           const bf16_t* gate, const void* li, const RouteOpts& o, int64_t N,
                           int D, int E, int gating, int need_ssum, bf16_t* lo, int64_t* ti,
                           float* tw, float* lse, int32_t* rl, RouteWs ws) {
#define FFMOE_RK(KM)                                                                           \
  launch_route_fl<ET, KM>(fl, grid, shm, st, x, gate, li, o, N, D, E, k, gating, need_ssum, \
                          lo, ti, tw, lse, rl, ws)
  if (k <= 2)
    FFMOE_RK(2);
  else if (k <= 4)
    FFMOE_RK(4);
  else if (k <= 8)
    FFMOE_RK(8);
  else
    FFMOE_RK(16);
#undef FFMOE_RK
}

// The route kernel has 8 instantiations per expert-count tier ET; each tier
// is compiled in a translation unit of its own (FFMOE_ROUTE_PART = ET), in
// parallel, and part 0 holds everything else.
#define FFMOE_ROUTE_K_INST(ETV)                                                                     \
  template void launch_route_k<ETV>(int, int, dim3, size_t, hipStream_t, const bf16_t*,          \
                                    const bf16_t*, const void*, const RouteOpts&, int64_t, int,   \
                                    int, int, int, bf16_t*, int64_t*, float*, float*, int32_t*,    \
                                    RouteWs)
#if FFMOE_ROUTE_PART > 0
FFMOE_ROUTE_K_INST(FFMOE_ROUTE_PART);
#else
#define FFMOE_ROUTE_K_EXT(ETV) extern FFMOE_ROUTE_K_INST(ETV)
FFMOE_ROUTE_K_EXT(1);
FFMOE_ROUTE_K_EXT(2);
FFMOE_ROUTE_K_EXT(4);
FFMOE_ROUTE_K_EXT(8);
FFMOE_ROUTE_K_EXT(16);
#undef FFMOE_ROUTE_K_EXT
#endif

}  // namespace ffmoe

#if FFMOE_ROUTE_PART == 0

using namespace ffmoe;

// Workspace: hist, psum, ssum [nb][E], zpart [nb], then (256-byte aligned)
// rank_local [N*k] int32.
static size_t rank_local_offset(int64_t N, int E) {
  const int64_t nb = route_blocks(N);
  return (static_cast<size_t>(nb * E * 3 + nb) * 4 + 255) / 256 * 256;
}

extern "C" size_t ffmoe_route_workspace_bytes(int64_t N, int E, int k) {
  return rank_local_offset(N, E) + static_cast<size_t>(N) * k * 4;
}

static int route_fwd_impl(const void* x, const void* gate, const void* logits_in, RouteOpts o,
                          int64_t N, int D, int E, int k, int gating, int need_sigmoid_sum,
                          void* logits_out, int64_t* topk_idx, float* topk_w, float* lse,
                          void* workspace, void* stream, bool logits_f32 = false) {
  if (N <= 0) return set_error("ffmoe_route_fwd: N must be positive");
  if (E < 1 || E > FFMOE_MAX_EXPERTS) return set_error("ffmoe_route_fwd: E out of range [1, 256]");
  if (k < 1 || k > E || k > FFMOE_MAX_TOPK)
    return set_error("ffmoe_route_fwd: top_k must be in [1, min(E, 16)]");
  if (logits_in == nullptr && (D <= 0 || D % 8 != 0))
    return set_error("ffmoe_route_fwd: D must be a positive multiple of 8");
  if (gating != FFMOE_GATING_SOFTMAX && gating != FFMOE_GATING_SIGMOID)
    return set_error("ffmoe_route_fwd: unknown gating");
  if (workspace == nullptr || topk_idx == nullptr || topk_w == nullptr)
    return set_error("ffmoe_route_fwd: null output");
  if (o.n_group > 0) {
    if (E % o.n_group != 0)
      return set_error("ffmoe_route_fwd: E (" + std::to_string(E) + ") must be divisible by n_group (" +
                       std::to_string(o.n_group) + ")");
    if (o.topk_group < 1 || o.topk_group > o.n_group || o.topk_group > FFMOE_MAX_TOPK)
      return set_error("ffmoe_route_fwd: topk_group must be in [1, min(n_group, 16)]");
    if (o.topk_group * (E / o.n_group) < k)
      return set_error("ffmoe_route_fwd: topk_group groups hold fewer than top_k experts");
  }
  if (o.noise != nullptr && logits_in != nullptr)
    return set_error("ffmoe_route_fwd: input jitter needs the gate GEMM (no logits_in)");
  if (gating != FFMOE_GATING_SOFTMAX) o.pre_softmax = 0;  // the reference ignores it there
  const int ET = E <= 16 ? 1 : E <= 32 ? 2 : E <= 64 ? 4 : E <= 128 ? 8 : 16;
  const size_t lsz = logits_f32 ? 4 : 2;
  const int LS = ET * 16 + static_cast<int>(4 / lsz);  // logits per LDS row (rows padded by 4 bytes)
  const size_t shm = static_cast<size_t>(kRouteTokens) * LS * lsz +
                     (2 * static_cast<size_t>(kRouteTokens) * k + kRouteTokens) * 4;
  RouteWs ws = route_ws(workspace, N, E);
  int32_t* rl = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + rank_local_offset(N, E));
  const dim3 grid(static_cast<unsigned>(route_blocks(N)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int fl = logits_in == nullptr ? kGateGemm : (logits_f32 ? kLogitsF32 : kLogitsBf16);
  auto xb = static_cast<const bf16_t*>(x);
  auto gb = static_cast<const bf16_t*>(gate);
  const void* lb = logits_in;
  auto lo = static_cast<bf16_t*>(logits_out);
#define FFMOE_RE(ETV)                                                                           \
  launch_route_k<ETV>(k, fl, grid, shm, st, xb, gb, lb, o, N, D, E, gating, need_sigmoid_sum,   \
                      lo, topk_idx, topk_w, lse, rl, ws)
  switch (ET) {
    case 1: FFMOE_RE(1); break;
    case 2: FFMOE_RE(2); break;
    case 4: FFMOE_RE(4); break;
    case 8: FFMOE_RE(8); break;
    default: FFMOE_RE(16); break;
  }
#undef FFMOE_RE
  if (check_launch("route_fwd_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_route_fwd(const void* x, const void* gate, const void* logits_in,
                               const float* expert_bias, int64_t N, int D, int E, int k,
                               int gating, int need_sigmoid_sum, void* logits_out,
                               int64_t* topk_idx, float* topk_w, float* lse, void* workspace,
                               void* stream) {
  RouteOpts o{expert_bias, 0, 0, 0.0f, 0, 0, nullptr};
  return route_fwd_impl(x, gate, logits_in, o, N, D, E, k, gating, need_sigmoid_sum, logits_out,
                        topk_idx, topk_w, lse, workspace, stream);
}

extern "C" int ffmoe_route_fwd_ex(const void* x, const void* gate, const void* logits_in,
                                  const float* expert_bias, int bias_round_bf16, int pre_softmax,
                                  float scoring_factor, int n_group, int topk_group,
                                  const void* jitter_noise, int64_t N, int D, int E, int k,
                                  int gating, int need_sigmoid_sum, void* logits_out,
                                  int64_t* topk_idx, float* topk_w, float* lse, void* workspace,
                                  void* stream) {
  RouteOpts o{expert_bias, bias_round_bf16, pre_softmax, scoring_factor, n_group, topk_group,
              static_cast<const bf16_t*>(jitter_noise)};
  return route_fwd_impl(x, gate, logits_in, o, N, D, E, k, gating, need_sigmoid_sum, logits_out,
                        topk_idx, topk_w, lse, workspace, stream);
}

extern "C" int ffmoe_route_logits_f32(const float* logits, const float* expert_bias, int pre_softmax,
                                      float scoring_factor, int n_group, int topk_group, int64_t N, int E,
                                      int k, int gating, int need_sigmoid_sum, int64_t* topk_idx,
                                      float* topk_w, float* lse, void* workspace, void* stream) {
  if (logits == nullptr) return set_error("ffmoe_route_logits_f32: null logits");
  RouteOpts o{expert_bias, 0, pre_softmax, scoring_factor, n_group, topk_group, nullptr};
  return route_fwd_impl(nullptr, nullptr, logits, o, N, 0, E, k, gating, need_sigmoid_sum, nullptr, topk_idx,
                        topk_w, lse, workspace, stream, true);
}

extern "C" int ffmoe_route_scan(int64_t N, int E, int k, int mt, int gemm_bm, float aux_coeff,
                                float z_coeff, int gating, void* workspace, int32_t* counts,
                                int32_t* offsets, int32_t* tile_offsets, float* stats,
                                int32_t* istats, float* aux_out, float* z_out, void* stream) {
  if (N <= 0 || E < 1 || E > FFMOE_MAX_EXPERTS) return set_error("ffmoe_route_scan: bad N/E");
  if (mt < 0 || gemm_bm <= 0) return set_error("ffmoe_route_scan: bad mt/gemm_bm");
  RouteWs ws = route_ws(workspace, N, E);
  // four experts per thread: 16-byte loads of the per-block arrays
  if (E % 4 == 0 && reinterpret_cast<uintptr_t>(workspace) % 16 == 0)
    hipLaunchKernelGGL(route_scan_kernel<4>, dim3(1), dim3(kScanThreads), 0, static_cast<hipStream_t>(stream),
                       N, route_blocks(N), E, k, mt, gemm_bm, aux_coeff, z_coeff, gating, ws, counts,
                       offsets, tile_offsets, stats, istats, aux_out, z_out);
  else
    hipLaunchKernelGGL(route_scan_kernel<1>, dim3(1), dim3(kScanThreads), 0, static_cast<hipStream_t>(stream),
                       N, route_blocks(N), E, k, mt, gemm_bm, aux_coeff, z_coeff, gating, ws, counts,
                       offsets, tile_offsets, stats, istats, aux_out, z_out);
  if (check_launch("route_scan_kernel")) return 1;
  return clear_error();
}

static int permute_impl(const void* x, const int64_t* topk_idx, float* topk_w, const int32_t* offsets,
                        const int32_t* counts, int64_t N, int64_t row_bytes, int E, int k, int mt,
                        int capacity_mode, void* workspace, void* x_sorted, int32_t* row_of, void* stream,
                        const char* name) {
  if (N <= 0 || row_bytes <= 0 || row_bytes % 16 != 0 || row_bytes / 16 > 0x7fffffff)
    return set_error(std::string(name) + ": rows must be a positive multiple of 16 bytes");
  if (k < 1 || k > FFMOE_MAX_TOPK || E < 1 || E > FFMOE_MAX_EXPERTS)
    return set_error(std::string(name) + ": bad k/E");
  RouteWs ws = route_ws(workspace, N, E);
  const int32_t* rl =
      reinterpret_cast<const int32_t*>(static_cast<char*>(workspace) + rank_local_offset(N, E));
  const dim3 grid(static_cast<unsigned>((N + kPermTokens - 1) / kPermTokens));
  hipLaunchKernelGGL(permute_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(x), topk_idx, topk_w, offsets, counts, rl, ws.hist, N,
                     static_cast<int>(row_bytes / 16), E, k, mt, capacity_mode, static_cast<uint4*>(x_sorted),
                     row_of);
  if (check_launch("permute_kernel")) return 1;
  return clear_error();
}

extern "C" int ffmoe_permute(const void* x, const int64_t* topk_idx, float* topk_w,
                             const int32_t* offsets, const int32_t* counts, int64_t N, int D, int E,
                             int k, int mt, int capacity_mode, void* workspace, void* x_sorted,
                             int32_t* row_of, void* stream) {
  if (D <= 0 || D % 8 != 0) return set_error("ffmoe_permute: D must be a positive multiple of 8");
  return permute_impl(x, topk_idx, topk_w, offsets, counts, N, static_cast<int64_t>(D) * 2, E, k, mt,
                      capacity_mode, workspace, x_sorted, row_of, stream, "ffmoe_permute");
}

extern "C" int ffmoe_t_permute(int dtype, const void* x, const int64_t* topk_idx, float* topk_w,
                               const int32_t* offsets, const int32_t* counts, int64_t N, int D, int E,
                               int k, int mt, int capacity_mode, void* workspace, void* x_sorted,
                               int32_t* row_of, void* stream) {
  const int es = dtype == FFMOE_DTYPE_F32 ? 4 : dtype == FFMOE_DTYPE_F64 ? 8 : 0;
  if (es == 0) return set_error("ffmoe_t_permute: dtype must be FFMOE_DTYPE_F32 or FFMOE_DTYPE_F64");
  if (D <= 0 || D % 8 != 0) return set_error("ffmoe_t_permute: D must be a positive multiple of 8");
  return permute_impl(x, topk_idx, topk_w, offsets, counts, N, static_cast<int64_t>(D) * es, E, k, mt,
                      capacity_mode, workspace, x_sorted, row_of, stream, "ffmoe_t_permute");
}

#endif  // FFMOE_ROUTE_PART == 0
