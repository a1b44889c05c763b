// Router: fp32 softmax over experts + top-k + renormalisation + cast.
//
// Replaces models/layers.py:606-610 of the reference:
//   probs = F.softmax(logits, -1, dtype=float32)
//   w, idx = torch.topk(probs, k);  w = w / w.sum(-1).clamp_min(1e-12);  w.to(dtype)
//
// Layout: LPR lanes (a quad, or a DPP row of 16) own one token row; lane q
// holds the contiguous experts [q*C, (q+1)*C) with C = NP2/LPR (NP2 = padded
// expert count).  Cross-lane steps are DPP moves inside the row: quad
// permutations for lane distances 1 and 2, row rotations for 4 and 8.  The
// launcher uses quads: the ordering network and weight sum run once per row
// group of a wave, so 16 rows per wave issue fewer instructions in total than
// 4 rows per wave, even though each selection round is longer.
//
// Bit-exactness with torch on the device:
//  * softmax: torch's persistent softmax reduces a row across a wavefront with
//    an xor butterfly.  For padded size NP2 that is the pairwise tree
//    S_i <- S_i + S_{i+o}, o = NP2/2 ... 1.  Levels o >= C pair lanes q and
//    q ^ (o/C); levels o < C stay inside a lane.  Levels run from the largest
//    distance down, so when a rotation by 4 replaces xor 4 the lanes it
//    reads hold the same sums as their xor partners (rotation by 8 is xor 8
//    in a row of 16).  Additions are commutative, so every lane of the row ends
//    with the same bits.  exp is expf, and the division is IEEE.  Padding
//    experts hold exp(-inf) = 0, which leaves every partial sum unchanged.
//  * top-k: selection in (value desc, index asc) order, then torch's output
//    order and weight-sum order from topk_order.h.
#include <stdlib.h>

#include <mutex>

#include "common.h"
#include "route_wave.h"
#include "topk_order.h"

namespace hrm {
namespace {

constexpr int kRouterMaxExperts = 128;

// One selection round over the row's lanes: the largest remaining key, ties
// to the lower expert index; the winner's key is cleared in the lane that holds it.
template <int C, int LPR>
__device__ __forceinline__ void select_round(uint32_t (&key)[C], int e0, uint32_t& out_key, int& out_idx) {
  uint32_t bk = 0u;
  int be = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const bool b = key[j] > bk;
    bk = b ? key[j] : bk;
    be = b ? e0 + j : be;
  }
  auto merge = [&](uint32_t ok, int oe) __attribute__((always_inline)) {
    const bool b = ok > bk || (ok == bk && oe < be);
    bk = b ? ok : bk;
    be = b ? oe : be;
  };
  if constexpr (LPR == 16) {
    merge(xlane<8>(bk), (int)xlane<8>((uint32_t)be));
    merge(xlane<4>(bk), (int)xlane<4>((uint32_t)be));
  }
  merge(xlane<2>(bk), (int)xlane<2>((uint32_t)be));
  merge(xlane<1>(bk), (int)xlane<1>((uint32_t)be));
#pragma unroll
  for (int j = 0; j < C; ++j) key[j] = (e0 + j == be) ? 0u : key[j];
  out_key = bk;
  out_idx = be;
}

// KFIX: k == SLOTS, known at compile time (the usual top-2/4/8).
// RANK (k <= 8 only): also the first step of the dispatch for this block's
// RPB * k routed slots (flat index row * k + j): each slot's rank among the
// block's slots of the same expert bucket (bucket E holds ids outside [0, E)),
// and the block's per-bucket counts, counts[blockIdx.x][E + 1].  Same method
// as the dispatch's rank kernel (LDS bitmask per bucket, rank = popcount of
// the lower bits), so the stable order does not depend on atomic ordering.
// Outputs of the whole dispatch, written by a single-block launch (SOLO).
struct DispatchOut {
  int64_t* tokens_per_expert;
  int32_t* expert_offsets;
  int32_t* sorted_token_idx;
  int64_t* sort_idx;
  int32_t* slot_to_row;
};

// SOLO (with RANK, one block, T <= 64): the block's counts are the totals, so
// it also finishes the dispatch (bucket offsets, sorted rows) that the
// scan + scatter kernel does for larger T, saving that launch at decode sizes.
template <int NP2, int SLOTS, int LPR, bool KFIX, bool RANK = false, bool SOLO = false>
__global__ __launch_bounds__(256) void router_topk_kernel(const void* __restrict__ logits, int ldt, int64_t T, int E,
                                                          int k_rt, int norm, float* __restrict__ probs,
                                                          int64_t* __restrict__ idx_out, void* __restrict__ w_out,
                                                          int wdt, int32_t* __restrict__ rank_out,
                                                          int32_t* __restrict__ counts_out, DispatchOut dout) {
  static_assert(!SOLO || RANK, "the single-block dispatch needs the rank step");
  static_assert(!RANK || SLOTS <= 8, "the fused rank step runs in the register (k <= 8) path");
  constexpr int C = NP2 / LPR;
  constexpr int RPB = 256 / LPR;  // rows per block
  constexpr int KC = KFIX ? SLOTS : 0;
  const int k = KFIX ? SLOTS : k_rt;
  static_assert(LPR == 4 || LPR == 16, "4 or 16 lanes per row");
  static_assert(C >= 1 && (C & (C - 1)) == 0, "experts per lane");
  const int q = threadIdx.x % LPR;
  const int lr = threadIdx.x / LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + lr;
  const bool active = row < T;  // inactive lanes still take part in the row exchanges
  const int e0 = q * C;

  float s[C];
  float mx = -INFINITY;
  // Loads use a clamped (always valid) address and a select instead of a
  // branch per element.  With E a multiple of 8, 16-bit logits come in as
  // 16-byte vectors, each wholly inside or wholly outside the row.
  const int64_t rr = active ? row : T - 1;
  if (ldt != HRM_MOE_F32 && (E % 8) == 0 && (C % 8) == 0) {
    const uint16_t* base = reinterpret_cast<const uint16_t*>(logits) + rr * E;
#pragma unroll
    for (int v = 0; v < C / 8; ++v) {
      const int ev = e0 + v * 8;
      const bool in = active && ev < E;
      const u32x4 raw = *reinterpret_cast<const u32x4*>(base + (in ? ev : 0));
#pragma unroll
      for (int q2 = 0; q2 < 8; ++q2) {
        const uint16_t h = (uint16_t)(q2 & 1 ? raw[q2 >> 1] >> 16 : raw[q2 >> 1] & 0xffffu);
        const float f = ldt == HRM_MOE_BF16 ? BF16::to_f(h) : F16::to_f(h);
        s[v * 8 + q2] = in ? f : -INFINITY;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int e = e0 + j;
      const bool in = active && e < E;
      const float f = load_logit(logits, ldt, rr * E + (in ? e : 0));
      s[j] = in ? f : -INFINITY;
    }
  }
#pragma unroll
  for (int j = 0; j < C; ++j) mx = fmaxf(mx, s[j]);
  if constexpr (LPR == 16) {
    mx = fmaxf(mx, xlanef<8>(mx));
    mx = fmaxf(mx, xlanef<4>(mx));
  }
  mx = fmaxf(mx, xlanef<2>(mx));
  mx = fmaxf(mx, xlanef<1>(mx));

  float t[C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    s[j] = expf(s[j] - mx);
    t[j] = s[j];
  }
  // Pairwise tree of the wavefront butterfly: cross-lane levels first.
  if constexpr (LPR == 16) {
#pragma unroll
    for (int j = 0; j < C; ++j) t[j] = t[j] + xlanef<8>(t[j]);
#pragma unroll
    for (int j = 0; j < C; ++j) t[j] = t[j] + xlanef<4>(t[j]);
  }
#pragma unroll
  for (int j = 0; j < C; ++j) t[j] = t[j] + xlanef<2>(t[j]);
#pragma unroll
  for (int j = 0; j < C; ++j) t[j] = t[j] + xlanef<1>(t[j]);
#pragma unroll
  for (int o = C / 2; o > 0; o /= 2) {
#pragma unroll
    for (int i = 0; i < o; ++i) t[i] = t[i] + t[i + o];
  }
  const float total = t[0];

  uint32_t key[C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    s[j] = s[j] / total;
    const bool ok = active && e0 + j < E;
    key[j] = ok ? (__float_as_uint(s[j]) + 1u) : 0u;  // 0 marks "not selectable"
  }
  // The lane's C probabilities are contiguous in the row: 16-byte stores when
  // the lane's range lies inside the row and the rows are 16-byte aligned
  // (16 single stores per lane cost 2.6 us more at 16384 tokens, 64 experts).
  if (probs != nullptr && active) {
    if ((C % 4) == 0 && (E % 4) == 0 && e0 + C <= E && (reinterpret_cast<uintptr_t>(probs) & 15) == 0) {
#pragma unroll
      for (int v = 0; v < C / 4; ++v)
        *reinterpret_cast<float4*>(probs + row * E + e0 + 4 * v) = float4{s[4 * v], s[4 * v + 1], s[4 * v + 2],
                                                                          s[4 * v + 3]};
    } else {
#pragma unroll
      for (int j = 0; j < C; ++j)
        if (e0 + j < E) probs[row * E + e0 + j] = s[j];
    }
  }

  // Top-k selection in (value desc, index asc) order: k rounds of a row-wide
  // argmax (ties to the lower expert index), each removing its winner.
  if constexpr (SLOTS <= 8) {
    uint32_t sk[SLOTS];
    int si[SLOTS];
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
      sk[r] = 0u;
      si[r] = 0;
      if (r < k) select_round<C, LPR>(key, e0, sk[r], si[r]);
    }
    if (!RANK && !active) return;  // with RANK every thread reaches the block barriers below
    uint32_t gk[SLOTS];
    int gi[SLOTS];
    torch_topk_order<SLOTS, KC>(sk, si, k, gk, gi);
    float w[SLOTS];
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) w[j] = __uint_as_float(gk[j] - 1u);
    if (norm) {
      float sum = torch_row_sum<SLOTS, KC>(w, k);
      sum = (sum != sum) ? sum : fmaxf(sum, 1e-12f);
#pragma unroll
      for (int j = 0; j < SLOTS; ++j) w[j] = w[j] / sum;
    }
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      if (active && j < k && (j % LPR) == q) {
        idx_out[row * k + j] = (int64_t)gi[j];
        store_weight(w_out, wdt, row * k + j, w[j]);
      }
    }
    if constexpr (RANK) {
      constexpr int SBMAX = RPB * 8;
      __shared__ uint32_t s_mask[(kRouterMaxExperts + 1) * (SBMAX / 32)];
      __shared__ uint32_t s_pref[(kRouterMaxExperts + 1) * (SBMAX / 32)];
      const int nbk = E + 1;
      // bitmask words for the slots of the rows this block holds (a single row at T = 1)
      const int rows_here = (int)min((int64_t)RPB, T - (int64_t)blockIdx.x * RPB);
      const int words = (rows_here * k + 31) / 32;
      for (int i = threadIdx.x; i < nbk * words; i += 256) s_mask[i] = 0u;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < SLOTS; ++j) {
        if (active && j < k && (j % LPR) == q) {
          const int ls = lr * k + j;
          const int b = (gi[j] >= 0 && gi[j] < E) ? gi[j] : E;
          atomicOr(&s_mask[b * words + (ls >> 5)], 1u << (ls & 31));
        }
      }
      __syncthreads();
      __shared__ int32_t s_off[kRouterMaxExperts + 1];
      for (int b = threadIdx.x; b < nbk; b += 256) {
        uint32_t run = 0;
        for (int w2 = 0; w2 < words; ++w2) {
          s_pref[b * words + w2] = run;
          run += __popc(s_mask[b * words + w2]);
        }
        if constexpr (SOLO) s_off[b] = (int32_t)run;
        else counts_out[(int64_t)blockIdx.x * nbk + b] = (int32_t)run;
      }
      __syncthreads();
      if constexpr (SOLO) {
        // bucket totals -> exclusive offsets (wave 0), tokens_per_expert
        if (threadIdx.x < 64) {
          const int lane = threadIdx.x;
          int32_t carry = 0;
          for (int c = 0; c < nbk; c += 64) {
            const int b = c + lane;
            const int32_t v = b < nbk ? s_off[b] : 0;
            int32_t incl = v;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
              const int32_t u = __shfl_up(incl, o, 64);
              if (lane >= o) incl += u;
            }
            if (b < nbk) {
              if (b < E) dout.tokens_per_expert[b] = (int64_t)v;
              s_off[b] = carry + incl - v;
              dout.expert_offsets[b] = carry + incl - v;  // [E]: start of the out-of-range ids
            }
            carry += __shfl(incl, 63, 64);
          }
        }
        __syncthreads();
      }
#pragma unroll
      for (int j = 0; j < SLOTS; ++j) {
        if (active && j < k && (j % LPR) == q) {
          const int ls = lr * k + j;
          const int b = (gi[j] >= 0 && gi[j] < E) ? gi[j] : E;
          const uint32_t below = s_mask[b * words + (ls >> 5)] & ((1u << (ls & 31)) - 1u);
          const int32_t rk = (int32_t)(s_pref[b * words + (ls >> 5)] + __popc(below));
          if constexpr (SOLO) {
            const int64_t sl = row * k + j;
            const int32_t dst = s_off[b] + rk;
            dout.sorted_token_idx[dst] = (int32_t)row;
            if (dout.sort_idx) dout.sort_idx[dst] = sl;
            dout.slot_to_row[sl] = dst;
          } else {
            rank_out[row * k + j] = rk;
          }
        }
      }
    }
  } else {
    // k > 8: the ordering runs in loop form on this row's LDS arrays (one lane per row).
    __shared__ uint32_t s_sk[RPB][SLOTS];
    __shared__ int s_si[RPB][SLOTS];
    __shared__ uint32_t s_gk[RPB][SLOTS];
    __shared__ int s_gi[RPB][SLOTS];
    __shared__ bool s_gv[RPB][SLOTS];
    for (int r = 0; r < k; ++r) {
      uint32_t bk;
      int be;
      select_round<C, LPR>(key, e0, bk, be);
      if (q == 0) {
        s_sk[lr][r] = bk;
        s_si[lr][r] = be;
      }
    }
    if (!active || q != 0) return;
    torch_topk_order_mem(s_sk[lr], s_si[lr], k, SLOTS, s_gk[lr], s_gi[lr], s_gv[lr]);
    float w[SLOTS];
    for (int j = 0; j < k; ++j) w[j] = __uint_as_float(s_gk[lr][j] - 1u);
    float sum = 1.0f;
    if (norm) {
      sum = torch_row_sum_mem(w, k);
      sum = (sum != sum) ? sum : fmaxf(sum, 1e-12f);
    }
    for (int j = 0; j < k; ++j) {
      idx_out[row * k + j] = (int64_t)s_gi[lr][j];
      store_weight(w_out, wdt, row * k + j, norm ? w[j] / sum : w[j]);
    }
  }
}

// Router with the fused rank step (k <= 8): RPB * k slots per rank block.
template <int NP2>
int launch_router_rank(const void* logits, int ldt, int64_t T, int E, int k, int norm, float* probs, int64_t* idx,
                       void* w, int wdt, int32_t* rank, int32_t* counts, const DispatchOut& dout, bool solo,
                       void* stream) {
  constexpr int LPR = 4, RPB = 256 / LPR;
  dim3 grid((unsigned)((T + RPB - 1) / RPB)), block(256);
#define HRM_RTR(SL, KF)                                                                                                \
  do {                                                                                                                 \
    if (solo)                                                                                                          \
      HRM_LAUNCH((router_topk_kernel<NP2, SL, LPR, KF, true, true>), grid, block, 0, stream, logits, ldt, T, E, k,   \
                 norm, probs, idx, w, wdt, rank, counts, dout);                                                        \
    else                                                                                                               \
      HRM_LAUNCH((router_topk_kernel<NP2, SL, LPR, KF, true>), grid, block, 0, stream, logits, ldt, T, E, k, norm,    \
                 probs, idx, w, wdt, rank, counts, dout);                                                              \
  } while (0)
  if (k == 2) HRM_RTR(2, true);
  else if (k == 4) HRM_RTR(4, true);
  else if (k == 8) HRM_RTR(8, true);
  else if (k <= 2) HRM_RTR(2, false);
  else if (k <= 4) HRM_RTR(4, false);
  else if (k <= 8) HRM_RTR(8, false);
  else return HRM_MOE_ERR_UNSUPPORTED;
#undef HRM_RTR
  return HRM_MOE_OK;
}

template <int NP2, int LPR>
int launch_router_np2(const void* logits, int ldt, int64_t T, int E, int k, int norm, float* probs, int64_t* idx,
                      void* w, int wdt, void* stream) {
  constexpr int RPB = 256 / LPR;
  dim3 grid((unsigned)((T + RPB - 1) / RPB)), block(256);
#define HRM_RT(SL, KF)                                                                                              \
  HRM_LAUNCH((router_topk_kernel<NP2, SL, LPR, KF>), grid, block, 0, stream, logits, ldt, T, E, k, norm, probs, idx, w, \
             wdt, (int32_t*)nullptr, (int32_t*)nullptr, DispatchOut{})
  if (k == 2) HRM_RT(2, true);
  else if (k == 4) HRM_RT(4, true);
  else if (k == 8) HRM_RT(8, true);
  else if (k <= 2) HRM_RT(2, false);
  else if (k <= 4) HRM_RT(4, false);
  else if (k <= 8) HRM_RT(8, false);
  else if constexpr (NP2 >= 16) {
    if (k <= 16) HRM_RT(16, false);
    else if constexpr (NP2 >= 32) {
      HRM_RT(32, false);
    } else {
      return HRM_MOE_ERR_UNSUPPORTED;
    }
  } else {
    return HRM_MOE_ERR_UNSUPPORTED;
  }
#undef HRM_RT
  return HRM_MOE_OK;
}

// Backward of the router (models/layers.py:606-610) as torch autograd computes it:
//   v_j = p[idx_j],  s = sum_j v_j,  c = max(s, 1e-12)
//   dv_j = g_w[j] / c - (sum_i g_w[i] v_i) / c^2 * [s >= 1e-12]   (norm_topk_prob; else dv_j = g_w[j])
//   dp_e = g_probs[e] + sum_{j: idx_j = e} dv_j                   (topk backward scatters to the chosen experts)
//   dlogits_e = p_e * (dp_e - sum_e' p_e' dp_e')                  (softmax backward)
// One wave per token; lane l holds experts l + 64 h, h < NE (NE = 2 up to 128
// experts).  The two sums over a row are fixed xor butterflies, so results
// are deterministic.
constexpr int kBwdTokPerBlock = 4;
template <int NE>
__global__ __launch_bounds__(kBwdTokPerBlock * 64) void router_bwd_kernel(
    const float* __restrict__ probs, const int64_t* __restrict__ idx, const void* __restrict__ g_w, int gw_dt,
    const float* __restrict__ g_probs, int64_t gp_stride, int64_t T, int E, int k, int norm, void* __restrict__ dlogits,
    int out_dt) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * kBwdTokPerBlock + (threadIdx.x >> 6);
  if (t >= T) return;  // no barriers below
  auto wsum = [](float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
  };
  const float* prow = probs + t * E;
  int ej = -1;
  float gj = 0.0f, vj = 0.0f;
  if (lane < k) {
    ej = (int)idx[t * k + lane];
    gj = load_logit(g_w, gw_dt, t * k + lane);
    vj = (ej >= 0 && ej < E) ? prow[ej] : 0.0f;
  }
  float dv = gj;
  if (norm) {
    const float sum = wsum(vj);
    const float dot = wsum(gj * vj);
    const float c = fmaxf(sum, 1e-12f);
    dv = gj / c - (sum >= 1e-12f ? dot / (c * c) : 0.0f);
  }
  float p[NE], dp[NE];
#pragma unroll
  for (int h = 0; h < NE; ++h) {
    const int e = lane + 64 * h;
    p[h] = e < E ? prow[e] : 0.0f;
    dp[h] = (e < E && g_probs) ? g_probs[t * gp_stride + e] : 0.0f;  // stride 0: one row for all tokens
  }
  for (int j = 0; j < k; ++j) {
    const int e = __shfl(ej, j, 64);
    const float d = __shfl(dv, j, 64);
#pragma unroll
    for (int h = 0; h < NE; ++h) dp[h] += (lane + 64 * h == e) ? d : 0.0f;
  }
  float part = p[0] * dp[0];
#pragma unroll
  for (int h = 1; h < NE; ++h) part = part + p[h] * dp[h];
  const float pd = wsum(part);
#pragma unroll
  for (int h = 0; h < NE; ++h) {
    const int e = lane + 64 * h;
    if (e < E) store_weight(dlogits, out_dt, t * E + e, p[h] * (dp[h] - pd));
  }
}

// Decode sizes (T <= 16 tokens, E <= 64, k <= 8): router and the whole
// dispatch in one block, one wave per token, lane e holding expert e.  A
// wave of the quad kernel runs the same serial chain (k arg-max rounds over
// 16 experts per lane, then the ordering network) whether it holds 16 rows or
// one; here each step is a handful of instructions.  Same arithmetic as
// router_topk_kernel, so the outputs are the same bits.  The per-token part
// is route_token_wave (route_wave.h), which the one-launch decode layer
// shares:
//  * softmax: the xor butterfly over lanes at distances 32 ... 1 is the
//    pairwise tree S_e <- S_e + S_(e^o) that the quad kernel evaluates
//    (cross-lane levels, then in-lane levels); fp32 addition commutes, so
//    both lanes of a pair hold the same bits.  Padding lanes hold 0.
//  * selection: each lane counts the (key, ~index) pairs above its own, i.e.
//    its rank in (key desc, index asc) order; ranks 0..k-1 are the k arg-max
//    rounds' winners in round order.  A round with no selectable key left
//    (key 0) yields index INT_MAX, as in the arg-max rounds.
//  * torch's output order equals that order unless two of the k keys are
//    equal (the network sorts distinct keys descending), so the ordering
//    network runs only then: a wave-uniform branch, one token per wave.
//  * weight sum in torch's order, IEEE division.
//  * dispatch: stable counting sort of the T*k slots by bucket (expert, or E
//    for an id outside [0, E)) with the rank step's LDS bitmasks.
//  * RANK (more than 16 tokens): blocks of 16 tokens, each writing its slots'
//    ranks within their bucket and its bucket counts (the rank step's output);
//    the scan + scatter launch then finishes the dispatch.
constexpr int kWaveRouterMaxTokens = 16;

template <int SLOTS, bool KFIX, bool RANK = false>
__global__ __launch_bounds__(64 * kWaveRouterMaxTokens) void router_dispatch_wave_kernel(
    const void* __restrict__ logits, int ldt, int T, int E, int k_rt, int norm, float* __restrict__ probs,
    int64_t* __restrict__ idx_out, void* __restrict__ w_out, int wdt, DispatchOut dout, int32_t* __restrict__ rank_out,
    int32_t* __restrict__ counts_out) {
  static_assert(SLOTS <= 8, "k <= 8");
  constexpr int kMaxWords = (kWaveRouterMaxTokens * 8 + 31) / 32;
  const int k = KFIX ? SLOTS : k_rt;
  const int lane = threadIdx.x & 63;
  const int tl = threadIdx.x >> 6;  // this wave's token within the block
  // RANK: blocks of 16 tokens, the last one possibly partial (its idle waves
  // still pass every barrier); otherwise one block of T waves
  const int t = RANK ? blockIdx.x * kWaveRouterMaxTokens + tl : tl;
  const int Tb = RANK ? min(kWaveRouterMaxTokens, T - (int)blockIdx.x * kWaveRouterMaxTokens) : T;
  const bool active = t < T;
  __shared__ uint64_t s_ck[kWaveRouterMaxTokens][64];
  __shared__ uint32_t s_sk[kWaveRouterMaxTokens][SLOTS];
  __shared__ int32_t s_si[kWaveRouterMaxTokens][SLOTS];
  __shared__ uint32_t s_mask[65 * kMaxWords];
  __shared__ uint32_t s_pref[65 * kMaxWords];
  __shared__ int32_t s_off[65];

  int my_i;
  float my_w;
  route_token_wave<SLOTS, KFIX>(logits, ldt, t, active, E, k, norm, probs, s_ck[tl], s_sk[tl], s_si[tl], my_i, my_w);
  const bool slot = active && lane < k;
  const int ls = t * k + lane;    // flat slot index
  const int lb = tl * k + lane;   // slot index within the block
  if (slot) {
    idx_out[ls] = (int64_t)my_i;
    store_weight(w_out, wdt, ls, my_w);
  }

  // dispatch of the block's Tb*k slots
  const int nbk = E + 1;
  const int words = (Tb * k + 31) / 32;
  for (int i = threadIdx.x; i < nbk * words; i += blockDim.x) s_mask[i] = 0u;
  __syncthreads();
  const int b = (my_i >= 0 && my_i < E) ? my_i : E;
  if (slot) atomicOr(&s_mask[b * words + (lb >> 5)], 1u << (lb & 31));
  __syncthreads();
  for (int c = threadIdx.x; c < nbk; c += blockDim.x) {
    uint32_t run = 0;
    for (int w2 = 0; w2 < words; ++w2) {
      s_pref[c * words + w2] = run;
      run += __popc(s_mask[c * words + w2]);
    }
    s_off[c] = (int32_t)run;
    if constexpr (RANK) counts_out[(int64_t)blockIdx.x * nbk + c] = (int32_t)run;
  }
  __syncthreads();
  if constexpr (RANK) {
    if (slot) {
      const uint32_t below = s_mask[b * words + (lb >> 5)] & ((1u << (lb & 31)) - 1u);
      rank_out[ls] = (int32_t)(s_pref[b * words + (lb >> 5)] + __popc(below));
    }
    return;
  }
  if (threadIdx.x < 64) {  // bucket totals -> exclusive offsets
    int32_t carry = 0;
    for (int c0 = 0; c0 < nbk; c0 += 64) {
      const int c = c0 + lane;
      const int32_t v = c < nbk ? s_off[c] : 0;
      int32_t incl = v;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int32_t u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
      }
      if (c < nbk) {
        if (c < E) dout.tokens_per_expert[c] = (int64_t)v;
        s_off[c] = carry + incl - v;
        dout.expert_offsets[c] = carry + incl - v;
      }
      carry += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
  if (slot) {
    const uint32_t below = s_mask[b * words + (lb >> 5)] & ((1u << (lb & 31)) - 1u);
    const int32_t dst = s_off[b] + (int32_t)(s_pref[b * words + (lb >> 5)] + __popc(below));
    dout.sorted_token_idx[dst] = t;
    if (dout.sort_idx) dout.sort_idx[dst] = ls;
    dout.slot_to_row[ls] = dst;
  }
}

// T <= 16 tokens, E <= 64, k <= 8: one block of T waves.  With rank/counts
// (more tokens): blocks of 16 waves, the rank step's output for the scan +
// scatter launch.
int launch_router_dispatch_wave(const void* logits, int ldt, int64_t T, int E, int k, int norm, float* probs,
                                int64_t* idx, void* w, int wdt, const DispatchOut& dout, void* stream,
                                int32_t* rank = nullptr, int32_t* counts = nullptr) {
  const bool rk = rank != nullptr;
  const dim3 grid(rk ? (unsigned)((T + kWaveRouterMaxTokens - 1) / kWaveRouterMaxTokens) : 1u),
      block((unsigned)(64 * (rk ? kWaveRouterMaxTokens : T)));
#define HRM_RW(SL, KF)                                                                                              \
  do {                                                                                                              \
    if (rk)                                                                                                         \
      HRM_LAUNCH((router_dispatch_wave_kernel<SL, KF, true>), grid, block, 0, stream, logits, ldt, (int)T, E, k,   \
                 norm, probs, idx, w, wdt, dout, rank, counts);                                                     \
    else                                                                                                            \
      HRM_LAUNCH((router_dispatch_wave_kernel<SL, KF>), grid, block, 0, stream, logits, ldt, (int)T, E, k, norm,   \
                 probs, idx, w, wdt, dout, rank, counts);                                                           \
  } while (0)
  if (k == 2) HRM_RW(2, true);
  else if (k == 4) HRM_RW(4, true);
  else if (k == 8) HRM_RW(8, true);
  else if (k <= 2) HRM_RW(2, false);
  else if (k <= 4) HRM_RW(4, false);
  else HRM_RW(8, false);
#undef HRM_RW
  return HRM_MOE_OK;
}

// Rows of 129 to 1024 experts: one wave per token, lane l holding experts
// l + 64 j, j < NE = next_pow2(E) / 64, which is how torch's warp softmax
// holds rows of up to 1024 fp32 values (persistent softmax, warp size 64):
// padding elements are -inf, the row maximum and then the sum are taken per
// lane in j order (the sum starting from 0) and finished with the xor
// butterfly at distances 32 ... 1; p = e / sum.  Top-k as in the other
// kernels: k rounds of a row-wide arg-max in (key desc, index asc) order, then
// torch's ordering network and weight sum.
constexpr int kWideTokPerBlock = 4;
template <int NE, int SLOTS, bool KFIX>
__global__ __launch_bounds__(kWideTokPerBlock * 64) void router_topk_wide_kernel(
    const void* __restrict__ logits, int ldt, int64_t T, int E, int k_rt, int norm, float* __restrict__ probs,
    int64_t* __restrict__ idx_out, void* __restrict__ w_out, int wdt) {
  constexpr int KC = KFIX ? SLOTS : 0;
  const int k = KFIX ? SLOTS : k_rt;
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * kWideTokPerBlock + (threadIdx.x >> 6);
  if (t >= T) return;  // no block barriers below
  float s[NE];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    const int e = lane + 64 * j;
    const bool in = e < E;
    const float f = load_logit(logits, ldt, t * E + (in ? e : 0));
    s[j] = in ? f : -INFINITY;
    mx = fmaxf(mx, s[j]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    s[j] = expf(s[j] - mx);
    sum = sum + s[j];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum = sum + __shfl_xor(sum, o, 64);
  uint32_t key[NE];
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    const float p = s[j] / sum;
    const int e = lane + 64 * j;
    const bool ok = e < E;
    if (ok && probs != nullptr) probs[t * E + e] = p;
    key[j] = ok ? (__float_as_uint(p) + 1u) : 0u;  // 0 marks "not selectable"
  }
  uint32_t sk[SLOTS];
  int si[SLOTS];
#pragma unroll
  for (int r = 0; r < SLOTS; ++r) {
    sk[r] = 0u;
    si[r] = 0;
    if (r < k) {
      uint32_t bk = 0u;
      int be = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < NE; ++j) {
        const bool b = key[j] > bk;
        bk = b ? key[j] : bk;
        be = b ? lane + 64 * j : be;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const uint32_t ok = (uint32_t)__shfl_xor((int)bk, o, 64);
        const int oe = __shfl_xor(be, o, 64);
        const bool b = ok > bk || (ok == bk && oe < be);
        bk = b ? ok : bk;
        be = b ? oe : be;
      }
#pragma unroll
      for (int j = 0; j < NE; ++j) key[j] = (lane + 64 * j == be) ? 0u : key[j];
      sk[r] = bk;
      si[r] = be;
    }
  }
  uint32_t gk[SLOTS];
  int gi[SLOTS];
  torch_topk_order<SLOTS, KC>(sk, si, k, gk, gi);
  float w[SLOTS];
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) w[j] = __uint_as_float(gk[j] - 1u);
  if (norm) {
    float wsum = torch_row_sum<SLOTS, KC>(w, k);
    wsum = (wsum != wsum) ? wsum : fmaxf(wsum, 1e-12f);
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) w[j] = w[j] / wsum;
  }
  int my_i = 0;
  float my_w = 0.0f;
#pragma unroll
  for (int j = 0; j < SLOTS; ++j) {
    my_i = lane == j ? gi[j] : my_i;
    my_w = lane == j ? w[j] : my_w;
  }
  if (lane < k) {
    idx_out[t * k + lane] = (int64_t)my_i;
    store_weight(w_out, wdt, t * k + lane, my_w);
  }
}

template <int NE>
int launch_router_wide(const void* logits, int ldt, int64_t T, int E, int k, int norm, float* probs, int64_t* idx,
                       void* w, int wdt, void* stream) {
  const dim3 grid((unsigned)((T + kWideTokPerBlock - 1) / kWideTokPerBlock)), block(kWideTokPerBlock * 64);
#define HRM_RWD(SL, KF)                                                                                          \
  HRM_LAUNCH((router_topk_wide_kernel<NE, SL, KF>), grid, block, 0, stream, logits, ldt, T, E, k, norm, probs, idx, \
             w, wdt)
  if (k == 2) HRM_RWD(2, true);
  else if (k == 4) HRM_RWD(4, true);
  else if (k == 8) HRM_RWD(8, true);
  else if (k <= 2) HRM_RWD(2, false);
  else if (k <= 4) HRM_RWD(4, false);
  else if (k <= 8) HRM_RWD(8, false);
  else if (k <= 16) HRM_RWD(16, false);
  else HRM_RWD(32, false);
#undef HRM_RWD
  return HRM_MOE_OK;
}

}  // namespace
}  // namespace hrm

extern "C" int hrm_moe_router_topk(const void* logits, int logits_dtype, int64_t num_tokens, int32_t num_experts,
                                   int32_t top_k, int32_t norm_topk_prob, float* probs, int64_t* topk_idx,
                                   void* topk_weight, int weight_dtype, void* stream) {
  if (num_tokens < 0 || num_experts < 1 || top_k < 1 || top_k > num_experts) return HRM_MOE_ERR_INVALID;
  if (logits_dtype < HRM_MOE_BF16 || logits_dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (weight_dtype < HRM_MOE_BF16 || weight_dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (num_experts > 1024 || top_k > 32) return HRM_MOE_ERR_UNSUPPORTED;
  if (num_tokens == 0) return HRM_MOE_OK;
  if (!logits || !topk_idx || !topk_weight) return HRM_MOE_ERR_INVALID;
  const int E = num_experts, k = top_k;
  if (E > 128) {
#define HRM_WIDE(NE) \
  hrm::launch_router_wide<NE>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx, topk_weight, weight_dtype, stream)
    if (E <= 256) return HRM_WIDE(4);
    if (E <= 512) return HRM_WIDE(8);
    return HRM_WIDE(16);
#undef HRM_WIDE
  }
  if (E <= 8) return hrm::launch_router_np2<8, 4>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx, topk_weight, weight_dtype, stream);
  if (E <= 64) return hrm::launch_router_np2<64, 4>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx, topk_weight, weight_dtype, stream);
  return hrm::launch_router_np2<128, 4>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx, topk_weight, weight_dtype, stream);
}

extern "C" int hrm_moe_router_topk_backward(const float* probs, const int64_t* topk_idx, const void* grad_weight,
                                            int grad_weight_dtype, const float* grad_probs,
                                            int64_t grad_probs_row_stride, int64_t num_tokens,
                                            int32_t num_experts, int32_t top_k, int32_t norm_topk_prob,
                                            void* grad_logits, int logits_dtype, void* stream) {
  if (num_tokens < 0 || num_experts < 1 || top_k < 1 || top_k > num_experts) return HRM_MOE_ERR_INVALID;
  if (grad_probs && grad_probs_row_stride != 0 && grad_probs_row_stride < num_experts) return HRM_MOE_ERR_INVALID;
  if (grad_weight_dtype < HRM_MOE_BF16 || grad_weight_dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (logits_dtype < HRM_MOE_BF16 || logits_dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (num_experts > 1024 || top_k > 32) return HRM_MOE_ERR_UNSUPPORTED;
  if (num_tokens == 0) return HRM_MOE_OK;
  if (!probs || !topk_idx || !grad_weight || !grad_logits) return HRM_MOE_ERR_INVALID;
  const dim3 grid((unsigned)((num_tokens + hrm::kBwdTokPerBlock - 1) / hrm::kBwdTokPerBlock));
#define HRM_RB(NE)                                                                                                 \
  hipLaunchKernelGGL(hrm::router_bwd_kernel<NE>, grid, dim3(hrm::kBwdTokPerBlock * 64), 0, (hipStream_t)stream,    \
                     probs, topk_idx, grad_weight, grad_weight_dtype, grad_probs, grad_probs_row_stride, num_tokens, \
                     num_experts, top_k, norm_topk_prob, grad_logits, logits_dtype)
  if (num_experts <= 128) HRM_RB(2);
  else if (num_experts <= 256) HRM_RB(4);
  else if (num_experts <= 512) HRM_RB(8);
  else HRM_RB(16);
#undef HRM_RB
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? HRM_MOE_OK : (int)err;
}

// Router + dispatch in two launches: the router kernel with its fused rank step,
// then one scan + scatter kernel.  Outputs are those of hrm_moe_router_topk
// followed by hrm_moe_permute on its topk_idx.
namespace hrm {
namespace {
// From 65 up to this many tokens (E <= 64) the one-wave-per-token router runs
// with the rank step, in blocks of 16 tokens, and the scan + scatter launch
// follows; decode layer at T = 256 (graph replay) 96.5 -> 94.0 us.  Up to 64
// tokens the single-block quad kernel finishes the dispatch in one launch in
// the same time (T = 64: 84.0 us either way); at 8192 tokens and more the wave
// kernel's per-token instruction count makes it the slower one.
constexpr int64_t kWaveRankMaxTokens = 256;
// rank blocks the router + dispatch workspace holds counts for: 16 tokens each
// up to kWaveRankMaxTokens (the wave kernel's blocks), else 64 (the quad kernel's)
inline int64_t router_dispatch_blocks(int64_t T) {
  return T <= kWaveRankMaxTokens ? (T + kWaveRouterMaxTokens - 1) / kWaveRouterMaxTokens : (T + 63) / 64;
}
inline size_t router_dispatch_ws(int64_t T, int E, int k) {
  const size_t r = (size_t)T * (size_t)k;
  return ((sizeof(int32_t) * r + 255) & ~size_t(255)) +
         ((sizeof(int32_t) * (size_t)router_dispatch_blocks(T) * (size_t)(E + 1) + 255) & ~size_t(255)) + 256;
}
}  // namespace
}  // namespace hrm

extern "C" size_t hrm_moe_router_dispatch_workspace_size(int64_t num_tokens, int32_t num_experts, int32_t top_k) {
  if (num_tokens < 0 || num_experts < 1 || num_experts > 128 || top_k < 1 || top_k > 8) return 0;
  return hrm::router_dispatch_ws(num_tokens, num_experts, top_k);
}

namespace hrm {
namespace {

int check_router_dispatch(const void* logits, int logits_dtype, int64_t num_tokens, int32_t num_experts,
                          int32_t top_k, const int64_t* topk_idx, const void* topk_weight, int weight_dtype,
                          const int64_t* tokens_per_expert, const int32_t* expert_offsets,
                          const int32_t* sorted_token_idx, const int32_t* slot_to_row) {
  if (num_tokens < 0 || num_experts < 1 || top_k < 1 || top_k > num_experts) return HRM_MOE_ERR_INVALID;
  if (logits_dtype < HRM_MOE_BF16 || logits_dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (weight_dtype < HRM_MOE_BF16 || weight_dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (num_experts > 128 || top_k > 8 || num_tokens * top_k >= (int64_t(1) << 31)) return HRM_MOE_ERR_UNSUPPORTED;
  if (!tokens_per_expert || !expert_offsets) return HRM_MOE_ERR_INVALID;
  if (num_tokens > 0 && (!logits || !topk_idx || !topk_weight || !sorted_token_idx || !slot_to_row))
    return HRM_MOE_ERR_INVALID;
  return HRM_MOE_OK;
}

// Router + dispatch over a scratch area of at least router_dispatch_ws bytes:
// rank[T*k] and counts[nb][E+1].  The rank step writes every entry of both
// that the scan + scatter launch reads, so the scratch need not start zeroed.
int router_dispatch(const void* logits, int logits_dtype, int64_t num_tokens, int32_t num_experts, int32_t top_k,
                    int32_t norm_topk_prob, float* probs, int64_t* topk_idx, void* topk_weight, int weight_dtype,
                    int64_t* tokens_per_expert, int32_t* expert_offsets, int32_t* sorted_token_idx,
                    int64_t* sort_idx, int32_t* slot_to_row, void* workspace, void* stream) {
  const int E = num_experts, k = top_k;
  const int64_t R = num_tokens * k;
  const int nb = (int)((num_tokens + 63) / 64);  // the quad kernel's rank blocks: 64 tokens
  char* p = static_cast<char*>(workspace);
  int32_t* rank = reinterpret_cast<int32_t*>(p);
  p += (sizeof(int32_t) * (size_t)R + 255) & ~size_t(255);
  int32_t* counts = reinterpret_cast<int32_t*>(p);
  if (num_tokens > 0) {
    // up to 64 tokens: one router block finishes the dispatch itself (no second launch)
    const bool solo = nb == 1;
    const DispatchOut dout{tokens_per_expert, expert_offsets, sorted_token_idx, sort_idx, slot_to_row};
    // up to 16 tokens and 64 experts: one wave per token (HRM_MOE_WAVE_ROUTER=0
    // selects the quad kernel instead; tests compare both)
    if (num_tokens <= kWaveRouterMaxTokens && E <= 64 && config().wave_router)
      return launch_router_dispatch_wave(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx,
                                         topk_weight, weight_dtype, dout, stream);
    if (num_tokens > 64 && num_tokens <= kWaveRankMaxTokens && E <= 64 && config().wave_router) {
      const int st = launch_router_dispatch_wave(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs,
                                                 topk_idx, topk_weight, weight_dtype, dout, stream, rank, counts);
      if (st) return st;
      const int nbw = (int)((num_tokens + kWaveRouterMaxTokens - 1) / kWaveRouterMaxTokens);
      return dispatch_from_ranks(topk_idx, R, E, k, kWaveRouterMaxTokens * k, nbw, rank, counts, tokens_per_expert,
                                 expert_offsets, sorted_token_idx, sort_idx, slot_to_row, stream);
    }
    int st;
    if (E <= 8)
      st = launch_router_rank<8>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx,
                                 topk_weight, weight_dtype, rank, counts, dout, solo, stream);
    else if (E <= 64)
      st = launch_router_rank<64>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx,
                                  topk_weight, weight_dtype, rank, counts, dout, solo, stream);
    else
      st = launch_router_rank<128>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx,
                                   topk_weight, weight_dtype, rank, counts, dout, solo, stream);
    if (st) return st;
    if (solo) return HRM_MOE_OK;
  }
  return dispatch_from_ranks(topk_idx, R, E, k, 64 * k, nb, rank, counts, tokens_per_expert, expert_offsets,
                             sorted_token_idx, sort_idx, slot_to_row, stream);
}

// The no-allocation entry point's scratch: rank[T*k] and counts[nb][E+1] for
// up to 32768 tokens at E <= 128 and k <= 8 (1.25 MiB).  Each GPU the library
// runs on holds its own copy until the process ends.  In host code the array's
// name is not a device address: set-up takes each device's address with
// hipGetSymbolAddress and only that address is passed on.
constexpr size_t kScratchBytes = ((sizeof(int32_t) * 32768 * 8 + 255) & ~size_t(255)) +
                                 ((sizeof(int32_t) * ((32768 + 63) / 64) * (128 + 1) + 255) & ~size_t(255)) + 256;
}  // namespace
__device__ __align__(256) char scratch[kScratchBytes];
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch` (looked up once per device, with the device current).
int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return (int)err;
  if (dev < 0 || dev >= kMaxDevices) return HRM_MOE_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return (int)err;
    if (!p) return HRM_MOE_ERR_INVALID;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HRM_MOE_OK;
}

}  // namespace
}  // namespace hrm

extern "C" int hrm_moe_router_topk_dispatch(const void* logits, int logits_dtype, int64_t num_tokens,
                                            int32_t num_experts, int32_t top_k, int32_t norm_topk_prob, float* probs,
                                            int64_t* topk_idx, void* topk_weight, int weight_dtype,
                                            int64_t* tokens_per_expert, int32_t* expert_offsets,
                                            int32_t* sorted_token_idx, int64_t* sort_idx, int32_t* slot_to_row,
                                            void* workspace, size_t workspace_bytes, void* stream) {
  const int st = hrm::check_router_dispatch(logits, logits_dtype, num_tokens, num_experts, top_k, topk_idx,
                                            topk_weight, weight_dtype, tokens_per_expert, expert_offsets,
                                            sorted_token_idx, slot_to_row);
  if (st) return st;
  if (!workspace || workspace_bytes < hrm::router_dispatch_ws(num_tokens, num_experts, top_k))
    return HRM_MOE_ERR_WORKSPACE;
  return hrm::router_dispatch(logits, logits_dtype, num_tokens, num_experts, top_k, norm_topk_prob, probs, topk_idx,
                              topk_weight, weight_dtype, tokens_per_expert, expert_offsets, sorted_token_idx,
                              sort_idx, slot_to_row, workspace, stream);
}

extern "C" size_t hrm_moe_router_dispatch_noalloc_max_bytes(void) { return hrm::kScratchBytes; }

extern "C" int hrm_moe_router_topk_dispatch_noalloc(const void* logits, int logits_dtype, int64_t num_tokens,
                                                    int32_t num_experts, int32_t top_k, int32_t norm_topk_prob,
                                                    float* probs, int64_t* topk_idx, void* topk_weight,
                                                    int weight_dtype, int64_t* tokens_per_expert,
                                                    int32_t* expert_offsets, int32_t* sorted_token_idx,
                                                    int64_t* sort_idx, int32_t* slot_to_row, void* stream) {
  int st = hrm::check_router_dispatch(logits, logits_dtype, num_tokens, num_experts, top_k, topk_idx, topk_weight,
                                      weight_dtype, tokens_per_expert, expert_offsets, sorted_token_idx, slot_to_row);
  if (st) return st;
  if (hrm::router_dispatch_ws(num_tokens, num_experts, top_k) > hrm::kScratchBytes) return HRM_MOE_ERR_UNSUPPORTED;
  void* ws = nullptr;
  st = hrm::scratch_for_current_device(&ws);
  if (st) return st;
  return hrm::router_dispatch(logits, logits_dtype, num_tokens, num_experts, top_k, norm_topk_prob, probs, topk_idx,
                              topk_weight, weight_dtype, tokens_per_expert, expert_offsets, sorted_token_idx,
                              sort_idx, slot_to_row, ws, stream);
}
