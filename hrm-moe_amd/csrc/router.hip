// Router: fp32 softmax over experts + top-k + renormalisation + cast.
//
// Replaces models/layers.py:606-610 of the reference:
//   probs = F.softmax(logits, -1, dtype=float32)
//   w, idx = torch.topk(probs, k);  w = w / w.sum(-1).clamp_min(1e-12);  w.to(dtype)
//
// Layout: four lanes own one token row; lane q holds the contiguous experts
// [q*C, (q+1)*C) with C = NP2/4 (NP2 = padded expert count).  Cross-lane
// steps use quad DPP moves, so a wave handles 16 rows.
//
// Bit-exactness with torch on the device:
//  * softmax: torch's persistent softmax reduces a row across a wavefront with
//    an xor butterfly.  For padded size NP2 that is the pairwise tree
//    S_i <- S_i + S_{i+o}, o = NP2/2 ... 1.  Levels o >= C pair lanes (xor 2,
//    xor 1); levels o < C stay inside a lane.  exp is expf, and the division is
//    IEEE.  Padding experts hold exp(-inf) = 0, which leaves every partial sum unchanged.
//  * top-k: selection in (value desc, index asc) order, then torch's output
//    order and weight-sum order from topk_order.h.
#include "common.h"
#include "topk_order.h"

namespace hrm {
namespace {

__device__ __forceinline__ float dpp_xor1(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
}
__device__ __forceinline__ float dpp_xor2(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
}
__device__ __forceinline__ uint32_t dpp_xor1u(uint32_t x) { return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ uint32_t dpp_xor2u(uint32_t x) { return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, false); }

__device__ __forceinline__ float load_logit(const void* p, int dt, int64_t i) {
  if (dt == HRM_MOE_BF16) return BF16::to_f(reinterpret_cast<const uint16_t*>(p)[i]);
  if (dt == HRM_MOE_F16) return F16::to_f(reinterpret_cast<const uint16_t*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_weight(void* p, int dt, int64_t i, float w) {
  if (dt == HRM_MOE_BF16) reinterpret_cast<uint16_t*>(p)[i] = BF16::from_f(w);
  else if (dt == HRM_MOE_F16) reinterpret_cast<uint16_t*>(p)[i] = F16::from_f(w);
  else reinterpret_cast<float*>(p)[i] = w;
}

// One selection round over a quad: the largest remaining key, ties to the lower
// expert index; the winner's key is cleared in the lane that holds it.
template <int C>
__device__ __forceinline__ void select_round(uint32_t (&key)[C], int e0, uint32_t& out_key, int& out_idx) {
  uint32_t bk = 0u;
  int be = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    if (key[j] > bk) { bk = key[j]; be = e0 + j; }
  }
  uint32_t ok = dpp_xor1u(bk);
  int oe = (int)dpp_xor1u((uint32_t)be);
  if (ok > bk || (ok == bk && oe < be)) { bk = ok; be = oe; }
  ok = dpp_xor2u(bk);
  oe = (int)dpp_xor2u((uint32_t)be);
  if (ok > bk || (ok == bk && oe < be)) { bk = ok; be = oe; }
#pragma unroll
  for (int j = 0; j < C; ++j) {
    if (e0 + j == be) key[j] = 0u;
  }
  out_key = bk;
  out_idx = be;
}

template <int NP2, int SLOTS>
__global__ __launch_bounds__(256) void router_topk_kernel(const void* __restrict__ logits, int ldt, int64_t T, int E,
                                                          int k, int norm, float* __restrict__ probs,
                                                          int64_t* __restrict__ idx_out, void* __restrict__ w_out,
                                                          int wdt) {
  constexpr int C = NP2 / 4;
  const int q = threadIdx.x & 3;
  const int64_t row = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 2);
  const bool active = row < T;  // inactive lanes still take part in the quad exchanges
  const int e0 = q * C;

  float s[C];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const int e = e0 + j;
    float x = -INFINITY;
    if (active && e < E) x = load_logit(logits, ldt, row * E + e);
    s[j] = x;
    mx = fmaxf(mx, x);
  }
  mx = fmaxf(mx, dpp_xor1(mx));
  mx = fmaxf(mx, dpp_xor2(mx));

  float t[C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    s[j] = expf(s[j] - mx);
    t[j] = s[j];
  }
  // Pairwise tree of the wavefront butterfly: cross-lane levels first.
#pragma unroll
  for (int j = 0; j < C; ++j) t[j] = t[j] + dpp_xor2(t[j]);
#pragma unroll
  for (int j = 0; j < C; ++j) t[j] = t[j] + dpp_xor1(t[j]);
#pragma unroll
  for (int o = C / 2; o > 0; o /= 2) {
#pragma unroll
    for (int i = 0; i < o; ++i) t[i] = t[i] + t[i + o];
  }
  const float total = t[0];

  uint32_t key[C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const float p = s[j] / total;
    const int e = e0 + j;
    const bool ok = active && e < E;
    if (ok && probs != nullptr) probs[row * E + e] = p;
    key[j] = ok ? (__float_as_uint(p) + 1u) : 0u;  // 0 marks "not selectable"
  }

  // Top-k selection in (value desc, index asc) order: k rounds of a quad-wide
  // argmax (ties to the lower expert index), each removing its winner.
  if constexpr (SLOTS <= 8) {
    uint32_t sk[SLOTS];
    int si[SLOTS];
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
      sk[r] = 0u;
      si[r] = 0;
      if (r < k) select_round<C>(key, e0, sk[r], si[r]);
    }
    if (!active) return;
    uint32_t gk[SLOTS];
    int gi[SLOTS];
    torch_topk_order<SLOTS>(sk, si, k, gk, gi);
    float w[SLOTS];
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) w[j] = __uint_as_float(gk[j] - 1u);
    if (norm) {
      float sum = torch_row_sum<SLOTS>(w, k);
      sum = (sum != sum) ? sum : fmaxf(sum, 1e-12f);
#pragma unroll
      for (int j = 0; j < SLOTS; ++j) w[j] = w[j] / sum;
    }
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      if (j < k && (j & 3) == q) {
        idx_out[row * k + j] = (int64_t)gi[j];
        store_weight(w_out, wdt, row * k + j, w[j]);
      }
    }
  } else {
    // k > 8: the ordering runs in loop form on this row's LDS arrays (one lane per row).
    __shared__ uint32_t s_sk[64][SLOTS];
    __shared__ int s_si[64][SLOTS];
    __shared__ uint32_t s_gk[64][SLOTS];
    __shared__ int s_gi[64][SLOTS];
    __shared__ bool s_gv[64][SLOTS];
    const int lr = threadIdx.x >> 2;
    for (int r = 0; r < k; ++r) {
      uint32_t bk;
      int be;
      select_round<C>(key, e0, bk, be);
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

template <int NP2>
int launch_router_np2(const void* logits, int ldt, int64_t T, int E, int k, int norm, float* probs, int64_t* idx,
                      void* w, int wdt, void* stream) {
  dim3 grid((unsigned)((T + 63) / 64)), block(256);
  if (k <= 2) HRM_LAUNCH((router_topk_kernel<NP2, 2>), grid, block, 0, stream, logits, ldt, T, E, k, norm, probs, idx, w, wdt);
  else if (k <= 4) HRM_LAUNCH((router_topk_kernel<NP2, 4>), grid, block, 0, stream, logits, ldt, T, E, k, norm, probs, idx, w, wdt);
  else if (k <= 8) HRM_LAUNCH((router_topk_kernel<NP2, 8>), grid, block, 0, stream, logits, ldt, T, E, k, norm, probs, idx, w, wdt);
  else if constexpr (NP2 >= 16) {
    if (k <= 16) HRM_LAUNCH((router_topk_kernel<NP2, 16>), grid, block, 0, stream, logits, ldt, T, E, k, norm, probs, idx, w, wdt);
    else if constexpr (NP2 >= 32) {
      HRM_LAUNCH((router_topk_kernel<NP2, 32>), grid, block, 0, stream, logits, ldt, T, E, k, norm, probs, idx, w, wdt);
    } else {
      return HRM_MOE_ERR_UNSUPPORTED;
    }
  } else {
    return HRM_MOE_ERR_UNSUPPORTED;
  }
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
  if (num_experts > 128 || top_k > 32) return HRM_MOE_ERR_UNSUPPORTED;
  if (num_tokens == 0) return HRM_MOE_OK;
  if (!logits || !topk_idx || !topk_weight) return HRM_MOE_ERR_INVALID;
  const int E = num_experts, k = top_k;
  if (E <= 8) return hrm::launch_router_np2<8>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx, topk_weight, weight_dtype, stream);
  if (E <= 64) return hrm::launch_router_np2<64>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx, topk_weight, weight_dtype, stream);
  return hrm::launch_router_np2<128>(logits, logits_dtype, num_tokens, E, k, norm_topk_prob, probs, topk_idx, topk_weight, weight_dtype, stream);
}
