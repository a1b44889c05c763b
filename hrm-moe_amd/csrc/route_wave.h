// One token routed by one wave: fp32 softmax over E <= 64 experts (lane e
// holds expert e), top-k in torch's order, optional renormalisation.
//
// Shared by the decode-size router (router.hip, router_dispatch_wave_kernel)
// and the one-launch decode layer (decode.hip), so both produce the same bits.
// Replaces models/layers.py:606-610 of the reference for one row:
//   probs = F.softmax(logits, -1, dtype=float32)
//   w, idx = torch.topk(probs, k);  w = w / w.sum(-1).clamp_min(1e-12)
//
// Bit-exactness with torch on the device:
//  * softmax: torch's persistent softmax over a row of up to 64 values reduces
//    across the wave with an xor butterfly at distances 32 ... 1 (maximum,
//    then the sum of exp(x - max)); exp is expf and the division is IEEE.
//    The same sums are formed here with cheaper lane moves (route_token_select).
//    Lanes past E hold -inf, so exp gives 0 and the sums are unchanged.
//  * top-k: the rank of each lane's (p, 63 - lane) pair among the wave's 64
//    unique pairs selects the k largest in (value desc, index asc) order.
//    torch's output order differs from plain descending order only when two
//    selected keys are equal, so the ordering network of topk_order.h runs
//    only then: a wave-uniform branch.
//  * weight sum in torch's order (topk_order.h), IEEE division.
#pragma once
#include "common.h"
#include "topk_order.h"

namespace hrm {

// Value of the lane at distance D inside the row (D = 1, 2: xor; D = 4, 8:
// rotation within a row of 16 lanes).
template <int D>
__device__ __forceinline__ uint32_t xlane(uint32_t x) {
  constexpr int ctrl = D == 1 ? 0xB1 : D == 2 ? 0x4E : D == 4 ? 0x124 : 0x128;  // quad_perm / row_ror
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, ctrl, 0xF, 0xF, false);
}
template <int D>
__device__ __forceinline__ float xlanef(float x) {
  return __uint_as_float(xlane<D>(__float_as_uint(x)));
}
// Value of lane ^ 16 (within each half of the wave), by swizzle: and-mask 31,
// or-mask 0, xor-mask 16.
__device__ __forceinline__ float xor16f(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
}

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

// First half of routing token t (row t of logits [*, E]) with the calling
// wave: softmax and selection.  `active` false for a wave without a token (it
// still passes both barriers).  Every wave of the workgroup must call this
// together: it holds two workgroup barriers.  s_ck[64], s_sk[SLOTS],
// s_si[SLOTS]: this wave's LDS scratch, left holding the k selected (key,
// expert) pairs in (key desc, index asc) order for route_token_finish.
// probs (may be null): the wave writes the token's E probabilities.
// s_sel (may be null): receives the set of selected experts as a bit mask,
// visible to the whole workgroup when this returns.
template <int SLOTS, bool KFIX>
__device__ __forceinline__ void route_token_select(const void* __restrict__ logits, int ldt, int64_t t, bool active,
                                                   int E, int k_rt, float* __restrict__ probs, uint64_t* s_ck,
                                                   uint32_t* s_sk, int32_t* s_si, uint64_t* s_sel) {
  static_assert(SLOTS <= 8, "k <= 8");
  const int k = KFIX ? SLOTS : k_rt;
  const int lane = threadIdx.x & 63;
  const bool ok = active && lane < E;
  const float x = ok ? load_logit(logits, ldt, t * E + lane) : -INFINITY;
  // xor butterfly at distances 32 ... 1 (torch's order): a permute for 32, a
  // swizzle for 16 (lane ^ 16 within each half), then DPP row moves.  Rotation
  // by 8 within a row of 16 is xor 8; at the distance-4 step every lane's value
  // depends only on its index mod 8, so rotation by 4 reads the same value as
  // xor 4; the sums are the butterfly's, bit for bit (and any order gives the
  // same maximum).  Six permutes through LDS, each waited for before the next,
  // took about 0.4 us of the one-launch decode kernel.
  float mx = x;
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  mx = fmaxf(mx, xor16f(mx));
  mx = fmaxf(mx, xlanef<8>(mx));
  mx = fmaxf(mx, xlanef<4>(mx));
  mx = fmaxf(mx, xlanef<2>(mx));
  mx = fmaxf(mx, xlanef<1>(mx));
  const float s = expf(x - mx);
  float total = s;
  total = total + __shfl_xor(total, 32, 64);
  total = total + xor16f(total);
  total = total + xlanef<8>(total);
  total = total + xlanef<4>(total);
  total = total + xlanef<2>(total);
  total = total + xlanef<1>(total);
  const float p = s / total;
  if (ok && probs != nullptr) probs[t * E + lane] = p;
  const uint32_t key = ok ? (__float_as_uint(p) + 1u) : 0u;  // 0 marks "not selectable"

  // rank among the wave's 64 unique (key, 63 - lane) pairs
  const uint64_t ck = ((uint64_t)key << 32) | (uint32_t)(63 - lane);
  s_ck[lane] = ck;
  __syncthreads();
  int rank = 0;
#pragma unroll
  for (int j = 0; j < 64; ++j) rank += s_ck[j] > ck ? 1 : 0;
  if (rank < k) {
    s_sk[rank] = key;
    s_si[rank] = key != 0u ? lane : 0x7fffffff;
  }
  const uint64_t sel = __ballot(rank < k && key != 0u);
  if (s_sel != nullptr && lane == 0) *s_sel = sel;
  __syncthreads();
}

// Second half, no barriers: torch's output order and the weights of the
// selected pairs.  Result, in lanes j < k of an active wave: slot j's expert
// (my_i) and weight (my_w, fp32 before the cast to the weight dtype).  A wave
// without a token returns my_i = 0, my_w = 0 at once: its keys are all equal
// (zero), so it would take the tie branch and run the whole ordering network
// (the one-launch decode kernel at one token waited 3.3 of its 12 us for that).
template <int SLOTS, bool KFIX>
__device__ __forceinline__ void route_token_finish(bool active, int k_rt, int norm, const uint32_t* s_sk,
                                                   const int32_t* s_si, int& my_i, float& my_w) {
  constexpr int KC = KFIX ? SLOTS : 0;
  const int k = KFIX ? SLOTS : k_rt;
  const int lane = threadIdx.x & 63;
  my_i = 0;
  my_w = 0.0f;
  if (!active) return;
  uint32_t sk[SLOTS];
  int si[SLOTS];
#pragma unroll
  for (int r = 0; r < SLOTS; ++r) {
    sk[r] = r < k ? s_sk[r] : 0u;
    si[r] = r < k ? s_si[r] : 0;
  }
  bool tie = false;
#pragma unroll
  for (int r = 0; r + 1 < SLOTS; ++r) tie = tie || (r + 1 < k && sk[r] == sk[r + 1]);
  uint32_t gk[SLOTS];
  int gi[SLOTS];
  if (__builtin_amdgcn_readfirstlane((int)tie)) {
    torch_topk_order<SLOTS, KC>(sk, si, k, gk, gi);
  } else {
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
      gk[r] = sk[r];
      gi[r] = si[r];
    }
  }
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
    my_i = lane == j ? gi[j] : my_i;
    my_w = lane == j ? w[j] : my_w;
  }
}

// Both halves: routes token t with the calling wave (all waves of the
// workgroup call it together; it holds two workgroup barriers).
template <int SLOTS, bool KFIX>
__device__ __forceinline__ void route_token_wave(const void* __restrict__ logits, int ldt, int64_t t, bool active,
                                                 int E, int k_rt, int norm, float* __restrict__ probs,
                                                 uint64_t* s_ck, uint32_t* s_sk, int32_t* s_si, int& my_i,
                                                 float& my_w) {
  route_token_select<SLOTS, KFIX>(logits, ldt, t, active, E, k_rt, probs, s_ck, s_sk, s_si, nullptr);
  route_token_finish<SLOTS, KFIX>(active, k_rt, norm, s_sk, s_si, my_i, my_w);
}

}  // namespace hrm
