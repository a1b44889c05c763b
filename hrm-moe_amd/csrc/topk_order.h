// Ordering of the k selected experts exactly as torch.topk returns them on ROCm.
//
// Shared by the router kernel and a host-compiled test library (hostcheck.cpp), so
// the CPU test suite exercises the same code the kernel runs.
//
// torch.topk (sorted) takes every value above the k-th largest in ascending
// index order, then values equal to it in ascending index order.  It then
// orders the k pairs with a descending bitonic network on 32 slots.  That
// network builds runs of size 2..16, then does one final merge.  A
// compare-exchange of slots (a, b) in direction d computes
//   swap = (key[a] > key[b] && valid[a]) || !valid[b]
// and exchanges when swap == d.  Equal keys are therefore exchanged whenever
// d is false.  Slots past the first SLOTS (SLOTS = next power of two >= k)
// hold invalid entries that never move into the first SLOTS, so the network
// is evaluated on SLOTS slots.  The build stages for sizes above SLOTS, and
// the final merge, act on those slots as merges with direction false.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define HRM_HD __host__ __device__ __forceinline__
#else
#define HRM_HD inline
#endif

namespace hrm {

// Written with selects only, so a wave whose rows take different branches
// does not split: every lane runs the same straight-line code.
HRM_HD void bitonic_ce(uint32_t& ka, int& ia, bool& va, uint32_t& kb, int& ib, bool& vb, bool dir) {
  const bool x = ((((ka > kb) && va) || !vb)) == dir;
  const uint32_t ka2 = x ? kb : ka, kb2 = x ? ka : kb;
  const int ia2 = x ? ib : ia, ib2 = x ? ia : ib;
  const bool va2 = x ? vb : va, vb2 = x ? va : vb;
  ka = ka2;
  kb = kb2;
  ia = ia2;
  ib = ib2;
  va = va2;
  vb = vb2;
}

// Number of direction-false merges over the first SLOTS slots: the build
// stages of sizes 2*SLOTS..16 plus the final merge.
template <int SLOTS>
struct TopkMerges {
  static constexpr int value = (SLOTS >= 16 ? 0 : (SLOTS >= 8 ? 1 : (SLOTS >= 4 ? 2 : 3))) + 1;
};

// The same compare-exchange with validity carried by the key: valid keys are
// >= 1 and invalid slots hold 0.  Then ((ka > kb) && va) || !vb equals
// (ka > kb) || (kb == 0) in all four valid/invalid cases, and no per-lane
// flag arrays are needed (registers only).
HRM_HD void bitonic_ce_k(uint32_t& ka, int& ia, uint32_t& kb, int& ib, bool dir) {
  const bool x = ((ka > kb) || (kb == 0u)) == dir;
  const uint32_t ka2 = x ? kb : ka, kb2 = x ? ka : kb;
  const int ia2 = x ? ib : ia, ib2 = x ? ia : ib;
  ka = ka2;
  kb = kb2;
  ia = ia2;
  ib = ib2;
}

// torch's network over SLOTS slots; keys >= 1 are valid, 0 marks an empty slot.
template <int SLOTS>
HRM_HD void torch_topk_network(uint32_t (&key)[SLOTS], int (&idx)[SLOTS]) {
  constexpr int kBuildMax = SLOTS < 16 ? SLOTS : 16;
#pragma unroll
  for (int size = 2; size <= kBuildMax; size *= 2) {
#pragma unroll
    for (int stride = size / 2; stride > 0; stride /= 2) {
#pragma unroll
      for (int t = 0; t < SLOTS / 2; ++t) {
        const int a = 2 * t - (t & (stride - 1));
        bitonic_ce_k(key[a], idx[a], key[a + stride], idx[a + stride], (t & (size / 2)) != 0);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < TopkMerges<SLOTS>::value; ++m) {
#pragma unroll
    for (int stride = SLOTS / 2; stride > 0; stride /= 2) {
#pragma unroll
      for (int t = 0; t < SLOTS / 2; ++t) {
        const int a = 2 * t - (t & (stride - 1));
        bitonic_ce_k(key[a], idx[a], key[a + stride], idx[a + stride], false);
      }
    }
  }
}

// From the k selected (key, index) pairs in (key desc, index asc) order
// (sk, si; entries >= k unused) to torch's output order (gk, gi).  Keys are
// order-preserving uint32 images of the probabilities, offset by one so that
// every selected key is >= 1.
// KC > 0 fixes k = KC at compile time (the k argument is then ignored), which
// removes every k-dependent predicate from the unrolled code.
template <int SLOTS, int KC = 0>
HRM_HD void torch_topk_order(const uint32_t (&sk)[SLOTS], const int (&si)[SLOTS], int k_rt, uint32_t (&gk)[SLOTS],
                             int (&gi)[SLOTS]) {
  static_assert(KC >= 0 && KC <= SLOTS, "compile-time k");
  const int k = KC > 0 ? KC : k_rt;
  uint32_t kth = 0u;
#pragma unroll
  for (int r = 0; r < SLOTS; ++r) kth = (r == k - 1) ? sk[r] : kth;
  int n_greater = 0;
#pragma unroll
  for (int r = 0; r < SLOTS; ++r) n_greater += (r < k && sk[r] > kth) ? 1 : 0;
  int pos[SLOTS];
#pragma unroll
  for (int r = 0; r < SLOTS; ++r) {
    const bool gr = sk[r] > kth;
    int p = gr ? 0 : n_greater;
#pragma unroll
    for (int u = 0; u < SLOTS; ++u) p += (u < k && ((sk[u] > kth) == gr) && si[u] < si[r]) ? 1 : 0;
    pos[r] = (r < k) ? p : SLOTS;
  }
#pragma unroll
  for (int p = 0; p < SLOTS; ++p) {
    uint32_t kk = 0u;  // positions >= k stay 0: empty slots
    int ii = 0;
#pragma unroll
    for (int r = 0; r < SLOTS; ++r) {
      const bool hit = pos[r] == p;
      kk = hit ? sk[r] : kk;
      ii = hit ? si[r] : ii;
    }
    gk[p] = kk;
    gi[p] = ii;
  }
  torch_topk_network<SLOTS>(gk, gi);
}

// Sum of the k weights in the order torch's reduction kernel uses for a
// [rows, k] tensor reduced over k: block_width = last_pow2(k) threads, thread
// x accumulating elements x, x + bw, ... in order, then a shfl_down tree.
template <int SLOTS, int KC = 0>
HRM_HD float torch_row_sum(const float (&w)[SLOTS], int k_rt) {
  static_assert(KC >= 0 && KC <= SLOTS, "compile-time k");
  const int k = KC > 0 ? KC : k_rt;
  int bw = 1;  // last power of two <= k
#pragma unroll
  for (int b = 2; b <= SLOTS; b *= 2) bw = (b <= k) ? b : bw;
  float part[SLOTS];
#pragma unroll
  for (int x = 0; x < SLOTS; ++x) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) acc = (j < k && j >= x && ((j - x) & (bw - 1)) == 0) ? acc + w[j] : acc;
    part[x] = acc;
  }
#pragma unroll
  for (int o = 1; o < SLOTS; o *= 2) {
#pragma unroll
    for (int x = 0; x + o < SLOTS; x += 2 * o) part[x] = (o < bw) ? part[x] + part[x + o] : part[x];
  }
  return part[0];
}

// Loop form of torch_topk_order + torch_row_sum on caller-provided arrays of
// `slots` entries (slots = next power of two >= k, 2..32).  The router runs this
// form for k > 8 on per-row LDS arrays, which keeps the large networks out of
// registers.
HRM_HD void torch_topk_order_mem(const uint32_t* sk, const int* si, int k, int slots, uint32_t* gk, int* gi,
                                 bool* gv) {
  uint32_t kth = sk[k - 1];
  int n_greater = 0;
  for (int r = 0; r < k; ++r) n_greater += sk[r] > kth ? 1 : 0;
  for (int p = 0; p < slots; ++p) {
    gk[p] = 0u;
    gi[p] = 0;
    gv[p] = p < k;
  }
  for (int r = 0; r < k; ++r) {
    const bool gr = sk[r] > kth;
    int p = gr ? 0 : n_greater;
    for (int u = 0; u < k; ++u)
      if (((sk[u] > kth) == gr) && si[u] < si[r]) ++p;
    gk[p] = sk[r];
    gi[p] = si[r];
  }
  const int build_max = slots < 16 ? slots : 16;
  for (int size = 2; size <= build_max; size *= 2)
    for (int stride = size / 2; stride > 0; stride /= 2)
      for (int t = 0; t < slots / 2; ++t) {
        const int a = 2 * t - (t & (stride - 1));
        bitonic_ce(gk[a], gi[a], gv[a], gk[a + stride], gi[a + stride], gv[a + stride], (t & (size / 2)) != 0);
      }
  const int merges = (slots >= 16 ? 0 : (slots >= 8 ? 1 : (slots >= 4 ? 2 : 3))) + 1;
  for (int m = 0; m < merges; ++m)
    for (int stride = slots / 2; stride > 0; stride /= 2)
      for (int t = 0; t < slots / 2; ++t) {
        const int a = 2 * t - (t & (stride - 1));
        bitonic_ce(gk[a], gi[a], gv[a], gk[a + stride], gi[a + stride], gv[a + stride], false);
      }
}

HRM_HD float torch_row_sum_mem(const float* w, int k) {
  int bw = 1;
  while (bw * 2 <= k) bw *= 2;
  float part[32];
  for (int x = 0; x < bw; ++x) {
    float acc = 0.0f;
    for (int j = x; j < k; j += bw) acc = acc + w[j];
    part[x] = acc;
  }
  for (int o = 1; o < bw; o *= 2)
    for (int x = 0; x + o < bw; x += 2 * o) part[x] = part[x] + part[x + o];
  return part[0];
}

}  // namespace hrm
