// Dispatch: stable counting sort of the T*k routed slots by expert.
//
// Replaces models/layers.py:312-322 of the reference (flat expert ids,
// repeat_interleave token ids, torch.sort(stable=True), index_select, bincount)
// with three deterministic kernels and no host synchronisation:
//   1. rank:    blocks of SB (32..512) consecutive slots.  Each slot sets its bit in an
//               LDS bitmask row of its bucket.  A slot's rank in the block is the
//               popcount of the bucket's bits below it (OR is order-free, so
//               the ranks do not depend on atomic ordering).
//   2. scan:    one workgroup turns the per-block bucket counts into bucket
//               offsets and per-block bases, and writes tokens_per_expert and
//               expert_offsets.
//   3. scatter: row = base[block][bucket] + rank; writes sorted_token_idx,
//               sort_idx and slot_to_row.
// Buckets are the E experts plus one trailing bucket for ids outside [0, E),
// whose rows land after every valid row.
#include "common.h"

namespace hrm {
namespace {

constexpr int kPermThreads = 256;
constexpr int kMaxExperts = 1024;

// Slots per rank block: keeps (E+1) * SB / 8 bytes of bitmask (and as much
// again of prefix counts) under 17 KB each, so a block needs at most 34 KB of LDS.
// Smaller blocks give more of them (parallelism) at the cost of a longer scan.
// 512 slots (one router block of 64 tokens at top-8) when that fits.
inline int slots_per_block(int E) {
  int sb = 512;
  while (sb > 32 && (int64_t)(E + 1) * sb / 8 > 17 * 1024) sb /= 2;
  return sb;
}

struct PermWs {
  int32_t* rank;    // [R]
  int32_t* counts;  // [nb][E+1]
  int32_t* base;    // [nb][E+1]
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline PermWs carve(void* ws, int64_t R, int nb, int E) {
  char* p = static_cast<char*>(ws);
  PermWs w;
  w.rank = reinterpret_cast<int32_t*>(p);
  p += align256(sizeof(int32_t) * (size_t)R);
  w.counts = reinterpret_cast<int32_t*>(p);
  p += align256(sizeof(int32_t) * (size_t)nb * (E + 1));
  w.base = reinterpret_cast<int32_t*>(p);
  return w;
}

inline size_t ws_bytes(int64_t R, int nb, int E) {
  const size_t n = align256(sizeof(int32_t) * (size_t)R) + 2 * align256(sizeof(int32_t) * (size_t)nb * (E + 1));
  return n < 256 ? 256 : n;
}

__device__ __forceinline__ int bucket_of(int64_t e, int E) { return (e >= 0 && e < E) ? (int)e : E; }

__global__ __launch_bounds__(kPermThreads) void permute_rank_kernel(const int64_t* __restrict__ idx, int64_t R, int E,
                                                                    int SB, int32_t* __restrict__ rank,
                                                                    int32_t* __restrict__ counts) {
  extern __shared__ uint32_t smem[];
  const int words = SB / 32;
  const int nbk = E + 1;
  uint32_t* mask = smem;                            // [nbk][words]
  uint32_t* pref = smem + (size_t)nbk * words;      // [nbk][words]
  const int64_t s0 = (int64_t)blockIdx.x * SB;
  const int per = SB >= kPermThreads ? SB / kPermThreads : 1;  // consecutive slots per thread
  for (int i = threadIdx.x; i < nbk * words; i += kPermThreads) mask[i] = 0u;
  __syncthreads();
  for (int i = 0; i < per; ++i) {
    const int ls = threadIdx.x * per + i;
    const int64_t s = s0 + ls;
    if (ls < SB && s < R) {
      const int b = bucket_of(idx[s], E);
      atomicOr(&mask[b * words + (ls >> 5)], 1u << (ls & 31));
    }
  }
  __syncthreads();
  for (int b = threadIdx.x; b < nbk; b += kPermThreads) {
    uint32_t run = 0;
    for (int w = 0; w < words; ++w) {
      pref[b * words + w] = run;
      run += __popc(mask[b * words + w]);
    }
    counts[(int64_t)blockIdx.x * nbk + b] = (int32_t)run;
  }
  __syncthreads();
  for (int i = 0; i < per; ++i) {
    const int ls = threadIdx.x * per + i;
    const int64_t s = s0 + ls;
    if (ls < SB && s < R) {
      const int b = bucket_of(idx[s], E);
      const uint32_t below = mask[b * words + (ls >> 5)] & ((1u << (ls & 31)) - 1u);
      rank[s] = (int32_t)(pref[b * words + (ls >> 5)] + __popc(below));
    }
  }
}

// Inclusive scan across the 64 lanes of a wave.
__device__ __forceinline__ int32_t wave_incl_scan(int32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

// One workgroup of 1024 threads.  The per-block counts form a [nb][E+1]
// matrix.  With E + 1 <= 512 buckets, G = 1024 / (E+1) groups of E+1
// consecutive threads each own a contiguous range of blocks, so a group reads
// and writes whole matrix rows (coalesced).  Each thread sums its bucket over
// its range; one thread per bucket scans the G partials; wave 0 scans the
// bucket totals; each thread then writes the bases of its range.  With more
// buckets each thread walks whole buckets.
__global__ __launch_bounds__(1024) void permute_scan_kernel(const int32_t* __restrict__ counts, int nb, int E,
                                                            int32_t* __restrict__ base,
                                                            int64_t* __restrict__ tokens_per_expert,
                                                            int32_t* __restrict__ expert_offsets) {
  __shared__ int32_t part[1024];
  __shared__ int32_t tot[kMaxExperts + 2];
  __shared__ int32_t off[kMaxExperts + 2];
  const int nbk = E + 1;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const bool split = nbk <= 512;
  const int G = split ? 1024 / nbk : 1;
  const int per = (nb + G - 1) / G;
  const int b = tid % nbk, g = tid / nbk;
  const bool on = split && g < G;
  const int j0 = g * per, j1 = min(nb, j0 + per);
  if (split) {
    int32_t sum = 0;
    if (on) {
#pragma unroll 8
      for (int j = j0; j < j1; ++j) sum += counts[(int64_t)j * nbk + b];
    }
    part[tid] = sum;
    __syncthreads();
    if (on && g == 0) {
      int32_t run = 0;
      for (int u = 0; u < G; ++u) {
        const int32_t v = part[u * nbk + b];
        part[u * nbk + b] = run;
        run += v;
      }
      tot[b] = run;
    }
  } else {
    for (int bb = tid; bb < nbk; bb += 1024) {
      int32_t t = 0;
      for (int j = 0; j < nb; ++j) t += counts[(int64_t)j * nbk + bb];
      tot[bb] = t;
    }
  }
  __syncthreads();
  if (tid < 64) {  // exclusive scan of the bucket totals, 64 at a time
    int32_t carry = 0;
    for (int c = 0; c < nbk; c += 64) {
      const int bb = c + lane;
      const int32_t v = bb < nbk ? tot[bb] : 0;
      const int32_t incl = wave_incl_scan(v, lane);
      if (bb < nbk) off[bb] = carry + incl - v;
      carry += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
  if (split) {
    if (on) {
      int32_t run = off[b] + part[tid];
#pragma unroll 8
      for (int j = j0; j < j1; ++j) {
        const int32_t c = counts[(int64_t)j * nbk + b];
        base[(int64_t)j * nbk + b] = run;
        run += c;
      }
    }
  } else {
    for (int bb = tid; bb < nbk; bb += 1024) {
      int32_t run = off[bb];
      for (int j = 0; j < nb; ++j) {
        base[(int64_t)j * nbk + bb] = run;
        run += counts[(int64_t)j * nbk + bb];
      }
    }
  }
  for (int bb = tid; bb < nbk; bb += 1024) {
    if (bb < E) tokens_per_expert[bb] = (int64_t)tot[bb];
    expert_offsets[bb] = off[bb];  // expert_offsets[E] = start of the dropped rows
  }
}

__global__ __launch_bounds__(256) void permute_scatter_kernel(const int64_t* __restrict__ idx, int64_t R, int E, int k,
                                                              int SB, const int32_t* __restrict__ rank,
                                                              const int32_t* __restrict__ base,
                                                              int32_t* __restrict__ sorted_token_idx,
                                                              int64_t* __restrict__ sort_idx,
                                                              int32_t* __restrict__ slot_to_row) {
  const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= R) return;
  const int b = bucket_of(idx[s], E);
  const int32_t row = base[(s / SB) * (E + 1) + b] + rank[s];
  sorted_token_idx[row] = (int32_t)(s / k);
  if (sort_idx) sort_idx[row] = s;
  slot_to_row[s] = row;
}

// Scan and scatter in one launch, after a rank step that wrote rank[R] and
// counts[nb][E+1] for rank blocks of SB slots (the router kernel's fused rank
// step).  Workgroup g handles rank blocks [g*G, g*G+G).  It recomputes, from
// the whole counts matrix, every bucket's total and its own blocks' prefix:
// workgroups never wait on one another, and each reads nb*(E+1) ints.
// Workgroup 0 also writes tokens_per_expert and expert_offsets.  Rows and
// their order are those of the three-kernel path.  Needs E + 1 <= 512.
constexpr int kScatterChunk = 16;  // rank blocks scattered together
__global__ __launch_bounds__(1024) void permute_scan_scatter_kernel(
    const int64_t* __restrict__ idx, int64_t R, int E, int k, int SB, int nb, int G, const int32_t* __restrict__ rank,
    const int32_t* __restrict__ counts, int64_t* __restrict__ tokens_per_expert, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ sorted_token_idx, int64_t* __restrict__ sort_idx, int32_t* __restrict__ slot_to_row) {
  __shared__ int32_t part[1024];
  __shared__ int32_t part_pre[1024];
  __shared__ int32_t tot[513], off[513], base[513];
  __shared__ int32_t cbase[kScatterChunk][513];
  const int nbk = E + 1;
  const int tid = threadIdx.x, lane = tid & 63;
  const int rb0 = blockIdx.x * G, rb1 = min(nb, rb0 + G);
  const int NG = 1024 / nbk;  // groups of nbk threads, each summing a range of rows
  const int per = (nb + NG - 1) / NG;
  const int b = tid % nbk, g = tid / nbk;
  const bool on = g < NG;
  int32_t all = 0, pre = 0;
  if (on) {
    const int j0 = g * per, j1 = min(nb, j0 + per);
#pragma unroll 8
    for (int j = j0; j < j1; ++j) {
      const int32_t c = counts[(int64_t)j * nbk + b];
      all += c;
      pre += j < rb0 ? c : 0;
    }
  }
  part[tid] = all;
  part_pre[tid] = pre;
  __syncthreads();
  if (on && g == 0) {
    int32_t t = 0, p = 0;
    for (int u = 0; u < NG; ++u) {
      t += part[u * nbk + b];
      p += part_pre[u * nbk + b];
    }
    tot[b] = t;
    base[b] = p;
  }
  __syncthreads();
  if (tid < 64) {  // exclusive scan of the bucket totals, 64 at a time
    int32_t carry = 0;
    for (int c = 0; c < nbk; c += 64) {
      const int bb = c + lane;
      const int32_t v = bb < nbk ? tot[bb] : 0;
      const int32_t incl = wave_incl_scan(v, lane);
      if (bb < nbk) off[bb] = carry + incl - v;
      carry += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
  if (tid < nbk) {
    base[tid] += off[tid];
    if (blockIdx.x == 0) {
      if (tid < E) tokens_per_expert[tid] = (int64_t)tot[tid];
      expert_offsets[tid] = off[tid];  // expert_offsets[E] = start of the dropped rows
    }
  }
  __syncthreads();
  // Scatter, kScatterChunk rank blocks at a time: first each bucket's start
  // row in every rank block of the chunk (a running sum over the chunk's
  // counts), then every slot of the chunk at once.
  for (int c0 = rb0; c0 < rb1; c0 += kScatterChunk) {
    const int n = min(kScatterChunk, rb1 - c0);
    if (tid < nbk) {
      int32_t cnt[kScatterChunk];
#pragma unroll
      for (int i = 0; i < kScatterChunk; ++i) cnt[i] = i < n ? counts[(int64_t)(c0 + i) * nbk + tid] : 0;
      int32_t run = base[tid];
#pragma unroll
      for (int i = 0; i < kScatterChunk; ++i) {
        cbase[i][tid] = run;
        run += cnt[i];
      }
      base[tid] = run;
    }
    __syncthreads();
    for (int it = tid; it < n * SB; it += 1024) {
      const int i = it / SB;
      const int64_t sl = (int64_t)c0 * SB + it;
      if (sl < R) {
        const int bk = bucket_of(idx[sl], E);
        const int32_t row = cbase[i][bk] + rank[sl];
        sorted_token_idx[row] = (int32_t)(sl / k);
        if (sort_idx) sort_idx[row] = sl;
        slot_to_row[sl] = row;
      }
    }
    __syncthreads();
  }
}

}  // namespace

// Second dispatch stage after a rank step that wrote rank[R] and counts[nb][E+1]
// with SB slots per rank block (used by the router's fused entry point).
int dispatch_from_ranks(const int64_t* topk_idx, int64_t R, int E, int k, int SB, int nb, const int32_t* rank,
                        const int32_t* counts, int64_t* tokens_per_expert, int32_t* expert_offsets,
                        int32_t* sorted_token_idx, int64_t* sort_idx, int32_t* slot_to_row, void* stream) {
  if (E + 1 > 512) return HRM_MOE_ERR_UNSUPPORTED;
  // about 256 workgroups: each re-reads the whole counts matrix for its prefix,
  // but more of them scatter in parallel (L: 9.5 -> 6.2 us against 32 workgroups;
  // T = 32768, E = 128: 17.6 -> 10.4 us)
  const int G = nb <= 256 ? 1 : (nb + 255) / 256;
  const int blocks = nb == 0 ? 1 : (nb + G - 1) / G;
  HRM_LAUNCH(permute_scan_scatter_kernel, dim3(blocks), dim3(1024), 0, stream, topk_idx, R, E, k, SB, nb, G, rank,
             counts, tokens_per_expert, expert_offsets, sorted_token_idx, sort_idx, slot_to_row);
  return HRM_MOE_OK;
}

}  // namespace hrm

extern "C" size_t hrm_moe_permute_workspace_size(int64_t num_tokens, int32_t num_experts, int32_t top_k) {
  if (num_tokens < 0 || num_experts < 1 || num_experts > hrm::kMaxExperts || top_k < 1) return 0;
  const int64_t R = num_tokens * top_k;
  const int sb = hrm::slots_per_block(num_experts);
  const int nb = (int)((R + sb - 1) / sb);
  return hrm::ws_bytes(R, nb, num_experts);
}

extern "C" int hrm_moe_permute(const int64_t* topk_idx, int64_t num_tokens, int32_t num_experts, int32_t top_k,
                               int64_t* tokens_per_expert, int32_t* expert_offsets, int32_t* sorted_token_idx,
                               int64_t* sort_idx, int32_t* slot_to_row, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (num_tokens < 0 || num_experts < 1 || top_k < 1) return HRM_MOE_ERR_INVALID;
  if (num_experts > hrm::kMaxExperts) return HRM_MOE_ERR_UNSUPPORTED;
  const int64_t R = num_tokens * top_k;
  if (R >= (int64_t(1) << 31)) return HRM_MOE_ERR_UNSUPPORTED;
  if (!tokens_per_expert || !expert_offsets) return HRM_MOE_ERR_INVALID;
  if (R > 0 && (!topk_idx || !sorted_token_idx || !slot_to_row)) return HRM_MOE_ERR_INVALID;
  const int E = num_experts;
  const int sb = hrm::slots_per_block(E);
  const int nb = (int)((R + sb - 1) / sb);
  const size_t need = hrm::ws_bytes(R, nb, E);
  if (!workspace || workspace_bytes < need) return HRM_MOE_ERR_WORKSPACE;
  hrm::PermWs w = hrm::carve(workspace, R, nb, E);
  if (nb > 0) {
    const size_t lds = sizeof(uint32_t) * 2 * (size_t)(E + 1) * (sb / 32);
    HRM_LAUNCH(hrm::permute_rank_kernel, dim3(nb), dim3(hrm::kPermThreads), lds, stream, topk_idx, R, E, sb, w.rank,
               w.counts);
  }
  HRM_LAUNCH(hrm::permute_scan_kernel, dim3(1), dim3(1024), 0, stream, w.counts, nb, E, w.base, tokens_per_expert,
             expert_offsets);
  if (R > 0) {
    HRM_LAUNCH(hrm::permute_scatter_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, stream, topk_idx, R, E,
               top_k, sb, w.rank, w.base, sorted_token_idx, sort_idx, slot_to_row);
  }
  return HRM_MOE_OK;
}
