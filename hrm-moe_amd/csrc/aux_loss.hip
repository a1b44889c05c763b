// Auxiliary load-balancing loss of the router and the layer's expert counts.
//
// Replaces models/layers.py:163-170 (load_balancing_loss_func) and :619-632
// (the counts appended to the MoE context) of the reference, whose torch form
// is about nine small kernels per layer:
//   f[e]    = tokens_per_expert[e] * (1 / T)           (fp32; torch divides a tensor
//                                                       by a scalar as a product with its reciprocal)
//   mean[e] = sum_t probs[t, e] * (1 / T)              (fp32, the column mean)
//   aux     = (sum_e f[e] * mean[e]) * E
//   counts  = tokens_per_expert as fp32
// Here it is two launches: per-block column sums of probs, then one block that
// adds the block sums and finishes.  Both reductions run in a fixed order, so
// every run gives the same bits (they differ from torch's reduction order by
// rounding only).
// The backward is the same for every token: d probs[t, e] = ((g * E) * f[e]) * (1 / T),
// torch's order for this expression, one row of E values that the router
// backward reads with a zero row stride.
#include "common.h"

namespace hrm {
namespace {

constexpr int kAuxThreads = 256;
constexpr int kAuxMaxBlocks = 128;
constexpr int kAuxMaxExperts = 1024;

inline int aux_blocks(int64_t T) {
  const int64_t b = (T + 127) / 128;
  return (int)(b < kAuxMaxBlocks ? (b < 1 ? 1 : b) : kAuxMaxBlocks);
}

// Column sums of a row-major [rows][E] fp32 array over rows [r0, r1), for the
// column chunk [c0, c0 + width): G = 256 / width thread groups take rows
// g, g + G, ... (ascending, 8 loads in flight per thread), then thread c of
// the chunk adds the G group sums in group order.  Returns the chunk column's
// sum in threads tid < width.  Every thread of the block must call it.
__device__ __forceinline__ float block_colsum(const float* __restrict__ a, int64_t r0, int64_t r1, int E, int c0,
                                              int width, float* s_part) {
  const int tid = threadIdx.x;
  const int groups = kAuxThreads / width;
  const int g = tid / width, e = c0 + tid % width;
  float acc = 0.0f;
  if (g < groups) {
    int64_t r = r0 + g;
    for (; r + 7 * (int64_t)groups < r1; r += 8 * (int64_t)groups) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = a[(r + u * (int64_t)groups) * E + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; r < r1; r += groups) acc += a[r * E + e];
  }
  s_part[tid] = acc;
  __syncthreads();
  float s = 0.0f;
  if (tid < width)
    for (int q = 0; q < groups; ++q) s += s_part[q * width + tid];
  __syncthreads();
  return s;
}

// partial[b][e] = sum of probs[t][e] over block b's rows.
__global__ __launch_bounds__(kAuxThreads) void aux_colsum_kernel(const float* __restrict__ probs, int64_t T, int E,
                                                                 int64_t rows_per_block, float* __restrict__ partial) {
  __shared__ float s_part[kAuxThreads];
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < T ? r0 + rows_per_block : T;
  for (int c0 = 0; c0 < E; c0 += kAuxThreads) {
    const int width = E - c0 < kAuxThreads ? E - c0 : kAuxThreads;
    const float s = block_colsum(probs, r0, r1, E, c0, width, s_part);
    if ((int)threadIdx.x < width) partial[(int64_t)blockIdx.x * E + c0 + threadIdx.x] = s;
  }
}

// One block: column sums over the block partials (the same fixed order), then
// f, counts and the loss; the sum over experts is a fixed tree over the 256
// threads' ascending partial sums.
__global__ __launch_bounds__(kAuxThreads) void aux_finish_kernel(const float* __restrict__ partial, int nblocks,
                                                                 const int64_t* __restrict__ tpe, int64_t T, int E,
                                                                 float* __restrict__ aux, float* __restrict__ counts,
                                                                 float* __restrict__ frac) {
  __shared__ float s_part[kAuxThreads];
  __shared__ float s_sum[kAuxThreads];
  const int tid = threadIdx.x;
  const float inv_t = 1.0f / (float)T;
  float local = 0.0f;
  for (int c0 = 0; c0 < E; c0 += kAuxThreads) {
    const int width = E - c0 < kAuxThreads ? E - c0 : kAuxThreads;
    const float s = block_colsum(partial, 0, nblocks, E, c0, width, s_part);
    if (tid < width) {
      const int e = c0 + tid;
      const float mean = s * inv_t;
      const float cnt = (float)tpe[e];
      const float f = cnt * inv_t;
      counts[e] = cnt;
      frac[e] = f;
      local += f * mean;
    }
  }
  s_sum[tid] = local;
  __syncthreads();
  for (int o = kAuxThreads / 2; o > 0; o >>= 1) {
    if (tid < o) s_sum[tid] += s_sum[tid + o];
    __syncthreads();
  }
  if (tid == 0) aux[0] = s_sum[0] * (float)E;
}

__global__ __launch_bounds__(kAuxThreads) void aux_backward_kernel(const float* __restrict__ g_aux,
                                                                   const float* __restrict__ frac, int64_t T, int E,
                                                                   float* __restrict__ g_row) {
  const float ge = g_aux[0] * (float)E;
  const float inv_t = 1.0f / (float)T;
  for (int e = blockIdx.x * kAuxThreads + threadIdx.x; e < E; e += gridDim.x * kAuxThreads)
    g_row[e] = (ge * frac[e]) * inv_t;
}

}  // namespace
}  // namespace hrm

extern "C" size_t hrm_moe_aux_loss_workspace_size(int64_t num_tokens, int32_t num_experts) {
  if (num_tokens < 1 || num_experts < 1 || num_experts > hrm::kAuxMaxExperts) return 0;
  return sizeof(float) * (size_t)hrm::aux_blocks(num_tokens) * (size_t)num_experts;
}

extern "C" int hrm_moe_aux_loss(const float* probs, int64_t num_tokens, int32_t num_experts,
                                const int64_t* tokens_per_expert, float* aux_loss, float* expert_counts,
                                float* expert_fraction, void* workspace, size_t workspace_bytes, void* stream) {
  if (num_tokens < 1 || num_experts < 1) return HRM_MOE_ERR_INVALID;
  if (num_experts > hrm::kAuxMaxExperts) return HRM_MOE_ERR_UNSUPPORTED;
  if (!probs || !tokens_per_expert || !aux_loss || !expert_counts || !expert_fraction) return HRM_MOE_ERR_INVALID;
  if (!workspace || workspace_bytes < hrm_moe_aux_loss_workspace_size(num_tokens, num_experts))
    return HRM_MOE_ERR_WORKSPACE;
  const int nb = hrm::aux_blocks(num_tokens);
  const int64_t rows = (num_tokens + nb - 1) / nb;
  float* partial = static_cast<float*>(workspace);
  HRM_LAUNCH(hrm::aux_colsum_kernel, dim3(nb), dim3(hrm::kAuxThreads), 0, stream, probs, num_tokens, num_experts,
             rows, partial);
  HRM_LAUNCH(hrm::aux_finish_kernel, dim3(1), dim3(hrm::kAuxThreads), 0, stream, partial, nb, tokens_per_expert,
             num_tokens, num_experts, aux_loss, expert_counts, expert_fraction);
  return HRM_MOE_OK;
}

extern "C" int hrm_moe_aux_loss_backward(const float* grad_aux, const float* expert_fraction, int64_t num_tokens,
                                         int32_t num_experts, float* grad_probs_row, void* stream) {
  if (num_tokens < 1 || num_experts < 1) return HRM_MOE_ERR_INVALID;
  if (!grad_aux || !expert_fraction || !grad_probs_row) return HRM_MOE_ERR_INVALID;
  const int blocks = (num_experts + hrm::kAuxThreads - 1) / hrm::kAuxThreads;
  HRM_LAUNCH(hrm::aux_backward_kernel, dim3(blocks), dim3(hrm::kAuxThreads), 0, stream, grad_aux, expert_fraction,
             num_tokens, num_experts, grad_probs_row);
  return HRM_MOE_OK;
}
