// Router, dispatch and gate/up + SwiGLU of one or two tokens, in one launch.
//
// Replaces, for a decode step of one or two tokens, models/layers.py:606-610
// (softmax router + top-k), :312-322 (dispatch) and :325-329 (gate/up grouped
// linear + SwiGLU).  At these sizes each of them is a few microseconds of
// latency, so the router launch costs as much as its work.  Here every
// workgroup selects the tokens' experts itself (route_token_select, the code
// of the decode-size router, so the routing is the same bits), derives the
// dispatch rows from the selection masks and issues its weight loads at once;
// workgroup 0 also finishes the routing (route_token_finish: torch's order and
// the weights) and writes the router and dispatch outputs while its loads fly.
// Workgroup (j, cb) runs the decode-size grouped GEMM's weight-streaming step
// (skinny_step.h, as mgemm_skinny_kernel runs it with one 16-row block and
// every K chunk in flight) for the j-th expert with rows and output columns
// [16 cb, 16 cb + 16), with the SwiGLU epilogue.  The down projection and the
// combine follow in one more launch (hrm_moe_down_combine_decode), which reads
// act after this kernel has ended.
//
// Taking the down projection and the combine into this launch as well was
// measured slower: workgroups that wait for every gate/up result (a counter in
// memory, the act rows read through coherent loads or after an L2
// invalidate) took 34-52 us per layer at T = 1 against 19.8 us for the three
// launches (everything after the gate GEMM, graphs of 8 layers), because each
// hand-over between workgroups on different XCDs costs several dependent
// memory round trips.
#include <stdio.h>

#include "common.h"
#include "route_wave.h"
#include "skinny_step.h"

namespace hrm {
namespace {

constexpr int kDecMaxTokens = 2;

struct DecodeArgs {
  const void* logits;         // [T, E] in ldt
  const uint16_t* x;          // [T, H]
  const uint16_t* w_gu;       // [E, 2I, H]: gate rows [0, I), up rows [I, 2I)
  float* probs;               // [T, E] or null
  int64_t* idx_out;           // [T, k]
  uint16_t* w_out;            // [T, k]
  int64_t* tokens_per_expert; // [E]
  int32_t* expert_offsets;    // [E + 1]
  int32_t* sorted_token_idx;  // [T k]
  int64_t* sort_idx;          // [T k] or null
  int32_t* slot_to_row;       // [T k]
  uint16_t* act;              // [T k, I], rows in dispatch order
  int ldt, T, E, norm, H, I;  // top-k is the kernel's SLOTS
};

template <typename TR, int SLOTS, int CPW>
__global__ __launch_bounds__(256) void router_gate_up_decode_kernel(DecodeArgs a) {
  __shared__ uint64_t s_ck[4][64];
  __shared__ uint32_t s_sk[4][SLOTS];
  __shared__ int32_t s_si[4][SLOTS];
  __shared__ uint64_t s_sel[4];  // token -> its selected experts, as a bit mask
  __shared__ SkinnyRed<true, 1> red;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int k = SLOTS;
  const int T = a.T, E = a.E;
  const bool writer = blockIdx.x == 0;

  // ---- selection: wave w selects token w's experts (waves past T pass the barriers idle)
  route_token_select<SLOTS, true>(a.logits, a.ldt, wave, wave < T, E, k, writer ? a.probs : nullptr, s_ck[wave],
                                  s_sk[wave], s_si[wave], &s_sel[wave]);
  // Rows in dispatch order are expert-major and, within an expert, in flat slot
  // order (token 0's row before token 1's), so the masks give every row: expert
  // e's rows start at the number of selected slots with a smaller expert.  (Each
  // token selects k distinct experts with nonzero keys, all inside [0, E): E >= k
  // experts have a nonzero key and rank above the padding lanes.)
  const uint64_t sel0 = s_sel[0];
  const uint64_t sel1 = T > 1 ? s_sel[1] : 0ull;
  auto rows_below = [&](int e) __attribute__((always_inline)) -> int {
    const uint64_t below = e >= 64 ? ~0ull : ((1ull << e) - 1ull);
    return __popcll(sel0 & below) + __popcll(sel1 & below);
  };

  // ---- gate/up: expert j (the j-th with rows, ascending id), columns [c0, c0 + 16).
  // Its loads go out first; workgroup 0's routing outputs are computed while they fly.
  const uint64_t any = sel0 | sel1;
  const int cblk = a.I / 16;
  const int j = blockIdx.x / cblk;
  const int c0 = (blockIdx.x - j * cblk) * 16;
  const bool has = j < __popcll(any);  // uniform over the workgroup
  const int N = a.I, K = a.H;
  const int nc = K / 32;
  const int kc0 = wave * nc / 4, kc1 = (wave + 1) * nc / 4;
  int rs = 0, re = 0;
  SkinnyChunks<TR, true, 1, CPW> ch;
  if (has) {
    const int my_rank = __popcll(any & ((1ull << lane) - 1ull));
    const uint64_t hit = __ballot(((any >> lane) & 1ull) && my_rank == j);
    const int e = __ffsll((unsigned long long)hit) - 1;
    const int b0 = (int)((sel0 >> e) & 1ull), b1 = (int)((sel1 >> e) & 1ull);
    rs = rows_below(e);
    re = rs + b0 + b1;
    int rr = lane & 15;
    rr = rr < re - rs ? rr : re - rs - 1;  // rows past the expert repeat a valid one; their columns are never stored
    const int tok = (b0 && b1) ? rr : (b0 ? 0 : 1);
    const uint16_t* wg = a.w_gu + ((int64_t)e * 2 * N + c0 + (lane & 15)) * K + (lane >> 4) * 8;
    const uint16_t* wu = wg + (int64_t)N * K;
    const uint16_t* const xr[1] = {a.x + (int64_t)tok * K + (lane >> 4) * 8};
    ch.load(wg, wu, xr, kc0, kc1);
  }

  if (writer) {
    // torch's output order and the weights of each token's k slots, then the dispatch tensors
    int my_i;
    float my_w;
    route_token_finish<SLOTS, true>(wave < T, k, a.norm, s_sk[wave], s_si[wave], my_i, my_w);
    if (wave < T && lane < k) {
      const int ls = wave * k + lane;
      a.idx_out[ls] = (int64_t)my_i;
      a.w_out[ls] = TR::from_f(my_w);
      const int dst = rows_below(my_i) + ((wave == 1 && ((sel0 >> my_i) & 1ull)) ? 1 : 0);
      a.sorted_token_idx[dst] = wave;
      if (a.sort_idx) a.sort_idx[dst] = ls;
      a.slot_to_row[ls] = dst;
    }
    if (tid <= E) {
      if (tid < E) a.tokens_per_expert[tid] = (int64_t)(((sel0 >> tid) & 1ull) + ((sel1 >> tid) & 1ull));
      a.expert_offsets[tid] = rows_below(tid);
    }
  }

  if (has) {
    floatx4 ag[1] = {floatx4{0.f, 0.f, 0.f, 0.f}}, au[1] = {floatx4{0.f, 0.f, 0.f, 0.f}};
    ch.mma(kc0, kc1, ag, au);
    skinny_publish<true, 1>(red, wave, lane, ag, au);
  }
  __syncthreads();
  if (has) skinny_store<TR, true, 1>(red, wave, lane, rs, re, a.act, N, c0);
}

template <typename TR, int SLOTS>
int launch_router_gate_up_decode(const DecodeArgs& a, int cpw, dim3 grid, void* stream) {
  if (cpw == 4) HRM_LAUNCH((router_gate_up_decode_kernel<TR, SLOTS, 4>), grid, dim3(256), 0, stream, a);
  else if (cpw == 8) HRM_LAUNCH((router_gate_up_decode_kernel<TR, SLOTS, 8>), grid, dim3(256), 0, stream, a);
  else if (cpw == 12) HRM_LAUNCH((router_gate_up_decode_kernel<TR, SLOTS, 12>), grid, dim3(256), 0, stream, a);
  else HRM_LAUNCH((router_gate_up_decode_kernel<TR, SLOTS, 16>), grid, dim3(256), 0, stream, a);
  return HRM_MOE_OK;
}

}  // namespace
}  // namespace hrm

extern "C" int hrm_moe_router_gate_up_decode_supported(int64_t num_tokens, int64_t hidden_size, int64_t inter_size,
                                                       int32_t num_experts, int32_t top_k) {
  if (num_tokens < 1 || num_tokens > hrm::kDecMaxTokens) return 0;
  if (top_k != 2 && top_k != 4 && top_k != 8) return 0;
  if (num_experts < top_k || num_experts > 64 || num_tokens * top_k * 4 > num_experts) return 0;
  if (hidden_size < 64 || hidden_size % 64 || hidden_size > 2048) return 0;
  if (inter_size < 16 || inter_size % 16) return 0;
  return 1;
}

extern "C" int hrm_moe_router_gate_up_decode(const void* logits, int logits_dtype, const void* hidden,
                                             const void* gate_up_weight, int64_t num_tokens, int64_t hidden_size,
                                             int64_t inter_size, int32_t num_experts, int32_t top_k,
                                             int32_t norm_topk_prob, int dtype, float* probs, int64_t* topk_idx,
                                             void* topk_weight, int64_t* tokens_per_expert,
                                             int32_t* expert_offsets, int32_t* sorted_token_idx, int64_t* sort_idx,
                                             int32_t* slot_to_row, void* act, void* stream) {
  if (num_tokens < 0 || hidden_size < 1 || inter_size < 1 || num_experts < 1 || top_k < 1 || top_k > num_experts)
    return HRM_MOE_ERR_INVALID;
  if (dtype != HRM_MOE_BF16 && dtype != HRM_MOE_F16) return HRM_MOE_ERR_DTYPE;
  if (logits_dtype < HRM_MOE_BF16 || logits_dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (num_tokens == 0) return HRM_MOE_OK;
  if (!hrm_moe_router_gate_up_decode_supported(num_tokens, hidden_size, inter_size, num_experts, top_k))
    return HRM_MOE_ERR_UNSUPPORTED;
  if (!logits || !hidden || !gate_up_weight || !topk_idx || !topk_weight || !tokens_per_expert || !expert_offsets ||
      !sorted_token_idx || !slot_to_row || !act)
    return HRM_MOE_ERR_INVALID;
  hrm::DecodeArgs a;
  a.logits = logits;
  a.x = static_cast<const uint16_t*>(hidden);
  a.w_gu = static_cast<const uint16_t*>(gate_up_weight);
  a.probs = probs;
  a.idx_out = topk_idx;
  a.w_out = static_cast<uint16_t*>(topk_weight);
  a.tokens_per_expert = tokens_per_expert;
  a.expert_offsets = expert_offsets;
  a.sorted_token_idx = sorted_token_idx;
  a.sort_idx = sort_idx;
  a.slot_to_row = slot_to_row;
  a.act = static_cast<uint16_t*>(act);
  a.ldt = logits_dtype;
  a.T = (int)num_tokens;
  a.E = num_experts;
  a.norm = norm_topk_prob ? 1 : 0;
  a.H = (int)hidden_size;
  a.I = (int)inter_size;
  // one workgroup group per expert that can have rows (at most T k of them), I / 16 column blocks each
  const int64_t experts_max = num_tokens * top_k < num_experts ? num_tokens * top_k : num_experts;
  const dim3 grid((unsigned)(experts_max * (inter_size / 16)));
  // K chunks per wave (4 waves split H in 32-wide chunks), all in flight at once
  const int need = (int)((hidden_size / 32 + 3) / 4);
  const int cpw = need <= 4 ? 4 : (need <= 8 ? 8 : (need <= 12 ? 12 : 16));
  char name[96];
  snprintf(name, sizeof(name), "router_gate_up_decode_kernel<%s, %d, %d>",
           dtype == HRM_MOE_BF16 ? "hrm::BF16" : "hrm::F16", (int)top_k, cpw);
  hrm::set_last_gemm_kernel(1, name);
#define HRM_RG(TR_)                                                                            \
  do {                                                                                         \
    if (top_k == 2) return hrm::launch_router_gate_up_decode<TR_, 2>(a, cpw, grid, stream);    \
    if (top_k == 4) return hrm::launch_router_gate_up_decode<TR_, 4>(a, cpw, grid, stream);    \
    return hrm::launch_router_gate_up_decode<TR_, 8>(a, cpw, grid, stream);                    \
  } while (0)
  if (dtype == HRM_MOE_BF16) HRM_RG(hrm::BF16);
  HRM_RG(hrm::F16);
#undef HRM_RG
}
