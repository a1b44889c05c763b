/*
 * hrm_moe.h - C ABI of the MI355X (gfx950) kernels for HRM-MoE's routed
 * SwiGLU MoE FFN (the reference's `grouped_triton` path).
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise.
 *     Tensors are dense and row-major (C order), with the shapes given in [].
 *   - `stream` is a hipStream_t (NULL = the default stream).  Every call only
 *     enqueues work on it: no entry point synchronises with the host,
 *     allocates memory, or reads device data on the host.
 *   - dtype codes: HRM_MOE_BF16, HRM_MOE_F16, HRM_MOE_F32.
 *   - Return value: HRM_MOE_OK (0); a negative HRM_MOE_ERR_* code for an
 *     argument the entry point rejects before launching anything; or a
 *     positive hipError_t from the HIP runtime.
 *   - Scratch memory is passed in by the caller (`workspace`, at least
 *     `*_workspace_size(...)` bytes, 256-byte aligned).
 *   - Calls that share a workspace must be ordered on one stream.
 *
 * Reference citations are paths relative to the reference repository
 * (XiaoYee/HRM-MoE).
 */
#ifndef HRM_MOE_H_
#define HRM_MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HRM_MOE_ABI_VERSION 1

enum hrm_moe_status {
  HRM_MOE_OK = 0,
  HRM_MOE_ERR_INVALID = -1,     /* null pointer, negative size, inconsistent sizes */
  HRM_MOE_ERR_DTYPE = -2,       /* dtype not supported by this entry point */
  HRM_MOE_ERR_UNSUPPORTED = -3, /* shape outside the kernels' limits (see each entry point) */
  HRM_MOE_ERR_WORKSPACE = -4    /* workspace null or smaller than required */
};

enum hrm_moe_dtype { HRM_MOE_BF16 = 0, HRM_MOE_F16 = 1, HRM_MOE_F32 = 2 };

/* ABI version of the loaded library (HRM_MOE_ABI_VERSION). */
int hrm_moe_abi_version(void);

/* Static description of a status code (never NULL). */
const char* hrm_moe_status_string(int status);

/*
 * Tuning configuration.  The library reads its knobs from the environment on
 * first use and keeps that snapshot; launches never read the environment.
 * hrm_moe_reload_config() reads it again (not safe while another thread
 * launches).  Returns HRM_MOE_OK, or HRM_MOE_ERR_INVALID when a value is
 * malformed (that knob keeps its default).
 *   HRM_MOE_HIP_CU_MARGIN, else HRM_MOE_TRITON_SM_MARGIN, else XTUNER_SM_MARGIN:
 *       compute units left out of the persistent GEMM grids, a non-negative
 *       integer.  Replaces SM_MARGIN of models/moe_triton_grouped_gemm.py:24-52
 *       (grid = max(1, SMs - margin)); here grid = max(1, CUs - margin) x
 *       workgroups per CU, rounded down to a multiple of 8, at least 8.
 *   HRM_MOE_GEMM_CFG, HRM_MOE_SKINNY, HRM_MOE_WGRAD_STAGES,
 *   HRM_MOE_GATE_SPLIT_ROWS, HRM_MOE_WAVE_ROUTER: kernel and tile choices
 *       (tests and tuning), replacing the reference's BLOCK_M / autotune knobs
 *       (models/moe_triton_grouped_gemm.py:48,70-110).
 */
int hrm_moe_reload_config(void);
/* The CU margin of the current configuration. */
int hrm_moe_cu_margin(void);

/*
 * Diagnostic, with no counterpart in the reference: the kernel instantiation
 * the latest M-grouped GEMM launch of `kind` used (0 = NT, the down
 * projection and forward grouped linear; 1 = gather + gate_up + SwiGLU,
 * including hrm_moe_router_gate_up_decode; 2 = NN, dgrad), as it appears
 * inside a profiler's demangled kernel name,
 * e.g. "mgemm_dma_kernel<hrm::BF16, 1, 128, 128, 2, 4, 64, 0, false>".
 * Empty before the first launch of that kind.  Lets a benchmark check that a
 * counter summary describes the kernel it timed.
 */
const char* hrm_moe_last_gemm_kernel(int kind);

/*
 * Router: fp32 softmax over experts, top-k, optional renormalisation, cast.
 * Replaces models/layers.py:606-610:
 *   probs = F.softmax(logits, -1, dtype=float32); w, idx = torch.topk(probs, k)
 *   if norm: w = w / w.sum(-1, keepdim=True).clamp_min(1e-12); w = w.to(dtype)
 * The softmax reproduces torch's device softmax bit for bit; top-k
 * reproduces torch.topk's order on ROCm, ties included.
 *   logits       [T, E] in logits_dtype (bf16, f16 or f32)
 *   probs        [T, E] fp32, may be NULL (needed only for the aux loss)
 *   topk_idx     [T, k] int64
 *   topk_weight  [T, k] in weight_dtype
 * Limits: 1 <= E <= 1024, 1 <= k <= min(E, 32) (torch's warp softmax, which
 * the kernels follow, covers rows of up to 1024 fp32 values).
 */
int hrm_moe_router_topk(const void* logits, int logits_dtype, int64_t num_tokens, int32_t num_experts,
                        int32_t top_k, int32_t norm_topk_prob, float* probs, int64_t* topk_idx,
                        void* topk_weight, int weight_dtype, void* stream);

/*
 * Dispatch: stable counting sort of the T*k routed slots by expert.
 * Replaces models/layers.py:312-322 (flatten, repeat_interleave,
 * torch.sort(stable=True), index_select of token ids, torch.bincount):
 *   tokens_per_expert [E]    int64  bincount(topk_idx, minlength=E)
 *   expert_offsets    [E+1]  int32  exclusive cumsum of tokens_per_expert
 *   sorted_token_idx  [T*k]  int32  token of each expert-contiguous row
 *   sort_idx          [T*k]  int64  slot t*k+j of each row (torch.sort's indices); may be NULL
 *   slot_to_row       [T*k]  int32  row of slot t*k+j (inverse permutation)
 * Rows of one expert are in ascending slot order (a stable sort).  Slots whose
 * expert id lies outside [0, E) are placed after every valid row (rows
 * >= expert_offsets[E]) and counted in no expert.
 * Limits: 1 <= E <= 1024, T*k < 2^31.
 */
size_t hrm_moe_permute_workspace_size(int64_t num_tokens, int32_t num_experts, int32_t top_k);
int hrm_moe_permute(const int64_t* topk_idx, int64_t num_tokens, int32_t num_experts, int32_t top_k,
                    int64_t* tokens_per_expert, int32_t* expert_offsets, int32_t* sorted_token_idx,
                    int64_t* sort_idx, int32_t* slot_to_row, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * Router and dispatch in two launches (one up to 64 tokens): hrm_moe_router_topk,
 * then hrm_moe_permute on its topk_idx, with the same outputs.  The router
 * kernel also ranks each block's routed slots within their expert, and one
 * scan + scatter kernel finishes the dispatch; with a single router block the
 * router kernel finishes it itself.  Up to 16 tokens with E <= 64, one block
 * with a wave per token (lane e holds expert e) does all of it; environment
 * HRM_MOE_WAVE_ROUTER=0 keeps the quad-layout kernel there.  Outputs are the
 * same bits either way.  Replaces models/layers.py:606-610 and
 * :312-322 back to back.  sort_idx may be NULL.
 * Limits: E <= 128, k <= 8, T*k < 2^31.  Workspace:
 * hrm_moe_router_dispatch_workspace_size.
 */
size_t hrm_moe_router_dispatch_workspace_size(int64_t num_tokens, int32_t num_experts, int32_t top_k);
int hrm_moe_router_topk_dispatch(const void* logits, int logits_dtype, int64_t num_tokens, int32_t num_experts,
                                 int32_t top_k, int32_t norm_topk_prob, float* probs, int64_t* topk_idx,
                                 void* topk_weight, int weight_dtype, int64_t* tokens_per_expert,
                                 int32_t* expert_offsets, int32_t* sorted_token_idx, int64_t* sort_idx,
                                 int32_t* slot_to_row, void* workspace, size_t workspace_bytes, void* stream);

/*
 * hrm_moe_router_topk_dispatch without a workspace argument: same arguments
 * (minus workspace and workspace_bytes), same outputs, same limits.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid allocation).  Its scratch (rank[T*k] and counts[ceil(T/64)][E+1])
 * is a fixed array inside the library, one copy per GPU, held until the
 * process ends; hrm_moe_router_dispatch_noalloc_max_bytes() gives its size,
 * 1.25 MiB: enough for 32768 tokens at E <= 128 and k <= 8.  A call whose
 * scratch need (hrm_moe_router_dispatch_workspace_size) exceeds it returns
 * HRM_MOE_ERR_UNSUPPORTED.  The call allocates nothing and needs nothing
 * zeroed; every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU (other streams, other threads) race: order them on one
 * stream.
 */
size_t hrm_moe_router_dispatch_noalloc_max_bytes(void);
int hrm_moe_router_topk_dispatch_noalloc(const void* logits, int logits_dtype, int64_t num_tokens,
                                         int32_t num_experts, int32_t top_k, int32_t norm_topk_prob, float* probs,
                                         int64_t* topk_idx, void* topk_weight, int weight_dtype,
                                         int64_t* tokens_per_expert, int32_t* expert_offsets,
                                         int32_t* sorted_token_idx, int64_t* sort_idx, int32_t* slot_to_row,
                                         void* stream);

/*
 * Grouped GEMMs over expert-contiguous row groups: rows
 * [sum(tpe[:e]), sum(tpe[:e+1])) belong to expert e.  tokens_per_expert is
 * int64 on the device and is never read on the host.  fp32 accumulation,
 * one rounding to dtype at the store.  dtype: bf16 or f16.  Limits: K and N
 * multiples of 8, E <= 1024, M < 2^31.  Rows past sum(tpe) are not written.
 */
size_t hrm_moe_grouped_gemm_workspace_size(int64_t num_rows, int32_t num_experts);

/* C[M,N] = A[M,K] . W[e][N,K]^T for the rows of expert e.
 * Replaces moe_triton_grouped_gemm.py:358-417 with trans_b=True
 * (_repeat_interleave_kernel :263-274, _m_grouped_gemm_bk_kernel :113-184):
 * the forward of triton_grouped_linear (:461-464, :478-485). */
int hrm_moe_grouped_gemm_nt(const void* A, const void* W, const int64_t* tokens_per_expert, int64_t M,
                            int64_t N, int64_t K, int32_t num_experts, int dtype, void* C, void* workspace,
                            size_t workspace_bytes, void* stream);

/* C[M,N] = A[M,K] . W[e][K,N] for the rows of expert e (dgrad).
 * Replaces moe_triton_grouped_gemm.py:358-417 with trans_b=False
 * (_m_grouped_gemm_bn_kernel :187-260), called from the backward at :472. */
int hrm_moe_grouped_gemm_nn(const void* A, const void* W, const int64_t* tokens_per_expert, int64_t M,
                            int64_t N, int64_t K, int32_t num_experts, int dtype, void* C, void* workspace,
                            size_t workspace_bytes, void* stream);

/* C[e][Na,Nb] = A[rows_e]^T . B[rows_e] with A [M,Na], B [M,Nb] (wgrad); an
 * expert without rows gets zeros.
 * Replaces _k_grouped_gemm (moe_triton_grouped_gemm.py:420-456) and
 * _k_grouped_gemm_kernel (:277-347), called from the backward at :474.
 * Workspace: at least hrm_moe_grouped_gemm_workspace_size(M, E).  With
 * hrm_moe_grouped_wgrad_workspace_size(M, Na, Nb, E) bytes, an expert holding
 * more than twice the mean rows (and at least 2048) is reduced in row
 * chunks into fp32 partial sums that are added in chunk order and rounded
 * once, so skewed loads keep every workgroup busy; results stay
 * deterministic and independent of the grid size. */
size_t hrm_moe_grouped_wgrad_workspace_size(int64_t num_rows, int64_t Na, int64_t Nb, int32_t num_experts);
int hrm_moe_grouped_gemm_tn(const void* A, const void* B, const int64_t* tokens_per_expert, int64_t M,
                            int64_t Na, int64_t Nb, int32_t num_experts, int dtype, void* C, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Fused expert input projection: row gather + gate_up grouped GEMM + SwiGLU.
 *   act[r, i] = silu(h[tok(r)] . Wgu[e][i]) * (h[tok(r)] . Wgu[e][I+i])
 * with tok = sorted_token_idx and e the expert owning row r (rows are
 * grouped by tokens_per_expert, as in the grouped GEMMs).  Rounding follows the reference: gate and up are rounded
 * to dtype, silu(gate) is rounded, then the product.
 * Replaces models/layers.py:320 (hidden_states.index_select), :325-326
 * (triton_grouped_linear on gate_up_weight) and :327-329 (silu(gate) * up).
 *   hidden [T,H], sorted_token_idx [R] (values in [0,T)), tokens_per_expert [E]
 *   int64, gate_up_weight [E,2I,H], act [R,I].  Workspace as for the grouped
 *   GEMMs (hrm_moe_grouped_gemm_workspace_size(R, E)).  dtype bf16 or f16.
 * Limits: H and I multiples of 8, E <= 1024.
 */
int hrm_moe_gate_up_swiglu(const void* hidden, const int32_t* sorted_token_idx, const int64_t* tokens_per_expert,
                           const void* gate_up_weight, int64_t num_tokens, int64_t num_rows, int64_t hidden_size,
                           int64_t inter_size, int32_t num_experts, int dtype, void* act, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Weighted combine back to token order.
 *   out[t] = round( sum over the token's slots j, in ascending row order, of
 *                   round(expert_out[slot_to_row[t*k+j]] * topk_weight[t,j]) )
 * with fp32 accumulation, which is what the reference's multiply and bf16
 * index_add_ compute on the CPU (models/layers.py:333-334).  Slots whose row
 * is >= expert_offsets[E] (dropped expert ids) contribute nothing.
 *   expert_out [R,H], topk_weight [T,k], out [T,H]; dtype bf16, f16 or f32.
 * topk_weight may be NULL: every weight is 1, the un-permute of the layer's
 * backward (sum of each token's rows, same order and single rounding).
 * Limits: H a multiple of 8, 1 <= k <= 32.
 */
int hrm_moe_combine(const void* expert_out, const int32_t* slot_to_row, const void* topk_weight,
                    const int32_t* expert_offsets, int64_t num_tokens, int32_t top_k, int64_t hidden_size,
                    int32_t num_experts, int dtype, void* out, void* stream);

/*
 * Down projection and combine in one launch, for one or two tokens
 * (models/layers.py:331-334: the down grouped linear, the weighting and the
 * index_add_).  For each token t and column c:
 *   out[t,c] = sum over t's slots j in ascending row order of
 *              round( round(act[row_j] . down_weight[e_j][c]) * topk_weight[t,j] )
 * with fp32 accumulation and one final rounding (row_j = slot_to_row[t*k+j],
 * e_j = topk_idx[t*k+j]).  The dot products take the decode-size grouped
 * GEMM's fp32 order (4 K quarters of 16x16x32 MFMA steps, added in order), so
 * where hrm_moe_grouped_gemm_nt picks its skinny kernel (T*k <= E/4, H a
 * multiple of 16) the result equals hrm_moe_grouped_gemm_nt followed by
 * hrm_moe_combine bit for bit.  Slots whose row is >= expert_offsets[E]
 * contribute nothing.  At these sizes the down GEMM only streams weights, and
 * one workgroup per 2 output columns computes the rows it needs and combines
 * them, so no [T*k, H] intermediate is written and no combine launch follows.
 *   act [T*k, I] (rows in dispatch order), down_weight [E, H, I],
 *   topk_weight [T, k] in dtype, out [T, H]; dtype bf16 or f16.
 * Limits: T <= 2, k <= 8, H even, I a multiple of 32 and <= 512.
 */
int hrm_moe_down_combine_decode(const void* act, const void* down_weight, const int32_t* slot_to_row,
                                const int64_t* topk_idx, const void* topk_weight, const int32_t* expert_offsets,
                                int64_t num_tokens, int32_t top_k, int64_t hidden_size, int64_t inter_size,
                                int32_t num_experts, int dtype, void* out, void* stream);

/*
 * Router, dispatch and gate/up grouped linear + SwiGLU in one launch, for one
 * or two tokens (models/layers.py:606-610, :312-322 and :325-329 of a decode
 * step).  Its outputs are the bits of hrm_moe_router_topk_dispatch followed by
 * hrm_moe_gate_up_swiglu on the same inputs (routing, probabilities, the
 * dispatch tensors and act), where hrm_moe_router_gate_up_decode_supported
 * says the call is covered: at these sizes the router launch costs as much as
 * its work.  hrm_moe_down_combine_decode then finishes the layer.
 *   logits [T,E] (logits_dtype), hidden [T,H], gate_up_weight [E,2I,H];
 *   outputs probs [T,E] fp32 (may be NULL), topk_idx [T,k] int64, topk_weight
 *   [T,k] in dtype, tokens_per_expert [E] int64, expert_offsets [E+1],
 *   sorted_token_idx [T*k], sort_idx [T*k] int64 (may be NULL), slot_to_row
 *   [T*k], act [T*k, I] (the SwiGLU rows in dispatch order); dtype bf16 or
 *   f16 for hidden, weights, topk_weight and act.
 * Limits (hrm_moe_router_gate_up_decode_supported): 1 <= T <= 2, k in
 * {2, 4, 8}, 4*T*k <= E <= 64, H a multiple of 64 and <= 2048, I a multiple
 * of 16.
 */
int hrm_moe_router_gate_up_decode_supported(int64_t num_tokens, int64_t hidden_size, int64_t inter_size,
                                            int32_t num_experts, int32_t top_k);
int hrm_moe_router_gate_up_decode(const void* logits, int logits_dtype, const void* hidden,
                                  const void* gate_up_weight, int64_t num_tokens, int64_t hidden_size,
                                  int64_t inter_size, int32_t num_experts, int32_t top_k, int32_t norm_topk_prob,
                                  int dtype, float* probs, int64_t* topk_idx, void* topk_weight,
                                  int64_t* tokens_per_expert, int32_t* expert_offsets, int32_t* sorted_token_idx,
                                  int64_t* sort_idx, int32_t* slot_to_row, void* act, void* stream);

/*
 * Training path.  The reference differentiates the grouped composition of
 * models/layers.py:317-334 with torch autograd; these entry points compute the
 * same quantities with the reference's rounding points.
 */

/* hrm_moe_gate_up_swiglu, also storing the rounded gate and up values
 * gate_up [R, 2I] (gate in columns [0,I), up in [I,2I)): the reference's
 * gate_up tensor (models/layers.py:326), saved for the backward of
 * silu(gate) * up.  Limits as hrm_moe_gate_up_swiglu, and H a multiple of 64. */
int hrm_moe_gate_up_swiglu_save(const void* hidden, const int32_t* sorted_token_idx,
                                const int64_t* tokens_per_expert, const void* gate_up_weight, int64_t num_tokens,
                                int64_t num_rows, int64_t hidden_size, int64_t inter_size, int32_t num_experts,
                                int dtype, void* act, void* gate_up, void* workspace, size_t workspace_bytes,
                                void* stream);

/* Down projection dgrad with the SwiGLU backward fused into its epilogue:
 *   dact[r]        = round(grad_expert_out[r] . down_weight[e])    [R, I]
 *   d_up[r,i]      = round(dact * round(silu(gate)))
 *   d_gate[r,i]    = round(round(dact * up) * sig * (1 + gate * (1 - sig))),  sig = sigmoid(gate)
 * written to grad_gate_up [R, 2I] as [d_gate | d_up].  This is the backward of
 * triton_grouped_linear on down_weight (moe_triton_grouped_gemm.py:472) followed
 * by torch autograd through silu(gate) * up (models/layers.py:328-329).
 *   grad_expert_out [R,H], down_weight [E,H,I], gate_up [R,2I].
 * Limits: H a multiple of 64, I a multiple of 8, E <= 1024. */
int hrm_moe_down_dgrad_swiglu(const void* grad_expert_out, const void* down_weight, const int64_t* tokens_per_expert,
                              const void* gate_up, int64_t num_rows, int64_t inter_size, int64_t hidden_size,
                              int32_t num_experts, int dtype, void* grad_gate_up, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Backward of the weighted combine (models/layers.py:333-334 under autograd):
 *   grad_expert_out[slot_to_row[t*k+j]] = round(grad_out[t] * topk_weight[t,j])
 *   grad_weight[t,j] = round(sum_h round(grad_out[t,h] * expert_out[row,h]))
 * The sum over h is in fp32 with a fixed order, so results are deterministic.
 * Slots with a dropped row (>= expert_offsets[E]) get grad_weight 0 and no
 * row write.  grad_out [T,H], expert_out and grad_expert_out [R,H],
 * topk_weight and grad_weight [T,k].  Limits: H a multiple of 8, 1 <= k <= 32. */
int hrm_moe_combine_backward(const void* grad_out, const void* expert_out, const int32_t* slot_to_row,
                             const void* topk_weight, const int32_t* expert_offsets, int64_t num_tokens,
                             int32_t top_k, int64_t hidden_size, int32_t num_experts, int dtype,
                             void* grad_expert_out, void* grad_weight, void* stream);

/* Backward of hrm_moe_router_topk (models/layers.py:606-610 under autograd):
 *   v_j = probs[t, idx_j], s = sum_j v_j, c = max(s, 1e-12)
 *   dv_j = g_w[t,j] / c - (sum_i g_w[t,i] v_i) / c^2 * [s >= 1e-12]   (norm_topk_prob; else dv_j = g_w[t,j])
 *   dp[t,e] = grad_probs[t,e] + sum over j with idx_j = e of dv_j
 *   grad_logits[t,e] = probs[t,e] * (dp[t,e] - sum_e' probs[t,e'] dp[t,e'])
 * probs [T,E] fp32 (the forward's output), topk_idx [T,k] int64, grad_weight
 * [T,k], grad_probs fp32 or NULL (no gradient reaches the probabilities):
 * row t at grad_probs + t * grad_probs_row_stride, the stride E for a [T,E]
 * tensor or 0 for one row shared by every token (the auxiliary loss's gradient,
 * which is the same for all tokens).  grad_logits [T,E] in logits_dtype.
 * Deterministic.  Limits: E <= 1024, k <= 32. */
int hrm_moe_router_topk_backward(const float* probs, const int64_t* topk_idx, const void* grad_weight,
                                 int grad_weight_dtype, const float* grad_probs, int64_t grad_probs_row_stride,
                                 int64_t num_tokens,
                                 int32_t num_experts, int32_t top_k, int32_t norm_topk_prob, void* grad_logits,
                                 int logits_dtype, void* stream);

/* Router gate weight gradient: grad_gate_weight[E,H] = grad_logits[T,E]^T . hidden[T,H],
 * the weight grad of F.linear(hidden, gate.weight) (models/layers.py:605, :89-90)
 * that torch autograd computes.  The T rows are split into S <= 128 groups
 * whose fp32 partial products are summed in group order and rounded once, so
 * results are deterministic.  Workspace: hrm_moe_gate_wgrad_workspace_size.
 * dtype bf16 or f16.  Limits: E and H multiples of 8, T*H*2 and T*E*2 < 2^32. */
size_t hrm_moe_gate_wgrad_workspace_size(int64_t num_tokens, int32_t num_experts, int64_t hidden_size);
int hrm_moe_gate_wgrad(const void* grad_logits, const void* hidden, int64_t num_tokens, int32_t num_experts,
                       int64_t hidden_size, int dtype, void* grad_gate_weight, void* workspace,
                       size_t workspace_bytes, void* stream);

/* hrm_moe_grouped_gemm_tn with the B operand's rows gathered:
 *   C[e][Na,Nb] = A[rows_e]^T . B[b_row_index[rows_e]]
 * with B [b_rows, Nb] and b_row_index [M] (values in [0, b_rows); others read
 * as zero rows).  This is the gate_up grad_weight of the reference
 * (moe_triton_grouped_gemm.py:474 on the rows index_select-ed at
 * models/layers.py:320) without materialising the gathered rows.
 * Limits as hrm_moe_grouped_gemm_tn, and b_rows * Nb * 2 < 2^32. */
int hrm_moe_grouped_gemm_tn_gather(const void* A, const void* B, const int32_t* b_row_index, int64_t b_rows,
                                   const int64_t* tokens_per_expert, int64_t M, int64_t Na, int64_t Nb,
                                   int32_t num_experts, int dtype, void* C, void* workspace, size_t workspace_bytes,
                                   void* stream);

/*
 * Auxiliary load-balancing loss and expert counts of the layer
 * (models/layers.py:163-170 load_balancing_loss_func, :619-632 counts):
 *   f[e] = tokens_per_expert[e] * (1/T),  mean[e] = sum_t probs[t,e] * (1/T)
 *   aux_loss[0] = (sum_e f[e] * mean[e]) * E,  expert_counts[e] = tokens_per_expert[e]
 * and expert_fraction[e] = f[e] for the backward.  probs [T,E] fp32 (the
 * router's), tokens_per_expert [E] int64 (the dispatch's counts, equal to
 * the reference's bincount).  Sums run in a fixed order (deterministic).
 * Workspace: hrm_moe_aux_loss_workspace_size.  Limits: T >= 1, E <= 1024.
 */
size_t hrm_moe_aux_loss_workspace_size(int64_t num_tokens, int32_t num_experts);
int hrm_moe_aux_loss(const float* probs, int64_t num_tokens, int32_t num_experts, const int64_t* tokens_per_expert,
                     float* aux_loss, float* expert_counts, float* expert_fraction, void* workspace,
                     size_t workspace_bytes, void* stream);
/* Its gradient, the same for every token: grad_probs_row[e] = ((grad_aux[0] * E) * f[e]) * (1/T),
 * to pass to hrm_moe_router_topk_backward with grad_probs_row_stride = 0. */
int hrm_moe_aux_loss_backward(const float* grad_aux, const float* expert_fraction, int64_t num_tokens,
                              int32_t num_experts, float* grad_probs_row, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HRM_MOE_H_ */
