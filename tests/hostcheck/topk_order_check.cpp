// Host build of the router's ordering code (hrm-moe_amd/csrc/topk_order.h),
// so the CPU tests check the exact functions the kernel runs.
#include <stdint.h>

#include "topk_order.h"

namespace {
// KC > 0: the compile-time-k form the router uses when k == SLOTS.
template <int SLOTS, int KC = 0>
void order_rows(int k, int64_t rows, const uint32_t* sel_keys, const int32_t* sel_idx, int32_t* out_idx,
                float* out_sum) {
  for (int64_t r = 0; r < rows; ++r) {
    uint32_t sk[SLOTS] = {};
    int si[SLOTS] = {};
    for (int j = 0; j < k; ++j) {
      sk[j] = sel_keys[r * k + j];
      si[j] = sel_idx[r * k + j];
    }
    uint32_t gk[SLOTS];
    int gi[SLOTS];
    hrm::torch_topk_order<SLOTS, KC>(sk, si, k, gk, gi);
    float w[SLOTS];
    for (int j = 0; j < SLOTS; ++j) {
      union { uint32_t u; float f; } c;
      c.u = gk[j] - 1u;
      w[j] = c.f;
    }
    for (int j = 0; j < k; ++j) out_idx[r * k + j] = gi[j];
    out_sum[r] = hrm::torch_row_sum<SLOTS, KC>(w, k);
  }
}
}  // namespace

void order_rows_mem(int k, int64_t rows, const uint32_t* sel_keys, const int32_t* sel_idx, int32_t* out_idx,
                    float* out_sum) {
  int slots = 2;
  while (slots < k) slots *= 2;
  for (int64_t r = 0; r < rows; ++r) {
    uint32_t gk[32];
    int gi[32];
    bool gv[32];
    int si[32];
    for (int j = 0; j < k; ++j) si[j] = sel_idx[r * k + j];
    hrm::torch_topk_order_mem(sel_keys + r * k, si, k, slots, gk, gi, gv);
    float w[32];
    for (int j = 0; j < k; ++j) {
      union { uint32_t u; float f; } c;
      c.u = gk[j] - 1u;
      w[j] = c.f;
      out_idx[r * k + j] = gi[j];
    }
    out_sum[r] = hrm::torch_row_sum_mem(w, k);
  }
}

// sel_keys / sel_idx: [rows, k] selected pairs in (key desc, index asc) order,
// keys = float bits + 1.  Writes torch's output order and the weight sum,
// using the unrolled register form (loop_form 0), the loop form (1) or the
// register form with k fixed at compile time (2; k a power of two).
extern "C" int topk_order_check(int32_t k, int64_t rows, const uint32_t* sel_keys, const int32_t* sel_idx,
                                int32_t* out_idx, float* out_sum, int32_t loop_form) {
  if (k < 1 || k > 32) return -1;
  if (loop_form == 1) {
    order_rows_mem(k, rows, sel_keys, sel_idx, out_idx, out_sum);
    return 0;
  }
  if (loop_form == 2) {  // compile-time k == SLOTS
    if (k == 2) order_rows<2, 2>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
    else if (k == 4) order_rows<4, 4>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
    else if (k == 8) order_rows<8, 8>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
    else if (k == 16) order_rows<16, 16>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
    else if (k == 32) order_rows<32, 32>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
    else return -2;
    return 0;
  }
  if (k <= 2) order_rows<2>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
  else if (k <= 4) order_rows<4>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
  else if (k <= 8) order_rows<8>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
  else if (k <= 16) order_rows<16>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
  else order_rows<32>(k, rows, sel_keys, sel_idx, out_idx, out_sum);
  return 0;
}
