// Weighted combine of expert rows back to token order.
//
// Replaces models/layers.py:333-334 of the reference:
//   expert_output = expert_output * sorted_weights[:, None]
//   final_hidden_states.index_add_(0, sorted_token_idx, expert_output)
// as a gather instead of a scatter.  Each token's k rows (slot_to_row) are
// read and each is multiplied by its routing weight with a rounding to the
// element type (the reference multiplies 16-bit tensors); the products are
// added in fp32 in ascending row order and rounded once at the end.  That is
// the arithmetic of the reference's index_add_ on the CPU.  The gather does
// no atomics, so the result is the same on every run.
#include "common.h"

namespace hrm {
namespace {

// Expert rows are read exactly once: non-temporal loads keep them from
// evicting other lines (L combine 79.3 -> 70.9 us with the same block shape).
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

template <int DT>
struct Elem;
template <>
struct Elem<HRM_MOE_BF16> {
  static constexpr int kPer16 = 8;
  static __device__ __forceinline__ float get(const u32x4& v, int q) {
    const uint32_t w = v[q >> 1];
    return BF16::to_f((uint16_t)((q & 1) ? (w >> 16) : (w & 0xffff)));
  }
  static __device__ __forceinline__ float round(float f) { return BF16::to_f(BF16::from_f(f)); }
  static __device__ __forceinline__ float mul(float a, float b) { return round(a * b); }
  static __device__ __forceinline__ float weight(const void* p, int64_t i) { return BF16::to_f(reinterpret_cast<const uint16_t*>(p)[i]); }
  static __device__ __forceinline__ void store1(void* p, int64_t i, float v) { reinterpret_cast<uint16_t*>(p)[i] = BF16::from_f(v); }
  static __device__ __forceinline__ u32x4 pack(const float* a) {
    return u32x4{pack2(BF16::from_f(a[0]), BF16::from_f(a[1])), pack2(BF16::from_f(a[2]), BF16::from_f(a[3])),
                 pack2(BF16::from_f(a[4]), BF16::from_f(a[5])), pack2(BF16::from_f(a[6]), BF16::from_f(a[7]))};
  }
};
template <>
struct Elem<HRM_MOE_F16> {
  static constexpr int kPer16 = 8;
  static __device__ __forceinline__ float get(const u32x4& v, int q) {
    const uint32_t w = v[q >> 1];
    return F16::to_f((uint16_t)((q & 1) ? (w >> 16) : (w & 0xffff)));
  }
  static __device__ __forceinline__ float round(float f) { return F16::to_f(F16::from_f(f)); }
  static __device__ __forceinline__ float mul(float a, float b) { return round(a * b); }
  static __device__ __forceinline__ float weight(const void* p, int64_t i) { return F16::to_f(reinterpret_cast<const uint16_t*>(p)[i]); }
  static __device__ __forceinline__ void store1(void* p, int64_t i, float v) { reinterpret_cast<uint16_t*>(p)[i] = F16::from_f(v); }
  static __device__ __forceinline__ u32x4 pack(const float* a) {
    return u32x4{pack2(F16::from_f(a[0]), F16::from_f(a[1])), pack2(F16::from_f(a[2]), F16::from_f(a[3])),
                 pack2(F16::from_f(a[4]), F16::from_f(a[5])), pack2(F16::from_f(a[6]), F16::from_f(a[7]))};
  }
};
template <>
struct Elem<HRM_MOE_F32> {
  static constexpr int kPer16 = 4;
  static __device__ __forceinline__ float get(const u32x4& v, int q) { return __uint_as_float(v[q]); }
  static __device__ __forceinline__ float round(float f) { return f; }
  static __device__ __forceinline__ float weight(const void* p, int64_t i) { return reinterpret_cast<const float*>(p)[i]; }
  // the product is rounded before the add, as the reference's separate
  // multiply is: device code contracts a * b + c into an FMA by default
  static __device__ __forceinline__ float mul(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
  }
  static __device__ __forceinline__ void store1(void* p, int64_t i, float v) { reinterpret_cast<float*>(p)[i] = v; }
  static __device__ __forceinline__ u32x4 pack(const float* a) {
    return u32x4{__float_as_uint(a[0]), __float_as_uint(a[1]), __float_as_uint(a[2]), __float_as_uint(a[3])};
  }
};

// 2 tokens per block (of 256 threads): L combine 69.5 us at 4, 67.4 us at 2 (8: 79.3 us before the
// non-temporal loads)
constexpr int kTokPerBlock = 2;
constexpr int kBlock = 256;     // threads per pass when the columns are split over blocks (small T)
constexpr int kMaxBlock = 512;  // otherwise one thread per (token, chunk) item, up to this many
constexpr int kMaxTopK = 32;    // kTokPerBlock * kMaxTopK <= kBlock: one thread per routed slot

// A block combines kTokPerBlock consecutive tokens over one slice of the
// columns (blockIdx.y of gridDim.y slices; one slice except at small T, where
// the slices spread the loads of a few tokens over many CUs).  Its threads
// first rank each token's k rows (ascending row order is the summation order)
// into LDS, then stride over (token, 16-byte chunk) items, so no lane idles
// when a token's chunk count is not a multiple of the wave size.
// KU > 0: top-k fixed at compile time, so every row load of an item is issued
// before the first product is added (all k loads in flight per lane).
// KU == 0: any top-k up to kMaxTopK, rows loaded one after another.
template <int DT, int KU>
__global__ __launch_bounds__(kMaxBlock) void combine_kernel(const char* __restrict__ Y,
                                                        const int32_t* __restrict__ slot_to_row,
                                                        const void* __restrict__ wts,
                                                        const int32_t* __restrict__ expert_offsets, int64_t T,
                                                        int k, int64_t H, int E, char* __restrict__ out) {
  using El = Elem<DT>;
  constexpr int P = El::kPer16;
  constexpr int ESZ = 16 / P;
  __shared__ int32_t s_raw[kTokPerBlock * kMaxTopK];
  __shared__ int32_t s_row[kTokPerBlock][kMaxTopK];
  __shared__ float s_w[kTokPerBlock][kMaxTopK];
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.x * kTokPerBlock;
  const int ntok = (int)(T - t0 < kTokPerBlock ? T - t0 : kTokPerBlock);
  const int nslot = ntok * k;
  const int32_t r_valid = expert_offsets[E];
  int32_t row = 0;
  float w = 0.0f;
  if (tid < nslot) {
    row = slot_to_row[t0 * k + tid];
    w = wts ? El::weight(wts, t0 * k + tid) : 1.0f;  // no weights: the un-permute (round(y * 1) = y)
    s_raw[tid] = row;
  }
  __syncthreads();
  // Rank of this slot's row among its token's k rows (rows are distinct).
  if (tid < nslot) {
    const int tk = tid / k;
    const int32_t* rows = s_raw + tk * k;
    int rank = 0;
    for (int j = 0; j < k; ++j) rank += rows[j] < row ? 1 : 0;
    s_row[tk][rank] = row;
    s_w[tk][rank] = w;
  }
  __syncthreads();
  const int all_chunks = (int)(H / P);
  const int per = (all_chunks + (int)gridDim.y - 1) / (int)gridDim.y;
  const int c_lo = (int)blockIdx.y * per;
  const int chunks = min(per, all_chunks - c_lo);  // this block's slice (may be empty)
  const int items = ntok * chunks;
  for (int it = tid; it < items; it += (int)blockDim.x) {
    const int tk = it / chunks;
    const int c = c_lo + (it - tk * chunks);
    float acc[P];
#pragma unroll
    for (int q = 0; q < P; ++q) acc[q] = 0.0f;
    if constexpr (KU > 0) {
      u32x4 y[KU];
      bool ok[KU];
#pragma unroll
      for (int j = 0; j < KU; ++j) {
        const int32_t r = s_row[tk][j];
        ok[j] = r < r_valid;  // dropped rows hold no expert output
        y[j] = ld16_nt(Y + ((int64_t)(ok[j] ? r : 0) * H + (int64_t)c * P) * ESZ);
      }
#pragma unroll
      for (int j = 0; j < KU; ++j) {
        const float wj = s_w[tk][j];
#pragma unroll
        for (int q = 0; q < P; ++q) acc[q] = ok[j] ? acc[q] + El::mul(El::get(y[j], q), wj) : acc[q];
      }
    } else {
      for (int j = 0; j < k; ++j) {
        const int32_t r = s_row[tk][j];
        if (r >= r_valid) continue;
        const float wj = s_w[tk][j];
        const u32x4 y = ld16(Y + ((int64_t)r * H + (int64_t)c * P) * ESZ);
#pragma unroll
        for (int q = 0; q < P; ++q) acc[q] += El::mul(El::get(y, q), wj);
      }
    }
    st16(out + ((t0 + tk) * H + (int64_t)c * P) * ESZ, El::pack(acc));
  }
}

// Backward of the weighted combine, as torch autograd differentiates
// models/layers.py:333-334 (expert_output * sorted_weights[:, None], then
// index_add_):
//   d_rows[row(t,j)] = round(dout[t] * w[t,j])
//   d_w[t,j]         = round(sum_h round(dout[t,h] * rows[row(t,j),h]))
// One wave per token, lanes striding over 16-byte chunks.  The per-slot sums
// are reduced over the wave by a fixed xor butterfly, so every run gives the
// same bits.  Slots whose row is a dropped one (>= expert_offsets[E]) get
// d_w = 0 and no d_rows write.
// KU > 0: top-k fixed at compile time, all slots handled per chunk.
// KU == 0: any top-k, one slot at a time.
constexpr int kBwdWaves = 4;
template <int DT, int KU>
__global__ __launch_bounds__(kBwdWaves * 64) void combine_bwd_kernel(const char* __restrict__ dout,
                                                                    const char* __restrict__ Y,
                                                                    const int32_t* __restrict__ slot_to_row,
                                                                    const void* __restrict__ wts,
                                                                    const int32_t* __restrict__ expert_offsets,
                                                                    int64_t T, int k, int64_t H, int E,
                                                                    char* __restrict__ dY, void* __restrict__ dW) {
  using El = Elem<DT>;
  constexpr int P = El::kPer16;
  constexpr int ESZ = 16 / P;
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * kBwdWaves + (threadIdx.x >> 6);
  if (t >= T) return;  // no barriers below
  const int32_t r_valid = expert_offsets[E];
  int32_t my_row = 0;
  float my_w = 0.0f;
  if (lane < k) {
    my_row = slot_to_row[t * k + lane];
    my_w = El::weight(wts, t * k + lane);
  }
  const int chunks = (int)(H / P);
  const char* drow = dout + t * H * ESZ;
  auto reduce = [](float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
  };
  if constexpr (KU > 0) {
    int32_t row[KU];
    float wj[KU], part[KU];
    bool ok[KU];
#pragma unroll
    for (int j = 0; j < KU; ++j) {
      row[j] = __shfl(my_row, j, 64);
      wj[j] = __shfl(my_w, j, 64);
      ok[j] = row[j] < r_valid;
      part[j] = 0.0f;
    }
    for (int c = lane; c < chunks; c += 64) {
      const u32x4 g = ld16(drow + (int64_t)c * 16);
      u32x4 y[KU];
#pragma unroll
      for (int j = 0; j < KU; ++j) y[j] = ld16_nt(Y + ((int64_t)(ok[j] ? row[j] : 0) * H + (int64_t)c * P) * ESZ);
#pragma unroll
      for (int j = 0; j < KU; ++j) {
        float dy[P];
#pragma unroll
        for (int q = 0; q < P; ++q) {
          const float gq = El::get(g, q);
          part[j] += El::mul(gq, El::get(y[j], q));
          dy[q] = El::mul(gq, wj[j]);
        }
        if (ok[j]) st16(dY + ((int64_t)row[j] * H + (int64_t)c * P) * ESZ, El::pack(dy));
      }
    }
#pragma unroll
    for (int j = 0; j < KU; ++j) {
      const float sj = reduce(part[j]);
      if (lane == 0) El::store1(dW, t * k + j, ok[j] ? sj : 0.0f);
    }
  } else {
    for (int j = 0; j < k; ++j) {
      const int32_t r = __shfl(my_row, j, 64);
      const float wj = __shfl(my_w, j, 64);
      const bool ok = r < r_valid;
      float part = 0.0f;
      if (ok) {
        for (int c = lane; c < chunks; c += 64) {
          const u32x4 g = ld16(drow + (int64_t)c * 16);
          const u32x4 y = ld16(Y + ((int64_t)r * H + (int64_t)c * P) * ESZ);
          float dy[P];
#pragma unroll
          for (int q = 0; q < P; ++q) {
            const float gq = El::get(g, q);
            part += El::mul(gq, El::get(y, q));
            dy[q] = El::mul(gq, wj);
          }
          st16(dY + ((int64_t)r * H + (int64_t)c * P) * ESZ, El::pack(dy));
        }
      }
      const float sj = reduce(part);  // every lane takes part: the shuffles need the whole wave
      if (lane == 0) El::store1(dW, t * k + j, ok ? sj : 0.0f);
    }
  }
}

template <int DT>
void launch_combine_bwd(void* stream, const char* dout, const char* Y, const int32_t* slot_to_row, const void* wts,
                        const int32_t* offs, int64_t T, int k, int64_t H, int E, char* dY, void* dW) {
  dim3 grid((unsigned)((T + kBwdWaves - 1) / kBwdWaves)), block(kBwdWaves * 64);
  hipStream_t s = (hipStream_t)stream;
  if (k == 8)
    hipLaunchKernelGGL((combine_bwd_kernel<DT, 8>), grid, block, 0, s, dout, Y, slot_to_row, wts, offs, T, k, H, E, dY, dW);
  else if (k == 2)
    hipLaunchKernelGGL((combine_bwd_kernel<DT, 2>), grid, block, 0, s, dout, Y, slot_to_row, wts, offs, T, k, H, E, dY, dW);
  else if (k == 4)
    hipLaunchKernelGGL((combine_bwd_kernel<DT, 4>), grid, block, 0, s, dout, Y, slot_to_row, wts, offs, T, k, H, E, dY, dW);
  else
    hipLaunchKernelGGL((combine_bwd_kernel<DT, 0>), grid, block, 0, s, dout, Y, slot_to_row, wts, offs, T, k, H, E, dY, dW);
}

template <int DT>
void launch_combine(dim3 grid, dim3 block, void* stream, const char* Y, const int32_t* slot_to_row, const void* wts,
                    const int32_t* offs, int64_t T, int k, int64_t H, int E, char* O) {
  if (k == 8)
    hipLaunchKernelGGL((combine_kernel<DT, 8>), grid, block, 0, (hipStream_t)stream, Y, slot_to_row, wts, offs, T, k, H,
                       E, O);
  else if (k == 2)
    hipLaunchKernelGGL((combine_kernel<DT, 2>), grid, block, 0, (hipStream_t)stream, Y, slot_to_row, wts, offs, T, k, H,
                       E, O);
  else if (k == 4)
    hipLaunchKernelGGL((combine_kernel<DT, 4>), grid, block, 0, (hipStream_t)stream, Y, slot_to_row, wts, offs, T, k, H,
                       E, O);
  else
    hipLaunchKernelGGL((combine_kernel<DT, 0>), grid, block, 0, (hipStream_t)stream, Y, slot_to_row, wts, offs, T, k, H,
                       E, O);
}

// Down projection and combine in one launch for one or two tokens (at most
// 16 routed rows, where the down GEMM only streams each touched expert's
// weights once).  Workgroup (column pair cb, token t) computes, for each of
// t's k <= 8 slots, y = round(act[row] . W_dn[e][c]) for columns c0, c0 + 1,
// then applies the combine's arithmetic: round(y * w) per slot, summed in
// fp32 in ascending row order and rounded once (combine_kernel's order).
// Slots whose row lies past the valid rows contribute nothing.  Workgroups
// never exchange data, so one launch replaces the down GEMM and the combine.
// The dot products follow the skinny down GEMM (mgemm_skinny_kernel) step for
// step, so at the sizes that kernel serves the output is bit-identical to the
// two launches: the 16 weight rows (slot s = row / 2, column c0 + row % 2) are
// the A operand of v_mfma_f32_16x16x32, the slots' act rows the B operand
// (lane l: row / column l % 16, k = 8 (l / 16) .. +7), the 4 waves take K
// quarters of 32-wide chunks in order, and their partial sums are added in
// wave order.  D[row][s] for slot s's two rows lands in lane 16 (s / 2) + s.
// Index loads are clamped to valid slots and the operand loads to row 0 /
// expert 0, so every load is in bounds and issued unconditionally (one round
// trip for the indices, one for the operands); dead slots are zeroed after.
template <typename TR>
__global__ __launch_bounds__(256) void down_combine_decode_kernel(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ W, const int32_t* __restrict__ slot_to_row,
    const int64_t* __restrict__ topk_idx, const uint16_t* __restrict__ wts, const int32_t* __restrict__ expert_offsets,
    int k, int H, int I, int E, uint16_t* __restrict__ out) {
  __shared__ floatx4 red[4][64];
  __shared__ int32_t s_row[8];
  __shared__ float s_p[8][2];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.y;
  const int c0 = blockIdx.x * 2;
  const int64_t tk = (int64_t)t * k;
  const int32_t r_valid = expert_offsets[E];
  // B operand: column l % 16 = slot sb's act row; A operand: weight row
  // l % 16 = slot sa's column c0 + l % 2 (the three index loads go out together)
  const int sb = lane & 15;
  const int sa = (lane & 15) >> 1;
  const int32_t rb = slot_to_row[tk + (sb < k ? sb : k - 1)];
  const int32_t ra = slot_to_row[tk + (sa < k ? sa : k - 1)];
  const int64_t ea = topk_idx[tk + (sa < k ? sa : k - 1)];
  const bool live_b = sb < k && rb >= 0 && rb < r_valid;
  const bool live_a = sa < k && ra >= 0 && ra < r_valid && ea >= 0 && ea < E;
  const uint16_t* wa = W + ((int64_t)(live_a ? ea : 0) * H + c0 + (lane & 1)) * I + (lane >> 4) * 8;
  const uint16_t* xb = act + (int64_t)(live_b ? rb : 0) * I + (lane >> 4) * 8;
  const int nc = I / 32;
  const int kc0 = wave * nc / 4, kc1 = (wave + 1) * nc / 4;
  // chunks past the wave's range (or all four, when I < 128 leaves it none)
  // reload a valid one and skip its MFMA: no branch separates the index loads
  // from the operand loads
  const int kc_hi = kc1 > kc0 ? kc1 - 1 : kc0;
  u32x4 a[4], b[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int kk = (kc0 + u < kc_hi ? kc0 + u : kc_hi) * 32;
    a[u] = ld16(wa + kk);
    b[u] = ld16(xb + kk);
  }
  const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (kc0 + u < kc1) acc = TR::mfma16(live_a ? a[u] : zero, live_b ? b[u] : zero, acc);
  red[wave][lane] = acc;
  if (wave == 0 && lane < 8) s_row[lane] = live_b ? rb : 0x7fffffff;  // lane < 8: sb = lane
  __syncthreads();
  // slot sb's columns c0, c0 + 1 are D rows 2 sb, 2 sb + 1: lane 16 (sb / 2) + sb, v = 2 (sb % 2) + 0, 1
  if (wave == 0 && sb == 2 * (lane >> 4) + (sb & 1) && live_b) {
    floatx4 g = red[0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) g += red[w][lane];
    int rank = 0;
    for (int v = 0; v < k; ++v) rank += s_row[v] < rb ? 1 : 0;
    const float w = TR::to_f(wts[tk + sb]);
    const int v0 = 2 * (sb & 1);
    s_p[rank][0] = TR::to_f(TR::from_f(TR::to_f(TR::from_f(g[v0])) * w));
    s_p[rank][1] = TR::to_f(TR::from_f(TR::to_f(TR::from_f(g[v0 + 1])) * w));
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    int n_live = 0;
    for (int v = 0; v < k; ++v) n_live += s_row[v] != 0x7fffffff ? 1 : 0;
    float o = 0.0f;
    for (int r = 0; r < n_live; ++r) o += s_p[r][threadIdx.x];
    out[(int64_t)t * H + c0 + threadIdx.x] = TR::from_f(o);
  }
}

}  // namespace
}  // namespace hrm

extern "C" int hrm_moe_combine(const void* expert_out, const int32_t* slot_to_row, const void* topk_weight,
                               const int32_t* expert_offsets, int64_t num_tokens, int32_t top_k, int64_t hidden_size,
                               int32_t num_experts, int dtype, void* out, void* stream) {
  if (num_tokens < 0 || top_k < 1 || hidden_size < 1 || num_experts < 1) return HRM_MOE_ERR_INVALID;
  if (dtype < HRM_MOE_BF16 || dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (top_k > hrm::kMaxTopK || hidden_size % 8) return HRM_MOE_ERR_UNSUPPORTED;
  if (num_tokens == 0) return HRM_MOE_OK;
  if (!expert_out || !slot_to_row || !expert_offsets || !out) return HRM_MOE_ERR_INVALID;  // weights may be NULL
  if (hidden_size / 8 > (int64_t(1) << 27)) return HRM_MOE_ERR_UNSUPPORTED;  // items per block fit an int
  // Column slices: enough for about 1024 blocks, but no more than one pass of
  // the block's threads over its items needs (T = 8 at H = 1536: 4 token
  // blocks of 2 slices; with 8 tokens per block that was 6 dependent load
  // rounds in a single block).
  const int64_t tok_blocks = (num_tokens + hrm::kTokPerBlock - 1) / hrm::kTokPerBlock;
  const int64_t items = hrm::kTokPerBlock * (hidden_size / (dtype == HRM_MOE_F32 ? 4 : 8));
  int64_t slices = (items + hrm::kBlock - 1) / hrm::kBlock;
  const int64_t want = (1024 + tok_blocks - 1) / tok_blocks;
  slices = slices < want ? slices : want;
  slices = slices < 1 ? 1 : slices;
  // threads: one per item of a block's slice, so no second pass with one busy
  // wave in four (L, H = 1280: 2 tokens x 160 chunks = 320 threads; combine
  // 67.8 -> 65.9 us; XL, H = 1536: 80.9 -> 78.3 us)
  const int64_t slice_items = hrm::kTokPerBlock * ((items / hrm::kTokPerBlock + slices - 1) / slices);
  int64_t threads = (slice_items + 63) / 64 * 64;
  threads = threads < hrm::kBlock ? hrm::kBlock : (threads > hrm::kMaxBlock ? hrm::kMaxBlock : threads);
  dim3 grid((unsigned)tok_blocks, (unsigned)slices), block((unsigned)threads);
  const char* Y = static_cast<const char*>(expert_out);
  char* O = static_cast<char*>(out);
  if (dtype == HRM_MOE_BF16)
    hrm::launch_combine<HRM_MOE_BF16>(grid, block, stream, Y, slot_to_row, topk_weight, expert_offsets, num_tokens,
                                      top_k, hidden_size, num_experts, O);
  else if (dtype == HRM_MOE_F16)
    hrm::launch_combine<HRM_MOE_F16>(grid, block, stream, Y, slot_to_row, topk_weight, expert_offsets, num_tokens,
                                     top_k, hidden_size, num_experts, O);
  else
    hrm::launch_combine<HRM_MOE_F32>(grid, block, stream, Y, slot_to_row, topk_weight, expert_offsets, num_tokens,
                                     top_k, hidden_size, num_experts, O);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  return HRM_MOE_OK;
}

extern "C" int hrm_moe_combine_backward(const void* grad_out, const void* expert_out, const int32_t* slot_to_row,
                                        const void* topk_weight, const int32_t* expert_offsets, int64_t num_tokens,
                                        int32_t top_k, int64_t hidden_size, int32_t num_experts, int dtype,
                                        void* grad_expert_out, void* grad_weight, void* stream) {
  if (num_tokens < 0 || top_k < 1 || hidden_size < 1 || num_experts < 1) return HRM_MOE_ERR_INVALID;
  if (dtype < HRM_MOE_BF16 || dtype > HRM_MOE_F32) return HRM_MOE_ERR_DTYPE;
  if (top_k > hrm::kMaxTopK || hidden_size % 8 || hidden_size / 8 > (int64_t(1) << 27)) return HRM_MOE_ERR_UNSUPPORTED;
  if (num_tokens == 0) return HRM_MOE_OK;
  if (!grad_out || !expert_out || !slot_to_row || !topk_weight || !expert_offsets || !grad_expert_out || !grad_weight)
    return HRM_MOE_ERR_INVALID;
  const char* G = static_cast<const char*>(grad_out);
  const char* Y = static_cast<const char*>(expert_out);
  char* DY = static_cast<char*>(grad_expert_out);
  if (dtype == HRM_MOE_BF16)
    hrm::launch_combine_bwd<HRM_MOE_BF16>(stream, G, Y, slot_to_row, topk_weight, expert_offsets, num_tokens, top_k,
                                          hidden_size, num_experts, DY, grad_weight);
  else if (dtype == HRM_MOE_F16)
    hrm::launch_combine_bwd<HRM_MOE_F16>(stream, G, Y, slot_to_row, topk_weight, expert_offsets, num_tokens, top_k,
                                         hidden_size, num_experts, DY, grad_weight);
  else
    hrm::launch_combine_bwd<HRM_MOE_F32>(stream, G, Y, slot_to_row, topk_weight, expert_offsets, num_tokens, top_k,
                                         hidden_size, num_experts, DY, grad_weight);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  return HRM_MOE_OK;
}

extern "C" int hrm_moe_down_combine_decode(const void* act, const void* down_weight, const int32_t* slot_to_row,
                                           const int64_t* topk_idx, const void* topk_weight,
                                           const int32_t* expert_offsets, int64_t num_tokens, int32_t top_k,
                                           int64_t hidden_size, int64_t inter_size, int32_t num_experts, int dtype,
                                           void* out, void* stream) {
  if (num_tokens < 0 || top_k < 1 || hidden_size < 1 || inter_size < 1 || num_experts < 1) return HRM_MOE_ERR_INVALID;
  if (dtype != HRM_MOE_BF16 && dtype != HRM_MOE_F16) return HRM_MOE_ERR_DTYPE;
  if (num_tokens > 2 || top_k > 8 || hidden_size % 2 || inter_size % 32 || inter_size > 512 ||
      hidden_size > (int64_t(1) << 24))
    return HRM_MOE_ERR_UNSUPPORTED;
  if (num_tokens == 0) return HRM_MOE_OK;
  if (!act || !down_weight || !slot_to_row || !topk_idx || !topk_weight || !expert_offsets || !out)
    return HRM_MOE_ERR_INVALID;
  const dim3 grid((unsigned)(hidden_size / 2), (unsigned)num_tokens), block(256);
#define HRM_DC(TR_)                                                                                                  \
  HRM_LAUNCH(hrm::down_combine_decode_kernel<TR_>, grid, block, 0, stream, (const uint16_t*)act,                     \
             (const uint16_t*)down_weight, slot_to_row, topk_idx, (const uint16_t*)topk_weight, expert_offsets, top_k, \
             (int)hidden_size, (int)inter_size, num_experts, (uint16_t*)out)
  if (dtype == HRM_MOE_BF16) HRM_DC(hrm::BF16);
  else HRM_DC(hrm::F16);
#undef HRM_DC
  return HRM_MOE_OK;
}
