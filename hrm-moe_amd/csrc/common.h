// Shared device types and helpers for the gfx950 MoE kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hrm_moe.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define HRM_LDS __attribute__((address_space(3)))

namespace hrm {

constexpr int kWave = 64;

// 16-bit element types the GEMMs accept.  Storage is raw 16-bit; the traits
// give the MFMA and the conversions.
struct BF16 {
  static __device__ __forceinline__ float to_f(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }
  static __device__ __forceinline__ uint16_t from_f(float f) {
    __bf16 b = static_cast<__bf16>(f);  // round to nearest even (v_cvt_pk_bf16_f32)
    return __builtin_bit_cast(uint16_t, b);
  }
  static __device__ __forceinline__ floatx16 mfma32(u32x4 a, u32x4 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ floatx4 mfma16(u32x4 a, u32x4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

struct F16 {
  static __device__ __forceinline__ float to_f(uint16_t v) { return float(__builtin_bit_cast(_Float16, v)); }
  static __device__ __forceinline__ uint16_t from_f(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }
  static __device__ __forceinline__ floatx16 mfma32(u32x4 a, u32x4 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(halfx8, a), __builtin_bit_cast(halfx8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ floatx4 mfma16(u32x4 a, u32x4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(halfx8, a), __builtin_bit_cast(halfx8, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) { return uint32_t(lo) | (uint32_t(hi) << 16); }

// 16-byte global load / store helpers (addresses must be 16-byte aligned).
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

template <typename TR>
__device__ __forceinline__ u32x2 pack4(float a, float b, float c, float d) {
  return u32x2{pack2(TR::from_f(a), TR::from_f(b)), pack2(TR::from_f(c), TR::from_f(d))};
}

// silu(gate) * up with the reference's rounding points (gate, up, silu and the
// product each rounded to the element type), using the hardware exp2 and
// reciprocal; it stays within one rounding of torch's expf / IEEE-divide silu.
template <typename TR>
__device__ __forceinline__ float swiglu_fast(float g, float u) {
  const float gr = TR::to_f(TR::from_f(g));
  const float ur = TR::to_f(TR::from_f(u));
  const float e = __builtin_amdgcn_exp2f(-gr * 1.4426950408889634f);
  const float sl = TR::to_f(TR::from_f(gr * __builtin_amdgcn_rcpf(1.0f + e)));
  return sl * ur;
}

inline int ceil_div(int64_t a, int64_t b) { return int((a + b - 1) / b); }

// Tuning knobs of the library, read from the environment on first use and
// again by hrm_moe_reload_config().  Launchers read this snapshot, never the
// environment itself.  Reloading while another thread launches is not safe.
struct Config {
  int cu_margin = 0;         // CUs left out of persistent grids (HRM_MOE_HIP_CU_MARGIN,
                             // else HRM_MOE_TRITON_SM_MARGIN, else XTUNER_SM_MARGIN)
  int gemm_bm = 0, gemm_bn = 0, gemm_stages = 0, gemm_waves = 4, gemm_bk = 64;  // HRM_MOE_GEMM_CFG, 0 = per call
  int skinny = -1;           // HRM_MOE_SKINNY: -1 automatic, 0 off, 1 forced up to 16 rows per expert
  int wgrad_stages = 0;      // HRM_MOE_WGRAD_STAGES: 0 automatic, 2 or 3 = 128 x 128 kernel with that ring
  int64_t gate_split_rows = 1024;  // HRM_MOE_GATE_SPLIT_ROWS: rows per split of the gate weight gradient
  bool wave_router = true;   // HRM_MOE_WAVE_ROUTER=0 turns the one-wave-per-token decode router off
};
const Config& config();
// Re-reads the environment; returns HRM_MOE_OK, or HRM_MOE_ERR_INVALID when a
// value is malformed (that knob then keeps its default).
int reload_config();

// Records the kernel instantiation the latest launch of a GEMM kind used
// (0 NT, 1 gate/up, 2 NN), read back by hrm_moe_last_gemm_kernel; kernels
// outside grouped_gemm.hip that do a kind's work record themselves here.
void set_last_gemm_kernel(int kind, const char* name);

// Second dispatch stage (permute.hip), after a rank step that wrote rank[R] and
// counts[nb][E+1] for rank blocks of SB slots: one scan + scatter launch.
int dispatch_from_ranks(const int64_t* topk_idx, int64_t R, int E, int k, int SB, int nb, const int32_t* rank,
                        const int32_t* counts, int64_t* tokens_per_expert, int32_t* expert_offsets,
                        int32_t* sorted_token_idx, int64_t* sort_idx, int32_t* slot_to_row, void* stream);

}  // namespace hrm

// Launch helper: returns the launch status as an int.
#define HRM_LAUNCH(kernel, grid, block, shmem, stream, ...)                                   \
  do {                                                                                          \
    hipLaunchKernelGGL(kernel, grid, block, shmem, (hipStream_t)(stream), __VA_ARGS__);         \
    hipError_t e_ = hipGetLastError();                                                          \
    if (e_ != hipSuccess) return int(e_);                                                       \
  } while (0)
