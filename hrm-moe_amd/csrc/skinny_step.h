// The weight-streaming step of the decode-size grouped GEMM, shared by
// mgemm_skinny_kernel (grouped_gemm.hip) and router_gate_up_decode_kernel
// (decode.hip), so the two give the same bits by construction.
//
// A workgroup of 4 waves computes 16 output columns for up to 16 NRB rows of
// one expert with v_mfma_f32_16x16x32: the 16 weight rows are the MFMA A
// operand and the rows the B operand, both loaded from global memory straight
// into the operand layout (lane l: row l % 16, k = 8 (l / 16) .. +7, 16
// contiguous bytes).  The 4 waves split K into quarters of 32-wide chunks;
// their partial sums are added in wave order.
#pragma once
#include "common.h"

namespace hrm {

// All of a wave's 32-wide K chunks [kc0, kc1) (at most CPW) of the weight rows
// (wg, and wu for the up half of a gate/up pair) and of the NRB 16-row blocks
// (xr) are loaded at once (load), then the MFMAs run in K order, each waiting
// only for its own chunk (mma).  Slots past kc1 reload the wave's last chunk
// and skip their MFMA, so every load is in bounds and issued unconditionally.
// A caller may do other work between the two while the loads are in flight.
template <typename TR, bool SW, int NRB, int CPW>
struct SkinnyChunks {
  u32x4 bg[CPW], bu[CPW], bx[CPW][NRB];

  __device__ __forceinline__ void load(const uint16_t* wg, const uint16_t* wu, const uint16_t* const (&xr)[NRB],
                                       int kc0, int kc1) {
    if (kc1 <= kc0) return;
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int k = (kc0 + u < kc1 ? kc0 + u : kc1 - 1) * 32;
      bg[u] = ld16(wg + k);
      if constexpr (SW) bu[u] = ld16(wu + k);
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) bx[u][rb] = ld16(xr[rb] + k);
    }
  }

  __device__ __forceinline__ void mma(int kc0, int kc1, floatx4 (&ag)[NRB], floatx4 (&au)[NRB]) const {
    if (kc1 <= kc0) return;
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      if (kc0 + u < kc1) {
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
          ag[rb] = TR::mfma16(bg[u], bx[u][rb], ag[rb]);
          if constexpr (SW) au[rb] = TR::mfma16(bu[u], bx[u][rb], au[rb]);
        }
      }
    }
  }
};

template <typename TR, bool SW, int NRB, int CPW>
__device__ __forceinline__ void skinny_chunks(const uint16_t* wg, const uint16_t* wu, const uint16_t* const (&xr)[NRB],
                                              int kc0, int kc1, floatx4 (&ag)[NRB], floatx4 (&au)[NRB]) {
  SkinnyChunks<TR, SW, NRB, CPW> c;
  c.load(wg, wu, xr, kc0, kc1);
  c.mma(kc0, kc1, ag, au);
}

// Partial sums of the 4 waves, [wave][row block][gate, up][lane].
template <bool SW, int NRB>
using SkinnyRed = floatx4[4][NRB][SW ? 2 : 1][64];

template <bool SW, int NRB>
__device__ __forceinline__ void skinny_publish(SkinnyRed<SW, NRB>& red, int wave, int lane,
                                               const floatx4 (&ag)[NRB], const floatx4 (&au)[NRB]) {
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    red[wave][rb][0][lane] = ag[rb];
    if constexpr (SW) red[wave][rb][1][lane] = au[rb];
  }
}

// After a barrier behind skinny_publish: wave rb < NRB adds the 4 K quarters of
// row block rb in wave order and stores its rows [row0 + 16 rb, + 16) below
// row_end of columns [c0, c0 + 16) of C [*, N] (SwiGLU of the gate/up pair
// for SW, with the reference's rounding points).  The MFMA result layout puts
// columns c0 + 4 (l / 16) + v of row l % 16 in lane l.
template <typename TR, bool SW, int NRB>
__device__ __forceinline__ void skinny_store(const SkinnyRed<SW, NRB>& red, int wave, int lane, int row0, int row_end,
                                             uint16_t* __restrict__ C, int N, int c0) {
  if (wave >= NRB) return;
  const int rb = wave;
  floatx4 g = red[0][rb][0][lane], u = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (SW) u = red[0][rb][1][lane];
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    g += red[w][rb][0][lane];
    if constexpr (SW) u += red[w][rb][1][lane];
  }
  const int r = row0 + rb * 16 + (lane & 15);
  if (r < row_end) {
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) o[v] = SW ? swiglu_fast<TR>(g[v], u[v]) : g[v];
    st8(C + (int64_t)r * N + c0 + (lane >> 4) * 4, pack4<TR>(o[0], o[1], o[2], o[3]));
  }
}

}  // namespace hrm
