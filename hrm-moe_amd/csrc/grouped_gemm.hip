// Grouped GEMMs over expert-contiguous rows, for gfx950 MFMA.
//
// Replaces the reference's Triton kernels (models/moe_triton_grouped_gemm.py):
//   _m_grouped_gemm_bk_kernel :113-184  -> KIND_NT       (C = A . W[e]^T)
//   _m_grouped_gemm_bn_kernel :187-260  -> KIND_NN       (C = A . W[e], dgrad)
//   _k_grouped_gemm_kernel    :277-347  -> wgrad kernel  (C[e] = A_e^T . B_e)
//   _repeat_interleave_kernel :263-274  -> plan kernel   (tile table on device)
// plus KIND_GATHER_SWIGLU, which fuses the row gather and the SwiGLU of
// models/layers.py:320,326-329 into the gate_up GEMM.
//
// Work decomposition
//  * A plan kernel turns tokens_per_expert (device int64) into a table of
//    M-tiles {expert, first row, end row}, so nothing is read on the host.
//  * M-grouped kernels are persistent.  Workgroup w runs on XCD w % 8, and
//    each XCD owns one contiguous eighth of the tile list (M-tile major,
//    N-tile minor), so an expert's weights stay in one XCD's L2.
//  * A workgroup is 4 waves (2 x 2).  It computes a BM x BN tile; each wave owns
//    (BM/2) x (BN/2) as 32x32 MFMA blocks of v_mfma_f32_32x32x16_{bf16,f16}.
//    Operand roles are swapped (W rows feed the MFMA A operand) so each lane
//    ends with four consecutive output columns and stores 8 bytes.
//  * K is consumed 64 at a time through a ring of LDS stages.  Row-major
//    K-contiguous tiles are stored as [rows][64] with a swizzled 16-byte chunk
//    index (kc_swz).  K-strided tiles (dgrad's W, both wgrad operands) are
//    stored as [k][cols] (kr_swz) and read with ds_read_b64_tr_b16, which
//    transposes 4x16 blocks of 16-bit values inside each 16-lane group.
#include <stdio.h>
#include <type_traits>
#include <stdlib.h>

#include "common.h"
#include "skinny_step.h"

namespace hrm {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 64;
constexpr int kMaxExperts = 1024;

enum { KIND_NT = 0, KIND_GATHER_SWIGLU = 1, KIND_NN = 2 };
// Epilogue modes of the DMA kernels (training path):
//   EPI_PLAIN       store C
//   EPI_SAVE_GU     gate/up kernel: also store the rounded gate and up values
//                   (the reference's gate_up tensor, models/layers.py:326) to aux [M, 2N]
//   EPI_SWIGLU_BWD  NN kernel computing dAct = dY . W_dn[e]: apply the backward of
//                   silu(gate) * up (models/layers.py:328-329) with gate/up read from
//                   aux [M, 2N] and store d(gate_up) [M, 2N] to C
enum { EPI_PLAIN = 0, EPI_SAVE_GU = 1, EPI_SWIGLU_BWD = 2 };

struct MTile {
  int32_t expert, row_start, row_end, pad;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// ---------------------------------------------------------------------------
// Plan: tile table from tokens_per_expert
// ---------------------------------------------------------------------------
// Writes tiles[0..count) and count, plus row_offsets[0..E] (exclusive prefix of
// clamped counts).  Rows are clamped to [0, M): a tokens_per_expert that sums
// past M never makes a kernel touch rows >= M.  Also zeroes the work counter.
__global__ __launch_bounds__(1024) void plan_kernel(const int64_t* __restrict__ tpe, int E, int64_t M, int BM,
                                                    MTile* __restrict__ tiles, int max_tiles, int* __restrict__ count,
                                                    int* __restrict__ row_offsets, int* __restrict__ work_counter) {
  __shared__ int64_t s_rows[kMaxExperts + 1];
  __shared__ int s_ntile[kMaxExperts + 1];
  __shared__ int s_rs[kMaxExperts];
  __shared__ int s_re[kMaxExperts];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += blockDim.x) {
    int64_t n = tpe[e];
    s_rows[e] = n > 0 ? n : 0;
  }
  __syncthreads();
  // Inclusive Hillis-Steele scan of row counts over E <= 1024 entries.
  for (int off = 1; off < E; off *= 2) {
    int64_t v = 0;
    if (tid < E && tid >= off) v = s_rows[tid - off];
    __syncthreads();
    if (tid < E && tid >= off) s_rows[tid] += v;
    __syncthreads();
  }
  if (tid < E) {
    const int64_t end = s_rows[tid];
    const int64_t n = tid == 0 ? end : end - s_rows[tid - 1];
    int64_t rs = end - n, re = end;
    rs = rs < M ? rs : M;
    re = re < M ? re : M;
    s_rs[tid] = (int)rs;
    s_re[tid] = (int)re;
    s_ntile[tid] = (int)((re - rs + BM - 1) / BM);
    row_offsets[tid] = (int)rs;
    if (tid == E - 1) row_offsets[E] = (int)re;
  }
  __syncthreads();
  for (int off = 1; off < E; off *= 2) {
    int v = 0;
    if (tid < E && tid >= off) v = s_ntile[tid - off];
    __syncthreads();
    if (tid < E && tid >= off) s_ntile[tid] += v;
    __syncthreads();
  }
  int total = s_ntile[E - 1];
  total = total < max_tiles ? total : max_tiles;
  for (int i = tid; i < total; i += blockDim.x) {
    int lo = 0, hi = E - 1;  // first e with inclusive prefix > i
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_ntile[mid] > i) hi = mid; else lo = mid + 1;
    }
    const int before = lo == 0 ? 0 : s_ntile[lo - 1];
    const int j = i - before;
    MTile t;
    t.expert = lo;
    t.row_start = s_rs[lo] + j * BM;
    const int e2 = t.row_start + BM;
    t.row_end = e2 < s_re[lo] ? e2 : s_re[lo];
    t.pad = 0;
    tiles[i] = t;
  }
  if (tid == 0) *count = total;
  if (tid < 8) work_counter[tid] = 0;  // one work counter per XCD
}

struct GemmWs {
  MTile* tiles;
  int* count;
  int* row_offsets;
  int* work_counter;
};

// work_counter points at 8 ints (one per XCD) inside the 256-byte counter block.
inline size_t gemm_ws_bytes(int64_t M, int E, int bm_min) {
  const int64_t max_tiles = (M + bm_min - 1) / bm_min + E;
  return align256(sizeof(MTile) * (size_t)max_tiles) + align256(sizeof(int) * 4) + align256(sizeof(int) * (E + 1));
}

inline GemmWs carve(void* ws, int64_t M, int E, int bm_min) {
  const int64_t max_tiles = (M + bm_min - 1) / bm_min + E;
  char* p = static_cast<char*>(ws);
  GemmWs w;
  w.tiles = reinterpret_cast<MTile*>(p);
  p += align256(sizeof(MTile) * (size_t)max_tiles);
  w.count = reinterpret_cast<int*>(p);
  w.work_counter = w.count + 1;
  p += align256(sizeof(int) * 4);
  w.row_offsets = reinterpret_cast<int*>(p);
  return w;
}

// ---------------------------------------------------------------------------
// LDS addressing
// ---------------------------------------------------------------------------
// LDS serves 64 four-byte banks (256 bytes) per cycle.  The swizzles below
// make the MFMA operand reads conflict-free under that model.
// [rows][64] tile, K contiguous: 128 B per row; 16-byte chunk c of row r sits
// at chunk c ^ ((r >> 1) & 7).  A ds_read_b128 of 16 consecutive rows at one
// logical chunk then covers 16 distinct (row parity, chunk) bank groups.
__device__ __forceinline__ int kc_swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ uint32_t kc_off(int row, int chunk) { return uint32_t(row * 128 + ((chunk ^ kc_swz(row)) << 4)); }
// The same layout for K slices of other widths: rows of PITCH bytes (64 or
// 128), chunk index XOR (row / rows-per-256-bytes) mod chunks-per-row.  Each
// group of 16 lanes reading one chunk column of 16 consecutive rows then
// covers 256 contiguous bytes, all 64 banks once.
template <int PITCH>
__device__ __forceinline__ int kcp_swz(int row) { return (row / (256 / PITCH)) % (PITCH / 16); }
template <int PITCH>
__device__ __forceinline__ uint32_t kcp_off(int row, int chunk) {
  return uint32_t(row * PITCH + ((chunk ^ kcp_swz<PITCH>(row)) << 4));
}
// [64 k][COLS] tile, columns contiguous: 16-byte chunk c of row k sits at
// chunk c ^ ((k & 3) << 2).  A transpose read covers 4 rows x 4 chunks per
// 32 lanes; the XOR spreads the 4 rows over distinct quarters of the bank space.
__device__ __forceinline__ int kr_swz(int k) { return (k & 3) << 2; }
template <int COLS>
__device__ __forceinline__ uint32_t kr_off(int k, int chunk) { return uint32_t(k * (COLS * 2) + ((chunk ^ kr_swz(k)) << 4)); }

// LDS pointers are plain pointers into __shared__ arrays; the compiler infers
// the LDS address space.  The transpose load takes an explicit LDS pointer.
__device__ __forceinline__ u32x4 lds_read16(const char* base, uint32_t off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}
__device__ __forceinline__ void lds_write16(char* base, uint32_t off, u32x4 v) {
  *reinterpret_cast<u32x4*>(base + off) = v;
}
__device__ __forceinline__ u32x2 lds_read_tr16(const char* base, uint32_t off) {
  shortx4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((HRM_LDS shortx4*)(base + off));
  return __builtin_bit_cast(u32x2, v);
}

// MFMA operand (8 values along the reduction) for output index i = l % 32 of a
// 32-wide block whose columns start at col0, from a [64 k][COLS] tile, at
// reduction sub-step s (16 values).  Lane l of 16-lane group g reads row
// k = s*16 + (g>>1)*8 + kk + (i>>2), columns col0 + (g&1)*16 + 4*(i&3) .. +3;
// the transpose hands lane j of the group column col0 + (g&1)*16 + j.
template <int COLS>
__device__ __forceinline__ u32x4 tr_operand(const char* base, int col0, int s, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int col = col0 + (g & 1) * 16 + 4 * (i & 3);
  const int kb = s * 16 + (g >> 1) * 8 + (i >> 2);
  const uint32_t o0 = kr_off<COLS>(kb, col >> 3) + (col & 7) * 2;
  const uint32_t o1 = kr_off<COLS>(kb + 4, col >> 3) + (col & 7) * 2;
  const u32x2 lo = lds_read_tr16(base, o0);
  const u32x2 hi = lds_read_tr16(base, o1);
  return u32x4{lo.x, lo.y, hi.x, hi.y};
}

// silu(gate) * up with the reference's roundings: gate, up, silu(gate) and the
// product are each rounded to the element type (models/layers.py:328-329 on
// 16-bit tensors; torch's silu computes x / (1 + exp(-x)) in fp32).
template <typename TR>
__device__ __forceinline__ float swiglu_ref(float g, float u) {
  const float gr = TR::to_f(TR::from_f(g));
  const float ur = TR::to_f(TR::from_f(u));
  const float s = TR::to_f(TR::from_f(gr / (1.0f + expf(-gr))));
  return s * ur;
}

// ---------------------------------------------------------------------------
// M-grouped GEMM (persistent)
// ---------------------------------------------------------------------------
// KIND_NT:            C[M,N]  = A[M,K] . W[e][N,K]^T
// KIND_GATHER_SWIGLU: C[M,I]  = swiglu(A[gather[m]] . W[e][2I,K]^T), N = I
// KIND_NN:            C[M,N]  = A[M,K] . W[e][K,N]
template <typename TR, int KIND, int BM, int BN>
__global__ __launch_bounds__(kThreads, 1) void mgemm_kernel(const uint16_t* __restrict__ A,
                                                           const int32_t* __restrict__ gather,
                                                           const uint16_t* __restrict__ W, uint16_t* __restrict__ C,
                                                           const MTile* __restrict__ tiles,
                                                           const int* __restrict__ tile_count, int N, int K,
                                                           int tiles_n) {
  constexpr int MB = BM / 64;  // 32-row blocks per wave
  constexpr int NB = BN / 64;  // 32-col blocks per wave
  constexpr int A_BYTES = BM * kBK * 2;
  constexpr int B_BYTES = BN * kBK * 2;
  constexpr int A_LOADS = BM / 32;                       // 16-byte loads per thread per stage
  constexpr int B_LOADS = KIND == KIND_NN ? 4 : BN / 32;  // NN: 64 k-rows x BN/8 chunks
  static_assert(KIND != KIND_NN || BN == 128, "NN tile loader assumes BN == 128");
  __shared__ __attribute__((aligned(16))) char smem[2 * (A_BYTES + B_BYTES)];
  char* lds = smem;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int total = (*tile_count) * tiles_n;
  const int xcd = blockIdx.x & 7;
  const int nloc = gridDim.x >> 3;
  const int chunk = (total + 7) >> 3;
  const int64_t w_rows = KIND == KIND_GATHER_SWIGLU ? 2 * (int64_t)N : (KIND == KIND_NN ? (int64_t)K : (int64_t)N);
  const int64_t w_cols = KIND == KIND_NN ? (int64_t)N : (int64_t)K;
  const int nk = (K + kBK - 1) / kBK;

  for (int j = blockIdx.x >> 3; j < chunk; j += nloc) {
    const int t = xcd * chunk + j;
    if (t >= total) break;
    const MTile ti = tiles[t / tiles_n];
    const int nt = t - (t / tiles_n) * tiles_n;
    const int rs = ti.row_start, re = ti.row_end;
    const uint16_t* Wexp = W + (int64_t)ti.expert * w_rows * w_cols;

    // ---- global source pointers for this tile
    const uint16_t* a_src[A_LOADS];
    const int ca = tid & 7;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      int r = rs + (tid >> 3) + 32 * i;
      r = r < re ? r : re - 1;
      const int64_t src = KIND == KIND_GATHER_SWIGLU ? (int64_t)gather[r] : (int64_t)r;
      a_src[i] = A + src * K + ca * 8;
    }
    const uint16_t* b_src[B_LOADS];
    int n0;
    if constexpr (KIND == KIND_NN) {
      n0 = nt * BN;
      int col = n0 + (tid & 15) * 8;
      col = col < N ? col : N - 8;
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) b_src[i] = Wexp + (int64_t)((tid >> 4) + 16 * i) * N + col;
    } else if constexpr (KIND == KIND_GATHER_SWIGLU) {
      n0 = nt * (BN / 2);  // first intermediate column of the tile
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) {
        const int jr = (tid >> 3) + 32 * i;  // 0..BN-1: first half gate rows, second half up rows
        int c = n0 + (jr % (BN / 2));
        c = c < N ? c : N - 1;
        const int64_t wr = jr < BN / 2 ? c : (int64_t)N + c;
        b_src[i] = Wexp + wr * K + ca * 8;
      }
    } else {
      n0 = nt * BN;
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) {
        int n = n0 + (tid >> 3) + 32 * i;
        n = n < N ? n : N - 1;
        b_src[i] = Wexp + (int64_t)n * K + ca * 8;
      }
    }

    u32x4 ra[A_LOADS], rb[B_LOADS];
    auto gload = [&](int kt) {
      const int k0 = kt * kBK;
      const bool ka_ok = k0 + ca * 8 < K;
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) ra[i] = ka_ok ? ld16(a_src[i] + k0) : u32x4{0, 0, 0, 0};
      if constexpr (KIND == KIND_NN) {
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
          const int kr = k0 + (tid >> 4) + 16 * i;
          rb[i] = kr < K ? ld16(b_src[i] + (int64_t)k0 * N) : u32x4{0, 0, 0, 0};
        }
      } else {
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) rb[i] = ka_ok ? ld16(b_src[i] + k0) : u32x4{0, 0, 0, 0};
      }
    };
    auto sstore = [&](int buf) {
      char* la = lds + buf * (A_BYTES + B_BYTES);
      char* lb = la + A_BYTES;
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) lds_write16(la, kc_off((tid >> 3) + 32 * i, ca), ra[i]);
      if constexpr (KIND == KIND_NN) {
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) lds_write16(lb, kr_off<BN>((tid >> 4) + 16 * i, tid & 15), rb[i]);
      } else {
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) lds_write16(lb, kc_off((tid >> 3) + 32 * i, ca), rb[i]);
      }
    };

    floatx16 acc[NB][MB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int a = 0; a < MB; ++a)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][a][v] = 0.0f;

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) gload(kt + 1);
      const char* la = lds + (kt & 1) * (A_BYTES + B_BYTES);
      const char* lb = la + A_BYTES;
#pragma unroll
      for (int s = 0; s < kBK / 16; ++s) {
        u32x4 fw[NB], fa[MB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          int r0;
          if constexpr (KIND == KIND_GATHER_SWIGLU) r0 = b * (BN / 2) + wn * 32;
          else r0 = wn * (BN / 2) + b * 32;
          if constexpr (KIND == KIND_NN) fw[b] = tr_operand<BN>(lb, r0, s, lane);
          else fw[b] = lds_read16(lb, kc_off(r0 + (lane & 31), s * 2 + (lane >> 5)));
        }
#pragma unroll
        for (int a = 0; a < MB; ++a) {
          const int r = wm * (BM / 2) + a * 32 + (lane & 31);
          fa[a] = lds_read16(la, kc_off(r, s * 2 + (lane >> 5)));
        }
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int a = 0; a < MB; ++a) acc[b][a] = TR::mfma32(fw[b], fa[a], acc[b][a]);
      }
      if (kt + 1 < nk) sstore((kt + 1) & 1);
      __syncthreads();
    }

    // ---- epilogue: lane holds rows m = base + (lane & 31), columns g*8 + (lane>>5)*4 + 0..3
#pragma unroll
    for (int a = 0; a < MB; ++a) {
      const int m = rs + wm * (BM / 2) + a * 32 + (lane & 31);
      if (m >= re) continue;
      if constexpr (KIND == KIND_GATHER_SWIGLU) {
        uint16_t* crow = C + (int64_t)m * N;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int c = n0 + wn * 32 + g * 8 + (lane >> 5) * 4;
          if (c < N) {
            float o[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = swiglu_ref<TR>(acc[0][a][g * 4 + q], acc[1][a][g * 4 + q]);
            st8(crow + c, pack4<TR>(o[0], o[1], o[2], o[3]));
          }
        }
      } else {
        uint16_t* crow = C + (int64_t)m * N;
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int c = n0 + wn * (BN / 2) + b * 32 + g * 8 + (lane >> 5) * 4;
            if (c < N)
              st8(crow + c, pack4<TR>(acc[b][a][g * 4 + 0], acc[b][a][g * 4 + 1], acc[b][a][g * 4 + 2],
                                      acc[b][a][g * 4 + 3]));
          }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Wgrad: C[e][Na,Nb] = A[rows_e]^T . B[rows_e]  (persistent, work queue)
// ---------------------------------------------------------------------------
// Output tile BA x BB (Na x Nb); reduction over the expert's rows, 64 at a
// time; both operands are [64 rows][cols] LDS tiles read with the transpose
// load.  MFMA A operand = B-tile (output columns nb, contiguous in C), MFMA B
// operand = A-tile (output rows na).
template <typename TR, int BA, int BB>
__global__ __launch_bounds__(kThreads, 1) void wgrad_kernel(const uint16_t* __restrict__ A,
                                                           const uint16_t* __restrict__ B, uint16_t* __restrict__ C,
                                                           const int* __restrict__ row_offsets, int E, int Na, int Nb,
                                                           int* __restrict__ work_counter) {
  static_assert(BA == 128 && BB == 128, "wgrad loader assumes 128 x 128 tiles");
  constexpr int MB = BA / 64, NB = BB / 64;
  constexpr int T_BYTES = kBK * 128 * 2;
  __shared__ __attribute__((aligned(16))) char smem[2 * 2 * T_BYTES];
  __shared__ int s_tile;
  char* lds = smem;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wa = wave >> 1, wb = wave & 1;
  const int ta_n = (Na + BA - 1) / BA, tb_n = (Nb + BB - 1) / BB;
  const int per_e = ta_n * tb_n;
  const int total = E * per_e;
  const int cc = tid & 15;  // 16-byte chunk within a 128-column row

  while (true) {
    if (tid == 0) s_tile = atomicAdd(work_counter, 1);
    __syncthreads();
    const int t = s_tile;
    __syncthreads();
    if (t >= total) break;
    const int e = t / per_e;
    const int rem = t - e * per_e;
    const int a0 = (rem / tb_n) * BA, b0 = (rem % tb_n) * BB;
    const int rs = row_offsets[e], re = row_offsets[e + 1];
    const int nk = (re - rs + kBK - 1) / kBK;
    int ca_col = a0 + cc * 8;
    ca_col = ca_col < Na ? ca_col : Na - 8;
    int cb_col = b0 + cc * 8;
    cb_col = cb_col < Nb ? cb_col : Nb - 8;

    u32x4 ra[4], rb[4];
    auto gload = [&](int kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rs + kt * kBK + (tid >> 4) + 16 * i;
        const bool ok = r < re;
        ra[i] = ok ? ld16(A + (int64_t)r * Na + ca_col) : u32x4{0, 0, 0, 0};
        rb[i] = ok ? ld16(B + (int64_t)r * Nb + cb_col) : u32x4{0, 0, 0, 0};
      }
    };
    auto sstore = [&](int buf) {
      char* la = lds + buf * 2 * T_BYTES;
      char* lb = la + T_BYTES;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lds_write16(la, kr_off<128>((tid >> 4) + 16 * i, cc), ra[i]);
        lds_write16(lb, kr_off<128>((tid >> 4) + 16 * i, cc), rb[i]);
      }
    };

    floatx16 acc[NB][MB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int a = 0; a < MB; ++a)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][a][v] = 0.0f;

    if (nk > 0) {
      gload(0);
      sstore(0);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) gload(kt + 1);
      const char* la = lds + (kt & 1) * 2 * T_BYTES;
      const char* lb = la + T_BYTES;
#pragma unroll
      for (int s = 0; s < kBK / 16; ++s) {
        u32x4 fb[NB], fa[MB];
#pragma unroll
        for (int b = 0; b < NB; ++b) fb[b] = tr_operand<128>(lb, wb * (BB / 2) + b * 32, s, lane);
#pragma unroll
        for (int a = 0; a < MB; ++a) fa[a] = tr_operand<128>(la, wa * (BA / 2) + a * 32, s, lane);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int a = 0; a < MB; ++a) acc[b][a] = TR::mfma32(fb[b], fa[a], acc[b][a]);
      }
      if (kt + 1 < nk) sstore((kt + 1) & 1);
      __syncthreads();
    }

    uint16_t* Ce = C + (int64_t)e * Na * Nb;
#pragma unroll
    for (int a = 0; a < MB; ++a) {
      const int na = a0 + wa * (BA / 2) + a * 32 + (lane & 31);
      if (na >= Na) continue;
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int nb = b0 + wb * (BB / 2) + b * 32 + g * 8 + (lane >> 5) * 4;
          if (nb < Nb)
            st8(Ce + (int64_t)na * Nb + nb, pack4<TR>(acc[b][a][g * 4 + 0], acc[b][a][g * 4 + 1],
                                                     acc[b][a][g * 4 + 2], acc[b][a][g * 4 + 3]));
        }
    }
  }
}

// Row counts of S equal splits of T rows (the first T % S splits one longer),
// the "experts" of the split-K router gate weight gradient.
__global__ void split_rows_kernel(int64_t* __restrict__ tpe, int S, int64_t T) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s < S) tpe[s] = T / S + (s < T % S ? 1 : 0);
}

// out[i] = round(sum_s part[s][i]) over the S partials in split order (deterministic).
template <typename TR>
__global__ __launch_bounds__(256) void sum_splits_kernel(const float* __restrict__ part, int S, int64_t n,
                                                         uint16_t* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; ++s) acc += *reinterpret_cast<const floatx4*>(part + (int64_t)s * n + i);
  st8(out + i, pack4<TR>(acc[0], acc[1], acc[2], acc[3]));
}

// ---------------------------------------------------------------------------
// Wgrad work plan: row groups, split and balanced by cost
// ---------------------------------------------------------------------------
// A wgrad work item is one output tile of one group of rows.  A group is an
// expert's rows or, for an expert holding more than `chunk` rows, one chunk
// of at most `chunk` consecutive rows of it.  The groups of a chunked expert
// accumulate into fp32 partial slots that wgrad_finish_kernel adds in chunk
// order and rounds once, so results are deterministic and independent of
// the grid.  An item's cost is about its group's row count, so the plan:
//   * cuts the group list (expert order) into 8 contiguous runs of about
//     equal total rows, one per XCD, so each expert's rows stay in one L2;
//   * orders each run by rows, largest first, so the longest items start
//     first and the XCD's workgroups finish together.
// (The reference's K-grouped kernel walks an expert's whole row range for
// every output tile, models/moe_triton_grouped_gemm.py:341-345, so one
// heavily loaded expert bounds its time.)
struct WGroup {
  int32_t expert, row_start, row_end, slot;  // slot: fp32 partial slot, or -1 to store C[expert] directly
};
constexpr int kChunkMin = 2048;  // smallest chunk: near-uniform loads (2 x the mean at most) are never split

inline int wgrad_gmax(int E) { return E + E / 2 + 2; }  // groups: E + M / chunk with chunk >= 2 M / E
inline size_t wgrad_plan_bytes(int E) {
  const int g = wgrad_gmax(E);
  return align256(sizeof(int) * (E + 1)) + align256(sizeof(WGroup) * g) + align256(sizeof(int) * g) +
         align256(sizeof(int) * 64) + align256(sizeof(int4) * E);
}
// chunk rows of a plan with partial slots: 2 x the mean rows per expert, at least kChunkMin
inline int64_t wgrad_chunk(int64_t M, int E) {
  const int64_t c = 2 * ((M + E - 1) / E);
  return c < kChunkMin ? kChunkMin : c;
}
// partial slots the first chunk size can need: chunked experts hold more than
// `chunk` rows each, so their chunks number less than 2 M / chunk (and E)
inline int wgrad_slots_needed(int64_t M, int E) {
  const int64_t s = 2 * M / wgrad_chunk(M, E);
  return (int)(s < E ? s : E);
}

struct WgradPlan {
  int* row_offsets;  // [E + 1]
  WGroup* groups;    // [gmax]
  int* order;        // [gmax]: group ids, the 8 XCD runs one after another, each largest first
  int* info;         // [64]: run start and count per XCD [0, 16), group count [16], split count [17],
                     //       work counters [32, 40)
  int4* splits;      // [E]: chunked expert, first slot, chunks
  float* partials;   // [max_slots][Na * Nb]
  int max_slots;
};

inline WgradPlan carve_wgrad(void* ws, size_t ws_bytes, int E, int64_t na_nb) {
  char* p = static_cast<char*>(ws);
  const int g = wgrad_gmax(E);
  WgradPlan w;
  w.row_offsets = reinterpret_cast<int*>(p);
  p += align256(sizeof(int) * (E + 1));
  w.groups = reinterpret_cast<WGroup*>(p);
  p += align256(sizeof(WGroup) * g);
  w.order = reinterpret_cast<int*>(p);
  p += align256(sizeof(int) * g);
  w.info = reinterpret_cast<int*>(p);
  p += align256(sizeof(int) * 64);
  w.splits = reinterpret_cast<int4*>(p);
  p += align256(sizeof(int4) * E);
  w.partials = reinterpret_cast<float*>(p);
  const size_t used = wgrad_plan_bytes(E);
  const size_t slot_bytes = sizeof(float) * (size_t)na_nb;
  size_t slots = ws_bytes > used && slot_bytes ? (ws_bytes - used) / slot_bytes : 0;
  w.max_slots = (int)(slots > (size_t)E ? (size_t)E : slots);
  return w;
}

// Inclusive scan of v[0, n) in LDS, n <= 2048, by a 1024-thread block.
__device__ void block_scan_i64(int64_t* v, int n) {
  for (int off = 1; off < n; off <<= 1) {
    int64_t a = 0, b = 0;
    const int i0 = threadIdx.x, i1 = threadIdx.x + 1024;
    if (i0 < n && i0 >= off) a = v[i0 - off];
    if (i1 < n && i1 >= off) b = v[i1 - off];
    __syncthreads();
    if (i0 < n && i0 >= off) v[i0] += a;
    if (i1 < n && i1 >= off) v[i1] += b;
    __syncthreads();
  }
}

// One block of 1024 threads; E <= 1024.  max_slots = 0 keeps every expert whole.
__global__ __launch_bounds__(1024) void wgrad_plan_kernel(const int64_t* __restrict__ tpe, int E, int64_t M,
                                                          int64_t chunk0, WgradPlan w) {
  __shared__ int64_t s_a[2048];  // scans (per expert, then per group)
  __shared__ uint64_t s_key[2048];
  __shared__ int s_rs[1024], s_n[1024], s_c[1024], s_gb[1024], s_sb[1024];
  __shared__ int64_t s_chunk;
  __shared__ int s_need;
  const int tid = threadIdx.x;
  // expert row ranges: prefix of the counts, clamped to M
  for (int e = tid; e < 1024; e += 1024) s_a[e] = e < E && tpe[e] > 0 ? tpe[e] : 0;
  __syncthreads();
  block_scan_i64(s_a, E);
  if (tid < E) {
    const int64_t end = s_a[tid], start = tid == 0 ? 0 : s_a[tid - 1];
    const int rs = (int)(start < M ? start : M), re = (int)(end < M ? end : M);
    s_rs[tid] = rs;
    s_n[tid] = re - rs;
    w.row_offsets[tid] = rs;
    if (tid == E - 1) w.row_offsets[E] = re;
  }
  if (tid == 0) s_chunk = w.max_slots > 0 ? chunk0 : ((int64_t)1 << 40);
  __syncthreads();
  // chunk size: the smallest power-of-two multiple of chunk0 whose chunks fit the partial slots
  while (true) {
    if (tid == 0) s_need = 0;
    __syncthreads();
    const int64_t ch = s_chunk;
    if (tid < E && s_n[tid] > ch) atomicAdd(&s_need, (int)((s_n[tid] + ch - 1) / ch));
    __syncthreads();
    const bool fits = s_need <= w.max_slots;
    __syncthreads();
    if (fits) break;
    if (tid == 0) s_chunk = ch * 2;
    __syncthreads();
  }
  const int64_t ch = s_chunk;
  // groups and partial slots per expert: exclusive prefixes
  if (tid < E) s_c[tid] = s_n[tid] > ch ? (int)((s_n[tid] + ch - 1) / ch) : 1;
  for (int e = tid; e < 1024; e += 1024) s_a[e] = e < E ? s_c[e] : 0;
  __syncthreads();
  block_scan_i64(s_a, E);
  if (tid < E) s_gb[tid] = (int)(s_a[tid] - s_c[tid]);
  const int G = (int)s_a[E - 1];
  __syncthreads();
  for (int e = tid; e < 1024; e += 1024) s_a[e] = e < E && s_c[e] > 1 ? s_c[e] : 0;
  __syncthreads();
  block_scan_i64(s_a, E);
  if (tid < E) s_sb[tid] = (int)(s_a[tid] - (s_c[tid] > 1 ? s_c[tid] : 0));
  __syncthreads();
  for (int e = tid; e < 1024; e += 1024) s_a[e] = e < E && s_c[e] > 1 ? 1 : 0;
  __syncthreads();
  block_scan_i64(s_a, E);
  if (tid < E && s_c[tid] > 1) w.splits[s_a[tid] - 1] = int4{tid, s_sb[tid], s_c[tid], 0};
  const int nsplit = (int)s_a[E - 1];
  __syncthreads();
  // the groups, their costs and their prefix
  for (int g = tid; g < 2048; g += 1024) {
    int64_t cost = 0;
    if (g < G) {
      int lo = 0, hi = E - 1;  // expert of group g: the last e with s_gb[e] <= g
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_gb[mid] <= g) lo = mid; else hi = mid - 1;
      }
      const int e = lo, c = g - s_gb[e];
      WGroup grp;
      grp.expert = e;
      grp.row_start = s_rs[e] + (int)(c * ch);
      const int64_t end = (int64_t)grp.row_start + ch;
      grp.row_end = (int)(end < s_rs[e] + s_n[e] ? end : s_rs[e] + s_n[e]);
      grp.slot = s_c[e] > 1 ? s_sb[e] + c : -1;
      w.groups[g] = grp;
      cost = (int64_t)(grp.row_end - grp.row_start) + 64;  // + a tile's fixed cost, so empty groups count
    }
    s_a[g] = cost;
  }
  __syncthreads();
  block_scan_i64(s_a, G);
  const int64_t total = s_a[G - 1];
  // XCD of a group: where its cost's midpoint falls in eighths of the total; then
  // sort by (XCD, cost descending, group id)
  for (int g = tid; g < 2048; g += 1024) {
    uint64_t key = ~0ull;
    if (g < G) {
      const int64_t cost = g == 0 ? s_a[0] : s_a[g] - s_a[g - 1];
      int64_t x = ((s_a[g] - cost / 2) * 8) / total;
      x = x < 7 ? x : 7;
      key = ((uint64_t)x << 56) | ((uint64_t)(0xFFFFFFFFu - (uint32_t)cost) << 16) | (uint64_t)g;
    }
    s_key[g] = key;
  }
  __syncthreads();
  int P = 1;
  while (P < G) P <<= 1;
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < P; i += 1024) {
        const int l = i ^ j;
        if (l > i) {
          const uint64_t a = s_key[i], b = s_key[l];
          const bool up = (i & k) == 0;
          if ((a > b) == up) {
            s_key[i] = b;
            s_key[l] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  if (tid < 16) w.info[tid] = 0;
  if (tid >= 32 && tid < 40) w.info[tid] = 0;  // work counters
  __syncthreads();
  for (int i = tid; i < G; i += 1024) {
    const uint64_t key = s_key[i];
    const int x = (int)(key >> 56);
    w.order[i] = (int)(key & 0xFFFF);
    if (i == 0 || (int)(s_key[i - 1] >> 56) != x) w.info[2 * x] = i;
    if (i == G - 1 || (int)(s_key[i + 1] >> 56) != x) w.info[2 * x + 1] = i + 1;  // end, made a count below
  }
  __syncthreads();
  if (tid < 8) {
    const int end = w.info[2 * tid + 1];
    w.info[2 * tid + 1] = end > 0 ? end - w.info[2 * tid] : 0;
  }
  if (tid == 0) {
    w.info[16] = G;
    w.info[17] = nsplit;
  }
}

// ---------------------------------------------------------------------------
// DMA-fed kernels: buffer_load ... lds fills a ring of LDS stages directly
// ---------------------------------------------------------------------------
// Each buffer_load_dwordx4 ... lds writes the 16 bytes of lane L to
// LDS[M0 + 16 L], so one wave instruction fills 1 KB of a stage.  Each lane
// therefore chooses its source address so that the bytes land in the
// swizzled layouts above:
//   [rows][64] tiles: 8 rows per instruction, lane L -> row L/8, physical
//                     chunk L%8, logical chunk (L%8) ^ kc_swz(row)
//   [64 k][128] tiles: 4 rows per instruction, lane L -> row L/16, physical
//                     chunk L%16, logical chunk (L%16) ^ kr_swz(row)
// Loads through a buffer resource return zeros past num_records, which zero-fills
// the wgrad row tails without branches.  The ring is synchronised with
// an explicit vmcnt wait plus a bare s_barrier per K step.  A workgroup
// barrier with a memory fence would drain the loads still in flight for
// later stages.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
template <int CPOL = 0>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* lds_dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (HRM_LDS void*)lds_dst, 16, voff, soff, 0, CPOL);
}
// 4 bytes per lane into LDS (lane l's dword at lds_dst + 4 l), as inline assembly like dma16t
__device__ __forceinline__ void dma4t(__amdgpu_buffer_rsrc_t r, char* lds_dst, uint32_t voff) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(HRM_LDS void*)lds_dst);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(lds), "v"(voff), "s"(r)
               : "memory", "m0");
}
// 4 bytes per lane straight into LDS (lane l's dword at lds_dst + 4 l)
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, char* lds_dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (HRM_LDS void*)lds_dst, 4, voff, 0, 0, 0);
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | 0x70 | 0xF00 | ((N >> 4) << 14));
}
// Barrier that orders LDS use without waiting for outstanding vector memory
// operations; the empty asm statements keep the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void barrier_lds() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// Wait until at most `ahead` stages of `per` loads each are still in flight.
template <int PER, int MAX_AHEAD>
__device__ __forceinline__ void wait_stages(int ahead) {
  static_assert(MAX_AHEAD <= 3 && 3 * PER < 64, "vmcnt range");
  if constexpr (MAX_AHEAD >= 3) {
    if (ahead >= 3) { wait_vmcnt<3 * PER>(); return; }
  }
  if constexpr (MAX_AHEAD >= 2) {
    if (ahead >= 2) { wait_vmcnt<2 * PER>(); return; }
  }
  if constexpr (MAX_AHEAD >= 1) {
    if (ahead >= 1) { wait_vmcnt<PER>(); return; }
  }
  wait_vmcnt<0>();
}

// Backward of silu(g) * u for one element, with the reference's rounding
// points (torch autograd on 16-bit tensors): the saved silu output is rounded,
// d_up = da * silu(g) and d_silu = da * u are rounded products, and silu's
// backward is computed in fp32 as d_silu * sig * (1 + g * (1 - sig)) and rounded.
// sig = 1 / (1 + e^-g) uses the hardware exp2 and reciprocal, as the forward's
// swiglu_fast does: an exact expf and two IEEE divisions made this epilogue
// cost more VALU time per tile than the tile's MFMAs.
template <typename TR>
__device__ __forceinline__ void swiglu_bwd(float da, float g, float u, float& dg, float& du) {
  const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
  const float sl = TR::to_f(TR::from_f(g * sig));
  du = TR::to_f(TR::from_f(da * sl));
  const float ds = TR::to_f(TR::from_f(da * u));
  dg = TR::to_f(TR::from_f(ds * sig * (1.0f + g * (1.0f - sig))));
}

__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

// Non-temporal (nt) cache policy bit, for stores of output that nothing
// re-reads from L2 soon (and for the weight loads of the decode-size tiles).  The persistent kernels' first wait of the next tile also waits for
// the previous tile's stores, and nt stores are acknowledged sooner: the NT
// GEMM at L (131072 x 1280 x 448) measured 177 against 204 us, and the L
// training step (dgrad and wgrad outputs too) 2384 against 2398 us.
constexpr int kCpolNT = 2;
// The same DMA issued as inline assembly, for kernels that read their tiles
// with ds_read_b64_tr_b16.  The compiler treats that read as possibly
// aliasing any LDS written by a DMA it knows of, and put an
// s_waitcnt vmcnt(0) before the first transposed read of every K step: each
// step then waited for the DMA of the step after it, which the ring issues
// just before, so no DMA overlapped any MFMA.  DMAs it cannot see are not
// tracked; these kernels order their DMAs with explicit vmcnt waits and
// barriers anyway.  Loads the compiler issues itself are still waited for
// correctly: extra operations in flight only make its vmcnt counts stricter.
// The LDS address goes to m0 and the scalar offset to an SGPR, so both must be
// wave-uniform, as they are at every call.  No other code in these kernels
// uses m0 (checked in the generated code: only these writes of it appear).
template <int CPOL = 0>
__device__ __forceinline__ void dma16t(__amdgpu_buffer_rsrc_t r, char* lds_dst, uint32_t voff, uint32_t soff) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(HRM_LDS void*)lds_dst);
  soff = __builtin_amdgcn_readfirstlane(soff);
  if constexpr (CPOL == kCpolNT)
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds" ::"s"(lds), "v"(voff), "s"(r),
                 "s"(soff)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(r),
                 "s"(soff)
                 : "memory", "m0");
}
__device__ __forceinline__ void bstore8(__amdgpu_buffer_rsrc_t r, uint32_t voff, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, voff, 0, 0);
}
// CPOL: cache policy bits of the store (0, or kCpolNT)
template <int CPOL = 0>
__device__ __forceinline__ void bstore16(__amdgpu_buffer_rsrc_t r, uint32_t voff, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, CPOL);
}

// M-grouped GEMM fed by DMA, persistent, with the K steps of consecutive tiles
// streamed through one LDS ring: while a tile's last steps compute, the ring
// already receives the next tile's first steps, and that tile's metadata and
// gathered row ids were loaded early in the current tile.  Requires K % 64 == 0.
// Output stores go through a buffer resource covering the tile's rows; lanes
// with nothing to store get an offset past it, so every wave issues the same
// stores and no branch is taken.
// 4-wave variants are sized for two workgroups per CU (at most 256 registers
// per lane, two waves per SIMD); 8-wave variants run one per CU.
// WNT: weight rows are loaded non-temporally (each expert's weights are read
// by about one M tile: decode and mid-size token counts).
template <typename TR, int KIND, int BM, int BN, int STAGES, int NW, int BK, int EPI = EPI_PLAIN, bool WNT = false>
__global__ __launch_bounds__(NW * 64, NW == 4 ? 2 : 1) void mgemm_dma_kernel(const uint16_t* __restrict__ A,
                                                               const int32_t* __restrict__ gather,
                                                               const uint16_t* __restrict__ W,
                                                               uint16_t* __restrict__ C,
                                                               const int64_t* __restrict__ tpe, int E, int M, int N,
                                                               int K, int tiles_n, uint32_t a_bytes,
                                                               uint16_t* __restrict__ aux) {
  static_assert(EPI == EPI_PLAIN || (EPI == EPI_SAVE_GU && KIND == KIND_GATHER_SWIGLU) ||
                    (EPI == EPI_SWIGLU_BWD && KIND == KIND_NN),
                "epilogue mode does not fit the kernel kind");
  constexpr int WGM = BM == 32 ? 1 : 2;                      // waves along M (32-row tiles: all along N)
  constexpr int WGN = NW / WGM;                              // waves along N
  constexpr int MB = BM / WGM / 32;                          // 32-row blocks per wave
  constexpr int NB = BN / WGN / 32;                          // 32-column blocks per wave
  constexpr int PK = BK * 2;                                 // bytes per K-contiguous tile row
  constexpr int LPRK = BK / 8;                               // DMA lanes per K-contiguous row
  constexpr int RPIK = 64 / LPRK;                            // K-contiguous rows per 1 KB instruction
  constexpr int A_BYTES = BM * BK * 2;
  constexpr int B_BYTES = BN * BK * 2;
  constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  constexpr int A_ROWS = BM / NW;                            // A rows loaded per wave
  constexpr int A_INSTR = A_ROWS / RPIK;
  constexpr int NN_RPI = 1024 / (BN * 2);                    // NN: [BK k][BN] rows per 1 KB instruction
  constexpr int NN_LPR = BN / 8;                             // NN: lanes per row
  constexpr int NN_KR = BK / NW;                             // NN: k rows loaded per wave
  constexpr int B_ROWS = BN / NW;                            // NT: B rows loaded per wave
  constexpr int B_INSTR = KIND == KIND_NN ? NN_KR / NN_RPI : B_ROWS / RPIK;
  static_assert(BK == 32 || BK == 64, "K step is 32 or 64");
  constexpr int PER = A_INSTR + B_INSTR;                     // loads per wave per stage
  // 8 waves, 2-stage ring: the second half of the waves issues its share of a
  // stage after its first sub-step of MFMAs.  Issued by every wave right after
  // the K-step barrier, the CU's 64 DMA instructions of a stage queue at the
  // texture unit together for about 1000 cycles, and a wave cannot issue
  // MFMAs behind its queued instructions.  Paired launches: down GEMM L
  // 179 -> 172 us, dgrad L 244 -> 227 us, XL128 510 -> 472 us; gather +
  // gate/up at XL128 796 -> 780 us, XL-skew 388 -> 382 us (XL-skew training
  // step 2.874 -> 2.863 ms with the gate/up-saving variant too).
  constexpr bool STAGGER = NW == 8 && STAGES == 2;
  static_assert(NW == 4 || NW == 8, "4 or 8 waves");
  static_assert(BN == 128 || BN == 256, "BN is 128 or 256");
  static_assert(A_INSTR >= 1 && B_INSTR >= 1 && NB >= 1 && (KIND != KIND_GATHER_SWIGLU || NB % 2 == 0), "tile split");
  static_assert(STAGES >= 2 && STAGES <= 5, "2..5 stages");
  // the ring plus the tile plan (3 ints per expert, dynamic) must fit one
  // workgroup's 160 KB of LDS, or the dispatch is rejected
  static_assert(STAGES * STAGE_BYTES + 3 * 4 * kMaxExperts +
                        (KIND == KIND_GATHER_SWIGLU ? NW * A_INSTR * 64 * 4 : 0) <= 160 * 1024,
                "LDS budget exceeds 160 KB");
  // gate/up kernel: the ring, then the gathered source rows of the prefetched tile
  constexpr int GIDX_BYTES = KIND == KIND_GATHER_SWIGLU ? NW * A_INSTR * 64 * 4 : 0;
  __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE_BYTES + GIDX_BYTES];
  extern __shared__ int plan_lds[];  // [3][E]: row start, row end, inclusive M-tile prefix

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  // M-tile plan from tokens_per_expert, built by wave 0 of every workgroup:
  // expert e owns rows [s_rs[e], s_re[e]) (prefix sums clamped to M) and
  // M-tiles [s_tp[e-1], s_tp[e]).
  int* s_rs = plan_lds;
  int* s_re = plan_lds + E;
  int* s_tp = plan_lds + 2 * E;
  if (wave == 0) {
    int64_t carry_rows = 0;
    int carry_t = 0;
    for (int c = 0; c < E; c += 64) {
      const int e = c + lane;
      int64_t n = e < E ? tpe[e] : 0;
      n = n > 0 ? n : 0;
      int64_t v = n;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int64_t u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
      }
      const int64_t end = carry_rows + v;
      const int rs = (int)(end - n < M ? end - n : M);
      const int re = (int)(end < M ? end : M);
      int it = (re - rs + BM - 1) / BM;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(it, o, 64);
        if (lane >= o) it += u;
      }
      if (e < E) {
        s_rs[e] = rs;
        s_re[e] = re;
        s_tp[e] = carry_t + it;
      }
      carry_rows += __shfl(v, 63, 64);
      carry_t += __shfl(it, 63, 64);
    }
  }
  __syncthreads();
  const int total = s_tp[E - 1] * tiles_n;
  const int xcd = blockIdx.x & 7;
  const int nloc = gridDim.x >> 3;
  const int chunk = (total + 7) >> 3;
  const int64_t w_rows = KIND == KIND_GATHER_SWIGLU ? 2 * (int64_t)N : (KIND == KIND_NN ? (int64_t)K : (int64_t)N);
  const int64_t w_cols = KIND == KIND_NN ? (int64_t)N : (int64_t)K;
  const int nk = K / BK;
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(A, a_bytes);
  const int lrowk = lane / LPRK;  // row within a DMA instruction
  const int lchk = lane % LPRK;   // physical 16-byte chunk within that row

  // i-th tile of this workgroup (XCD-contiguous order), or -1
  auto tile_at = [&](int i) __attribute__((always_inline)) -> int {
    const int jj = (blockIdx.x >> 3) + i * nloc;
    if (jj >= chunk) return -1;
    const int t = xcd * chunk + jj;
    return t < total ? t : -1;
  };

  // ---- issue side: the tile whose K steps are being fed into the ring.  The
  // host keeps STAGES - 1 <= K/64, so it is at most one tile ahead of compute.
  uint32_t a_off[A_INSTR];
  uint32_t b_off[B_INSTR];
  __amdgpu_buffer_rsrc_t rB = make_rsrc(W, 0);
  int iss_rs = 0, iss_re = 0, iss_n0 = 0;
  int iss_seq = 0;      // sequence number of the issue-side tile
  int iss_step = 0;     // next local K step to issue
  bool iss_valid = false;
  // metadata prefetched for tile iss_seq + 1
  int pf_t = -1;
  MTile pf_m = MTile{0, 0, 0, 0};
  uint32_t pf_src[A_INSTR];
#pragma unroll
  for (int i = 0; i < A_INSTR; ++i) pf_src[i] = 0;
  // Gathered source rows of the prefetched tile (gate/up kernel): DMA'd into
  // LDS, one dword per lane, and read back when the tile is taken, a whole
  // tile later.  Loaded into registers, they were copied at once into the
  // registers that carry them across the loop, and that copy waited for the
  // load, and so for every DMA in flight, at each tile switch.  By the time
  // they are read, the K-step waits (vmcnt, which counts in issue order)
  // have covered their DMA.
  constexpr bool GIDX = KIND == KIND_GATHER_SWIGLU;
  uint32_t* const gidx = reinterpret_cast<uint32_t*>(smem + STAGES * STAGE_BYTES);  // [NW][A_INSTR][64]
  const __amdgpu_buffer_rsrc_t rG = make_rsrc(gather, GIDX ? (uint32_t)M * 4u : 0u);

  auto load_src = [&](const MTile& m) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
      int r = m.row_start + wave * A_ROWS + i * RPIK + lrowk;
      r = r < m.row_end ? r : m.row_end - 1;
      if constexpr (GIDX) {
        // the previous tile's indices have been read back (that ds_read is done) before the DMA overwrites them
        if (i == 0) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        dma4(rG, reinterpret_cast<char*>(gidx + (wave * A_INSTR + i) * 64), (uint32_t)r * 4u);
      } else {
        pf_src[i] = (uint32_t)r;
      }
    }
  };
  auto prefetch = [&](int seq) __attribute__((always_inline)) {
    pf_t = tile_at(seq);
    if (pf_t >= 0) {
      // expert of M-tile mt: the first e whose inclusive tile prefix exceeds mt
      const int mt = pf_t / tiles_n;
      int ex = 0;
      for (int c = 0; c < E; c += 64) {
        const int ee = c + lane;
        const uint64_t hit = __ballot(ee < E && s_tp[ee] > mt);
        if (hit) {
          ex = c + __ffsll((unsigned long long)hit) - 1;
          break;
        }
      }
      const int before = ex == 0 ? 0 : s_tp[ex - 1];
      pf_m.expert = ex;
      pf_m.row_start = s_rs[ex] + (mt - before) * BM;
      pf_m.row_end = min(pf_m.row_start + BM, s_re[ex]);
      load_src(pf_m);
    }
  };
  // builds the issue-side context from the prefetched metadata
  auto take_prefetched = [&]() __attribute__((always_inline)) {
    // tile metadata is wave-uniform: keep it in SGPRs so descriptors built from
    // it need no per-lane (waterfall) handling
    // N tile of list entry pf_t, rotated by mt * tiles_n / nloc: a workgroup
    // walks the list with stride nloc, i.e. nloc / tiles_n M tiles per step,
    // so the rotation advances by one N tile per step and every workgroup sees
    // each N tile equally often (the gate/up kernel's last N tile may be a
    // cheaper half tile).
    const int mt_ = pf_t / tiles_n;
    const int rot = (int)(((int64_t)mt_ * tiles_n) / nloc);
    const int nt = __builtin_amdgcn_readfirstlane((pf_t - mt_ * tiles_n + rot) % tiles_n);
    iss_rs = __builtin_amdgcn_readfirstlane(pf_m.row_start);
    iss_re = __builtin_amdgcn_readfirstlane(pf_m.row_end);
    const int ex = __builtin_amdgcn_readfirstlane(pf_m.expert);
    rB = make_rsrc(W + (int64_t)ex * w_rows * w_cols, (uint32_t)(w_rows * w_cols * 2));
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
      const int row = wave * A_ROWS + i * RPIK + lrowk;
      const int lc = lchk ^ kcp_swz<PK>(row);
      const uint32_t src = GIDX ? gidx[(wave * A_INSTR + i) * 64 + lane] : pf_src[i];
      a_off[i] = (src * (uint32_t)K + lc * 8) * 2;
    }
    if constexpr (KIND == KIND_NN) {
      iss_n0 = nt * BN;
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i) {
        const int kr = wave * NN_KR + i * NN_RPI + lane / NN_LPR;
        const int lc = (lane % NN_LPR) ^ kr_swz(kr);
        int col = iss_n0 + lc * 8;
        col = col < N ? col : N - 8;
        b_off[i] = ((uint32_t)kr * (uint32_t)N + (uint32_t)col) * 2;
      }
    } else if constexpr (KIND == KIND_GATHER_SWIGLU) {
      iss_n0 = nt * (BN / 2);
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i) {
        const int jr = wave * B_ROWS + i * RPIK + lrowk;
        const int lc = lchk ^ kcp_swz<PK>(jr);
        int cc = iss_n0 + (jr % (BN / 2));
        cc = cc < N ? cc : N - 1;
        const uint32_t wr = jr < BN / 2 ? (uint32_t)cc : (uint32_t)(N + cc);
        b_off[i] = (wr * (uint32_t)K + lc * 8) * 2;
      }
    } else {
      iss_n0 = nt * BN;
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i) {
        const int jr = wave * B_ROWS + i * RPIK + lrowk;
        const int lc = lchk ^ kcp_swz<PK>(jr);
        int n = iss_n0 + jr;
        n = n < N ? n : N - 1;
        b_off[i] = ((uint32_t)n * (uint32_t)K + lc * 8) * 2;
      }
    }
  };

  int issued = 0;  // global K steps issued so far; step g sits in ring slot g % STAGES
  auto issue_next = [&]() __attribute__((always_inline)) -> bool {
    if (iss_step == nk) {
      if (pf_t < 0) return false;
      take_prefetched();
      ++iss_seq;
      iss_step = 0;
      prefetch(iss_seq + 1);
    }
    char* sa = smem + (issued % STAGES) * STAGE_BYTES;
    char* sb = sa + A_BYTES;
    const uint32_t ka = (uint32_t)iss_step * (BK * 2);
    if constexpr (KIND == KIND_NN) {  // the W tile is read transposed: DMA the compiler cannot see
#pragma unroll
      for (int i = 0; i < A_INSTR; ++i) dma16t(rA, sa + (wave * A_ROWS + i * RPIK) * PK, a_off[i], ka);
    } else {
#pragma unroll
      for (int i = 0; i < A_INSTR; ++i) dma16(rA, sa + (wave * A_ROWS + i * RPIK) * PK, a_off[i], ka);
    }
    if constexpr (KIND == KIND_NN) {
      const uint32_t kb = (uint32_t)iss_step * BK * (uint32_t)N * 2;
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i) dma16t(rB, sb + (wave * NN_KR + i * NN_RPI) * (BN * 2), b_off[i], kb);
    } else {
      // 32-row tiles run at decode sizes, where each expert's weight rows are
      // read once: non-temporal loads (decode layer T = 8 82.9 -> 73.8 us,
      // T = 64 99.4 -> 88.3 us).  Larger tiles re-read them from L2 across M
      // tiles, except with few rows per expert (WNT).
      constexpr int BPOL = (BM == 32 || WNT) ? kCpolNT : 0;
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i) dma16<BPOL>(rB, sb + (wave * B_ROWS + i * RPIK) * PK, b_off[i], ka);
    }
    ++iss_step;
    ++issued;
    return true;
  };

  // first tile
  prefetch(0);
  if (pf_t < 0) return;
  if constexpr (GIDX) wait_vmcnt<0>();  // its gathered source rows are in LDS
  take_prefetched();
  iss_valid = true;
  prefetch(1);
  (void)iss_valid;
  int comp_rs = iss_rs, comp_re = iss_re, comp_n0 = iss_n0;
#pragma unroll
  for (int s2 = 0; s2 < STAGES - 1; ++s2) issue_next();

  int g0 = 0;  // global index of the computing tile's step 0

  // One tile: K loop and epilogue.  A "half" tile (gate/up kernel with 8 waves
  // and 256-row weight tiles, when at most 64 gate columns remain) puts the 8
  // waves on a 4 x 2 grid of 64 rows x (32 gate + 32 up) columns, so the last
  // N tile of a width that is an odd multiple of 64 keeps every wave busy on
  // valid columns.  Its B tile rows past the valid ones are loaded but unused.
  auto tile = [&](auto half_tag) __attribute__((always_inline)) {
    constexpr bool H = decltype(half_tag)::value;
    constexpr int MBH = H ? 2 : MB;                               // 32-row blocks per wave
    const int row_base = H ? (wave >> 1) * 64 : wm * (BM / WGM);  // first tile row of this wave
    const int col_blk = H ? (wave & 1) * 32 : wn * (BN / 2 / WGN);  // gate/up column block (gate/up kernel)
    floatx16 acc[NB][MBH];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int a = 0; a < MBH; ++a)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][a][v] = 0.0f;

    // K loop over MBV of the wave's MBH 32-row blocks: blocks wholly past the
    // tile's last row (an expert's ragged last M tile) get no fragment reads
    // and no MFMAs, which leaves the SIMD's matrix pipe to the other wave on
    // it (down GEMM: L 184 -> 181 us, XL128 471 -> 461 us).  Their accumulators stay zero; the epilogue's stores past the last
    // row fall outside the output's buffer range.  Every wave still waits,
    // passes each barrier and issues its share of the DMA.
    auto kloop = [&](auto mbv_tag) __attribute__((always_inline)) {
      constexpr int MBV = decltype(mbv_tag)::value;
      for (int kt = 0; kt < nk; ++kt) {
        const int gs = g0 + kt;
        wait_stages<PER, STAGES - 2>(min(STAGES - 2, issued - gs - 1));
        barrier_lds();
        const bool late = STAGGER && wave >= NW / 2 && MBV > 0;
        const bool due = issued == gs + STAGES - 1;
        if (due && !late) issue_next();
        if constexpr (MBV > 0) {
          const char* la = smem + (gs % STAGES) * STAGE_BYTES;
          const char* lb = la + A_BYTES;
          u32x4 fw[2][NB], fa[2][MBV];
          auto load_frags = [&](int s, u32x4 (&w)[NB], u32x4 (&x)[MBV]) __attribute__((always_inline)) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              int r0;
              if constexpr (KIND == KIND_GATHER_SWIGLU)  // gate blocks, then the matching up blocks
                r0 = (b < NB / 2 ? 0 : BN / 2) + col_blk + (b % (NB / 2)) * 32;
              else
                r0 = wn * (BN / WGN) + b * 32;
              if constexpr (KIND == KIND_NN) w[b] = tr_operand<BN>(lb, r0, s, lane);
              else w[b] = lds_read16(lb, kcp_off<PK>(r0 + (lane & 31), s * 2 + (lane >> 5)));
            }
#pragma unroll
            for (int a = 0; a < MBV; ++a)
              x[a] = lds_read16(la, kcp_off<PK>(row_base + a * 32 + (lane & 31), s * 2 + (lane >> 5)));
          };
          load_frags(0, fw[0], fa[0]);
#pragma unroll
          for (int s = 0; s < BK / 16; ++s) {
            if (s + 1 < BK / 16) load_frags(s + 1, fw[(s + 1) & 1], fa[(s + 1) & 1]);
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
              for (int a = 0; a < MBV; ++a) acc[b][a] = TR::mfma32(fw[s & 1][b], fa[s & 1][a], acc[b][a]);
            if (s == 0 && due && late) issue_next();
          }
        }
      }
    };
    // The gather + gate/up kernel takes kloop only for tiles with a row block
    // past their last row and keeps the plain loop for full tiles: built
    // through kloop for every tile it measured 1-2% slower (L gate_up +3 us,
    // XL128 +14 us, paired launches), even with every row block valid.  With
    // the split: XL128 gate_up 770 -> 755 us, XL-skew 394 -> 389 us, L the
    // same (paired launches, bit-identical).
    // this wave's 32-row blocks that hold a row of the tile (wave-uniform)
    const int vrows = __builtin_amdgcn_readfirstlane(comp_re - comp_rs) - row_base;
    const int nvb = vrows <= 0 ? 0 : min((vrows + 31) / 32, MBH);
    auto ragged_kloop = [&]() __attribute__((always_inline)) {
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using I3 = std::integral_constant<int, 3>;
      if (nvb >= MBH) {
        kloop(std::integral_constant<int, MBH>{});
      } else if constexpr (MBH == 4) {
        if (nvb == 3) kloop(I3{});
        else if (nvb == 2) kloop(I2{});
        else if (nvb == 1) kloop(I1{});
        else kloop(I0{});
      } else if constexpr (MBH == 2) {
        if (nvb == 1) kloop(I1{});
        else kloop(I0{});
      } else {
        kloop(I0{});
      }
    };
    if constexpr (H || KIND == KIND_GATHER_SWIGLU) {
      if (!H && nvb < MBH) {
        if constexpr (!H) ragged_kloop();
      } else {
      for (int kt = 0; kt < nk; ++kt) {
        const int gs = g0 + kt;
        wait_stages<PER, STAGES - 2>(min(STAGES - 2, issued - gs - 1));
        barrier_lds();
        const bool late = STAGGER && wave >= NW / 2;
        const bool due = issued == gs + STAGES - 1;
        if (due && !late) issue_next();
        const char* la = smem + (gs % STAGES) * STAGE_BYTES;
        const char* lb = la + A_BYTES;
        u32x4 fw[2][NB], fa[2][MBH];
        auto load_frags = [&](int s, u32x4 (&w)[NB], u32x4 (&x)[MBH]) __attribute__((always_inline)) {
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            int r0;
            if constexpr (KIND == KIND_GATHER_SWIGLU)  // gate blocks, then the matching up blocks
              r0 = (b < NB / 2 ? 0 : BN / 2) + col_blk + (b % (NB / 2)) * 32;
            else
              r0 = wn * (BN / WGN) + b * 32;
            if constexpr (KIND == KIND_NN) w[b] = tr_operand<BN>(lb, r0, s, lane);
            else w[b] = lds_read16(lb, kcp_off<PK>(r0 + (lane & 31), s * 2 + (lane >> 5)));
          }
#pragma unroll
          for (int a = 0; a < MBH; ++a)
            x[a] = lds_read16(la, kcp_off<PK>(row_base + a * 32 + (lane & 31), s * 2 + (lane >> 5)));
        };
        load_frags(0, fw[0], fa[0]);
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
          if (s + 1 < BK / 16) load_frags(s + 1, fw[(s + 1) & 1], fa[(s + 1) & 1]);
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int a = 0; a < MBH; ++a) acc[b][a] = TR::mfma32(fw[s & 1][b], fa[s & 1][a], acc[b][a]);
          if (s == 0 && due && late) issue_next();
        }
      }
      }
    } else {
      ragged_kloop();
    }

    // Epilogue, staged through LDS so that every store writes whole row segments.
    // The ring slot of the tile's last K step is free once all waves have
    // passed the barrier below: the next DMA into it is issued only after the
    // barrier at the top of the next K step.  Each wave stages its own region,
    // so between its writes and its read-back only in-order LDS execution is
    // needed.  Staged rows are swizzled at 8-byte granularity (chunk ^ g(row))
    // so both the 8-byte writes and the 16-byte read-back are conflict-free.
    const int c_rs = __builtin_amdgcn_readfirstlane(comp_rs);
    const int c_rows = __builtin_amdgcn_readfirstlane(comp_re - comp_rs);
    // C rows hold N values, or 2N for the d(gate_up) output of EPI_SWIGLU_BWD;
    // aux rows (gate/up) hold 2N
    constexpr int CMUL = EPI == EPI_SWIGLU_BWD ? 2 : 1;
    const __amdgpu_buffer_rsrc_t rC =
        make_rsrc(C + (int64_t)c_rs * N * CMUL, (uint32_t)c_rows * (uint32_t)N * 2 * CMUL);
    const __amdgpu_buffer_rsrc_t rX = EPI == EPI_PLAIN
                                          ? rC
                                          : make_rsrc(aux + (int64_t)c_rs * N * 2, (uint32_t)c_rows * (uint32_t)N * 4);
    constexpr int WCOLS = KIND == KIND_GATHER_SWIGLU ? BN / 2 / WGN : BN / WGN;  // output columns per wave
    constexpr int PITCH = WCOLS * 2;                                      // staged row bytes
    constexpr int C8 = PITCH / 8;                                         // 8-byte chunks per row
    constexpr int RP = 256 / PITCH;                                       // rows per 256 bytes
    constexpr int REGION = STAGE_BYTES / NW;                              // staging bytes per wave
    constexpr int FIT = REGION / (32 * PITCH);                            // 32-row blocks that fit
    constexpr int APP = FIT >= 4 && MBH >= 4 ? 4 : (FIT >= 2 && MBH >= 2 ? 2 : 1);  // blocks per pass
    constexpr int LPR = PITCH / 16;                                       // read-back lanes per row
    constexpr int RPI = 64 / LPR;                                         // rows per read-back
    constexpr int NPASS = EPI == EPI_SAVE_GU ? 3 : 1;                     // act, then gate, then up
    static_assert(FIT >= 1 && MBH % APP == 0 && RP * C8 == 32, "staging layout");
    char* stg = smem + ((g0 + nk - 1) % STAGES) * STAGE_BYTES + wave * REGION;
    const int col0 = comp_n0 + (KIND == KIND_GATHER_SWIGLU ? col_blk : wn * WCOLS);
    barrier_lds();
#pragma unroll
    for (int pass = 0; pass < NPASS; ++pass) {
#pragma unroll
      for (int a0 = 0; a0 < MBH; a0 += APP) {
#pragma unroll
        for (int a = a0; a < a0 + APP; ++a) {
          const int r = (a - a0) * 32 + (lane & 31);
          const int g = (r / RP) % C8;
#pragma unroll
          for (int b = 0; b < WCOLS / 32; ++b)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              float o[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                if constexpr (KIND == KIND_GATHER_SWIGLU) {
                  const float x = acc[b][a][gq * 4 + q], y = acc[b + NB / 2][a][gq * 4 + q];
                  o[q] = pass == 0 ? swiglu_fast<TR>(x, y) : (pass == 1 ? x : y);
                } else {
                  o[q] = acc[b][a][gq * 4 + q];
                }
              }
              const int ch8 = (b * 32 + gq * 8) / 4 + (lane >> 5);
              *reinterpret_cast<u32x2*>(stg + r * PITCH + ((ch8 ^ g) << 3)) = pack4<TR>(o[0], o[1], o[2], o[3]);
            }
        }
        constexpr int ITER = APP * 32 / RPI;  // read-back rows per lane in this pass
        // EPI_SWIGLU_BWD: byte offset of the gate values of read-back i's row and columns
        auto xoff_of = [&](int i) __attribute__((always_inline)) -> uint32_t {
          const uint32_t ml = (uint32_t)(row_base + a0 * 32 + i * RPI + lane / LPR);
          const int c = col0 + (lane % LPR) * 8;
          return c < N ? (ml * (uint32_t)N * 2 + (uint32_t)c) * 2 : 0x80000000u;
        };
        u32x4 g_next = u32x4{0u, 0u, 0u, 0u}, u_next = g_next;
        if constexpr (EPI == EPI_SWIGLU_BWD) {  // first row's gate/up, in flight during the staging reads
          g_next = bload16(rX, xoff_of(0));
          u_next = bload16(rX, xoff_of(0) + (uint32_t)N * 2);
        }
#pragma unroll
        for (int i = 0; i < ITER; ++i) {
          const int r = i * RPI + lane / LPR;
          const int c16 = lane % LPR;
          const int g = (r / RP) % C8;
          u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * PITCH + ((c16 ^ (g >> 1)) << 4));
          if (g & 1) v = u32x4{v[2], v[3], v[0], v[1]};
          const uint32_t ml = (uint32_t)(row_base + a0 * 32 + r);
          const int c = col0 + c16 * 8;
          if constexpr (EPI == EPI_SWIGLU_BWD) {
            // v holds dAct (rounded); gate and up of the same elements come from aux,
            // loaded one read-back ahead
            const uint32_t xoff = xoff_of(i);
            const u32x4 gv = g_next, uv = u_next;
            if (i + 1 < ITER) {
              g_next = bload16(rX, xoff_of(i + 1));
              u_next = bload16(rX, xoff_of(i + 1) + (uint32_t)N * 2);
            }
            u32x4 dgv, duv;
#pragma unroll
            for (int h2 = 0; h2 < 4; ++h2) {
              float dg0, du0, dg1, du1;
              swiglu_bwd<TR>(TR::to_f((uint16_t)(v[h2] & 0xffff)), TR::to_f((uint16_t)(gv[h2] & 0xffff)),
                             TR::to_f((uint16_t)(uv[h2] & 0xffff)), dg0, du0);
              swiglu_bwd<TR>(TR::to_f((uint16_t)(v[h2] >> 16)), TR::to_f((uint16_t)(gv[h2] >> 16)),
                             TR::to_f((uint16_t)(uv[h2] >> 16)), dg1, du1);
              dgv[h2] = pack2(TR::from_f(dg0), TR::from_f(dg1));
              duv[h2] = pack2(TR::from_f(du0), TR::from_f(du1));
            }
            bstore16(rC, xoff, dgv);
            bstore16(rC, xoff + (uint32_t)N * 2, duv);
          } else if (pass == 0) {
            const uint32_t voff = c < N ? (ml * (uint32_t)N + (uint32_t)c) * 2 : 0x80000000u;
            // the down projection's rows (and dgrad's d(hidden) rows) go to the combine /
            // un-permute, which reads them from HBM; the gate/up kernel's act rows
            // are re-read by the down GEMM right away
            bstore16<(KIND == KIND_NT || KIND == KIND_NN) ? kCpolNT : 0>(rC, voff, v);
          } else {
            // EPI_SAVE_GU: gate to columns [0, N), up to [N, 2N) of aux
            const uint32_t xoff =
                c < N ? (ml * (uint32_t)N * 2 + (uint32_t)c + (pass == 2 ? (uint32_t)N : 0u)) * 2 : 0x80000000u;
            bstore16(rX, xoff, v);
          }
        }
      }
    }
  };

  constexpr bool HALF_OK = KIND == KIND_GATHER_SWIGLU && NW == 8 && BN == 256 && NB == 2;
  while (true) {
    if constexpr (HALF_OK) {
      if (N - comp_n0 <= BN / 4) tile(std::true_type{});
      else tile(std::false_type{});
    } else {
      tile(std::false_type{});
    }

    g0 += nk;
    if (issued <= g0) break;  // the ring holds no step of a further tile: this was the last one
    // the issue side has moved on to the next tile (it runs STAGES - 1 >= 1 steps ahead)
    comp_rs = iss_rs;
    comp_re = iss_re;
    comp_n0 = iss_n0;
  }
  // drain: no DMA may still be writing LDS when the workgroup retires
  wait_vmcnt<0>();
}

// Skinny M-grouped GEMM for decode-sized inputs (a few rows per expert).  Its
// load + MFMA step with every K chunk in flight and its epilogue are
// skinny_step.h's, shared with the decode kernel that also routes.
// Workgroup (e, cb) computes output columns [16 cb, 16 cb + 16) for every row
// of expert e with v_mfma_f32_16x16x32: the 16 weight rows are the MFMA A
// operand and up to 16 rows of the expert the B operand, both loaded from
// global memory straight into the operand layout (lane l: row l % 16,
// k = 8 (l / 16) .. +7, 16 contiguous bytes), so the kernel streams each
// weight row once with no LDS staging.  The 4 waves split K; each keeps PD
// 32-wide K chunks of loads in flight (a register ring) and the 4 partial
// sums are added in LDS in wave order.  Rows come in passes of 16 NRB; the
// weights are re-read per pass, which only matters for experts far above the
// decode sizes this kernel is chosen for.
// The grid holds min(E, M) x cblk_n workgroups: workgroup group j serves the
// j-th expert that has rows (found with a ballot over tokens_per_expert), so
// at a token or two no workgroups are spent on the many empty experts.
// CPW > 0: each wave loads exactly CPW 32-wide K chunks (its own, the last
// one repeated past its range), all in flight at once, and the loop is
// unrolled so every MFMA waits only for its own chunk.  In the PD ring the
// loop-carried loads made each iteration wait for every load in flight, one
// memory round trip per PD chunks.  CPW = 0 keeps the ring (large K).
template <typename TR, int KIND, int NRB, int PD, int CPW = 0>
__global__ __launch_bounds__(256) void mgemm_skinny_kernel(const uint16_t* __restrict__ A,
                                                           const int32_t* __restrict__ gather,
                                                           const uint16_t* __restrict__ W, uint16_t* __restrict__ C,
                                                           const int64_t* __restrict__ tpe, int E, int M, int N, int K,
                                                           int cblk_n) {
  static_assert(KIND == KIND_NT || KIND == KIND_GATHER_SWIGLU, "skinny kernel: NT or gate/up");
  constexpr bool SW = KIND == KIND_GATHER_SWIGLU;
  __shared__ SkinnyRed<SW, NRB> red;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = blockIdx.x / cblk_n;  // rank of this group's expert among the experts with rows
  const int c0 = (blockIdx.x - j * cblk_n) * 16;

  // expert e = the j-th with rows, and its first row: prefix of tokens_per_expert, clamped to M
  int e = -1, seen = 0;
  int64_t before = 0;
  for (int c = 0; c < E && e < 0; c += 64) {
    const int ee = c + lane;
    int64_t v = ee < E ? tpe[ee] : 0;
    v = v > 0 ? v : 0;
    const uint64_t nz = __ballot(v > 0);
    const int n_nz = __popcll(nz);
    int64_t part = v;
    if (seen + n_nz > j) {
      const int want = j - seen;
      const int my_rank = __popcll(nz & ((1ull << lane) - 1ull));
      const uint64_t hit = __ballot(v > 0 && my_rank == want);
      const int p = __ffsll((unsigned long long)hit) - 1;
      e = c + p;
      part = lane < p ? v : 0;
    }
    seen += n_nz;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
    before += part;
  }
  if (e < 0) return;  // fewer experts with rows than groups; uniform over the workgroup
  int64_t cnt = tpe[e];
  cnt = cnt > 0 ? cnt : 0;
  const int rs = (int)(before < M ? before : M);
  const int re = (int)(before + cnt < M ? before + cnt : M);
  if (re <= rs) return;  // uniform over the workgroup

  const int w_rows = SW ? 2 * N : N;
  const uint16_t* wg = W + ((int64_t)e * w_rows + c0 + (lane & 15)) * K + (lane >> 4) * 8;
  const uint16_t* wu = SW ? wg + (int64_t)N * K : wg;
  const int nc = K / 32;
  const int kc0 = wave * nc / 4, kc1 = (wave + 1) * nc / 4;

  for (int p = rs; p < re; p += 16 * NRB) {
    const uint16_t* xr[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      int r = p + rb * 16 + (lane & 15);
      r = r < re ? r : re - 1;  // rows past the expert repeat a valid one; their columns are never stored
      const int64_t src = SW ? (int64_t)gather[r] : (int64_t)r;
      xr[rb] = A + src * K + (lane >> 4) * 8;
    }
    floatx4 ag[NRB], au[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      ag[rb] = floatx4{0.f, 0.f, 0.f, 0.f};
      au[rb] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (CPW > 0) {
      skinny_chunks<TR, SW, NRB, CPW>(wg, wu, xr, kc0, kc1, ag, au);
    } else if (kc1 > kc0) {
      u32x4 bg[PD], bu[PD], bx[PD][NRB];
      // loads of chunk kc into ring slot u; chunks past the wave's range reload its last one
      auto load = [&](int u, int kc) __attribute__((always_inline)) {
        const int k = (kc < kc1 ? kc : kc1 - 1) * 32;
        bg[u] = ld16(wg + k);
        if constexpr (SW) bu[u] = ld16(wu + k);
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) bx[u][rb] = ld16(xr[rb] + k);
      };
#pragma unroll
      for (int u = 0; u < PD; ++u) load(u, kc0 + u);
      for (int kc = kc0; kc < kc1; kc += PD) {
#pragma unroll
        for (int u = 0; u < PD; ++u) {
          if (kc + u < kc1) {
#pragma unroll
            for (int rb = 0; rb < NRB; ++rb) {
              ag[rb] = TR::mfma16(bg[u], bx[u][rb], ag[rb]);
              if constexpr (SW) au[rb] = TR::mfma16(bu[u], bx[u][rb], au[rb]);
            }
            load(u, kc + u + PD);
          }
        }
      }
    }
    skinny_publish<SW, NRB>(red, wave, lane, ag, au);
    __syncthreads();
    // waves 0..NRB-1 reduce one row block each: the 4 K quarters in wave order
    skinny_store<TR, SW, NRB>(red, wave, lane, p, re, C, N, c0);
    __syncthreads();  // red[] is reused by the next pass
  }
}

// Wgrad with 8 waves on BA x BB = 256 x 256 tiles of C[e] (128 x 64 per
// wave), both operands DMA-fed as [64 k][cols] slices of a row group and
// read transposed.  Work items are (row group, na-tile, nb-tile), taken
// with one atomic counter per XCD from that XCD's run of the wgrad plan
// (wgrad_plan_kernel: runs of about equal rows, largest groups first), so
// an expert's rows stay in one L2 and skewed loads still balance.  The
// epilogue of a whole expert is staged through the idle ring like the
// M-grouped kernels'; a chunk of a split expert stores fp32 partial sums.
// GB: the B operand's rows are gathered, B[b_index[row]] (B is [b_rows, Nb]),
// as the gate_up wgrad reads the hidden rows of the expert's tokens.  Each lane
// keeps the source rows of its k rows for the next step to be issued, loaded
// one step ahead; the 2-stage ring's wait for all loads before each issue also
// covers those index loads.
template <typename TR, int BA, int BB, int NW, int STAGES, bool GB = false>
__global__ __launch_bounds__(NW * 64, 1) void wgrad_dma8_kernel(const uint16_t* __restrict__ A,
                                                                const uint16_t* __restrict__ B,
                                                                uint16_t* __restrict__ C, WgradPlan plan, int Na,
                                                                int Nb, const int32_t* __restrict__ b_index,
                                                                uint32_t b_bytes) {
  static_assert(!GB || STAGES == 2, "gathered B needs the 2-stage ring (its issue waits for every load)");
  constexpr int WGN = NW / 2;
  constexpr int MB = BA / 64;             // 32-row (na) blocks per wave, 2 waves along na
  constexpr int NB = BB / WGN / 32;       // 32-column (nb) blocks per wave
  constexpr int TA_BYTES = kBK * BA * 2;
  constexpr int TB_BYTES = kBK * BB * 2;
  constexpr int STAGE_BYTES = TA_BYTES + TB_BYTES;
  constexpr int RPI_A = 1024 / (BA * 2), RPI_B = 1024 / (BB * 2);  // k rows per 1 KB instruction
  constexpr int LPR_A = BA / 8, LPR_B = BB / 8;                     // lanes per k row
  constexpr int KR = kBK / NW;                                       // k rows loaded per wave
  constexpr int IA = KR / RPI_A, IB = KR / RPI_B;
  constexpr int PER = IA + IB;
  static_assert(IA >= 1 && IB >= 1 && NB >= 1, "tile split");
  static_assert(STAGES * STAGE_BYTES <= 160 * 1024, "LDS ring exceeds 160 KB");
  __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE_BYTES];
  __shared__ int s_tile;
  __shared__ uint32_t s_gi[GB ? NW : 1][GB ? IB : 1][64];
  const __amdgpu_buffer_rsrc_t rI = make_rsrc(b_index, GB ? 0x7ffffffcu : 0u);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  const int ta_n = (Na + BA - 1) / BA, tb_n = (Nb + BB - 1) / BB;
  const int per_e = ta_n * tb_n;
  const int xcd = blockIdx.x & 7;
  const int run0 = plan.info[2 * xcd];
  const int items = plan.info[2 * xcd + 1] * per_e;

  while (true) {
    if (tid == 0) s_tile = atomicAdd(&plan.info[32 + xcd], 1);
    __syncthreads();  // also orders the previous tile's staging reads before this tile's DMA
    const int t = s_tile;
    __syncthreads();
    if (t >= items) break;
    const WGroup grp = plan.groups[plan.order[run0 + t / per_e]];
    const int rem = t % per_e;
    const int a0 = (rem / tb_n) * BA, b0 = (rem % tb_n) * BB;
    const int e = grp.expert, rs = grp.row_start, re = grp.row_end;
    const int slot = __builtin_amdgcn_readfirstlane(grp.slot);
    const int nk = (re - rs + kBK - 1) / kBK;
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(A + (int64_t)rs * Na, (uint32_t)(re - rs) * (uint32_t)Na * 2);
    const __amdgpu_buffer_rsrc_t rB =
        GB ? make_rsrc(B, b_bytes) : make_rsrc(B + (int64_t)rs * Nb, (uint32_t)(re - rs) * (uint32_t)Nb * 2);
    uint32_t oa[IA], ob[IB];
    // GB: source rows of this wave's B k rows for the next step to issue, DMA'd
    // into s_gi (one dword per lane) during the step before and read back at
    // the issue; the step's vmcnt(0) wait (2-stage ring) covers that DMA
#pragma unroll
    for (int i = 0; i < IA; ++i) {
      const int kr = wave * KR + i * RPI_A + lane / LPR_A;
      const int lc = (lane % LPR_A) ^ kr_swz(kr);
      int ca = a0 + lc * 8;
      ca = ca < Na ? ca : Na - 8;
      oa[i] = ((uint32_t)kr * (uint32_t)Na + (uint32_t)ca) * 2;
    }
#pragma unroll
    for (int i = 0; i < IB; ++i) {
      const int kr = wave * KR + i * RPI_B + lane / LPR_B;
      const int lc = (lane % LPR_B) ^ kr_swz(kr);
      int cb = b0 + lc * 8;
      cb = cb < Nb ? cb : Nb - 8;
      ob[i] = GB ? (uint32_t)cb * 2 : ((uint32_t)kr * (uint32_t)Nb + (uint32_t)cb) * 2;
    }
    auto gi_row = [&](int kt, int i) __attribute__((always_inline)) {
      return rs + kt * kBK + wave * KR + i * RPI_B + lane / LPR_B;
    };
    auto load_gi = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        const int row = gi_row(kt, i);
        dma4t(rI, reinterpret_cast<char*>(&s_gi[wave][i][0]), (uint32_t)(row < re ? row : re - 1) * 4u);
      }
    };
    if constexpr (GB) {
      if (nk > 0) {
        load_gi(0);
        wait_vmcnt<0>();
      }
    }
    auto issue = [&](int kt, int stage) __attribute__((always_inline)) {
      char* sa = smem + stage * STAGE_BYTES;
      char* sb = sa + TA_BYTES;
      const uint32_t sofa = (uint32_t)kt * kBK * (uint32_t)Na * 2;
      const uint32_t sofb = (uint32_t)kt * kBK * (uint32_t)Nb * 2;
#pragma unroll
      for (int i = 0; i < IA; ++i) dma16t(rA, sa + (wave * KR + i * RPI_A) * (BA * 2), oa[i], sofa);
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        if constexpr (GB)
          dma16t(rB, sb + (wave * KR + i * RPI_B) * (BB * 2),
                 gi_row(kt, i) < re ? s_gi[wave][i][lane] * (uint32_t)Nb * 2 + ob[i] : 0x80000000u, 0);
        else
          dma16t(rB, sb + (wave * KR + i * RPI_B) * (BB * 2), ob[i], sofb);
      }
      if constexpr (GB) load_gi(kt + 1);
    };

    floatx16 acc[NB][MB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int a = 0; a < MB; ++a)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][a][v] = 0.0f;

#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st)
      if (st < nk) issue(st, st);
    // 2-stage ring: the second half of the waves issues its share of a stage
    // after its first sub-step of MFMAs (see mgemm_dma_kernel's STAGGER)
    constexpr bool STAGGER = NW == 8 && STAGES == 2;
    const bool late = STAGGER && wave >= NW / 2;
    for (int kt = 0; kt < nk; ++kt) {
      wait_stages<PER, STAGES - 2>(min(STAGES - 2, nk - 1 - kt));
      barrier_lds();
      const bool due = kt + STAGES - 1 < nk;
      if (due && !late) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
      const char* la = smem + (kt % STAGES) * STAGE_BYTES;
      const char* lb = la + TA_BYTES;
      u32x4 fb[2][NB], fa[2][MB];
      auto load_frags = [&](int sub, u32x4 (&xb)[NB], u32x4 (&xa)[MB]) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < NB; ++b) xb[b] = tr_operand<BB>(lb, wn * (BB / WGN) + b * 32, sub, lane);
#pragma unroll
        for (int a = 0; a < MB; ++a) xa[a] = tr_operand<BA>(la, wm * (BA / 2) + a * 32, sub, lane);
      };
      load_frags(0, fb[0], fa[0]);
#pragma unroll
      for (int sub = 0; sub < kBK / 16; ++sub) {
        if (sub + 1 < kBK / 16) load_frags(sub + 1, fb[(sub + 1) & 1], fa[(sub + 1) & 1]);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int a = 0; a < MB; ++a) acc[b][a] = TR::mfma32(fb[sub & 1][b], fa[sub & 1][a], acc[b][a]);
        if (sub == 0 && due && late) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
      }
    }

    // Epilogue: no DMA is in flight (every issued step was consumed), so once
    // all waves pass the barrier the whole ring is free for staging.
    if (slot >= 0) {
      // a chunk of a split expert: fp32 partial sums straight from the accumulators
      float* P = plan.partials + (int64_t)slot * Na * Nb;
#pragma unroll
      for (int a = 0; a < MB; ++a) {
        const int na = a0 + wm * (BA / 2) + a * 32 + (lane & 31);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int nb = b0 + wn * (BB / WGN) + b * 32 + gq * 8 + (lane >> 5) * 4;
            if (na < Na && nb < Nb)
              *reinterpret_cast<floatx4*>(P + (int64_t)na * Nb + nb) =
                  floatx4{acc[b][a][gq * 4 + 0], acc[b][a][gq * 4 + 1], acc[b][a][gq * 4 + 2], acc[b][a][gq * 4 + 3]};
          }
      }
    } else {
      constexpr int WCOLS = BB / WGN;                     // output columns (nb) per wave
      constexpr int PITCH = WCOLS * 2;
      constexpr int C8 = PITCH / 8;
      constexpr int RP = 256 / PITCH;
      constexpr int REGION = STAGES * STAGE_BYTES / NW;
      constexpr int FIT = REGION / (32 * PITCH);
      constexpr int APP = FIT >= 4 && MB >= 4 ? 4 : (FIT >= 2 && MB >= 2 ? 2 : 1);
      constexpr int LPR = PITCH / 16;
      constexpr int RPI = 64 / LPR;
      static_assert(FIT >= 1 && MB % APP == 0 && RP * C8 == 32, "staging layout");
      const int rows = min(BA, Na - a0);
      const __amdgpu_buffer_rsrc_t rC =
          make_rsrc(C + ((int64_t)e * Na + a0) * Nb, (uint32_t)rows * (uint32_t)Nb * 2);
      char* stg = smem + wave * REGION;
      const int col0 = b0 + wn * WCOLS;
      barrier_lds();
#pragma unroll
      for (int p0 = 0; p0 < MB; p0 += APP) {
#pragma unroll
        for (int a = p0; a < p0 + APP; ++a) {
          const int r = (a - p0) * 32 + (lane & 31);
          const int g = (r / RP) % C8;
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              const int ch8 = (b * 32 + gq * 8) / 4 + (lane >> 5);
              *reinterpret_cast<u32x2*>(stg + r * PITCH + ((ch8 ^ g) << 3)) =
                  pack4<TR>(acc[b][a][gq * 4 + 0], acc[b][a][gq * 4 + 1], acc[b][a][gq * 4 + 2], acc[b][a][gq * 4 + 3]);
            }
        }
#pragma unroll
        for (int i = 0; i < APP * 32 / RPI; ++i) {
          const int r = i * RPI + lane / LPR;
          const int c16 = lane % LPR;
          const int g = (r / RP) % C8;
          u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * PITCH + ((c16 ^ (g >> 1)) << 4));
          if (g & 1) v = u32x4{v[2], v[3], v[0], v[1]};
          const uint32_t ml = (uint32_t)(wm * (BA / 2) + p0 * 32 + r);
          const int c = col0 + c16 * 8;
          const uint32_t voff = c < Nb ? (ml * (uint32_t)Nb + (uint32_t)c) * 2 : 0x80000000u;
          bstore16<kCpolNT>(rC, voff, v);  // weight gradients: written once, read by the optimizer
        }
      }
    }
  }
  wait_vmcnt<0>();
}

// Wgrad fed by DMA: both operands are [64 rows][128 cols] tiles of a row
// group; rows past the group's end read as zeros (buffer bounds).  Work
// items (group, na-tile, nb-tile) come from one atomic counter over all
// groups of the wgrad plan in its order.
// GB: gathered B rows, as in wgrad_dma8_kernel.  F32OUT: C is fp32 (the
// per-split partial sums of the router gate's weight gradient).
template <typename TR, int STAGES, bool GB = false, bool F32OUT = false>
__global__ __launch_bounds__(kThreads, 1) void wgrad_dma_kernel(const uint16_t* __restrict__ A,
                                                               const uint16_t* __restrict__ B,
                                                               uint16_t* __restrict__ C, WgradPlan plan, int Na,
                                                               int Nb, const int32_t* __restrict__ b_index,
                                                               uint32_t b_bytes) {
  static_assert(!GB || STAGES == 2, "gathered B needs the 2-stage ring (its issue waits for every load)");
  constexpr int BA = 128, BB = 128;
  constexpr int MB = BA / 64, NB = BB / 64;
  constexpr int T_BYTES = kBK * 128 * 2;
  constexpr int STAGE_BYTES = 2 * T_BYTES;
  constexpr int PER = 8;  // 4 + 4 loads per wave per stage
  __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE_BYTES];
  __shared__ int s_tile;
  __shared__ uint32_t s_gi[GB ? 4 : 1][GB ? 4 : 1][64];  // [wave][i][lane], as in wgrad_dma8_kernel
  const __amdgpu_buffer_rsrc_t rI = make_rsrc(b_index, GB ? 0x7ffffffcu : 0u);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wa = wave >> 1, wb = wave & 1;
  const int ta_n = (Na + BA - 1) / BA, tb_n = (Nb + BB - 1) / BB;
  const int per_e = ta_n * tb_n;
  const int total = plan.info[16] * per_e;

  while (true) {
    if (tid == 0) s_tile = atomicAdd(&plan.info[32], 1);
    __syncthreads();
    const int t = s_tile;
    __syncthreads();
    if (t >= total) break;
    const WGroup grp = plan.groups[plan.order[t / per_e]];
    const int rem = t % per_e;
    const int a0 = (rem / tb_n) * BA, b0 = (rem % tb_n) * BB;
    const int e = grp.expert, rs = grp.row_start, re = grp.row_end;
    const int slot = __builtin_amdgcn_readfirstlane(grp.slot);
    const int nk = (re - rs + kBK - 1) / kBK;
    const __amdgpu_buffer_rsrc_t rA = make_rsrc(A + (int64_t)rs * Na, (uint32_t)(re - rs) * (uint32_t)Na * 2);
    const __amdgpu_buffer_rsrc_t rB =
        GB ? make_rsrc(B, b_bytes) : make_rsrc(B + (int64_t)rs * Nb, (uint32_t)(re - rs) * (uint32_t)Nb * 2);
    uint32_t oa[4], ob[4];
    // GB: source rows of this wave's B k rows for the next step to issue, in s_gi (see wgrad_dma8_kernel)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kr = wave * 16 + i * 4 + (lane >> 4);
      const int lc = (lane & 15) ^ kr_swz(kr);
      int ca = a0 + lc * 8, cb = b0 + lc * 8;
      ca = ca < Na ? ca : Na - 8;
      cb = cb < Nb ? cb : Nb - 8;
      oa[i] = ((uint32_t)kr * (uint32_t)Na + (uint32_t)ca) * 2;
      ob[i] = GB ? (uint32_t)cb * 2 : ((uint32_t)kr * (uint32_t)Nb + (uint32_t)cb) * 2;
    }
    auto gi_row = [&](int kt, int i) __attribute__((always_inline)) {
      return rs + kt * kBK + wave * 16 + i * 4 + (lane >> 4);
    };
    auto load_gi = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = gi_row(kt, i);
        dma4t(rI, reinterpret_cast<char*>(&s_gi[wave][i][0]), (uint32_t)(row < re ? row : re - 1) * 4u);
      }
    };
    if constexpr (GB) {
      if (nk > 0) {
        load_gi(0);
        wait_vmcnt<0>();
      }
    }
    auto issue = [&](int kt, int stage) {
      char* sa = smem + stage * STAGE_BYTES;
      char* sb = sa + T_BYTES;
      const uint32_t sofa = (uint32_t)kt * kBK * (uint32_t)Na * 2;
      const uint32_t sofb = (uint32_t)kt * kBK * (uint32_t)Nb * 2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dma16t(rA, sa + (wave * 16 + i * 4) * 256, oa[i], sofa);
        if constexpr (GB)
          dma16t(rB, sb + (wave * 16 + i * 4) * 256,
                 gi_row(kt, i) < re ? s_gi[wave][i][lane] * (uint32_t)Nb * 2 + ob[i] : 0x80000000u, 0);
        else
          dma16t(rB, sb + (wave * 16 + i * 4) * 256, ob[i], sofb);
      }
      if constexpr (GB) load_gi(kt + 1);
    };

    floatx16 acc[NB][MB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int a = 0; a < MB; ++a)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[b][a][v] = 0.0f;

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
      if (s < nk) issue(s, s);
    for (int kt = 0; kt < nk; ++kt) {
      wait_stages<PER, STAGES - 2>(min(STAGES - 2, nk - 1 - kt));
      barrier_lds();
      if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
      const char* la = smem + (kt % STAGES) * STAGE_BYTES;
      const char* lb = la + T_BYTES;
      u32x4 fb[2][NB], fa[2][MB];
      auto load_frags = [&](int s, u32x4 (&xb)[NB], u32x4 (&xa)[MB]) {
#pragma unroll
        for (int b = 0; b < NB; ++b) xb[b] = tr_operand<128>(lb, wb * (BB / 2) + b * 32, s, lane);
#pragma unroll
        for (int a = 0; a < MB; ++a) xa[a] = tr_operand<128>(la, wa * (BA / 2) + a * 32, s, lane);
      };
      load_frags(0, fb[0], fa[0]);
#pragma unroll
      for (int s = 0; s < kBK / 16; ++s) {
        if (s + 1 < kBK / 16) load_frags(s + 1, fb[(s + 1) & 1], fa[(s + 1) & 1]);
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int a = 0; a < MB; ++a) acc[b][a] = TR::mfma32(fb[s & 1][b], fa[s & 1][a], acc[b][a]);
      }
    }
    barrier_lds();

    uint16_t* Ce = C + (int64_t)e * Na * Nb;
    // fp32 destination: a split expert's partial slot, or C itself for F32OUT
    float* Cf = slot >= 0 ? plan.partials + (int64_t)slot * Na * Nb : reinterpret_cast<float*>(C) + (int64_t)e * Na * Nb;
#pragma unroll
    for (int a = 0; a < MB; ++a) {
      const int na = a0 + wa * (BA / 2) + a * 32 + (lane & 31);
      if (na >= Na) continue;
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int nb = b0 + wb * (BB / 2) + b * 32 + g * 8 + (lane >> 5) * 4;
          if (nb >= Nb) continue;
          if (F32OUT || slot >= 0)
            *reinterpret_cast<floatx4*>(Cf + (int64_t)na * Nb + nb) =
                floatx4{acc[b][a][g * 4 + 0], acc[b][a][g * 4 + 1], acc[b][a][g * 4 + 2], acc[b][a][g * 4 + 3]};
          else
            st8(Ce + (int64_t)na * Nb + nb, pack4<TR>(acc[b][a][g * 4 + 0], acc[b][a][g * 4 + 1],
                                                     acc[b][a][g * 4 + 2], acc[b][a][g * 4 + 3]));
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int kBMMin = 128;  // smallest BM any launch uses (sizes the tile table)

// Persistent grid: (CUs - margin, at least 1) x resident workgroups per CU,
// rounded down to a multiple of 8 (at least 8: the tile lists are split over
// the 8 XCDs).  As the reference's grid of SM count - SM_MARGIN, at least 1
// (models/moe_triton_grouped_gemm.py:50-52).  CU count and occupancy are
// queried once per kernel (and LDS size); the margin is read per launch from
// the library configuration.
struct GridCache {
  int cus = 0, occ = 0;
  size_t lds = ~size_t(0);
  template <typename KernelT>
  int get(KernelT kernel, int threads = kThreads, size_t dyn_lds = 0) {
    if (occ == 0 || lds != dyn_lds) {
      int dev = 0, c = 0, o = 1;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c < 1)
        c = 8;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, kernel, threads, dyn_lds) != hipSuccess || o < 1) o = 1;
      cus = c;
      occ = o;
      lds = dyn_lds;
    }
    const int usable = cus - config().cu_margin;
    int g = (usable < 1 ? 1 : usable) * occ;
    g = (g / 8) * 8;
    return g < 8 ? 8 : g;
  }
};

int check_common(int64_t M, int32_t E, int dtype, const void* ws, size_t ws_bytes) {
  if (M < 0 || E < 1) return HRM_MOE_ERR_INVALID;
  if (dtype != HRM_MOE_BF16 && dtype != HRM_MOE_F16) return HRM_MOE_ERR_DTYPE;
  if (E > kMaxExperts || M >= (int64_t(1) << 31)) return HRM_MOE_ERR_UNSUPPORTED;
  // the size hrm_moe_grouped_gemm_workspace_size reports: the M-tile plan or the wgrad plan
  const size_t need = gemm_ws_bytes(M, E, kBMMin) > wgrad_plan_bytes(E) ? gemm_ws_bytes(M, E, kBMMin)
                                                                         : wgrad_plan_bytes(E);
  if (!ws || ws_bytes < need) return HRM_MOE_ERR_WORKSPACE;
  return HRM_MOE_OK;
}

// Name of the kernel instantiation the latest launch of each kind used, in
// the form a profiler's demangled kernel name contains (for matching traces
// and counter summaries to what ran).
char g_last_kernel[3][128];
template <typename TR>
constexpr const char* tr_name() { return std::is_same<TR, BF16>::value ? "hrm::BF16" : "hrm::F16"; }

template <typename TR, int KIND, int BM, int BN>
int launch_mgemm(const void* A, const int32_t* gather, const void* W, const int64_t* tpe, int64_t M, int N, int K,
                 int E, void* C, void* workspace, void* stream) {
  GemmWs w = carve(workspace, M, E, kBMMin);
  const int max_tiles = (int)((M + BM - 1) / BM + E);
  HRM_LAUNCH(plan_kernel, dim3(1), dim3(1024), 0, stream, tpe, E, M, BM, w.tiles, max_tiles, w.count, w.row_offsets,
             w.work_counter);
  const int tiles_n = KIND == KIND_GATHER_SWIGLU ? (N + BN / 2 - 1) / (BN / 2) : (N + BN - 1) / BN;
  auto kern = mgemm_kernel<TR, KIND, BM, BN>;
  snprintf(g_last_kernel[KIND], sizeof(g_last_kernel[KIND]), "mgemm_kernel<%s, %d, %d, %d>", tr_name<TR>(), KIND, BM,
           BN);
  static GridCache gc;
  const int grid = gc.get(kern);
  HRM_LAUNCH(kern, dim3(grid), dim3(kThreads), 0, stream, (const uint16_t*)A, gather, (const uint16_t*)W,
             (uint16_t*)C, w.tiles, w.count, N, K, tiles_n);
  return HRM_MOE_OK;
}

template <typename TR, int KIND, int BM, int BN, int STAGES, int NW, int BK, int EPI = EPI_PLAIN, bool WNT = false>
int launch_mgemm_dma(const void* A, const int32_t* gather, const void* W, const int64_t* tpe, int64_t M, int N,
                     int K, int E, int64_t a_rows, void* C, void* workspace, void* stream, void* aux = nullptr) {
  (void)workspace;  // the DMA kernels plan their tiles themselves
  const int tiles_n = KIND == KIND_GATHER_SWIGLU ? (N + BN / 2 - 1) / (BN / 2) : (N + BN - 1) / BN;
  auto kern = mgemm_dma_kernel<TR, KIND, BM, BN, STAGES, NW, BK, EPI, WNT>;
  snprintf(g_last_kernel[KIND], sizeof(g_last_kernel[KIND]), "mgemm_dma_kernel<%s, %d, %d, %d, %d, %d, %d, %d, %s>",
           tr_name<TR>(), KIND, BM, BN, STAGES, NW, BK, EPI, WNT ? "true" : "false");
  const size_t plan_bytes = sizeof(int) * 3 * (size_t)E;
  static GridCache gc;
  const int grid = gc.get(kern, NW * 64, plan_bytes);
  HRM_LAUNCH(kern, dim3(grid), dim3(NW * 64), plan_bytes, stream, (const uint16_t*)A, gather, (const uint16_t*)W,
             (uint16_t*)C, tpe, E, (int)M, N, K, tiles_n, (uint32_t)(a_rows * K * 2), (uint16_t*)aux);
  return HRM_MOE_OK;
}

// Tile shape, pipeline depth, waves and K step of the DMA kernels.
// Default: 256 x 256 tiles with 8 waves (2 per SIMD, 128 x 64 per wave) and 2
// stages of 64-wide K steps (128 KB of LDS) when experts average at least 256
// rows and the weight rows split into whole 256-row tiles (the gate/up kernel
// also supports a last half tile of 64 gate + 64 up rows when selected
// explicitly); when experts average at most 16 rows, 32 x 256 tiles (4 waves
// along N, 4 stages, 144 KB) for gate/up and 32 x 128 tiles (5 stages, 100 KB)
// for the down projection (a 32 x 128 choice for gate/up runs 32 x 256);
// up to 48 rows, 64 x 128 tiles with 3 stages (72 KB, two workgroups per CU);
// otherwise 128 x 128 tiles, 4 waves, 2 stages (64 KB of LDS, two workgroups
// per CU).  The large
// tile halves LDS and L2 traffic per flop; the small one wastes less on ragged
// experts and on widths that are not multiples of 256.
// HRM_MOE_GEMM_CFG="<rows>x<cols>x<stages>x<waves>x<kstep>" (e.g.
// "256x256x4x8x32") overrides the choice with one of the built variants.
struct MCfg {
  int bm, bn, stages, waves, bk;
};
bool mcfg_built(const MCfg& c) {
  if (c.bm == 32)
    return c.waves == 4 && c.bk == 64 && ((c.bn == 256 && c.stages == 4) || (c.bn == 128 && (c.stages == 4 || c.stages == 5)));
  if (c.bm == 256 && c.bn == 128 && c.waves == 4) return c.bk == 32 && (c.stages == 2 || c.stages == 3);
  if (c.bm == 128 && c.bn == 128 && c.waves == 4)
    return (c.bk == 64 && (c.stages == 2 || c.stages == 3)) || (c.bk == 32 && (c.stages == 4 || c.stages == 5));
  if (c.bm == 64 && c.bn == 128 && c.waves == 4) return c.bk == 64 && (c.stages == 3 || c.stages == 5);
  if (c.bm == 256 && c.bn == 256 && c.waves == 8)
    return (c.bk == 64 && c.stages == 2) || (c.bk == 32 && c.stages == 4);
  return false;
}
MCfg mgemm_cfg(int64_t M, int E, int64_t w_rows, bool gate_up, bool nn = false) {
  const Config& cf = config();  // HRM_MOE_GEMM_CFG (tests switch variants and reload the configuration)
  if (cf.gemm_bm) {
    const MCfg c{cf.gemm_bm, cf.gemm_bn, cf.gemm_stages, cf.gemm_waves, cf.gemm_bk};
    if (mcfg_built(c)) return c;
  }
  // 256 x 256 tiles with 8 waves when experts average >= 256 rows and the
  // weight rows fill whole tiles (for the gate/up kernel: 2I a multiple of 256;
  // at XL, I = 512, the layer measured 792 against 814 us, and 1550 against
  // 1650 us at XL128).  L's gate/up (2I = 896) stays on 128 x 128: with a half
  // tile for its last N tile it measured no faster.
  // The NN (dgrad) kernel takes 256 x 256 tiles even when its width is not a
  // multiple of 256: at L's dact (N = 448) they measured 203 us against 272 us
  // for 128 x 128 tiles, whose higher LDS and DMA traffic per flop costs more
  // than the idle columns of the last N tile.
  if (M >= (int64_t)E * 256 && (nn || w_rows % 256 == 0)) return MCfg{256, 256, 2, 8, 64};
  // Decode sizes (experts average at most 16 rows): the GEMM streams weights,
  // and 32-row tiles leave LDS for 4 stages of 256 weight rows (3 K steps in
  // flight).  Decode layer at H = 1536, I = 512: T = 8 88.8 -> 82.8 us,
  // T = 64 104.8 -> 100.8 us; at T = 256 (32 rows per expert) 128 x 128 stays
  // faster (111.5 against 120.1 us).  The down projection takes 32 x 128
  // tiles with 5 stages: twice the workgroups, each streaming half the weight
  // rows, so all CUs stream at T = 8 (255 -> 510 tiles; layer 62.6 -> 61.3 us,
  // T = 64 85.0 -> 83.8 us).  The gate/up pair needs two 32-column blocks per
  // wave, so its N tile stays 256.
  if (!nn && M <= (int64_t)E * 16) return gate_up ? MCfg{32, 256, 4, 4, 64} : MCfg{32, 128, 5, 4, 64};
  // Up to 48 rows per expert on average: 64 x 128 tiles with 3 stages (72 KB,
  // two workgroups per CU), each expert's rows mostly in one M tile, weight
  // rows two K steps ahead.  Decode layer at T = 256 (32 rows per expert):
  // 94.3/93.1 -> 87.7/87.7 us against 128 x 128 with 2 stages; 5 stages (one
  // workgroup per CU) 89.3/88.5 us.
  if (!nn && M <= (int64_t)E * 48) return MCfg{64, 128, 3, 4, 64};
  return MCfg{128, 128, 2, 4, 64};
}

template <typename TR, int KIND>
int dispatch_mgemm_t(const void* A, const int32_t* gather, const void* W, const int64_t* tpe, int64_t M, int N, int K,
                     int E, int64_t a_rows, void* C, void* workspace, void* stream) {
  const int64_t w_rows = KIND == KIND_GATHER_SWIGLU ? 2 * (int64_t)N : (KIND == KIND_NN ? (int64_t)K : (int64_t)N);
  const int64_t w_cols = KIND == KIND_NN ? (int64_t)N : (int64_t)K;
  const bool dma = K % kBK == 0 && a_rows * K * 2 < (int64_t(1) << 32) && w_rows * w_cols * 2 < (int64_t(1) << 32);
  if (!dma) {
    // K not a multiple of 64 (or operands beyond 32-bit buffer offsets): register-staged kernel
    return M >= (int64_t)E * 192 ? launch_mgemm<TR, KIND, 256, 128>(A, gather, W, tpe, M, N, K, E, C, workspace, stream)
                                 : launch_mgemm<TR, KIND, 128, 128>(A, gather, W, tpe, M, N, K, E, C, workspace, stream);
  }
  // weight rows spanned by the N tiles: 2N for the gate/up pair, else N
  // Decode sizes: at most one row per four experts on average (a token or two
  // at top-8 of 64) -> weight-streaming skinny kernel.  Measured against the
  // tiled kernels it wins only there (T = 1: gate_up 17 vs 26 us); from about
  // one row per expert the tiled DMA kernels stream weights faster.
  // HRM_MOE_SKINNY=1 forces it up to 16 rows per expert, =0 turns it off
  // (tests compare both paths).
  if constexpr (KIND != KIND_NN) {
    const bool force = config().skinny == 1, off = config().skinny == 0;
    const int64_t limit = force ? (int64_t)E * 16 : (int64_t)E / 4;
    const bool skinny_ok = !off && M <= limit && K % 32 == 0 && N % 16 == 0;
    if (skinny_ok) {
      const int cblk_n = N / 16;
      const int groups = (int)(M < (int64_t)E ? M : (int64_t)E);  // at most one group per expert with rows
      const dim3 grid((unsigned)(groups * cblk_n));
#define HRM_SK(NRB_, CPW_)                                                                                  \
  HRM_LAUNCH((mgemm_skinny_kernel<TR, KIND, NRB_, 4, CPW_>), grid, dim3(256), 0, stream, (const uint16_t*)A, \
             gather, (const uint16_t*)W, (uint16_t*)C, tpe, E, (int)M, N, K, cblk_n)
      // chunks per wave (4 waves split K in 32-wide chunks): all of a wave's loads in flight at once up to 16
      const int need = (K / 32 + 3) / 4;
      const int cpw = need <= 4 ? 4 : (need <= 8 ? 8 : (need <= 12 ? 12 : (need <= 16 ? 16 : 0)));
      const int nrb = M <= (int64_t)E * 4 ? 1 : 2;  // up to 4 rows per expert on average: one 16-row block per pass
      snprintf(g_last_kernel[KIND], sizeof(g_last_kernel[KIND]), "mgemm_skinny_kernel<%s, %d, %d, 4, %d>",
               tr_name<TR>(), KIND, nrb, cpw);
      if (nrb == 1) {
        if (cpw == 4) HRM_SK(1, 4);
        else if (cpw == 8) HRM_SK(1, 8);
        else if (cpw == 12) HRM_SK(1, 12);
        else if (cpw == 16) HRM_SK(1, 16);
        else HRM_SK(1, 0);
      } else {
        if (cpw == 4) HRM_SK(2, 4);
        else if (cpw == 8) HRM_SK(2, 8);
        else if (cpw == 12) HRM_SK(2, 12);
        else if (cpw == 16) HRM_SK(2, 16);
        else HRM_SK(2, 0);
      }
#undef HRM_SK
      return HRM_MOE_OK;
    }
  }
  MCfg c = mgemm_cfg(M, E, KIND == KIND_GATHER_SWIGLU ? 2 * (int64_t)N : (int64_t)N, KIND == KIND_GATHER_SWIGLU,
                     KIND == KIND_NN);
  if (K % c.bk != 0) c = MCfg{128, 128, 2, 4, 64};
  // the ring may run at most one tile ahead: STAGES - 1 <= K / BK.  The
  // 32- and 64-row tiles are built with 3 to 5 stages only, so short K (the
  // down projection of experts narrower than 256, or gate/up below a hidden
  // size of 192) takes the 2-stage 128 x 128 tile.
  if (c.stages - 1 > K / c.bk) {
    if (c.bm == 32 || c.bm == 64) c = MCfg{128, 128, 2, 4, 64};
    else if (c.bk == 32) c = MCfg{c.bm, c.bn, 2, c.waves, 64};
    else c.stages = 2;
  }
#define HRM_MG(BM_, BN_, ST_, NW_, BK_) \
  return launch_mgemm_dma<TR, KIND, BM_, BN_, ST_, NW_, BK_>(A, gather, W, tpe, M, N, K, E, a_rows, C, workspace, stream)
  if constexpr (KIND != KIND_GATHER_SWIGLU) {
    if (c.bm == 32 && c.bn == 128) {
      if (c.stages == 5) HRM_MG(32, 128, 5, 4, 64);
      HRM_MG(32, 128, 4, 4, 64);
    }
  }
  if (c.bm == 32) HRM_MG(32, 256, 4, 4, 64);
  if (c.bm == 64) {
    if (KIND != KIND_NN && M <= (int64_t)E * 128) {
      if (c.stages == 5)
        return launch_mgemm_dma<TR, KIND, 64, 128, 5, 4, 64, EPI_PLAIN, true>(A, gather, W, tpe, M, N, K, E, a_rows, C,
                                                                             workspace, stream);
      return launch_mgemm_dma<TR, KIND, 64, 128, 3, 4, 64, EPI_PLAIN, true>(A, gather, W, tpe, M, N, K, E, a_rows, C,
                                                                           workspace, stream);
    }
    if (c.stages == 5) HRM_MG(64, 128, 5, 4, 64);
    HRM_MG(64, 128, 3, 4, 64);
  }
  if (c.bm == 256 && c.bn == 128) {
    if (c.stages == 2) HRM_MG(256, 128, 2, 4, 32);
    HRM_MG(256, 128, 3, 4, 32);
  }
  if (c.bm == 256) {
    if (c.bk == 32) HRM_MG(256, 256, 4, 8, 32);
    HRM_MG(256, 256, 2, 8, 64);
  }
  if (c.bk == 32) {
    if (c.stages == 5) HRM_MG(128, 128, 5, 4, 32);
    HRM_MG(128, 128, 4, 4, 32);
  }
  if (c.stages == 3) HRM_MG(128, 128, 3, 4, 64);
  // experts averaging at most 128 rows (one M tile): weights read once, so
  // loaded non-temporally (decode T = 256 108.6 -> 99.4 us, T = 512 113.5 ->
  // 104.7 us; at L's 2048 rows per expert the same loads were much slower)
  if (KIND != KIND_NN && M <= (int64_t)E * 128)
    return launch_mgemm_dma<TR, KIND, 128, 128, 2, 4, 64, EPI_PLAIN, true>(A, gather, W, tpe, M, N, K, E, a_rows, C,
                                                                          workspace, stream);
  HRM_MG(128, 128, 2, 4, 64);
#undef HRM_MG
}

// Training-path epilogues (EPI_SAVE_GU, EPI_SWIGLU_BWD): DMA kernels only,
// on the two default tile shapes.
template <typename TR, int KIND, int EPI>
int dispatch_mgemm_epi_t(const void* A, const int32_t* gather, const void* W, const int64_t* tpe, int64_t M, int N,
                         int K, int E, int64_t a_rows, void* C, void* aux, void* stream) {
  const int64_t w_rows = KIND == KIND_GATHER_SWIGLU ? 2 * (int64_t)N : (KIND == KIND_NN ? (int64_t)K : (int64_t)N);
  const int64_t w_cols = KIND == KIND_NN ? (int64_t)N : (int64_t)K;
  const int64_t c_cols = EPI == EPI_SWIGLU_BWD ? 2 * (int64_t)N : (int64_t)N;
  if (K % kBK != 0 || a_rows * K * 2 >= (int64_t(1) << 32) || w_rows * w_cols * 2 >= (int64_t(1) << 32) ||
      M * 2 * (int64_t)N * 2 >= (int64_t(1) << 32) || M * c_cols * 2 >= (int64_t(1) << 32))
    return HRM_MOE_ERR_UNSUPPORTED;
  const MCfg c = mgemm_cfg(M, E, KIND == KIND_GATHER_SWIGLU ? 2 * (int64_t)N : (int64_t)N, KIND == KIND_GATHER_SWIGLU,
                           KIND == KIND_NN);
  if (c.bm == 256 && c.bn == 256 && c.waves == 8 && c.bk == 64 && c.stages == 2)
    return launch_mgemm_dma<TR, KIND, 256, 256, 2, 8, 64, EPI>(A, gather, W, tpe, M, N, K, E, a_rows, C, nullptr,
                                                               stream, aux);
  return launch_mgemm_dma<TR, KIND, 128, 128, 2, 4, 64, EPI>(A, gather, W, tpe, M, N, K, E, a_rows, C, nullptr, stream,
                                                             aux);
}

template <int KIND, int EPI>
int dispatch_mgemm_epi(int dtype, const void* A, const int32_t* gather, const void* W, const int64_t* tpe, int64_t M,
                       int N, int K, int E, int64_t a_rows, void* C, void* aux, void* stream) {
  if (dtype == HRM_MOE_BF16)
    return dispatch_mgemm_epi_t<BF16, KIND, EPI>(A, gather, W, tpe, M, N, K, E, a_rows, C, aux, stream);
  return dispatch_mgemm_epi_t<F16, KIND, EPI>(A, gather, W, tpe, M, N, K, E, a_rows, C, aux, stream);
}

template <int KIND>
int dispatch_mgemm(int dtype, const void* A, const int32_t* gather, const void* W, const int64_t* tpe, int64_t M,
                   int N, int K, int E, int64_t a_rows, void* C, void* workspace, void* stream) {
  if (dtype == HRM_MOE_BF16) return dispatch_mgemm_t<BF16, KIND>(A, gather, W, tpe, M, N, K, E, a_rows, C, workspace, stream);
  return dispatch_mgemm_t<F16, KIND>(A, gather, W, tpe, M, N, K, E, a_rows, C, workspace, stream);
}

// Adds each split expert's partial slots in chunk order and rounds once into
// C[e]; a grid-stride loop over (split expert, 4 elements), so a plan without
// splits costs one short launch.
template <typename TR>
__global__ __launch_bounds__(256) void wgrad_finish_kernel(const float* __restrict__ partials,
                                                           const int4* __restrict__ splits,
                                                           const int* __restrict__ info, int64_t n,
                                                           uint16_t* __restrict__ C) {
  const int64_t quads = n / 4;
  const int64_t total = (int64_t)info[17] * quads;
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < total; q += (int64_t)gridDim.x * 256) {
    const int64_t si = q / quads;
    const int64_t i = (q - si * quads) * 4;
    const int4 sp = splits[si];
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < sp.z; ++c) acc += *reinterpret_cast<const floatx4*>(partials + (int64_t)(sp.y + c) * n + i);
    st8(C + (int64_t)sp.x * n + i, pack4<TR>(acc[0], acc[1], acc[2], acc[3]));
  }
}

// Workspace of the wgrad entry points: the tile plan of the register-staged
// fallback or the wgrad plan, whichever is larger; with room for partial slots
// beyond it, heavily loaded experts are split (hrm_moe_grouped_wgrad_workspace_size).
inline size_t wgrad_base_bytes(int64_t M, int E) {
  const size_t a = gemm_ws_bytes(M, E, kBMMin), b = wgrad_plan_bytes(E);
  return a > b ? a : b;
}
inline size_t wgrad_full_bytes(int64_t M, int E, int64_t Na, int64_t Nb) {
  return wgrad_base_bytes(M, E) + align256(sizeof(float) * (size_t)wgrad_slots_needed(M, E) * (size_t)(Na * Nb));
}

template <typename TR>
int launch_wgrad(const void* A, const void* B, const int64_t* tpe, int64_t M, int Na, int Nb, int E, void* C,
                 void* workspace, size_t ws_bytes, void* stream, const int32_t* b_index = nullptr,
                 int64_t b_rows = 0) {
  const bool gather = b_index != nullptr;
  const int64_t b_span = gather ? b_rows : M;
  const bool dma = M * (int64_t)Na * 2 < (int64_t(1) << 32) && b_span * (int64_t)Nb * 2 < (int64_t(1) << 32);
  const uint32_t b_bytes = (uint32_t)(b_span * (int64_t)Nb * 2);
  if (!dma) {
    if (gather) return HRM_MOE_ERR_UNSUPPORTED;  // operands beyond 32-bit buffer offsets
    GemmWs w = carve(workspace, M, E, kBMMin);
    const int max_tiles = (int)((M + kBMMin - 1) / kBMMin + E);
    HRM_LAUNCH(plan_kernel, dim3(1), dim3(1024), 0, stream, tpe, E, M, kBMMin, w.tiles, max_tiles, w.count,
               w.row_offsets, w.work_counter);
    auto kern = wgrad_kernel<TR, 128, 128>;
    static GridCache gc;
    const int grid = gc.get(kern);
    HRM_LAUNCH(kern, dim3(grid), dim3(kThreads), 0, stream, (const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C,
               w.row_offsets, E, Na, Nb, w.work_counter);
    return HRM_MOE_OK;
  }
  // the plan sits after the fallback's tile plan region, so both fit the base size
  const size_t skip = align256(wgrad_base_bytes(M, E) - wgrad_plan_bytes(E));
  WgradPlan plan = carve_wgrad(static_cast<char*>(workspace) + skip, ws_bytes - skip, E, (int64_t)Na * Nb);
  HRM_LAUNCH(wgrad_plan_kernel, dim3(1), dim3(1024), 0, stream, tpe, E, M, wgrad_chunk(M, E), plan);
  // 256 x 256 tiles with 8 waves when both widths fill them and experts have
  // enough rows to amortise a tile; HRM_MOE_WGRAD_STAGES=2|3 selects the
  // 128 x 128 four-wave kernel instead (gathered B: 2 stages).
  const int wstages = config().wgrad_stages;  // 0: automatic choice
  if (wstages == 0 && Na >= 256 && Nb >= 256 && M >= (int64_t)E * 256) {
    if (gather) {
      auto kern = wgrad_dma8_kernel<TR, 256, 256, 8, 2, true>;
      static GridCache gc;
      const int grid = gc.get(kern, 512);
      HRM_LAUNCH(kern, dim3(grid), dim3(512), 0, stream, (const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C, plan,
                 Na, Nb, b_index, b_bytes);
    } else {
      auto kern = wgrad_dma8_kernel<TR, 256, 256, 8, 2>;
      static GridCache gc;
      const int grid = gc.get(kern, 512);
      HRM_LAUNCH(kern, dim3(grid), dim3(512), 0, stream, (const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C, plan,
                 Na, Nb, nullptr, 0u);
    }
  } else {
    const int stages = gather || wstages == 2 ? 2 : 3;
    if (gather) {
      auto kern = wgrad_dma_kernel<TR, 2, true>;
      static GridCache gc;
      const int grid = gc.get(kern);
      HRM_LAUNCH(kern, dim3(grid), dim3(kThreads), 0, stream, (const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C,
                 plan, Na, Nb, b_index, b_bytes);
    } else if (stages == 2) {
      auto kern = wgrad_dma_kernel<TR, 2>;
      static GridCache gc;
      const int grid = gc.get(kern);
      HRM_LAUNCH(kern, dim3(grid), dim3(kThreads), 0, stream, (const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C,
                 plan, Na, Nb, nullptr, 0u);
    } else {
      auto kern = wgrad_dma_kernel<TR, 3>;
      static GridCache gc;
      const int grid = gc.get(kern);
      HRM_LAUNCH(kern, dim3(grid), dim3(kThreads), 0, stream, (const uint16_t*)A, (const uint16_t*)B, (uint16_t*)C,
                 plan, Na, Nb, nullptr, 0u);
    }
  }
  if (plan.max_slots >= 2) {
    const int64_t n = (int64_t)Na * Nb;
    const int64_t blocks = (n / 4 * (plan.max_slots / 2) + 255) / 256;
    HRM_LAUNCH(wgrad_finish_kernel<TR>, dim3((unsigned)(blocks < 2048 ? blocks : 2048)), dim3(256), 0, stream,
               plan.partials, plan.splits, plan.info, n, (uint16_t*)C);
  }
  return HRM_MOE_OK;
}

// Router gate weight gradient dW[E,H] = dlogits[T,E]^T . h[T,H]: a wgrad over
// S row splits with fp32 partials, then one ordered sum.  One long reduction
// (T rows) into a small output is what library GEMMs tile poorly.
// Rows per split: HRM_MOE_GATE_SPLIT_ROWS (default 1024).  At T = 16384,
// E = 64, H = 1280: 256 / 512 / 1024 / 2048 rows measured 50 / 37 / 36 / 47 us
// (torch's matmul: 101 us); short splits are dominated by each tile's pipeline
// fill and epilogue, long ones leave CUs idle.
inline int gate_wgrad_splits(int64_t T) {
  int64_t s = T / config().gate_split_rows;
  return (int)(s < 1 ? 1 : (s > 128 ? 128 : s));
}
inline size_t gate_wgrad_ws_bytes(int64_t T, int E, int64_t H) {
  const int S = gate_wgrad_splits(T);
  return align256(sizeof(int64_t) * S) + align256(wgrad_plan_bytes(S)) + align256(sizeof(float) * S * E * H);
}

template <typename TR>
int launch_gate_wgrad(const void* dlogits, const void* hidden, int64_t T, int E, int H, void* out, void* ws,
                      void* stream) {
  const int S = gate_wgrad_splits(T);
  char* p = static_cast<char*>(ws);
  int64_t* tpe = reinterpret_cast<int64_t*>(p);
  p += align256(sizeof(int64_t) * S);
  // the splits are the groups of a plan without partial slots
  const WgradPlan plan = carve_wgrad(p, wgrad_plan_bytes(S), S, (int64_t)E * H);
  p += align256(wgrad_plan_bytes(S));
  float* part = reinterpret_cast<float*>(p);
  HRM_LAUNCH(split_rows_kernel, dim3((S + 255) / 256), dim3(256), 0, stream, tpe, S, T);
  HRM_LAUNCH(wgrad_plan_kernel, dim3(1), dim3(1024), 0, stream, tpe, S, T, (int64_t)T, plan);
  auto kern = wgrad_dma_kernel<TR, 2, false, true>;
  static GridCache gc;
  const int grid = gc.get(kern);
  HRM_LAUNCH(kern, dim3(grid), dim3(kThreads), 0, stream, (const uint16_t*)dlogits, (const uint16_t*)hidden,
             (uint16_t*)part, plan, E, H, nullptr, 0u);
  const int64_t n = (int64_t)E * H;
  HRM_LAUNCH(sum_splits_kernel<TR>, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, stream, part, S, n,
             (uint16_t*)out);
  return HRM_MOE_OK;
}

}  // namespace
}  // namespace hrm

namespace hrm {
void set_last_gemm_kernel(int kind, const char* name) {
  if (kind < 0 || kind > 2 || !name) return;
  snprintf(g_last_kernel[kind], sizeof(g_last_kernel[kind]), "%s", name);
}
}  // namespace hrm

extern "C" const char* hrm_moe_last_gemm_kernel(int kind) {
  if (kind < 0 || kind > 2) return "";
  return hrm::g_last_kernel[kind];
}

extern "C" size_t hrm_moe_gate_wgrad_workspace_size(int64_t num_tokens, int32_t num_experts, int64_t hidden_size) {
  if (num_tokens < 0 || num_experts < 1 || hidden_size < 1) return 0;
  return hrm::gate_wgrad_ws_bytes(num_tokens, num_experts, hidden_size);
}

extern "C" int hrm_moe_gate_wgrad(const void* grad_logits, const void* hidden, int64_t num_tokens, int32_t num_experts,
                                  int64_t hidden_size, int dtype, void* grad_gate_weight, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (num_tokens < 0 || num_experts < 1 || hidden_size < 1) return HRM_MOE_ERR_INVALID;
  if (dtype != HRM_MOE_BF16 && dtype != HRM_MOE_F16) return HRM_MOE_ERR_DTYPE;
  if (num_experts % 8 || hidden_size % 8 || num_experts >= (1 << 20) || hidden_size >= (1 << 30) ||
      num_tokens >= (int64_t(1) << 31) || num_tokens * hidden_size * 2 >= (int64_t(1) << 32) ||
      num_tokens * (int64_t)num_experts * 2 >= (int64_t(1) << 32))
    return HRM_MOE_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < hrm::gate_wgrad_ws_bytes(num_tokens, num_experts, hidden_size))
    return HRM_MOE_ERR_WORKSPACE;
  if (!grad_logits || !hidden || !grad_gate_weight) return HRM_MOE_ERR_INVALID;
  if (num_tokens == 0) return HRM_MOE_ERR_INVALID;
  if (dtype == HRM_MOE_BF16)
    return hrm::launch_gate_wgrad<hrm::BF16>(grad_logits, hidden, num_tokens, num_experts, (int)hidden_size,
                                            grad_gate_weight, workspace, stream);
  return hrm::launch_gate_wgrad<hrm::F16>(grad_logits, hidden, num_tokens, num_experts, (int)hidden_size,
                                         grad_gate_weight, workspace, stream);
}

extern "C" size_t hrm_moe_grouped_gemm_workspace_size(int64_t num_rows, int32_t num_experts) {
  if (num_rows < 0 || num_experts < 1 || num_experts > hrm::kMaxExperts) return 0;
  return hrm::wgrad_base_bytes(num_rows, num_experts);
}

extern "C" size_t hrm_moe_grouped_wgrad_workspace_size(int64_t num_rows, int64_t Na, int64_t Nb,
                                                       int32_t num_experts) {
  if (num_rows < 0 || num_experts < 1 || num_experts > hrm::kMaxExperts || Na < 1 || Nb < 1) return 0;
  return hrm::wgrad_full_bytes(num_rows, num_experts, Na, Nb);
}

extern "C" int hrm_moe_grouped_gemm_nt(const void* A, const void* W, const int64_t* tokens_per_expert, int64_t M,
                                       int64_t N, int64_t K, int32_t num_experts, int dtype, void* C, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  int st = hrm::check_common(M, num_experts, dtype, workspace, workspace_bytes);
  if (st) return st;
  if (N < 1 || K < 1) return HRM_MOE_ERR_INVALID;
  if (N % 8 || K % 8 || N >= (1 << 30) || K >= (1 << 30)) return HRM_MOE_ERR_UNSUPPORTED;
  if (M == 0) return HRM_MOE_OK;
  if (!A || !W || !tokens_per_expert || !C) return HRM_MOE_ERR_INVALID;
  return hrm::dispatch_mgemm<hrm::KIND_NT>(dtype, A, nullptr, W, tokens_per_expert, M, (int)N, (int)K, num_experts, M,
                                           C, workspace, stream);
}

extern "C" int hrm_moe_grouped_gemm_nn(const void* A, const void* W, const int64_t* tokens_per_expert, int64_t M,
                                       int64_t N, int64_t K, int32_t num_experts, int dtype, void* C, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  int st = hrm::check_common(M, num_experts, dtype, workspace, workspace_bytes);
  if (st) return st;
  if (N < 1 || K < 1) return HRM_MOE_ERR_INVALID;
  if (N % 8 || K % 8 || N >= (1 << 30) || K >= (1 << 30)) return HRM_MOE_ERR_UNSUPPORTED;
  if (M == 0) return HRM_MOE_OK;
  if (!A || !W || !tokens_per_expert || !C) return HRM_MOE_ERR_INVALID;
  return hrm::dispatch_mgemm<hrm::KIND_NN>(dtype, A, nullptr, W, tokens_per_expert, M, (int)N, (int)K, num_experts, M,
                                           C, workspace, stream);
}

extern "C" int hrm_moe_grouped_gemm_tn(const void* A, const void* B, const int64_t* tokens_per_expert, int64_t M,
                                       int64_t Na, int64_t Nb, int32_t num_experts, int dtype, void* C,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  int st = hrm::check_common(M, num_experts, dtype, workspace, workspace_bytes);
  if (st) return st;
  if (Na < 1 || Nb < 1) return HRM_MOE_ERR_INVALID;
  if (Na % 8 || Nb % 8 || Na >= (1 << 30) || Nb >= (1 << 30)) return HRM_MOE_ERR_UNSUPPORTED;
  if (!tokens_per_expert || !C || (M > 0 && (!A || !B))) return HRM_MOE_ERR_INVALID;
  if (workspace_bytes < hrm::wgrad_base_bytes(M, num_experts)) return HRM_MOE_ERR_WORKSPACE;
  if (dtype == HRM_MOE_BF16)
    return hrm::launch_wgrad<hrm::BF16>(A, B, tokens_per_expert, M, (int)Na, (int)Nb, num_experts, C, workspace,
                                        workspace_bytes, stream);
  return hrm::launch_wgrad<hrm::F16>(A, B, tokens_per_expert, M, (int)Na, (int)Nb, num_experts, C, workspace,
                                     workspace_bytes, stream);
}

extern "C" int hrm_moe_gate_up_swiglu(const void* hidden, const int32_t* sorted_token_idx,
                                      const int64_t* tokens_per_expert, const void* gate_up_weight,
                                      int64_t num_tokens, int64_t num_rows, int64_t hidden_size, int64_t inter_size,
                                      int32_t num_experts, int dtype, void* act, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  int st = hrm::check_common(num_rows, num_experts, dtype, workspace, workspace_bytes);
  if (st) return st;
  if (num_tokens < 0 || hidden_size < 1 || inter_size < 1) return HRM_MOE_ERR_INVALID;
  if (hidden_size % 8 || inter_size % 8 || hidden_size >= (1 << 30) || inter_size >= (1 << 29))
    return HRM_MOE_ERR_UNSUPPORTED;
  if (num_rows == 0) return HRM_MOE_OK;
  if (num_tokens == 0) return HRM_MOE_ERR_INVALID;  // rows need tokens to gather from
  if (!hidden || !sorted_token_idx || !tokens_per_expert || !gate_up_weight || !act) return HRM_MOE_ERR_INVALID;
  return hrm::dispatch_mgemm<hrm::KIND_GATHER_SWIGLU>(dtype, hidden, sorted_token_idx, gate_up_weight,
                                                      tokens_per_expert, num_rows, (int)inter_size, (int)hidden_size,
                                                      num_experts, num_tokens, act, workspace, stream);
}

extern "C" int hrm_moe_gate_up_swiglu_save(const void* hidden, const int32_t* sorted_token_idx,
                                           const int64_t* tokens_per_expert, const void* gate_up_weight,
                                           int64_t num_tokens, int64_t num_rows, int64_t hidden_size,
                                           int64_t inter_size, int32_t num_experts, int dtype, void* act,
                                           void* gate_up, void* workspace, size_t workspace_bytes, void* stream) {
  int st = hrm::check_common(num_rows, num_experts, dtype, workspace, workspace_bytes);
  if (st) return st;
  if (num_tokens < 0 || hidden_size < 1 || inter_size < 1) return HRM_MOE_ERR_INVALID;
  if (hidden_size % 64 || inter_size % 8 || hidden_size >= (1 << 30) || inter_size >= (1 << 29))
    return HRM_MOE_ERR_UNSUPPORTED;
  if (num_rows == 0) return HRM_MOE_OK;
  if (num_tokens == 0) return HRM_MOE_ERR_INVALID;
  if (!hidden || !sorted_token_idx || !tokens_per_expert || !gate_up_weight || !act || !gate_up)
    return HRM_MOE_ERR_INVALID;
  return hrm::dispatch_mgemm_epi<hrm::KIND_GATHER_SWIGLU, hrm::EPI_SAVE_GU>(
      dtype, hidden, sorted_token_idx, gate_up_weight, tokens_per_expert, num_rows, (int)inter_size, (int)hidden_size,
      num_experts, num_tokens, act, gate_up, stream);
}

extern "C" int hrm_moe_down_dgrad_swiglu(const void* grad_expert_out, const void* down_weight,
                                         const int64_t* tokens_per_expert, const void* gate_up, int64_t num_rows,
                                         int64_t inter_size, int64_t hidden_size, int32_t num_experts, int dtype,
                                         void* grad_gate_up, void* workspace, size_t workspace_bytes, void* stream) {
  int st = hrm::check_common(num_rows, num_experts, dtype, workspace, workspace_bytes);
  if (st) return st;
  if (hidden_size < 1 || inter_size < 1) return HRM_MOE_ERR_INVALID;
  if (hidden_size % 64 || inter_size % 8 || hidden_size >= (1 << 30) || inter_size >= (1 << 29))
    return HRM_MOE_ERR_UNSUPPORTED;
  if (num_rows == 0) return HRM_MOE_OK;
  if (!grad_expert_out || !down_weight || !tokens_per_expert || !gate_up || !grad_gate_up) return HRM_MOE_ERR_INVALID;
  return hrm::dispatch_mgemm_epi<hrm::KIND_NN, hrm::EPI_SWIGLU_BWD>(
      dtype, grad_expert_out, nullptr, down_weight, tokens_per_expert, num_rows, (int)inter_size, (int)hidden_size,
      num_experts, num_rows, grad_gate_up, const_cast<void*>(gate_up), stream);
}

extern "C" int hrm_moe_grouped_gemm_tn_gather(const void* A, const void* B, const int32_t* b_row_index, int64_t b_rows,
                                              const int64_t* tokens_per_expert, int64_t M, int64_t Na, int64_t Nb,
                                              int32_t num_experts, int dtype, void* C, void* workspace,
                                              size_t workspace_bytes, void* stream) {
  int st = hrm::check_common(M, num_experts, dtype, workspace, workspace_bytes);
  if (st) return st;
  if (Na < 1 || Nb < 1 || b_rows < 0) return HRM_MOE_ERR_INVALID;
  if (Na % 8 || Nb % 8 || Na >= (1 << 30) || Nb >= (1 << 30)) return HRM_MOE_ERR_UNSUPPORTED;
  if (!tokens_per_expert || !C || (M > 0 && (!A || !B || !b_row_index || b_rows == 0))) return HRM_MOE_ERR_INVALID;
  if (workspace_bytes < hrm::wgrad_base_bytes(M, num_experts)) return HRM_MOE_ERR_WORKSPACE;
  if (dtype == HRM_MOE_BF16)
    return hrm::launch_wgrad<hrm::BF16>(A, B, tokens_per_expert, M, (int)Na, (int)Nb, num_experts, C, workspace,
                                        workspace_bytes, stream, b_row_index, b_rows);
  return hrm::launch_wgrad<hrm::F16>(A, B, tokens_per_expert, M, (int)Na, (int)Nb, num_experts, C, workspace,
                                     workspace_bytes, stream, b_row_index, b_rows);
}
