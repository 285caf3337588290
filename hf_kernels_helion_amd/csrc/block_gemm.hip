// Block-scaled w8a8 GEMM for gfx950:  C[M,N] = A[M,K] . B[N,K]^T with
//   C[m,n] = sum_kb dot_kb(m,n) * As[m,kb] * Bs[n/128,kb],
// the arithmetic of the Helion kernel in
// finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/fp8.py:28-38.
//
// MFMA path (block_n = block_k = 128):
//   * One K-block of 128 is exactly one v_mfma_f32_16x16x128_f8f6f4 per 16x16
//     output sub-tile, issued with a zero accumulator; its fp32 result is
//     folded into the running fp32 accumulator with one FMA by the product of
//     the row's activation scale and the tile's weight scale. No second set of
//     accumulators is needed.
//   * The weight tile is the MFMA's A operand and the activation tile its B
//     operand, so the 16x16 result holds one activation row per lane and four
//     consecutive output columns: the activation scale is one register per
//     lane and sub-tile row, the weight scale one scalar per wave.
//   * Both operand tiles stream global -> LDS with global_load_lds_dwordx4
//     (no VGPR staging) into two LDS stages. Each 128-byte tile row is kept as
//     eight 16-byte chunks, chunk c of row r stored at slot c ^ (r & 7), which
//     makes the per-lane fragment reads (16 rows x same chunk) hit distinct
//     banks.
//   * Ragged M/N: rows past the end are clamped to the last row when loading
//     and masked when storing. K must be a multiple of 128.
//   * Split-K writes fp32 partials to the caller's workspace; a second kernel
//     sums them in split order and applies the output conversion.
//
// Generic path (any block_n/block_k, ragged K, unaligned operands): a SIMT
// kernel with the same blockwise summation, used only where the MFMA path's
// preconditions do not hold.
#include "common.h"
#include "quant.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>

namespace fp8b {

struct GemmArgs {
  const uint8_t* A;
  const uint8_t* B;
  const float* As;
  const float* Bs;
  void* C;
  float* ws;
  int64_t lda, ldb, as_sm, as_sk, bs_sn, bs_sk, ldc;
  int M, N, K;
  int KB;            // number of 128-wide K-blocks
  int kb_per_split;  // K-blocks per grid.z slice
  int tiles_m, tiles_n;
  int out_dtype;     // fp8b_dtype; ignored when writing split-K partials
  int vec_store;     // 1 if 4 consecutive outputs can be stored as one vector
  // Pipelined kernels: 1 = scale windows by 4-byte DMA lanes (any scale
  // strides, any K-block count and split size); 0 = by 16-byte lanes (As and
  // Bs contiguous in K with 16-byte aligned rows, K-block count and split
  // size multiples of 4).
  int win4;
  // gemm_pipe128_kernel and gemm_tiny_kernel only: when rem_base >= 0,
  // workgroup w computes quarter w % 4 of tile rem_base + w / 4 of a
  // rem_tiles_m x rem_tiles_n grid of tiles twice as large (the tiles a
  // launch of rem_base workgroups on that grid left), instead of tile w:
  // 128x128 quarters of gemm_pipe256_kernel's tiles, 64x64 quarters of
  // gemm_pipe128_kernel's. gemm_pipe256x128_kernel: column half w % 2 of
  // tile rem_base + w / 2 of gemm_pipe256_kernel's grid.
  int rem_base, rem_tiles_m, rem_tiles_n;
  // gemm_pipe256_kernel<false, true> only (the gate/up GEMM that writes
  // silu(gate) * up quantised): C is the e4m3fn output [M, N/2] (row stride
  // ldc) and the group scale of (m, g) goes to Sq[m * sq_sm + g * sq_sg].
  float* Sq;
  int64_t sq_sm, sq_sg;
};

// Workgroup -> output tile of a tiles_m x tiles_n grid: XCD-contiguous runs
// (workgroup b runs on XCD b % 8, so b goes to tile (b % 8) * tiles/8 + b/8
// when 8 divides the tile count), walked in groups of 8 tile rows.
__device__ __forceinline__ void tile_of_bid(int bid, int tiles_m, int tiles_n, int& tm,
                                            int& tn) {
  const int tiles = tiles_m * tiles_n;
  if (tiles % 8 == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
  constexpr int GROUP_M = 8;
  const int group_size = GROUP_M * tiles_n;
  const int first_m = (bid / group_size) * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  tm = first_m + (bid % group_size) % gm;
  tn = (bid % group_size) / gm;
}

typedef __attribute__((address_space(3))) void lds_void;

// One 16x16x128 fp8 (e4m3) MFMA with a zero accumulator: 16 rows of a (the
// MFMA A operand, lane = row & 15, K bytes 32*(lane>>4)..+31) times 16 rows of
// b, summed over 128 K. With both scale operands 0 the compiler selects the
// unscaled v_mfma_f32_16x16x128_f8f6f4 (one 8-byte instruction) instead of
// the E8M0-scaled form with scale 127 = 1.0 (a v_mfma_ld_scale_b32 prefix
// plus the MFMA): the same product bit for bit, one instruction less per
// MFMA (measured 2.4% faster on the large GEMM at steady clock).
__device__ __forceinline__ v4f mfma16x16x128(const v8i& a, const v8i& b) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0,
                                                          0, 0, 0);
}

__device__ __forceinline__ void lds_dma16(const void* gsrc, uint8_t* ldst) {
  __builtin_amdgcn_global_load_lds(gsrc, (lds_void*)ldst, 16, 0, 0);
}

// Store four consecutive outputs (columns n..n+3 of row m).
__device__ __forceinline__ void store4(const GemmArgs& a, int m, int n, const v4f& v,
                                       bool partial_ws, int split) {
  if (m >= a.M || n >= a.N) return;
  if (partial_ws) {
    float* p = a.ws + ((int64_t)split * a.M + m) * a.N + n;
    if (n + 3 < a.N && a.vec_store) {
      *reinterpret_cast<v4f*>(p) = v;
    } else {
      for (int r = 0; r < 4 && n + r < a.N; ++r) p[r] = v[r];
    }
    return;
  }
  if (a.out_dtype == FP8B_F32) {
    float* p = reinterpret_cast<float*>(a.C) + (int64_t)m * a.ldc + n;
    if (n + 3 < a.N && a.vec_store) {
      *reinterpret_cast<v4f*>(p) = v;
    } else {
      for (int r = 0; r < 4 && n + r < a.N; ++r) p[r] = v[r];
    }
  } else {
    uint16_t* p = reinterpret_cast<uint16_t*>(a.C) + (int64_t)m * a.ldc + n;
    const bool bf = a.out_dtype == FP8B_BF16;
    const uint32_t lo = bf ? pack_bf16x2(v[0], v[1]) : pack_f16x2(v[0], v[1]);
    const uint32_t hi = bf ? pack_bf16x2(v[2], v[3]) : pack_f16x2(v[2], v[3]);
    if (n + 3 < a.N && a.vec_store) {
      v2i w;
      w[0] = (int)lo;
      w[1] = (int)hi;
      *reinterpret_cast<v2i*>(p) = w;
    } else {
      const uint16_t h[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi,
                             (uint16_t)(hi >> 16)};
      for (int r = 0; r < 4 && n + r < a.N; ++r) p[r] = h[r];
    }
  }
}

// fp32 tile of a workgroup (AR rows from m0 x BN columns from n0, 512
// threads) staged through LDS on its way to dst + row * ld + column (the
// split-K workspace slice, or fp32 C): each lane first puts its 16-byte
// pieces into a [rows][BN + 4] tile (rows padded against bank conflicts),
// then every store instruction writes whole row segments of BN * 4 bytes
// (full cache lines) instead of the 64-byte pieces of four lanes per row.
// Called by every thread once the operand stages are dead (each wave has
// waited for all its DMA). Rounds of RR rows when the whole tile does not
// fit the LDS: put(tile, pitch, r0) writes the calling lane's accumulators
// of tile rows r0..r0+RR-1 at row - r0.
template <int AR, int BN, int RR, typename Put>
__device__ __forceinline__ void f32_tile_lds(const GemmArgs& a, uint8_t* smem, int m0, int n0,
                                             float* dst, int64_t ld, Put put) {
  constexpr int P = BN + 4, TPR = BN / 4, RPP = 512 / TPR;
  static_assert(RR % RPP == 0 && AR % RR == 0, "whole passes of 512 threads per round");
  float* tile = reinterpret_cast<float*>(smem);
  const int t = threadIdx.x, c = 4 * (t % TPR);
#pragma unroll
  for (int r0 = 0; r0 < AR; r0 += RR) {
    __syncthreads();
    put(tile, P, r0);
    __syncthreads();
#pragma unroll
    for (int p = 0; p < RR / RPP; ++p) {
      const int m = p * RPP + t / TPR;
      if (m0 + r0 + m < a.M)
        *reinterpret_cast<v4f*>(dst + (int64_t)(m0 + r0 + m) * ld + n0 + c) =
            *reinterpret_cast<const v4f*>(tile + m * P + c);
    }
  }
}

// Where a workgroup's fp32 tile (BN columns from n0) goes through
// f32_tile_lds: the split-K workspace slice of its split, or fp32 C when
// the launch is unsplit; nullptr when it keeps per-lane stores (a partial
// column tile, no vector stores, or 16-bit C).
__device__ __forceinline__ float* f32_tile_dest(const GemmArgs& a, int n0, int BN, int split,
                                                int64_t& ld) {
  if (!a.vec_store || n0 + BN > a.N) return nullptr;
  if (gridDim.z > 1) {
    if (a.N & 3) return nullptr;
    ld = a.N;
    return a.ws + (int64_t)split * a.M * a.N;
  }
  if (a.out_dtype != FP8B_F32) return nullptr;
  ld = a.ldc;
  return reinterpret_cast<float*>(a.C);
}

__device__ __forceinline__ void lds_dma4(const void* gsrc, uint8_t* ldst) {
  __builtin_amdgcn_global_load_lds(gsrc, (lds_void*)ldst, 4, 0, 0);
}

__device__ __forceinline__ v8i lds_frag(const uint8_t* row, int c0, int r7) {
  const v4i lo = *reinterpret_cast<const v4i*>(row + ((c0 ^ r7) << 4));
  const v4i hi = *reinterpret_cast<const v4i*>(row + (((c0 + 1) ^ r7) << 4));
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// 16-bit epilogue of one wave's WM x WN tile (rows mw.., columns nw..): the
// wave writes its packed sub-tiles to its own LDS area (pitch WN*2+16 bytes,
// conflict-free), then stores whole 16-byte runs of each output row. Every
// wave of the workgroup must call it (it contains a barrier).
template <int WM, int WN>
__device__ __forceinline__ void stage16(uint8_t* wbase, const v4f (&acc)[WM / 16][WN / 16],
                                        int lane, bool bf) {
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int EPI_PITCH = WN * 2 + 16;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const v4f v = acc[i][j];
      v2i w;
      w[0] = (int)(bf ? pack_bf16x2(v[0], v[1]) : pack_f16x2(v[0], v[1]));
      w[1] = (int)(bf ? pack_bf16x2(v[2], v[3]) : pack_f16x2(v[2], v[3]));
      *reinterpret_cast<v2i*>(wbase + (i * 16 + (lane & 15)) * EPI_PITCH +
                              (j * 16 + 4 * (lane >> 4)) * 2) = w;
    }
  }
}

template <int WM, int WN>
__device__ __forceinline__ void epilogue16(const GemmArgs& a, uint8_t* wbase,
                                           const v4f (&acc)[WM / 16][WN / 16], int mw, int nw,
                                           int lane) {
  constexpr int EPI_PITCH = WN * 2 + 16;
  stage16<WM, WN>(wbase, acc, lane, a.out_dtype == FP8B_BF16);
  __syncthreads();
  constexpr int CPR = WN / 8;   // 16-byte chunks per wave row
  constexpr int RPP = 64 / CPR; // rows per pass
  const int c = lane % CPR;
  const int n = nw + c * 8;
  uint16_t* C = reinterpret_cast<uint16_t*>(a.C);
#pragma unroll
  for (int p = 0; p < WM / RPP; ++p) {
    const int r = p * RPP + lane / CPR;
    const int m = mw + r;
    const v4i v = *reinterpret_cast<const v4i*>(wbase + r * EPI_PITCH + c * 16);
    if (m >= a.M || n >= a.N) continue;
    uint16_t* dst = C + (int64_t)m * a.ldc + n;
    if (n + 8 <= a.N && a.vec_store) {
      // streaming store: 0.5-1.4% on 4096x4096x8192 and 3001x28672x4096
      // (steady and graph replay, eight alternating runs), no loss seen
      __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(dst));
    } else {
      for (int e = 0; e < 8 && n + e < a.N; ++e)
        dst[e] = (uint16_t)(((uint32_t)v[e >> 1]) >> ((e & 1) * 16));
    }
  }
}

__device__ __forceinline__ v8i lds_frag2(const uint8_t* p, int s_lo, int s_hi) {
  const v4i lo = *reinterpret_cast<const v4i*>(p + s_lo);
  const v4i hi = *reinterpret_cast<const v4i*>(p + s_hi);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// BM x BN output tile per workgroup, WM x WN per wavefront.
//
// LDS stage layout (two stages):
//   [0, (BM+BN)*128)        A rows then B rows, 128 bytes each, chunk-swizzled
//   [SA_OFF, +max(BM,64)*4) As[m0+r, kb] for r < BM (gathered by lane DMA)
//   [SB_OFF, +256)          Bs[n0/128 + j, kb] for the tile's 128-column blocks
// Every operand and scale of a K-block arrives by global_load_lds, so the
// only wait on vector memory in the main loop is the one per K-block that
// also guards the double buffer.
template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
gemm_bs128_kernel(GemmArgs a) {
  constexpr int NWM = BM / WM, NWN = BN / WN, NW = NWM * NWN;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int ROWS = BM + BN;
  constexpr int SA_OFF = ROWS * 128;
  constexpr int SA_LOADS = (BM + 63) / 64;
  constexpr int SB_OFF = SA_OFF + SA_LOADS * 256;
  constexpr int STAGE = SB_OFF + 256;
  constexpr int LOADS = ROWS / 8;  // 1 KiB wave-loads of operand rows per stage
  constexpr int NB_TILE = BN / 128;
  constexpr int EPI_PITCH = WN * 2 + 16;  // bf16 epilogue row pitch (conflict-free)
  constexpr int EPI = NW * WM * EPI_PITCH;
  constexpr int SMEM = (2 * STAGE > EPI) ? 2 * STAGE : EPI;
  static_assert(LOADS % NW == 0, "stage loads must split evenly over waves");
  static_assert(BN % 128 == 0 && WN <= 128 && 128 % WN == 0,
                "a wave's columns must sit in one 128-column scale block");
  static_assert(FN % 2 == 0, "weight fragments are consumed in two halves");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int wm = wid / NWN, wn = wid % NWN;

  // Workgroup -> tile. Consecutive workgroup ids go round-robin over the 8
  // XCDs; regroup so each XCD owns a contiguous run of tiles, then walk the
  // run in column-major groups of 8 tile rows so neighbouring workgroups
  // share A row-panels and B column-panels in their XCD's L2.
  const int tiles = a.tiles_m * a.tiles_n;
  int bid = blockIdx.x;
  if (tiles % 8 == 0) bid = (bid & 7) * (tiles >> 3) + (bid >> 3);
  constexpr int GROUP_M = 8;
  const int group_size = GROUP_M * a.tiles_n;
  const int first_m = (bid / group_size) * GROUP_M;
  const int gm = min(a.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (bid % group_size) % gm;
  const int tn = (bid % group_size) / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  const int split = blockIdx.z;
  const int kb_begin = split * a.kb_per_split;
  const int kb_end = min(kb_begin + a.kb_per_split, a.KB);

  // Per-lane global source of each operand wave-load: row r of the stage,
  // logical chunk (lane&7) ^ (r&7) so that it lands in LDS slot lane&7.
  const uint8_t* src[LOADS / NW];
#pragma unroll
  for (int i = 0; i < LOADS / NW; ++i) {
    const int L = wid + i * NW;
    const int r = L * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ (r & 7);
    if (L * 8 < BM) {
      const int gmr = min(m0 + r, a.M - 1);
      src[i] = a.A + (int64_t)gmr * a.lda + chunk * 16;
    } else {
      const int gnr = min(n0 + r - BM, a.N - 1);
      src[i] = a.B + (int64_t)gnr * a.ldb + chunk * 16;
    }
  }
  // Scale gathers: waves 0..SA_LOADS-1 fetch 64 activation-scale rows each,
  // the last wave fetches the tile's weight-scale blocks (rows and blocks past
  // the matrix edge are clamped; their values only reach masked outputs).
  const float* sa_src =
      a.As + (int64_t)min(m0 + min(wid * 64 + lane, BM - 1), a.M - 1) * a.as_sm;
  const float* sb_src =
      a.Bs + (int64_t)min((n0 >> 7) + min(lane, NB_TILE - 1), (a.N - 1) >> 7) * a.bs_sn;

  auto issue = [&](int kb, int stage) {
    uint8_t* base = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < LOADS / NW; ++i) {
      const int L = wid + i * NW;
      lds_dma16(src[i] + (int64_t)kb * 128, base + L * 1024);
    }
    if (wid < SA_LOADS) lds_dma4(sa_src + (int64_t)kb * a.as_sk, base + SA_OFF + wid * 256);
    if (wid == NW - 1) lds_dma4(sb_src + (int64_t)kb * a.bs_sk, base + SB_OFF);
  };

  // LDS byte offsets of this lane's fragment rows; the two 16-byte chunks of
  // a fragment are logical chunks 2*(lane>>4) and 2*(lane>>4)+1.
  const int c0 = 2 * (lane >> 4);
  const int r7 = lane & 7;  // fragment rows start at multiples of 16
  const int a_row = (wm * WM + (lane & 15)) * 128;
  const int b_row = (BM + wn * WN + (lane & 15)) * 128;
  const int sa_row = SA_OFF + (wm * WM + (lane & 15)) * 4;
  const int sb_slot = SB_OFF + ((wn * WN) >> 7) * 4;

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  if (kb_begin < kb_end) issue(kb_begin, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  for (int kb = kb_begin; kb < kb_end; ++kb) {
    const int stage = (kb - kb_begin) & 1;
    if (kb + 1 < kb_end) issue(kb + 1, stage ^ 1);

    const uint8_t* sbase = smem + stage * STAGE;
    const float sbv = *reinterpret_cast<const float*>(sbase + sb_slot);
    float sc[FM];
    v8i xf[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      sc[i] = *reinterpret_cast<const float*>(sbase + sa_row + i * 64) * sbv;
      xf[i] = lds_frag(sbase + a_row + i * 16 * 128, c0, r7);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v8i wf[FN / 2];
#pragma unroll
      for (int j = 0; j < FN / 2; ++j)
        wf[j] = lds_frag(sbase + b_row + (h * FN / 2 + j) * 16 * 128, c0, r7);
      // Software pipeline: the FMAs of one sub-tile run under the next MFMA.
      v4f prev = mfma16x16x128(wf[0], xf[0]);
#pragma unroll
      for (int t = 1; t <= FM * (FN / 2); ++t) {
        v4f cur = prev;
        if (t < FM * (FN / 2)) {
          const int i = t / (FN / 2), j = t % (FN / 2);
          cur = mfma16x16x128(wf[j], xf[i]);
        }
        const int pi = (t - 1) / (FN / 2), pj = h * (FN / 2) + (t - 1) % (FN / 2);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[pi][pj][r] = fmaf(prev[r], sc[pi], acc[pi][pj][r]);
        prev = cur;
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  // Epilogue: lane holds row (lane & 15) and columns 4*(lane>>4)+0..3 of each
  // 16x16 sub-tile.
  const bool to_ws = gridDim.z > 1;
  if (to_ws || a.out_dtype == FP8B_F32) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + wm * WM + i * 16 + (lane & 15);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * WN + j * 16 + 4 * (lane >> 4);
        store4(a, m, n, acc[i][j], to_ws, split);
      }
    }
    return;
  }
  // 16-bit outputs: staged through LDS (the operand stages are dead after
  // the loop's last barrier).
  epilogue16<WM, WN>(a, smem + wid * WM * EPI_PITCH, acc, m0 + wm * WM, n0 + wn * WN, lane);
}

// Epilogue of a wave's WM x WN accumulator tile at rows mw.., columns nw..
// (lane: row lane & 15 and columns 4*(lane>>4)..+3 of each 16x16 sub-tile):
// fp32 partials to the split-K workspace or fp32 C directly, 16-bit outputs
// staged through LDS by epilogue16. Every wave of the workgroup must call it
// (the 16-bit path has a barrier); the operand stages in smem must be dead.
template <int WM, int WN>
__device__ __forceinline__ void tile_epilogue(const GemmArgs& a, uint8_t* smem,
                                              const v4f (&acc)[WM / 16][WN / 16], int mw,
                                              int nw, int wid, int lane, int split) {
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int EPI_PITCH = WN * 2 + 16;
  const bool to_ws = gridDim.z > 1;
  if (to_ws || a.out_dtype == FP8B_F32) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = mw + i * 16 + (lane & 15);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = nw + j * 16 + 4 * (lane >> 4);
        store4(a, m, n, acc[i][j], to_ws, split);
      }
    }
    return;
  }
  epilogue16<WM, WN>(a, smem + wid * WM * EPI_PITCH, acc, mw, nw, lane);
}

// SWIGLU epilogue of a BM x 256 tile whose columns 0..127 are gate columns
// and 128..255 the matching up columns (8 waves of WM x 64, wave w at rows
// WM*(w/4), columns 64*(w%4)): the waves stage their bf16 tiles in LDS as
// epilogue16 does, then thread t takes tile row 32p + t/16 in pass p and
// output columns 8(t%16)..+7 of the row's 128-wide group, forms
// silu(gate) * up in bf16 (silu_mul_bf16x8) and quantises the group
// (quant_row16_8): e4m3fn codes to C [M, N/2], the scale to Sq. Every thread
// of the workgroup must call it.
template <int BM, int WM, int WN>
__device__ __forceinline__ void swiglu_epilogue(const GemmArgs& a, uint8_t* smem,
                                                const v4f (&acc)[WM / 16][WN / 16], int m0,
                                                int tn, int wid, int lane) {
  constexpr int NWN = 4, EPI_PITCH = WN * 2 + 16;
  static_assert(WN == 64 && BM % 32 == 0, "a 256-column tile of 64-column waves");
  const int tid = threadIdx.x;
  stage16<WM, WN>(smem + wid * WM * EPI_PITCH, acc, lane, true);
  __syncthreads();
  // Gate values of row r, columns 8(t%16).. sit in wave (r/WM, (t%16)/8)'s
  // staging area, the up values two waves further.
  const int sub = tid & 15;
  const int cb = (sub & 7) * 16;
  const int half = sub >> 3;
  uint8_t* qout = reinterpret_cast<uint8_t*>(a.C) + tn * 128 + sub * 8;
  // All LDS reads first (the accumulators are dead, so registers are
  // plentiful), then the rows' arithmetic back to back.
  constexpr int NP = BM / 32;
  v4i gv[NP], uv[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int r = p * 32 + (tid >> 4);
    const uint8_t* row = smem + (r % WM) * EPI_PITCH + cb;
    const int wg = (r / WM) * NWN + half;
    gv[p] = *reinterpret_cast<const v4i*>(row + wg * WM * EPI_PITCH);
    uv[p] = *reinterpret_cast<const v4i*>(row + (wg + 2) * WM * EPI_PITCH);
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int r = p * 32 + (tid >> 4);
    float v[8];
    const v4i h = silu_mul_bf16x8(gv[p], uv[p], v);
    uint32_t w0, w1;
    float scale;
    quant_row16_8(v, max_mag_bf16x8(h), w0, w1, scale);
    const int m = m0 + r;
    if (m < a.M) {
      v2i packed;
      packed[0] = (int)w0;
      packed[1] = (int)w1;
      *reinterpret_cast<v2i*>(qout + (int64_t)m * a.ldc) = packed;
      if (sub == 0) a.Sq[(int64_t)m * a.sq_sm + (int64_t)tn * a.sq_sg] = scale;
    }
  }
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Before a wave refills an LDS slot by DMA without a barrier: its own LDS
// reads of that slot must have completed. The compiler waits for a ds_read
// only where the value is used, which can be after the refill is issued
// (then the DMA's write can overtake the pending read).
__device__ __forceinline__ void lds_reads_done() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------
// Pipelined 256x256 kernel (the large-GEMM path).
//
// Same arithmetic as gemm_bs128_kernel (one zero-accumulator MFMA per 16x16
// sub-tile and K-block, folded by one FMA with the product of the two
// scales), scheduled so that LDS reads, DMA and the workgroup barrier overlap
// the MFMA stream:
//   * 8 waves, each owning a 128x64 (activation rows x weight rows) piece:
//     eight 16-row activation fragments and four weight fragments per
//     K-block. The 32 MFMAs of a K-block run in a fixed order (rows 0-1 and
//     6-7 column-major in pairs, rows 2-5 row-major), so every fragment is
//     read from LDS several MFMAs before its first use and its registers are
//     refilled right after its last use.
//   * One barrier per K-block, placed before MFMA 24: by then every wave has
//     read all of the current stage and its DMA of the next stage has landed.
//     After it the wave reads the next K-block's first fragments and issues
//     the DMA of K-block kb+2 into the stage just released, one instruction
//     per MFMA, while its last 8 MFMAs run.
//   * Each MFMA result is folded two MFMAs later, so the FMAs never wait on
//     the MFMA that produced them.
//   * Activation and weight scales arrive in windows of 8 K-blocks (32 bytes
//     per activation row: two 16-byte DMA lanes) instead of one 4-byte
//     gather per row and K-block; a window is double-buffered and issued with
//     the operand DMA two K-blocks ahead.
//   * The DMA is issued from inline asm (global_load_lds_dwordx4 with an
//     SGPR base and a 32-bit VGPR offset). The compiler does not see these
//     loads, so it neither tracks them (the kernel waits on vmcnt itself,
//     before each barrier) nor treats them as LGKM events of unknown order,
//     which would force lgkmcnt(0) before every fragment read.
// Precondition (checked by the host): 255 * max(lda, ldb) + K below 2^32 for
// the 32-bit DMA offsets. Scale windows take 16-byte DMA lanes when As and
// Bs are contiguous along K with 16-byte aligned rows and KB and the split
// size are multiples of 4, else (a.win4) 4-byte lanes with every K-block
// clamped into range (win4_rows, win4_blocks): any strides and counts.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void dma16_soff(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma16_ptr(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4_ptr(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(g), "{m0}"(lds) : "memory");
}
// Scale window of 8 K-blocks by 4-byte DMA lanes, for any scale strides and
// K-block counts: rows r0..r0+31 (each clamped to rmax) into 32-byte row
// slots at lds (slot s: K-block kb0 + s, clamped to kb_end - 1), four
// instructions of 8 rows; lane i of instruction j writes row 8j + i/8, slot
// i%8 (LDS DMA lane i lands at M0 + 4i).
__device__ __forceinline__ void win4_rows(const float* S, int64_t sm, int64_t sk, int r0, int rmax,
                                          int kb0, int kb_end, uint32_t lds, int lane) {
  const int64_t kofs = (int64_t)min(kb0 + (lane & 7), kb_end - 1) * sk;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int r = min(r0 + 8 * j + (lane >> 3), rmax);
    asm volatile("" : "+v"(r));
    dma4_ptr(S + (int64_t)r * sm + kofs, lds + j * 256);
  }
}
// The weight-block scales of a window: nb 128-column blocks from row b0
// (clamped to bmax), 8 slots each, lanes 0..8nb-1.
__device__ __forceinline__ void win4_blocks(const float* S, int64_t sm, int64_t sk, int b0, int bmax,
                                            int nb, int kb0, int kb_end, uint32_t lds, int lane) {
  if (lane < 8 * nb) {
    const int b = min(b0 + (lane >> 3), bmax);
    const int kb = min(kb0 + (lane & 7), kb_end - 1);
    dma4_ptr(S + (int64_t)b * sm + (int64_t)kb * sk, lds);
  }
}

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <int KIND> struct PipeKind { static constexpr int value = KIND; };

// PR (per-row weight scales, block_n = 1): the window also holds the 256
// weight rows' scales slot-major (slot s: K-block kb0 + s, consecutive floats;
// 4-byte DMA lanes, one per row); each fold multiplies the row scale by the
// lane's four column scales, read once per K-block per weight fragment as one
// 16-byte load, each into the register its previous value just left.
//
// SWIGLU (gate/up GEMM of a gated MLP, weights interleaved in 128-row blocks
// so that columns 0..127 of every 256-column tile are gate columns and
// 128..255 the matching up columns): the epilogue stages the bf16 tile in LDS
// as epilogue16 does, then each 16-lane DPP row takes one tile row, forms
// silu(gate) * up in bf16 (silu_mul_bits) and quantises the 128 results as
// one group: e4m3fn codes to C [M, N/2], the scale to Sq. Bit-identical to
// storing the bf16 tile, then silu_and_mul_quant.
template <bool PR, bool SWIGLU = false>
__global__ void __launch_bounds__(512) gemm_pipe256_kernel(GemmArgs a) {
  constexpr int BM = 256, BN = 256, WM = 128, WN = 64, NWN = BN / WN, NW = 8;
  constexpr int FM = WM / 16, FN = WN / 16;       // 8 activation, 4 weight fragments
  constexpr int STAGE = (BM + BN) * 128;          // operand rows of one K-block
  constexpr int WIN_SA = BM * 32;                 // 8 K-blocks of As per row
  constexpr int WIN = WIN_SA + (PR ? 8 * BN * 4 : 256);  // + Bs of the tile
  constexpr int SW_OFF = 2 * STAGE;
  constexpr int EPI_PITCH = WN * 2 + 16;
  constexpr int EPI = NW * WM * EPI_PITCH;
  constexpr int SMEM = (2 * STAGE + 2 * WIN > EPI) ? 2 * STAGE + 2 * WIN : EPI;
  static_assert(FM == 8 && FN == 4, "the MFMA order below is written for 8x4 fragments");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid / NWN, wn = wid % NWN;

  int tm, tn;
  tile_of_bid((int)blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int split = blockIdx.z;
  const int kb_begin = split * a.kb_per_split;
  const int kb_end = min(kb_begin + a.kb_per_split, a.KB);
  const int nkb = kb_end - kb_begin;

  const uint32_t lds0 = lds_u32(smem);
  // Operand DMA: wave-load L = wid + 8i brings stage rows 8L..8L+7 (A rows
  // for L < 32, B rows after), eight lanes per 128-byte row; lane l fetches
  // chunk (l&7)^(l>>3) of row 8L + (l>>3), i.e. chunk c of row r lands in
  // slot c^(r&7). Rows past the matrix edge are clamped to the last row.
  const int r8 = lane >> 3;
  const uint8_t* a_base = a.A + (int64_t)m0 * a.lda;
  const uint8_t* b_base = a.B + (int64_t)n0 * a.ldb;
  const int a_lim = a.M - 1 - m0, b_lim = a.N - 1 - n0;
  // Block L of a stage (1 KiB, 8 segments of 128 bytes) holds the rows
  // 64*(L/8) + 8*s + (L%8), s = 0..7, with chunk c of each row in slot
  // c ^ (L%8): a 16-row fragment then spans eight blocks (two segments
  // each), the layout that ds_read_b128 serves fastest (measured ~1.5x the
  // row-contiguous tile).
  auto issue_op = [&](int kb, int stage, int i) {
    const int L = wid + i * NW;
    const uint32_t lds = lds0 + stage * STAGE + L * 1024;
    const int Lr = L & 31;
    const int row = (Lr >> 3) * 64 + r8 * 8 + (Lr & 7);
    const int c16 = ((lane & 7) ^ (Lr & 7)) * 16;
    if (i < 4) {
      const uint32_t voff = (uint32_t)min(row, a_lim) * (uint32_t)a.lda + c16;
      dma16_soff(voff, a_base + (int64_t)kb * 128, lds);
    } else {
      const uint32_t voff = (uint32_t)min(row, b_lim) * (uint32_t)a.ldb + c16;
      dma16_soff(voff, b_base + (int64_t)kb * 128, lds);
    }
  };
  // Scale window of 8 K-blocks from kb0: wave w brings As rows 32w..32w+31
  // (16-byte lanes: two per row, 4 K-blocks each); wave 7 also brings the Bs
  // rows of the tile's two 128-column blocks. With 16-byte lanes a
  // half-window past kb_end re-reads the first half (KB is then a multiple
  // of 4), so no lane reads past the row.
  const float* saw_src =
      a.As + (int64_t)min(m0 + wid * 32 + (lane >> 1), a.M - 1) * a.as_sm + 4 * (lane & 1);
  const float* sbw_src =
      a.Bs + (int64_t)min((n0 >> 7) + min(lane >> 1, 1), (a.N - 1) >> 7) * a.bs_sn + 4 * (lane & 1);
  auto issue_win = [&](int kb0, int wbuf) {
    const int kk = (kb0 + 4 * (lane & 1) < kb_end) ? kb0 : kb0 - 4 * (lane & 1);
    const uint32_t lb = lds0 + SW_OFF + wbuf * WIN;
    if (a.win4)
      win4_rows(a.As, a.as_sm, a.as_sk, m0 + wid * 32, a.M - 1, kb0, kb_end, lb + wid * 1024, lane);
    else
      dma16_ptr(saw_src + kk, lb + wid * 1024);
    if constexpr (PR) {
      // wave w: slot w, rows 64h + lane for h = 0..3
      // (the row is pinned so that the addresses are formed here, once per
      // window, instead of being held in registers across the loop)
      const int kbs = min(kb0 + wid, kb_end - 1);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        int row = n0 + h * 64 + lane;
        asm volatile("" : "+v"(row));
        dma4_ptr(a.Bs + (int64_t)min(row, a.N - 1) * a.bs_sn + (int64_t)kbs * a.bs_sk,
                 lb + WIN_SA + wid * 1024 + h * 256);
      }
    } else if (wid == NW - 1) {
      if (a.win4)
        win4_blocks(a.Bs, a.bs_sn, a.bs_sk, n0 >> 7, (a.N - 1) >> 7, 2, kb0, kb_end, lb + WIN_SA, lane);
      else if (lane < 4)
        dma16_ptr(sbw_src + kk, lb + WIN_SA);
    }
  };

  // Fragment reads: rows (lane & 15) of a 16-row group, logical chunks
  // 2*(lane>>4) and 2*(lane>>4)+1 at their swizzled slots.
  const int r7 = lane & 7, g2 = 2 * (lane >> 4);
  const int slo = (g2 ^ r7) << 4, shi = ((g2 + 1) ^ r7) << 4;
  // Fragment f (rows 16f..16f+15 of an operand tile): lane row q = lane&15
  // at block 8*(f/4) + q%8, segment 2*(f%4) + q/8.
  const int q_off = (lane & 7) * 1024 + ((lane >> 3) & 1) * 128;
  const int a_off = wm * (WM / 64) * 8192 + q_off;
  const int b_off = BM * 128 + wn * (WN / 64) * 8192 + q_off;
  auto frag_off = [](int f) { return (f >> 2) * 8192 + (f & 3) * 256; };
  auto rdx = [&](int stage, int i) {
    return lds_frag2(smem + stage * STAGE + a_off + frag_off(i), slo, shi);
  };
  auto rdw = [&](int stage, int j) {
    return lds_frag2(smem + stage * STAGE + b_off + frag_off(j), slo, shi);
  };
  const int sa_off = SW_OFF + (wm * WM + (lane & 15)) * 32;
  const int sb_off = SW_OFF + WIN_SA + ((wn * WN) >> 7) * 32;
  auto rdsa = [&](int rel, int i) {
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 4;
    return *reinterpret_cast<const float*>(smem + sa_off + o + i * 512);
  };
  auto rdsb = [&](int rel) {
    if constexpr (PR) return 1.0f;
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 4;
    return *reinterpret_cast<const float*>(smem + sb_off + o);
  };
  // PR: the lane's four column scales of weight fragment j at K-block rel
  auto rdsbj = [&](int rel, int j) {
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 1024;
    return *reinterpret_cast<const v4f*>(smem + SW_OFF + WIN_SA + o +
                                         (wn * WN + j * 16 + 4 * (lane >> 4)) * 4);
  };

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // MFMA order of a K-block; activation row i lives in fragment slot i & 3.
  constexpr int ORD_I[32] = {0, 1, 0, 1, 0, 1, 0, 1, 2, 2, 2, 2, 3, 3, 3, 3,
                             4, 4, 4, 4, 5, 5, 5, 5, 6, 7, 6, 7, 6, 7, 6, 7};
  constexpr int ORD_J[32] = {0, 0, 1, 1, 2, 2, 3, 3, 0, 1, 2, 3, 0, 1, 2, 3,
                             0, 1, 2, 3, 0, 1, 2, 3, 0, 0, 1, 1, 2, 2, 3, 3};
  v8i w[FN], xs[4];
  float sc[FM], sa_t[FM], sb_n = 0.f, sc6_old = 0.f, sc7_old = 0.f;
  v4f sbj[PR ? FN : 1];
#pragma unroll
  for (int j = 0; j < (PR ? FN : 1); ++j) sbj[j] = v4f{0.f, 0.f, 0.f, 0.f};
  v4f r1 = v4f{0.f, 0.f, 0.f, 0.f}, r2 = r1;  // results of MFMAs p-1 and p-2

  if (nkb > 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) issue_op(kb_begin, 0, i);
    issue_win(kb_begin, 0);
    if (nkb > 1) {
#pragma unroll
      for (int i = 0; i < 8; ++i) issue_op(kb_begin + 1, 1, i);
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    w[0] = rdw(0, 0); w[1] = rdw(0, 1); w[2] = rdw(0, 2);
    xs[0] = rdx(0, 0); xs[1] = rdx(0, 1);
    sb_n = rdsb(0);
    sa_t[0] = rdsa(0, 0); sa_t[1] = rdsa(0, 1);
    if constexpr (PR) { sbj[0] = rdsbj(0, 0); sbj[1] = rdsbj(0, 1); }
  }

  // One K-block. KIND 0: steady state (reads the next K-block, DMA of
  // kb+2); 1: next K-block exists but no kb+2; 2: last K-block.
  // The empty asm statements pin each MFMA result and accumulator update in
  // program order (LLVM would otherwise sink the pure MFMA/FMA chain past the
  // barrier), and sched_barrier keeps the machine scheduler from regrouping
  // the reads and the DMA.
  auto body = [&](int kb, auto tag) {
    constexpr int KIND = decltype(tag)::value;
    const int rel = kb - kb_begin;
    const int s = rel & 1;
    const float sb = sb_n;
#pragma unroll
    for (int p = 0; p < 32; ++p) {
      const int i = ORD_I[p], j = ORD_J[p];
      if (p == 24 && KIND < 2) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __syncthreads();
        if (KIND == 0 && ((rel + 2) & 7) == 0) issue_win(kb + 2, ((rel + 2) >> 3) & 1);
      }
      v4f res = mfma16x16x128(w[j], xs[i & 3]);
      asm volatile("" : "+v"(res));
      // Within the step: MFMA, then the LDS reads and DMA, then the folds of
      // MFMA p-2 (measured 2-3% faster than folding before the reads).
      __builtin_amdgcn_sched_barrier(0);
      // This K-block's remaining fragments and activation scales.
      if (p == 0) w[3] = rdw(s, 3);
      if (p == 1) { xs[2] = rdx(s, 2); sa_t[2] = rdsa(rel, 2); }
      if (p == 3) { xs[3] = rdx(s, 3); sa_t[3] = rdsa(rel, 3); }
      if (p == 7) { xs[0] = rdx(s, 4); sa_t[4] = rdsa(rel, 4); }
      if (p == 8) { xs[1] = rdx(s, 5); sa_t[5] = rdsa(rel, 5); }
      if (p == 12) { xs[2] = rdx(s, 6); sa_t[6] = rdsa(rel, 6); }
      if (p == 16) { xs[3] = rdx(s, 7); sa_t[7] = rdsa(rel, 7); }
      // PR: column scales of fragments 2 and 3, each read once the previous
      // K-block's last fold with it has been issued
      if constexpr (PR) {
        if (p == 0) sbj[2] = rdsbj(rel, 2);
        if (p == 2) sbj[3] = rdsbj(rel, 3);
      }
      // Scale of row i, computed just before the FMA of its first MFMA.
      if (p == 1) { sc[0] = sa_t[0] * sb; sc[1] = sa_t[1] * sb; }
      if (p == 9) sc[2] = sa_t[2] * sb;
      if (p == 13) sc[3] = sa_t[3] * sb;
      if (p == 17) sc[4] = sa_t[4] * sb;
      if (p == 21) sc[5] = sa_t[5] * sb;
      if (p == 25) { sc[6] = sa_t[6] * sb; sc[7] = sa_t[7] * sb; }
      // After the barrier: the next K-block's first fragments (stage s^1)
      // and the DMA of K-block kb+2 into stage s.
      if (KIND < 2 && p >= 24) {
        if (KIND == 0) issue_op(kb + 2, s, p - 24);
        if (p == 24) { xs[0] = rdx(s ^ 1, 0); sb_n = rdsb(rel + 1); sa_t[0] = rdsa(rel + 1, 0); }
        if (p == 25) { xs[1] = rdx(s ^ 1, 1); sa_t[1] = rdsa(rel + 1, 1); }
        if (p == 26) w[0] = rdw(s ^ 1, 0);
        if (p == 28) w[1] = rdw(s ^ 1, 1);
        if (p == 30) w[2] = rdw(s ^ 1, 2);
        if constexpr (PR) {
          if (p == 28) sbj[0] = rdsbj(rel + 1, 0);
          if (p == 30) sbj[1] = rdsbj(rel + 1, 1);
        }
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if (p >= 2) {
        const int qi = ORD_I[p - 2], qj = ORD_J[p - 2];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[qi][qj][e] = fmaf(r2[e], PR ? sc[qi] * sbj[qj % (PR ? FN : 1)][e] : sc[qi],
                                acc[qi][qj][e]);
        asm volatile("" : "+v"(acc[qi][qj]));
      } else {
        // the previous K-block's last two MFMAs: rows 6 and 7, column 3
        // (PR: fragment 3's column scales are reloaded only at p == 2)
        const int qi = 6 + p;
        const float so = p == 0 ? sc6_old : sc7_old;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[qi][3][e] = fmaf(r2[e], PR ? so * sbj[PR ? 3 : 0][e] : so, acc[qi][3][e]);
        asm volatile("" : "+v"(acc[qi][3]));
      }
      r2 = r1;
      r1 = res;
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
    sc6_old = sc[6];
    sc7_old = sc[7];
  };

  int kb = kb_begin;
  for (; kb + 2 < kb_end; ++kb) body(kb, PipeKind<0>{});
  if (kb + 1 < kb_end) {
    body(kb, PipeKind<1>{});
    ++kb;
  }
  if (kb < kb_end) {
    body(kb, PipeKind<2>{});
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[6][3][e] = fmaf(r2[e], PR ? sc[6] * sbj[PR ? 3 : 0][e] : sc[6], acc[6][3][e]);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[7][3][e] = fmaf(r1[e], PR ? sc[7] * sbj[PR ? 3 : 0][e] : sc[7], acc[7][3][e]);
  }
  // The last K-block has no barrier: wait for every wave before the epilogue
  // reuses the operand stages.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  if constexpr (SWIGLU) {
    swiglu_epilogue<BM, WM, WN>(a, smem, acc, m0, tn, wid, lane);
    return;
  } else {
    int64_t ld = 0;
    if (float* dst = f32_tile_dest(a, n0, BN, split, ld)) {
      // two rounds of 128 rows (waves 0-3, then 4-7): the padded 256 x 256
      // tile exceeds the dead stages
      static_assert(128 * (BN + 4) * 4 <= SMEM && WM == 128, "half the fp32 tile fits");
      f32_tile_lds<BM, BN, 128>(a, smem, m0, n0, dst, ld, [&](float* tile, int pitch, int r0) {
        if (wm * WM != r0) return;  // wave-uniform
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            *reinterpret_cast<v4f*>(tile + (i * 16 + (lane & 15)) * pitch + wn * WN + j * 16 +
                                    4 * (lane >> 4)) = acc[i][j];
      });
      return;
    }
  }
  tile_epilogue<WM, WN>(a, smem, acc, m0 + wm * WM, n0 + wn * WN, wid, lane, split);
}

// ---------------------------------------------------------------------------
// Pipelined 192x256 kernel: the scheme of gemm_pipe256_kernel on a tile of
// 192 activation rows, for grids that 256x256 tiles leave with a partial last
// wave while 192-row tiles fill whole waves (M = 3001: the gate/up GEMM of
// the MLP has 16 x 112 = 7 x 256 tiles against 12 x 112 = 5.25 waves, the
// down projection 16 x 16 = 256 against 192). Per output the arithmetic is
// the other kernels' (one zero-accumulator MFMA per 16x16 sub-tile and
// K-block, folded as acc + dot * (As * Bs) in K order), so the result bits
// are the same as on any unsplit plan.
//   * 8 waves of 96x64 (2 x 4): six activation and four weight fragments,
//     24 MFMAs per K-block, all six activation fragments in registers
//     (no slot reuse inside a K-block).
//   * MFMA order: rows 0-1 column-major in pairs, rows 2-3 row-major, rows
//     4-5 column-major in pairs. Rows 4-5 and weight fragment 3 of a K-block
//     are read at its MFMAs 0-3; one barrier per K-block before MFMA 16 (every
//     wave has read the whole current stage, and its DMA of the next stage has
//     landed); after it the next K-block's rows 0-3 and weight fragments 0-2
//     are read into the registers their last use just freed, and the DMA of
//     K-block kb+2 goes into the released stage, one instruction per MFMA.
//   * Stage: 192 + 256 rows of 128 bytes (56 KiB) in the block layout of
//     gemm_pipe256_kernel (A blocks 0-23, B blocks 24-55), two stages; scale
//     windows of 8 K-blocks as there.
// SWIGLU: the gate/up epilogue of gemm_pipe256_kernel on 192-row tiles.
// Preconditions: those of gemm_pipe256_kernel (pipe_ok), block_n = 128.
// ---------------------------------------------------------------------------
template <bool SWIGLU = false>
__global__ void __launch_bounds__(512) gemm_pipe192_kernel(GemmArgs a) {
  constexpr int BM = 192, BN = 256, WM = 96, WN = 64, NWN = BN / WN, NW = 8;
  constexpr int FM = WM / 16, FN = WN / 16;       // 6 activation, 4 weight fragments
  constexpr int NP = FM * FN;                     // 24 MFMAs per K-block
  constexpr int STAGE = (BM + BN) * 128;          // 56 KiB
  constexpr int LPW = (BM + BN) / 8 / NW;         // 7 wave-loads per wave per K-block
  constexpr int A_LOADS = BM / 64;                // wave-loads i < 3 bring A rows
  constexpr int WIN_SA = BM * 32;
  constexpr int WIN = WIN_SA + 256;
  constexpr int SW_OFF = 2 * STAGE;
  constexpr int EPI_PITCH = WN * 2 + 16;
  constexpr int EPI = NW * WM * EPI_PITCH;
  constexpr int SMEM = (2 * STAGE + 2 * WIN > EPI) ? 2 * STAGE + 2 * WIN : EPI;
  constexpr int BAR = 16;                         // MFMA index of the barrier
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert(LPW <= NP - BAR, "one DMA instruction per MFMA after the barrier");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid / NWN, wn = wid % NWN;

  int tm, tn;
  tile_of_bid((int)blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int split = blockIdx.z;
  const int kb_begin = split * a.kb_per_split;
  const int kb_end = min(kb_begin + a.kb_per_split, a.KB);
  const int nkb = kb_end - kb_begin;

  const uint32_t lds0 = lds_u32(smem);
  const int r8 = lane >> 3;
  const uint8_t* a_base = a.A + (int64_t)m0 * a.lda;
  const uint8_t* b_base = a.B + (int64_t)n0 * a.ldb;
  const int a_lim = a.M - 1 - m0, b_lim = a.N - 1 - n0;
  // wave-load L = wid + 8i: stage block L (A blocks 0..23, B blocks 24..55)
  auto issue_op = [&](int kb, int stage, int i) {
    const int L = wid + i * NW;
    const uint32_t lds = lds0 + stage * STAGE + L * 1024;
    const int Lr = i < A_LOADS ? L : L - BM / 8;
    const int row = (Lr >> 3) * 64 + r8 * 8 + (Lr & 7);
    const int c16 = ((lane & 7) ^ (Lr & 7)) * 16;
    if (i < A_LOADS) {
      const uint32_t voff = (uint32_t)min(row, a_lim) * (uint32_t)a.lda + c16;
      dma16_soff(voff, a_base + (int64_t)kb * 128, lds);
    } else {
      const uint32_t voff = (uint32_t)min(row, b_lim) * (uint32_t)a.ldb + c16;
      dma16_soff(voff, b_base + (int64_t)kb * 128, lds);
    }
  };
  // Scale window of 8 K-blocks: waves 0..5 bring As rows 32w..32w+31, wave 7
  // the Bs rows of the tile's two 128-column blocks.
  const float* saw_src =
      a.As + (int64_t)min(m0 + min(wid * 32 + (lane >> 1), BM - 1), a.M - 1) * a.as_sm +
      4 * (lane & 1);
  const float* sbw_src =
      a.Bs + (int64_t)min((n0 >> 7) + min(lane >> 1, 1), (a.N - 1) >> 7) * a.bs_sn + 4 * (lane & 1);
  auto issue_win = [&](int kb0, int wbuf) {
    const int kk = (kb0 + 4 * (lane & 1) < kb_end) ? kb0 : kb0 - 4 * (lane & 1);
    const uint32_t lb = lds0 + SW_OFF + wbuf * WIN;
    if (a.win4) {
      if (wid < BM / 32)
        win4_rows(a.As, a.as_sm, a.as_sk, m0 + wid * 32, a.M - 1, kb0, kb_end, lb + wid * 1024,
                  lane);
      if (wid == NW - 1)
        win4_blocks(a.Bs, a.bs_sn, a.bs_sk, n0 >> 7, (a.N - 1) >> 7, 2, kb0, kb_end, lb + WIN_SA, lane);
    } else {
      if (wid < BM / 32) dma16_ptr(saw_src + kk, lb + wid * 1024);
      if (wid == NW - 1 && lane < 4) dma16_ptr(sbw_src + kk, lb + WIN_SA);
    }
  };

  const int r7 = lane & 7, g2 = 2 * (lane >> 4);
  const int slo = (g2 ^ r7) << 4, shi = ((g2 + 1) ^ r7) << 4;
  const int q_off = (lane & 7) * 1024 + ((lane >> 3) & 1) * 128;
  // 16-row fragment F of an operand: block 8*(F/4) + q%8, segment 2*(F%4) + q/8
  auto frag_off = [](int f) { return (f >> 2) * 8192 + (f & 3) * 256; };
  auto rdx = [&](int stage, int i) {
    return lds_frag2(smem + stage * STAGE + q_off + frag_off(wm * FM + i), slo, shi);
  };
  auto rdw = [&](int stage, int j) {
    return lds_frag2(smem + stage * STAGE + BM * 128 + q_off + frag_off(wn * FN + j), slo, shi);
  };
  const int sa_off = SW_OFF + (wm * WM + (lane & 15)) * 32;
  const int sb_off = SW_OFF + WIN_SA + ((wn * WN) >> 7) * 32;
  auto rdsa = [&](int rel, int i) {
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 4;
    return *reinterpret_cast<const float*>(smem + sa_off + o + i * 512);
  };
  auto rdsb = [&](int rel) {
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 4;
    return *reinterpret_cast<const float*>(smem + sb_off + o);
  };

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  constexpr int ORD_I[NP] = {0, 1, 0, 1, 0, 1, 0, 1, 2, 2, 2, 2,
                             3, 3, 3, 3, 4, 5, 4, 5, 4, 5, 4, 5};
  constexpr int ORD_J[NP] = {0, 0, 1, 1, 2, 2, 3, 3, 0, 1, 2, 3,
                             0, 1, 2, 3, 0, 0, 1, 1, 2, 2, 3, 3};
  v8i w[FN], xs[FM];
  float sc[FM], sa_t[FM], sb_n = 0.f;
  v4f r1 = v4f{0.f, 0.f, 0.f, 0.f}, r2 = r1;  // results of MFMAs p-1 and p-2

  if (nkb > 0) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) issue_op(kb_begin, 0, i);
    issue_win(kb_begin, 0);
    if (nkb > 1) {
#pragma unroll
      for (int i = 0; i < LPW; ++i) issue_op(kb_begin + 1, 1, i);
      wait_vmcnt<LPW>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();
    w[0] = rdw(0, 0); w[1] = rdw(0, 1); w[2] = rdw(0, 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) { xs[i] = rdx(0, i); sa_t[i] = rdsa(0, i); }
    sb_n = rdsb(0);
  }

  // One K-block. KIND 0: steady state (reads the next K-block, DMA of
  // kb+2); 1: next K-block exists but no kb+2; 2: last K-block. Empty asm
  // statements and sched_barrier keep the MFMAs, reads and folds in the
  // written order, as in gemm_pipe256_kernel.
  auto body = [&](int kb, auto tag) {
    constexpr int KIND = decltype(tag)::value;
    const int rel = kb - kb_begin;
    const int s = rel & 1;
    const float sb = sb_n;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int i = ORD_I[p], j = ORD_J[p];
      if (p == BAR && KIND < 2) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __syncthreads();
        if (KIND == 0 && ((rel + 2) & 7) == 0) issue_win(kb + 2, ((rel + 2) >> 3) & 1);
      }
      v4f res = mfma16x16x128(w[j], xs[i]);
      asm volatile("" : "+v"(res));
      __builtin_amdgcn_sched_barrier(0);
      // this K-block's last fragments and activation scales
      if (p == 0) w[3] = rdw(s, 3);
      if (p == 1) { xs[4] = rdx(s, 4); sa_t[4] = rdsa(rel, 4); }
      if (p == 3) { xs[5] = rdx(s, 5); sa_t[5] = rdsa(rel, 5); }
      // scale of row i, just before the fold of its first MFMA
      if (p == 1) { sc[0] = sa_t[0] * sb; sc[1] = sa_t[1] * sb; }
      if (p == 9) sc[2] = sa_t[2] * sb;
      if (p == 13) sc[3] = sa_t[3] * sb;
      if (p == 17) { sc[4] = sa_t[4] * sb; sc[5] = sa_t[5] * sb; }
      // after the barrier: the next K-block's first fragments (stage s^1)
      // and the DMA of K-block kb+2 into stage s
      if (KIND < 2 && p >= BAR) {
        if (KIND == 0 && p - BAR < LPW) issue_op(kb + 2, s, p - BAR);
        if (p == BAR) { xs[0] = rdx(s ^ 1, 0); sb_n = rdsb(rel + 1); sa_t[0] = rdsa(rel + 1, 0); }
        if (p == BAR + 1) { xs[1] = rdx(s ^ 1, 1); sa_t[1] = rdsa(rel + 1, 1); }
        if (p == BAR + 2) w[0] = rdw(s ^ 1, 0);
        if (p == BAR + 3) { xs[2] = rdx(s ^ 1, 2); sa_t[2] = rdsa(rel + 1, 2); }
        if (p == BAR + 4) w[1] = rdw(s ^ 1, 1);
        if (p == BAR + 5) { xs[3] = rdx(s ^ 1, 3); sa_t[3] = rdsa(rel + 1, 3); }
        if (p == BAR + 6) w[2] = rdw(s ^ 1, 2);
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if (p >= 2) {
        const int qi = ORD_I[p - 2], qj = ORD_J[p - 2];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[qi][qj][e] = fmaf(r2[e], sc[qi], acc[qi][qj][e]);
        asm volatile("" : "+v"(acc[qi][qj]));
      } else {
        // the previous K-block's last two MFMAs: rows 4 and 5, column 3
        // (their scales are rewritten only at MFMA 17)
        const int qi = FM - 2 + p;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[qi][3][e] = fmaf(r2[e], sc[qi], acc[qi][3][e]);
        asm volatile("" : "+v"(acc[qi][3]));
      }
      r2 = r1;
      r1 = res;
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // sc starts at zero so the first K-block's two "previous" folds add 0.
#pragma unroll
  for (int i = 0; i < FM; ++i) sc[i] = 0.f;
  int kb = kb_begin;
  for (; kb + 2 < kb_end; ++kb) body(kb, PipeKind<0>{});
  if (kb + 1 < kb_end) {
    body(kb, PipeKind<1>{});
    ++kb;
  }
  if (kb < kb_end) {
    body(kb, PipeKind<2>{});
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[FM - 2][3][e] = fmaf(r2[e], sc[FM - 2], acc[FM - 2][3][e]);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[FM - 1][3][e] = fmaf(r1[e], sc[FM - 1], acc[FM - 1][3][e]);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  if constexpr (SWIGLU) {
    swiglu_epilogue<BM, WM, WN>(a, smem, acc, m0, tn, wid, lane);
    return;
  }
  tile_epilogue<WM, WN>(a, smem, acc, m0 + wm * WM, n0 + wn * WN, wid, lane, split);
}

// ---------------------------------------------------------------------------
// Pipelined 256x128 kernel: the scheme of gemm_pipe192_kernel on tiles of 256
// activation rows by one 128-column weight block, for grids where 256x256
// tiles leave CUs idle while 128x128 tiles need extra waves (M x N = 2048 x
// 4096: 128 tiles of 256x256, 512 of 128x128, 256 of 256x128 on 256 CUs).
// Per output the arithmetic is the other kernels' (one zero-accumulator MFMA
// per 16x16 sub-tile and K-block, folded as acc + dot * (As * Bs) in K
// order), so the result bits are those of any unsplit plan.
//   * 8 waves of 64x64 (4 x 2): four activation and four weight fragments,
//     16 MFMAs per K-block.
//   * MFMA order: rows 0-1, then rows 2-3, each pair column-major. Weight
//     fragment 3 and rows 2-3 of a K-block are read at its MFMAs 0-3; one
//     barrier per K-block before MFMA 8 (every wave has read the whole
//     current stage, and its DMA of the next stage has landed); after it the
//     next K-block's rows 0-1 and weight fragments 0-2 are read into the
//     registers their last use just freed, and the DMA of K-block kb+2 goes
//     into the released stage, one instruction per MFMA.
//   * Stage: 256 + 128 rows of 128 bytes (48 KiB) in the block layout of
//     gemm_pipe256_kernel (A blocks 0-31, B blocks 32-47), two stages; scale
//     windows of 8 K-blocks as there, with the tile's single weight-scale row
//     (one scale per K-block for all 128 columns).
// PR (per-row weight scales, block_n = 1): as in gemm_pipe256_kernel, the
// window holds the 128 weight rows' scales slot-major (4-byte DMA lanes) and
// each fold multiplies the row scale by the lane's four column scales, read
// per weight fragment and K-block as one 16-byte load into the register its
// previous value just left.
// Preconditions: those of gemm_pipe256_kernel (pipe_ok); block_n = 128, or
// 1 with PR.
// ---------------------------------------------------------------------------
template <bool PR>
__global__ void __launch_bounds__(512) gemm_pipe256x128_kernel(GemmArgs a) {
  constexpr int BM = 256, BN = 128, WM = 64, WN = 64, NWN = BN / WN, NW = 8;
  constexpr int FM = WM / 16, FN = WN / 16;       // 4 activation, 4 weight fragments
  constexpr int NP = FM * FN;                     // 16 MFMAs per K-block
  constexpr int STAGE = (BM + BN) * 128;          // 48 KiB
  constexpr int LPW = (BM + BN) / 8 / NW;         // 6 wave-loads per wave per K-block
  constexpr int A_LOADS = BM / 64;                // wave-loads i < 4 bring A rows
  constexpr int WIN_SA = BM * 32;
  constexpr int WIN = WIN_SA + (PR ? 8 * BN * 4 : 256);
  constexpr int SW_OFF = 2 * STAGE;
  constexpr int EPI_PITCH = WN * 2 + 16;
  constexpr int EPI = NW * WM * EPI_PITCH;
  constexpr int SMEM = (2 * STAGE + 2 * WIN > EPI) ? 2 * STAGE + 2 * WIN : EPI;
  constexpr int BAR = 8;                          // MFMA index of the barrier
  static_assert(SMEM <= 160 * 1024, "LDS budget");
  static_assert(LPW <= NP - BAR, "one DMA instruction per MFMA after the barrier");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid / NWN, wn = wid % NWN;

  int tm, tn;
  if (a.rem_base >= 0) {
    // a 128-column half of one of the 256x256 tiles a gemm_pipe256_kernel
    // launch left
    tile_of_bid(a.rem_base + (int)blockIdx.x / 2, a.rem_tiles_m, a.rem_tiles_n, tm, tn);
    tn = 2 * tn + ((int)blockIdx.x & 1);
  } else {
    tile_of_bid((int)blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  }
  const int m0 = tm * BM, n0 = tn * BN;
  if (n0 >= a.N) return;  // a half past the matrix edge (whole workgroup)

  const int split = blockIdx.z;
  const int kb_begin = split * a.kb_per_split;
  const int kb_end = min(kb_begin + a.kb_per_split, a.KB);
  const int nkb = kb_end - kb_begin;

  const uint32_t lds0 = lds_u32(smem);
  const int r8 = lane >> 3;
  const uint8_t* a_base = a.A + (int64_t)m0 * a.lda;
  const uint8_t* b_base = a.B + (int64_t)n0 * a.ldb;
  const int a_lim = a.M - 1 - m0, b_lim = a.N - 1 - n0;
  // wave-load L = wid + 8i: stage block L (A blocks 0..31, B blocks 32..47)
  auto issue_op = [&](int kb, int stage, int i) {
    const int L = wid + i * NW;
    const uint32_t lds = lds0 + stage * STAGE + L * 1024;
    const int Lr = i < A_LOADS ? L : L - BM / 8;
    const int row = (Lr >> 3) * 64 + r8 * 8 + (Lr & 7);
    const int c16 = ((lane & 7) ^ (Lr & 7)) * 16;
    if (i < A_LOADS) {
      const uint32_t voff = (uint32_t)min(row, a_lim) * (uint32_t)a.lda + c16;
      dma16_soff(voff, a_base + (int64_t)kb * 128, lds);
    } else {
      const uint32_t voff = (uint32_t)min(row, b_lim) * (uint32_t)a.ldb + c16;
      dma16_soff(voff, b_base + (int64_t)kb * 128, lds);
    }
  };
  // Scale window of 8 K-blocks: wave w brings As rows 32w..32w+31 (two lanes
  // per row, 4 K-blocks each); lanes 0-1 of wave 7 also bring the tile's Bs
  // row (PR: wave w brings slot w, the 128 rows' scales of K-block kb0 + w).
  // With 16-byte lanes a half-window past kb_end re-reads the first half (KB
  // is then a multiple of 4), so no lane reads past the row.
  const float* saw_src =
      a.As + (int64_t)min(m0 + wid * 32 + (lane >> 1), a.M - 1) * a.as_sm + 4 * (lane & 1);
  const float* sbw_src = a.Bs + (int64_t)(n0 >> 7) * a.bs_sn + 4 * (lane & 1);
  auto issue_win = [&](int kb0, int wbuf) {
    const int kk = (kb0 + 4 * (lane & 1) < kb_end) ? kb0 : kb0 - 4 * (lane & 1);
    const uint32_t lb = lds0 + SW_OFF + wbuf * WIN;
    if (a.win4)
      win4_rows(a.As, a.as_sm, a.as_sk, m0 + wid * 32, a.M - 1, kb0, kb_end, lb + wid * 1024, lane);
    else
      dma16_ptr(saw_src + kk, lb + wid * 1024);
    if constexpr (PR) {
      const int kbs = min(kb0 + wid, kb_end - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int row = n0 + h * 64 + lane;
        asm volatile("" : "+v"(row));
        dma4_ptr(a.Bs + (int64_t)min(row, a.N - 1) * a.bs_sn + (int64_t)kbs * a.bs_sk,
                 lb + WIN_SA + wid * 512 + h * 256);
      }
    } else if (wid == NW - 1) {
      if (a.win4)
        win4_blocks(a.Bs, a.bs_sn, a.bs_sk, n0 >> 7, (a.N - 1) >> 7, 1, kb0, kb_end, lb + WIN_SA, lane);
      else if (lane < 2)
        dma16_ptr(sbw_src + kk, lb + WIN_SA);
    }
  };

  const int r7 = lane & 7, g2 = 2 * (lane >> 4);
  const int slo = (g2 ^ r7) << 4, shi = ((g2 + 1) ^ r7) << 4;
  const int q_off = (lane & 7) * 1024 + ((lane >> 3) & 1) * 128;
  // 16-row fragment F of an operand: block 8*(F/4) + q%8, segment 2*(F%4) + q/8
  auto frag_off = [](int f) { return (f >> 2) * 8192 + (f & 3) * 256; };
  auto rdx = [&](int stage, int i) {
    return lds_frag2(smem + stage * STAGE + q_off + frag_off(wm * FM + i), slo, shi);
  };
  auto rdw = [&](int stage, int j) {
    return lds_frag2(smem + stage * STAGE + BM * 128 + q_off + frag_off(wn * FN + j), slo, shi);
  };
  const int sa_off = SW_OFF + (wm * WM + (lane & 15)) * 32;
  auto rdsa = [&](int rel, int i) {
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 4;
    return *reinterpret_cast<const float*>(smem + sa_off + o + i * 512);
  };
  auto rdsb = [&](int rel) {
    if constexpr (PR) return 1.0f;
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 4;
    return *reinterpret_cast<const float*>(smem + SW_OFF + WIN_SA + o);
  };
  // PR: the lane's four column scales of weight fragment j at K-block rel
  auto rdsbj = [&](int rel, int j) {
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 512;
    return *reinterpret_cast<const v4f*>(smem + SW_OFF + WIN_SA + o +
                                         (wn * WN + j * 16 + 4 * (lane >> 4)) * 4);
  };

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  constexpr int ORD_I[NP] = {0, 1, 0, 1, 0, 1, 0, 1, 2, 3, 2, 3, 2, 3, 2, 3};
  constexpr int ORD_J[NP] = {0, 0, 1, 1, 2, 2, 3, 3, 0, 0, 1, 1, 2, 2, 3, 3};
  v8i w[FN], xs[FM];
  float sc[FM], sa_t[FM], sb_n = 0.f;
  v4f sbj[PR ? FN : 1];
#pragma unroll
  for (int j = 0; j < (PR ? FN : 1); ++j) sbj[j] = v4f{0.f, 0.f, 0.f, 0.f};
  v4f r1 = v4f{0.f, 0.f, 0.f, 0.f}, r2 = r1;  // results of MFMAs p-1 and p-2

  if (nkb > 0) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) issue_op(kb_begin, 0, i);
    issue_win(kb_begin, 0);
    if (nkb > 1) {
#pragma unroll
      for (int i = 0; i < LPW; ++i) issue_op(kb_begin + 1, 1, i);
      wait_vmcnt<LPW>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();
    w[0] = rdw(0, 0); w[1] = rdw(0, 1); w[2] = rdw(0, 2);
    xs[0] = rdx(0, 0); xs[1] = rdx(0, 1);
    sa_t[0] = rdsa(0, 0); sa_t[1] = rdsa(0, 1);
    sb_n = rdsb(0);
    if constexpr (PR) { sbj[0] = rdsbj(0, 0); sbj[1] = rdsbj(0, 1); }
  }

  // One K-block. KIND 0: steady state (reads the next K-block, DMA of
  // kb+2); 1: next K-block exists but no kb+2; 2: last K-block. Empty asm
  // statements and sched_barrier keep the MFMAs, reads and folds in the
  // written order, as in gemm_pipe256_kernel.
  auto body = [&](int kb, auto tag) {
    constexpr int KIND = decltype(tag)::value;
    const int rel = kb - kb_begin;
    const int s = rel & 1;
    const float sb = sb_n;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int i = ORD_I[p], j = ORD_J[p];
      if (p == BAR && KIND < 2) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __syncthreads();
        if (KIND == 0 && ((rel + 2) & 7) == 0) issue_win(kb + 2, ((rel + 2) >> 3) & 1);
      }
      v4f res = mfma16x16x128(w[j], xs[i]);
      asm volatile("" : "+v"(res));
      __builtin_amdgcn_sched_barrier(0);
      // this K-block's last weight fragment, rows 2-3 and their scales
      if (p == 0) w[3] = rdw(s, 3);
      if (p == 1) { xs[2] = rdx(s, 2); sa_t[2] = rdsa(rel, 2); }
      if (p == 3) { xs[3] = rdx(s, 3); sa_t[3] = rdsa(rel, 3); }
      // PR: column scales of fragments 2 and 3, each read once the previous
      // K-block's last fold with it has been issued
      if constexpr (PR) {
        if (p == 0) sbj[2] = rdsbj(rel, 2);
        if (p == 2) sbj[3] = rdsbj(rel, 3);
      }
      // scale of row i, just before the fold of its first MFMA
      if (p == 1) { sc[0] = sa_t[0] * sb; sc[1] = sa_t[1] * sb; }
      if (p == 9) { sc[2] = sa_t[2] * sb; sc[3] = sa_t[3] * sb; }
      // after the barrier: the next K-block's rows 0-1 and weight fragments
      // 0-2 (stage s^1) and the DMA of K-block kb+2 into stage s
      if (KIND < 2 && p >= BAR) {
        if (KIND == 0 && p - BAR < LPW) issue_op(kb + 2, s, p - BAR);
        if (p == BAR) { xs[0] = rdx(s ^ 1, 0); sb_n = rdsb(rel + 1); sa_t[0] = rdsa(rel + 1, 0); }
        if (p == BAR + 1) { xs[1] = rdx(s ^ 1, 1); sa_t[1] = rdsa(rel + 1, 1); }
        if (p == BAR + 2) w[0] = rdw(s ^ 1, 0);
        if (p == BAR + 4) w[1] = rdw(s ^ 1, 1);
        if (p == BAR + 6) w[2] = rdw(s ^ 1, 2);
        // PR: the next K-block's column scales of fragments 0 and 1, after
        // this K-block's last folds with them (MFMAs 9 and 11)
        if constexpr (PR) {
          if (p == 12) sbj[0] = rdsbj(rel + 1, 0);
          if (p == 14) sbj[1] = rdsbj(rel + 1, 1);
        }
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if (p >= 2) {
        const int qi = ORD_I[p - 2], qj = ORD_J[p - 2];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[qi][qj][e] = fmaf(r2[e], PR ? sc[qi] * sbj[qj % (PR ? FN : 1)][e] : sc[qi],
                                acc[qi][qj][e]);
        asm volatile("" : "+v"(acc[qi][qj]));
      } else {
        // the previous K-block's last two MFMAs: rows 2 and 3, column 3
        // (their scales are rewritten only at MFMA 9; PR: fragment 3's
        // column scales only at MFMA 2)
        const int qi = FM - 2 + p;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[qi][3][e] = fmaf(r2[e], PR ? sc[qi] * sbj[PR ? 3 : 0][e] : sc[qi], acc[qi][3][e]);
        asm volatile("" : "+v"(acc[qi][3]));
      }
      r2 = r1;
      r1 = res;
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // sc starts at zero so the first K-block's two "previous" folds add 0.
#pragma unroll
  for (int i = 0; i < FM; ++i) sc[i] = 0.f;
  int kb = kb_begin;
  for (; kb + 2 < kb_end; ++kb) body(kb, PipeKind<0>{});
  if (kb + 1 < kb_end) {
    body(kb, PipeKind<1>{});
    ++kb;
  }
  if (kb < kb_end) {
    body(kb, PipeKind<2>{});
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[FM - 2][3][e] =
          fmaf(r2[e], PR ? sc[FM - 2] * sbj[PR ? 3 : 0][e] : sc[FM - 2], acc[FM - 2][3][e]);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[FM - 1][3][e] =
          fmaf(r1[e], PR ? sc[FM - 1] * sbj[PR ? 3 : 0][e] : sc[FM - 1], acc[FM - 1][3][e]);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int64_t ld = 0;
  if (float* dst = f32_tile_dest(a, n0, BN, split, ld)) {
    // two rounds of 128 rows: the padded 256-row tile exceeds the stages
    static_assert(128 * (BN + 4) * 4 <= SMEM, "half the fp32 tile fits the dead stages");
    f32_tile_lds<BM, BN, 128>(a, smem, m0, n0, dst, ld, [&](float* tile, int pitch, int r0) {
      if (wm * WM < r0 || wm * WM >= r0 + 128) return;  // wave-uniform
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          *reinterpret_cast<v4f*>(tile + (wm * WM - r0 + i * 16 + (lane & 15)) * pitch +
                                  wn * WN + j * 16 + 4 * (lane >> 4)) = acc[i][j];
    });
    return;
  }
  tile_epilogue<WM, WN>(a, smem, acc, m0 + wm * WM, n0 + wn * WN, wid, lane, split);
}

// ---------------------------------------------------------------------------
// Pipelined 128x128 kernel (grids below one 256x256 tile per CU, and the
// split-K path). Waves of WM x WN (two per SIMD for 64x32); with half the operand
// reuse of a 256x256 tile this size is bound by the operand stream, so it
// keeps three K-blocks of DMA in flight: four LDS stages of 32 KiB, the DMA
// of K-block kb+4 issued right after the barrier that opens K-block kb. Each
// K-block's fragments are read from LDS during the previous K-block's MFMAs
// into the other of two register sets; scale windows and asm DMA as in
// gemm_pipe256_kernel.
// ---------------------------------------------------------------------------
template <int WM, int WN, bool PR>
__global__ void __launch_bounds__((128 / WM) * (128 / WN) * 64) gemm_pipe128_kernel(GemmArgs a) {
  constexpr int BM = 128, BN = 128, NWN = BN / WN, NW = (BM / WM) * NWN;
  constexpr int FM = WM / 16, FN = WN / 16;
  static_assert(FM * FN >= FM + FN + 1, "next-K-block reads must fit between the MFMAs");
  static_assert(NW >= BM / 32, "one scale-window instruction per 32 activation rows");
  constexpr int NSTAGE = 4;
  constexpr int STAGE = (BM + BN) * 128;   // 32 KiB
  constexpr int WIN_SA = BM * 32;
  // PR (per-row weight scales, block_n = 1): Bs rows of the tile in the
  // window as the As rows are (32 bytes per row: 8 K-blocks).
  constexpr int WIN = WIN_SA + (PR ? BN * 32 : 256);
  constexpr int SW_OFF = NSTAGE * STAGE;
  constexpr int EPI_PITCH = WN * 2 + 16;
  constexpr int EPI = NW * WM * EPI_PITCH;
  constexpr int SMEM = (SW_OFF + 2 * WIN > EPI) ? SW_OFF + 2 * WIN : EPI;
  constexpr int LPW = (BM + BN) / 8 / NW;  // wave-loads per wave per K-block (8)
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid / NWN, wn = wid % NWN;

  int tm, tn;
  if (a.rem_base >= 0) {
    // a quarter of one of the 256x256 tiles a gemm_pipe256_kernel launch left
    tile_of_bid(a.rem_base + (int)blockIdx.x / 4, a.rem_tiles_m, a.rem_tiles_n, tm, tn);
    tm = 2 * tm + (((int)blockIdx.x >> 1) & 1);
    tn = 2 * tn + ((int)blockIdx.x & 1);
  } else {
    tile_of_bid((int)blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  }
  const int m0 = tm * BM, n0 = tn * BN;
  if (m0 >= a.M || n0 >= a.N) return;  // a quarter past the matrix edge (whole workgroup)

  const int split = blockIdx.z;
  const int kb_begin = split * a.kb_per_split;
  const int kb_end = min(kb_begin + a.kb_per_split, a.KB);
  const int nkb = kb_end - kb_begin;

  const uint32_t lds0 = lds_u32(smem);
  const int r8 = lane >> 3;
  const uint8_t* a_base = a.A + (int64_t)m0 * a.lda;
  const uint8_t* b_base = a.B + (int64_t)n0 * a.ldb;
  const int a_lim = a.M - 1 - m0, b_lim = a.N - 1 - n0;
  // Block layout of gemm_pipe256_kernel: block L of an operand holds rows
  // 64*(L/8) + 8*s + (L%8), chunk c in slot c ^ (L%8).
  auto issue_op = [&](int kb, int stage, int i) {
    const int L = wid + i * NW;
    const uint32_t lds = lds0 + stage * STAGE + L * 1024;
    const bool is_a = L < BM / 8;
    const int Lr = is_a ? L : L - BM / 8;
    const int row = (Lr >> 3) * 64 + r8 * 8 + (Lr & 7);
    const int c16 = ((lane & 7) ^ (Lr & 7)) * 16;
    if (is_a) {
      const uint32_t voff = (uint32_t)min(row, a_lim) * (uint32_t)a.lda + c16;
      dma16_soff(voff, a_base + (int64_t)kb * 128, lds);
    } else {
      const uint32_t voff = (uint32_t)min(row, b_lim) * (uint32_t)a.ldb + c16;
      dma16_soff(voff, b_base + (int64_t)kb * 128, lds);
    }
  };
  const float* saw_src =
      a.As + (int64_t)min(m0 + wid * 32 + (lane >> 1), a.M - 1) * a.as_sm + 4 * (lane & 1);
  const float* sbw_src = a.Bs + (int64_t)(n0 >> 7) * a.bs_sn + 4 * (lane & 1);
  auto issue_win = [&](int kb0, int wbuf) {
    const int kk = (kb0 + 4 * (lane & 1) < kb_end) ? kb0 : kb0 - 4 * (lane & 1);
    const uint32_t lb = lds0 + SW_OFF + wbuf * WIN;
    if (wid < BM / 32) {
      if (a.win4)
        win4_rows(a.As, a.as_sm, a.as_sk, m0 + wid * 32, a.M - 1, kb0, kb_end, lb + wid * 1024,
                  lane);
      else
        dma16_ptr(saw_src + kk, lb + wid * 1024);
    }
    if constexpr (PR) {
      // slot-major (slot s: the 128 rows' scales of K-block kb0 + s as
      // consecutive floats), so a lane reads its four rows in one 16-byte
      // load: waves NW-4..NW-1 issue 4 instructions each, one 4-byte lane
      // per row, for (slot, 64-row half) = (i/2, i%2), i = 4q + j
      if (wid >= NW - 4) {
        const int q = wid - (NW - 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = q * 4 + j, sl = i >> 1, h = i & 1;
          const int kbs = min(kb0 + sl, kb_end - 1);
          dma4_ptr(a.Bs + (int64_t)min(n0 + h * 64 + lane, a.N - 1) * a.bs_sn +
                       (int64_t)kbs * a.bs_sk,
                   lb + WIN_SA + sl * 512 + h * 256);
        }
      }
    } else if (wid == NW - 1) {
      if (a.win4)
        win4_blocks(a.Bs, a.bs_sn, a.bs_sk, n0 >> 7, (a.N - 1) >> 7, 1, kb0, kb_end, lb + WIN_SA, lane);
      else if (lane < 2)
        dma16_ptr(sbw_src + kk, lb + WIN_SA);
    }
  };
  // DMA of one K-block (and, at a window start, its scale window).
  auto issue_kb = [&](int kb) {
    const int rel = kb - kb_begin;
    if ((rel & 7) == 0) issue_win(kb, (rel >> 3) & 1);
#pragma unroll
    for (int i = 0; i < LPW; ++i) issue_op(kb, rel % NSTAGE, i);
  };

  const int r7 = lane & 7, g2 = 2 * (lane >> 4);
  const int slo = (g2 ^ r7) << 4, shi = ((g2 + 1) ^ r7) << 4;
  const int q_off = (lane & 7) * 1024 + ((lane >> 3) & 1) * 128;
  // operand fragment f: block 8*(f/4) + q%8, segment 2*(f%4) + q/8
  auto frag_off = [](int f) { return (f >> 2) * 8192 + (f & 3) * 256; };
  const int sa_off = SW_OFF + (wm * WM + (lane & 15)) * 32;
  const int sb_off = SW_OFF + WIN_SA;

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  v8i xf[2][FM], wf[2][FN];
  float sc[2][FM];
  v4f sbr[2][PR ? FN : 1];  // PR: the weight-row scales of the lane's 4 columns
  v4f r1 = v4f{0.f, 0.f, 0.f, 0.f}, r2 = r1;
  // Scale of output (row i, column group j, element e) in register set S.
  auto scale_of = [&](int S, int i, int j, int e) {
    if constexpr (PR) return sc[S][i] * sbr[S][j][e];
    else return sc[S][i];
  };

  // Fragments and scales of K-block kb into register set S (reads spread
  // over the caller's MFMAs by the caller's sched barriers).
  auto read_frag = [&](int kb, int S, int f) {
    const uint8_t* st = smem + ((kb - kb_begin) % NSTAGE) * STAGE;
    if (f < FM) xf[S][f] = lds_frag2(st + q_off + frag_off(wm * FM + f), slo, shi);
    else wf[S][f - FM] = lds_frag2(st + BM * 128 + q_off + frag_off(wn * FN + f - FM), slo, shi);
  };
  auto read_scales = [&](int kb, int S) {
    const int rel = kb - kb_begin;
    const int o = ((rel >> 3) & 1) * WIN + (rel & 7) * 4;
    if constexpr (PR) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        sc[S][i] = *reinterpret_cast<const float*>(smem + sa_off + o + i * 512);
      const int ob = ((rel >> 3) & 1) * WIN + (rel & 7) * 512;
#pragma unroll
      for (int j = 0; j < FN; ++j)
        sbr[S][j] = *reinterpret_cast<const v4f*>(
            smem + sb_off + ob + (wn * WN + j * 16 + 4 * (lane >> 4)) * 4);
    } else {
      const float sb = *reinterpret_cast<const float*>(smem + sb_off + o);
#pragma unroll
      for (int i = 0; i < FM; ++i)
        sc[S][i] = *reinterpret_cast<const float*>(smem + sa_off + o + i * 512) * sb;
    }
  };

  // Waits until this wave's DMA of a K-block has landed, given how many
  // K-blocks' DMAs it issued after that one (window instructions in between
  // only make the wait stricter).
  auto wait_after = [&](int n_after) {
    if (n_after >= 3) wait_vmcnt<3 * LPW>();
    else if (n_after == 2) wait_vmcnt<2 * LPW>();
    else if (n_after == 1) wait_vmcnt<LPW>();
    else wait_vmcnt<0>();
  };

  if (nkb > 0) {
    for (int k = 0; k < NSTAGE && k < nkb; ++k) issue_kb(kb_begin + k);
    wait_after(min(NSTAGE, nkb) - 1);
    __syncthreads();
#pragma unroll
    for (int f = 0; f < FM + FN; ++f) read_frag(kb_begin, 0, f);
    read_scales(kb_begin, 0);
  }

  auto body = [&](int kb, auto set_tag) {
    constexpr int S = decltype(set_tag)::value, T = S ^ 1;
    const bool more = kb + 1 < kb_end;
    if (more) {
      // outstanding: the DMAs of kb+1 .. min(kb+3, kb_end-1)
      wait_after(min(2, kb_end - kb - 2));
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __syncthreads();
      if (kb + NSTAGE < kb_end) issue_kb(kb + NSTAGE);
    }
#pragma unroll
    for (int p = 0; p < FM * FN; ++p) {
      const int i = p / FN, j = p % FN;
      v4f res = mfma16x16x128(wf[S][j], xf[S][i]);
      asm volatile("" : "+v"(res));
      if (p >= 2) {
        const int qi = (p - 2) / FN, qj = (p - 2) % FN;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[qi][qj][e] = fmaf(r2[e], scale_of(S, qi, qj, e), acc[qi][qj][e]);
        asm volatile("" : "+v"(acc[qi][qj]));
      } else {
        const int qj = FN - 2 + p;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[FM - 1][qj][e] = fmaf(r2[e], scale_of(T, FM - 1, qj, e), acc[FM - 1][qj][e]);
        asm volatile("" : "+v"(acc[FM - 1][qj]));
      }
      r2 = r1;
      r1 = res;
      if (more) {
        if (p < FM + FN) read_frag(kb + 1, T, p);
        if (p == FM + FN) read_scales(kb + 1, T);
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // sc[1] starts at zero so the first K-block's two "previous" folds add 0.
#pragma unroll
  for (int i = 0; i < FM; ++i) sc[1][i] = 0.f;
#pragma unroll
  for (int j = 0; j < (PR ? FN : 1); ++j) sbr[1][j] = v4f{0.f, 0.f, 0.f, 0.f};
  int kb = kb_begin;
  for (; kb + 1 < kb_end; kb += 2) {
    body(kb, PipeKind<0>{});
    body(kb + 1, PipeKind<1>{});
  }
  int last_set = 1;
  if (kb < kb_end) {
    body(kb, PipeKind<0>{});
    last_set = 0;
  }
  if (nkb > 0) {
    const int L = last_set;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[FM - 1][FN - 2][e] = fmaf(r2[e], L == 0 ? scale_of(0, FM - 1, FN - 2, e)
                                                  : scale_of(1, FM - 1, FN - 2, e),
                                    acc[FM - 1][FN - 2][e]);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[FM - 1][FN - 1][e] = fmaf(r1[e], L == 0 ? scale_of(0, FM - 1, FN - 1, e)
                                                  : scale_of(1, FM - 1, FN - 1, e),
                                    acc[FM - 1][FN - 1][e]);
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();
  int64_t ld = 0;
  if (float* dst = f32_tile_dest(a, n0, BN, split, ld)) {
    static_assert(BM * (BN + 4) * 4 <= SMEM && NW == 8, "the fp32 tile fits the dead stages");
    f32_tile_lds<BM, BN, BM>(a, smem, m0, n0, dst, ld, [&](float* tile, int pitch, int) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          *reinterpret_cast<v4f*>(tile + (wm * WM + i * 16 + (lane & 15)) * pitch + wn * WN +
                                  j * 16 + 4 * (lane >> 4)) = acc[i][j];
    });
    return;
  }
  tile_epilogue<WM, WN>(a, smem, acc, m0 + wm * WM, n0 + wn * WN, wid, lane, split);
}

// s_waitcnt vmcnt(n) for a run-time n in [0, 15].
__device__ __forceinline__ void wait_vmcnt_rt(int n) {
  switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    case 4: wait_vmcnt<4>(); break;
    case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;
    case 7: wait_vmcnt<7>(); break;
    case 8: wait_vmcnt<8>(); break;
    case 9: wait_vmcnt<9>(); break;
    case 10: wait_vmcnt<10>(); break;
    case 11: wait_vmcnt<11>(); break;
    case 12: wait_vmcnt<12>(); break;
    case 13: wait_vmcnt<13>(); break;
    case 14: wait_vmcnt<14>(); break;
    default: wait_vmcnt<15>(); break;
  }
}

// ---------------------------------------------------------------------------
// Decode GEMM (M <= 16*FM <= 64): bound by the weight stream from HBM. A
// 512-thread workgroup owns 128 weight rows (output columns n0..n0+127) and a
// K-range of kb_per_split K-blocks; grid.z splits K so that the grid fills
// the CUs about once (partials go to the workspace and splitk_reduce_kernel
// sums them in split order). Each K-block stages 128 weight rows (a wave owns 16) and
// the 16*FM activation rows once for all 8 waves, so activations cost
// 16*FM/128 of the weight bytes in L2->LDS traffic. NS LDS stages keep the
// DMA of the next K-blocks in flight; the stage of K-block kb-1 is refilled
// right after the barrier that opens K-block kb. Activation and weight-block
// scales arrive per window of 8 K-blocks by 4-byte DMA (any strides; the
// activation scales slot-major, 32 rows per slot).
// Preconditions (checked by the host, decode_offsets_ok): the 32-bit DMA
// offsets row * ldb + 127 (row <= 127) and row * lda + 127 (row < 16*FM) fit.
// ---------------------------------------------------------------------------
template <int FM, bool PR = false, int NSX = 0> struct DecodeCfg {
  static constexpr int NW = 8, BN = 128, AR = 16 * FM;
  // measured: deeper rings only lengthen the start-up burst. NSX = 3 (grids
  // above one workgroup per CU, which the planner now makes only where one
  // split less would leave 32 K-blocks per split): the smaller ring lets two
  // workgroups share a CU, so the whole grid is resident (32x28672x4096
  // split in two, 448 workgroups: 29.7 us against 33.7 with four stages).
  static constexpr int NS = NSX ? NSX : 4;
  static constexpr int STAGE = (BN + AR) * 128;
  static constexpr int ACT_LOADS = AR / 8;                 // 1 KiB wave-loads per K-block
  static constexpr int WIN_SA = 8 * 32 * 4 * ((FM + 1) / 2);
  // PR (per-row weight scales): Bs of the 128 rows, slot-major (8 x 512 B).
  static constexpr int WIN = WIN_SA + (PR ? 8 * BN * 4 : 256);
  static constexpr int SW_OFF = NS * STAGE;
  static constexpr int SMEM = SW_OFF + 2 * WIN;
};

template <int FM, bool PR = false, int NSX = 0>
__global__ void __launch_bounds__(512) gemm_decode_kernel(GemmArgs a) {
  using Cfg = DecodeCfg<FM, PR, NSX>;
  constexpr int NW = Cfg::NW, BN = Cfg::BN, NS = Cfg::NS;
  constexpr int STAGE = Cfg::STAGE, WIN_SA = Cfg::WIN_SA, WIN = Cfg::WIN;
  constexpr int SW_OFF = Cfg::SW_OFF, ACT_LOADS = Cfg::ACT_LOADS;
  static_assert(Cfg::SMEM <= 160 * 1024, "LDS budget");
  static_assert(Cfg::AR * 132 * 4 <= Cfg::SMEM, "the partial tile fits the dead stages");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::SMEM];

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * BN;
  const int split = blockIdx.z;
  const int kb_begin = split * a.kb_per_split;
  const int kb_end = min(kb_begin + a.kb_per_split, a.KB);
  const int nkb = kb_end - kb_begin;

  const uint32_t lds0 = lds_u32(smem);
  const int r8 = lane >> 3;
  const int c16 = ((lane & 7) ^ r8) * 16;
  const uint8_t* b_base = a.B + (int64_t)n0 * a.ldb;
  const int b_lim = a.N - 1 - n0, a_lim = a.M - 1;
  // Activation wave-loads of this wave per K-block (waves w, w+8, ...).
  const int act_loads = (ACT_LOADS - wid + NW - 1) / NW;
  // Wave w stages weight rows 16w..16w+15 (wave-loads 2w and 2w+1 of the
  // stage) and activation wave-loads w, w+8, ...: rows 8L..8L+7, eight lanes
  // per 128-byte row, chunk-swizzled.
  auto issue_kb = [&](int kb) {
    const int stage = (kb - kb_begin) % NS;
    const uint32_t lds = lds0 + stage * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = (wid * 2 + h) * 8 + r8;
      const uint32_t voff = (uint32_t)min(r, b_lim) * (uint32_t)a.ldb + c16;
      dma16_soff(voff, b_base + (int64_t)kb * 128, lds + (wid * 2 + h) * 1024);
    }
    for (int L = wid; L < ACT_LOADS; L += NW) {
      const uint32_t voff = (uint32_t)min(L * 8 + r8, a_lim) * (uint32_t)a.lda + c16;
      dma16_soff(voff, a.A + (int64_t)kb * 128, lds + (16 + L) * 1024);
    }
  };
  // Window from kb0: instruction j (wave j) brings slots 2j, 2j+1 for 32
  // activation rows (lane i: row i & 31, slot 2j + (i >> 5)); waves 4..7 do
  // rows 32..63 when FM = 3. The last wave brings the 8 weight-block scales.
  // K-blocks past kb_end repeat kb_end - 1.
  auto issue_win = [&](int kb0) {
    const int wbuf = ((kb0 - kb_begin) >> 3) & 1;
    const uint32_t lb = lds0 + SW_OFF + wbuf * WIN;
    constexpr int SA_INS = 4 * ((FM + 1) / 2);
    if (wid < SA_INS) {
      const int j = wid & 3, rb = (wid >> 2) * 32;
      const int kb = min(kb0 + 2 * j + (lane >> 5), kb_end - 1);
      const int m = min(rb + (lane & 31), a_lim);
      dma4_ptr(a.As + (int64_t)m * a.as_sm + (int64_t)kb * a.as_sk, lb + wid * 256);
    }
    if constexpr (PR) {
      // wave w: slot w for rows 0..63 and 64..127 (lane = row)
      const int kb = min(kb0 + wid, kb_end - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int n = min(n0 + h * 64 + lane, a.N - 1);
        dma4_ptr(a.Bs + (int64_t)n * a.bs_sn + (int64_t)kb * a.bs_sk,
                 lb + WIN_SA + wid * 512 + h * 256);
      }
    } else {
      if (wid == NW - 1 && lane < 8) {
        const int kb = min(kb0 + lane, kb_end - 1);
        dma4_ptr(a.Bs + (int64_t)(n0 >> 7) * a.bs_sn + (int64_t)kb * a.bs_sk, lb + WIN_SA);
      }
    }
  };
  auto issue_next = [&](int kb) {
    if (((kb - kb_begin) & 7) == 0) issue_win(kb);
    issue_kb(kb);
  };
  // Waits until this wave's DMA of a K-block has landed, given how many
  // K-blocks' DMAs it issued after that one (window instructions in between
  // only make the wait stricter).
  const int per_kb = 2 + act_loads;
  auto wait_after = [&](int n_after) { wait_vmcnt_rt(min(n_after * per_kb, 15)); };

  // Fragment offsets: this wave's 16 weight rows and the activation rows.
  const int r7 = lane & 7, g2 = 2 * (lane >> 4);
  const int slo = (g2 ^ r7) << 4, shi = ((g2 + 1) ^ r7) << 4;
  const int w_off = (wid * 16 + (lane & 15)) * 128;
  const int x_off = (BN + (lane & 15)) * 128;

  v4f acc[FM];
#pragma unroll
  for (int f = 0; f < FM; ++f) acc[f] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int k = 0; k < NS - 1 && k < nkb; ++k) issue_next(kb_begin + k);

  for (int kb = kb_begin; kb < kb_end; ++kb) {
    const int rel = kb - kb_begin;
    // DMAs issued after K-block kb's: those of kb+1..kb+NS-2 that exist
    wait_after(min(NS - 2, kb_end - 1 - kb));
    __syncthreads();
    if (kb + NS - 1 < kb_end) issue_next(kb + NS - 1);
    const uint8_t* st = smem + (rel % NS) * STAGE;
    const uint8_t* win = smem + SW_OFF + ((rel >> 3) & 1) * WIN;
    const int slot = rel & 7;
    v4f sbv;
    if constexpr (PR) {
      sbv = *reinterpret_cast<const v4f*>(win + WIN_SA + slot * 512 +
                                          (wid * 16 + 4 * (lane >> 4)) * 4);
    } else {
      const float sb = *reinterpret_cast<const float*>(win + WIN_SA + slot * 4);
      sbv = v4f{sb, sb, sb, sb};
    }
    const v8i w = lds_frag2(st + w_off, slo, shi);
#pragma unroll
    for (int f = 0; f < FM; ++f) {
      const int m = f * 16 + (lane & 15);
      const v8i x = lds_frag2(st + x_off + f * 2048, slo, shi);
      const float sa =
          *reinterpret_cast<const float*>(win + (m >> 5) * 1024 + slot * 128 + (m & 31) * 4);
      const v4f t = mfma16x16x128(w, x);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[f][r] = fmaf(t[r], sa * sbv[r], acc[f][r]);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  int64_t ld = 0;
  if (float* dst = f32_tile_dest(a, n0, BN, split, ld)) {
    f32_tile_lds<Cfg::AR, BN, Cfg::AR>(a, smem, 0, n0, dst, ld, [&](float* tile, int pitch, int) {
#pragma unroll
      for (int f = 0; f < FM; ++f)
        *reinterpret_cast<v4f*>(tile + (f * 16 + (lane & 15)) * pitch + wid * 16 +
                                4 * (lane >> 4)) = acc[f];
    });
    return;
  }
  const bool to_ws = gridDim.z > 1;
#pragma unroll
  for (int f = 0; f < FM; ++f)
    store4(a, f * 16 + (lane & 15), n0 + wid * 16 + 4 * (lane >> 4), acc[f], to_ws, split);
}

// ---------------------------------------------------------------------------
// One lane's share of quantising bf16 rows inside a GEMM kernel: row qm of
// the rows at `src` (256 bytes each, unswizzled), values QE*qsub..+QE-1
// (quant_load), then the act-quant's arithmetic over the 128/QE lanes of the
// row's group (a DPP row, half-row or quad: quant_row16_8, quant_row8_16,
// quant_row4_32) with the codes to row qm of `frag` in the MFMA fragment
// layout (128 bytes per row, 16-byte chunk c at slot c ^ (row & 7)) and the
// group scale to scales[qm] by the row's first lane (quant_codes). Every
// lane of the group must call quant_codes.
template <int QE> struct QuantRaw {
  static_assert(QE == 8 || QE == 16 || QE == 32, "8, 16 or 32 values per lane");
  v4i r[QE / 8];
};

template <int QE>
__device__ __forceinline__ QuantRaw<QE> quant_load(const uint8_t* src, int qm, int qsub) {
  QuantRaw<QE> raw;
#pragma unroll
  for (int i = 0; i < QE / 8; ++i)
    raw.r[i] = *reinterpret_cast<const v4i*>(src + qm * 256 + qsub * (QE * 2) + i * 16);
  return raw;
}

template <int QE>
__device__ __forceinline__ void quant_codes(const QuantRaw<QE>& raw, int qm, int qsub,
                                            uint8_t* frag, float* scales) {
  float v[QE];
  uint32_t mag = 0;
#pragma unroll
  for (int i = 0; i < QE / 8; ++i) mag = max(mag, unpack_bf16x8(raw.r[i], v + 8 * i));
  float scale;
  uint8_t* row = frag + qm * 128;
  if constexpr (QE == 8) {
    uint32_t w0, w1;
    quant_row16_8(v, mag, w0, w1, scale);
    v2i packed;
    packed[0] = (int)w0;
    packed[1] = (int)w1;
    *reinterpret_cast<v2i*>(row + (((qsub >> 1) ^ (qm & 7)) << 4) + (qsub & 1) * 8) = packed;
  } else if constexpr (QE == 16) {
    uint32_t w[4];
    quant_row8_16(v, mag, w, scale);
    v4i packed;
    for (int i = 0; i < 4; ++i) packed[i] = (int)w[i];
    *reinterpret_cast<v4i*>(row + ((qsub ^ (qm & 7)) << 4)) = packed;
  } else {
    uint32_t w[8];
    quant_row4_32(v, mag, w, scale);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i packed;
      for (int i = 0; i < 4; ++i) packed[i] = (int)w[4 * h + i];
      *reinterpret_cast<v4i*>(row + (((2 * qsub + h) ^ (qm & 7)) << 4)) = packed;
    }
  }
  if (qsub == 0) scales[qm] = scale;
}

// ---------------------------------------------------------------------------
// Decode GEMM with the group-128 act-quant inside it (fp8b_act_quant_matmul
// on decode plans, M <= 32): gemm_decode_kernel's grid, K split and fold,
// with the activations read as bf16. The waves split the work: waves 0-3
// run the MFMAs of 32 weight rows each, waves 4-7 quantise activation rows,
// and every wave DMAs exactly the bytes it consumes, so it waits on its own
// vmcnt only. Stage j of the LDS ring holds weight K-block j (128 rows,
// chunk-swizzled as in gemm_decode_kernel; MFMA wave w brings rows
// 32w..32w+31) and the bf16 rows of activation K-block j + 1 (16*FM rows of
// 256 bytes, unswizzled; quantiser wave q brings the rows it quantises); the
// rows of the split's first K-block arrive ahead of the ring, in the
// activation area of the last stage, which the ring first refills after
// they are read. A quantiser wave keeps the next K-block's rows in
// registers (read as soon as its own DMA of them has landed), quantises
// them with the act-quant's own arithmetic (QE values per lane, one DPP row
// or half-row per 128-value group: quant_row16_8 / quant_row8_16) into a
// double-buffered fp8 slab in the MFMA fragment layout, and writes the group
// scales beside it; the one barrier per K-block publishes the slab to the
// MFMA waves and frees the other buffer. The quantiser's VALU work (every
// column tile repeats it for the same rows) so runs beside the MFMA chain,
// and no global read is a compiler-generated load whose wait would drain
// the weight ring. Codes, scales, split and fold order equal act-quant
// followed by gemm_decode_kernel, so the results are bit-identical to that
// two-kernel path.
// Preconditions (checked by the host): x 16-byte aligned with a row stride
// (a.lda, in bytes) that is a multiple of 16, and the 32-bit DMA offsets
// row * ldb + 127 (row <= 127) and row * a.lda + 255 (row < 16*FM) fit.
// ---------------------------------------------------------------------------
template <int FM, int NSX, int QE> struct DecodeQuantCfg {
  static constexpr int BN = 128, AR = 16 * FM;
  static constexpr int NS = NSX;
  static constexpr int LPR = 128 / QE;                // quantiser lanes per row
  static constexpr int QROWS = 64 / LPR;              // rows per quantiser wave
  static constexpr int QLOADS = QROWS / 4;            // its 1 KiB bf16 wave-loads per stage
  static constexpr int XB = BN * 128;                 // bf16 rows within a stage
  static constexpr int STAGE = XB + AR * 256;
  static constexpr int Q_OFF = NS * STAGE;            // fp8 slabs, 2 x AR x 128 B
  static constexpr int S_OFF = Q_OFF + 2 * AR * 128;  // group scales, 2 x AR floats
  static constexpr int W_OFF = S_OFF + 2 * AR * 4;    // weight-block scale windows, 2 x 8
  static constexpr int SMEM = W_OFF + 2 * 256;
};

template <int FM, int NSX, int QE>
__global__ void __launch_bounds__(512) gemm_decode_quant_kernel(GemmArgs a) {
  using Cfg = DecodeQuantCfg<FM, NSX, QE>;
  constexpr int BN = Cfg::BN, NS = Cfg::NS, AR = Cfg::AR, LPR = Cfg::LPR;
  constexpr int QROWS = Cfg::QROWS, QLOADS = Cfg::QLOADS;
  constexpr int STAGE = Cfg::STAGE, XB = Cfg::XB;
  constexpr int Q_OFF = Cfg::Q_OFF, S_OFF = Cfg::S_OFF, W_OFF = Cfg::W_OFF;
  static_assert(QE == 8 || QE == 16, "8 or 16 values per lane");
  static_assert(4 * QROWS == AR && QLOADS >= 1, "four quantiser waves cover the rows");
  static_assert(NS >= 2 && Cfg::SMEM <= 160 * 1024, "LDS budget");
  static_assert(AR * 132 * 4 <= Cfg::SMEM, "the partial tile fits the dead stages");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::SMEM];

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool mfma_wave = wid < 4;
  const int n0 = blockIdx.x * BN;
  const int split = blockIdx.z;
  const int kb_begin = split * a.kb_per_split;
  const int kb_end = min(kb_begin + a.kb_per_split, a.KB);
  const int nkb = kb_end - kb_begin;
  const int pro = min(NS - 1, nkb);

  const uint32_t lds0 = lds_u32(smem);
  // Quantiser wave q = wid - 4: rows QROWS*q .. +QROWS-1; lane -> row
  // QROWS*q + lane/LPR, values QE*(lane%LPR) .. +QE-1.
  const int q = wid - 4;
  const int qm = q * QROWS + lane / LPR, qsub = lane % LPR;
  // bf16 rows of K-block kb into the activation area at lds (this
  // quantiser wave's QLOADS wave-loads: rows 4L..4L+3, sixteen lanes per
  // 256-byte row).
  auto issue_rows = [&](int kb, uint32_t lds) {
#pragma unroll
    for (int i = 0; i < QLOADS; ++i) {
      const int L = q * QLOADS + i;
      const uint32_t voff =
          (uint32_t)min(L * 4 + (lane >> 4), a.M - 1) * (uint32_t)a.lda + (lane & 15) * 16;
      dma16_soff(voff, a.A + (int64_t)kb * 256, lds + L * 1024);
    }
  };
  // MFMA wave w: weight rows 32w..32w+31 of K-block kb (four wave-loads of
  // eight lanes per 128-byte row, chunk-swizzled); wave 0 also brings the
  // weight-block scales of K-blocks kb..kb+7 at a window start.
  const int r8 = lane >> 3;
  const int c16 = ((lane & 7) ^ r8) * 16;
  const uint8_t* b_base = a.B + (int64_t)n0 * a.ldb;
  const int b_lim = a.N - 1 - n0;
  auto issue_weights = [&](int kb) {
    const int rel = kb - kb_begin;
    if (wid == 0 && (rel & 7) == 0 && lane < 8) {
      const int kbs = min(kb + lane, kb_end - 1);
      dma4_ptr(a.Bs + (int64_t)(n0 >> 7) * a.bs_sn + (int64_t)kbs * a.bs_sk,
               lds0 + W_OFF + ((rel >> 3) & 1) * 256);
    }
    const uint32_t lds = lds0 + (rel % NS) * STAGE;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int r = (wid * 4 + h) * 8 + r8;
      const uint32_t voff = (uint32_t)min(r, b_lim) * (uint32_t)a.ldb + c16;
      dma16_soff(voff, b_base + (int64_t)kb * 128, lds + (wid * 4 + h) * 1024);
    }
  };
  // Stage of K-block kb, this wave's part: weights, or the rows of K-block
  // kb + 1 (the last K-block's own again at the end of the split, unused).
  auto issue_stage = [&](int kb) {
    if (mfma_wave) issue_weights(kb);
    else issue_rows(min(kb + 1, kb_end - 1), lds0 + ((kb - kb_begin) % NS) * STAGE + XB);
  };
  const int per_kb = mfma_wave ? 4 : QLOADS;
  auto wait_after = [&](int n_after) { wait_vmcnt_rt(min(n_after * per_kb, 15)); };

  // Quantiser: this lane's bf16 values of a row (read from LDS into
  // registers), and their codes into slab `buf` with the group scale beside
  // it.
  QuantRaw<QE> raw;
  auto read_rows = [&](const uint8_t* src) { raw = quant_load<QE>(src, qm, qsub); };
  auto quantise = [&](int buf) {
    quant_codes<QE>(raw, qm, qsub, smem + Q_OFF + buf * (AR * 128),
                    reinterpret_cast<float*>(smem + S_OFF + buf * (AR * 4)));
  };

  // MFMA waves: fragment offsets of weight rows 32w + 16j + (lane & 15) and
  // of the activation rows.
  const int r7 = lane & 7, g2 = 2 * (lane >> 4);
  const int slo = (g2 ^ r7) << 4, shi = ((g2 + 1) ^ r7) << 4;
  const int w_off = (wid * 32 + (lane & 15)) * 128;
  const int x_off = (lane & 15) * 128;
  v4f acc[2][FM];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int f = 0; f < FM; ++f) acc[j][f] = v4f{0.f, 0.f, 0.f, 0.f};

  // Prologue. Quantiser waves: the first K-block's rows (into the last
  // stage's activation area), then their part of the ring; once the first
  // rows have landed (at most the ring's DMAs pending), quantise them into
  // slab 0 and read the next K-block's rows as soon as they land. MFMA
  // waves: their part of the ring.
  const int x0 = (NS - 1) * STAGE + XB;
  if (!mfma_wave) issue_rows(kb_begin, lds0 + x0);
  for (int k = 0; k < pro; ++k) issue_stage(kb_begin + k);
  if (!mfma_wave) {
    wait_vmcnt_rt(min(pro * per_kb, 15));
    read_rows(smem + x0);
    quantise(0);
    if (nkb > 1) {
      wait_after(pro - 1);
      read_rows(smem + XB);
    }
  }

  for (int kb = kb_begin; kb < kb_end; ++kb) {
    const int rel = kb - kb_begin;
    // MFMA waves: their weights of K-block kb (DMAs issued after them: the
    // stages of kb+1..kb+NS-2 that exist). The barrier publishes slab rel&1
    // and frees slab (rel+1)&1.
    if (mfma_wave) wait_after(min(NS - 2, kb_end - 1 - kb));
    __syncthreads();
    if (kb + NS - 1 < kb_end) issue_stage(kb + NS - 1);
    if (mfma_wave) {
      const uint8_t* st = smem + (rel % NS) * STAGE;
      const uint8_t* qs = smem + Q_OFF + (rel & 1) * (AR * 128);
      const float* ss = reinterpret_cast<const float*>(smem + S_OFF + (rel & 1) * (AR * 4));
      const float sb =
          *reinterpret_cast<const float*>(smem + W_OFF + ((rel >> 3) & 1) * 256 + (rel & 7) * 4);
      const v8i w0 = lds_frag2(st + w_off, slo, shi);
      const v8i w1 = lds_frag2(st + w_off + 2048, slo, shi);
#pragma unroll
      for (int f = 0; f < FM; ++f) {
        const v8i x = lds_frag2(qs + x_off + f * 2048, slo, shi);
        const float sab = ss[f * 16 + (lane & 15)] * sb;
        const v4f t0 = mfma16x16x128(w0, x);
        const v4f t1 = mfma16x16x128(w1, x);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          acc[0][f][r] = fmaf(t0[r], sab, acc[0][f][r]);
          acc[1][f][r] = fmaf(t1[r], sab, acc[1][f][r]);
        }
      }
    } else if (kb + 1 < kb_end) {
      // rows of K-block kb+1 (in registers) -> slab (rel+1)&1; then the
      // rows of kb+2 from stage rel+1 once this wave's DMA of them has
      // landed (DMAs issued after it: the stages of kb+2..kb+NS-1 that exist)
      quantise((rel + 1) & 1);
      if (kb + 2 < kb_end) {
        wait_after(min(NS - 2, kb_end - kb - 2));
        read_rows(smem + ((rel + 1) % NS) * STAGE + XB);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  int64_t ld = 0;
  if (float* dst = f32_tile_dest(a, n0, BN, split, ld)) {
    f32_tile_lds<AR, BN, AR>(a, smem, 0, n0, dst, ld, [&](float* tile, int pitch, int) {
      if (!mfma_wave) return;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int f = 0; f < FM; ++f)
          *reinterpret_cast<v4f*>(tile + (f * 16 + (lane & 15)) * pitch + wid * 32 + j * 16 +
                                  4 * (lane >> 4)) = acc[j][f];
    });
    return;
  }
  if (mfma_wave) {
    const bool to_ws = gridDim.z > 1;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int f = 0; f < FM; ++f)
        store4(a, f * 16 + (lane & 15), n0 + wid * 32 + j * 16 + 4 * (lane >> 4), acc[j][f],
               to_ws, split);
  }
}

// Skinny GEMM (M <= 16*FM <= 48, the decode shapes): bandwidth-bound on the
// weight stream. A 512-thread workgroup owns 16 weight rows (output columns
// n0..n0+15) over the whole K; its 8 waves split the K-blocks into
// contiguous ranges. Each wave streams its K-blocks through a private ring
// of SK LDS slots filled by global_load_lds only (weight rows, activation
// rows and their scales), so the only waits in the loop are explicit vmcnt
// waits on this ring. Rows are staged eight lanes per 128-byte row (whole
// cache lines per request) with the chunk swizzle of the tiled kernel. Each
// K-block is one 16x16x128 MFMA per 16 activation rows (weights as the A
// operand: the weight scale is wave-uniform and the activation scale is one
// register per lane). The 8 partial tiles are summed in wave order through
// LDS: deterministic, no workspace, no second kernel.
// Only the first 8*XG activation rows (XG = ceil(M/8) groups of 8) are
// staged: lanes of the MFMA operand past them read a staged row with the
// same swizzle key, and their outputs (rows >= M) are never stored. Each
// DMA instruction that is not issued saves the L2 -> LDS traffic of 1 KiB
// per K-block and wave (1x4096x14336: 2 KiB of activation rows per K-block
// cost as much time as the 2 KiB of weights beside them).
template <int FM, int XG>
__global__ void __launch_bounds__(512) gemm_skinny_kernel(GemmArgs a) {
  static_assert(XG >= 1 && XG <= 2 * FM, "staged activation row groups");
  constexpr int NWAVE = 8;
  constexpr int SK = FM <= 2 ? 3 : 2;          // K-blocks in flight per wave
  constexpr int ROWS = 16 + 8 * XG;            // weight rows, then staged activation rows
  constexpr int LOADS = ROWS / 8;              // 1 KiB DMA instructions per K-block
  constexpr int SCALE_OFF = ROWS * 128;        // 64 fp32: sa rows 0..16FM-1, sb at 63
  constexpr int SLOT = SCALE_OFF + 256;
  constexpr int PER_KB = LOADS + 1;            // DMA instructions per K-block
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NWAVE][SK][SLOT];
  const int lane = threadIdx.x & 63;
  // Wave index as a scalar, so K ranges and loop conditions are uniform.
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16;
  const int kb0 = (int)((int64_t)a.KB * wid / NWAVE);
  const int kb1 = (int)((int64_t)a.KB * (wid + 1) / NWAVE);
  const int row = lane & 15;

  // DMA sources: load L brings staged rows 8L..8L+7 (0..15 weights, then
  // activations), lane i the logical chunk (i&7) ^ (r&7) of row 8L + (i>>3).
  const uint8_t* src[LOADS];
#pragma unroll
  for (int L = 0; L < LOADS; ++L) {
    const int r = L * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ (r & 7);
    src[L] = r < 16 ? a.B + (int64_t)min(n0 + r, a.N - 1) * a.ldb + chunk * 16
                    : a.A + (int64_t)min(r - 16, a.M - 1) * a.lda + chunk * 16;
  }
  // Scale DMA (4 bytes per lane): lanes 0..16FM-1 the activation rows' scale,
  // the remaining lanes the weight block's scale.
  const float* ssrc = lane < 16 * FM ? a.As + (int64_t)min(lane, a.M - 1) * a.as_sm
                                     : a.Bs + (int64_t)(min(n0, a.N - 1) >> 7) * a.bs_sn;
  const int64_t sstep = lane < 16 * FM ? a.as_sk : a.bs_sk;
  const int c0 = 2 * (lane >> 4);
  const int r7 = row & 7;

  auto issue = [&](int kb, int slot) {
    uint8_t* dst = &ring[wid][slot][0];
#pragma unroll
    for (int L = 0; L < LOADS; ++L) lds_dma16(src[L] + (int64_t)kb * 128, dst + L * 1024);
    lds_dma4(ssrc + (int64_t)kb * sstep, dst + SCALE_OFF);
  };

  v4f acc[FM];
#pragma unroll
  for (int f = 0; f < FM; ++f) acc[f] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int u = 0; u < SK; ++u)
    if (kb0 + u < kb1) issue(kb0 + u, u);
  for (int kb = kb0; kb < kb1; kb += SK) {
#pragma unroll
    for (int u = 0; u < SK; ++u) {
      if (kb + u < kb1) {
        // In steady state the DMAs of the next SK-1 K-blocks were issued
        // after this slot's, so allowing that many outstanding retires it;
        // near the end of the range fewer exist: wait for all.
        if (kb + u + SK - 1 < kb1) wait_vmcnt<PER_KB * (SK - 1)>();
        else wait_vmcnt<0>();
        const uint8_t* sl = &ring[wid][u][0];
        const v8i w = lds_frag(sl + row * 128, c0, r7);
        const float sb = *reinterpret_cast<const float*>(sl + SCALE_OFF + 63 * 4);
#pragma unroll
        for (int f = 0; f < FM; ++f) {
          const int xr = f * 16 + row < 8 * XG ? f * 16 + row : 8 * (XG - 1) + r7;
          const v8i x = lds_frag(sl + (16 + xr) * 128, c0, r7);
          const float sc = *reinterpret_cast<const float*>(sl + SCALE_OFF + (f * 16 + row) * 4) * sb;
          const v4f t = mfma16x16x128(w, x);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[f][r] = fmaf(t[r], sc, acc[f][r]);
        }
        // refill the slot once this wave's reads of it are complete
        if (kb + u + SK < kb1) {
          lds_reads_done();
          issue(kb + u + SK, u);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // Partial tiles reuse the ring: [wave][f][r][lane] floats.
  float* part = reinterpret_cast<float*>(&ring[0][0][0]);
#pragma unroll
  for (int f = 0; f < FM; ++f)
#pragma unroll
    for (int r = 0; r < 4; ++r) part[((wid * FM + f) * 4 + r) * 64 + lane] = acc[f][r];
  __syncthreads();
  if (wid != 0) return;
  // Wave 0 sums the 8 partial tiles in wave order and stores: lane holds
  // row m = 16f + (lane & 15) and columns n0 + 4*(lane>>4) + 0..3.
#pragma unroll
  for (int f = 0; f < FM; ++f) {
    v4f sum = {0.f, 0.f, 0.f, 0.f};
    for (int w = 0; w < NWAVE; ++w)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum[r] += part[((w * FM + f) * 4 + r) * 64 + lane];
    store4(a, f * 16 + row, n0 + 4 * (lane >> 4), sum, false, 0);
  }
}

// ---------------------------------------------------------------------------
// Skinny GEMM with the group-128 act-quant inside it (fp8b_act_quant_matmul
// on skinny plans, M <= QR <= 8): gemm_skinny_kernel<1, XG>'s grid, K ranges and
// fold, with the activations read as bf16. Each wave streams its K-blocks
// through a private ring of LDS slots (its 16 weight rows, chunk-swizzled;
// the QR bf16 activation rows, unswizzled; the weight block's scale), all by
// DMA counted by its own waits, and before each K-block's MFMA quantises
// the slot's QR rows with the act-quant's own arithmetic (one task of 2*QR
// values per lane: quant_row16_8 for 4 rows, quant_row8_16 for 8) into its
// fp8 fragment buffer and scale buffer, which its MFMA then reads (LDS
// operations of one wave complete in order). Rows QR..15 of the fragment are
// never written and never stored. Codes, scales, K ranges, fold and the sum
// of the eight partial tiles equal act-quant followed by gemm_skinny_kernel,
// so the results are bit-identical to that two-kernel path.
// Preconditions (checked by the host): M <= QR, x 16-byte aligned with a row
// stride (a.lda, in bytes) that is a multiple of 16.
// ---------------------------------------------------------------------------
template <int QR>
__global__ void __launch_bounds__(512) gemm_skinny_quant_kernel(GemmArgs a) {
  constexpr int NWAVE = 8;
  constexpr int SK = 3;                        // K-blocks in flight per wave
  constexpr int QE = 2 * QR;                   // values per lane
  constexpr int LPR = 128 / QE;                // lanes per row
  constexpr int XLOADS = QR / 4;               // 1 KiB DMA instructions of bf16 rows
  constexpr int X_OFF = 16 * 128;              // bf16 rows after the 16 weight rows
  constexpr int S_OFF = X_OFF + QR * 256;      // the weight block's scale
  constexpr int SLOT = S_OFF + 64;
  constexpr int PER_KB = 2 + XLOADS + 1;       // DMA instructions per K-block
  static_assert(QR == 4 || QR == 8, "4 or 8 activation rows");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NWAVE][SK][SLOT];
  __shared__ __attribute__((aligned(1024))) uint8_t qbuf[NWAVE][16 * 128 + 64];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16;
  const int kb0 = (int)((int64_t)a.KB * wid / NWAVE);
  const int kb1 = (int)((int64_t)a.KB * (wid + 1) / NWAVE);
  const int row = lane & 15;

  // DMA sources: weight loads L = 0, 1 bring rows 8L..8L+7 (lane i: the
  // logical chunk (i&7) ^ (r&7) of row 8L + (i>>3)); bf16 load L brings
  // activation rows 4L..4L+3 (lane i: bytes 16(i&15).. of row 4L + (i>>4)).
  const uint8_t* wsrc[2];
#pragma unroll
  for (int L = 0; L < 2; ++L) {
    const int r = L * 8 + (lane >> 3);
    wsrc[L] = a.B + (int64_t)min(n0 + r, a.N - 1) * a.ldb + ((lane & 7) ^ (r & 7)) * 16;
  }
  const uint8_t* xsrc[XLOADS];
#pragma unroll
  for (int L = 0; L < XLOADS; ++L)
    xsrc[L] = a.A + (int64_t)min(L * 4 + (lane >> 4), a.M - 1) * a.lda + (lane & 15) * 16;
  const float* bsrc = a.Bs + (int64_t)(min(n0, a.N - 1) >> 7) * a.bs_sn;
  const uint32_t ring0 = lds_u32(&ring[wid][0][0]);

  auto issue = [&](int kb, int slot) {
    const uint32_t dst = ring0 + slot * SLOT;
#pragma unroll
    for (int L = 0; L < 2; ++L) dma16_ptr(wsrc[L] + (int64_t)kb * 128, dst + L * 1024);
#pragma unroll
    for (int L = 0; L < XLOADS; ++L) dma16_ptr(xsrc[L] + (int64_t)kb * 256, dst + X_OFF + L * 1024);
    if (lane == 0) dma4_ptr(bsrc + (int64_t)kb * a.bs_sk, dst + S_OFF);
  };

  // This lane's quantiser task: row qm, values QE*qsub..+QE-1.
  const int qm = lane / LPR, qsub = lane % LPR;
  uint8_t* qb = &qbuf[wid][0];
  float* qs = reinterpret_cast<float*>(qb + 16 * 128);
  auto quantise = [&](const uint8_t* sl) {
    quant_codes<QE>(quant_load<QE>(sl + X_OFF, qm, qsub), qm, qsub, qb, qs);
  };

  const int c0 = 2 * (lane >> 4);
  const int r7 = row & 7;
  v4f acc = {0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int u = 0; u < SK; ++u)
    if (kb0 + u < kb1) issue(kb0 + u, u);
  for (int kb = kb0; kb < kb1; kb += SK) {
#pragma unroll
    for (int u = 0; u < SK; ++u) {
      if (kb + u < kb1) {
        // as in gemm_skinny_kernel: the next SK-1 K-blocks' DMAs were issued
        // after this slot's, or fewer near the end of the range
        if (kb + u + SK - 1 < kb1) wait_vmcnt<PER_KB * (SK - 1)>();
        else wait_vmcnt<0>();
        const uint8_t* sl = &ring[wid][u][0];
        quantise(sl);
        const v8i w = lds_frag(sl + row * 128, c0, r7);
        const float sb = *reinterpret_cast<const float*>(sl + S_OFF);
        const v8i x = lds_frag(qb + row * 128, c0, r7);
        const float sc = qs[row] * sb;
        const v4f t = mfma16x16x128(w, x);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(t[r], sc, acc[r]);
        // refill the slot once this wave's reads of it are complete
        if (kb + u + SK < kb1) {
          lds_reads_done();
          issue(kb + u + SK, u);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // Partial tiles reuse the ring: [wave][r][lane] floats, summed by wave 0
  // in wave order (row m = lane & 15, columns n0 + 4*(lane>>4) + 0..3).
  float* part = reinterpret_cast<float*>(&ring[0][0][0]);
#pragma unroll
  for (int r = 0; r < 4; ++r) part[(wid * 4 + r) * 64 + lane] = acc[r];
  __syncthreads();
  if (wid != 0) return;
  v4f sum = {0.f, 0.f, 0.f, 0.f};
  for (int w = 0; w < NWAVE; ++w)
#pragma unroll
    for (int r = 0; r < 4; ++r) sum[r] += part[(w * 4 + r) * 64 + lane];
  store4(a, row, n0 + 4 * (lane >> 4), sum, false, 0);
}

// Small-grid GEMM (grids of 128x128 tiles that would leave most CUs idle,
// e.g. 512x512x2048): one workgroup per TM x TN output tile (TM = 16*FM,
// TN = 16*FN: 32x32 or 64x64), so the grid spreads the operand stream over
// many more CUs than 128x128 tiles, with no workspace and no second kernel.
// Each of its NW waves takes a contiguous range of the K-blocks and streams
// the tile's TM activation and TN weight rows ((TM+TN)/8 DMA instructions of
// 1 KiB per K-block, the chunk swizzle of gemm_bs128_kernel) and their
// scales (4-byte DMA lanes: the TM activation rows' scales, then TN weight
// scales: the block's, or each weight row's with PR) through a private ring
// of NS LDS slots, so the only waits in the loop are vmcnt waits on its own
// DMA. Per K-block: FM x FN 16x16x128 MFMAs (weights as the A operand), each
// folded as acc + dot * (As * Bs), or dot * (As * Bs[n]) per output column
// with PR, as the other kernels do. With NW = 1 that is the arithmetic of
// every other unsplit plan, bit for bit; with NW > 1 the NW partial tiles
// are summed through LDS in wave order (deterministic), which keeps more
// K-blocks in flight per CU: the loop is bound by DMA latency.
template <int FM, int FN, int NW, int NS, bool PR = false>
__global__ void __launch_bounds__(64 * NW) gemm_tiny_kernel(GemmArgs a) {
  constexpr int TM = 16 * FM, TN = 16 * FN;
  constexpr int ROWS = TM + TN;               // activation rows, then weight rows
  constexpr int SCALES = TM + TN;             // sa of the TM rows, then TN weight scales
  constexpr int SDMA = (SCALES + 63) / 64;    // 4-byte DMA instructions per K-block
  constexpr int SCALE_OFF = ROWS * 128;
  constexpr int SLOT = SCALE_OFF + SDMA * 256;
  constexpr int PER_KB = ROWS / 8 + SDMA;     // DMA instructions per K-block
  static_assert(TM <= 128 && TN <= 128, "tile shape");
  // at most NS K-blocks of DMA are outstanding per wave: within the 6-bit vmcnt
  static_assert(PER_KB * NS <= 63, "vmcnt is a 6-bit counter");
  static_assert(NW == 1 || NS * SLOT >= FM * FN * 4 * 64 * 4, "partials reuse the ring");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NW][NS][SLOT];
  const int lane = threadIdx.x & 63;
  // wave index as a scalar, so K ranges and loop conditions are uniform
  const int wid = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tm, tn;
  if (a.rem_base >= 0) {
    // a quarter of one of the tiles of twice the size a launch left
    tile_of_bid(a.rem_base + (int)blockIdx.x / 4, a.rem_tiles_m, a.rem_tiles_n, tm, tn);
    tm = 2 * tm + (((int)blockIdx.x >> 1) & 1);
    tn = 2 * tn + ((int)blockIdx.x & 1);
  } else {
    tile_of_bid((int)blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  }
  const int m0 = tm * TM, n0 = tn * TN;
  if (m0 >= a.M || n0 >= a.N) return;  // a quarter past the matrix edge (whole workgroup)
  const int kb0 = (int)((int64_t)a.KB * wid / NW);
  const int kb1 = (int)((int64_t)a.KB * (wid + 1) / NW);

  // load L brings rows 8L..8L+7 of the slot; lane i the logical chunk
  // (i&7) ^ (r&7) of row 8L + (i>>3), so chunk c of row r sits in slot c^(r&7)
  const uint8_t* src[ROWS / 8];
#pragma unroll
  for (int L = 0; L < ROWS / 8; ++L) {
    const int r = L * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ (r & 7);
    src[L] = r < TM ? a.A + (int64_t)min(m0 + r, a.M - 1) * a.lda + chunk * 16
                    : a.B + (int64_t)min(n0 + r - TM, a.N - 1) * a.ldb + chunk * 16;
  }
  // scale entry e = 64 d + lane of DMA d: e < TM the activation row m0 + e,
  // else weight scale e - TM (the block's, or weight row n0 + e - TM with PR;
  // entries past TM + TN repeat a valid address and are not read)
  const float* ssrc[SDMA];
  int64_t sstep[SDMA];
#pragma unroll
  for (int d = 0; d < SDMA; ++d) {
    const int e = d * 64 + lane;
    const int64_t b_row = PR ? min(max(n0 + e - TM, 0), a.N - 1) : (min(n0, a.N - 1) >> 7);
    ssrc[d] = e < TM ? a.As + (int64_t)min(m0 + e, a.M - 1) * a.as_sm : a.Bs + b_row * a.bs_sn;
    sstep[d] = e < TM ? a.as_sk : a.bs_sk;
  }
  auto issue = [&](int kb, int slot) {
    uint8_t* dst = &ring[wid][slot][0];
#pragma unroll
    for (int L = 0; L < ROWS / 8; ++L) lds_dma16(src[L] + (int64_t)kb * 128, dst + L * 1024);
#pragma unroll
    for (int d = 0; d < SDMA; ++d)
      lds_dma4(ssrc[d] + (int64_t)kb * sstep[d], dst + SCALE_OFF + d * 256);
  };

  const int row = lane & 15, c0 = 2 * (lane >> 4), r7 = row & 7;
  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int u = 0; u < NS && kb0 + u < kb1; ++u) issue(kb0 + u, u);
  for (int kb = kb0; kb < kb1; ++kb) {
    const int slot = (kb - kb0) % NS;
    // the DMAs of the next NS-1 K-blocks were issued after this slot's
    // (fewer near the end of the range: then wait for all)
    if (kb + NS - 1 < kb1) wait_vmcnt<PER_KB * (NS - 1)>();
    else wait_vmcnt<0>();
    const uint8_t* sl = &ring[wid][slot][0];
    const float* sv = reinterpret_cast<const float*>(sl + SCALE_OFF);
    v8i x[FM], w[FN];
#pragma unroll
    for (int f = 0; f < FM; ++f) x[f] = lds_frag(sl + (f * 16 + row) * 128, c0, r7);
#pragma unroll
    for (int f = 0; f < FN; ++f) w[f] = lds_frag(sl + (TM + f * 16 + row) * 128, c0, r7);
    if constexpr (PR) {
      // output (i, j, e): activation row 16i + row, weight row 16j + 4*(lane>>4) + e
      float sa[FM];
      v4f sbv[FN];
#pragma unroll
      for (int f = 0; f < FM; ++f) sa[f] = sv[f * 16 + row];
#pragma unroll
      for (int f = 0; f < FN; ++f)
        sbv[f] = *reinterpret_cast<const v4f*>(sv + TM + f * 16 + 4 * (lane >> 4));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const v4f t = mfma16x16x128(w[j], x[i]);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(t[e], sa[i] * sbv[j][e], acc[i][j][e]);
        }
    } else {
      const float sb = sv[TM];
      float sc[FM];
#pragma unroll
      for (int f = 0; f < FM; ++f) sc[f] = sv[f * 16 + row] * sb;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const v4f t = mfma16x16x128(w[j], x[i]);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(t[e], sc[i], acc[i][j][e]);
        }
    }
    // refill the slot once this wave's reads of it are complete
    if (kb + NS < kb1) {
      lds_reads_done();
      issue(kb + NS, slot);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if constexpr (NW == 1) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        store4(a, m0 + i * 16 + row, n0 + j * 16 + 4 * (lane >> 4), acc[i][j], false, 0);
  } else {
    // partial tiles reuse the ring: [wave][i][j][e][lane] floats; wave q
    // then sums sub-tiles q, q + NW, ... of every wave in wave order
    __syncthreads();
    float* part = reinterpret_cast<float*>(&ring[0][0][0]);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          part[(((wid * FM + i) * FN + j) * 4 + e) * 64 + lane] = acc[i][j][e];
    __syncthreads();
    for (int q = wid; q < FM * FN; q += NW) {
      const int i = q / FN, j = q % FN;
      v4f sum = {0.f, 0.f, 0.f, 0.f};
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[e] += part[(((w * FM + i) * FN + j) * 4 + e) * 64 + lane];
      store4(a, m0 + i * 16 + row, n0 + j * 16 + 4 * (lane >> 4), sum, false, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Small-grid GEMM with the group-128 act-quant inside it
// (fp8b_act_quant_matmul on small-grid plans of 32-row tiles, M <= QR <= 16):
// gemm_tiny_kernel's grid, K ranges, fold and wave-order sum for the first
// 16 rows of the tile (rows 16..31 do not exist). Each wave's
// ring slots carry its TN weight rows (chunk-swizzled), the QR bf16
// activation rows (unswizzled) and the weight block's scale, and the wave
// quantises a slot's rows (one task of 2*QR values per lane, the
// act-quant's arithmetic: quant_codes) into its own fragment and scale
// buffers right before that slot's MFMAs (LDS operations of one wave
// complete in order). Same codes, scales and sums as act-quant followed by
// gemm_tiny_kernel, so the same output bits.
// Preconditions (checked by the host): M <= QR, x 16-byte aligned with a row
// stride (a.lda, in bytes) that is a multiple of 16; a.tiles_m = 1.
// ---------------------------------------------------------------------------
template <int FN, int NW, int QR>
__global__ void __launch_bounds__(64 * NW) gemm_tiny_quant_kernel(GemmArgs a) {
  constexpr int NS = 2;
  constexpr int TN = 16 * FN;
  constexpr int QE = 2 * QR;                   // values per lane
  constexpr int LPR = 128 / QE;                // lanes per row
  constexpr int WLOADS = TN / 8, XLOADS = QR / 4;
  constexpr int X_OFF = TN * 128;              // bf16 rows after the weight rows
  constexpr int S_OFF = X_OFF + QR * 256;      // the weight block's scale
  constexpr int SLOT = S_OFF + 64;
  constexpr int PER_KB = WLOADS + XLOADS + 1;  // DMA instructions per K-block
  static_assert(QR == 4 || QR == 8 || QR == 16, "4, 8 or 16 activation rows");
  static_assert(NW == 1 || NS * SLOT >= FN * 4 * 64 * 4, "partials reuse the ring");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NW][NS][SLOT];
  __shared__ __attribute__((aligned(1024))) uint8_t qbuf[NW][16 * 128 + 64];
  const int lane = threadIdx.x & 63;
  const int wid = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tm, tn;
  tile_of_bid((int)blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int n0 = tn * TN;
  if (n0 >= a.N) return;
  const int kb0 = (int)((int64_t)a.KB * wid / NW);
  const int kb1 = (int)((int64_t)a.KB * (wid + 1) / NW);

  const uint8_t* wsrc[WLOADS];
#pragma unroll
  for (int L = 0; L < WLOADS; ++L) {
    const int r = L * 8 + (lane >> 3);
    wsrc[L] = a.B + (int64_t)min(n0 + r, a.N - 1) * a.ldb + ((lane & 7) ^ (r & 7)) * 16;
  }
  const uint8_t* xsrc[XLOADS];
#pragma unroll
  for (int L = 0; L < XLOADS; ++L)
    xsrc[L] = a.A + (int64_t)min(L * 4 + (lane >> 4), a.M - 1) * a.lda + (lane & 15) * 16;
  const float* bsrc = a.Bs + (int64_t)(min(n0, a.N - 1) >> 7) * a.bs_sn;
  const uint32_t ring0 = lds_u32(&ring[wid][0][0]);
  auto issue = [&](int kb, int slot) {
    const uint32_t dst = ring0 + slot * SLOT;
#pragma unroll
    for (int L = 0; L < WLOADS; ++L) dma16_ptr(wsrc[L] + (int64_t)kb * 128, dst + L * 1024);
#pragma unroll
    for (int L = 0; L < XLOADS; ++L) dma16_ptr(xsrc[L] + (int64_t)kb * 256, dst + X_OFF + L * 1024);
    if (lane == 0) dma4_ptr(bsrc + (int64_t)kb * a.bs_sk, dst + S_OFF);
  };

  const int qm = lane / LPR, qsub = lane % LPR;
  uint8_t* qb = &qbuf[wid][0];
  float* qs = reinterpret_cast<float*>(qb + 16 * 128);
  auto quantise = [&](const uint8_t* sl) {
    quant_codes<QE>(quant_load<QE>(sl + X_OFF, qm, qsub), qm, qsub, qb, qs);
  };

  const int row = lane & 15, c0 = 2 * (lane >> 4), r7 = row & 7;
  v4f acc[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int u = 0; u < NS && kb0 + u < kb1; ++u) issue(kb0 + u, u);
  for (int kb = kb0; kb < kb1; ++kb) {
    const int slot = (kb - kb0) % NS;
    // as in gemm_tiny_kernel: the next NS-1 K-blocks' DMAs were issued after
    // this slot's, or fewer near the end of the range
    if (kb + NS - 1 < kb1) wait_vmcnt<PER_KB * (NS - 1)>();
    else wait_vmcnt<0>();
    const uint8_t* sl = &ring[wid][slot][0];
    quantise(sl);
    const v8i x = lds_frag(qb + row * 128, c0, r7);
    const float sc = qs[row] * *reinterpret_cast<const float*>(sl + S_OFF);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const v8i w = lds_frag(sl + (j * 16 + row) * 128, c0, r7);
      const v4f t = mfma16x16x128(w, x);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[j][e] = fmaf(t[e], sc, acc[j][e]);
    }
    // refill the slot once this wave's reads of it are complete
    if (kb + NS < kb1) {
      lds_reads_done();
      issue(kb + NS, slot);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if constexpr (NW == 1) {
#pragma unroll
    for (int j = 0; j < FN; ++j) store4(a, row, n0 + j * 16 + 4 * (lane >> 4), acc[j], false, 0);
  } else {
    // partial tiles reuse the ring: [wave][j][e][lane] floats; wave q sums
    // sub-tiles q, q + NW, ... of every wave in wave order
    __syncthreads();
    float* part = reinterpret_cast<float*>(&ring[0][0][0]);
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) part[((wid * FN + j) * 4 + e) * 64 + lane] = acc[j][e];
    __syncthreads();
    for (int j = wid; j < FN; j += NW) {
      v4f sum = {0.f, 0.f, 0.f, 0.f};
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[e] += part[((w * FN + j) * 4 + e) * 64 + lane];
      store4(a, row, n0 + j * 16 + 4 * (lane >> 4), sum, false, 0);
    }
  }
}

// Sum split-K partials in split order and convert: 4 outputs per thread. The
// partial loads go out eight splits at a time before any is added, so the
// kernel costs about one memory latency per eight splits.
__global__ void __launch_bounds__(256)
splitk_reduce_kernel(GemmArgs a, int splits) {
  const int64_t quads_per_row = (a.N + 3) / 4;
  const int64_t qi = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (qi >= (int64_t)a.M * quads_per_row) return;
  const int m = (int)(qi / quads_per_row);
  const int n = (int)(qi - (int64_t)m * quads_per_row) * 4;
  v4f s = {0.f, 0.f, 0.f, 0.f};
  const int64_t plane = (int64_t)a.M * a.N;
  const float* p = a.ws + (int64_t)m * a.N + n;
  const bool vec = n + 3 < a.N && a.vec_store;
  for (int z0 = 0; z0 < splits; z0 += 8) {
    v4f v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int z = z0 + u;
      if (z < splits) {
        if (vec) {
          v[u] = *reinterpret_cast<const v4f*>(p + z * plane);
        } else {
          for (int r = 0; r < 4; ++r) v[u][r] = (n + r < a.N) ? p[z * plane + r] : 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (z0 + u < splits) s += v[u];
  }
  store4(a, m, n, s, false, 0);
}

// The same sum for the decode grids whose column-tile count is a multiple of
// 8: workgroup (x, z) of the decode grid runs on XCD x % 8 for every split z
// (workgroups go round-robin over the 8 XCDs), so the partials of column
// tile x sit in that XCD's L2. Block b here runs on XCD b % 8 and sums 8
// rows of a column tile of that XCD: tile x = b % 8 + 8 * ((b / 8) %
// (tiles_n / 8)), rows 8 * (b / tiles_n) ..; thread t takes row + t / 32,
// columns 4 * (t % 32) .. of the tile. Placement only changes where the
// loads hit; the sum and its order are splitk_reduce_kernel's.
__global__ void __launch_bounds__(256)
splitk_reduce_xcd_kernel(GemmArgs a, int splits) {
  const int b = (int)blockIdx.x;
  const int x = (b & 7) + 8 * ((b >> 3) % (a.tiles_n >> 3));
  const int m = 8 * (b / a.tiles_n) + (int)(threadIdx.x >> 5);
  const int n = x * 128 + 4 * (int)(threadIdx.x & 31);
  if (m >= a.M || n >= a.N) return;
  v4f s = {0.f, 0.f, 0.f, 0.f};
  const int64_t plane = (int64_t)a.M * a.N;
  const float* p = a.ws + (int64_t)m * a.N + n;
  const bool vec = n + 3 < a.N && a.vec_store;
  for (int z0 = 0; z0 < splits; z0 += 8) {
    v4f v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int z = z0 + u;
      if (z < splits) {
        if (vec) {
          v[u] = *reinterpret_cast<const v4f*>(p + z * plane);
        } else {
          for (int r = 0; r < 4; ++r) v[u][r] = (n + r < a.N) ? p[z * plane + r] : 0.f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (z0 + u < splits) s += v[u];
  }
  store4(a, m, n, s, false, 0);
}

// Generic SIMT kernel: 32x32 outputs per 256-thread block, 2x2 per thread.
// For each K-block: part = sum_k A*B over the block (fp32 FMA chain in k
// order), then acc += part * As * Bs, as in fp8.py:31-37.
struct GenericArgs {
  const uint8_t* A;
  const uint8_t* B;
  const float* As;
  const float* Bs;
  void* C;
  int64_t lda, ldb, as_sm, as_sk, bs_sn, bs_sk, ldc;
  int64_t M, N, K, block_n, block_k;
  int out_dtype;
};

__global__ void __launch_bounds__(256) gemm_generic_kernel(GenericArgs g) {
  __shared__ float sA[32][33];
  __shared__ float sB[32][33];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t mb = (int64_t)blockIdx.y * 32, nbase = (int64_t)blockIdx.x * 32;
  float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  const int64_t KB = (g.K + g.block_k - 1) / g.block_k;
  for (int64_t kb = 0; kb < KB; ++kb) {
    float part[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
    const int64_t kbeg = kb * g.block_k, kend = min(kbeg + g.block_k, g.K);
    for (int64_t k0 = kbeg; k0 < kend; k0 += 32) {
      for (int e = threadIdx.x; e < 32 * 32; e += 256) {
        const int r = e >> 5, c = e & 31;
        const int64_t k = k0 + c;
        const int64_t m = mb + r, n = nbase + r;
        sA[r][c] = (m < g.M && k < kend) ? fp8e4m3_to_f32(g.A[m * g.lda + k]) : 0.f;
        sB[r][c] = (n < g.N && k < kend) ? fp8e4m3_to_f32(g.B[n * g.ldb + k]) : 0.f;
      }
      __syncthreads();
      for (int c = 0; c < 32; ++c) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            part[i][j] = fmaf(sA[ty * 2 + i][c], sB[tx * 2 + j][c], part[i][j]);
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t m = min(mb + ty * 2 + i, g.M - 1);
      const float sa = g.As[m * g.as_sm + kb * g.as_sk];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t n = min(nbase + tx * 2 + j, g.N - 1);
        const float sb = g.Bs[(n / g.block_n) * g.bs_sn + kb * g.bs_sk];
        acc[i][j] = acc[i][j] + part[i][j] * sa * sb;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t m = mb + ty * 2 + i;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = nbase + tx * 2 + j;
      if (n >= g.N) continue;
      const float v = acc[i][j];
      if (g.out_dtype == FP8B_F32) {
        reinterpret_cast<float*>(g.C)[m * g.ldc + n] = v;
      } else if (g.out_dtype == FP8B_BF16) {
        reinterpret_cast<uint16_t*>(g.C)[m * g.ldc + n] = f32_to_bf16_bits(v);
      } else {
        _Float16 h = (_Float16)v;
        reinterpret_cast<uint16_t*>(g.C)[m * g.ldc + n] = __builtin_bit_cast(uint16_t, h);
      }
    }
  }
}

}  // namespace fp8b

using namespace fp8b;

namespace {

// Tile configurations of the MFMA path.
enum TileCfg {
  CFG_256x256 = 0,
  CFG_192x256 = 1,
  CFG_128x128 = 2,
  CFG_SKINNY = 3,
  CFG_DECODE = 4,
  CFG_TINY = 5,
  CFG_256x128 = 6,
  CFG_COUNT
};

// What runs the last partial wave of an unsplit grid.
enum TailKind {
  TAIL_NONE = 0,
  TAIL_Q128 = 1,      // 256x256 tiles: as 128x128 quarters on gemm_pipe128_kernel
  TAIL_H256X128 = 2,  // 256x256 tiles: as 256x128 halves on gemm_pipe256x128_kernel
  TAIL_Q64 = 3        // 128x128 tiles: as 64x64 quarters on gemm_tiny_kernel
};

struct Plan {
  int cfg;
  int bm, bn;
  int splits;
  int kb_per_split;
  int tail;
};

// CU count of the current device, queried once per device.
int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 256;
  if (dev >= 0 && dev < 64) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Environment switches for A/B measurements, read once per process:
//   FP8B_DECODE=0   M <= 48 always takes the skinny kernel (no split-K
//                   decode kernel; per-row scales then take the 128x128 path);
//   FP8B_PIPE=0     no pipelined kernels (gemm_bs128_kernel instead);
//   FP8B_TAIL128=0  no 128x128 quarters for a small last wave of 256x256 tiles;
//   FP8B_TILE192=0  no 192x256 tiles;
//   FP8B_TINY=0     no small-grid kernel (32x32, 32x16, 64x64 tiles);
//   FP8B_TAIL64=0   no 64x64 quarters for a small last wave of 128x128 tiles;
//   FP8B_TILE256X128=0  no 256x128 tiles;
//   FP8B_FUSED_DECODE=0 fp8b_act_quant_matmul runs act-quant and the GEMM as
//                   two kernels on decode, skinny and small-grid plans too;
//   FP8B_TINY16=0   M <= 16 small grids run the 32-row tiles whole;
//   FP8B_REDUCE_XCD=0  split-K sums of decode grids in row order.
bool env_flag_on(const char* name) {
  const char* e = getenv(name);
  return !(e && e[0] == '0');
}
bool use_decode_kernel() {
  static const bool v = env_flag_on("FP8B_DECODE");
  return v;
}
bool use_pipelined_kernels() {
  static const bool v = env_flag_on("FP8B_PIPE");
  return v;
}
bool use_tail128() {
  static const bool v = env_flag_on("FP8B_TAIL128");
  return v;
}
bool use_tile192() {
  static const bool v = env_flag_on("FP8B_TILE192");
  return v;
}
bool use_tiny() {
  static const bool v = env_flag_on("FP8B_TINY");
  return v;
}
bool use_tail64() {
  static const bool v = env_flag_on("FP8B_TAIL64");
  return v;
}
bool use_tile256x128() {
  static const bool v = env_flag_on("FP8B_TILE256X128");
  return v;
}
bool use_tiny16() {
  static const bool v = env_flag_on("FP8B_TINY16");
  return v;
}
bool use_reduce_xcd() {
  static const bool v = env_flag_on("FP8B_REDUCE_XCD");
  return v;
}
bool use_fused_decode() {
  static const bool v = env_flag_on("FP8B_FUSED_DECODE");
  return v;
}

// ---------------------------------------------------------------------------
// Cost model of the MFMA-bound plans: grids past the small-grid and decode
// ranges, where the choice is a tile shape (256x256, 192x256, 256x128 or
// 128x128), what runs a last partial wave, and how often to split K. Every
// candidate is priced as the sum over its waves of workgroups (one workgroup
// per CU for every pipelined kernel, by its LDS) of
//   first K-block latency
//   + K-blocks x time per K-block of the tile x the wave's power factor
//   + the wave's output stores,
// plus, for a K split, the fp32 partials and the split-K sum kernel; the
// cheapest wins. Time per K-block of one tile on one CU of a fully busy
// chip (MI355X, realistic operand bits, power-limited clock): 256x256
// 1.72 us, 192x256 1.37, 256x128 0.95, 128x128 0.71; 64x64 quarters on the
// small-grid kernel 0.40. A wave that keeps a fraction f of the CUs busy
// runs each tile faster, the power limit then allowing a higher clock:
// factor max(0.8, 1 - 0.8 (1 - f)) (a 192-tile wave of 256x256 tiles takes
// 1.41 us per K-block). The model reproduces the measured order of the
// plans it chooses between, e.g. (us, steady clock):
//   3001x4096x14336   192x256 one wave 157.8 < 256x256 partial wave 160.3
//                     < 128x128 three waves 241
//   3001x28672x4096   256x256 + last wave as 128x128 quarters 320.3
//                     < 192x256 seven waves 331.4
//   2048x4096x4096    256x128 one wave 34.8 < 128x128 two waves 47.1
//   2048x2048x4096    128x128 one wave 25.3 < 256x128 half a wave 30.1
//   2048x6144x4096    256x256 partial wave 47.1 < 256x128 two waves 61.2
//   4096x6144x14336   256x256 + last wave as 256x128 halves 298.9
//                     < 256x256 two waves 326.0
//   2048x2560x4096    128x128 + last wave as 64x64 quarters 37.9
//                     < 128x128 two waves 45.3
//   1024x4096x14336   256x128 split in two 69.6 < 128x128 one wave 75.2
//   512x4096x14336    256x128 split four ways 44.4 < 128x128 split two 51.7
// A K split is considered only while the split grid fits one wave of
// workgroups (a second wave costs more than the idle CUs: 1536x1536x4096
// 40.2 us split in two, 24.2 unsplit); 256x256 and 192x256 grids are never
// split. Two exclusions the model does not reproduce, each measured on
// several shapes with the weights streamed from HBM: 256x128 tiles are not
// split over 8 or fewer column tiles (N = 1024: 2048x1024x14336 56.0 us
// split four ways against 48.1 for 128x128 tiles split two ways,
// 1536x1024x14336 49.5 against 45.8, 1280x1024x14336 47.6 against 44.7),
// nor below 256 rows (M = 200: 200x14336x14336 82.0 split two ways against
// 76.6 on 128x128 tiles, 200x16384x14336 86.0 against 81.6, 200x11008x14336
// 77.5 against 74.5; unsplit they stay ahead: 200x28672x4096 47.0 against
// 53.0 on 192x256 tiles). Per-row weight scales (one more multiply per
// fold) slow the tiles unevenly: x1.10 for 256x256, x1.08 for 256x128,
// x1.20 for 128x128 (fitted to 72 shapes, 69 of their 72 choices right or
// within 2%).
// FP8B_TILE192=0, FP8B_TILE256X128=0, FP8B_TAIL128=0 and FP8B_TAIL64=0
// take the corresponding candidates out.
// ---------------------------------------------------------------------------
struct TileCost {
  int cfg, bm, bn;
  double kb_us;   // per K-block of one tile on one CU of a fully busy chip
  double per_row; // factor with per-row weight scales (one more multiply per fold)
};
constexpr TileCost kTileCosts[] = {{CFG_256x256, 256, 256, 1.62, 1.10},
                                   {CFG_192x256, 192, 256, 1.31, 1.0},
                                   {CFG_256x128, 256, 128, 1.08, 1.08},
                                   {CFG_128x128, 128, 128, 0.67, 1.20}};
constexpr double kQuarter64KbUs = 0.40;     // 64x64 quarters on gemm_tiny_kernel
constexpr double kFirstKbUs = 4.7;          // launch and first K-block, per wave
constexpr double kStoreBytesPerUs = 9.4e6;  // a wave's output stores
constexpr double kSplitSumUs = 3.1;         // split-K sum kernel and its launch
constexpr double kSplitBytesPerUs = 7.0e6;  // fp32 partials written and read back

double power_factor(int64_t active, int cus) {
  const double f = std::min(1.0, (double)active / (double)cus);
  return std::max(0.93, 1.0 - 0.85 * (1.0 - f));
}

double tile_kb_us(int cfg, bool per_row = false) {
  for (const TileCost& tc : kTileCosts)
    if (tc.cfg == cfg) return tc.kb_us * (per_row ? tc.per_row : 1.0);
  return 1.0;
}

// One wave of `active` workgroups, each a bm x bn tile over kbs K-blocks,
// storing out_bytes per output element.
double wave_us(double kb_us, int bm, int bn, int64_t active, int kbs, double out_bytes,
               int cus) {
  return kFirstKbUs + kbs * kb_us * power_factor(active, cus) +
         (double)active * bm * bn * out_bytes / kStoreBytesPerUs;
}

// Full waves of t tiles, then the last partial wave.
double grid_us(double kb_us, int bm, int bn, int64_t t, int kbs, double out_bytes, int cus) {
  const int64_t full = t / cus, rest = t % cus;
  return full * wave_us(kb_us, bm, bn, cus, kbs, out_bytes, cus) +
         (rest ? wave_us(kb_us, bm, bn, rest, kbs, out_bytes, cus) : 0.0);
}

bool tile_enabled(int cfg, bool per_row) {
  if (cfg == CFG_192x256) return !per_row && use_tile192();
  if (cfg == CFG_256x128) return use_tile256x128();
  return true;
}

// The cheapest MFMA-bound plan by the cost model above.
Plan large_tile_plan(int64_t M, int64_t N, int64_t K, bool per_row, int cus) {
  const int KB = (int)(K / 128);
  const double q64_us = kQuarter64KbUs * (per_row ? tile_kb_us(CFG_128x128, true) /
                                                        tile_kb_us(CFG_128x128) : 1.0);
  Plan best{CFG_128x128, 128, 128, 1, KB, TAIL_NONE};
  double best_us = 1e300;
  auto consider = [&](const Plan& p, double us) {
    if (us < best_us) {
      best = p;
      best_us = us;
    }
  };
  for (const TileCost& tc : kTileCosts) {
    if (!tile_enabled(tc.cfg, per_row)) continue;
    const int64_t tn = (N + tc.bn - 1) / tc.bn;
    const int64_t t = ((M + tc.bm - 1) / tc.bm) * tn;
    const double kb_us = tile_kb_us(tc.cfg, per_row);
    consider({tc.cfg, tc.bm, tc.bn, 1, KB, TAIL_NONE},
             grid_us(kb_us, tc.bm, tc.bn, t, KB, 2.0, cus));
    // The last partial wave on smaller tiles (same per-output arithmetic):
    // 256x256 tiles as 128x128 quarters or 256x128 halves, 128x128 tiles
    // as 64x64 quarters, when the smaller tiles fit one per CU.
    const int64_t full = t / cus, rest = t % cus;
    if (full > 0 && rest > 0) {
      const double base = full * wave_us(kb_us, tc.bm, tc.bn, cus, KB, 2.0, cus);
      if (tc.cfg == CFG_256x256 && use_tail128() && 4 * rest <= cus)
        consider({tc.cfg, tc.bm, tc.bn, 1, KB, TAIL_Q128},
                 base + wave_us(tile_kb_us(CFG_128x128, per_row), 128, 128, 4 * rest, KB, 2.0, cus));
      if (tc.cfg == CFG_256x256 && use_tile256x128() && 2 * rest <= cus)
        consider({tc.cfg, tc.bm, tc.bn, 1, KB, TAIL_H256X128},
                 base + wave_us(tile_kb_us(CFG_256x128, per_row), 256, 128, 2 * rest, KB, 2.0, cus));
      if (tc.cfg == CFG_128x128 && use_tiny() && use_tail64() && 4 * rest <= cus)
        consider({tc.cfg, tc.bm, tc.bn, 1, KB, TAIL_Q64},
                 base + wave_us(q64_us, 64, 64, 4 * rest, KB, 2.0, cus));
    }
    // K splits, in whole scale half-windows (multiples of 4 K-blocks, which
    // keep the 16-byte window lanes) when KB allows, at least four K-blocks
    // per split.
    if ((tc.cfg == CFG_128x128 || (tc.cfg == CFG_256x128 && tn > 8 && M >= 256)) && t < cus) {
      for (int s = 2; t * s <= cus && KB / s >= 4; s *= 2) {
        int kbs = (KB + s - 1) / s;
        if (KB % 4 == 0) kbs = (kbs + 3) / 4 * 4;
        const int splits = (KB + kbs - 1) / kbs;
        if (t * splits > cus) break;
        const double us = wave_us(kb_us, tc.bm, tc.bn, t * splits, kbs, 4.0, cus) +
                          kSplitSumUs + 2.0 * splits * (double)M * N * 4.0 / kSplitBytesPerUs;
        consider({tc.cfg, tc.bm, tc.bn, splits, kbs, TAIL_NONE}, us);
      }
    }
  }
  return best;
}

// Grids for gemm_tiny_kernel: at most 8 tiles of 32x32 per CU and at most
// 128 tile K-blocks per CU. Measured (HIP-graph replay, against the
// 128x128 kernel split along K within one wave of workgroups): 512x512x2048
// 4.6 against 11.7 us, 512x512x7168 7.9 against 16.0, 768x768x4096 11.1
// against 16.5, 2048x1024x2048 14.1 against 20.7; past 128 K-blocks per CU
// the split 128x128 grid wins (1024x2048x4096: 24.6 against 23.2).
bool tiny_grid(int64_t t32, int KB, int cus) {
  return t32 <= 8 * (int64_t)cus && t32 * KB <= 128 * (int64_t)cus;
}

// Tile of gemm_tiny_kernel for a small grid, or false when the grid is not
// one (grids this small never take the 256x256 plans). Measured in HIP-graph
// replay against the plans they replace; for M <= 64 with the weights
// streamed from HBM (each launch of the graph on another weight copy, 600 MB
// of copies past the 256 MB MALL, as a decode step over a model's layers):
//  * 64x64 tiles for a band of mid-size grids, M > 64 with 16..64 K-blocks
//    and about one to two tiles per CU: 1024x2048x4096 19.1 against 22.8 us
//    (split 128x128), 2048x1024x2048 12.5 against 14.0, 960x1024x4096 12.1
//    against 14.6, 1024x1024x8192 19.5 against 24.2. Outside it they lost:
//    1024x2048x14336 52.3 against 47.6, 1536x1536x4096 (576 tiles, a second
//    partial round) 33.8 against 24.3, 768x768x4096 (144 tiles) 11.6
//    against 11.1. Between one and two tiles per CU only 24..48 K-blocks
//    gain (steady clock, 384 tiles: 768x2048x4096 18.1 against 20.8 us;
//    16 K-blocks 11.9 against 10.7, 64 K-blocks 31.8 against 30.3); at two
//    tiles per CU only up to 32 K-blocks (weights streamed: 256x8192x2048
//    14.7 against 18.3, 1024x2048x4096 21.4 against 23.4; 48 and 64
//    K-blocks lost: 256x8192x6144 36.6 against 30.9, 256x8192x8192 47.0
//    against 38.2, 1024x2048x8192 37.3 against 33.8). Between one and two
//    tiles per CU, with the weights streamed, only while N <= 16 M: wider
//    grids of few rows lost (128x11008x4096 27.6 against 24.9, 128x11008x6144
//    41.0 against 32.0, 256x6144x4096 24.7 against 22.7), 384x4096x4096
//    (21.8 against 22.4) and 768x2048x4096 (20.9 against 22.0) gained. At
//    7/8 to one tile per CU past 32 K-blocks likewise: per-row 128x8192x8192
//    33.2 against 30.7, 96x7168x8192 29.9 against 27.4 (block scales
//    128x8192x8192 28.6 against 27.7), while 256x4096x8192 (N = 16 M) was
//    level and 32 K-blocks gained (per-row 128x4096x4096 13.4 against 21.0).
//  * 32x32 tiles (tiny_grid) up to 64 K-blocks for M > 64, replacing the
//    split 128x128 plan (512x512x2048 5.2 against 12.9 us, 128x4096x4096
//    12.0 against 19.8, 256x7168x2048 14.4 against 21.3; at 224 K-blocks
//    38.6 against 21.7 for 128x1024x28672, at 112 20.9 against 19.2 for
//    128x2048x14336), and at 49..64 rows, replacing the 64x128 tiles
//    (64x2048x4096 8.1 against 12.6; at 112 K-blocks 24.2 against 23.6;
//    with block scales make_plan keeps only grids below 48 K-blocks or of at
//    most one tile per CU here, the rest stream faster on the decode kernel);
//    at up to 48 rows up to 32 K-blocks,
//    replacing the decode and skinny kernels, once the grid has a tile per
//    CU (32x14336x4096 16.4 against 19.2; 1x8192x4096 9.5 against 11.3;
//    48x7168x2048 7.3 against 11.4), or half that with M > 16. Longer K
//    keeps the decode kernel's deeper weight stream (32x8192x14336 29.6
//    against 26.8, 32x16384x7168 31.1 against 26.9).
//  * 32x16 tiles at 9..32 rows and 16..64 K-blocks when they fill 3/4 to all
//    of the CUs once and 32x32 tiles would not fill them: 32x4096x4096 7.4
//    against 8.2 (skinny), 16x4096x7168 9.2 against 10.9 and 32x4096x7168
//    11.5 against 12.1 (decode + split-K sum); at 112 K-blocks the decode
//    kernel wins (32x4096x14336: 16.7 against 21.6).
bool small_grid_tile(int64_t M, int64_t N, int KB, int cus, int& tm, int& tn) {
  auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  const int64_t c = cus;
  const int64_t t64 = tiles(64, 64), t32 = tiles(32, 32), t16 = tiles(32, 16);
  tm = 32;
  if (M > 64 && KB >= 16 && KB <= 64 &&
      ((t64 == 2 * c && KB <= 32) ||
       (t64 > c && t64 < 2 * c && KB >= 24 && KB <= 48 && N <= 16 * M) ||
       (8 * t64 >= 7 * c && t64 <= c && (KB <= 32 || N <= 16 * M)))) {
    tm = tn = 64;
    return true;
  }
  tn = 32;
  // Past 48 K-blocks, 1 to 1.75 tiles per CU leave half the CUs with two
  // long tiles: the split 128x128 plan wins there (weights streamed, 384
  // tiles: 96x4096x7168 18.0 against 20.7 us, 80x4096x8192 18.0 against
  // 21.2, 128x3072x8192 18.8 against 22.0; per-row scales 96x4096x7168 20.0
  // against 23.9; 480 tiles keep the small grid: 72x5120x7168 18.8 against
  // 20.8).
  if (M > 64 && KB > 48 && t32 > c && 4 * t32 <= 7 * c) return false;
  if (M > 48) return tiny_grid(t32, KB, cus) && KB <= 64;
  if (tiny_grid(t32, KB, cus) && t32 >= c && KB <= 32) return true;
  if (M > 8 && M <= 32 && KB >= 16 && KB <= 64 && t16 <= c && 4 * t16 >= 3 * c) {
    tn = 16;
    return true;
  }
  return tiny_grid(t32, KB, cus) && 2 * t32 >= c && KB <= 32 && M > 16;
}

// per_row: weight scales per output row (block_n = 1, the deep-gemm layout);
// the decode kernel, gemm_tiny_kernel, gemm_pipe128_kernel, gemm_pipe256x128_kernel
// and gemm_pipe256_kernel implement it.
Plan make_plan(int64_t M, int64_t N, int64_t K, bool per_row, int cus) {
  const int KB = (int)(K / 128);
  Plan p{};
  auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  if (M <= 48 && !use_decode_kernel() && !per_row) {
    // Skinny path: 16 output columns per workgroup, K split inside it.
    p.cfg = CFG_SKINNY; p.bm = (int)(((M + 15) / 16) * 16); p.bn = 16;
    p.splits = 1;
    p.kb_per_split = KB;
    return p;
  }
  // 49..64 rows (weights streamed from HBM) take the decode kernel with 64
  // activation rows. Per-row scales: 64x8192x8192 24.5 against 31.3 us on
  // the small-grid kernel, 64x4096x14336 22.3 against 26.7 on 128x128
  // tiles, 50x6144x8192 20.7 against 26.6. Block scales: level with 128x128 tiles (half
  // of each tile's rows idle) within 2% (56x14336x14336 53.5 against 54.2
  // us, 64x28672x4096 33.8 against 34.0, 64x18432x8192 50.1 against 49.3)
  // and ahead of the 64x128 tiles of the non-pipelined kernel
  // (64x4096x14336 19.3 against 23.5, 64x57344x2048 26.4 against 28.2). The
  // small-grid kernel keeps short K and grids of at most one 32x32 tile per
  // CU; from 48 K-blocks on a larger grid the decode kernel's weight stream
  // is faster (64x8192x8192 22.9 against 27.0 us, 64x5120x8192 17.9 against
  // 24.5, 64x6144x6144 17.5 against 20.4, 50x6144x8192 18.7 against 22.7;
  // at 32 K-blocks 64x12288x4096 20.8 against 19.9, 56x11008x4096 19.9
  // against 19.0; at 256 tiles 64x4096x8192 15.8 against 14.8).
  const bool decode64 = M > 48 && M <= 64 && use_decode_kernel();
  // 17..48 rows and at least half as many 128-column tiles as CUs (at most
  // two decode splits): the decode kernel streams the weights faster than
  // the small-grid kernel's many 32x32 tiles (48x28672x2048 16.6 against
  // 20.5 us, 48x32768x1024 10.9 against 12.8, 48x16384x4096 20.6 against
  // 22.8, 17x28672x2048 14.0 against 15.1; per-row scales 48x28672x2048 17.8
  // against 22.6, 48x16384x4096 22.4 against 27.1); with
  // fewer tiles the small-grid kernel keeps them (48x14336x2048 12.7
  // against 14.5, 32x14336x4096 17.3 against 18.4), and at one row it
  // stays ahead at any width (1x28672x4096 25.2 against 30.7).
  // Up to 16 rows only where the decode grid is unsplit (more than half as
  // many column tiles as CUs) and K short: 1x28672x2048 13.1 against 14.1,
  // 16x28672x2048 13.6 against 14.8, 4x32768x1536 11.7 against 12.4; at 128
  // tiles (two splits) and at 32 K-blocks the small-grid kernel stays ahead
  // (8x16384x2048 9.1 against 11.5, 16x28672x4096 26.4 against 30.0).
  const int64_t t128 = (N + 127) / 128;
  const bool decode_wide =
      use_decode_kernel() && ((M > 16 && M <= 48 && 2 * t128 >= cus) ||
                              (M <= 16 && 2 * t128 > cus && KB <= 16));
  const bool tiny_ok = !(decode64 && KB >= 48 && tiles(32, 32) > cus) && !decode_wide;
  int tm = 0, tn = 0;
  if (use_tiny() && tiny_ok && small_grid_tile(M, N, KB, cus, tm, tn)) {
    p.cfg = CFG_TINY; p.bm = tm; p.bn = tn;
    p.splits = 1;
    p.kb_per_split = KB;
    return p;
  }
  if (use_decode_kernel() && (M <= 48 || decode64)) {
    // Decode path: 128 output columns per workgroup; split K as often as
    // the grid still fits one workgroup per CU. Splitting once more, until
    // the grid covers every CU, overfills it: the workgroups past the CU
    // count share CUs on a shallower ring (or, with per-row scales, run as
    // a second round), and the weight stream slows by more than the idle
    // CUs cost (weights streamed from HBM: 32x7168x8192 17.7 against 20.3
    // us, 8x13824x5120 17.8 against 20.3, 16x12800x14336 39.0 against
    // 45.6, 32x18432x8192 unsplit on 144 CUs 42.8 against 47.7). Except
    // where that leaves exactly 32 K-blocks per split on two or more
    // splits, which measured 6-10% slower than the overfilled grid
    // (16x12800x8192 31.7 against 29.0 us, 8x13824x8192 32.2 against 29.5;
    // 33 or 34 K-blocks per split were no faster).
    p.cfg = CFG_DECODE; p.bm = (int)(((M + 15) / 16) * 16); p.bn = 128;
    const int64_t t = (N + 127) / 128;
    int splits = 1;
    if (t < cus) {
      splits = (int)(cus / t);
      if (!per_row && splits >= 2 && (KB + splits - 1) / splits == 32)
        splits = (int)((cus + t - 1) / t);
    }
    splits = std::max(1, std::min(splits, KB));
    p.kb_per_split = (KB + splits - 1) / splits;
    p.splits = (KB + p.kb_per_split - 1) / p.kb_per_split;
    // Four or fewer K-blocks per split, or eight rows or fewer on an 8-way
    // split: the split-K partials and their sum cost more than the skinny
    // kernel's activation re-reads (measured 32x4096x4096: 11.5 us split-K,
    // 8.2 us skinny; 1..8x4096x14336: 14.7-15.0 against 13.2-13.6; but
    // 32x4096x14336: 16.1 against 21.5, 16x4096x14336 even, and 8x14336x4096
    // with 3 splits 16.7 against 20.6).
    if (!per_row && M <= 48 && (p.kb_per_split <= 4 || (M <= 8 && p.splits >= 8))) {
      p.cfg = CFG_SKINNY; p.bn = 16;
      p.splits = 1;
      p.kb_per_split = KB;
    }
    return p;
  }
  return large_tile_plan(M, N, K, per_row, cus);
}

// 32-bit DMA offsets of gemm_decode_kernel: weight rows up to 127 of a tile
// (row * ldb + 127) and activation rows up to 16*FM - 1 (row * lda + 127).
bool decode_offsets_ok(int64_t lda, int64_t ldb, int64_t M) {
  const int64_t rows = (M + 15) / 16 * 16;
  return 127 * ldb + 128 <= (int64_t(1) << 32) && (rows - 1) * lda + 128 <= (int64_t(1) << 32);
}

bool mfma_path_ok(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                  int64_t K, int64_t block_n, int64_t block_k) {
  return block_n == 128 && block_k == 128 && K % 128 == 0 && K > 0 && lda % 16 == 0 &&
         ldb % 16 == 0 && ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 &&
         M < (int64_t(1) << 30) && N < (int64_t(1) << 30) && K < (int64_t(1) << 30);
}

// Operand properties the kernel choice depends on, besides the sizes.
struct Operands {
  int64_t lda, ldb;
  bool mfma;    // mfma_path_ok
  bool scales;  // As, Bs contiguous in K with 16-byte aligned rows (16-byte window lanes)
};

// Operands of a plan query: contiguous, 16-byte aligned, K-contiguous scales.
Operands contiguous_operands(int64_t M, int64_t N, int64_t K, int64_t block_n,
                             int64_t block_k) {
  Operands o;
  o.lda = K;
  o.ldb = K;
  const bool per_row = block_n == 1 && block_k == 128;
  o.mfma = K > 0 && K % 16 == 0 &&
           mfma_path_ok(nullptr, K, nullptr, K, M, N, K, per_row ? 128 : block_n, block_k);
  o.scales = K % 512 == 0;  // K/128 scales per row: 16-byte rows when 4 | K/128
  return o;
}

// Precondition of the pipelined kernels: 32-bit DMA offsets within a
// 256-row tile. FP8B_PIPE=0 turns them off. Their scale windows take 16-byte
// DMA lanes when As and Bs are contiguous in K with 16-byte aligned rows and
// the K-block count and split size are multiples of 4 (win16_ok), else
// 4-byte lanes (any strides and counts; 4.4 against 1.1 DMA instructions
// per wave and 8 K-blocks).
bool pipe_ok(const Operands& o, int64_t K) {
  return use_pipelined_kernels() && 255 * std::max(o.lda, o.ldb) + K < (int64_t(1) << 32);
}
bool win16_ok(const Operands& o, int64_t K, int splits, int kb_per_split) {
  return o.scales && (K / 128) % 4 == 0 && (splits == 1 || kb_per_split % 4 == 0);
}

// Everything fp8b_w8a8_block_matmul launches for one call: the main kernel
// (grid `grid` workgroups of `waves` waves, splits along K in grid.z), an
// optional kernel for the last partial wave of the grid, and, when split,
// splitk_reduce_kernel. resolve() derives it from the plan and the
// operands; launch_dispatch() runs exactly it; fp8b_gemm_plan() reports it.
struct Dispatch {
  int kernel = FP8B_KERNEL_GENERIC;
  int bm = 32, bn = 32;
  int splits = 1, kb_per_split = 0;
  int waves = 4;
  int ring = 0;        // gemm_decode_kernel: LDS stages
  int64_t grid = 0;    // workgroups of the main launch (all splits)
  int tail_kernel = FP8B_KERNEL_NONE;
  int tail_bm = 0, tail_bn = 0;
  int64_t tail_grid = 0;
  bool per_row = false;
  bool win4 = false;   // pipelined kernels: scale windows by 4-byte DMA lanes
};

// One unsplit grid of 256x256 tiles on gemm_pipe256_kernel. When the tiles
// leave a last partial wave of at most a quarter of the CUs, that wave's
// tiles run as 128x128 quarters on gemm_pipe128_kernel (one wave), with the
// same arithmetic per output: MLP gate/up 3001x28672x4096 has 1344 tiles,
// five full waves and 64 left; the 64 tiles take 35 us as quarters against
// ~40 us as a sixth wave. FP8B_TAIL128=0 keeps the whole grid on
// gemm_pipe256_kernel. With more than a quarter and at most half of the CUs
// left, the wave runs as 256x128 halves on gemm_pipe256x128_kernel:
// 4096x6144x14336 (384 tiles, 128 left) 298.9 against 326.0 us,
// 2048x28672x4096 204.1 against 212.5; with per-row weight scales
// 1536x14336x7168 (80 left) 175.6 against 208.1; block scales with 80 left
// even (768x28672x14336 305.5 against 305.0).
void resolve_pipe256(Dispatch& d, int64_t tiles, int KB, int tail, int cus) {
  d.kernel = FP8B_KERNEL_PIPE256;
  d.waves = 8;
  d.grid = tiles;
  const int64_t full = tiles / cus * cus, rest = tiles - full;
  if ((tail != TAIL_Q128 && tail != TAIL_H256X128) || rest == 0 || d.kb_per_split < KB) return;
  d.grid = full;
  if (tail == TAIL_Q128) {
    d.tail_kernel = FP8B_KERNEL_PIPE128;
    d.tail_bm = d.tail_bn = 128;
    d.tail_grid = 4 * rest;
  } else {
    d.tail_kernel = FP8B_KERNEL_PIPE256X128;
    d.tail_bm = 256;
    d.tail_bn = 128;
    d.tail_grid = 2 * rest;
  }
}

// gemm_tiny_kernel with as many waves per tile as keep about eight waves
// per CU resident (two K-block slots per wave: 8448 B each for 32x32
// tiles). Measured per waves x slots on 512x512x2048: 8x2 4.6 us, 4x2 4.6,
// 2x2 5.8, 1x7 8.1; on 2048x1024x2048 (eight tiles per CU): 1x2 13.3, 2x2
// 16.2, 8x2 23.1. Four waves up to 2.5 tiles per CU (weights streamed,
// 576 tiles: 96x6144x4096 17.1 against 18.7 us with two, 80x6144x4096 16.0
// against 17.9, per-row 96x6144x4096 19.0 against 21.4; 672 tiles level,
// 768 tiles 16.7 with two against 17.0). 64x64 tiles (16896 B per slot): four waves for up to one
// tile per CU, else two (1024x2048x4096: 2x2 19.1 us, 4x2 22.0, 1x2 28.9,
// 2x3 33.0).
int tiny_waves(int64_t t, int tile_n, int cus) {
  if (tile_n == 16) return 8;
  if (tile_n == 64) return t <= cus ? 4 : 2;
  if (t <= cus) return 8;
  if (2 * t <= 5 * (int64_t)cus) return 4;
  if (t <= 4 * (int64_t)cus) return 2;
  return 1;
}

// One grid of 128x128 tiles on gemm_pipe128_kernel. When the plan gives the
// last partial wave of an unsplit grid to 64x64 quarters, those run on
// gemm_tiny_kernel (four waves per quarter, one quarter per CU):
// 2048x2560x4096 has 320 tiles, one full wave and 64 left.
void resolve_pipe128(Dispatch& d, int64_t tiles, int tail, int cus) {
  d.kernel = FP8B_KERNEL_PIPE128;
  d.waves = 8;
  d.grid = tiles * d.splits;
  if (d.splits > 1 || tail != TAIL_Q64 || tiles % cus == 0) return;
  const int64_t full = tiles / cus * cus, rest = tiles - full;
  d.grid = full;
  d.tail_kernel = FP8B_KERNEL_TINY;
  d.tail_bm = d.tail_bn = 64;
  d.tail_grid = 4 * rest;
}

// The launches of one GEMM call (see Dispatch) on a device with `cus` CUs.
Dispatch resolve_uncached(int64_t M, int64_t N, int64_t K, int64_t block_n, int64_t block_k,
                          int cus, const Operands& o) {
  Dispatch d;
  const bool per_row = block_n == 1 && block_k == 128;
  d.per_row = per_row;
  if (!o.mfma) {
    d.bm = d.bn = 32;
    d.grid = ((N + 31) / 32) * ((M + 31) / 32);
    return d;  // gemm_generic_kernel
  }
  const int KB = (int)(K / 128);
  Plan p = make_plan(M, N, K, per_row, cus);
  // Leading dimensions too large for the decode kernel's 32-bit DMA offsets:
  // the skinny kernel (64-bit addresses, no workspace) or, for per-row
  // scales and more than 48 rows, the generic kernel.
  if (p.cfg == CFG_DECODE && !decode_offsets_ok(o.lda, o.ldb, M)) {
    if (per_row || M > 48) {
      d.grid = ((N + 31) / 32) * ((M + 31) / 32);
      return d;
    }
    p.cfg = CFG_SKINNY; p.bn = 16; p.splits = 1; p.kb_per_split = KB;
  }
  const bool pipe = pipe_ok(o, K);
  // 192x256 and 256x128 tiles exist only as pipelined kernels: without
  // their preconditions the grid goes back to 256x256 or 128x128 tiles.
  if (p.cfg == CFG_192x256 && !pipe) { p.cfg = CFG_256x256; p.bm = 256; p.tail = TAIL_NONE; }
  if (p.cfg == CFG_256x128 && !pipe) { p.cfg = CFG_128x128; p.bm = 128; p.tail = TAIL_NONE; }
  d.bm = p.bm;
  d.bn = p.bn;
  d.splits = p.splits;
  d.kb_per_split = p.kb_per_split;
  d.win4 = !win16_ok(o, K, p.splits, p.kb_per_split);
  const int64_t tiles = ((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn);
  switch (p.cfg) {
    case CFG_SKINNY:
      d.kernel = FP8B_KERNEL_SKINNY;
      d.bm = (int)(((M + 15) / 16) * 16);
      d.waves = 8;
      d.grid = (N + 15) / 16;
      break;
    case CFG_DECODE: {
      d.kernel = FP8B_KERNEL_DECODE;
      d.waves = 8;
      d.grid = ((N + 127) / 128) * p.splits;
      // Past one workgroup per CU, the three-stage ring lets two share a CU
      // instead of running a second, mostly empty round. Per-row scales
      // (up to 48 rows): 32x40960x8192 91.7 against 103.0 us, 48x36864x4096
      // 53.4 against 58.8 (grids of several rounds, e.g. 16x128256x4096, run
      // the same).
      const int fm = (int)((M + 15) / 16);
      d.ring = (d.grid > cus && (!per_row || fm <= 3)) ? 3 : 4;
      break;
    }
    case CFG_TINY:
      d.kernel = FP8B_KERNEL_TINY;
      d.waves = tiny_waves(tiles, p.bn, cus);
      d.grid = tiles;
      break;
    case CFG_256x256:
      if (pipe) {
        resolve_pipe256(d, tiles, KB, p.tail, cus);
      } else if (per_row) {
        d = Dispatch();
        d.per_row = true;
        d.grid = ((N + 31) / 32) * ((M + 31) / 32);
      } else {
        d.kernel = FP8B_KERNEL_BS128;
        d.waves = 8;
        d.grid = tiles * p.splits;
      }
      break;
    case CFG_192x256:
      d.kernel = FP8B_KERNEL_PIPE192;
      d.waves = 8;
      d.grid = tiles;
      break;
    case CFG_256x128:
      d.kernel = FP8B_KERNEL_PIPE256X128;
      d.waves = 8;
      d.grid = tiles * p.splits;
      break;
    default:  // CFG_128x128
      if (pipe) {
        resolve_pipe128(d, tiles, p.tail, cus);
      } else if (per_row) {
        d = Dispatch();
        d.per_row = true;
        d.grid = ((N + 31) / 32) * ((M + 31) / 32);
      } else {
        d.kernel = FP8B_KERNEL_BS128;
        d.waves = 4;
        d.grid = tiles * p.splits;
      }
      break;
  }
  return d;
}

// resolve() behind a per-thread cache of the last plans: the planner costs
// ~1-2 us of host time per call (the cost model prices every tile shape),
// as much as the rest of a small eager call. The key is everything the plan
// depends on (the environment switches are read once per process); 64
// direct-mapped entries, no locking, no allocation.
Dispatch resolve(int64_t M, int64_t N, int64_t K, int64_t block_n, int64_t block_k, int cus,
                 const Operands& o) {
  struct Entry {
    int64_t M = -1, N, K, bn, bk, lda, ldb;
    int cus;
    bool mfma, scales;
    Dispatch d;
  };
  thread_local Entry cache[64];
  uint64_t h = (uint64_t)M * 0x9E3779B97F4A7C15ull ^ (uint64_t)N * 0xC2B2AE3D27D4EB4Full ^
               (uint64_t)K * 0x165667B19E3779F9ull ^ (uint64_t)block_n * 31 ^ (uint64_t)block_k ^
               (uint64_t)o.lda * 0x27D4EB2F165667C5ull ^ (uint64_t)o.ldb * 0x85EBCA77C2B2AE63ull ^
               (uint64_t)cus << 7 ^ (uint64_t)o.mfma << 1 ^ (uint64_t)o.scales;
  Entry& e = cache[(h ^ (h >> 29)) & 63];
  if (e.M == M && e.N == N && e.K == K && e.bn == block_n && e.bk == block_k && e.lda == o.lda &&
      e.ldb == o.ldb && e.cus == cus && e.mfma == o.mfma && e.scales == o.scales)
    return e.d;
  const Dispatch d = resolve_uncached(M, N, K, block_n, block_k, cus, o);
  e.M = M; e.N = N; e.K = K; e.bn = block_n; e.bk = block_k; e.lda = o.lda; e.ldb = o.ldb;
  e.cus = cus; e.mfma = o.mfma; e.scales = o.scales; e.d = d;
  return d;
}

// gemm_tiny_quant_kernel for a small-grid plan of 32 x tile_n tiles.
template <int QR>
void launch_tiny_quant(const GemmArgs& a, int tile_n, int waves, int64_t grid, hipStream_t st) {
  const unsigned g = (unsigned)grid, thr = 64u * (unsigned)waves;
  if (tile_n == 16) gemm_tiny_quant_kernel<1, 8, QR><<<g, thr, 0, st>>>(a);
  else if (waves == 8) gemm_tiny_quant_kernel<2, 8, QR><<<g, thr, 0, st>>>(a);
  else if (waves == 4) gemm_tiny_quant_kernel<2, 4, QR><<<g, thr, 0, st>>>(a);
  else if (waves == 2) gemm_tiny_quant_kernel<2, 2, QR><<<g, thr, 0, st>>>(a);
  else gemm_tiny_quant_kernel<2, 1, QR><<<g, thr, 0, st>>>(a);
}

template <bool PR>
void launch_tiny(const GemmArgs& a, int tile_n, int waves, int64_t grid, hipStream_t st) {
  const unsigned g = (unsigned)grid, thr = 64u * (unsigned)waves;
  // M <= 16 on 32-row tiles with block scales: the first 16 rows only (half
  // the activation bytes per K-block; rows past M are never stored, so the
  // same bits): 1x14336x4096 12.6 against 13.5 us, 1x28672x4096 23.2
  // against 24.1, 16x14336x4096 14.0 against 14.6 (graph-replayed, rotating
  // weight copies). With per-row scales it measured slower (28.4 against
  // 26.2 us at 1x28672x4096).
  if (!PR && a.M <= 16 && tile_n != 64 && use_tiny16()) {
    if (tile_n == 16) gemm_tiny_kernel<1, 1, 8, 2, PR><<<g, thr, 0, st>>>(a);
    else if (waves == 8) gemm_tiny_kernel<1, 2, 8, 2, PR><<<g, thr, 0, st>>>(a);
    else if (waves == 4) gemm_tiny_kernel<1, 2, 4, 2, PR><<<g, thr, 0, st>>>(a);
    else if (waves == 2) gemm_tiny_kernel<1, 2, 2, 2, PR><<<g, thr, 0, st>>>(a);
    else gemm_tiny_kernel<1, 2, 1, 2, PR><<<g, thr, 0, st>>>(a);
    return;
  }
  if (tile_n == 16) gemm_tiny_kernel<2, 1, 8, 2, PR><<<g, thr, 0, st>>>(a);
  else if (tile_n == 64 && waves == 4) gemm_tiny_kernel<4, 4, 4, 2, PR><<<g, thr, 0, st>>>(a);
  else if (tile_n == 64) gemm_tiny_kernel<4, 4, 2, 2, PR><<<g, thr, 0, st>>>(a);
  else if (waves == 8) gemm_tiny_kernel<2, 2, 8, 2, PR><<<g, thr, 0, st>>>(a);
  else if (waves == 4) gemm_tiny_kernel<2, 2, 4, 2, PR><<<g, thr, 0, st>>>(a);
  else if (waves == 2) gemm_tiny_kernel<2, 2, 2, 2, PR><<<g, thr, 0, st>>>(a);
  else gemm_tiny_kernel<2, 2, 1, 2, PR><<<g, thr, 0, st>>>(a);
}

template <bool PR>
void launch_decode(const GemmArgs& a, int M, int ring, int splits, hipStream_t st) {
  const dim3 grid((unsigned)((a.N + 127) / 128), 1, (unsigned)splits);
  const int fm = (M + 15) / 16;
  if (ring == 3) {
    if (fm <= 1) gemm_decode_kernel<1, PR, 3><<<grid, 512, 0, st>>>(a);
    else if (fm == 2) gemm_decode_kernel<2, PR, 3><<<grid, 512, 0, st>>>(a);
    else if (fm == 3 || PR) gemm_decode_kernel<3, PR, 3><<<grid, 512, 0, st>>>(a);
    else gemm_decode_kernel<4, false, 3><<<grid, 512, 0, st>>>(a);
  } else {
    if (fm <= 1) gemm_decode_kernel<1, PR><<<grid, 512, 0, st>>>(a);
    else if (fm == 2) gemm_decode_kernel<2, PR><<<grid, 512, 0, st>>>(a);
    else if (fm == 3) gemm_decode_kernel<3, PR><<<grid, 512, 0, st>>>(a);
    else gemm_decode_kernel<4, PR><<<grid, 512, 0, st>>>(a);
  }
}

// The split-K sum of a call's partials (a.ws, splits planes of M x N): on
// decode grids whose column-tile count is a multiple of 8 the XCD-local
// form (32x4096x14336: act-quant GEMM step 17.0 against 17.4 us, the plain
// GEMM 16.2 against 16.4), else one thread per 4 outputs in row order.
void launch_splitk_reduce(const GemmArgs& a, const Dispatch& d, hipStream_t st) {
  if (d.kernel == FP8B_KERNEL_DECODE && a.tiles_n % 8 == 0 && use_reduce_xcd()) {
    const int64_t blocks = (int64_t)a.tiles_n * ((a.M + 7) / 8);
    splitk_reduce_xcd_kernel<<<(unsigned)blocks, 256, 0, st>>>(a, d.splits);
    return;
  }
  const int64_t quads = (int64_t)a.M * ((a.N + 3) / 4);
  splitk_reduce_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, st>>>(a, d.splits);
}

// gemm_decode_quant_kernel: the quantiser takes 8 values per lane for 16
// rows and 16 for 32 (four waves either way). LDS stages of 16 KiB of weights
// plus 16*FM bf16 rows, by measured step time (graph-replayed, bit-identical
// results): 32 rows on 3 stages, 32x4096x14336 17.0 us against 18.3 with 4,
// 19.3 with 5, 20.8 with 2 (act-quant + GEMM: 19.7); 16 rows on 4 stages,
// 16x4096x14336 15.5 us against 16.0 with 5 (act-quant + GEMM: 18.0).
int decode_quant_ring(int64_t M) { return M <= 16 ? 4 : 3; }
void launch_decode_quant(const GemmArgs& a, int M, int splits, hipStream_t st) {
  const dim3 grid((unsigned)((a.N + 127) / 128), 1, (unsigned)splits);
  if (M <= 16) gemm_decode_quant_kernel<1, 4, 8><<<grid, 512, 0, st>>>(a);
  else gemm_decode_quant_kernel<2, 3, 16><<<grid, 512, 0, st>>>(a);
}

// fp8b_act_quant_matmul takes gemm_skinny_quant_kernel when the plan is the
// skinny kernel, M <= 8 and the bf16 rows are 16-byte aligned.
bool skinny_quant_ok(const Dispatch& d, const void* x, int64_t ldx, int64_t M) {
  return use_fused_decode() && d.kernel == FP8B_KERNEL_SKINNY && M <= 8 &&
         ((uintptr_t)x & 15) == 0 && ldx % 8 == 0;
}

// ... and gemm_tiny_quant_kernel when the plan is one small grid of 32x16 or
// 32x32 tiles (no tail launch) and the rows are 16-byte aligned, for M <= 8,
// or M <= 16 with at most 4 K-blocks per wave: a wave quantises 16 rows in
// ~200 VALU instructions per K-block, which pays for the saved launch only
// over a short K range (12x8192x2048, 2 K-blocks per wave: 7.2 against
// 8.9 us; 16x4096x4096, 4: 8.5 against 8.8; 16x14336x4096, 8: 16.8 against
// 16.3; 16x28672x4096, 16: level). Measured the same way, the skinny kernel
// with 16 rows lost (9x2048x8192: 11.9 against 9.7 us).
bool tiny_quant_ok(const Dispatch& d, const void* x, int64_t ldx, int64_t M, int64_t K) {
  const int64_t kb_per_wave = (K / 128 + d.waves - 1) / d.waves;
  return use_fused_decode() && d.kernel == FP8B_KERNEL_TINY && d.tail_kernel == FP8B_KERNEL_NONE &&
         d.bm == 32 && (d.bn == 16 || d.bn == 32) && (M <= 8 || (M <= 16 && kb_per_wave <= 4)) &&
         ((uintptr_t)x & 15) == 0 && ldx % 8 == 0;
}

// fp8b_act_quant_matmul takes gemm_decode_quant_kernel when the plan is the
// decode kernel with one workgroup per CU (grids past the CU count run two
// smaller-ring workgroups per CU, for which the bf16 stages do not fit), the
// bf16 rows are 16-byte aligned, and the 32-bit DMA offsets fit.
bool fused_decode_ok(const Dispatch& d, const void* x, int64_t ldx, int64_t ldb, int64_t M) {
  if (!use_fused_decode() || d.kernel != FP8B_KERNEL_DECODE || d.per_row || d.ring != 4) return false;
  if (M > 32 || ((uintptr_t)x & 15) != 0 || ldx % 8 != 0) return false;
  const int64_t rows = (M + 15) / 16 * 16;
  return 127 * ldb + 128 <= (int64_t(1) << 32) && (rows - 1) * 2 * ldx + 256 <= (int64_t(1) << 32);
}

// Runs the main launch and the tail launch of d (not the split-K sum).
template <bool PR>
void launch_dispatch(const Dispatch& d, const GemmArgs& a, hipStream_t st) {
  const dim3 grid3((unsigned)(d.grid / d.splits), 1, (unsigned)d.splits);
  switch (d.kernel) {
    case FP8B_KERNEL_SKINNY: {
      const int fm = (a.M + 15) / 16;
      if constexpr (!PR) {
        // staged activation row groups: ceil(M / 8) (odd counts save a DMA)
        const int xg = (a.M + 7) / 8;
        const dim3 g((unsigned)d.grid);
        if (xg <= 1) gemm_skinny_kernel<1, 1><<<g, 512, 0, st>>>(a);
        else if (fm <= 1) gemm_skinny_kernel<1, 2><<<g, 512, 0, st>>>(a);
        else if (xg == 3) gemm_skinny_kernel<2, 3><<<g, 512, 0, st>>>(a);
        else if (fm == 2) gemm_skinny_kernel<2, 4><<<g, 512, 0, st>>>(a);
        else if (xg == 5) gemm_skinny_kernel<3, 5><<<g, 512, 0, st>>>(a);
        else gemm_skinny_kernel<3, 6><<<g, 512, 0, st>>>(a);
      }
      break;
    }
    case FP8B_KERNEL_DECODE:
      launch_decode<PR>(a, a.M, d.ring, d.splits, st);
      break;
    case FP8B_KERNEL_TINY:
      launch_tiny<PR>(a, d.bn, d.waves, d.grid, st);
      break;
    case FP8B_KERNEL_PIPE256:
      gemm_pipe256_kernel<PR><<<(unsigned)d.grid, 512, 0, st>>>(a);
      break;
    case FP8B_KERNEL_PIPE192:
      if constexpr (!PR) gemm_pipe192_kernel<false><<<(unsigned)d.grid, 512, 0, st>>>(a);
      break;
    case FP8B_KERNEL_PIPE256X128:
      gemm_pipe256x128_kernel<PR><<<grid3, 512, 0, st>>>(a);
      break;
    case FP8B_KERNEL_PIPE128:
      // 32x64 wave tiles (two activation and four weight fragments per
      // K-block) measured 3-6% faster than 64x32 on 2048x2048x4096; the
      // per-row-scale grids take 64x32
      if constexpr (PR) gemm_pipe128_kernel<64, 32, true><<<grid3, 512, 0, st>>>(a);
      else gemm_pipe128_kernel<32, 64, false><<<grid3, 512, 0, st>>>(a);
      break;
    case FP8B_KERNEL_BS128:
      if constexpr (!PR) {
        if (d.bm == 256) gemm_bs128_kernel<256, 256, 64, 128><<<grid3, 512, 0, st>>>(a);
        else gemm_bs128_kernel<128, 128, 64, 64><<<grid3, 256, 0, st>>>(a);
      }
      break;
    default:
      break;
  }
  if (d.tail_kernel == FP8B_KERNEL_NONE) return;
  GemmArgs r = a;
  r.rem_base = (int)d.grid;
  r.rem_tiles_m = a.tiles_m;
  r.rem_tiles_n = a.tiles_n;
  r.tiles_m = (a.M + d.tail_bm - 1) / d.tail_bm;
  r.tiles_n = (a.N + d.tail_bn - 1) / d.tail_bn;
  if (d.tail_kernel == FP8B_KERNEL_PIPE128)
    gemm_pipe128_kernel<64, 32, PR><<<(unsigned)d.tail_grid, 512, 0, st>>>(r);
  else if (d.tail_kernel == FP8B_KERNEL_PIPE256X128)
    gemm_pipe256x128_kernel<PR><<<(unsigned)d.tail_grid, 512, 0, st>>>(r);
  else
    gemm_tiny_kernel<4, 4, 4, 2, PR><<<(unsigned)d.tail_grid, 256, 0, st>>>(r);
}

const char* kernel_name(int k) {
  switch (k) {
    case FP8B_KERNEL_NONE: return "none";
    case FP8B_KERNEL_GENERIC: return "gemm_generic_kernel";
    case FP8B_KERNEL_SKINNY: return "gemm_skinny_kernel";
    case FP8B_KERNEL_DECODE: return "gemm_decode_kernel";
    case FP8B_KERNEL_TINY: return "gemm_tiny_kernel";
    case FP8B_KERNEL_PIPE128: return "gemm_pipe128_kernel";
    case FP8B_KERNEL_PIPE256: return "gemm_pipe256_kernel";
    case FP8B_KERNEL_PIPE192: return "gemm_pipe192_kernel";
    case FP8B_KERNEL_PIPE256X128: return "gemm_pipe256x128_kernel";
    case FP8B_KERNEL_BS128: return "gemm_bs128_kernel";
    case FP8B_KERNEL_DECODE_QUANT: return "gemm_decode_quant_kernel";
    case FP8B_KERNEL_SKINNY_QUANT: return "gemm_skinny_quant_kernel";
    case FP8B_KERNEL_TINY_QUANT: return "gemm_tiny_quant_kernel";
    default: return "unknown";
  }
}

// Operands of a call, as resolve() sees them.
Operands call_operands(const void* A, int64_t lda, const void* B, int64_t ldb, const float* As,
                       int64_t as_sm, int64_t as_sk, const float* Bs, int64_t bs_sn,
                       int64_t bs_sk, int64_t M, int64_t N, int64_t K, int64_t block_n,
                       int64_t block_k) {
  const bool per_row = block_n == 1 && block_k == 128;
  Operands o;
  o.lda = lda;
  o.ldb = ldb;
  o.mfma = mfma_path_ok(A, lda, B, ldb, M, N, K, per_row ? 128 : block_n, block_k);
  o.scales = as_sk == 1 && bs_sk == 1 && as_sm % 4 == 0 && bs_sn % 4 == 0 &&
             ((uintptr_t)As & 15) == 0 && ((uintptr_t)Bs & 15) == 0;
  return o;
}

bool plan_args_ok(int64_t M, int64_t N, int64_t K, int64_t block_n, int64_t block_k) {
  return M > 0 && N > 0 && K > 0 && block_n > 0 && block_k > 0;
}

}  // namespace

extern "C" size_t fp8b_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int64_t block_n,
                                           int64_t block_k) {
  const bool per_row = block_n == 1;
  if (M <= 0 || N <= 0 || K <= 0 || (block_n != 128 && !per_row) || block_k != 128 ||
      K % 128 != 0)
    return 0;
  const Plan p = make_plan(M, N, K, per_row, device_cu_count());
  if (p.splits <= 1) return 0;
  return (size_t)p.splits * (size_t)M * (size_t)N * sizeof(float);
}

extern "C" const char* fp8b_kernel_name(int kernel) { return kernel_name(kernel); }

namespace {
// The fp8b_plan_info of a Dispatch.
void fill_plan(const Dispatch& d, int64_t M, int64_t N, int cus, fp8b_plan_info* plan) {
  plan->kernel = d.kernel;
  plan->tile_m = d.bm;
  plan->tile_n = d.bn;
  plan->splits = d.splits;
  plan->kb_per_split = d.kb_per_split;
  plan->waves = d.waves;
  plan->ring = d.ring;
  plan->workgroups = d.grid;
  plan->tail_kernel = d.tail_kernel;
  plan->tail_tile_m = d.tail_bm;
  plan->tail_tile_n = d.tail_bn;
  plan->tail_workgroups = d.tail_grid;
  plan->reduce = d.splits > 1 ? 1 : 0;
  plan->workspace_bytes = d.splits > 1 ? (size_t)d.splits * (size_t)M * (size_t)N * sizeof(float) : 0;
  plan->cu_count = cus;
}
}  // namespace

extern "C" int fp8b_gemm_plan(int64_t M, int64_t N, int64_t K, int64_t block_n, int64_t block_k,
                              int cu_count, fp8b_plan_info* plan) {
  if (!plan) {
    set_error("fp8b_gemm_plan: null plan");
    return FP8B_ERR_NULL;
  }
  if (!plan_args_ok(M, N, K, block_n, block_k)) {
    set_error("fp8b_gemm_plan: need M, N, K, block_n, block_k > 0");
    return FP8B_ERR_DIMS;
  }
  const int cus = cu_count > 0 ? cu_count : device_cu_count();
  const Dispatch d = resolve(M, N, K, block_n, block_k, cus,
                             contiguous_operands(M, N, K, block_n, block_k));
  fill_plan(d, M, N, cus, plan);
  return FP8B_OK;
}

extern "C" int fp8b_act_quant_matmul_plan(int64_t M, int64_t N, int64_t K, int cu_count,
                                          fp8b_plan_info* plan) {
  if (!plan) {
    set_error("fp8b_act_quant_matmul_plan: null plan");
    return FP8B_ERR_NULL;
  }
  if (!plan_args_ok(M, N, K, 128, 128) || K % 128 != 0) {
    set_error("fp8b_act_quant_matmul_plan: need M, N, K > 0 and K % 128 == 0");
    return FP8B_ERR_DIMS;
  }
  const int cus = cu_count > 0 ? cu_count : device_cu_count();
  const Dispatch d = resolve(M, N, K, 128, 128, cus, contiguous_operands(M, N, K, 128, 128));
  fill_plan(d, M, N, cus, plan);
  if (fused_decode_ok(d, nullptr, K, K, M)) {
    plan->kernel = FP8B_KERNEL_DECODE_QUANT;
    plan->ring = decode_quant_ring(M);
  } else if (skinny_quant_ok(d, nullptr, K, M)) {
    plan->kernel = FP8B_KERNEL_SKINNY_QUANT;
  } else if (tiny_quant_ok(d, nullptr, K, M, K)) {
    plan->kernel = FP8B_KERNEL_TINY_QUANT;
  }
  plan->workspace_bytes = fp8b_act_quant_matmul_workspace_size(M, N, K);
  return FP8B_OK;
}

extern "C" int fp8b_w8a8_block_matmul(const void* A, int64_t lda, const void* B, int64_t ldb,
                                      const float* As, int64_t as_sm, int64_t as_sk,
                                      const float* Bs, int64_t bs_sn, int64_t bs_sk, void* C,
                                      int64_t ldc, int out_dtype, int64_t M, int64_t N,
                                      int64_t K, int64_t block_n, int64_t block_k,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  if (M < 0 || N < 0 || K < 0 || lda < K || ldb < K || ldc < N) {
    set_error("fp8b_w8a8_block_matmul: bad dims (need M,N,K >= 0, lda,ldb >= K, ldc >= N)");
    return FP8B_ERR_DIMS;
  }
  if (block_n <= 0 || block_k <= 0) {
    set_error("fp8b_w8a8_block_matmul: block_n and block_k must be positive");
    return FP8B_ERR_BLOCK;
  }
  if (out_dtype != FP8B_F32 && out_dtype != FP8B_BF16 && out_dtype != FP8B_F16) {
    set_error("fp8b_w8a8_block_matmul: out_dtype must be FP8B_F32, FP8B_BF16 or FP8B_F16");
    return FP8B_ERR_DTYPE;
  }
  if (M == 0 || N == 0) return FP8B_OK;
  if (!C || (K > 0 && (!A || !B || !As || !Bs))) {
    set_error("fp8b_w8a8_block_matmul: null pointer");
    return FP8B_ERR_NULL;
  }
  hipStream_t st = (hipStream_t)stream;
  const size_t esz = out_dtype == FP8B_F32 ? 4 : 2;

  // block_n = 1 (per-row weight scales, the deep-gemm layout) with
  // block_k = 128 has MFMA kernels too.
  const bool per_row = block_n == 1 && block_k == 128;
  const Dispatch d = resolve(M, N, K, block_n, block_k, device_cu_count(),
                             call_operands(A, lda, B, ldb, As, as_sm, as_sk, Bs, bs_sn, bs_sk, M,
                                           N, K, block_n, block_k));

  if (d.kernel == FP8B_KERNEL_GENERIC) {
    GenericArgs g;
    g.A = (const uint8_t*)A; g.B = (const uint8_t*)B; g.As = As; g.Bs = Bs; g.C = C;
    g.lda = lda; g.ldb = ldb; g.as_sm = as_sm; g.as_sk = as_sk; g.bs_sn = bs_sn;
    g.bs_sk = bs_sk; g.ldc = ldc; g.M = M; g.N = N; g.K = K; g.block_n = block_n;
    g.block_k = block_k; g.out_dtype = out_dtype;
    dim3 grid((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32));
    if ((M + 31) / 32 > 65535) {
      set_error("fp8b_w8a8_block_matmul: M too large for the generic kernel");
      return FP8B_ERR_DIMS;
    }
    gemm_generic_kernel<<<grid, 256, 0, st>>>(g);
    if (hipGetLastError() != hipSuccess) {
      set_error("fp8b_w8a8_block_matmul: generic kernel launch failed");
      return FP8B_ERR_LAUNCH;
    }
    return FP8B_OK;
  }

  const size_t need = d.splits > 1 ? (size_t)d.splits * M * N * sizeof(float) : 0;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("fp8b_w8a8_block_matmul: workspace smaller than fp8b_gemm_workspace_size()");
    return FP8B_ERR_WORKSPACE;
  }
  if (need > 0 && ((uintptr_t)workspace & 15) != 0) {
    set_error("fp8b_w8a8_block_matmul: workspace must be 16-byte aligned");
    return FP8B_ERR_ALIGN;
  }
  const int64_t tiles_m = (M + d.bm - 1) / d.bm, tiles_n = (N + d.bn - 1) / d.bn;
  if (tiles_m * tiles_n >= (int64_t(1) << 31)) {
    set_error("fp8b_w8a8_block_matmul: too many output tiles for one launch");
    return FP8B_ERR_DIMS;
  }
  // Vector stores: 4 fp32 (16 B) for fp32 C and split-K partials, 8 x 16-bit
  // (16 B) for bf16/fp16 C.
  const bool c_vec = esz == 4 ? (ldc % 4 == 0 && ((uintptr_t)C & 15) == 0)
                              : (ldc % 8 == 0 && ((uintptr_t)C & 15) == 0);
  const bool ws_vec = (N % 4 == 0);
  GemmArgs a;
  a.A = (const uint8_t*)A; a.B = (const uint8_t*)B; a.As = As; a.Bs = Bs; a.C = C;
  a.ws = (float*)workspace;
  a.lda = lda; a.ldb = ldb; a.as_sm = as_sm; a.as_sk = as_sk; a.bs_sn = bs_sn;
  a.bs_sk = bs_sk; a.ldc = ldc; a.M = (int)M; a.N = (int)N; a.K = (int)K;
  a.KB = (int)(K / 128);
  a.kb_per_split = d.kb_per_split;
  a.tiles_m = (int)tiles_m;
  a.tiles_n = (int)tiles_n;
  a.out_dtype = out_dtype;
  a.rem_base = -1; a.rem_tiles_m = 0; a.rem_tiles_n = 0;
  a.Sq = nullptr; a.sq_sm = 0; a.sq_sg = 0;
  a.vec_store = (d.splits > 1) ? (ws_vec ? 1 : 0) : (c_vec ? 1 : 0);
  a.win4 = d.win4 ? 1 : 0;

  if (per_row) launch_dispatch<true>(d, a, st);
  else launch_dispatch<false>(d, a, st);
  if (hipGetLastError() != hipSuccess) {
    set_error("fp8b_w8a8_block_matmul: MFMA kernel launch failed");
    return FP8B_ERR_LAUNCH;
  }
  if (d.splits > 1) {
    GemmArgs r = a;
    r.vec_store = (ws_vec && c_vec) ? 1 : 0;
    launch_splitk_reduce(r, d, st);
    if (hipGetLastError() != hipSuccess) {
      set_error("fp8b_w8a8_block_matmul: split-K reduce launch failed");
      return FP8B_ERR_LAUNCH;
    }
  }
  return FP8B_OK;
}

// ---------------------------------------------------------------------------
// fp8b_w8a8_block_matmul_noalloc: the split-K partials go to `scratch`, a
// library-owned device array (one copy per GPU, held until the process
// ends), so the call needs no workspace and allocates nothing. The array's
// name is a host-side stand-in in host code: its device address on the
// current GPU comes from hipGetSymbolAddress, taken once per device and kept
// in g_scratch_dev, and only that address is passed to kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[FP8B_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the current device (nullptr on failure,
// with the error text set).
void* scratch_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("fp8b_w8a8_block_matmul_noalloc: no current HIP device (or device index >= 64)");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      set_error("fp8b_w8a8_block_matmul_noalloc: hipGetSymbolAddress of the scratch array failed");
      return nullptr;
    }
    g_scratch_dev[dev] = ptr;
  }
  return g_scratch_dev[dev];
}
}  // namespace

extern "C" int fp8b_w8a8_block_matmul_noalloc(const void* A, int64_t lda, const void* B,
                                              int64_t ldb, const float* As, int64_t as_sm,
                                              int64_t as_sk, const float* Bs, int64_t bs_sn,
                                              int64_t bs_sk, void* C, int64_t ldc, int out_dtype,
                                              int64_t M, int64_t N, int64_t K, int64_t block_n,
                                              int64_t block_k, void* stream) {
  // Argument and null-pointer errors first, with the same codes and texts as
  // the allocating entry point (it returns before touching the workspace for
  // all of them).
  if (M < 0 || N < 0 || K < 0 || lda < K || ldb < K || ldc < N || block_n <= 0 ||
      block_k <= 0 || (out_dtype != FP8B_F32 && out_dtype != FP8B_BF16 &&
                       out_dtype != FP8B_F16) || M == 0 || N == 0 || !C ||
      (K > 0 && (!A || !B || !As || !Bs)))
    return fp8b_w8a8_block_matmul(A, lda, B, ldb, As, as_sm, as_sk, Bs, bs_sn, bs_sk, C, ldc,
                                  out_dtype, M, N, K, block_n, block_k, nullptr, 0, stream);
  // The plan the allocating entry point makes for these operands: the
  // generic kernel and unsplit plans need no scratch (whatever the plan for
  // aligned operands would need).
  const Dispatch d = resolve(M, N, K, block_n, block_k, device_cu_count(),
                             call_operands(A, lda, B, ldb, As, as_sm, as_sk, Bs, bs_sn, bs_sk, M,
                                           N, K, block_n, block_k));
  const size_t need = d.kernel != FP8B_KERNEL_GENERIC && d.splits > 1
                          ? (size_t)d.splits * (size_t)M * (size_t)N * sizeof(float)
                          : 0;
  if (need > (size_t)FP8B_NOALLOC_SCRATCH_BYTES) {
    set_error("fp8b_w8a8_block_matmul_noalloc: this shape's split-K partials need more than "
              "FP8B_NOALLOC_SCRATCH_BYTES (32 MiB); use fp8b_w8a8_block_matmul with a workspace");
    return FP8B_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  if (need > 0) {
    ws = scratch_on_current_device();
    if (ws == nullptr) return FP8B_ERR_LAUNCH;
  }
  return fp8b_w8a8_block_matmul(A, lda, B, ldb, As, as_sm, as_sk, Bs, bs_sn, bs_sk, C, ldc,
                                out_dtype, M, N, K, block_n, block_k, ws, need, stream);
}

namespace {
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
}  // namespace

// Act-quant then the block GEMM. On a decode plan with M <= 32 (one
// workgroup per CU) and 16-byte aligned bf16 rows, one launch of
// gemm_decode_quant_kernel quantises the rows inside the GEMM with the plan's
// split (then the split-K sum): 17.0 us per graph-replayed step at
// 32x4096x14336 against 19.7 us for the two launches below, and 15.5 against
// 18.0 at 16x4096x14336, bit-identical. On a skinny plan with M <= 8,
// gemm_skinny_quant_kernel: 12.8 against 15.7 us at 1x4096x14336, 15.0
// against 16.9 at 8x4096x14336; on a small-grid plan with M <= 8,
// gemm_tiny_quant_kernel: 24.1 against 27.5 us at 1x28672x4096. Otherwise
// two launches on the caller's stream: the quantiser writes (q, s) into the
// workspace and the GEMM reads them (plus its own split-K partials, at the
// start of the workspace).
// Earlier one-launch forms, measured slower and removed: quantisation by
// every wave after its MFMAs (the per-column-tile repetition of the act-quant
// work then sits on each K-block's critical path), per-split prologue
// quantisation, quantisation shared across workgroups through
// device-coherent memory or one XCD's L2 (hand-offs that cost what the saved
// launch does), and activation loads issued beside the weight stream as
// compiler-generated loads (their waits drain the weight ring).
extern "C" size_t fp8b_act_quant_matmul_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0) return 0;
  // GEMM workspace, then q [M,K] and s [M,K/128].
  const size_t gemm = fp8b_gemm_workspace_size(M, N, K, 128, 128);
  return align256(gemm) + align256((size_t)M * K) + (size_t)M * (K / 128) * sizeof(float);
}

extern "C" int fp8b_act_quant_matmul(const void* x, int64_t ldx, const void* B, int64_t ldb,
                                     const float* Bs, int64_t bs_sn, int64_t bs_sk, void* C,
                                     int64_t ldc, int out_dtype, int64_t M, int64_t N,
                                     int64_t K, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (M < 0 || N < 0 || K < 0 || K % 128 != 0 || ldx < K || ldb < K || ldc < N) {
    set_error("fp8b_act_quant_matmul: bad dims (need K % 128 == 0, ldx,ldb >= K, ldc >= N)");
    return FP8B_ERR_DIMS;
  }
  if (out_dtype != FP8B_F32 && out_dtype != FP8B_BF16 && out_dtype != FP8B_F16) {
    set_error("fp8b_act_quant_matmul: out_dtype must be FP8B_F32, FP8B_BF16 or FP8B_F16");
    return FP8B_ERR_DTYPE;
  }
  if (M == 0 || N == 0) return FP8B_OK;
  if (!C || (K > 0 && (!x || !B || !Bs))) {
    set_error("fp8b_act_quant_matmul: null pointer");
    return FP8B_ERR_NULL;
  }
  const size_t need = fp8b_act_quant_matmul_workspace_size(M, N, K);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("fp8b_act_quant_matmul: workspace smaller than fp8b_act_quant_matmul_workspace_size()");
    return FP8B_ERR_WORKSPACE;
  }
  if (need > 0 && ((uintptr_t)workspace & 255) != 0) {
    set_error("fp8b_act_quant_matmul: workspace must be 256-byte aligned");
    return FP8B_ERR_ALIGN;
  }
  if (K == 0) return fp8b_w8a8_block_matmul(nullptr, 0, B, ldb, nullptr, 1, 1, Bs, bs_sn, bs_sk,
                                           C, ldc, out_dtype, M, N, 0, 128, 128, nullptr, 0,
                                           stream);
  const int64_t KB = K / 128;
  const size_t gemm = fp8b_gemm_workspace_size(M, N, K, 128, 128);
  uint8_t* q = (uint8_t*)workspace + align256(gemm);
  float* s = (float*)(q + align256((size_t)M * K));
  // The GEMM the two-kernel path would run on the quantised rows; on a
  // decode plan one kernel quantises the bf16 rows itself with that plan's
  // split (the same result bits).
  const Dispatch d = resolve(M, N, K, 128, 128, device_cu_count(),
                             call_operands(q, K, B, ldb, s, KB, 1, Bs, bs_sn, bs_sk, M, N, K,
                                           128, 128));
  const bool small_m = skinny_quant_ok(d, x, ldx, M) || tiny_quant_ok(d, x, ldx, M, K);
  if (small_m || fused_decode_ok(d, x, ldx, ldb, M)) {
    // One kernel reads the bf16 rows (a.A, row stride a.lda in bytes) and
    // quantises them itself; decode plans write split-K partials to the
    // workspace and sum them after.
    hipStream_t st = (hipStream_t)stream;
    GemmArgs a;
    a.A = (const uint8_t*)x; a.B = (const uint8_t*)B; a.As = nullptr; a.Bs = Bs; a.C = C;
    a.ws = small_m ? nullptr : (float*)workspace;
    a.lda = 2 * ldx; a.ldb = ldb; a.as_sm = 0; a.as_sk = 0; a.bs_sn = bs_sn; a.bs_sk = bs_sk;
    a.ldc = ldc; a.M = (int)M; a.N = (int)N; a.K = (int)K; a.KB = (int)KB;
    a.kb_per_split = small_m ? (int)KB : d.kb_per_split;
    a.tiles_m = 1; a.tiles_n = (int)((N + d.bn - 1) / d.bn);
    a.out_dtype = out_dtype;
    a.rem_base = -1; a.rem_tiles_m = 0; a.rem_tiles_n = 0;
    a.Sq = nullptr; a.sq_sm = 0; a.sq_sg = 0;
    a.win4 = 1;
    const bool c_vec = out_dtype == FP8B_F32 ? (ldc % 4 == 0 && ((uintptr_t)C & 15) == 0)
                                             : (ldc % 8 == 0 && ((uintptr_t)C & 15) == 0);
    const bool ws_vec = (N % 4 == 0);
    a.vec_store = (!small_m && d.splits > 1) ? (ws_vec ? 1 : 0) : (c_vec ? 1 : 0);
    if (!small_m) {
      launch_decode_quant(a, (int)M, d.splits, st);
    } else if (d.kernel == FP8B_KERNEL_TINY) {
      if (M <= 4) launch_tiny_quant<4>(a, d.bn, d.waves, d.grid, st);
      else if (M <= 8) launch_tiny_quant<8>(a, d.bn, d.waves, d.grid, st);
      else launch_tiny_quant<16>(a, d.bn, d.waves, d.grid, st);
    } else if (M <= 4) {
      gemm_skinny_quant_kernel<4><<<(unsigned)d.grid, 512, 0, st>>>(a);
    } else {
      gemm_skinny_quant_kernel<8><<<(unsigned)d.grid, 512, 0, st>>>(a);
    }
    if (hipGetLastError() != hipSuccess) {
      set_error("fp8b_act_quant_matmul: act-quant GEMM kernel launch failed");
      return FP8B_ERR_LAUNCH;
    }
    if (!small_m && d.splits > 1) {
      GemmArgs r = a;
      r.vec_store = (ws_vec && c_vec) ? 1 : 0;
      launch_splitk_reduce(r, d, st);
      if (hipGetLastError() != hipSuccess) {
        set_error("fp8b_act_quant_matmul: split-K reduce launch failed");
        return FP8B_ERR_LAUNCH;
      }
    }
    return FP8B_OK;
  }
  int rc = fp8b_act_quant(x, ldx, q, K, s, KB, 1, M, K, 128, stream);
  if (rc != FP8B_OK) return rc;
  return fp8b_w8a8_block_matmul(q, K, B, ldb, s, KB, 1, Bs, bs_sn, bs_sk, C, ldc, out_dtype, M, N,
                                K, 128, 128, gemm ? workspace : nullptr, gemm, stream);
}

namespace {
// Tile rows of the fused gate/up kernel by the GEMM cost model: 192x256
// against 256x256 tiles, unsplit and without tail launches (the SWIGLU
// epilogue needs each gate block and its up block in one workgroup), each
// wave also paying the epilogue's SiLU and quantisation (~3.5 us per
// 256x256 tile while its matrix cores idle) and storing fp8 codes for half
// of its columns. M = 3001, I = 14336: 1792 tiles of 192x256 (seven waves)
// against 1344 of 256x256 (six, the last of 64 tiles), 517.7 against 528.4
// us for the gate/up + down chain.
bool gate_up_tile192(int64_t M, int64_t I, int64_t K, int cus) {
  if (!use_tile192()) return false;
  const int64_t tn = 2 * I / 256;
  const int KB = (int)(K / 128);
  auto cost = [&](int bm, double kb_us) {
    const int64_t t = ((M + bm - 1) / bm) * tn;
    const int64_t waves = (t + cus - 1) / cus;
    return grid_us(kb_us, bm, 256, t, KB, 0.5, cus) + waves * 3.5 * bm / 256.0;
  };
  return cost(192, tile_kb_us(CFG_192x256)) < cost(256, tile_kb_us(CFG_256x256));
}
}  // namespace

extern "C" int fp8b_gate_up_plan(int64_t M, int64_t I, int64_t K, int cu_count,
                                 fp8b_plan_info* plan) {
  if (!plan) {
    set_error("fp8b_gate_up_plan: null plan");
    return FP8B_ERR_NULL;
  }
  if (M <= 0 || I <= 0 || I % 128 != 0 || K <= 0 || K % 128 != 0) {
    set_error("fp8b_gate_up_plan: need M > 0, I a positive multiple of 128 and K a positive "
              "multiple of 128");
    return FP8B_ERR_DIMS;
  }
  const int cus = cu_count > 0 ? cu_count : device_cu_count();
  const bool t192 = gate_up_tile192(M, I, K, cus);
  *plan = fp8b_plan_info{};
  plan->kernel = t192 ? FP8B_KERNEL_PIPE192 : FP8B_KERNEL_PIPE256;
  plan->tile_m = t192 ? 192 : 256;
  plan->tile_n = 256;
  plan->splits = 1;
  plan->kb_per_split = (int)(K / 128);
  plan->waves = 8;
  plan->workgroups = ((M + plan->tile_m - 1) / plan->tile_m) * (2 * I / 256);
  plan->tail_kernel = FP8B_KERNEL_NONE;
  plan->cu_count = cus;
  return FP8B_OK;
}

extern "C" int fp8b_gate_up_silu_quant(const void* A, int64_t lda, const void* B, int64_t ldb,
                                       const float* As, int64_t as_sm, int64_t as_sk,
                                       const float* Bs, int64_t bs_sn, int64_t bs_sk, void* q,
                                       int64_t ldq, float* s, int64_t s_stride_m,
                                       int64_t s_stride_g, int64_t M, int64_t I, int64_t K,
                                       void* stream) {
  if (M < 0 || I < 0 || K < 0 || lda < K || ldb < K || ldq < I) {
    set_error("fp8b_gate_up_silu_quant: bad dims (need M,I,K >= 0, lda,ldb >= K, ldq >= I)");
    return FP8B_ERR_DIMS;
  }
  if (I % 128 != 0 || K % 128 != 0 || K == 0) {
    set_error("fp8b_gate_up_silu_quant: I must be a multiple of 128 and K a positive "
              "multiple of 128");
    return FP8B_ERR_DIMS;
  }
  if (M == 0 || I == 0) return FP8B_OK;
  if (!A || !B || !As || !Bs || !q || !s) {
    set_error("fp8b_gate_up_silu_quant: null pointer");
    return FP8B_ERR_NULL;
  }
  const int64_t N = 2 * I;
  if (!mfma_path_ok(A, lda, B, ldb, M, N, K, 128, 128) || ldq % 8 != 0 ||
      ((uintptr_t)q & 7) != 0) {
    set_error("fp8b_gate_up_silu_quant: need 16-byte aligned A, B (lda, ldb multiples of 16) "
              "and an 8-byte aligned q with ldq a multiple of 8");
    return FP8B_ERR_ALIGN;
  }
  if (255 * std::max(lda, ldb) + K >= (int64_t(1) << 32)) {
    set_error("fp8b_gate_up_silu_quant: leading dimensions too large for 32-bit tile offsets");
    return FP8B_ERR_DIMS;
  }
  GemmArgs a;
  a.A = (const uint8_t*)A; a.B = (const uint8_t*)B; a.As = As; a.Bs = Bs; a.C = q;
  a.ws = nullptr;
  a.lda = lda; a.ldb = ldb; a.as_sm = as_sm; a.as_sk = as_sk; a.bs_sn = bs_sn; a.bs_sk = bs_sk;
  a.ldc = ldq; a.M = (int)M; a.N = (int)N; a.K = (int)K; a.KB = (int)(K / 128);
  a.kb_per_split = a.KB;
  const bool tile192 = gate_up_tile192(M, I, K, device_cu_count());
  a.tiles_m = (int)(tile192 ? (M + 191) / 192 : (M + 255) / 256);
  a.tiles_n = (int)(N / 256);
  a.out_dtype = FP8B_BF16;
  a.vec_store = 0;
  Operands o;
  o.lda = lda;
  o.ldb = ldb;
  o.mfma = true;
  o.scales = as_sk == 1 && bs_sk == 1 && as_sm % 4 == 0 && bs_sn % 4 == 0 &&
             ((uintptr_t)As & 15) == 0 && ((uintptr_t)Bs & 15) == 0;
  a.win4 = win16_ok(o, K, 1, a.KB) ? 0 : 1;
  a.rem_base = -1; a.rem_tiles_m = 0; a.rem_tiles_n = 0;
  a.Sq = s; a.sq_sm = s_stride_m; a.sq_sg = s_stride_g;
  const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
  if (tiles >= (int64_t(1) << 31)) {
    set_error("fp8b_gate_up_silu_quant: too many tiles");
    return FP8B_ERR_DIMS;
  }
  if (tile192)
    gemm_pipe192_kernel<true><<<(unsigned)tiles, 512, 0, (hipStream_t)stream>>>(a);
  else
    gemm_pipe256_kernel<false, true><<<(unsigned)tiles, 512, 0, (hipStream_t)stream>>>(a);
  if (hipGetLastError() != hipSuccess) {
    set_error("fp8b_gate_up_silu_quant: kernel launch failed");
    return FP8B_ERR_LAUNCH;
  }
  return FP8B_OK;
}
