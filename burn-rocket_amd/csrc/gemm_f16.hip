// fp16 GEMM with f32 accumulation for gfx950: C[M,N] = A[M,K] · B[N,K]ᵀ.
//
// Stands in for the resident fp16 matmul of the reference
// (crates/rocket-npu/src/matmul/context.rs:497-513, run.rs:244/571): both
// operands are K-contiguous (activations [M,K], HF weights [N,K]), which is
// the natural MFMA operand order, so no transpose or repack is needed.
//
// Design
//   * Workgroup tile BM×BN, K-step 64, WM×WN waves; each wave owns a
//     (BM/WM)×(BN/WN) block of v_mfma_f32_16x16x32_f16 tiles.
//   * A STAGES-deep LDS ring is filled with global_load_lds_dwordx4 (one
//     16-byte chunk per lane, no VGPR staging). A stage holds BM + BN rows of
//     128 bytes; chunk c of row r sits at chunk c ^ (r & 7), so the eight rows
//     read by consecutive lanes of an MFMA fragment load hit distinct banks.
//   * One barrier per K-step: wait for this stage's copies (vmcnt), barrier,
//     refill the stage consumed in the previous step, compute.
//   * Rows past M/N are clamped (their results are never stored); chunks past
//     K read a zero block so the tail contributes nothing.
#include "common.hpp"
#include "kernels.hpp"

template <int BM, int BN, int WM, int WN, int STAGES>
__global__ __launch_bounds__(WM *WN * 64) void gemm_f16_nt_kernel(
    const f16 *__restrict__ A, const f16 *__restrict__ B, f16 *__restrict__ C,
    int M, int N, int K, int tiles_m) {
  constexpr int NW = WM * WN;
  constexpr int BK = 64;
  constexpr int ROWB = BK * 2;
  constexpr int STAGE_BYTES = (BM + BN) * ROWB;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int A_PER = BM / 8 / NW, B_PER = BN / 8 / NW;
  constexpr int L = A_PER + B_PER;
  static_assert(A_PER * 8 * NW == BM && B_PER * 8 * NW == BN, "tile/wave split");
  static_assert(TM * 16 * WM == BM && TN * 16 * WN == BN, "mfma split");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int tm = bid % tiles_m, tn = bid / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = (K + BK - 1) / BK;

  // DMA sources: lane covers row 8·instr + lane/8, physical chunk lane%8,
  // which holds logical chunk (lane%8) ^ (lane/8).
  const int r8 = lane >> 3;
  const int lchunk = (lane & 7) ^ r8;
  const f16 *a_src[A_PER];
  const f16 *b_src[B_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    int row = (wave * A_PER + i) * 8 + r8;
    int gm = min(m0 + row, M - 1);
    a_src[i] = A + (size_t)gm * K + lchunk * 8;
  }
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    int row = (wave * B_PER + i) * 8 + r8;
    int gn = min(n0 + row, N - 1);
    b_src[i] = B + (size_t)gn * K + lchunk * 8;
  }

  auto issue = [&](int kt) {
    uint8_t *sb = smem + (kt % STAGES) * STAGE_BYTES;
    const int k0 = kt * BK;
    const bool in = (k0 + lchunk * 8) < K;
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      dma16(in ? (const void *)(a_src[i] + k0) : (const void *)g_zero_chunk,
            sb + (wave * A_PER + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_PER; ++i)
      dma16(in ? (const void *)(b_src[i] + k0) : (const void *)g_zero_chunk,
            sb + BM * ROWB + (wave * B_PER + i) * 1024);
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int wm = wave / WN, wn = wave % WN;
  const int frow = lane & 15, fgrp = lane >> 4;

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KT) issue(s);

  for (int kt = 0; kt < KT; ++kt) {
    const int ahead = min(STAGES - 2, KT - 1 - kt);
    if (ahead >= 2 && STAGES >= 4) {
      WAIT_VMCNT(L * 2);
    } else if (ahead == 1) {
      WAIT_VMCNT(L);
    } else {
      WAIT_VMCNT(0);
    }
    WAIT_LGKMCNT0();
    BARRIER();
    if (kt + STAGES - 1 < KT) issue(kt + STAGES - 1);

    const uint8_t *sa = smem + (kt % STAGES) * STAGE_BYTES;
    const uint8_t *sbm = sa + BM * ROWB;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int c = kk * 4 + fgrp;
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        int row = wm * WTM + i * 16 + frow;
        af[i] = *(const half8 *)(sa + row * ROWB + ((c ^ (row & 7)) << 4));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        int row = wn * WTN + j * 16 + frow;
        bf[j] = *(const half8 *)(sbm + row * ROWB + ((c ^ (row & 7)) << 4));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue: lane holds C[row = 4·(lane/16) + r][col = lane%16] of each tile.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * WTN + j * 16 + frow;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * WTM + i * 16 + fgrp * 4 + r;
        if (m < M && n < N) C[(size_t)m * N + n] = (f16)acc[i][j][r];
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int STAGES>
static hipError_t launch_gemm_f16(const f16 *A, const f16 *B, f16 *C, int M, int N,
                                  int K, hipStream_t st) {
  constexpr int smem = STAGES * (BM + BN) * 128;
  auto kern = gemm_f16_nt_kernel<BM, BN, WM, WN, STAGES>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  hipLaunchKernelGGL(kern, dim3(tm * tn), dim3(WM * WN * 64), smem, st, A, B, C, M, N, K, tm);
  return hipGetLastError();
}

// Tile choice: the largest tile that still gives at least one workgroup per
// CU; small problems fall back to 64-row tiles.
hipError_t rk_launch_gemm_f16(const void *A, const void *B, void *C, int M, int N, int K,
                              int num_cus, hipStream_t st) {
  const f16 *a = (const f16 *)A;
  const f16 *b = (const f16 *)B;
  f16 *c = (f16 *)C;
  const long t128 = ((M + 127) / 128) * (long)((N + 127) / 128);
  if (t128 >= num_cus) return launch_gemm_f16<128, 128, 2, 2, 3>(a, b, c, M, N, K, st);
  const long t64x96 = ((M + 63) / 64) * (long)((N + 95) / 96);
  if (N % 96 == 0 && t64x96 >= num_cus / 2)
    return launch_gemm_f16<64, 96, 2, 2, 4>(a, b, c, M, N, K, st);
  return launch_gemm_f16<64, 64, 2, 2, 4>(a, b, c, M, N, K, st);
}
