// W8A8 / GGUF Q8_0 GEMM for gfx950 on int8 MFMA with exact int32 accumulators.
//
// Replaces the group-wise int8 resident context of the reference
// (crates/rocket-npu/src/matmul/int8.rs:644-676 matmul_gw, drain int8.rs:708-746,
// detile_accum_i8_scaled layout.rs:504-540) and its raw int32 form
// (I8Context::matmul, int8.rs:606-640).
//
//   a  int8 [M, K]  activation codes          (row-major, K-contiguous)
//   w  int8 [N, K]  weight codes              (row-major, K-contiguous)
//   ws f32  [N, KBp] weight scale per 32-value block (a K-group of 32·gb values
//                   repeats its scale over its gb blocks; KBp = K/32 rounded
//                   up to a multiple of 4, zero padded)
//   P_g[m,n] = Σ_{k in group g} a[m,k]·w[n,k]   exact int32
//
// Modes (template parameter MODE):
//   PER_TOKEN  c[m,n] = as[m] · Σ_g ws[n,g]·P_g        (per-token activations)
//   PER_GROUP  c[m,n] = Σ_g (as[m,g]·ws[n,g])·P_g      (reference matmul_gw)
//   RAW        c[m,n] = Σ_k a[m,k]·w[n,k]   as int32  (exact)
//   PARTIALS   p[m,n,g] = P_g                 as int32  (exactness checks)
//
// One v_mfma_i32_32x32x32_i8 covers exactly one 32-value block, so the int32
// result of a group is complete after gb MFMAs and is folded into an f32
// accumulator by one convert and one FMA per element; that epilogue is VALU
// work proportional to M·N·K/32 and bounds the kernel below the int8 MFMA
// peak. The lane that holds column n of an MFMA tile holds it for all 16 of
// its rows, so ws[n,g] is one LDS read per lane per tile.
//
// Pipeline: a STAGES-deep LDS ring filled by global_load_lds (16-byte chunks
// for codes, 4-byte elements for scales); a stage is 128 K-values (4 blocks).
// Code rows are 128 bytes with chunk c of row r at chunk c ^ (r & 7).
#include "common.hpp"
#include "kernels.hpp"

enum { MODE_PER_TOKEN = 0, MODE_PER_GROUP = 1, MODE_RAW = 2, MODE_PARTIALS = 3 };

__device__ __forceinline__ void dma4(const void *gsrc, void *lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, LDS_PTR(lds_base), 4, 0, 0);
}

template <int BM, int BN, int WM, int WN, int STAGES, int MODE, bool OUT_F16, bool GB1>
__global__ __launch_bounds__(WM *WN * 64) void gemm_i8_kernel(
    const int8_t *__restrict__ A, const float *__restrict__ AS, int as_stride, int a_gb,
    const int8_t *__restrict__ W, const float *__restrict__ WS, int ws_stride, int gb,
    void *__restrict__ Cout, int M, int N, int K, int tiles_m) {
  constexpr int NW = WM * WN;
  constexpr int ROWB = 128;  // 128 int8 K-values per stage row
  constexpr bool HAS_WS = (MODE == MODE_PER_TOKEN || MODE == MODE_PER_GROUP);
  constexpr bool HAS_AS = (MODE == MODE_PER_GROUP);
  constexpr int CODE_BYTES = (BM + BN) * ROWB;
  constexpr int WS_BYTES = HAS_WS ? BN * 16 : 0;
  constexpr int AS_BYTES = HAS_AS ? BM * 16 : 0;
  constexpr int STAGE_BYTES = CODE_BYTES + WS_BYTES + AS_BYTES;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int A_PER = BM / 8 / NW, B_PER = BN / 8 / NW;
  constexpr int WS_PER = HAS_WS ? (BN * 4 / 64) / NW : 0;
  constexpr int AS_PER = HAS_AS ? (BM * 4 / 64) / NW : 0;
  constexpr int L = A_PER + B_PER + WS_PER + AS_PER;
  static_assert(A_PER * 8 * NW == BM && B_PER * 8 * NW == BN, "tile/wave split");
  static_assert(!HAS_WS || WS_PER * 64 * NW == BN * 4, "scale split");
  static_assert(!HAS_AS || AS_PER * 64 * NW == BM * 4, "scale split");
  static_assert(TM * 32 * WM == BM && TN * 32 * WN == BN, "mfma split");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int tm = bid % tiles_m, tn = bid / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = (K + 127) / 128;
  const int KB = K / 32;

  const int r8 = lane >> 3;
  const int lchunk = (lane & 7) ^ r8;
  const int8_t *a_src[A_PER];
  const int8_t *b_src[B_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    int row = (wave * A_PER + i) * 8 + r8;
    a_src[i] = A + (size_t)min(m0 + row, M - 1) * K + lchunk * 16;
  }
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    int row = (wave * B_PER + i) * 8 + r8;
    b_src[i] = W + (size_t)min(n0 + row, N - 1) * K + lchunk * 16;
  }
  // Scale DMA: element e = 64·instr + lane of the [rows][4] stage tile.
  const float *ws_src[WS_PER > 0 ? WS_PER : 1];
  const float *as_row[AS_PER > 0 ? AS_PER : 1];
  int as_blk[AS_PER > 0 ? AS_PER : 1];
#pragma unroll
  for (int i = 0; i < WS_PER; ++i) {
    int e = (wave * WS_PER + i) * 64 + lane;
    ws_src[i] = WS + (size_t)min(n0 + e / 4, N - 1) * ws_stride + (e & 3);
  }
#pragma unroll
  for (int i = 0; i < AS_PER; ++i) {
    int e = (wave * AS_PER + i) * 64 + lane;
    as_row[i] = AS + (size_t)min(m0 + e / 4, M - 1) * as_stride;
    as_blk[i] = e & 3;
  }

  auto issue = [&](int kt) {
    uint8_t *sb = smem + (kt % STAGES) * STAGE_BYTES;
    const int k0 = kt * 128;
    const bool in = (k0 + lchunk * 16) < K;
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      dma16(in ? (const void *)(a_src[i] + k0) : (const void *)g_zero_chunk,
            sb + (wave * A_PER + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_PER; ++i)
      dma16(in ? (const void *)(b_src[i] + k0) : (const void *)g_zero_chunk,
            sb + BM * ROWB + (wave * B_PER + i) * 1024);
#pragma unroll
    for (int i = 0; i < WS_PER; ++i)
      dma4(ws_src[i] + kt * 4, sb + CODE_BYTES + (wave * WS_PER + i) * 256);
#pragma unroll
    for (int i = 0; i < AS_PER; ++i) {
      int blk = min(kt * 4 + as_blk[i], KB - 1);
      dma4(as_row[i] + blk / a_gb, sb + CODE_BYTES + WS_BYTES + (wave * AS_PER + i) * 256);
    }
  };

  const int wm = wave / WN, wn = wave % WN;
  const int fcol = lane & 31, fh = lane >> 5;

  // Integer accumulators (one group) and f32 accumulators.
  intx16 iacc[TM][TN];
  floatx16 facc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        iacc[i][j][r] = 0;
        facc[i][j][r] = 0.f;
      }
    }

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KT) issue(s);

  int gcount = 0;  // blocks folded into iacc since the last epilogue
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
    const float *sws = (const float *)(sa + CODE_BYTES);
    const float *sas = (const float *)(sa + CODE_BYTES + WS_BYTES);
    const int nblk = min(4, KB - kt * 4);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (b >= nblk) break;
      const int c = 2 * b + fh;
      intx4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        int row = wm * WTM + i * 32 + fcol;
        af[i] = *(const intx4 *)(sa + row * ROWB + ((c ^ (row & 7)) << 4));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        int row = wn * WTN + j * 32 + fcol;
        bf[j] = *(const intx4 *)(sbm + row * ROWB + ((c ^ (row & 7)) << 4));
      }
      // With one block per group every MFMA starts from zero (inline constant
      // C operand); otherwise the group's blocks accumulate in iacc.
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if constexpr (GB1)
            iacc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], intx16{}, 0, 0, 0);
          else
            iacc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], iacc[i][j], 0, 0, 0);
        }

      if constexpr (MODE == MODE_PARTIALS) {
        const int g = kt * 4 + b;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn * WTN + j * 32 + fcol;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int m = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
              if (m < M && n < N) ((int32_t *)Cout)[((size_t)m * N + n) * KB + g] = iacc[i][j][r];
            }
          }
      } else if constexpr (HAS_WS) {
        if (GB1 || ++gcount == gb) {
          gcount = 0;
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const float d = sws[(wn * WTN + j * 32 + fcol) * 4 + b];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                float s = d;
                if constexpr (HAS_AS) {
                  const int row = wm * WTM + i * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
                  s = sas[row * 4 + b] * d;
                }
                facc[i][j][r] = __builtin_fmaf((float)iacc[i][j][r], s, facc[i][j][r]);
                if constexpr (!GB1) iacc[i][j][r] = 0;
              }
            }
          }
        }
      }
    }
  }

  // Epilogue: lane holds rows 8·(r/4) + 4·(lane/32) + r%4, column lane%32.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * WTN + j * 32 + fcol;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
        if (m >= M || n >= N) continue;
        if constexpr (MODE == MODE_RAW) {
          ((int32_t *)Cout)[(size_t)m * N + n] = iacc[i][j][r];
        } else if constexpr (MODE == MODE_PER_TOKEN) {
          const float v = AS[(size_t)m * as_stride] * facc[i][j][r];
          if constexpr (OUT_F16)
            ((f16 *)Cout)[(size_t)m * N + n] = (f16)v;
          else
            ((float *)Cout)[(size_t)m * N + n] = v;
        } else if constexpr (MODE == MODE_PER_GROUP) {
          if constexpr (OUT_F16)
            ((f16 *)Cout)[(size_t)m * N + n] = (f16)facc[i][j][r];
          else
            ((float *)Cout)[(size_t)m * N + n] = facc[i][j][r];
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int STAGES, int MODE, bool OUT_F16, bool GB1>
static hipError_t launch_i8(const I8GemmArgs &g, hipStream_t st) {
  constexpr bool HAS_WS = (MODE == MODE_PER_TOKEN || MODE == MODE_PER_GROUP);
  constexpr bool HAS_AS = (MODE == MODE_PER_GROUP);
  constexpr int smem =
      STAGES * ((BM + BN) * 128 + (HAS_WS ? BN * 16 : 0) + (HAS_AS ? BM * 16 : 0));
  auto kern = gemm_i8_kernel<BM, BN, WM, WN, STAGES, MODE, OUT_F16, GB1>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  hipLaunchKernelGGL(kern, dim3(tm * tn), dim3(WM * WN * 64), smem, st, g.A, g.AS,
                     g.as_stride, g.a_gb, g.W, g.WS, g.ws_stride, g.gb, g.C, g.M, g.N,
                     g.K, tm);
  return hipGetLastError();
}

template <int MODE, bool OUT_F16, bool GB1>
static hipError_t dispatch_i8(const I8GemmArgs &g, hipStream_t st) {
  const long t128 = ((g.M + 127) / 128) * (long)((g.N + 127) / 128);
  if (t128 >= g.num_cus) return launch_i8<128, 128, 2, 2, 3, MODE, OUT_F16, GB1>(g, st);
  return launch_i8<64, 64, 2, 2, 4, MODE, OUT_F16, GB1>(g, st);
}

template <int MODE>
static hipError_t dispatch_scaled(const I8GemmArgs &g, hipStream_t st) {
  if (g.gb == 1)
    return g.out_f16 ? dispatch_i8<MODE, true, true>(g, st) : dispatch_i8<MODE, false, true>(g, st);
  return g.out_f16 ? dispatch_i8<MODE, true, false>(g, st) : dispatch_i8<MODE, false, false>(g, st);
}

hipError_t rk_launch_gemm_i8(const I8GemmArgs &g, hipStream_t st) {
  switch (g.mode) {
    case I8_PER_TOKEN:
      return dispatch_scaled<MODE_PER_TOKEN>(g, st);
    case I8_PER_GROUP:
      return dispatch_scaled<MODE_PER_GROUP>(g, st);
    case I8_RAW:
      return dispatch_i8<MODE_RAW, false, false>(g, st);
    case I8_PARTIALS:
      return launch_i8<64, 64, 2, 2, 4, MODE_PARTIALS, false, true>(g, st);
  }
  return hipErrorInvalidValue;
}
