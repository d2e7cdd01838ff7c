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
//   PER_GROUP  c[m,n] = Σ_g (as[m,g]·ws[n,g])·P_g      (reference matmul_gw;
//              group 32 on both sides runs on gemm_i8_q8_kernel below)
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
#include <type_traits>
#include <utility>

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

// ---------------------------------------------------------------------------
// Pipelined kernel for the two hot modes: per-token activations against a
// weight with one scale per 32-value block (GGUF Q8_0, group 32), and the raw
// int32 product. Compared with gemm_i8_kernel above it
//   * moves tiles with buffer→LDS copies whose K offset is a scalar, and whose
//     range check zero-fills rows past M/N (no per-stage vector address math);
//   * computes each lane's LDS fragment addresses once: stage, tile and block
//     offsets are instruction immediates (the K loop is unrolled over the
//     STAGES·4 blocks of the LDS ring);
//   * swizzles 16-byte chunks with (row >> 1) & 7, which keeps the 16 lanes of
//     each ds_read_b128 phase on distinct banks;
//   * prefetches the next block's fragments into a second register set and
//     interleaves every MFMA with the 32 VALU instructions (16 cvt + 16 fma)
//     that fold the previous tile's int32 block result into the f32
//     accumulator.
// The fold is 2 VALU instructions per output element and block (4 cycles
// each, wave64) against 32 cycles per 32x32x32 MFMA for 1024 elements, so the
// scaled mode is VALU-bound at 1/4 of the int8 MFMA rate.
// ---------------------------------------------------------------------------

// MLP glue applied to column pairs in the epilogue (GLU_SILU: silu(g)·u,
// GLU_GELU: gelu_tanh(g)·u, the formulas of host.rs:12-39 in f32 without FMA
// contraction). The weight rows come interleaved in 16-row groups, gate rows
// 16q..16q+15 at 32q..32q+15 and the matching up rows at 32q+16..32q+31, so
// in a 32-column MFMA tile lane l (l%32 < 16) holds a gate value and lane
// l+16 the up value of the same output (row m, column 16q + l%32).
enum { GLU_NONE = 0, GLU_SILU = 1, GLU_GELU = 2 };
template <int GLU>
__device__ __forceinline__ float glu_apply(float g, float u) {
#pragma clang fp contract(off)
  if constexpr (GLU == GLU_SILU) {
    const float sigmoid = 1.0f / (1.0f + expf(-g));
    return g * sigmoid * u;
  } else {
    constexpr float k = (float)(1.12837916709551257390 * 0.70710678118654752440);  // sqrt(2/pi)
    const float inner = (g + g * g * g * 0.044715f) * k;
    return ((g * (tanhf(inner) + 1.0f)) * 0.5f) * u;
  }
}

template <int BM, int BN, int WM, int WN, int STAGES, int MODE, bool OUT_F16, int MINW = 2,
          int GLU = GLU_NONE, bool WSF16 = false, int KG = 1>
__global__ __launch_bounds__(KG *WM *WN * 64, MINW) void gemm_i8_q8_kernel(
    const int8_t *__restrict__ A, const float *__restrict__ AS, const int8_t *__restrict__ W,
    const float *__restrict__ WS, int ws_stride, void *__restrict__ Cout, int M, int N, int K,
    int tiles_m, int tiles_n, int group_m, int n_out, int as_stride) {
  static_assert(MODE == MODE_PER_TOKEN || MODE == MODE_PER_GROUP || MODE == MODE_RAW,
                "per-token, per-group or raw");
  constexpr int NW = WM * WN;  // waves of one K-group
  constexpr int NT = KG * NW * 64;
  constexpr int ROWB = 128;  // K bytes of one stage row
  constexpr bool GROUPED = (MODE == MODE_PER_GROUP);
  // KG K-groups of NW waves each: group k walks stages [k·KT, (k+1)·KT) of the
  // tile's K range with its own LDS ring, and the groups' partial sums meet
  // in LDS at the end (group 0's first). A tile then keeps 4·KG waves per
  // SIMD busy on its own, which is what a lone workgroup (a grid of about
  // one tile per CU, or the last round of a larger one) lacks.
  static_assert(KG == 1 || !GROUPED, "K-groups: per-token and raw modes");
  constexpr bool SCALED = (MODE == MODE_PER_TOKEN) || GROUPED;
  constexpr int CODE_BYTES = (BM + BN) * ROWB;
  constexpr int WS_BYTES = SCALED ? BN * 16 : 0;
  constexpr int STAGE_BYTES = CODE_BYTES + WS_BYTES;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  // Copies of 8 code rows (1 KiB) per stage: QA for A, QB for B, dealt
  // round-robin to the waves (wave w issues copies w, w+NW, ...); QMIN is
  // the smallest number any wave issues.
  constexpr int QA = BM / 8, QB = BN / 8, QT = QA + QB;
  constexpr int CP = (QT + NW - 1) / NW, QMIN = QT / NW;
  constexpr int WS_INS = SCALED ? BN / 64 : 0;            // 64 scale rows per copy
  static_assert(QA % 2 == 0, "A copies keep the swizzle parity of B copies");
  static_assert(WS_INS <= NW && (!SCALED || WS_INS * 64 == BN), "scale split");
  static_assert(TM * 32 * WM == BM && TN * 32 * WN == BN, "mfma split");
  // Per-group activation scales as[m, g] of a stage (4 blocks) sit in their
  // own ring of STAGES + 1 slots, [block][row], filled by 4-byte copies
  // (AS_INS of 64 per stage): a slot outlives its stage's code slot, which is
  // refilled while the last block's last tile is still to be folded. One row
  // of 32 tiles per wave (TM = 1) keeps one 16-row scale set in registers,
  // shared by the wave's TN column tiles.
  constexpr int AS_SLOT = GROUPED ? BM * 16 : 0;
  constexpr int AS_INS = GROUPED ? BM * 4 / 64 : 0;
  static_assert(!GROUPED || TM == 1, "per-group mode: one row of 32x32 tiles per wave");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float *s_as = (float *)(smem + KG * STAGES * STAGE_BYTES);  // [BM] per-token activation scales
  uint8_t *s_asg = smem + STAGES * STAGE_BYTES;               // per-group ring (GROUPED)

  const int lane = lane_id();
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave_all / NW;    // K-group
  const int wave = wave_all % NW;   // wave within its K-group
  uint8_t *const gsm = smem + grp * STAGES * STAGE_BYTES;  // the group's LDS ring
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, gridDim.x), tiles_m, tiles_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // Stages (128 K-values) of this group; with KG > 1 the host guarantees
  // K % (128·KG) == 0, so each group has KT whole stages.
  const int KT = ((K + 127) / 128) / KG;
  const int kt0 = grp * KT;  // the group's first stage
  const int KB = K / 32;
  const int NBLK = KG == 1 ? KB : 4 * KT;  // blocks the main loop steps through

  const rsrc_t ra = make_rsrc(A + (size_t)m0 * K, (int64_t)(M - m0) * K);
  const rsrc_t rw = make_rsrc(W + (size_t)n0 * K, (int64_t)(N - n0) * K);
  const rsrc_t rs = make_rsrc(SCALED ? WS + (size_t)n0 * ws_stride : WS, (int64_t)(N - n0) * ws_stride * 4);

  // Copy geometry: lane covers tile row 8·q + lane/8 and physical chunk lane%8,
  // which holds logical chunk (lane%8) ^ ((row >> 1) & 7); the swizzle depends
  // on the parity of q only.
  const int r8 = lane >> 3, p8 = lane & 7;
  const uint32_t voff_even = r8 * K + ((p8 ^ (r8 >> 1)) << 4);
  const uint32_t voff_odd = r8 * K + ((p8 ^ (4 + (r8 >> 1))) << 4);
  const uint32_t voff_ws = lane * ws_stride * 4;
  // per-group scale copy c: float f = 64c + lane of the slot = (block f / BM, row f % BM)
  const rsrc_t ras = make_rsrc(GROUPED ? AS + (size_t)m0 * as_stride : AS,
                               GROUPED ? (int64_t)(M - m0) * as_stride * 4 : 0);
  auto as_voff = [&](int c) -> uint32_t {
    const int f = 64 * c + lane;
    return (uint32_t)(((f % BM) * as_stride + f / BM) * 4);
  };

  if constexpr (MODE == MODE_PER_TOKEN) {
    for (int r = threadIdx.x; r < BM; r += NT) s_as[r] = AS[min(m0 + r, M - 1)];
  }

  auto issue = [&](auto slot_c, int kt) {
    constexpr int slot = decltype(slot_c)::value;
    uint8_t *sb = gsm + slot * STAGE_BYTES;
    const uint32_t k0 = (kt0 + kt) * 128;
#pragma unroll
    for (int i = 0; i < CP; ++i) {
      const int q = wave + i * NW;  // wave-uniform
      if (CP * NW == QT || q < QT) {
        const uint32_t voff = (q & 1) ? voff_odd : voff_even;
        if (q < QA)
          bdma16(ra, sb + q * 1024, voff, q * 8 * K + k0);
        else
          bdma16(rw, sb + BM * ROWB + (q - QA) * 1024, voff, (q - QA) * 8 * K + k0);
      }
    }
    if constexpr (WS_INS > 0) {
      if (wave < WS_INS)
        bdma16(rs, sb + CODE_BYTES + wave * 1024, voff_ws, wave * 64 * ws_stride * 4 + (kt0 + kt) * 16);
    }
    if constexpr (AS_INS > 0) {
      // from the last wave down, away from the waves that copy weight scales
      uint8_t *ab = s_asg + (kt % (STAGES + 1)) * AS_SLOT;
#pragma unroll
      for (int c = 0; c < AS_INS; ++c)
        if (wave == NW - 1 - c % NW)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(ras, LDS_PTR(ab + c * 256), 4, as_voff(c),
                                                   (uint32_t)(kt * 16), 0, 0);
    }
  };
  // Make stage kt visible to every wave. Copies return in issue order, so
  // waiting until at most QMIN·later copies (the stages issued after kt)
  // remain is enough for every wave, also those that issue more copies per
  // stage (code rows or scales): they wait for a few later copies as well.
  auto stage_ready = [&](int kt) {
    if constexpr (STAGES >= 3) {
      const int later = min(STAGES - 2, KT - 1 - kt);
      if (later >= 2) {
        WAIT_VMCNT(QMIN * 2);
      } else if (later == 1) {
        WAIT_VMCNT(QMIN);
      } else {
        WAIT_VMCNT(0);
      }
    } else {
      WAIT_VMCNT(0);
    }
    WAIT_LGKMCNT0();
    BARRIER();
  };

  const int wm = wave / WN, wn = wave % WN;
  const int fcol = lane & 31, fh = lane >> 5;
  const int swz = (fcol >> 1) & 7;
  uint32_t a_off[4], b_off[4];  // lane's fragment byte offsets per block (stage 0)
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t ch = (uint32_t)(((2 * b + fh) ^ swz) << 4);
    a_off[b] = (wm * WTM + fcol) * ROWB + ch;
    b_off[b] = BM * ROWB + (wn * WTN + fcol) * ROWB + ch;
  }
  const uint32_t s_off = CODE_BYTES + (wn * WTN + fcol) * 16;
  // lane's 16 rows of a 32-row tile: 8·q + 4·(lane/32) + 0..3, q = 0..3
  const uint32_t asg_off = (uint32_t)((wm * WTM + fh * 4) * 4);
  floatx4 as_pend[4];  // per-group scales of the block whose tile is folded next
#pragma unroll
  for (int q = 0; q < 4; ++q) as_pend[q] = floatx4{0.f, 0.f, 0.f, 0.f};
  auto load_as = [&](floatx4(&dst)[4], int g) {
    const uint8_t *ab = s_asg + ((g >> 2) % (STAGES + 1)) * AS_SLOT + (g & 3) * BM * 4 + asg_off;
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = *(const floatx4 *)(ab + q * 32);
  };

  intx4 af[2][TM], bf[2][TN];
  float dsc[2][TN];
  // The column's 4 weight scales of a stage, read with one 16-byte LDS read
  // at the stage's first block (4-byte reads at a 16-byte lane stride would
  // conflict on the banks).
  floatx4 wsq[TN];
  auto load_frags = [&](auto buf_c, auto slot_c, auto b_c) {
    constexpr int buf = decltype(buf_c)::value, slot = decltype(slot_c)::value,
                  b = decltype(b_c)::value;
    const uint8_t *base = gsm + slot * STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < TM; ++i) af[buf][i] = *(const intx4 *)(base + a_off[b] + i * 32 * ROWB);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      bf[buf][j] = *(const intx4 *)(base + b_off[b] + j * 32 * ROWB);
      if constexpr (SCALED) {
        if constexpr (b == 0) wsq[j] = *(const floatx4 *)(base + s_off + j * 32 * 16);
        dsc[buf][j] = wsq[j][b];
      }
    }
  };

  intx16 iacc[TM][TN];
  floatx16 facc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        facc[i][j][r] = 0.f;
        iacc[i][j][r] = 0;
      }

  issue(ic<0>{}, 0);
  if constexpr (STAGES > 2) {
    if (1 < KT) issue(ic<1>{}, 1);
  }
  stage_ready(0);
  if (STAGES - 1 < KT) issue(ic<STAGES - 1>{}, STAGES - 1);
  load_frags(ic<0>{}, ic<0>{}, ic<0>{});

  // Scaled mode software pipeline. The block results of the T = TM·TN tiles
  // are produced into two alternating register sets (ires) and each is folded
  // one MFMA later: MFMA(u+1) is issued before the 32 VALU instructions that
  // fold tile u, so the MFMA of the next tile runs while the VALU folds the
  // previous one. The pending tile of a block is folded at the start of the
  // next block. sched_barrier(0) fences keep this issue order. Tile u of
  // block B (B = block index mod 4) uses set (B·T + u) & 1; a loop iteration
  // covers 4·STAGES blocks, an even count, so the sets alternate across
  // iterations too.
  constexpr int T = TM * TN;
  intx16 ires[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) ires[0][r] = ires[1][r] = 0;
  float dpend = 0.f;  // scale of the pending tile (the last tile of the previous block)
  // Per-group mode with fp16 weight scales (WSF16): each MFMA starts from the
  // int32 bits of 1.5·2^23 (GBIAS_BITS), so its result read as a float is
  // exactly 1.5·2^23 + P_g (|P_g| < 2^19); fma(F, d, -1.5·2^23·d) is then
  // P_g·d rounded once (an fp16 d makes 1.5·2^23·d exact), and a second FMA
  // applies as[m, g]: two VALU operations per element and block instead of a
  // convert, a multiply and an FMA. Other scales take the latter.
  constexpr bool BIASED = GROUPED && WSF16;
  constexpr int GBIAS_BITS = 0x4B400000;
  constexpr float GBIAS = 12582912.0f;
  intx16 cinit;
#pragma unroll
  for (int r = 0; r < 16; ++r) cinit[r] = BIASED ? GBIAS_BITS : 0;
  auto fold = [&](auto p_c, auto i_c, auto j_c, float d, const floatx4(&asr)[4]) {
    constexpr int P = decltype(p_c)::value, I = decltype(i_c)::value, J = decltype(j_c)::value;
    if constexpr (GROUPED && !WSF16) {
      // (as[m, g] · ws[n, g]) · P_g, the reference's order (emu_matmul_gw)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        facc[I][J][r] = __builtin_fmaf((float)ires[P][r], asr[r >> 2][r & 3] * d, facc[I][J][r]);
    } else if constexpr (GROUPED) {
      const float nbd = -GBIAS * d;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int bits = ires[P][r];  // element to a scalar first (ext-vector bit_cast)
        const float y = __builtin_fmaf(__int_as_float(bits), d, nbd);
        facc[I][J][r] = __builtin_fmaf(y, asr[r >> 2][r & 3], facc[I][J][r]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) facc[I][J][r] = __builtin_fmaf((float)ires[P][r], d, facc[I][J][r]);
    }
  };

  // Block step: global block g sits at slot S, block B of its stage, and uses
  // register set CUR (= B parity).
  auto step = [&](int g, auto s_c, auto b_c) {
    constexpr int S = decltype(s_c)::value, B = decltype(b_c)::value;
    constexpr int CUR = B & 1, NXT = CUR ^ 1;
    constexpr int NS = (B == 3) ? (S + 1) % STAGES : S, NB = (B + 1) & 3;
    const int gn = g + 1;
    if constexpr (B == 3) {
      if (gn < NBLK) {
        const int kt = gn >> 2;
        stage_ready(kt);
        if (kt + STAGES - 1 < KT) issue(ic<S>{}, kt + STAGES - 1);
      }
    }
    if constexpr (MODE == MODE_RAW) {
      // The prefetch of block g+1 is unconditional (past the last block it
      // reads stale, in-bounds LDS that is never used) so that it shares a
      // scheduling region with the MFMAs below.
      load_frags(ic<NXT>{}, ic<NS>{}, ic<NB>{});
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          iacc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[CUR][i], bf[CUR][j], iacc[i][j], 0, 0, 0);
    } else {
      // Tile 0 of this block first: its wait covers only the fragments read
      // in the previous step. Then the next block's fragments are read from
      // LDS (register set NXT is free: its MFMAs were all issued in the
      // previous step) and have a whole step to arrive, then the fold of the
      // previous block's last tile.
      constexpr int P0 = (B * T) & 1;
      const float dlast = dsc[CUR][TN - 1];
      ires[P0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[CUR][0], bf[CUR][0], cinit, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      load_frags(ic<NXT>{}, ic<NS>{}, ic<NB>{});
      __builtin_amdgcn_sched_barrier(0);
      fold(ic<P0 ^ 1>{}, ic<TM - 1>{}, ic<TN - 1>{}, dpend, as_pend);
      // the scales of this block's tile, folded in the next step
      if constexpr (GROUPED) load_as(as_pend, g);
      __builtin_amdgcn_sched_barrier(0);
      // Tiles 1..T-1: MFMA of tile u, then the fold of tile u-1.
      static_for<T - 1>([&](auto uc) {
        constexpr int u = decltype(uc)::value + 1;
        constexpr int I = u / TN, J = u % TN;
        constexpr int PI = (u - 1) / TN, PJ = (u - 1) % TN;
        ires[(P0 + u) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[CUR][I], bf[CUR][J], cinit, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        fold(ic<(P0 + u - 1) & 1>{}, ic<PI>{}, ic<PJ>{}, dsc[CUR][PJ], as_pend);
        __builtin_amdgcn_sched_barrier(0);
      });
      dpend = dlast;
    }
  };

  for (int g0 = 0; g0 < NBLK; g0 += 4 * STAGES) {
    auto stage = [&](auto s_c) {
      const int gs = g0 + 4 * decltype(s_c)::value;
      if (gs + 0 < NBLK) step(gs + 0, s_c, ic<0>{});
      if (gs + 1 < NBLK) step(gs + 1, s_c, ic<1>{});
      if (gs + 2 < NBLK) step(gs + 2, s_c, ic<2>{});
      if (gs + 3 < NBLK) step(gs + 3, s_c, ic<3>{});
    };
    stage(ic<0>{});
    if constexpr (STAGES > 1) stage(ic<1>{});
    if constexpr (STAGES > 2) stage(ic<2>{});
  }
  if constexpr (SCALED) {
    // The last block's last tile sits in set ((NBLK-1)·T + T-1) & 1.
    if (((NBLK * T - 1) & 1) != 0)
      fold(ic<1>{}, ic<TM - 1>{}, ic<TN - 1>{}, dpend, as_pend);
    else
      fold(ic<0>{}, ic<TM - 1>{}, ic<TN - 1>{}, dpend, as_pend);
  }

  if constexpr (KG > 1) {
    // Group 1 hands its partial sums to group 0 through LDS ([wave][tile]
    // [element][lane], lane-contiguous 4-byte words: conflict-free), and
    // group 0 adds them to its own: (first half of K) + (second half).
    static_assert(KG == 2, "two K-groups");
    static_assert(NW * T * 16 * 64 * 4 <= KG * STAGES * STAGE_BYTES, "exchange fits the rings");
    WAIT_VMCNT(0);
    WAIT_LGKMCNT0();
    BARRIER();  // every wave is past its last read of the rings
    float *xf = (float *)smem + wave * (T * 16 * 64) + lane;
    if (grp == 1) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int u = (i * TN + j) * 16 + r;
            if constexpr (MODE == MODE_RAW)
              xf[u * 64] = __int_as_float(iacc[i][j][r]);
            else
              xf[u * 64] = facc[i][j][r];
          }
    }
    WAIT_LGKMCNT0();
    BARRIER();
    if (grp == 1) return;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int u = (i * TN + j) * 16 + r;
          if constexpr (MODE == MODE_RAW)
            iacc[i][j][r] += __float_as_int(xf[u * 64]);
          else
            facc[i][j][r] = facc[i][j][r] + xf[u * 64];
        }
  }

  // Epilogue: lane holds rows 8·(r/4) + 4·(lane/32) + r%4 of column lane%32.
  // f32 and int32 outputs use non-temporal stores: written through rather than left
  // dirty in L2 for the end-of-kernel write-back (MI355X, M=3633 up / down
  // projections: 1.5-2 us of ~35 us). fp16 stores fill half lines and stay
  // ordinary.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    floatx4 as4[4];
    if constexpr (MODE == MODE_PER_TOKEN) {
#pragma unroll
      for (int q = 0; q < 4; ++q) as4[q] = *(const floatx4 *)(s_as + wm * WTM + i * 32 + q * 8 + fh * 4);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * WTN + j * 32 + fcol;
      if constexpr (GLU != GLU_NONE) {
        // gate lanes (fcol < 16) take the up value from lane + 16; output
        // column 16·(n/32) + fcol of an [M, n_out] matrix
        const int oc = ((n0 + wn * WTN + j * 32) >> 1) + fcol;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
          const float v = as4[r >> 2][r & 3] * facc[i][j][r];
          const float u = __int_as_float(
              __builtin_amdgcn_ds_bpermute((lane ^ 16) << 2, __float_as_int(v)));
          if (fcol < 16 && m < M && oc < n_out) {
            const float y = glu_apply<GLU>(v, u);
            if constexpr (OUT_F16)
              ((f16 *)Cout)[(size_t)m * n_out + oc] = (f16)y;
            else
              ((float *)Cout)[(size_t)m * n_out + oc] = y;
          }
        }
        continue;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
        if (m < M && n < N) {
          if constexpr (MODE == MODE_RAW) {
            __builtin_nontemporal_store(iacc[i][j][r], (int32_t *)Cout + (size_t)m * N + n);
          } else {
            const float v = GROUPED ? facc[i][j][r] : as4[r >> 2][r & 3] * facc[i][j][r];
            if constexpr (OUT_F16)
              ((f16 *)Cout)[(size_t)m * N + n] = (f16)v;
            else  // 32 lanes fill one 128-byte line of a row: streamed past L2
              __builtin_nontemporal_store(v, (float *)Cout + (size_t)m * N + n);
          }
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int STAGES, int MODE, bool OUT_F16, int MINW = 2,
          int GLU = GLU_NONE, bool WSF16 = false, int KG = 1>
static hipError_t launch_q8(const I8GemmArgs &g, hipStream_t st) {
  constexpr bool SCALED = MODE == MODE_PER_TOKEN || MODE == MODE_PER_GROUP;
  constexpr int smem = KG * STAGES * ((BM + BN) * 128 + (SCALED ? BN * 16 : 0)) +
                       (MODE == MODE_PER_GROUP ? (STAGES + 1) * BM * 16 : BM * 4);
  static_assert(smem <= 160 * 1024, "LDS");
  if (KG > 1 && g.K % (128 * KG) != 0) return hipErrorInvalidValue;
  auto kern = gemm_i8_q8_kernel<BM, BN, WM, WN, STAGES, MODE, OUT_F16, MINW, GLU, WSF16, KG>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  // Tiles in groups of 8 tile rows (row-fastest inside a group): one XCD's run
  // of consecutive tiles re-reads a few A row blocks from its L2 instead of
  // streaming all of A (M=3633 down-projection: 108 MB fetched per launch
  // row-fastest over the whole grid; 3-4 % faster on both projections).
  hipLaunchKernelGGL(kern, dim3(tm * tn), dim3(KG * WM * WN * 64), smem, st, g.A, g.AS, g.W, g.WS,
                     g.ws_stride, g.C, g.M, g.N, g.K, tm, tn, rk_knob("RK_TILE_GROUP_M", 8),
                     GLU != GLU_NONE ? g.n_out : g.N, g.as_stride);
  return hipGetLastError();
}

// Tile configurations of the per-token Q8_0 kernel. Default, by the number of
// 128x128 tiles against the CU count (measured on MI355X at M=3633: up
// 3072x1024 29.9 us with 10, down 1024x3072 29.4 us with 15):
//   >= 1 per CU:   128x128 tiles on 8 waves, 2 workgroups (4 waves per SIMD);
//   >= 3/4 per CU: 128x128 tiles on 16 waves, one tile per CU (4 waves per SIMD);
//   fewer:         128x64 tiles on 4 waves.
// RK_Q8_TILE selects a configuration by number.
// GLU epilogue launches: the three default configurations of launch_q8_cfg
// (below), chosen by the same tile count.
template <bool OUT_F16, int GLU>
static hipError_t launch_q8_glu(const I8GemmArgs &g, hipStream_t st) {
  const long t128 = ((g.M + 127) / 128) * (long)((g.N + 127) / 128);
  if (t128 >= g.num_cus)
    return launch_q8<128, 128, 2, 4, 2, MODE_PER_TOKEN, OUT_F16, 4, GLU>(g, st);
  if (4 * t128 >= 3L * g.num_cus)
    return launch_q8<128, 128, 4, 4, 2, MODE_PER_TOKEN, OUT_F16, 4, GLU>(g, st);
  return launch_q8<128, 64, 2, 2, 3, MODE_PER_TOKEN, OUT_F16, 2, GLU>(g, st);
}

template <bool OUT_F16>
static hipError_t launch_q8_cfg(const I8GemmArgs &g, hipStream_t st) {
  const long t128 = ((g.M + 127) / 128) * (long)((g.N + 127) / 128);
  const int dflt = t128 >= g.num_cus ? 10 : (4 * t128 >= 3L * g.num_cus ? 15 : 0);
  switch (rk_knob("RK_Q8_TILE", dflt)) {
    case 1:
      return launch_q8<128, 64, 2, 2, 3, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 2:
      return launch_q8<128, 128, 2, 2, 2, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 3:
      return launch_q8<128, 128, 2, 2, 3, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 4:
      return launch_q8<256, 64, 4, 1, 2, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 5:
      return launch_q8<64, 128, 1, 4, 3, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 6:
      return launch_q8<64, 64, 2, 1, 2, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 7:
      return launch_q8<64, 128, 2, 2, 2, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 8:
      return launch_q8<64, 64, 2, 1, 3, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 9:
      return launch_q8<64, 64, 1, 2, 2, MODE_PER_TOKEN, OUT_F16>(g, st);
    case 10:
      return launch_q8<128, 128, 2, 4, 2, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 11:
      return launch_q8<256, 128, 4, 4, 2, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 12:
      return launch_q8<128, 64, 2, 2, 2, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 13:
      return launch_q8<256, 192, 8, 2, 2, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 14:
      return launch_q8<256, 64, 8, 2, 2, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 15:
      return launch_q8<128, 128, 4, 4, 2, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 16:
      return launch_q8<192, 128, 6, 2, 2, MODE_PER_TOKEN, OUT_F16, 3>(g, st);
    case 17:
      return launch_q8<128, 192, 4, 2, 2, MODE_PER_TOKEN, OUT_F16, 2>(g, st);
    case 18:
      return launch_q8<256, 128, 8, 2, 2, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 19:
      return launch_q8<128, 128, 4, 4, 3, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 20:
      return launch_q8<256, 64, 8, 2, 3, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 21:
      return launch_q8<256, 128, 8, 2, 3, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 22:
      return launch_q8<128, 256, 4, 4, 2, MODE_PER_TOKEN, OUT_F16, 4>(g, st);
    case 23:
      return launch_q8<128, 128, 2, 4, 3, MODE_PER_TOKEN, OUT_F16, 2>(g, st);
    // two K-groups per workgroup (K % 256 == 0)
    case 24:
      return launch_q8<128, 128, 2, 4, 2, MODE_PER_TOKEN, OUT_F16, 4, GLU_NONE, false, 2>(g, st);
    case 25:
      return launch_q8<128, 128, 2, 2, 2, MODE_PER_TOKEN, OUT_F16, 2, GLU_NONE, false, 2>(g, st);
    case 26:
      return launch_q8<128, 64, 2, 2, 2, MODE_PER_TOKEN, OUT_F16, 2, GLU_NONE, false, 2>(g, st);
    case 27:
      return launch_q8<64, 128, 2, 2, 2, MODE_PER_TOKEN, OUT_F16, 2, GLU_NONE, false, 2>(g, st);
    default:
      return launch_q8<128, 64, 2, 2, 2, MODE_PER_TOKEN, OUT_F16>(g, st);
  }
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

// Group-32 activations on the pipelined kernel. Each wave owns one row of
// 32x32 tiles (its 16 activation scales per block serve every tile of the
// row). By default 128x128 tiles on 4 waves of 32x128 (7) when there are at
// least as many 128x128 tiles as CUs, else 128x64 on 4 waves of 32x64 (8):
// two workgroups per CU with up to 256 registers per wave. On MI355X at
// M=3633 the up-projection 3072x1024 takes 40.6 us with 7 against 46-49 us
// with 2 (64x128 on 8 waves of 32x32), the down-projection 1024x3072 40.4 us
// with 8 against 43.5 us. Wider wave tiles on 8 waves (3-6) spill under their
// 128-register budget. RK_Q8G_TILE selects a configuration by number.
template <bool OUT_F16, bool WSF16>
static hipError_t launch_q8g(int c, const I8GemmArgs &g, hipStream_t st) {
  if (c == 0) return launch_q8<128, 128, 4, 4, 2, MODE_PER_GROUP, OUT_F16, 4, GLU_NONE, WSF16>(g, st);
  if (c == 1) return launch_q8<128, 64, 4, 2, 2, MODE_PER_GROUP, OUT_F16, 4, GLU_NONE, WSF16>(g, st);
  if (c == 3) return launch_q8<128, 128, 4, 2, 2, MODE_PER_GROUP, OUT_F16, 4, GLU_NONE, WSF16>(g, st);
  if (c == 4) return launch_q8<128, 256, 4, 4, 2, MODE_PER_GROUP, OUT_F16, 4, GLU_NONE, WSF16>(g, st);
  if (c == 5) return launch_q8<256, 128, 8, 2, 2, MODE_PER_GROUP, OUT_F16, 4, GLU_NONE, WSF16>(g, st);
  if (c == 6) return launch_q8<64, 128, 2, 2, 2, MODE_PER_GROUP, OUT_F16, 4, GLU_NONE, WSF16>(g, st);
  if (c == 7) return launch_q8<128, 128, 4, 1, 2, MODE_PER_GROUP, OUT_F16, 2, GLU_NONE, WSF16>(g, st);
  if (c == 8) return launch_q8<128, 64, 4, 1, 2, MODE_PER_GROUP, OUT_F16, 2, GLU_NONE, WSF16>(g, st);
  if (c == 9) return launch_q8<64, 128, 2, 1, 2, MODE_PER_GROUP, OUT_F16, 2, GLU_NONE, WSF16>(g, st);
  if (c == 10) return launch_q8<128, 128, 4, 1, 3, MODE_PER_GROUP, OUT_F16, 2, GLU_NONE, WSF16>(g, st);
  return launch_q8<64, 128, 2, 4, 2, MODE_PER_GROUP, OUT_F16, 4, GLU_NONE, WSF16>(g, st);
}

hipError_t rk_launch_gemm_i8(const I8GemmArgs &g, hipStream_t st) {
  switch (g.mode) {
    case I8_PER_TOKEN:
      // One scale per 32-value block (GGUF Q8_0 / group 32): pipelined kernel.
      if (g.gb == 1) {
        if (g.glu == GLU_SILU)
          return g.out_f16 ? launch_q8_glu<true, GLU_SILU>(g, st) : launch_q8_glu<false, GLU_SILU>(g, st);
        if (g.glu == GLU_GELU)
          return g.out_f16 ? launch_q8_glu<true, GLU_GELU>(g, st) : launch_q8_glu<false, GLU_GELU>(g, st);
        return g.out_f16 ? launch_q8_cfg<true>(g, st) : launch_q8_cfg<false>(g, st);
      }
      if (g.glu != 0) return hipErrorInvalidValue;
      return dispatch_scaled<MODE_PER_TOKEN>(g, st);
    case I8_PER_GROUP:
      // Group-32 activations against a group-32 weight: pipelined kernel
      // (launch_q8g; RK_Q8G_TILE selects the tile).
      if (g.gb == 1 && g.a_gb == 1 && g.glu == 0) {
        const int knob = rk_knob("RK_Q8G_TILE", -1);
        const long t128 = ((g.M + 127) / 128) * (long)((g.N + 127) / 128);
        const int c = knob >= 0 ? knob : (t128 >= g.num_cus ? 7 : 8);
        return g.ws_f16 ? (g.out_f16 ? launch_q8g<true, true>(c, g, st) : launch_q8g<false, true>(c, g, st))
                        : (g.out_f16 ? launch_q8g<true, false>(c, g, st) : launch_q8g<false, false>(c, g, st));
      }
      return dispatch_scaled<MODE_PER_GROUP>(g, st);
    case I8_RAW: {
      // Two K-groups of waves per workgroup where the grid leaves a CU with
      // one workgroup (down-projection 3633x3072->1024: 18.6 against 19.3 us);
      // with two or more per CU the single group is faster (up-projection
      // 3633x1024->3072: 22.0 against 24.0 us). RK_Q8_RAW_TILE: 1 forces two
      // groups, 2 forces one.
      const int knob = rk_knob("RK_Q8_RAW_TILE", 0);
      const long t128 = ((g.M + 127) / 128) * (long)((g.N + 127) / 128);
      if (g.K % 256 == 0 && (knob == 1 || (knob == 0 && t128 < g.num_cus)))
        return launch_q8<128, 128, 2, 2, 2, MODE_RAW, false, 2, GLU_NONE, false, 2>(g, st);
      return launch_q8<128, 128, 2, 2, 2, MODE_RAW, false>(g, st);
    }
    case I8_PARTIALS:
      return launch_i8<64, 64, 2, 2, 4, MODE_PARTIALS, false, true>(g, st);
  }
  return hipErrorInvalidValue;
}
