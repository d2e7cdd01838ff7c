// fp16 GEMM with f32 accumulation for gfx950: C[M,N] = A[M,K] · B[N,K]ᵀ.
//
// Stands in for the resident fp16 matmul of the reference
// (crates/rocket-npu/src/matmul/context.rs:497-513, run.rs:244/571): both
// operands are K-contiguous (activations [M,K], HF weights [N,K]), which is
// the MFMA operand order, so no transpose or repack is needed.
//
// Design
//   * Workgroup tile BM×BN on WM×WN waves; each wave owns a (BM/WM)×(BN/WN)
//     block of v_mfma_f32_16x16x32_f16 tiles (the 16x16x32 form sustains a
//     higher fraction of the fp16 peak on gfx950 than 32x32x16).
//   * The K loop advances 64 values per stage. An ST-deep LDS ring holds one
//     stage per slot: BM + BN rows of 128 bytes, filled by buffer→LDS copies
//     of 8 whole rows (full 128-byte lines) per instruction, with no VGPR
//     staging. Rows past M/N and chunks past K are read at an out-of-range
//     offset, which the buffer unit returns as zeros, so ragged edges need no
//     extra code.
//   * Chunk c (16 bytes) of row r sits at chunk c ^ (r & 7). A fragment read
//     (16 rows, 4 chunks) is then free of LDS bank conflicts: measured on
//     MI355X with SQ_LDS_BANK_CONFLICT for both sub-steps' chunk sets, while
//     the unswizzled layout costs 12 and a (r & 7) ^ ((r >> 3) & 1) swizzle
//     4 conflict cycles per ds_read_b128.
//   * A stage is two MFMA sub-steps of 32 K-values. Sub-step 0's MFMAs run
//     while sub-step 1's fragments are read; then the next stage is waited
//     for (one barrier per stage), the slot of the stage just read is
//     refilled at once (ST-2 stages of copy latency hidden), and sub-step 1's
//     MFMAs run while the next stage's first fragments are read (two
//     register sets).
//   * The MFMA computes Cᵀ tiles (B fragment as the A operand), so a lane
//     holds four consecutive columns of one row of C: 8-byte stores.
//   * Split-K (ksplit > 1): the K stages of a tile are divided between
//     ksplit workgroups. Each stores its f32 partial tile with device-coherent
//     (sc1) 16-byte stores and counts its arrival; the workgroup that arrives
//     last sums the partials in split order (0, 1, ...: the result does not
//     depend on which finishes last), resets the count and runs the epilogue.
//     No workgroup waits for another. Grids that fill less than a round of
//     the CUs, or whose tiles are too small to keep the MFMAs fed from LDS,
//     trade the partials' traffic for more and larger tiles.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace {
constexpr int KS = 64;    // K values per stage
constexpr int ROWB = 128;  // bytes per LDS row of one stage
}  // namespace

// MLP glue of a gate|up product, in f32 in the reference's operation order
// with no FMA contraction (host.rs:12-39): 1 silu(g)·u, 2 gelu_tanh(g)·u.
template <int GLU>
__device__ __forceinline__ float f16_glu(float g, float u) {
#pragma clang fp contract(off)
  if constexpr (GLU == 1) {
    const float sigmoid = 1.0f / (1.0f + expf(-g));
    return g * sigmoid * u;
  } else {
    constexpr float k = (float)(1.12837916709551257390 * 0.70710678118654752440);  // sqrt(2/pi)
    const float inner = (g + g * g * g * 0.044715f) * k;
    return ((g * (tanhf(inner) + 1.0f)) * 0.5f) * u;
  }
}

// GLU = 0: C [M, N] fp16. GLU = 1 / 2: B holds gate and up rows interleaved
// per 16 (rows 32t..32t+15 gate rows 16t.., rows 32t+16.. the matching up
// rows), so tiles j (even) and j+1 of a lane hold gate and up of the same
// outputs; each is rounded to fp16 as the plain GEMM's output would be, the
// glue runs in f32, and C is [M, n_out] f32 (OUT_F16: fp16).
// SPLIT = false is the unsplit kernel (ksplit must be 1): the partial
// exchange is compiled out, and with it the registers it holds.
template <int BM, int BN, int WM, int WN, int ST, int MINW, int GLU = 0, bool OUT_F16 = true,
          bool SPLIT = false>
__global__ __launch_bounds__(WM *WN * 64, MINW) void gemm_f16_kernel(
    const f16 *__restrict__ A, const f16 *__restrict__ B, void *__restrict__ Cv, int M, int N, int K,
    int tiles_m, int tiles_n, int group_m, int n_out, int ksplit, float *__restrict__ part,
    unsigned *__restrict__ cnt) {
  constexpr int NW = WM * WN;
  constexpr int STAGE = (BM + BN) * ROWB;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  // One stage is A_INS + B_INS copies of 8 rows; wave w issues A copies w,
  // w + NW, ... and B copies likewise: LA of A then L - LA of B, the same
  // count on every wave and known at compile time, so the issue is straight
  // scalar code with no branches.
  constexpr int A_INS = BM / 8, B_INS = BN / 8;
  static_assert(A_INS % NW == 0 && B_INS % NW == 0, "copies split evenly over the waves");
  constexpr int LA = A_INS / NW;
  constexpr int L = (A_INS + B_INS) / NW;
  static_assert(TM * 16 * WM == BM && TN * 16 * WN == BN, "mfma split");
  static_assert(ST >= 2 && (ST - 1) * L <= 63, "pipeline depth");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tm, tn;
  // Split kj of tile `tile`: consecutive workgroup ids (one XCD's run) take
  // consecutive tiles of one split, so an XCD's L2 holds one K range of them.
  const int n_tiles = tiles_m * tiles_n;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int ks = SPLIT ? ksplit : 1;
  const int kj = SPLIT ? bid / n_tiles : 0, tile = bid - kj * n_tiles;
  tile_coords(tile, tiles_m, tiles_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT_ALL = (K + KS - 1) / KS;
  const int s_begin = SPLIT ? (int)((int64_t)KT_ALL * kj / ks) : 0;
  const int KT = SPLIT ? (int)((int64_t)KT_ALL * (kj + 1) / ks) - s_begin : KT_ALL;  // stages of this split

  const rsrc_t ra = make_rsrc(A + (size_t)m0 * K, (int64_t)min(M - m0, BM) * K * 2);
  const rsrc_t rb = make_rsrc(B + (size_t)n0 * K, (int64_t)min(N - n0, BN) * K * 2);

  // Copy geometry: copy q covers rows 8q..8q+7; lane → row r = 8q + lane/8,
  // physical chunk lane%8, which holds logical chunk (lane%8) ^ (r & 7) =
  // (lane%8) ^ (lane/8) for every q.
  const int crow = lane >> 3;
  const int lch = (lane & 7) ^ crow;
  const uint32_t voff0 = (uint32_t)(crow * K * 2 + lch * 16);
  const bool ktail = (K % KS) != 0;

  // Copies of stage s; stages past the end copy zeros (into a slot no later
  // stage reads), which keeps the loop body free of branches.
  auto issue = [&](int s) {
    uint8_t *sb = smem + (s % ST) * STAGE;
    const int k0 = (s_begin + s) * KS;
    const bool past = s >= KT;
    const uint32_t v0 = (past || (ktail && k0 + lch * 8 >= K)) ? OOB_OFFSET : voff0;
    static_for<L>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      if constexpr (I < LA) {
        const int q = wave + NW * I;  // wave-uniform
        bdma16(ra, sb + q * 1024, v0, (uint32_t)((q * 8 * K + k0) * 2));
      } else {
        const int q = wave + NW * (I - LA);
        bdma16(rb, sb + BM * ROWB + q * 1024, v0, (uint32_t)((q * 8 * K + k0) * 2));
      }
    });
  };

  // Fragment reads: lane → row lane%16 of a 16-row tile, K chunk 4·kk + lane/16.
  const int wm = wave / WN, wn = wave % WN;
  const int frow = lane & 15;
  const int ff = frow & 7;
  const uint32_t fch0 = (uint32_t)((((lane >> 4)) ^ ff) << 4);      // sub-step 0
  const uint32_t fch1 = (uint32_t)((((lane >> 4) + 4) ^ ff) << 4);  // sub-step 1
  const uint32_t a_row = (uint32_t)((wm * WTM + frow) * ROWB);
  const uint32_t b_row = (uint32_t)(BM * ROWB + (wn * WTN + frow) * ROWB);

  half8 fa[2][TM], fb[2][TN];
  auto load_frags = [&](auto buf_c, int s, uint32_t fch) {
    constexpr int BUF = decltype(buf_c)::value;
    const uint8_t *base = smem + (s % ST) * STAGE;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[BUF][i] = *(const half8 *)(base + a_row + fch + i * 16 * ROWB);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[BUF][j] = *(const half8 *)(base + b_row + fch + j * 16 * ROWB);
  };

  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  constexpr int T = TM * TN;
  auto mfmas = [&](auto buf_c) {
    constexpr int BUF = decltype(buf_c)::value;
    static_for<T>([&](auto u_c) {
      constexpr int U = decltype(u_c)::value, I = U / TN, J = U % TN;
      acc[I][J] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[BUF][J], fa[BUF][I], acc[I][J], 0, 0, 0);
    });
  };
  // One MFMA, one copy; one MFMA, one fragment read; then the rest.
  auto interleave = [&](auto ncopy_c) {
    constexpr int NC = decltype(ncopy_c)::value;
    if constexpr (T >= NC + TM + TN) {
      static_for<NC>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      });
      static_for<TM + TN>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      });
      __builtin_amdgcn_sched_group_barrier(0x008, T - NC - TM - TN, 0);
    }
  };

  // Prologue: stages 0..ST-1 in flight, stage 0 visible, its first fragments read.
#pragma unroll
  for (int s = 0; s < ST; ++s) issue(s);
  WAIT_VMCNT((ST - 1) * L);
  BARRIER();
  load_frags(ic<0>{}, 0, fch0);

  for (int s = 0; s < KT; ++s) {
    // Sub-step 0 (register set 0) while sub-step 1's fragments are read.
    load_frags(ic<1>{}, s, fch1);
    mfmas(ic<0>{});
    interleave(ic<0>{});
    __builtin_amdgcn_sched_barrier(0);
    // Stage s+1 visible to all waves (stages up to s+ST-1 were issued), and
    // every wave's reads of stage s complete: its slot is refilled at once
    // with stage s+ST, so a copy has ST-2 full stages to land. Sub-step 1 runs
    // while stage s+1's first fragments are read (past the last stage: stale,
    // unused).
    WAIT_VMCNT((ST - 2) * L);
    WAIT_LGKMCNT0();
    BARRIER();
    issue(s + ST);
    load_frags(ic<0>{}, s + 1, fch0);
    mfmas(ic<1>{});
    interleave(ic<L>{});
    __builtin_amdgcn_sched_barrier(0);
  }
  WAIT_VMCNT(0);  // no copy may still be writing LDS when the workgroup ends

  if constexpr (SPLIT) {
    // Partial slot of split j: [wave][tile u][lane] 16-byte entries.
    constexpr int SC1 = 16;  // cache policy bit: device scope
    constexpr uint32_t SLOT = (uint32_t)BM * BN * 4;
    const rsrc_t rp = make_rsrc(part + (size_t)tile * ksplit * BM * BN, (int64_t)ksplit * SLOT);
    const uint32_t lane_off = (uint32_t)((wave * T * 64 + lane) * 16);
    static_for<T>([&](auto u_c) {
      constexpr int U = decltype(u_c)::value, I = U / TN, J = U % TN;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4, acc[I][J]), rp,
                                             lane_off + (uint32_t)kj * SLOT + U * 1024, 0, SC1);
    });
    WAIT_VMCNT(0);  // the partial is stored before the arrival count
    WAIT_LGKMCNT0();
    BARRIER();  // every LDS read of the stages is done: the first word is free
    unsigned *flag = (unsigned *)smem;
    if (threadIdx.x == 0) {
      const unsigned prev = atomicAdd(cnt + tile, 1u);
      const unsigned last = prev == (unsigned)(ksplit - 1);
      if (last) atomicExch(cnt + tile, 0u);  // every split is in: reset for the next launch
      *flag = last;
      WAIT_LGKMCNT0();
    }
    BARRIER();
    if (!*flag) return;
    // The sum runs in split order: sum = p0 + p1 + ... (this split's own
    // partial from its registers); each split's loads are all issued before
    // the first add.
    floatx4 sum[TM][TN];
    for (int i = 0; i < ksplit; ++i) {
      floatx4 v[TM][TN];
      if (i == kj) {
        static_for<T>([&](auto u_c) {
          constexpr int U = decltype(u_c)::value, I = U / TN, J = U % TN;
          v[I][J] = acc[I][J];
        });
      } else {
        static_for<T>([&](auto u_c) {
          constexpr int U = decltype(u_c)::value, I = U / TN, J = U % TN;
          v[I][J] = __builtin_bit_cast(
              floatx4, __builtin_amdgcn_raw_buffer_load_b128(rp, lane_off + (uint32_t)i * SLOT + U * 1024, 0, SC1));
        });
      }
      static_for<T>([&](auto u_c) {
        constexpr int U = decltype(u_c)::value, I = U / TN, J = U % TN;
        sum[I][J] = i == 0 ? v[I][J] : sum[I][J] + v[I][J];
      });
    }
    static_for<T>([&](auto u_c) {
      constexpr int U = decltype(u_c)::value, I = U / TN, J = U % TN;
      acc[I][J] = sum[I][J];
    });
  }

  // Epilogue: lane holds C[row lane%16][cols 4·(lane/16) + 0..3] of each tile.
  if constexpr (GLU != 0) {
    static_assert(TN % 2 == 0 && WTN % 32 == 0, "gate/up tile pairs start at 32-row groups");
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + wm * WTM + i * 16 + frow;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < TN; j += 2) {
        // output column of element e: 16·(group) + 4·(lane/16) + e
        const int oc = ((n0 + wn * WTN + j * 16) >> 1) + 4 * (lane >> 4);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float g = (float)(f16)acc[i][j][e], u = (float)(f16)acc[i][j + 1][e];
          y[e] = f16_glu<GLU>(g, u);
        }
        if constexpr (OUT_F16) {
          f16 *crow_p = (f16 *)Cv + (size_t)m * n_out;
          if ((n_out % 4) == 0 && oc + 3 < n_out) {
            *(half4 *)(crow_p + oc) = half4{(f16)y[0], (f16)y[1], (f16)y[2], (f16)y[3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (oc + e < n_out) crow_p[oc + e] = (f16)y[e];
          }
        } else {
          float *crow_p = (float *)Cv + (size_t)m * n_out;
          if ((n_out % 4) == 0 && oc + 3 < n_out) {
            *(floatx4 *)(crow_p + oc) = floatx4{y[0], y[1], y[2], y[3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (oc + e < n_out) crow_p[oc + e] = y[e];
          }
        }
      }
    }
    return;
  }
  f16 *C = (f16 *)Cv;
  const bool vec = (N % 4) == 0;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WTM + i * 16 + frow;
    if (m >= M) continue;
    f16 *crow_p = C + (size_t)m * N;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * WTN + j * 16 + 4 * (lane >> 4);
      const half4 h = {(f16)acc[i][j][0], (f16)acc[i][j][1], (f16)acc[i][j][2], (f16)acc[i][j][3]};
      if (vec && n + 3 < N) {
        *(half4 *)(crow_p + n) = h;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < N) crow_p[n + e] = h[e];
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int ST, int MINW, int GLU = 0, bool OUT_F16 = true>
static hipError_t launch_gemm_f16(const f16 *A, const f16 *B, void *C, int M, int N, int K,
                                  int ksplit, float *part, unsigned *cnt, hipStream_t st, int n_out = 0) {
  constexpr int smem = ST * (BM + BN) * ROWB;
  static_assert(smem <= 160 * 1024, "LDS per workgroup");
  auto kern = ksplit > 1 ? gemm_f16_kernel<BM, BN, WM, WN, ST, MINW, GLU, OUT_F16, true>
                         : gemm_f16_kernel<BM, BN, WM, WN, ST, MINW, GLU, OUT_F16, false>;
  static bool attr_set[2] = {false, false};
  if (!attr_set[ksplit > 1]) {
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    attr_set[ksplit > 1] = true;
  }
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  // Tiles in groups of 3 tile rows (row-fastest inside a group): one XCD's
  // run of consecutive tiles then shares a few A row-blocks instead of
  // streaming all of A (vision fc2 2394x4304x1152: 40.6 -> 37.3 us on MI355X,
  // 185 MB fetched per launch row-fastest over the whole grid).
  hipLaunchKernelGGL(kern, dim3(tm * tn * ksplit), dim3(WM * WN * 64), smem, st, A, B, C, M, N, K, tm, tn,
                     rk_knob("RK_TILE_GROUP_M", 3), n_out, ksplit, part, cnt);
  return hipGetLastError();
}

namespace {
// Tile configurations: workgroup tile, workgroups per CU that fit in LDS, and
// the fraction of a CU's fp16 MFMA peak one tile sustains once running
// (fitted to every configuration timed on MI355X on the vision-layer and
// 512x1024x3072 shapes at K ~ 1-4k; the chooser then picks the fastest
// measured configuration for each of those five shapes).
struct F16Cfg {
  int bm, bn, per_cu;
  float eff;
};
constexpr F16Cfg F16_CFGS[] = {
    {256, 128, 1, .40f}, {192, 192, 1, .38f}, {128, 128, 1, .32f}, {128, 64, 2, .26f},
    {64, 64, 2, .27f},   {128, 256, 1, .41f}, {96, 128, 1, .27f},  {128, 192, 1, .34f},
    {192, 128, 1, .35f}, {64, 128, 2, .25f},  {192, 192, 1, .41f}, {192, 192, 1, .42f},
    {128, 128, 1, .33f}, {128, 192, 1, .36f}, {192, 128, 1, .42f}, {128, 192, 2, .36f},
    {192, 128, 2, .36f}, {128, 96, 1, .27f},  {128, 96, 2, .22f},  {128, 128, 2, .30f},
    {96, 128, 2, .22f},  {256, 192, 1, .42f}, {256, 192, 1, .425f}, {64, 96, 2, .26f},
};
constexpr int N_F16_CFGS = sizeof(F16_CFGS) / sizeof(F16_CFGS[0]);

hipError_t launch_cfg(int c, const f16 *a, const f16 *b, f16 *d, int M, int N, int K, int ks, float *part,
                      unsigned *cnt, hipStream_t st) {
  switch (c) {
    case 0: return launch_gemm_f16<256, 128, 4, 2, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 1: return launch_gemm_f16<192, 192, 2, 2, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 2: return launch_gemm_f16<128, 128, 2, 2, 4, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 3: return launch_gemm_f16<128, 64, 2, 2, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 4: return launch_gemm_f16<64, 64, 2, 2, 4, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 5: return launch_gemm_f16<128, 256, 2, 4, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 6: return launch_gemm_f16<96, 128, 2, 2, 4, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 7: return launch_gemm_f16<128, 192, 2, 2, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 8: return launch_gemm_f16<192, 128, 2, 2, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 9: return launch_gemm_f16<64, 128, 2, 2, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 10: return launch_gemm_f16<192, 192, 2, 4, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 11: return launch_gemm_f16<192, 192, 4, 2, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 12: return launch_gemm_f16<128, 128, 2, 4, 4, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 13: return launch_gemm_f16<128, 192, 2, 4, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 14: return launch_gemm_f16<192, 128, 4, 2, 3, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 15: return launch_gemm_f16<128, 192, 2, 4, 2, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 16: return launch_gemm_f16<192, 128, 4, 2, 2, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 17: return launch_gemm_f16<128, 96, 2, 2, 4, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 18: return launch_gemm_f16<128, 96, 2, 2, 2, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 19: return launch_gemm_f16<128, 128, 2, 2, 2, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 20: return launch_gemm_f16<96, 128, 2, 2, 2, 2>(a, b, d, M, N, K, ks, part, cnt, st);
    case 21: return launch_gemm_f16<256, 192, 2, 4, 2, 1>(a, b, d, M, N, K, ks, part, cnt, st);
    case 22: return launch_gemm_f16<256, 192, 4, 2, 2, 1>(a, b, d, M, N, K, ks, part, cnt, st);
    // 512x1024x3072 as one 64x96 tile per CU: 7.6-7.9 us against 7.9-8.2 us for 64x64 tiles
    case 23: return launch_gemm_f16<64, 96, 2, 2, 4, 2>(a, b, d, M, N, K, ks, part, cnt, st);
  }
  return hipErrorInvalidValue;
}

// The configurations whose waves hold whole 32-row gate|up groups (BN/WN a
// multiple of 32), the ones the glue epilogue is instantiated for.
constexpr int F16_GLU_CFGS[] = {0, 1, 2, 3, 4, 8, 22};

// Estimated time of configuration c with its K stages split over ks
// workgroups: rounds of workgroups over the CUs, each round a fixed ~3 us
// (launch, pipeline fill, output store) plus the work of the tiles one CU
// holds at that tile's sustained MFMA efficiency; a split adds its partial
// tiles' store and load (~1 us plus their bytes at ~10 TB/s). The split
// term is optimistic: measured on MI355X, splits cost 5-20 us more than this
// on the 512x1024x3072 and vision-layer shapes and won only on fc2
// (2394x4304x1152: 36.7 us split in two against 37.9 us), so the chooser
// only considers them when RK_F16_KSPLIT asks for one.
double cfg_time(int c, int ks, int M, int N, int K, int num_cus) {
  const F16Cfg &f = F16_CFGS[c];
  const long tiles = ((M + f.bm - 1) / f.bm) * (long)((N + f.bn - 1) / f.bn);
  const long wgs = tiles * ks;
  const long slots = (long)num_cus * f.per_cu;
  const long rounds = (wgs + slots - 1) / slots;
  const long held = std::min<long>(f.per_cu, (wgs + num_cus - 1) / num_cus);
  double t = rounds * (3e-6 + held * 2.0 * f.bm * f.bn * ((double)K / ks) / (9.83e12 * f.eff));
  if (ks > 1) t += 1e-6 + (double)wgs * f.bm * f.bn * 4 * 2 / 10e12;
  return t;
}
}  // namespace

F16Plan rk_gemm_f16_plan(int M, int N, int K, int num_cus, bool glu) {
  const int stages = (K + KS - 1) / KS;
  int cfg = rk_knob("RK_F16_TILE", -1);
  const bool cfg_ok = cfg >= 0 && cfg < N_F16_CFGS &&
                      (!glu || std::find(std::begin(F16_GLU_CFGS), std::end(F16_GLU_CFGS), cfg) !=
                                   std::end(F16_GLU_CFGS));
  int ks = rk_knob("RK_F16_KSPLIT", 1);
  if (ks > stages) ks = stages;
  F16Plan p;
  double best = 1e300;
  for (int c = 0; c < N_F16_CFGS; ++c) {
    if (cfg_ok && c != cfg) continue;
    if (glu && std::find(std::begin(F16_GLU_CFGS), std::end(F16_GLU_CFGS), c) == std::end(F16_GLU_CFGS))
      continue;
    for (int s = 1; s <= 4 && s <= stages; ++s) {
      if (ks >= 1 && s != ks) continue;
      const double t = cfg_time(c, s, M, N, K, num_cus);
      if (t < best) {
        best = t;
        p.cfg = c;
        p.ksplit = s;
      }
    }
  }
  if (p.ksplit > 1) {
    const F16Cfg &f = F16_CFGS[p.cfg];
    const int64_t tiles = (int64_t)((M + f.bm - 1) / f.bm) * ((N + f.bn - 1) / f.bn);
    p.part_floats = tiles * p.ksplit * f.bm * f.bn;
    p.n_cnt = tiles;
  }
  return p;
}

hipError_t rk_launch_gemm_f16(const F16Plan &p, const void *A, const void *B, void *C, int M, int N, int K,
                              float *part, unsigned *cnt, hipStream_t st) {
  return launch_cfg(p.cfg, (const f16 *)A, (const f16 *)B, (f16 *)C, M, N, K, p.ksplit, part, cnt, st);
}

namespace {
template <int GLU, bool OUT_F16>
hipError_t launch_glu_cfg(int c, const f16 *a, const f16 *b, void *d, int M, int N, int K, int n_out, int ks,
                          float *part, unsigned *cnt, hipStream_t st) {
  switch (c) {
    case 0: return launch_gemm_f16<256, 128, 4, 2, 3, 2, GLU, OUT_F16>(a, b, d, M, N, K, ks, part, cnt, st, n_out);
    case 1: return launch_gemm_f16<192, 192, 2, 2, 3, 2, GLU, OUT_F16>(a, b, d, M, N, K, ks, part, cnt, st, n_out);
    case 2: return launch_gemm_f16<128, 128, 2, 2, 4, 2, GLU, OUT_F16>(a, b, d, M, N, K, ks, part, cnt, st, n_out);
    case 3: return launch_gemm_f16<128, 64, 2, 2, 3, 2, GLU, OUT_F16>(a, b, d, M, N, K, ks, part, cnt, st, n_out);
    case 4: return launch_gemm_f16<64, 64, 2, 2, 4, 2, GLU, OUT_F16>(a, b, d, M, N, K, ks, part, cnt, st, n_out);
    case 8: return launch_gemm_f16<192, 128, 2, 2, 3, 2, GLU, OUT_F16>(a, b, d, M, N, K, ks, part, cnt, st, n_out);
    case 22: return launch_gemm_f16<256, 192, 4, 2, 2, 1, GLU, OUT_F16>(a, b, d, M, N, K, ks, part, cnt, st, n_out);
  }
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t rk_launch_gemm_f16_glu(const F16Plan &p, const void *A, const void *B, void *C, int M, int N, int K,
                                  int n_out, int glu, bool out_f16, float *part, unsigned *cnt, hipStream_t st) {
  const f16 *a = (const f16 *)A, *b = (const f16 *)B;
  const int c = p.cfg, ks = p.ksplit;
  if (glu == 1)
    return out_f16 ? launch_glu_cfg<1, true>(c, a, b, C, M, N, K, n_out, ks, part, cnt, st)
                   : launch_glu_cfg<1, false>(c, a, b, C, M, N, K, n_out, ks, part, cnt, st);
  if (glu == 2)
    return out_f16 ? launch_glu_cfg<2, true>(c, a, b, C, M, N, K, n_out, ks, part, cnt, st)
                   : launch_glu_cfg<2, false>(c, a, b, C, M, N, K, n_out, ks, part, cnt, st);
  return hipErrorInvalidValue;
}
