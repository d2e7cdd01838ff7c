// Grouped W8A8 GEMMs for the MoE expert FFN (Q8_0 expert weights), gfx950.
//
// Stands in for the reference's expert workers (src/clef/engine_npu.rs:75-207:
// gate|up matmul_gw, silu·up on the host, down matmul_gw, one expert per NPU
// core) and the per-token combine (src/clef/engine.rs:317-338). Tokens are
// bucketed per expert on the host (engine.rs:284-313); a tile table lists
// (expert, first bucket row, rows ≤ 128) entries, and the grid is tiles × N/64.
//
// Each workgroup streams one 64-column slice of one expert's weight through a
// 3-stage LDS ring while 4 waves each hold 32 gathered token rows, so an
// expert's weight bytes leave HBM once per row chunk. Waves past the tile's
// rows still move data and pass barriers but skip the MFMAs.
//
//   gate|up: weight rows are interleaved per 64-column slice t as
//            [gate 32t..32t+31 | up 32t..32t+31], so the lane holding gate
//            column j also holds up column j and the epilogue writes
//            act = silu(xs·g) · (xs·u) directly (silu(x) = x / (1 + e^-x),
//            src/clef/model.rs:491).
//   down:    yb[row] = (as·acc) · router weight of the row.
// Codes use one v_mfma_i32_32x32x32_i8 per Q8_0 block (exact int32) and one
// convert + FMA per element and block with the block's f32 scale.
#include "common.hpp"
#include "kernels.hpp"

namespace {
constexpr int BM = 128, BN = 64, NW = 4, STAGES = 3;
constexpr int ROWB = 128;
constexpr int CODE_BYTES = (BM + BN) * ROWB;
constexpr int WS_BYTES = BN * 16;
constexpr int STAGE_BYTES = CODE_BYTES + WS_BYTES;
constexpr int A_PER = BM / 8 / NW;         // 4
constexpr int B_PER = BN / 8 / NW;         // 2
constexpr int WS_PER = BN * 4 / 64 / NW;   // 1
constexpr int L = A_PER + B_PER + WS_PER;  // 7
}  // namespace

__device__ __forceinline__ void dma4_moe(const void *gsrc, void *lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, LDS_PTR(lds_base), 4, 0, 0);
}

template <bool GU>
__global__ __launch_bounds__(NW * 64) void moe_gemm_kernel(
    const int8_t *__restrict__ A, const float *__restrict__ AS, const int32_t *__restrict__ tok,
    const MoeTile *__restrict__ tiles, const int8_t *__restrict__ W,
    const float *__restrict__ WS, int64_t w_stride_e, int64_t ws_stride_e, int ws_stride,
    int N, int K, const float *__restrict__ row_w, float *__restrict__ out, int out_ld) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const MoeTile tile = tiles[blockIdx.y];
  const int n0 = blockIdx.x * BN;
  const int KT = (K + 127) / 128;
  const int KB = K / 32;
  const int8_t *We = W + (int64_t)tile.expert * w_stride_e;
  const float *WSe = WS + (int64_t)tile.expert * ws_stride_e;

  const int r8 = lane >> 3;
  const int lchunk = (lane & 7) ^ r8;
  const int8_t *a_src[A_PER];
  const int8_t *b_src[B_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int row = min((wave * A_PER + i) * 8 + r8, tile.rows - 1);
    const int64_t src_row = GU ? (int64_t)tok[tile.row0 + row] : (int64_t)(tile.row0 + row);
    a_src[i] = A + src_row * K + lchunk * 16;
  }
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int row = (wave * B_PER + i) * 8 + r8;
    b_src[i] = We + (int64_t)min(n0 + row, N - 1) * K + lchunk * 16;
  }
  const int e_ws = wave * 64 + lane;
  const float *ws_src = WSe + (int64_t)min(n0 + e_ws / 4, N - 1) * ws_stride + (e_ws & 3);

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
    dma4_moe(ws_src + kt * 4, sb + CODE_BYTES + wave * 256);
  };

  const bool active = wave * 32 < tile.rows;
  const int fcol = lane & 31, fh = lane >> 5;
  floatx16 facc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) facc[j][r] = 0.f;

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KT) issue(s);

  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) {
      WAIT_VMCNT(L);
    } else {
      WAIT_VMCNT(0);
    }
    WAIT_LGKMCNT0();
    BARRIER();
    if (kt + STAGES - 1 < KT) issue(kt + STAGES - 1);
    if (!active) continue;

    const uint8_t *sa = smem + (kt % STAGES) * STAGE_BYTES;
    const uint8_t *sbm = sa + BM * ROWB;
    const float *sws = (const float *)(sa + CODE_BYTES);
    const int nblk = min(4, KB - kt * 4);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (b >= nblk) break;
      const int c = 2 * b + fh;
      const int arow = wave * 32 + fcol;
      const intx4 af = *(const intx4 *)(sa + arow * ROWB + ((c ^ (arow & 7)) << 4));
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int brow = j * 32 + fcol;
        const intx4 bf = *(const intx4 *)(sbm + brow * ROWB + ((c ^ (brow & 7)) << 4));
        const intx16 p = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, intx16{}, 0, 0, 0);
        const float d = sws[brow * 4 + b];
#pragma unroll
        for (int r = 0; r < 16; ++r) facc[j][r] = __builtin_fmaf((float)p[r], d, facc[j][r]);
      }
    }
  }
  if (!active) return;

#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = wave * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
    if (row >= tile.rows) continue;
    const int brow = tile.row0 + row;
    if (GU) {
      const float xs = AS[tok[brow]];
      const float g = xs * facc[0][r];
      const float u = xs * facc[1][r];
      const int col = blockIdx.x * 32 + fcol;
      out[(int64_t)brow * out_ld + col] = g / (1.0f + expf(-g)) * u;
    } else {
      const int col = n0 + fcol;
      const float v0 = AS[brow] * facc[0][r];
      const float v1 = AS[brow] * facc[1][r];
      const float w = row_w[brow];
      if (col < N) out[(int64_t)brow * out_ld + col] = v0 * w;
      if (col + 32 < N) out[(int64_t)brow * out_ld + col + 32] = v1 * w;
    }
  }
}

static hipError_t launch_moe(bool gu, const int8_t *A, const float *AS, const int32_t *tok,
                             const MoeTile *tiles, int n_tiles, const int8_t *w, const float *ws,
                             int64_t w_stride_e, int64_t ws_stride_e, int ws_stride, int N,
                             int K, const float *row_w, float *out, int out_ld,
                             hipStream_t st) {
  if (n_tiles == 0) return hipSuccess;
  constexpr int smem = STAGES * STAGE_BYTES;
  static bool attr_set[2] = {false, false};
  auto kern = gu ? moe_gemm_kernel<true> : moe_gemm_kernel<false>;
  if (!attr_set[gu]) {
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    attr_set[gu] = true;
  }
  dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)n_tiles);
  hipLaunchKernelGGL(kern, grid, dim3(NW * 64), smem, st, A, AS, tok, tiles, w, ws, w_stride_e,
                     ws_stride_e, ws_stride, N, K, row_w, out, out_ld);
  return hipGetLastError();
}

hipError_t rk_launch_moe_gemm_gu(const int8_t *xq, const float *xs, const int32_t *tok,
                                 const MoeTile *tiles, int n_tiles, const int8_t *w,
                                 const float *ws, int64_t w_stride_e, int64_t ws_stride_e,
                                 int ws_stride, int N, int K, float *act, int num_cus,
                                 hipStream_t st) {
  (void)num_cus;
  return launch_moe(true, xq, xs, tok, tiles, n_tiles, w, ws, w_stride_e, ws_stride_e, ws_stride,
                    N, K, nullptr, act, N / 2, st);
}

hipError_t rk_launch_moe_gemm_down(const int8_t *aq, const float *as, const MoeTile *tiles,
                                   int n_tiles, const int8_t *w, const float *ws,
                                   int64_t w_stride_e, int64_t ws_stride_e, int ws_stride,
                                   int N, int K, const float *row_w, float *yb, int num_cus,
                                   hipStream_t st) {
  (void)num_cus;
  return launch_moe(false, aq, as, nullptr, tiles, n_tiles, w, ws, w_stride_e, ws_stride_e,
                    ws_stride, N, K, row_w, yb, N, st);
}

// y[t] = Σ_j yb[slot_rows[t, j]] with the slots of a token already sorted by
// ascending expert id (the deterministic order of combine, engine.rs:317-338).
__global__ void moe_combine_kernel(const float *__restrict__ yb,
                                   const int32_t *__restrict__ slot_rows, int top_k, int64_t h,
                                   float *__restrict__ y) {
  const int64_t t = blockIdx.y;
  const int64_t c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (c >= h) return;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < top_k; ++j) {
    const int64_t row = slot_rows[t * top_k + j];
    const floatx4 v = *(const floatx4 *)(yb + row * h + c);
    acc[0] += v[0];
    acc[1] += v[1];
    acc[2] += v[2];
    acc[3] += v[3];
  }
  *(floatx4 *)(y + t * h + c) = acc;
}

hipError_t rk_launch_moe_combine(const float *yb, const int32_t *slot_rows, int64_t s, int top_k,
                                 int64_t h, float *y, hipStream_t st) {
  if (s == 0) return hipSuccess;
  dim3 grid((unsigned)((h / 4 + 255) / 256), (unsigned)s);
  hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, st, yb, slot_rows, top_k, h, y);
  return hipGetLastError();
}
