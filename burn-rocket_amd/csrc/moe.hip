// Grouped W8A8 GEMMs for the MoE expert FFN (Q8_0 expert weights), gfx950.
//
// Stands in for the reference's expert workers (src/clef/engine_npu.rs:75-207:
// gate|up matmul_gw, silu·up on the host, down matmul_gw, one expert per NPU
// core; the exact host twin EmuWorker, src/clef/engine.rs:990-1043) and the
// per-token combine (src/clef/engine.rs:317-338). Tokens are bucketed per
// expert on the host (engine.rs:284-313); a tile table lists (expert, first
// bucket row, rows ≤ 128) entries.
//
// Arithmetic (the reference's matmul_gw, src/clef/int8.rs:101-158): the
// activations are quantized per row per 32-value group, the Q8_0 weights
// carry one scale per 32-value block, and
//   C[m, n] = Σ_b a_s[m, b] · w_s[n, b] · P_b[m, n],  P_b exact int32,
// accumulated in f32 in block order.
//
// The expert GEMMs are HBM-bound: 128 experts of Q8_0 weights are read once
// per call while each expert sees ~64 token rows. One workgroup takes one
// tile of ≤128 rows of one expert and a slice of BN = 32·NW weight columns;
// wave w owns the 32 columns [32w, 32w+32) for every 32-row block of the
// tile, so no wave idles on short tiles (only the row blocks that hold rows
// are computed: the body is instantiated for 1..4 row blocks).
//
// No two waves read the same weight bytes, so the weight codes and scales
// go straight from HBM into registers (buffer loads, 16 bytes per lane per
// block), PD stages of 128 K-values ahead of the MFMAs: with ~4 KB per wave
// and stage that keeps the HBM pipe full. The token rows of the tile, which
// every wave reads, are gathered into a (PD+1)-slot LDS ring by buffer→LDS
// copies with per-lane row offsets (16-byte chunks, swizzled by
// (row >> 1) & 7), and next to them the rows' activation scales of the
// stage's 4 blocks, stored [block][row]; rows past the tile read as zeros.
//
// One v_mfma_i32_32x32x32_i8 covers one Q8_0 block. It starts from the int32
// bits of 1.5·2^23 (0x4B400000), so its result read as a float is exactly
// F = 1.5·2^23 + P (|P| <= 32·127² < 2^22): no int→float conversion.
//   gate|up: acc = acc + fl(fl(a_s·d)·(F - 1.5·2^23)), the reference's own
//            rounding sequence (its results are quantized again, where any
//            difference could move a code);
//   down:    two FMAs, y = fma(F, d, -1.5·2^23·d) = P·d rounded once (d = the
//            f16 weight scale widened to f32, so 1.5·2^23·d is exact), then
//            acc = fma(y, a_s, acc).
// The MFMA of row block u+1 is issued before the fold of row block u so the
// two overlap.
//
//   gate|up: weight rows are interleaved per 16-row slice t as
//            [gate 16t..16t+15 | up 16t..16t+15], so the lane holding gate
//            column j and the lane 16 above it holding up column j swap
//            through ds_bpermute and the epilogue writes
//            act = silu(g) · u, silu(v) = v / (1 + e^-v) (src/clef/model.rs:
//            491-493) with e^-v rounded once from f64 (exp_rn).
//   down:    yb[row] = acc · router weight of the row (engine.rs:649-650),
//            then the combine (engine.rs:317-338) in the same launch: every
//            workgroup counts its rows in on a per-(token, column slice)
//            arrival counter, and the workgroup whose arrival completes a
//            token's top_k rows sums them in ascending expert id into y
//            (onto y's old value in accumulate mode). No workgroup waits on
//            another, and the sum's order does not depend on which one
//            arrives last, so y is the same from call to call.
#include "common.hpp"
#include "kernels.hpp"

namespace {
constexpr int MOE_ROWB = 128;  // K bytes of one stage row
constexpr int MOE_BIAS_BITS = 0x4B400000;  // 1.5·2^23 as f32 bits
constexpr float MOE_BIAS = 12582912.0f;

// Per BM-row tile (BM = 64 or 128, the host's tile size): token-row codes of
// one stage, their scales [block 0..3][row], one LDS ring slot.
template <int BM> constexpr int moe_a_stage() { return BM * MOE_ROWB; }
template <int BM> constexpr int moe_s_stage() { return 4 * BM * 4; }
template <int BM> constexpr int moe_slot() { return moe_a_stage<BM>() + moe_s_stage<BM>(); }

// LDS: the (PD+1)-slot ring of token-row stages with their scales, then the
// router weight of each tile row, and for the combine the tokens the
// workgroup completes, their slot rows and their count.
template <int PD, int BM>
constexpr int moe_smem() {
  return (PD + 1) * moe_slot<BM>() + BM * 4 + BM * 4 + BM * 8 * 4 + 16;
}
}  // namespace

// e^x rounded once to f32: the f64 exponential (error well below half an f32
// ulp) rounded to nearest. libm's expf, which the reference's f32::exp calls,
// is correctly rounded on all but ~0.06 % of arguments, so silu·up matches it
// bit for bit almost everywhere.
__device__ __forceinline__ float exp_rn(float x) { return (float)exp((double)x); }

__device__ __forceinline__ void bdma4(rsrc_t r, void *lds_base, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, LDS_PTR(lds_base), 4, voff, soff, 0, 0);
}

template <bool GU, int NW, int PD, int BM, int NRB>
__device__ __forceinline__ void moe_body(
    const int8_t *__restrict__ A, const float *__restrict__ AS, int as_stride,
    const int32_t *__restrict__ tok, int64_t a_rows, const MoeTile &tile,
    const int8_t *__restrict__ We, const float *__restrict__ WSe, int ws_stride, int N, int K,
    int n0, const float *__restrict__ row_w, float *__restrict__ out, int out_ld, const MoeCombine &cmb,
    uint8_t *smem) {
  constexpr int ROWB = MOE_ROWB, NSLOT = PD + 1;
  constexpr int MOE_A_STAGE = moe_a_stage<BM>(), MOE_SLOT = moe_slot<BM>();
  constexpr int QA = BM / 8;     // 8-row copies of token rows per stage
  constexpr int CPA = QA / NW;   // of them per wave
  constexpr int SC = BM / 16;    // 4-byte scale copies per stage: 4 blocks × BM/64 runs of 64 rows
  constexpr int SPW = SC / NW;   // of them per wave
  constexpr int VM = CPA + 4 + 1 + SPW;  // memory ops per wave and stage
  static_assert(CPA * NW == QA && SPW * NW == SC, "copies per wave");

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KT = (K + 127) / 128;
  const int KB = K / 32;

  // Router weights for the epilogue (visible after the first stage's barrier).
  float *s_rw = (float *)(smem + NSLOT * MOE_SLOT);
  if constexpr (!GU) {
    for (int row = threadIdx.x; row < BM; row += NW * 64)
      s_rw[row] = row < tile.rows ? row_w[tile.row0 + row] : 0.f;
  }

  // Expert weights are stored fragment-major: per 32-column block cb and
  // 128-value stage kt, 4 KB = [block b][lane][16 bytes] where lane
  // 32·h + j holds W[32cb + j][32(4kt + b) + 16h .. +16], and 512 bytes of
  // scales [j][b]. A wave's load of one block is one contiguous 1 KB read.
  const int KS = ws_stride / 4;  // stages per row (blocks padded to a multiple of 4)
  const int cb0 = n0 / 32, ncb = (N + 31) / 32;
  const rsrc_t ra = make_rsrc(A, a_rows * K);
  const rsrc_t ras = make_rsrc(AS, a_rows * as_stride * 4);
  const rsrc_t rw = make_rsrc(We + (size_t)cb0 * KS * 4096, (int64_t)(ncb - cb0) * KS * 4096);
  const rsrc_t rs = make_rsrc(WSe + (size_t)cb0 * KS * 128, (int64_t)(ncb - cb0) * KS * 512);

  // Token-row copy q covers stage rows 8q..8q+7: lane → row 8q + lane/8,
  // physical chunk lane%8 holding logical chunk (lane%8) ^ ((row >> 1) & 7).
  // Scale copy c covers block c%4 of rows 64·(c/4) + lane.
  const int r8 = lane >> 3, p8 = lane & 7;
  auto src_row = [&](int row) -> int64_t {
    if (row >= tile.rows) return -1;
    return GU ? (int64_t)tok[tile.row0 + row] : (int64_t)(tile.row0 + row);
  };
  uint32_t voff_a[CPA];
#pragma unroll
  for (int i = 0; i < CPA; ++i) {
    const int q = wave + i * NW;
    const int row = 8 * q + r8;
    const uint32_t ch = (uint32_t)((p8 ^ ((row >> 1) & 7)) << 4);
    const int64_t src = src_row(row);
    voff_a[i] = src >= 0 ? (uint32_t)(src * K) + ch : OOB_OFFSET;
  }
  uint32_t voff_as[SPW];
#pragma unroll
  for (int i = 0; i < SPW; ++i) {
    const int c = wave + i * NW;
    const int64_t src = src_row(64 * (c >> 2) + lane);
    voff_as[i] = src >= 0 ? (uint32_t)((src * as_stride + (c & 3)) * 4) : OOB_OFFSET;
  }
  const int fcol = lane & 31, fh = lane >> 5;
  const uint32_t voff_w = (uint32_t)(wave * KS * 4096 + lane * 16);
  const uint32_t voff_ws = (uint32_t)(wave * KS * 512 + fcol * 16);

  intx4 bq[NSLOT][4];
  floatx4 sq[NSLOT];
  auto issue = [&](auto slot_c, int kt) {
    constexpr int slot = decltype(slot_c)::value;
    uint8_t *sb = smem + slot * MOE_SLOT;
    const uint32_t k0 = kt * 128;
#pragma unroll
    for (int i = 0; i < CPA; ++i) bdma16(ra, sb + (wave + i * NW) * 1024, voff_a[i], k0);
#pragma unroll
    for (int b = 0; b < 4; ++b)
      bq[slot][b] = __builtin_amdgcn_raw_buffer_load_b128(rw, voff_w + 1024 * b, kt * 4096, 0);
    sq[slot] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff_ws, kt * 512, 0));
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const int c = wave + i * NW;
      bdma4(ras, sb + MOE_A_STAGE + (c & 3) * (BM * 4) + (c >> 2) * 256, voff_as[i], kt * 16);
    }
  };

  const int swz = (fcol >> 1) & 7;
  uint32_t a_off[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) a_off[b] = fcol * ROWB + ((((2 * b + fh) ^ swz)) << 4);

  intx4 af[2][NRB];
  auto load_afrag = [&](auto buf_c, auto slot_c, auto b_c) {
    constexpr int buf = decltype(buf_c)::value, slot = decltype(slot_c)::value,
                  b = decltype(b_c)::value;
    const uint8_t *base = smem + slot * MOE_SLOT;
#pragma unroll
    for (int i = 0; i < NRB; ++i) af[buf][i] = *(const intx4 *)(base + a_off[b] + i * 32 * ROWB);
  };
  // Activation scales of the lane's 16 rows of row block u for block b:
  // rows 32u + 8q + 4·fh + j for register 4q + j.
  auto load_as = [&](float(&v)[16], auto slot_c, auto b_c, auto u_c) {
    constexpr int slot = decltype(slot_c)::value, b = decltype(b_c)::value,
                  u = decltype(u_c)::value;
    const float *p = (const float *)(smem + slot * MOE_SLOT + MOE_A_STAGE + b * (BM * 4)) + u * 32 + fh * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const floatx4 t = *(const floatx4 *)(p + q * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[4 * q + j] = t[j];
    }
  };

  intx16 bias;
#pragma unroll
  for (int r = 0; r < 16; ++r) bias[r] = MOE_BIAS_BITS;
  floatx16 facc[NRB];
#pragma unroll
  for (int i = 0; i < NRB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) facc[i][r] = 0.f;
  intx16 ires[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) ires[0][r] = ires[1][r] = 0;
  // The pending fold (the last row block of the previous block): its weight
  // scale, bias correction and activation scales. Zero at the start, so the
  // first pending fold adds nothing.
  float dpend = 0.f, cpend = 0.f, asp[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) asp[r] = 0.f;
  auto fold = [&](auto p_c, auto i_c, float d, float c, const float(&as)[16]) {
    constexpr int P = decltype(p_c)::value, I = decltype(i_c)::value;
    if constexpr (GU) {
      // The reference's rounding sequence, acc + fl(fl(a_s·w_s)·P): gate|up
      // results feed the next quantizer, where a one-ulp difference could move
      // an int8 code, so they are computed exactly as the reference does.
      // Written as four passes over the 16 elements, so that no step waits on
      // the one before it for the same element.
#pragma clang fp contract(off)
      float pf[16], sc[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int bits = ires[P][r];  // element to a scalar before the bit cast
        pf[r] = __int_as_float(bits) - MOE_BIAS;  // P, exact
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = as[r] * d;
#pragma unroll
      for (int r = 0; r < 16; ++r) pf[r] = sc[r] * pf[r];
#pragma unroll
      for (int r = 0; r < 16; ++r) facc[I][r] = facc[I][r] + pf[r];
    } else {
      float y[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int bits = ires[P][r];
        y[r] = __builtin_fmaf(__int_as_float(bits), d, c);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) facc[I][r] = __builtin_fmaf(y[r], as[r], facc[I][r]);
    }
  };

  // Row block u of block b (b = block index within its stage) uses result set
  // (b·NRB + u) & 1; stages hold 4 blocks, so the sets alternate across stages.
  auto block = [&](auto s_c, auto b_c) {
    constexpr int S = decltype(s_c)::value, B = decltype(b_c)::value;
    constexpr int CUR = B & 1, NXT = CUR ^ 1;
    constexpr int P0 = (B * NRB) & 1;
    const float d = sq[S][B];
    const float c = -MOE_BIAS * d;
    ires[P0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[CUR][0], bq[S][B], bias, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (B < 3) load_afrag(ic<NXT>{}, ic<S>{}, ic<B + 1>{});
    __builtin_amdgcn_sched_barrier(0);
    fold(ic<P0 ^ 1>{}, ic<NRB - 1>{}, dpend, cpend, asp);
    __builtin_amdgcn_sched_barrier(0);
    static_for<NRB - 1>([&](auto uc) {
      constexpr int u = decltype(uc)::value + 1;
      float asv[16];
      load_as(asv, ic<S>{}, ic<B>{}, ic<u - 1>{});
      ires[(P0 + u) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[CUR][u], bq[S][B], bias, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      fold(ic<(P0 + u - 1) & 1>{}, ic<u - 1>{}, d, c, asv);
      __builtin_amdgcn_sched_barrier(0);
    });
    // The slot may be refilled before the pending fold runs: its scales go to
    // registers now (the next stage's lgkmcnt wait covers these reads).
    load_as(asp, ic<S>{}, ic<B>{}, ic<NRB - 1>{});
    dpend = d;
    cpend = c;
  };

  // Stage kt is ready once at most `later` stages' memory ops (those issued
  // after it) are outstanding; then the slot of stage kt-1 is free for kt+PD.
  auto stage = [&](auto s_c, int kt) {
    constexpr int S = decltype(s_c)::value;
    const int later = min(PD - 1, KT - 1 - kt);
    if constexpr (PD >= 4) {
      if (later >= 3) {
        WAIT_VMCNT(3 * VM);
      } else if (later == 2) {
        WAIT_VMCNT(2 * VM);
      } else if (later == 1) {
        WAIT_VMCNT(VM);
      } else {
        WAIT_VMCNT(0);
      }
    } else if constexpr (PD == 3) {
      if (later >= 2) {
        WAIT_VMCNT(2 * VM);
      } else if (later == 1) {
        WAIT_VMCNT(VM);
      } else {
        WAIT_VMCNT(0);
      }
    } else {
      if (later >= 1) {
        WAIT_VMCNT(VM);
      } else {
        WAIT_VMCNT(0);
      }
    }
    WAIT_LGKMCNT0();
    BARRIER();
    if (kt + PD < KT) issue(ic<(S + PD) % NSLOT>{}, kt + PD);
    load_afrag(ic<0>{}, ic<S>{}, ic<0>{});
    // One branch per block keeps each block's MFMAs and folds in their own
    // basic block, in the issue order written here.
    const int g = kt * 4;
    block(s_c, ic<0>{});
    if (g + 1 < KB) block(s_c, ic<1>{});
    if (g + 2 < KB) block(s_c, ic<2>{});
    if (g + 3 < KB) block(s_c, ic<3>{});
  };

  static_for<PD>([&](auto s_c) {
    if (decltype(s_c)::value < KT) issue(s_c, decltype(s_c)::value);
  });
  for (int kt0 = 0; kt0 < KT; kt0 += NSLOT) {
    static_for<NSLOT>([&](auto s_c) {
      const int kt = kt0 + decltype(s_c)::value;
      if (kt < KT) stage(s_c, kt);
    });
  }
  if (((KB * NRB - 1) & 1) != 0)
    fold(ic<1>{}, ic<NRB - 1>{}, dpend, cpend, asp);
  else
    fold(ic<0>{}, ic<NRB - 1>{}, dpend, cpend, asp);
  WAIT_VMCNT(0);  // no copy may still be writing LDS when the workgroup ends

  // Epilogue: lane holds rows 8·(r/4) + 4·(lane/32) + r%4 of each 32-row
  // block, column lane%32 of the wave's 32 columns.
  const int col = n0 + wave * 32 + fcol;
  constexpr int SC1 = 16;  // cache policy bit: device scope
  const rsrc_t ryb = make_rsrc(out + (int64_t)tile.row0 * out_ld, (int64_t)tile.rows * out_ld * 4);
#pragma unroll
  for (int i = 0; i < NRB; ++i) {
    if constexpr (GU) {
      // Gate column j is in lane j, up column j in lane j + 16 (of each half
      // wave). For the row pair (r, r+1) the lower lanes finish row r and the
      // upper lanes row r+1: one swap across the 16-lane halves gives each
      // lane the gate and up values of its row, so every lane computes one
      // output.
      const bool lo = (fcol & 16) == 0;
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const int rr = lo ? r : r + 1;
        const int row = i * 32 + (rr >> 2) * 8 + fh * 4 + (rr & 3);
        const float v0 = facc[i][r], v1 = facc[i][r + 1];
        // lower lanes send the gate of row r+1, upper lanes the up of row r
        const float x = __int_as_float(
            __builtin_amdgcn_ds_bpermute((lane ^ 16) << 2, __float_as_int(lo ? v1 : v0)));
        const float g = lo ? v0 : x, u = lo ? x : v1;
        if (row < tile.rows && col < N) {
          const int c = (n0 + wave * 32) / 2 + (fcol & 15);
          out[(int64_t)(tile.row0 + row) * out_ld + c] = g / (1.0f + exp_rn(-g)) * u;
        }
      }
    } else {
      // yb rows with device-coherent (sc1) stores: the workgroup that
      // completes a token may run on another XCD, whose L2 does not see this
      // one's.
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = i * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
        if (row < tile.rows && col < N)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(facc[i][r] * s_rw[row]), ryb,
                                                (uint32_t)((row * out_ld + col) * 4), 0, SC1);
      }
    }
  }
  if constexpr (!GU) {
    // Combine (engine.rs:317-338). Once every wave's rows are stored, each
    // row of the tile counts itself in on its token's counter for this
    // column slice; the row whose count completes the token's top_k rows
    // belongs to the workgroup that sums them. It resets the counter, so
    // every launch leaves the counters at zero.
    WAIT_VMCNT(0);
    int *s_tok = (int *)(smem + NSLOT * MOE_SLOT + BM * 4);  // [BM] tokens this workgroup completes
    int *s_sl = s_tok + BM;                                  // [BM][8] their slot rows (top_k <= 8)
    int *s_n = s_sl + BM * 8;
    if (threadIdx.x == 0) *s_n = 0;
    __syncthreads();
    const int n_cs = (N + 32 * NW - 1) / (32 * NW), cs = n0 / (32 * NW);
    const int top_k = cmb.top_k;
    const bool staged = top_k <= 8;
    for (int row = threadIdx.x; row < tile.rows; row += NW * 64) {
      const int t = cmb.tok[tile.row0 + row];
      unsigned *c = cmb.cnt + (int64_t)t * n_cs + cs;
      if (atomicAdd(c, 1u) == (unsigned)top_k - 1) {
        atomicExch(c, 0u);
        const int idx = atomicAdd(s_n, 1);
        s_tok[idx] = t;
        if (staged)
          for (int j = 0; j < top_k; ++j) s_sl[idx * 8 + j] = cmb.slot[(int64_t)t * top_k + j];
      }
    }
    __syncthreads();
    // y[t] (+)= Σ_j yb[slot j of t] over the token's rows in ascending
    // expert id: 4 columns per thread, 8·NW threads per row, U rows per
    // thread at a time with every row load issued before the first add (the
    // completing workgroups are the last ones to run, so their loads are
    // the launch's tail).
    constexpr int TPR = 8 * NW, NT = NW * 64, RPI = NT / TPR, U = 4;
    const int n_last = *s_n;
    const int c = n0 + 4 * ((int)threadIdx.x % TPR);
    const int sub = (int)threadIdx.x / TPR;
    const rsrc_t rall = make_rsrc(out, a_rows * out_ld * 4);
    if (c < N) {
      if (staged) {
        // Loads past the token's top_k or past the last row read zeros
        // (offsets outside the buffer) rather than sitting under a branch,
        // which would serialise them.
        const rsrc_t ry = make_rsrc(cmb.y, (int64_t)cmb.n_tok * N * 4);
        for (int i0 = 0; i0 < n_last; i0 += U * RPI) {
          floatx4 v[U][8], y0[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int idx = i0 + u * RPI + sub;
            const bool ok = idx < n_last;
            const int ic = ok ? idx : 0;
            const intx4 sa = *(const intx4 *)(s_sl + ic * 8), sb = *(const intx4 *)(s_sl + ic * 8 + 4);
            const int tk = s_tok[ic];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const int sv = j < 4 ? sa[j & 3] : sb[j & 3];
              const uint32_t off = (ok && j < top_k) ? (uint32_t)((sv * out_ld + c) * 4) : OOB_OFFSET;
              v[u][j] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rall, off, 0, SC1));
            }
            const uint32_t yoff = (ok && cmb.accumulate) ? (uint32_t)((tk * N + c) * 4) : OOB_OFFSET;
            y0[u] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(ry, yoff, 0, 0));
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            floatx4 acc = y0[u];
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (j < top_k)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] = acc[e] + v[u][j][e];
            const int idx = i0 + u * RPI + sub;
            if (idx < n_last) *(floatx4 *)(cmb.y + (int64_t)s_tok[idx] * N + c) = acc;
          }
        }
      } else {
        for (int idx = sub; idx < n_last; idx += RPI) {
          const int t = s_tok[idx];
          const int32_t *sl = cmb.slot + (int64_t)t * top_k;
          float *yr = cmb.y + (int64_t)t * N + c;
          floatx4 acc = {0.f, 0.f, 0.f, 0.f};
          if (cmb.accumulate) acc = *(const floatx4 *)yr;
          for (int j0 = 0; j0 < top_k; j0 += 8) {
            const int nj = min(8, top_k - j0);
            floatx4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (j < nj)
                v[j] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rall, (uint32_t)((sl[j0 + j] * out_ld + c) * 4), 0, SC1));
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (j < nj)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] = acc[e] + v[j][e];
          }
          *(floatx4 *)yr = acc;
        }
      }
    }
  }
}

template <bool GU, int NW, int PD, int BM>
__global__ __launch_bounds__(NW * 64, 2) void moe_q8_kernel(
    const int8_t *__restrict__ A, const float *__restrict__ AS, int as_stride,
    const int32_t *__restrict__ tok, int64_t a_rows, const MoeTile *__restrict__ tiles, int n_col_tiles,
    const int8_t *__restrict__ W, const float *__restrict__ WS, int64_t w_stride_e,
    int64_t ws_stride_e, int ws_stride, int N, int K, const float *__restrict__ row_w,
    float *__restrict__ out, int out_ld, MoeCombine cmb) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // Tile t runs on XCD t mod 8 (the dispatcher hands workgroup b to XCD
  // b mod 8), all its column slices there, sharing the tile's token rows in
  // that XCD's L2; each XCD takes its tiles in list order, longest first (the
  // plan sorts them). For down this also spreads the last tiles, whose
  // workgroups complete most tokens and run the combine's reads, over all
  // XCDs. The grid is padded to whole rounds of 8 tiles and the padding
  // workgroups exit at once.
  const int jb = blockIdx.x / 8;
  const int t = blockIdx.x % 8 + 8 * (jb / n_col_tiles);
  if (t >= cmb.n_tiles) return;
  const int L = t * n_col_tiles + jb % n_col_tiles;
  const MoeTile tile = tiles[L / n_col_tiles];
  const int n0 = (L % n_col_tiles) * 32 * NW;
  const int8_t *We = W + (int64_t)tile.expert * w_stride_e;
  const float *WSe = WS + (int64_t)tile.expert * ws_stride_e;
  // The body is instantiated per count of 32-row blocks holding rows; the
  // registers of the largest (BM / 32) set the kernel's.
  const int nrb = (tile.rows + 31) >> 5;
  static_for<BM / 32>([&](auto u_c) {
    constexpr int NRB = decltype(u_c)::value + 1;
    if (nrb == NRB || (NRB == BM / 32 && nrb > NRB))
      moe_body<GU, NW, PD, BM, NRB>(A, AS, as_stride, tok, a_rows, tile, We, WSe, ws_stride, N, K, n0,
                                    row_w, out, out_ld, cmb, smem);
  });
}

template <bool GU, int NW, int PD, int BM>
static hipError_t launch_moe_cfg(const int8_t *A, const float *AS, int as_stride, const int32_t *tok,
                                 int64_t a_rows, const MoeTile *tiles, int n_tiles,
                                 const int8_t *w, const float *ws, int64_t w_stride_e,
                                 int64_t ws_stride_e, int ws_stride, int N, int K,
                                 const float *row_w, float *out, int out_ld, const MoeCombine &cmb,
                                 hipStream_t st) {
  constexpr int smem = moe_smem<PD, BM>();
  static_assert(smem <= 160 * 1024, "LDS per workgroup");
  auto kern = moe_q8_kernel<GU, NW, PD, BM>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int n_col = (N + 32 * NW - 1) / (32 * NW);
  const int grid = (n_tiles + 7) / 8 * 8 * n_col;
  MoeCombine c = cmb;
  c.n_tiles = n_tiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(NW * 64), smem, st, A, AS, as_stride,
                     tok, a_rows, tiles, n_col, w, ws, w_stride_e, ws_stride_e, ws_stride, N, K,
                     row_w, out, out_ld, c);
  return hipGetLastError();
}

// Tiles of at most 128 rows by default: on MI355X a 30B-A3B expert layer (1024
// tokens, top-8 of 128 experts) takes 256 µs with 128-row tiles against
// 270-275 µs with 64-row tiles, both warm, in the same process. RK_MOE_ROWS=64
// selects the smaller tiles.
int rk_moe_tile_rows() { return rk_knob("RK_MOE_ROWS", 128) == 64 ? 64 : 128; }

// Workgroup shapes (RK_MOE_TILE) for tiles of ≤128 rows: 0 = 4 waves × 128
// columns, weights 2 stages ahead (two workgroups per CU); 1 = 8 waves × 256
// columns, 3 ahead; 2 = 4 waves, 3 ahead; 3 = 4 waves, 4 ahead (one workgroup
// per CU by LDS). Tiles of ≤64 rows (half the accumulator and fragment
// registers): 4 waves × 128 columns, weights PD stages ahead, RK_MOE_TILE
// 0 / 2 / 3 / 4 for PD = 4 / 2 / 3 / 5.
template <bool GU>
static hipError_t launch_moe(int tile_rows, const int8_t *A, const float *AS, int as_stride, const int32_t *tok,
                             int64_t a_rows,
                             const MoeTile *tiles, int n_tiles, const int8_t *w, const float *ws,
                             int64_t w_stride_e, int64_t ws_stride_e, int ws_stride, int N,
                             int K, const float *row_w, float *out, int out_ld, const MoeCombine &cmb,
                             hipStream_t st) {
  if (n_tiles == 0) return hipSuccess;
#define RK_MOE_ARGS A, AS, as_stride, tok, a_rows, tiles, n_tiles, w, ws, w_stride_e, ws_stride_e, ws_stride, N, K, \
                    row_w, out, out_ld, cmb, st
  if (tile_rows == 64) {
    switch (rk_knob("RK_MOE_TILE", 0)) {
      case 2: return launch_moe_cfg<GU, 4, 2, 64>(RK_MOE_ARGS);
      case 3: return launch_moe_cfg<GU, 4, 3, 64>(RK_MOE_ARGS);
      case 4: return launch_moe_cfg<GU, 4, 5, 64>(RK_MOE_ARGS);
      default: return launch_moe_cfg<GU, 4, 4, 64>(RK_MOE_ARGS);
    }
  }
  if (tile_rows != 128) return hipErrorInvalidValue;
  switch (rk_knob("RK_MOE_TILE", 0)) {
    case 1: return launch_moe_cfg<GU, 8, 3, 128>(RK_MOE_ARGS);
    case 2: return launch_moe_cfg<GU, 4, 3, 128>(RK_MOE_ARGS);
    case 3: return launch_moe_cfg<GU, 4, 4, 128>(RK_MOE_ARGS);
    default: return launch_moe_cfg<GU, 4, 2, 128>(RK_MOE_ARGS);
  }
#undef RK_MOE_ARGS
}

hipError_t rk_launch_moe_gemm_gu(int tile_rows, const int8_t *xq, const float *xs, int xs_stride,
                                 const int32_t *tok, int64_t s, const MoeTile *tiles, int n_tiles, const int8_t *w,
                                 const float *ws, int64_t w_stride_e, int64_t ws_stride_e,
                                 int ws_stride, int N, int K, float *act, hipStream_t st) {
  return launch_moe<true>(tile_rows, xq, xs, xs_stride, tok, s, tiles, n_tiles, w, ws, w_stride_e, ws_stride_e,
                          ws_stride, N, K, nullptr, act, N / 2, MoeCombine{}, st);
}

hipError_t rk_launch_moe_gemm_down(int tile_rows, const int8_t *aq, const float *as, int as_stride, int64_t rows,
                                   const MoeTile *tiles, int n_tiles, const int8_t *w,
                                   const float *ws, int64_t w_stride_e, int64_t ws_stride_e,
                                   int ws_stride, int N, int K, const float *row_w, float *yb,
                                   const MoeCombine &cmb, hipStream_t st) {
  return launch_moe<false>(tile_rows, aq, as, as_stride, nullptr, rows, tiles, n_tiles, w, ws, w_stride_e, ws_stride_e,
                           ws_stride, N, K, row_w, yb, N, cmb, st);
}

