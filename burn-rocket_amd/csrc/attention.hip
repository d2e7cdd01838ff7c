// Fused grouped-query flash attention for gfx950 (QKᵀ, online softmax, PV).
//
// Replaces the reference's three-step device attention (QK matmul on the NPU,
// host f32 softmax, AV matmul; crates/rocket-npu/src/attn/mod.rs:1541-1600) and
// the host layout passes around it (fill_heads / fill_heads_transposed /
// unpack_heads, ext.rs:2174-2220): Q, K and O are read and written in the
// caller's layout; only V is rewritten, once per call, into the transposed
// layout the PV product consumes (the reference's own V layout, [KV][D][n_kv],
// with keys permuted inside each 32-key chunk).
//
// Work decomposition. A workgroup owns one KV head and a query tile of 128
// rows, row r ↔ (query head g = r / BQ of the group, query qt·BQ + r % BQ),
// BQ = 128 / G, so every K/V tile staged in LDS serves all G query heads that
// read it. Its 8 waves form two key groups of 4 waves; wave w of a group owns
// rows 32w..32w+31 and the group walks every other 64-key tile (group 0 the
// even tiles, group 1 the odd ones). The two partial softmax states are
// merged through LDS at the end. Two waves per SIMD let one wave's softmax
// VALU work overlap the other's MFMAs. Query tiles are dispatched from the
// last one down, so under a causal mask the longest tiles start first and the
// short ones fill in behind them. Unmasked calls with head dims up to 80 may
// instead use 192-row tiles on two groups of 6 waves (3 per SIMD) when that
// takes fewer rounds of one workgroup per CU (launch_attn below). Head dim
// 256 walks 32-key tiles and splits Oᵀ into two 128-row chunks, one per
// workgroup (both form the same QKᵀ and P), so that the four K/Vᵀ buffers fit
// in LDS and the Oᵀ accumulators in registers. A launch with at most half as
// many query tiles as CUs splits each tile's key tiles between two workgroups
// whose softmax states meet in a workspace (KSPLIT, at the end of the kernel);
// a causal launch of one round splits its longest tiles only.
//
// Per wave and 64-key tile (v_mfma_f32_16x16x32_f16 throughout):
//   Sᵀ = K·Qᵀ   A = K rows from LDS, B = Q fragments held in VGPRs; a lane
//               owns one query column (lane % 16 of each 16-query block) and
//               keys 4·(lane/16)+e of each 16-key block, so the row max is
//               in-lane plus two lane swaps (v_permlane16/32_swap);
//   P          exp2 of the scaled scores, split into an unevaluated sum of
//               two fp16 values (hi = top 11 bits of the f32 probability, lo =
//               the rest): fp16-rounded P alone leaves ~2^-12 relative noise
//               per probability, above the parity gate for small outputs;
//   Oᵀ += Vᵀ·Pᵀ A = Vᵀ rows from LDS, B = P hi and lo; Oᵀ keeps the query per
//               lane, so the online-softmax rescale is a per-lane scalar. With
//               a padded head dim (72 → 80) Vᵀ row 72 is all ones in LDS and
//               Oᵀ row 72 is the row sum of P.
//
// LDS: per group two buffers of {K tile: 64 rows of KPC 16-byte chunks (8
// for d ≤ 64, else 16: 256-byte rows) with chunk c of row r at
// c ^ (r & (KPC-1)), Vᵀ tile: DV rows of 64 key slots with chunk c of row r
// at c ^ (r & 7)}, filled by buffer→LDS copies; keys past n_kv and head
// columns past D read as zeros. Both layouts were measured free of LDS bank
// conflicts for these fragment reads on MI355X (SQ_LDS_BANK_CONFLICT), where
// padded 272-byte K rows cost 4 conflict cycles per ds_read_b128.
//
// Masks are predicates on absolute positions (masks.rs:11-114); key tiles
// that no row of the tile can see are skipped. Scores follow fa_score
// (attn/oneshot.rs:193-199) without the lower clamp for visible keys: masked
// keys score -30000 only in tiles holding a row with no visible key at all,
// which then sweep every key so such a row averages V over all n_kv keys
// (flash_attn_ref, attn/oneshot.rs:118-127).
#include "common.hpp"
#include "kernels.hpp"
#include "vt_tile.hpp"

namespace {

// LDS fragment reads issued ahead of the MFMAs that use them: on MI355X the
// causal GQA S=3633 d=128 kernel takes 125, 108, 105, 104 and 101 µs with
// 1, 2, 3, 4 and 6 reads ahead (no spills up to d=128 at 6).
constexpr int LA = 6;
constexpr int BK = 64;          // keys per tile
constexpr int ROWS = 128;       // query rows per workgroup tile (4 waves per key group)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float MASKED_SCORE = -30000.0f;  // fa_score clamp (attn/softmax.rs:59)
constexpr float RESCALE = 8.0f;  // log2 headroom before the running max is raised

// Visible absolute key interval [lo, hi] of query t (hi may exceed the keys).
__device__ __forceinline__ void vis_range(int mode, int64_t w, int64_t t, int64_t &lo,
                                          int64_t &hi) {
  const int64_t INF = (int64_t)1 << 60;
  switch (mode) {
    case RK_MASK_CAUSAL:
      lo = -INF;
      hi = t;
      break;
    case RK_MASK_WINDOW:
      lo = t - w;
      hi = t + w;
      break;
    case RK_MASK_CAUSAL_WINDOW:
      lo = t - w + 1;
      hi = t;
      break;
    default:
      lo = -INF;
      hi = INF;
  }
}

// x - f32(h) for the low / high fp16 half of h in one v_fma_mix_f32 (the f16
// operand is widened exactly and the difference of a value and its
// truncation to fp16 is exact in f32), instead of a convert and a subtract.
__device__ __forceinline__ float minus_half_lo(unsigned h, float x) {
  float r;
  asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
  return r;
}
__device__ __forceinline__ float minus_half_hi(unsigned h, float x) {
  float r;
  asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(x));
  return r;
}

// max over lanes l, l^16, l^32, l^48 (the four lane groups holding one query).
__device__ __forceinline__ float max4groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum4groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Key tiles a query tile reads: its rows (query heads × queries q_lo..q_hi)
// see absolute keys in per-row intervals whose ends never decrease with the
// query position, so the union of the rows' intervals and "some row sees no
// key at all" (degenerate: then every key tile is swept) follow from the first
// and the last query. full_lo..full_hi: relative keys every row of the tile
// sees.
struct TileKeys {
  int kt_begin, kt_end, full_lo, full_hi;
  bool degenerate;
};
template <int TK>
__device__ __forceinline__ TileKeys tile_keys(const AttnArgs &a, int qt, int BQ) {
  const int n_kt = (a.n_kv + TK - 1) / TK;
  const int q_lo = qt * BQ, q_hi = min(qt * BQ + BQ, a.n_q) - 1;
  const int64_t t_min = a.q0 + q_lo, t_max = a.q0 + q_hi;
  const int64_t kabs0 = a.k0, kabs1 = a.k0 + a.n_kv - 1;
  int64_t lo_a, hi_a, lo_b, hi_b;
  vis_range(a.mask_mode, a.window, t_min, lo_a, hi_a);
  vis_range(a.mask_mode, a.window, t_max, lo_b, hi_b);
  TileKeys t;
  // a row t sees no key iff lo(t) > kabs1, hi(t) < kabs0 or lo(t) > hi(t);
  // lo - hi is the same for every row
  t.degenerate = hi_a < kabs0 || lo_b > kabs1 || lo_a > hi_a;
  t.full_lo = (int)min(max(lo_b - a.k0, (int64_t)0), (int64_t)a.n_kv);
  t.full_hi = (int)max(min(hi_a - a.k0, (int64_t)a.n_kv - 1), (int64_t)-1);
  t.kt_begin = 0;
  t.kt_end = n_kt;
  if (!t.degenerate) {
    const int64_t any_lo = max(lo_a, kabs0) - a.k0;  // relative key indices
    const int64_t any_hi = min(hi_b, kabs1) - a.k0;
    t.kt_begin = (int)(max(any_lo, (int64_t)0) / TK);
    t.kt_end = (int)min((any_hi / TK) + 1, (int64_t)n_kt);
  }
  return t;
}

// TK keys per tile (64; 32 for head dims above 128, to fit LDS). Head dims
// above 128 split Oᵀ into 128-row chunks, one workgroup each: each chunk's
// workgroup computes the whole Sᵀ and softmax and multiplies its own Vᵀ rows.
template <int D, int TK = BK>
struct AttnGeom {
  static constexpr int DQ = (D + 15) / 16 * 16;  // padded head dim
  static constexpr int NQC = DQ / 32;            // 32-wide d chunks of QKᵀ
  static constexpr bool TAIL16 = (DQ % 32) != 0;  // one 16-wide chunk (x16 MFMA)
  static constexpr int DV = DQ;
  static constexpr int DVC = DV <= 128 ? DV : 128;  // Oᵀ rows per workgroup
  static constexpr int NCH = DV / DVC;              // workgroups per query tile
  static constexpr int NDB = DVC / 16;           // 16-row d blocks of Oᵀ
  static constexpr int KPC = DQ <= 64 ? 8 : (DQ <= 128 ? 16 : DQ / 8);  // 16-byte chunks per K row
  static constexpr int KSW = (KPC < 16 ? KPC : 16) - 1;  // K chunk swizzle mask
  static constexpr int KROW = 16 * KPC;          // bytes per K row in LDS
  static constexpr int NKB = TK / 16;            // 16-key blocks per tile
  static constexpr int NC2 = TK / 32;            // 32-key chunks per tile
  static constexpr int VRB = TK * 2;             // bytes per Vᵀ row in LDS
  static constexpr int K_BYTES = TK * KROW;
  static constexpr int V_BYTES = DVC * VRB;
  static constexpr int BUF_BYTES = K_BYTES + V_BYTES;
  static constexpr int K_INS = TK * KPC / 64;    // 1 KB copies per K tile
  static constexpr int V_INS = V_BYTES / 1024;   // 1 KB copies per Vᵀ tile
  static constexpr int SMEM = 4 * BUF_BYTES;     // 2 groups × 2 buffers
  static_assert(DV % DVC == 0 && (TK == 64 || TK == 32), "tile geometry");
};

}  // namespace

template <int D, bool SOFTCAP, int NWG, int TK = BK, bool KSPLIT = false>
__global__ __launch_bounds__(2 * NWG * 64, NWG == 4 ? 2 : 1) void attn_fa_kernel(AttnArgs a, int G,
                                                                                int BQ,
                                                                                int n_qtiles) {
  using Gm = AttnGeom<D, TK>;
  constexpr int DQ = Gm::DQ, NQC = Gm::NQC, NDB = Gm::NDB, DV = Gm::DV;
  constexpr int DVC = Gm::DVC, NCH = Gm::NCH, NKB = Gm::NKB, NC2 = Gm::NC2, VRB = Gm::VRB;
  constexpr bool TAIL16 = Gm::TAIL16;
  constexpr int KROW = Gm::KROW, KPC = Gm::KPC;
  constexpr int K_BYTES = Gm::K_BYTES, BUF_BYTES = Gm::BUF_BYTES;
  constexpr int K_INS = Gm::K_INS;
  // A head dim padded to DV (72 → 80): Vᵀ row D of every LDS buffer holds ones,
  // so O row D of the PV product is the softmax row sum l (the MFMAs compute it
  // from the same hi + lo probabilities, and the rescale of O rescales it), and
  // the VALU slot keeps no sums. The rows D..DV-1 are written once and never
  // copied.
  constexpr bool LROW = D < DV;
  static_assert(!LROW || (D % 8 == 0 && TK == 64 && NCH == 1), "Vᵀ copies move 8-row groups");
  constexpr int V_INS = LROW ? D / 8 : Gm::V_INS;
  constexpr int CPW = (K_INS + V_INS + NWG - 1) / NWG;  // copies per wave of a group
  // Reads ahead: fewer with 3 waves per SIMD, whose register budget is 168.
  constexpr int LAW = NWG == 4 ? LA : 3;
  // (at most the fragments a slot reads: head dim 32 has four per product)
  constexpr int NF_ = NC2 * NDB, NR_ = NKB * (NQC + (TAIL16 ? 1 : 0));
  constexpr int LAWV = LAW < NF_ ? LAW : NF_, LAWK = LAW < NR_ ? LAW : NR_;
  static_assert(Gm::SMEM <= 160 * 1024, "LDS");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = (int)((unsigned)wave / NWG), wq = (int)((unsigned)wave % NWG);
  const int KV = a.n_kv_heads;
  // KSPLIT: for t < n_split, workgroups 2t and 2t+1 take the first and the
  // second half of the key tiles of query tile t (ks 0, 1); the workgroups
  // after them take the other tiles whole (ks -1).
  const int n_split = KSPLIT ? a.n_split : 0;
  const bool split_wg = KSPLIT && (int)blockIdx.x < 2 * n_split;
  const int ks = split_wg ? (int)(blockIdx.x & 1) : -1;
  const int bid = split_wg ? (int)(blockIdx.x >> 1) : (int)blockIdx.x - n_split;
  const int dch = bid % NCH;  // Oᵀ row chunk
  const int wgq = bid / NCH;
  const int kvh = wgq % KV;
  const int qt = n_qtiles - 1 - wgq / KV;  // longest causal tiles first
  const int l16 = lane & 15, lg = lane >> 4;

  // ---- copy geometry (per wave of a group, constant over tiles)
  const f16 *kbase = (const f16 *)a.k + (int64_t)kvh * a.k_head_stride;
  const rsrc_t rk =
      make_rsrc(kbase, ((int64_t)(a.n_kv - 1) * a.k_tok_stride + D) * 2);
  const f16 *vtbase = (const f16 *)a.vt + ((int64_t)kvh * DV + (int64_t)dch * DVC) * a.n_kv_pad;
  const rsrc_t rv = make_rsrc(vtbase, (int64_t)DVC * a.n_kv_pad * 2);
  const uint32_t kstride_b = (uint32_t)(a.k_tok_stride * 2);  // bytes between keys
  const uint32_t vrow_b = (uint32_t)(a.n_kv_pad * 2);         // bytes between Vᵀ rows
  // Per-lane byte offset of copy c (recomputed at issue time: a few integer
  // ops, instead of keeping one VGPR per copy live through the loop).
  auto copy_voff = [&](int c) -> uint32_t {
    if (c < K_INS) {
      const int p = 64 * c + lane, row = p / KPC;
      const int ch = (p % KPC) ^ (row & Gm::KSW);  // logical chunk of this slot
      return (ch < D / 8) ? (uint32_t)row * kstride_b + (uint32_t)(ch * 16) : OOB_OFFSET;
    }
    if constexpr (TK == 64) {  // 8 Vᵀ rows of 8 chunks, chunk c of row d at c ^ (d & 7)
      const int d = 8 * (c - K_INS) + (lane >> 3);
      const int lch = (lane & 7) ^ (d & 7);
      return (uint32_t)d * vrow_b + (uint32_t)(lch * 16);
    } else {  // 16 Vᵀ rows of 4 chunks, chunk c of row d at c ^ ((d >> 1) & 3): the
              // 64-byte rows pair up in 128 bytes, and eight consecutive rows
              // then cover the 128 bytes a fragment read serves at once
              // (d >> 2 left rows d and d + 2 on the same banks)
      const int d = 16 * (c - K_INS) + (lane >> 2);
      const int lch = (lane & 3) ^ ((d >> 1) & 3);
      return (uint32_t)d * vrow_b + (uint32_t)(lch * 16);
    }
  };
  // Copies of the K part of key tile tk into buffer bk and of the Vᵀ part of
  // key tile tv into buffer bv of this wave's group (a tile < 0: no copy).
  auto issue = [&](int tk, int bk, int tv, int bv) {
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int c = wq + NWG * i;  // wave-uniform
      if (c < K_INS) {
        if (tk >= 0)
          bdma16(rk, smem + (grp * 2 + bk) * BUF_BYTES + c * 1024, copy_voff(c),
                 (uint32_t)tk * (TK * kstride_b));
      } else if (c < K_INS + V_INS) {
        if (tv >= 0)
          bdma16(rv, smem + (grp * 2 + bv) * BUF_BYTES + K_BYTES + (c - K_INS) * 1024, copy_voff(c),
                 (uint32_t)(tv * TK * 2));
      }
    }
  };

  // ---- LDS fragment addresses (within a buffer)
  const int kf = l16 & Gm::KSW;
  uint32_t k_off[NQC > 0 ? NQC : 1];  // per 32-wide d chunk c; + kb·16·KROW
#pragma unroll
  for (int c = 0; c < NQC; ++c) k_off[c] = (uint32_t)(l16 * KROW + (((4 * c + lg) ^ kf) << 4));
  const uint32_t k_off16 =
      (uint32_t)(l16 * KROW + (((4 * NQC + (lg >> 1)) ^ kf) << 4) + (lg & 1) * 8);
  uint32_t v_off[NC2];  // per 32-key chunk c2; + db·16·VRB
#pragma unroll
  for (int c2 = 0; c2 < NC2; ++c2)
    v_off[c2] = TK == 64 ? (uint32_t)(K_BYTES + l16 * 128 + (((4 * c2 + lg) ^ (l16 & 7)) << 4))
                         : (uint32_t)(K_BYTES + l16 * 64 + ((lg ^ ((l16 >> 1) & 3)) << 4));

  const float C = SOFTCAP ? LOG2E : a.scale * LOG2E;
  {

    // ---- this lane's query rows (two 16-query blocks)
    int qi[2], hq[2];
    bool rok[2];
    int64_t tab[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int r = wq * 32 + qb * 16 + l16;
      const int g = r / BQ;
      qi[qb] = qt * BQ + (r % BQ);
      rok[qb] = (g < G) && (qi[qb] < a.n_q);
      hq[qb] = kvh * G + min(g, G - 1);
      tab[qb] = a.q0 + (rok[qb] ? qi[qb] : 0);
    }

    // ---- key range of the tile, degenerate rows
    const TileKeys tkeys = tile_keys<TK>(a, qt, BQ);
    const bool degenerate = tkeys.degenerate;
    const int full_lo = tkeys.full_lo, full_hi = tkeys.full_hi;
    int kt_begin = tkeys.kt_begin, kt_end = tkeys.kt_end;
    if (split_wg) {
      const int kt_mid = kt_begin + (kt_end - kt_begin + 1) / 2;
      if (ks == 0)
        kt_end = kt_mid;
      else
        kt_begin = kt_mid;
    }
    const float masked_x = degenerate ? MASKED_SCORE * LOG2E : -INFINITY;
    // Visible keys of each of this lane's queries as a relative key interval
    // [klo, khi] (every mask mode is an interval), clipped to [0, n_kv).
    int klo[2], khi[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      int64_t lo, hi;
      vis_range(a.mask_mode, a.window, tab[qb], lo, hi);
      lo = max(lo - a.k0, (int64_t)0);
      hi = min(hi - a.k0, (int64_t)a.n_kv - 1);
      klo[qb] = rok[qb] ? (int)min(lo, (int64_t)a.n_kv) : a.n_kv;
      khi[qb] = rok[qb] ? (int)max(hi, (int64_t)-1) : -1;
    }

    // ---- Q fragments (B operand of Sᵀ = K·Qᵀ): d = 32c + 8·lg + 0..7
    half8 qf[2][NQC > 0 ? NQC : 1];
    half4 qt16[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const f16 *qrow = (const f16 *)a.q + (int64_t)(rok[qb] ? qi[qb] : 0) * a.q_tok_stride +
                        (int64_t)hq[qb] * a.q_head_stride;
#pragma unroll
      for (int c = 0; c < NQC; ++c) {
        const int d0 = 32 * c + 8 * lg;
        qf[qb][c] = (rok[qb] && d0 < D) ? *(const half8 *)(qrow + d0) : half8{};
      }
      if constexpr (TAIL16) {
        const int d0 = 32 * NQC + 4 * lg;
        qt16[qb] = (rok[qb] && d0 < D) ? *(const half4 *)(qrow + d0) : half4{};
      }
    }

    floatx4 o[NDB][2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) o[db][qb] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY};  // running max (exp2 domain), per query
    float l_run[2] = {0.f, 0.f};              // this lane's partial row sums

    // ---- key loop. Group g walks tiles kt_begin + 2j + g, j < nj. Its work
    // alternates between an MFMA slot (PV of tile j-1, then Sᵀ of tile j) and
    // a VALU slot (softmax of tile j); group 1 runs one slot behind group 0,
    // so in every slot one wave of each SIMD multiplies while the other does
    // the softmax. Slots are separated by workgroup barriers. K(j+1) and Vᵀ(j)
    // are copied at the start of MFMA slot j (their buffers were last read in
    // slot j-1) and waited for at the end of VALU slot j.
    const int n_tiles = kt_end - kt_begin;
    const int nj = (n_tiles - grp + 1) / 2;
    const int nj_max = (n_tiles + 1) / 2;
    floatx4 sacc[NKB][2];
    half8 phi[2][NC2], plo[2][NC2];
    const bool mix_on = a.mix != 0;
    // Steady-state MFMA slot of 64-key tiles (MIX): the PV products of the
    // second 32-key chunk run interleaved with the Sᵀ products of the first
    // two 16-key blocks. Sᵀ alone reads a 1 KB K fragment per two MFMAs, which
    // on four waves is the LDS read rate of a CU; PV reads one per four. The
    // registers of P chunk 0 die before those of Sᵀ blocks 0-1 are born, so
    // the mix adds no live registers. Built for head dims 72 and 80 only: on
    // MI355X it took vision attention (S=2394, 16 heads, d72) 70.9 -> 68.7 us
    // and made d64 and d128 5-7 % slower (causal S=3633 d128 85 -> 90 us).
    constexpr bool MIX = NC2 == 2 && D > 64 && D <= 80;
    constexpr int NSQ = NQC + (TAIL16 ? 1 : 0);  // K fragments per 16-key block
    auto s_step = [&](const uint8_t *kbuf, auto c_c, auto kb_c) {
      constexpr int c = decltype(c_c)::value, kb = decltype(kb_c)::value;
      if constexpr (c < NQC) {
        const half8 kfr = *(const half8 *)(kbuf + k_off[c] + kb * 16 * KROW);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          sacc[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfr, qf[qb][c], sacc[kb][qb], 0, 0, 0);
      } else if constexpr (TAIL16) {
        const half4 kfr = *(const half4 *)(kbuf + k_off16 + kb * 16 * KROW);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          sacc[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x16f16(kfr, qt16[qb], sacc[kb][qb], 0, 0, 0);
      }
    };
    auto mixed_slot = [&](int j) {
      // (1 <= j < nj) the slot's copies, as in mfma_slot
      issue(j + 1 < nj ? kt_begin + 2 * (j + 1) + grp : -1, (j + 1) & 1, kt_begin + 2 * j + grp, j & 1);
      const uint8_t *vb = smem + (grp * 2 + ((j - 1) & 1)) * BUF_BYTES;
      const uint8_t *kbuf = smem + (grp * 2 + (j & 1)) * BUF_BYTES;
      // (a) PV of chunk 0: hi of fragment f, lo of fragment f-1.
      {
        half8 vprev = half8{};
        static_for<NDB + 1>([&](auto f_c) {
          constexpr int F = decltype(f_c)::value;
          half8 vcur = half8{};
          if constexpr (F < NDB) {
            vcur = *(const half8 *)(vb + v_off[0] + F * 16 * VRB);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
              o[F][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vcur, phi[qb][0], o[F][qb], 0, 0, 0);
          }
          if constexpr (F > 0) {
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
              o[F - 1][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vprev, plo[qb][0], o[F - 1][qb], 0, 0, 0);
          }
          vprev = vcur;
        });
        constexpr int LA_A = LAWV < NDB ? LAWV : NDB;
        __builtin_amdgcn_sched_group_barrier(0x100, LA_A, 0);
        static_for<NDB - LA_A>([&](auto) {
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        });
        __builtin_amdgcn_sched_group_barrier(0x008, 4 * LA_A, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      // (b) PV of chunk 1 interleaved with Sᵀ of blocks 0 and 1.
      {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) sacc[kb][qb] = floatx4{0.f, 0.f, 0.f, 0.f};
        constexpr int NS = 2 * NSQ;                       // Sᵀ steps: (c, kb), c-major
        constexpr int NB = (NDB + 1 > NS) ? NDB + 1 : NS;  // interleaved steps
        half8 vprev = half8{};
        static_for<NB>([&](auto i_c) {
          constexpr int I = decltype(i_c)::value;
          half8 vcur = half8{};
          if constexpr (I < NDB) {
            vcur = *(const half8 *)(vb + v_off[1] + I * 16 * VRB);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
              o[I][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vcur, phi[qb][1], o[I][qb], 0, 0, 0);
          }
          if constexpr (I > 0 && I <= NDB) {
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
              o[I - 1][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vprev, plo[qb][1], o[I - 1][qb], 0, 0, 0);
          }
          vprev = vcur;
          if constexpr (I < NS) s_step(kbuf, ic<I / 2>{}, ic<I % 2>{});
        });
        constexpr int NRB = NDB + NS, NMB = 4 * NDB + 2 * NS;
        constexpr int LA_B = LAW < NRB ? LAW : NRB;
        constexpr int STEPS = (NMB / 3 < NRB - LA_B) ? NMB / 3 : NRB - LA_B;
        __builtin_amdgcn_sched_group_barrier(0x100, LA_B, 0);
        static_for<STEPS>([&](auto) {
          __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        });
        __builtin_amdgcn_sched_group_barrier(0x008, NMB - 3 * STEPS, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      // (c) Sᵀ of blocks 2 and 3.
      {
#pragma unroll
        for (int kb = 2; kb < 4; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) sacc[kb][qb] = floatx4{0.f, 0.f, 0.f, 0.f};
        static_for<2 * NSQ>([&](auto i_c) {
          constexpr int I = decltype(i_c)::value;
          s_step(kbuf, ic<I / 2>{}, ic<2 + I % 2>{});
        });
        constexpr int NR = 2 * NSQ;
        constexpr int LA_C = LAWK < NR ? LAWK : NR;
        __builtin_amdgcn_sched_group_barrier(0x100, LA_C, 0);
        static_for<NR - LA_C>([&](auto) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        });
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * LA_C, 0);
      }
    };
    // MFMA slot j: PV of tile j-1, Sᵀ of tile j.
    auto mfma_slot = [&](int j) {
    if (j < nj) issue(j + 1 < nj ? kt_begin + 2 * (j + 1) + grp : -1, (j + 1) & 1, kt_begin + 2 * j + grp, j & 1);
    if (j >= 1 && j - 1 < nj) {
      // Oᵀ += Vᵀ·Pᵀ for tile j-1: the hi products of one V fragment, then
      // the lo products of the previous fragment, so that the two MFMAs into
      // one accumulator are four MFMAs apart.
      const uint8_t *vb = smem + (grp * 2 + ((j - 1) & 1)) * BUF_BYTES;
      constexpr int NF = NC2 * NDB;  // fragments: f = c2·NDB + db
      half8 vprev = half8{};
      static_for<NF + 1>([&](auto f_c) {
        constexpr int F = decltype(f_c)::value;
        half8 vcur = half8{};
        if constexpr (F < NF) {
          constexpr int C2 = F / NDB, DB = F % NDB;
          vcur = *(const half8 *)(vb + v_off[C2] + DB * 16 * VRB);
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            o[DB][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vcur, phi[qb][C2], o[DB][qb], 0, 0, 0);
        }
        if constexpr (F > 0) {
          constexpr int C2 = (F - 1) / NDB, DB = (F - 1) % NDB;
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            o[DB][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vprev, plo[qb][C2], o[DB][qb], 0, 0, 0);
        }
        vprev = vcur;
      });
      // Each fragment read LAWV reads ahead of its four MFMAs.
      __builtin_amdgcn_sched_group_barrier(0x100, LAWV, 0);
      static_for<NF - LAWV>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      });
      __builtin_amdgcn_sched_group_barrier(0x008, 4 * LAWV, 0);
    }
    // P of tile j-1 dies here, before S of tile j is produced (keeps the two
    // register sets from overlapping).
    __builtin_amdgcn_sched_barrier(0);
    if (j < nj) {
      // Sᵀ for the four 16-key blocks and two 16-query blocks of tile j.
      const uint8_t *kbuf = smem + (grp * 2 + (j & 1)) * BUF_BYTES;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) sacc[kb][qb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NQC; ++c) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const half8 kfr = *(const half8 *)(kbuf + k_off[c] + kb * 16 * KROW);
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            sacc[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfr, qf[qb][c], sacc[kb][qb], 0, 0, 0);
        }
      }
      if constexpr (TAIL16) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const half4 kfr = *(const half4 *)(kbuf + k_off16 + kb * 16 * KROW);
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            sacc[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x16f16(kfr, qt16[qb], sacc[kb][qb], 0, 0, 0);
        }
      }
      // Each fragment read LAWK reads ahead of its two MFMAs.
      constexpr int NR = NKB * (NQC + (TAIL16 ? 1 : 0));
      __builtin_amdgcn_sched_group_barrier(0x100, LAWK, 0);
      static_for<NR - LAWK>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      });
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * LAWK, 0);
    }
    };
    // VALU slot j: online softmax of tile j. Scores stay in the raw domain s
    // (softcap applied in place) and the exp2 argument is always one FMA,
    // s·C - m; on boundary tiles masked scores are first replaced in place by
    // raw values that map to the masked value under that FMA. The running max is
    // only raised (and O and l rescaled) when some query of the wave sees a score
    // more than 2^RESCALE above it; otherwise P is taken against the stale max
    // (values up to 2^RESCALE, exact after the final normalisation).
    auto valu_slot = [&](int j) {
      if (j >= nj) return;
      const int kb0 = (kt_begin + 2 * j + grp) * TK;
      if constexpr (SOFTCAP) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              sacc[kb][qb][e] = a.softcap * tanhf(sacc[kb][qb][e] * a.scale / a.softcap);
      }
      if (!((kb0 >= full_lo) && (kb0 + TK - 1 <= full_hi) && !degenerate)) {
        const float masked_raw = masked_x / C;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int key = kb0 + kb * 16 + 4 * lg + e;
              const float v = sacc[kb][qb][e];
              sacc[kb][qb][e] =
                  (key >= a.n_kv) ? -INFINITY : (key < klo[qb] || key > khi[qb]) ? masked_raw : v;
            }
      }
      float mt[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        float m = sacc[0][qb][0];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (kb | e) m = fmaxf(m, sacc[kb][qb][e]);
        mt[qb] = max4groups(m) * C;
      }
      // Raise the running max (wave-uniform decision).
      const bool up = mt[0] > m_run[0] + RESCALE || mt[1] > m_run[1] + RESCALE;
      if (__builtin_amdgcn_ballot_w64(up) != 0) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const float m_new = fmaxf(m_run[qb], mt[qb]);
          const float alpha = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run[qb] - m_new);
          m_run[qb] = m_new;
          l_run[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < NDB; ++db) o[db][qb] *= alpha;
        }
      }
      // P = exp2(s·C - m) as hi + lo fp16 halves, in the B-operand order of the
      // PV product: chunk c2 = keys 32·c2.., slot 8·lg + i ↔ block 2·c2 + i/4,
      // e = i%4.
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float nm = (m_run[qb] == -INFINITY) ? 0.f : -m_run[qb];
        float lsum = 0.f;
#pragma unroll
        for (int c2 = 0; c2 < NC2; ++c2) {
          uintx4 hw, lw;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int kb = 2 * c2 + (jj >> 1), e = 2 * (jj & 1);
            const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][qb][e], C, nm));
            const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][qb][e + 1], C, nm));
            lsum += e0 + e1;
            const unsigned int h = __builtin_bit_cast(unsigned int, __builtin_amdgcn_cvt_pkrtz(e0, e1));
            hw[jj] = h;
            lw[jj] = __builtin_bit_cast(unsigned int, __builtin_amdgcn_cvt_pkrtz(minus_half_lo(h, e0),
                                                                                minus_half_hi(h, e1)));
          }
          phi[qb][c2] = __builtin_bit_cast(half8, hw);
          plo[qb][c2] = __builtin_bit_cast(half8, lw);
        }
        if constexpr (!LROW) l_run[qb] += lsum;
      }
      WAIT_VMCNT(0);  // K(j+1) and Vᵀ(j) land before the next MFMA slot
    };
    if constexpr (LROW) {
      // Vᵀ rows D..DV-1 of the four buffers: row D = 1.0 per key slot, the rest 0.
      for (int i = threadIdx.x; i < 4 * (DV - D) * 8; i += 2 * NWG * 64) {
        const int buf = i / ((DV - D) * 8), j = i % ((DV - D) * 8);
        const int row = D + j / 8;
        const unsigned one2 = row == D ? 0x3c003c00u : 0u;  // two fp16 1.0
        *(uintx4 *)(smem + buf * BUF_BYTES + K_BYTES + row * 128 + (j % 8) * 16) =
            uintx4{one2, one2, one2, one2};
      }
      WAIT_LGKMCNT0();
    }
    issue(nj > 0 ? kt_begin + grp : -1, 0, -1, 0);
    WAIT_VMCNT(0);
    BARRIER();
    // One loop per group, so that only S (group 1) or only P (group 0) is
    // live across a loop iteration; both make 2·nj_max + 2 barriers.
    // With MIX the slots that hold both products (1 ≤ j < nj) run in a loop
    // of their own, so that no loop body joins two schedules of them.
    if (grp == 0) {
      int j = 0;
      if constexpr (MIX) {
        if (mix_on && nj >= 2) {
          mfma_slot(0);
          BARRIER();
          valu_slot(0);
          BARRIER();
          for (j = 1; j < nj; ++j) {
            mixed_slot(j);
            BARRIER();
            valu_slot(j);
            BARRIER();
          }
        }
      }
      for (; j <= nj_max; ++j) {
        mfma_slot(j);
        BARRIER();
        valu_slot(j);
        BARRIER();
      }
    } else {
      BARRIER();
      mfma_slot(0);
      BARRIER();
      int j = 0;
      if constexpr (MIX) {
        if (mix_on && nj >= 2) {
          for (; j + 1 < nj; ++j) {
            valu_slot(j);
            BARRIER();
            mixed_slot(j + 1);
            BARRIER();
          }
        }
      }
      for (; j < nj_max; ++j) {
        valu_slot(j);
        BARRIER();
        mfma_slot(j + 1);
        BARRIER();
      }
    }
    WAIT_VMCNT(0);

    // ---- merge the two key groups through LDS, normalise and store.
    // Group 1 writes (m, l, Oᵀ) per lane; group 0 combines.
    float *xch = (float *)smem + wq * 64 * (2 * 2 + NDB * 2 * 4);
    BARRIER();  // all compute done: the K/V buffers are free
    float lt[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      if constexpr (LROW) {
        // O row D (block D/16, lane group (D%16)/4, element D%4) of this query.
        lt[qb] = __shfl(o[D / 16][qb][D % 4], l16 + 16 * ((D % 16) / 4));
      } else {
        lt[qb] = sum4groups(l_run[qb]);
      }
    }
    if (grp == 1) {
      float *p = xch + lane;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        p[(2 * qb) * 64] = m_run[qb];
        p[(2 * qb + 1) * 64] = lt[qb];
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int e = 0; e < 4; ++e) p[(4 + (db * 2 + qb) * 4 + e) * 64] = o[db][qb][e];
    }
    BARRIER();
    float m_all[2] = {0.f, 0.f}, l_all[2] = {0.f, 0.f};  // KSPLIT: the merged state of this key half
    if (grp == 0) {
      const float *p = xch + lane;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float m1 = p[(2 * qb) * 64], l1 = p[(2 * qb + 1) * 64];
        const float m = fmaxf(m_run[qb], m1);
        const float mu = (m == -INFINITY) ? 0.f : m;
        const float a0 = __builtin_amdgcn_exp2f(m_run[qb] - mu);
        const float a1 = __builtin_amdgcn_exp2f(m1 - mu);
        const float l = lt[qb] * a0 + l1 * a1;
        if (split_wg) {
          m_all[qb] = m;
          l_all[qb] = l;
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              o[db][qb][e] = o[db][qb][e] * a0 + p[(4 + (db * 2 + qb) * 4 + e) * 64] * a1;
          continue;
        }
        const float inv = l > 0.f ? 1.0f / l : 0.f;
        if (rok[qb]) {
          f16 *orow = (f16 *)a.out + (int64_t)qi[qb] * a.o_tok_stride + (int64_t)hq[qb] * a.o_head_stride;
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const int d0 = dch * DVC + db * 16 + 4 * lg;
            if (d0 < D) {
              half4 h;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float o1 = p[(4 + (db * 2 + qb) * 4 + e) * 64];
                h[e] = (f16)((o[db][qb][e] * a0 + o1 * a1) * inv);
              }
              *(half4 *)(orow + d0) = h;
            }
          }
        }
      }
    }
    if (split_wg) {
      // Each half writes its state (m, l, unnormalised Oᵀ) to its slot, and
      // the second half to arrive merges the two, in split order whichever it
      // is, and stores O. Nothing waits on the other workgroup. The slots are
      // written and read with 16-byte device-coherent (sc1) accesses, so no
      // L2-wide write-back or invalidate is needed (those cost more than the
      // split gained). Slot of a half: [wave wq][j][lane] 16-byte entries,
      // j = 0 the (m, l) pairs of the two query blocks, j = 1 + 2·db + qb the
      // Oᵀ block (db, qb).
      constexpr int NJ = 1 + 2 * NDB;
      constexpr int SLOT_BYTES = NWG * NJ * 64 * 16;
      constexpr int SC1 = 16;  // cache policy bit: device scope
      const rsrc_t rp = make_rsrc(a.part + (size_t)bid * 2 * (SLOT_BYTES / 4), 2 * SLOT_BYTES);
      const uint32_t lane_off = (uint32_t)((wq * NJ * 64 + lane) * 16);
      const uint32_t mine = lane_off + (uint32_t)(ks * SLOT_BYTES);
      const uint32_t other = lane_off + (uint32_t)((ks ^ 1) * SLOT_BYTES);
      if (grp == 0) {
        const floatx4 ml = {m_all[0], l_all[0], m_all[1], l_all[1]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4, ml), rp, mine, 0, SC1);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uintx4, o[db][qb]), rp,
                                                   mine + (uint32_t)((1 + 2 * db + qb) * 1024), 0, SC1);
        WAIT_VMCNT(0);  // the state is stored before the arrival count
      }
      BARRIER();  // every read of the exchange area is done: its first word is free
      unsigned *flag = (unsigned *)smem;
      if (threadIdx.x == 0) {
        const unsigned prev = atomicAdd(a.cnt + bid, 1u);
        if (prev != 0) atomicExch(a.cnt + bid, 0u);  // both halves are in: reset for the next launch
        *flag = prev;
        WAIT_LGKMCNT0();
      }
      BARRIER();
      if (*flag == 0 || grp != 0) return;
      // Every load of the other state is issued before the first use (the
      // loads go to memory; one at a time they cost a latency each).
      const floatx4 mlo = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rp, other, 0, SC1));
      floatx4 ot[NDB][2];
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          ot[db][qb] = __builtin_bit_cast(
              floatx4, __builtin_amdgcn_raw_buffer_load_b128(rp, other + (uint32_t)((1 + 2 * db + qb) * 1024), 0, SC1));
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float mo = mlo[2 * qb], lo = mlo[2 * qb + 1];
        const float m0 = ks == 0 ? m_all[qb] : mo, m1 = ks == 0 ? mo : m_all[qb];
        const float l0 = ks == 0 ? l_all[qb] : lo, l1 = ks == 0 ? lo : l_all[qb];
        const float m = fmaxf(m0, m1);
        const float mu = (m == -INFINITY) ? 0.f : m;
        const float a0 = __builtin_amdgcn_exp2f(m0 - mu);
        const float a1 = __builtin_amdgcn_exp2f(m1 - mu);
        const float l = l0 * a0 + l1 * a1;
        const float inv = l > 0.f ? 1.0f / l : 0.f;
        if (rok[qb]) {
          f16 *orow = (f16 *)a.out + (int64_t)qi[qb] * a.o_tok_stride + (int64_t)hq[qb] * a.o_head_stride;
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const int d0 = dch * DVC + db * 16 + 4 * lg;
            if (d0 < D) {
              const floatx4 oo = ot[db][qb];
              half4 h;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float o0 = ks == 0 ? o[db][qb][e] : oo[e], o1 = ks == 0 ? oo[e] : o[db][qb][e];
                h[e] = (f16)((o0 * a0 + o1 * a1) * inv);
              }
              *(half4 *)(orow + d0) = h;
            }
          }
        }
      }
    }
  }
}

// V [n_kv] × (head g, d) → Vt (layout and tile order: vt_tile.hpp); one
// 64-key × 64-d tile per block.
__global__ __launch_bounds__(256) void v_transpose_kernel(const f16 *__restrict__ v,
                                                          int64_t tok_stride, int64_t head_stride,
                                                          int64_t d_stride, int n_kv, int n_kv_pad,
                                                          int D, int DVp, f16 *__restrict__ vt) {
  __shared__ vt_half8 tile[64][8];
  vt_tile(v, tok_stride, head_stride, d_stride, n_kv, n_kv_pad, D, DVp, vt, blockIdx.x, blockIdx.y,
          blockIdx.z, tile, threadIdx.x);
}

int rk_attn_dv_pad(int head_dim) { return (head_dim + 15) / 16 * 16; }
int rk_attn_kv_tile() { return BK; }

hipError_t rk_launch_v_transpose(const void *v, int64_t v_tok_stride, int64_t v_head_stride,
                                 int n_kv, int n_kv_pad, int n_kv_heads, int head_dim,
                                 int dv_pad, void *vt, hipStream_t st) {
  dim3 grid((unsigned)(n_kv_pad / 64), (unsigned)((dv_pad + 63) / 64), (unsigned)n_kv_heads);
  hipLaunchKernelGGL(v_transpose_kernel, grid, dim3(256), 0, st, (const f16 *)v, v_tok_stride,
                     v_head_stride, (int64_t)1, n_kv, n_kv_pad, head_dim, dv_pad, (f16 *)vt);
  return hipGetLastError();
}

hipError_t rk_launch_v_transpose_strided(const void *v, int64_t tok_stride, int64_t head_stride,
                                         int64_t d_stride, int n_kv, int n_kv_pad,
                                         int n_kv_heads, int head_dim, int dv_pad, void *vt,
                                         hipStream_t st) {
  dim3 grid((unsigned)(n_kv_pad / 64), (unsigned)((dv_pad + 63) / 64), (unsigned)n_kv_heads);
  hipLaunchKernelGGL(v_transpose_kernel, grid, dim3(256), 0, st, (const f16 *)v, tok_stride,
                     head_stride, d_stride, n_kv, n_kv_pad, head_dim, dv_pad, (f16 *)vt);
  return hipGetLastError();
}

template <int D, int NWG, int TK = BK, bool KSPLIT = false>
static hipError_t launch_attn_nwg(const AttnArgs &a, hipStream_t st) {
  const int G = a.n_head / a.n_kv_heads;
  const int BQ = 32 * NWG / G;
  const int n_qtiles = (a.n_q + BQ - 1) / BQ;
  const int grid = n_qtiles * a.n_kv_heads * AttnGeom<D, TK>::NCH + (KSPLIT ? a.n_split : 0);
  auto kern0 = attn_fa_kernel<D, false, NWG, TK, KSPLIT>;
  auto kern1 = attn_fa_kernel<D, true, NWG, TK, KSPLIT>;
  constexpr int smem = AttnGeom<D, TK>::SMEM;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)kern0,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void *)kern1, hipFuncAttributeMaxDynamicSharedMemorySize,
                              smem);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  // RK_ATTN_MIX = 0 keeps the PV and Sᵀ products of a slot apart (kernels
  // that have the mixed slot: head dims 72 and 80).
  AttnArgs b = a;
  b.mix = rk_knob("RK_ATTN_MIX", 1) != 0;
  if (a.softcap != 0.f)
    hipLaunchKernelGGL(kern1, dim3((unsigned)grid), dim3(2 * NWG * 64), smem, st, b, G, BQ,
                       n_qtiles);
  else
    hipLaunchKernelGGL(kern0, dim3((unsigned)grid), dim3(2 * NWG * 64), smem, st, b, G, BQ,
                       n_qtiles);
  return hipGetLastError();
}

// One workgroup per CU (LDS). Without a mask every workgroup walks all keys,
// so a grid of slightly more tiles than CUs runs a short second round on few
// CUs; 192-row tiles (6 waves per key group, 3 per SIMD) then cover the
// queries in fewer rounds (vision S=2394, 16 heads: 304 tiles of 128 rows =
// 2 rounds, 208 tiles of 192 rows = 1). Head dims up to 80 fit 3 waves per
// SIMD in registers.
//
// A grid that fills at most half of the CUs (few query heads, short
// sequences) leaves the rest idle for the whole launch: given the workspace,
// such a launch splits each query tile's key tiles between two workgroups. A
// causal grid of one round splits its first a.n_split tiles, the longest
// (rk_attn_split_tiles).
template <int D>
static hipError_t launch_attn(const AttnArgs &a, hipStream_t st) {
  const bool split = a.part != nullptr && a.cnt != nullptr && a.n_split > 0;
  // Head dims above 128: 32-key tiles and 128-row Oᵀ chunks (LDS).
  if constexpr (D > 128) {
    if (split) return launch_attn_nwg<D, 4, 32, true>(a, st);
    return launch_attn_nwg<D, 4, 32>(a, st);
  } else {
  if (split) return launch_attn_nwg<D, 4, BK, true>(a, st);
  if constexpr (D <= 80) {
    // RK_ATTN_ROWS = 128 or 192 forces the tile height (any mask).
    const int G = a.n_head / a.n_kv_heads;
    const int knob = rk_knob("RK_ATTN_ROWS", 0);
    bool six = knob == 192;
    if (knob == 0 && a.mask_mode == RK_MASK_NONE) {
      const long cus = a.num_cus > 0 ? a.num_cus : 256;
      const long t4 = (long)((a.n_q + 128 / G - 1) / (128 / G)) * a.n_kv_heads;
      const long t6 = (long)((a.n_q + 192 / G - 1) / (192 / G)) * a.n_kv_heads;
      six = (t6 + cus - 1) / cus * 192 < (t4 + cus - 1) / cus * 128;
    }
    if (six && G <= 192) return launch_attn_nwg<D, 6>(a, st);
  }
  return launch_attn_nwg<D, 4>(a, st);
  }
}

long rk_attn_split_floats(int head_dim) {
  const int dv = rk_attn_dv_pad(head_dim);
  const int ndb = (dv <= 128 ? dv : 128) / 16;
  return 4L * 64 * (4 + 8 * ndb);  // four waves of 64 lanes (the exchange layout)
}

// RK_ATTN_SPLIT: 0 (default) splits grids of at most half the CUs, 1 never
// splits, 2 splits every launch that has the workspace.
long rk_attn_split_tiles(const AttnArgs &a) {
  const int knob = rk_knob("RK_ATTN_SPLIT", 0);
  if (knob == 1 || a.n_kv_heads <= 0 || a.n_head % a.n_kv_heads) return 0;
  const int G = a.n_head / a.n_kv_heads;
  if (G < 1 || G > ROWS) return 0;
  const int dv = rk_attn_dv_pad(a.head_dim);
  const long nch = dv <= 128 ? 1 : dv / 128;
  const int BQ = ROWS / G;
  const long tiles = (long)((a.n_q + BQ - 1) / BQ) * a.n_kv_heads * nch;
  const long cus = a.num_cus > 0 ? a.num_cus : 256;
  if (knob == 2 || 2 * tiles <= cus) return tiles;
  // One round under a causal mask: the longest tiles set the time.
  const bool causal = a.mask_mode == RK_MASK_CAUSAL || a.mask_mode == RK_MASK_CAUSAL_WINDOW;
  const int forced = rk_knob("RK_ATTN_SPLIT_TILES", -1);
  if (causal && forced >= 0) return std::min<long>(tiles, forced);
  if (causal && tiles <= cus) return std::min(tiles, (cus - tiles) / 2 + tiles / 8);
  return 0;
}

hipError_t rk_launch_attention(const AttnArgs &a, hipStream_t st) {
  const int G = a.n_head / a.n_kv_heads;
  if (G < 1 || G > ROWS || a.n_head % a.n_kv_heads) return hipErrorInvalidValue;
  switch (a.head_dim) {
    case 32:
      return launch_attn<32>(a, st);
    case 48:
      return launch_attn<48>(a, st);
    case 64:
      return launch_attn<64>(a, st);
    case 72:
      return launch_attn<72>(a, st);
    case 80:
      return launch_attn<80>(a, st);
    case 96:
      return launch_attn<96>(a, st);
    case 112:
      return launch_attn<112>(a, st);
    case 128:
      return launch_attn<128>(a, st);
    case 256:
      return launch_attn<256>(a, st);
  }
  return hipErrorInvalidValue;
}
