// Fused grouped-query flash attention for gfx950 (QKᵀ, online softmax, PV).
//
// Replaces the reference's three-step device attention (QK matmul on the NPU,
// host f32 softmax, AV matmul; crates/rocket-npu/src/attn/mod.rs:1541-1600) and
// the host layout passes around it (fill_heads / fill_heads_transposed /
// unpack_heads, ext.rs:2174-2220): Q, K and O are read and written in the
// caller's token-major layout; only V is rewritten, once per call, into the
// transposed layout the PV product consumes (the reference's own V layout,
// [KV][D][n_kv], with keys permuted inside each 16-key chunk).
//
// One workgroup = one query tile of one KV head, covering all G = H/KV query
// heads that read it: 4 waves × 32 rows, row r ↔ (head g = r / BQ, query
// qt·BQ + r % BQ). K/V tiles of 64 keys are staged once in LDS and used by all
// G·BQ rows.
//
// Per wave and 32-key block the kernel computes Sᵀ = K·Qᵀ with
// v_mfma_f32_32x32x16_f16 (A = K rows from LDS, B = Q fragment held in VGPRs),
// so each lane owns one query column and 16 of its keys; the row max and row
// sum are in-lane plus one exchange with lane ^ 32. P is converted to fp16 in
// registers and fed straight back as the B operand of Oᵀ = Vᵀ·Pᵀ (A = Vᵀ rows
// from LDS); Oᵀ keeps the same query-per-lane ownership, so the online-softmax
// rescale is a per-lane scalar.
//
// Masks are predicates on absolute positions (masks.rs:11-114); key tiles that
// no row of the workgroup can see are skipped. Scores follow fa_score
// (attn/oneshot.rs:193-199) without the lower clamp for visible keys: masked
// keys score -30000 only in workgroups holding a row with no visible key at
// all, which then sweep every key so such a row averages V over all n_kv keys
// (flash_attn_ref, attn/oneshot.rs:118-127).
#include "common.hpp"
#include "kernels.hpp"

namespace {

constexpr int BK = 64;         // keys per tile
constexpr int NWAVES = 4;      // waves per workgroup
constexpr int ROWS = NWAVES * 32;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float MASKED_SCORE = -30000.0f;  // fa_score clamp (attn/softmax.rs:59)

// Does absolute query t see absolute key j?
__device__ __forceinline__ bool visible(int mode, int64_t w, int64_t t, int64_t j) {
  switch (mode) {
    case RK_MASK_CAUSAL:
      return j <= t;
    case RK_MASK_WINDOW:
      return (t - j <= w) && (j - t <= w);
    case RK_MASK_CAUSAL_WINDOW:
      return j <= t && t - j < w;
    default:
      return true;
  }
}

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

}  // namespace

template <int DQ, int DV, bool SOFTCAP>
__global__ __launch_bounds__(NWAVES * 64) void attn_fwd_kernel(AttnArgs a, int G, int BQ,
                                                           int n_qtiles) {
  static_assert(DQ % 16 == 0 && DV % 32 == 0, "head padding");
  constexpr int KROW = DQ + 8;   // halfs per K row in LDS (16-byte pad)
  constexpr int VROW = BK + 8;   // halfs per Vᵀ row in LDS
  constexpr int K_TILE = BK * KROW;
  constexpr int V_TILE = DV * VROW;
  constexpr int NQC = DQ / 16;   // Q fragments (K=16 each)
  constexpr int NDB = DV / 32;   // output d-blocks
  constexpr int THREADS = NWAVES * 64;
  constexpr int K_CHUNKS = BK * DQ / 8;
  constexpr int V_CHUNKS = DV * BK / 8;
  constexpr int K_PER = (K_CHUNKS + THREADS - 1) / THREADS;
  constexpr int V_PER = (V_CHUNKS + THREADS - 1) / THREADS;

  __shared__ __attribute__((aligned(16))) f16 sK[2][K_TILE];
  __shared__ __attribute__((aligned(16))) f16 sV[2][V_TILE];
  __shared__ int s_flags[2];

  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int KV = a.n_kv_heads;
  const int kvh = blockIdx.x % KV;
  const int qt = n_qtiles - 1 - (int)(blockIdx.x / KV);  // heaviest causal tiles first
  const int D = a.head_dim;

  // ---- this lane's query row
  const int r = wave * 32 + (lane & 31);
  const int hh = lane >> 5;
  const int g = r / BQ;
  const int qi = qt * BQ + (r % BQ);
  const bool row_ok = (g < G) && (qi < a.n_q);
  const int h = kvh * G + min(g, G - 1);
  const int64_t t_abs = a.q0 + (row_ok ? qi : 0);

  // ---- workgroup query range and degenerate-row check
  const int q_lo = qt * BQ, q_hi = min(qt * BQ + BQ, a.n_q) - 1;
  const int64_t t_min = a.q0 + q_lo, t_max = a.q0 + q_hi;
  const int64_t kabs0 = a.k0, kabs1 = a.k0 + a.n_kv - 1;
  if (threadIdx.x == 0) s_flags[0] = 0;
  __syncthreads();
  if (row_ok) {
    int64_t lo, hi;
    vis_range(a.mask_mode, a.window, t_abs, lo, hi);
    if (max(lo, kabs0) > min(hi, kabs1)) s_flags[0] = 1;  // no visible key
  }
  __syncthreads();
  const bool degenerate = s_flags[0] != 0;

  int kt_begin = 0, kt_end = (a.n_kv + BK - 1) / BK;
  int64_t full_lo = kabs0, full_hi = kabs1;  // keys visible to every row
  {
    int64_t lo_a, hi_a, lo_b, hi_b;
    vis_range(a.mask_mode, a.window, t_min, lo_a, hi_a);
    vis_range(a.mask_mode, a.window, t_max, lo_b, hi_b);
    full_lo = max(lo_b, kabs0);
    full_hi = min(hi_a, kabs1);
    if (!degenerate) {
      const int64_t any_lo = max(lo_a, kabs0) - a.k0;  // relative key indices
      const int64_t any_hi = min(hi_b, kabs1) - a.k0;
      kt_begin = (int)(max(any_lo, (int64_t)0) / BK);
      kt_end = (int)min((any_hi / BK) + 1, (int64_t)kt_end);
    }
  }
  const float masked_x = degenerate ? MASKED_SCORE * LOG2E : -INFINITY;

  // ---- Q fragments (B operand of Sᵀ = K·Qᵀ): d = 16c + 8·hh + 0..7
  half8 qf[NQC];
  {
    const f16 *qrow = (const f16 *)a.q + (int64_t)(row_ok ? qi : 0) * a.q_tok_stride +
                      (int64_t)h * a.q_head_stride;
#pragma unroll
    for (int c = 0; c < NQC; ++c) {
      const int d0 = 16 * c + 8 * hh;
      if (row_ok && d0 < D)
        qf[c] = *(const half8 *)(qrow + d0);
      else
        qf[c] = half8{};
    }
  }

  // ---- K / Vᵀ tile staging (global → VGPR → LDS)
  const f16 *kbase = (const f16 *)a.k + (int64_t)kvh * a.k_head_stride;
  const f16 *vtbase = (const f16 *)a.vt + (int64_t)kvh * DV * a.n_kv_pad;
  uintx4 kreg[K_PER], vreg[V_PER];
  auto load_tile = [&](int kt) {
    const int kb = kt * BK;
#pragma unroll
    for (int i = 0; i < K_PER; ++i) {
      const int cidx = i * THREADS + threadIdx.x;
      const int key = cidx / (DQ / 8), ch = cidx % (DQ / 8);
      uintx4 v = {0u, 0u, 0u, 0u};
      if (cidx < K_CHUNKS && ch * 8 < D) {
        const int kk = min(kb + key, a.n_kv - 1);
        v = *(const uintx4 *)(kbase + (int64_t)kk * a.k_tok_stride + ch * 8);
      }
      kreg[i] = v;
    }
#pragma unroll
    for (int i = 0; i < V_PER; ++i) {
      const int cidx = i * THREADS + threadIdx.x;
      const int d = cidx / (BK / 8), ch = cidx % (BK / 8);
      uintx4 v = {0u, 0u, 0u, 0u};
      if (cidx < V_CHUNKS) v = *(const uintx4 *)(vtbase + (int64_t)d * a.n_kv_pad + kb + ch * 8);
      vreg[i] = v;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < K_PER; ++i) {
      const int cidx = i * THREADS + threadIdx.x;
      if (cidx < K_CHUNKS) {
        const int key = cidx / (DQ / 8), ch = cidx % (DQ / 8);
        *(uintx4 *)(&sK[buf][key * KROW + ch * 8]) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < V_PER; ++i) {
      const int cidx = i * THREADS + threadIdx.x;
      if (cidx < V_CHUNKS) {
        const int d = cidx / (BK / 8), ch = cidx % (BK / 8);
        *(uintx4 *)(&sV[buf][d * VROW + ch * 8]) = vreg[i];
      }
    }
  };

  floatx16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m_run = -INFINITY;  // running max (exp2 domain), same on lane and lane^32
  float l_run = 0.f;        // this lane's partial row sum
  const float C = SOFTCAP ? LOG2E : a.scale * LOG2E;

  if (kt_begin < kt_end) {
    load_tile(kt_begin);
    store_tile(0);
  }
  __syncthreads();

  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const int buf = (kt - kt_begin) & 1;
    if (kt + 1 < kt_end) load_tile(kt + 1);

    // Sᵀ for the two 32-key blocks of the tile.
    floatx16 s[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[sb][i] = 0.f;
      const f16 *krow = &sK[buf][(sb * 32 + (lane & 31)) * KROW + 8 * hh];
#pragma unroll
      for (int c = 0; c < NQC; ++c) {
        const half8 kf = *(const half8 *)(krow + 16 * c);
        s[sb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[c], s[sb], 0, 0, 0);
      }
    }

    // Scores in the exp2 domain with masking.
    const int kb = kt * BK;
    const bool interior = (a.k0 + kb >= full_lo) && (a.k0 + kb + BK - 1 <= full_hi) &&
                          (kb + BK <= a.n_kv) && !degenerate;
    float mt = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float x = s[sb][i];
        if constexpr (SOFTCAP) x = a.softcap * tanhf(x * a.scale / a.softcap);
        x *= C;
        if (!interior) {
          const int key = kb + sb * 32 + 8 * (i >> 2) + 4 * hh + (i & 3);
          if (key >= a.n_kv)
            x = -INFINITY;
          else if (!row_ok || !visible(a.mask_mode, a.window, t_abs, a.k0 + key))
            x = masked_x;
        }
        s[sb][i] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;

    // P as an unevaluated sum of two fp16 values: hi keeps the top 11 bits of
    // the f32 probability (exactly representable, so the round-toward-zero
    // pack is exact) and lo = p - hi carries the rest. Rounding P itself to
    // fp16 would leave ~2^-12 relative noise per probability in O.
    half8 phi[4], plo[4];
    float lsum = 0.f;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        uintx4 hw, lw;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e0 = __builtin_amdgcn_exp2f(s[sb][8 * c2 + 2 * j] - m_use);
          const float e1 = __builtin_amdgcn_exp2f(s[sb][8 * c2 + 2 * j + 1] - m_use);
          lsum += e0 + e1;
          const float h0 = __uint_as_float(__float_as_uint(e0) & 0xffffe000u);
          const float h1 = __uint_as_float(__float_as_uint(e1) & 0xffffe000u);
          hw[j] = __builtin_bit_cast(unsigned int, __builtin_amdgcn_cvt_pkrtz(h0, h1));
          lw[j] = __builtin_bit_cast(unsigned int, __builtin_amdgcn_cvt_pkrtz(e0 - h0, e1 - h1));
        }
        phi[sb * 2 + c2] = __builtin_bit_cast(half8, hw);
        plo[sb * 2 + c2] = __builtin_bit_cast(half8, lw);
      }
    }
    l_run = l_run * alpha + lsum;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[db][i] *= alpha;

    // Oᵀ += Vᵀ·Pᵀ over the four 16-key chunks (hi and lo parts).
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const half8 vf =
            *(const half8 *)(&sV[buf][(db * 32 + (lane & 31)) * VROW + 16 * c + 8 * hh]);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, phi[c], o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, plo[c], o[db], 0, 0, 0);
      }
    }

    if (kt + 1 < kt_end) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and store Oᵀ: lane holds d = 32·db + 8·(i/4) + 4·hh + i%4
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (row_ok) {
    f16 *orow = (f16 *)a.out + (int64_t)qi * a.o_tok_stride + (int64_t)h * a.o_head_stride;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d0 = 32 * db + 8 * i4 + 4 * hh;
        if (d0 < D) {
          half4 v = {(f16)(o[db][4 * i4 + 0] * inv), (f16)(o[db][4 * i4 + 1] * inv),
                     (f16)(o[db][4 * i4 + 2] * inv), (f16)(o[db][4 * i4 + 3] * inv)};
          *(half4 *)(orow + d0) = v;
        }
      }
    }
  }
}

// V [n_kv] × (head g, d) → Vt[g][d][p] for p in [0, n_kv_pad), where position
// p of each 16-key chunk holds key 8·((p%8)/4) + 4·(p/8 % 2) + p%4 of the
// chunk (the order in which the PV operand lanes consume keys). Rows d ≥ D and
// keys ≥ n_kv are zero.
__global__ void v_transpose_kernel(const f16 *__restrict__ v, int64_t tok_stride,
                                   int64_t head_stride, int64_t d_stride, int n_kv, int n_kv_pad,
                                   int D, int DVp, f16 *__restrict__ vt) {
  __shared__ f16 tile[64][65];
  const int g = blockIdx.z;
  const int key0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  const f16 *vg = v + (int64_t)g * head_stride;
  for (int idx = threadIdx.x; idx < 64 * 64; idx += blockDim.x) {
    const int kk = idx / 64, dd = idx % 64;
    const int key = key0 + kk, d = d0 + dd;
    f16 val = (f16)0.f;
    if (key < n_kv && d < D) val = vg[(int64_t)key * tok_stride + (int64_t)d * d_stride];
    tile[kk][dd] = val;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 64 * 64; idx += blockDim.x) {
    const int dd = idx / 64, p = idx % 64;
    const int d = d0 + dd;
    if (d >= DVp) continue;
    const int pc = p & 15;
    const int key_in_chunk = 8 * ((pc & 7) >> 2) + 4 * (pc >> 3) + (pc & 3);
    const int kk = (p & ~15) + key_in_chunk;
    vt[((int64_t)g * DVp + d) * n_kv_pad + key0 + p] = tile[kk][dd];
  }
}

int rk_attn_dv_pad(int head_dim) { return (head_dim + 31) / 32 * 32; }
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

template <int DQ, int DV>
static hipError_t launch_attn(const AttnArgs &a, hipStream_t st) {
  const int G = a.n_head / a.n_kv_heads;
  const int BQ = ROWS / G;
  const int n_qtiles = (a.n_q + BQ - 1) / BQ;
  dim3 grid((unsigned)(n_qtiles * a.n_kv_heads));
  if (a.softcap != 0.f)
    hipLaunchKernelGGL((attn_fwd_kernel<DQ, DV, true>), grid, dim3(NWAVES * 64), 0, st, a, G, BQ,
                       n_qtiles);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<DQ, DV, false>), grid, dim3(NWAVES * 64), 0, st, a, G,
                       BQ, n_qtiles);
  return hipGetLastError();
}

hipError_t rk_launch_attention(const AttnArgs &a, hipStream_t st) {
  const int G = a.n_head / a.n_kv_heads;
  if (G < 1 || G > ROWS || a.n_head % a.n_kv_heads) return hipErrorInvalidValue;
  switch (a.head_dim) {
    case 64:
      return launch_attn<64, 64>(a, st);
    case 72:
    case 80:
      return launch_attn<80, 96>(a, st);
    case 96:
      return launch_attn<96, 96>(a, st);
    case 112:
      return launch_attn<112, 128>(a, st);
    case 128:
      return launch_attn<128, 128>(a, st);
  }
  return hipErrorInvalidValue;
}
