// Row normalisation and rotary position embedding on the GPU.
//
// RMSNorm: out = x·inv·w, or x·inv with no weight, inv = 1/sqrt(Σx²/d + eps)
// over each row of d values (rocket_rms_norm / rocket_rms_norm_noscale,
// ext.rs:75-80 and 611-615, rms_norm_impl ext.rs:1093-1123, row formula
// host.rs:40-56).
// RoPE, rotate-half form, x [B, S, H, D] with cos/sin [S, D/2]:
//   out[j]     = x[j]·cos[j] − x[D/2 + j]·sin[j]
//   out[D/2+j] = x[D/2 + j]·cos[j] + x[j]·sin[j]
// (rocket_rope, ext.rs:82-84 and 617-619, rope_impl ext.rs:1125-1152, row
// formula host.rs:58-75).
//
// Both compute in f32 in the reference's operation order with no FMA
// contraction; x and out are f32, fp16 or bf16 (out rounded to nearest even
// in x's type); the weight and the cos/sin tables may have another float
// type. out may be the same buffer as x. Both kernels are HBM-bound: each
// value of x is read once and each value of out written once.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "vt_tile.hpp"

namespace {
constexpr int es_of(int dt) { return dt == RK_DTYPE_F32 ? 4 : 2; }
}  // namespace

// ---------------------------------------------------------------------------
// RMSNorm. A row is shared by LPR lanes (a wave holds 64/LPR rows). The row is
// cut into chunks of CV values (16 bytes when VEC, else one value); lane l
// takes chunks l, l + LPR, l + 2·LPR, ... With NC > 0 a lane keeps its (at
// most NC) chunks in registers between the sum and the scaling, so x is read
// once; NC == 0 is for rows too long for that and reads each row twice, the
// second time from cache.
// The sum of squares: each lane adds its values in order (chunk, then value),
// then the LPR partial sums meet in a butterfly. The order is fixed, so the
// result is deterministic; it differs from the reference's left-to-right sum
// only by the rounding of a different summation order.
// WT: weight element type, or -1 for no weight. The VEC kernels read CV weight
// values per chunk in one access.
// ---------------------------------------------------------------------------
template <int DT, int WT, bool VEC, int LPR, int NC>
__global__ __launch_bounds__(256) void rms_norm_kernel(const void *__restrict__ x,
                                                       const void *__restrict__ w,
                                                       void *__restrict__ out, int64_t rows, int d,
                                                       float eps) {
#pragma clang fp contract(off)
  constexpr int CV = VEC ? 16 / es_of(DT) : 1;
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, li = lane % LPR;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const int nch = d / CV;
  const float fd = (float)d;
  // the loop bound is the same for every lane of a wave (the shuffles need all 64)
  for (int64_t r0 = wave * RPW; r0 < rows; r0 += n_waves * RPW) {
    const int64_t row = r0 + lane / LPR;
    const bool live = row < rows;
    const int64_t base = row * (int64_t)d;
    float acc = 0.f;
    float v[NC > 0 ? NC : 1][CV];
    // rows of at most two chunks per lane load their weight chunks with x,
    // so the wave waits for memory once
    constexpr bool PRE = WT >= 0 && NC > 0 && NC <= 2;
    float wpre[PRE ? NC : 1][CV];
    if constexpr (NC > 0) {
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int ch = li + LPR * i;
        if (live && ch < nch) {
          dt_load_vec<DT, CV>(x, base + (int64_t)ch * CV, v[i]);
          if constexpr (PRE) dt_load_vec<WT, CV>(w, (int64_t)ch * CV, wpre[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int ch = li + LPR * i;
        if (live && ch < nch) {
#pragma unroll
          for (int e = 0; e < CV; ++e) acc += v[i][e] * v[i][e];
        }
      }
    } else {
      if (live)
        for (int ch = li; ch < nch; ch += LPR) {
          dt_load_vec<DT, CV>(x, base + (int64_t)ch * CV, v[0]);
#pragma unroll
          for (int e = 0; e < CV; ++e) acc += v[0][e] * v[0][e];
        }
    }
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    const float inv = 1.0f / sqrtf(acc / fd + eps);
    auto emit = [&](int ch, float *f, const float *wp) {
      float o[CV];
      if constexpr (WT >= 0) {
        float wv[CV];
        if (wp) {
#pragma unroll
          for (int e = 0; e < CV; ++e) wv[e] = wp[e];
        } else {
          dt_load_vec<WT, CV>(w, (int64_t)ch * CV, wv);
        }
#pragma unroll
        for (int e = 0; e < CV; ++e) o[e] = f[e] * inv * wv[e];
      } else {
#pragma unroll
        for (int e = 0; e < CV; ++e) o[e] = f[e] * inv;
      }
      dt_store_vec<DT, CV>(out, base + (int64_t)ch * CV, o);
    };
    if constexpr (NC > 0) {
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int ch = li + LPR * i;
        if (live && ch < nch) emit(ch, v[i], PRE ? wpre[PRE ? i : 0] : nullptr);
      }
    } else {
      if (live)
        for (int ch = li; ch < nch; ch += LPR) {
          dt_load_vec<DT, CV>(x, base + (int64_t)ch * CV, v[0]);
          emit(ch, v[0], nullptr);
        }
    }
  }
}

// Scalar-path kernel for weight types that differ from x's and misaligned
// buffers: one value per chunk, rows read twice, weight type at run time.
template <int DT>
__global__ __launch_bounds__(256) void rms_norm_any_kernel(const void *__restrict__ x,
                                                           const void *__restrict__ w, int wt,
                                                           void *__restrict__ out, int64_t rows,
                                                           int d, float eps) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const float fd = (float)d;
  for (int64_t row = wave; row < rows; row += n_waves) {
    const int64_t base = row * (int64_t)d;
    float acc = 0.f;
    for (int c = lane; c < d; c += 64) {
      const float f = dt_load<DT>(x, base + c);
      acc += f * f;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    const float inv = 1.0f / sqrtf(acc / fd + eps);
    for (int c = lane; c < d; c += 64) {
      const float f = dt_load<DT>(x, base + c);
      dt_store<DT>(out, base + c, w ? f * inv * dt_load_any(w, c, wt) : f * inv);
    }
  }
}

namespace {
template <int DT, int WT, bool VEC, int LPR, int NC>
hipError_t launch_rms_cfg(const void *x, const void *w, void *out, int64_t rows, int d, float eps,
                          hipStream_t st) {
  const int64_t rows_per_block = 4 * (64 / LPR);
  const unsigned blocks =
      (unsigned)std::min<int64_t>((rows + rows_per_block - 1) / rows_per_block, 16384);
  hipLaunchKernelGGL((rms_norm_kernel<DT, WT, VEC, LPR, NC>), dim3(blocks), dim3(256), 0, st, x,
                     w, out, rows, d, eps);
  return hipGetLastError();
}

// Chunks per row → (lanes per row, chunks per lane). Longer rows stream: more
// than 512 chunks of 16-bit values (holding 1024 decoded chunks measured slower
// than streaming), more than 1024 chunks of f32 (4096 values).
template <int DT, int WT>
hipError_t launch_rms_vec(const void *x, const void *w, void *out, int64_t rows, int d, float eps,
                          hipStream_t st) {
  const int nch = d / (16 / es_of(DT));
  if (nch <= 8) return launch_rms_cfg<DT, WT, true, 8, 1>(x, w, out, rows, d, eps, st);
  if (nch <= 16) return launch_rms_cfg<DT, WT, true, 16, 1>(x, w, out, rows, d, eps, st);
  if (nch <= 32) return launch_rms_cfg<DT, WT, true, 32, 1>(x, w, out, rows, d, eps, st);
  if (nch <= 64) return launch_rms_cfg<DT, WT, true, 64, 1>(x, w, out, rows, d, eps, st);
  if (nch <= 128) return launch_rms_cfg<DT, WT, true, 64, 2>(x, w, out, rows, d, eps, st);
  if (nch <= 256) return launch_rms_cfg<DT, WT, true, 64, 4>(x, w, out, rows, d, eps, st);
  if (nch <= 512) return launch_rms_cfg<DT, WT, true, 64, 8>(x, w, out, rows, d, eps, st);
  if constexpr (DT == RK_DTYPE_F32)
    if (nch <= 1024) return launch_rms_cfg<DT, WT, true, 64, 16>(x, w, out, rows, d, eps, st);
  return launch_rms_cfg<DT, WT, true, 64, 0>(x, w, out, rows, d, eps, st);
}

template <int DT>
hipError_t launch_rms_t(const void *x, const void *w, int wt, void *out, int64_t rows, int d,
                        float eps, hipStream_t st) {
  constexpr int CV = 16 / es_of(DT);
  const bool xo_vec = d % CV == 0 && (((uintptr_t)x | (uintptr_t)out) & 15) == 0;
  if (xo_vec && !w) return launch_rms_vec<DT, -1>(x, w, out, rows, d, eps, st);
  if (xo_vec && wt == DT && ((uintptr_t)w & 15) == 0)
    return launch_rms_vec<DT, DT>(x, w, out, rows, d, eps, st);
  const unsigned blocks = (unsigned)std::min<int64_t>((rows + 3) / 4, 16384);
  hipLaunchKernelGGL((rms_norm_any_kernel<DT>), dim3(blocks), dim3(256), 0, st, x, w, wt, out,
                     rows, d, eps);
  return hipGetLastError();
}
}  // namespace

hipError_t rk_launch_rms_norm(const void *x, const void *w, int w_dtype, void *out, int64_t rows,
                              int d, float eps, int dtype, hipStream_t st) {
  if (rows <= 0 || d <= 0) return hipSuccess;
  switch (dtype) {
    case RK_DTYPE_F32: return launch_rms_t<RK_DTYPE_F32>(x, w, w_dtype, out, rows, d, eps, st);
    case RK_DTYPE_F16: return launch_rms_t<RK_DTYPE_F16>(x, w, w_dtype, out, rows, d, eps, st);
    case RK_DTYPE_BF16: return launch_rms_t<RK_DTYPE_BF16>(x, w, w_dtype, out, rows, d, eps, st);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// RoPE. A thread rotates CV consecutive pairs (j, D/2 + j) of one row
// (b, s, h); a block covers 256/hc whole rows, hc = (D/2)/CV, or one row in
// steps of 256 when hc > 256. Row r = (b·S + s)·H + h reads table row s =
// (r / H) mod S.
// ---------------------------------------------------------------------------
template <int DT, int CT, int CV>
__global__ __launch_bounds__(256) void rope_kernel(const void *__restrict__ x,
                                                   const void *__restrict__ cs,
                                                   const void *__restrict__ sn,
                                                   void *__restrict__ out, int rows, int S, int H,
                                                   int half) {
#pragma clang fp contract(off)
  const int hc = half / CV;
  const int rpb = hc >= 256 ? 1 : 256 / hc;
  const int t = threadIdx.x;
  const int rl = t / hc;
  const int row = blockIdx.x * rpb + rl;
  if (rl >= rpb || row >= rows) return;
  const int si = (row / H) % S;
  const int64_t xb = (int64_t)row * (2 * half), tb = (int64_t)si * half;
  for (int jc = t % hc; jc < hc; jc += 256) {
    const int j = jc * CV;
    float x1[CV], x2[CV], c[CV], s[CV], o1[CV], o2[CV];
    dt_load_vec<DT, CV>(x, xb + j, x1);
    dt_load_vec<DT, CV>(x, xb + half + j, x2);
    dt_load_vec<CT, CV>(cs, tb + j, c);
    dt_load_vec<CT, CV>(sn, tb + j, s);
#pragma unroll
    for (int e = 0; e < CV; ++e) {
      o1[e] = x1[e] * c[e] - x2[e] * s[e];
      o2[e] = x2[e] * c[e] + x1[e] * s[e];
    }
    dt_store_vec<DT, CV>(out, xb + j, o1);
    dt_store_vec<DT, CV>(out, xb + half + j, o2);
  }
}

namespace {
template <int DT, int CT, int CV>
hipError_t launch_rope_cfg(const void *x, const void *cs, const void *sn, void *out, int rows,
                           int S, int H, int half, hipStream_t st) {
  const int hc = half / CV;
  const int rpb = hc >= 256 ? 1 : 256 / hc;
  const unsigned blocks = (unsigned)((rows + rpb - 1) / rpb);
  hipLaunchKernelGGL((rope_kernel<DT, CT, CV>), dim3(blocks), dim3(256), 0, st, x, cs, sn, out,
                     rows, S, H, half);
  return hipGetLastError();
}

// The widest CV (at most 16 bytes of x) that divides D/2 and that every
// buffer's alignment allows.
template <int DT, int CT>
hipError_t launch_rope_t(const void *x, const void *cs, const void *sn, void *out, int rows, int S,
                         int H, int half, hipStream_t st) {
  const uintptr_t xa = (uintptr_t)x | (uintptr_t)out, ca = (uintptr_t)cs | (uintptr_t)sn;
  auto fits = [&](int cv) {
    return half % cv == 0 && xa % (cv * es_of(DT)) == 0 && ca % (cv * es_of(CT)) == 0;
  };
  if constexpr (DT != RK_DTYPE_F32)
    if (fits(8)) return launch_rope_cfg<DT, CT, 8>(x, cs, sn, out, rows, S, H, half, st);
  if (fits(4)) return launch_rope_cfg<DT, CT, 4>(x, cs, sn, out, rows, S, H, half, st);
  if (fits(2)) return launch_rope_cfg<DT, CT, 2>(x, cs, sn, out, rows, S, H, half, st);
  return launch_rope_cfg<DT, CT, 1>(x, cs, sn, out, rows, S, H, half, st);
}

template <int DT>
hipError_t launch_rope_x(const void *x, const void *cs, const void *sn, int ct, void *out,
                         int rows, int S, int H, int half, hipStream_t st) {
  switch (ct) {
    case RK_DTYPE_F32: return launch_rope_t<DT, RK_DTYPE_F32>(x, cs, sn, out, rows, S, H, half, st);
    case RK_DTYPE_F16: return launch_rope_t<DT, RK_DTYPE_F16>(x, cs, sn, out, rows, S, H, half, st);
    case RK_DTYPE_BF16: return launch_rope_t<DT, RK_DTYPE_BF16>(x, cs, sn, out, rows, S, H, half, st);
  }
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t rk_launch_rope(const void *x, const void *cs, const void *sn, int cs_dtype, void *out,
                          int rows, int S, int H, int half, int dtype, hipStream_t st) {
  if (rows <= 0 || half <= 0) return hipSuccess;
  switch (dtype) {
    case RK_DTYPE_F32: return launch_rope_x<RK_DTYPE_F32>(x, cs, sn, cs_dtype, out, rows, S, H, half, st);
    case RK_DTYPE_F16: return launch_rope_x<RK_DTYPE_F16>(x, cs, sn, cs_dtype, out, rows, S, H, half, st);
    case RK_DTYPE_BF16: return launch_rope_x<RK_DTYPE_BF16>(x, cs, sn, cs_dtype, out, rows, S, H, half, st);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Attention prologue of a fused q|k|v projection (the Qwen3 layer,
// src/qwen3_embedding/model.rs:355-376): per head, RMSNorm over the head dim
// with the q or k norm weight, the result rounded to the element type (as the
// reference's separate rms_norm op returns it), then rotate-half RoPE at the
// token's position; in place, over the HQ q heads and the HK k heads that
// follow them in each token's row. V is not touched.
// A head row of D values is nch = D/CV chunks, one per lane, on LPR lanes
// (a power of two >= nch); RoPE partners chunk c with chunk c ± D/(2·CV),
// taken from the partner lane by a cross-lane read. The sum of squares
// follows the order of rms_norm_kernel with the same CV and LPR.
// ---------------------------------------------------------------------------
template <int DT, int CT, int CV, int G>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(void *__restrict__ qkv,
                                                           int64_t row_stride, int S, int HQ,
                                                           int HK, int D, int lpr,
                                                           const void *__restrict__ wq,
                                                           const void *__restrict__ wk, float eps,
                                                           const void *__restrict__ cs,
                                                           const void *__restrict__ sn,
                                                           QknrVt vtj) {
#pragma clang fp contract(off)
  // Blocks from vtj.nb_norm on rewrite V (the HK heads after the k heads) as
  // the attention kernel's Vᵀ, one 64-key × 64-d tile each.
  if ((int)blockIdx.x >= vtj.nb_norm) {
    __shared__ vt_half8 tile[64][8];
    const int t = (int)blockIdx.x - vtj.nb_norm;
    const int kb = t % vtj.tiles_k, rest = t / vtj.tiles_k;
    const int db = rest % vtj.tiles_d, g = rest / vtj.tiles_d;
    const f16 *v = (const f16 *)qkv + (int64_t)(HQ + HK) * D;
    vt_tile(v, row_stride, D, 1, S, vtj.n_kv_pad, D, vtj.dv_pad, (f16 *)vtj.vt, kb, db, g, tile,
            threadIdx.x);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int li = lane & (lpr - 1), grp0 = lane - li;
  const int rpw = 64 / lpr;
  const int nch = D / CV, hc = nch / 2, half = D / 2;
  const int heads = HQ + HK;
  const int64_t rows = (int64_t)S * heads;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n_waves = ((int64_t)vtj.nb_norm * blockDim.x) >> 6;
  const float fd = (float)D;
  const bool has_w = wq != nullptr;
  const int partner = grp0 + (li < hc ? li + hc : li - hc);
  const bool lo = li < hc;
  const int j = (lo ? li : li - hc) * CV;
  // G row groups per pass; all their loads (x, weight, table entries) are
  // issued before any arithmetic, so a wave keeps G groups in flight
  for (int64_t r0 = wave * rpw * G; r0 < rows; r0 += n_waves * rpw * G) {
    dt_raw<DT, CV> xr[G], wr[G];
    dt_raw<CT, CV> cr[G], sr[G];
    bool live[G];
    int64_t base[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t row = r0 + g * rpw + lane / lpr;
      live[g] = row < rows && li < nch;
      // rows < 2^31 (checked by the caller): 32-bit division
      const int t = (int)((uint32_t)row / (uint32_t)heads);
      const int hh = (int)row - t * heads;
      base[g] = (int64_t)t * row_stride + (int64_t)hh * D + (int64_t)li * CV;
#pragma unroll
      for (int k = 0; k < dt_raw<DT, CV>::WORDS; ++k) xr[g].w[k] = wr[g].w[k] = 0;
#pragma unroll
      for (int k = 0; k < dt_raw<CT, CV>::WORDS; ++k) cr[g].w[k] = sr[g].w[k] = 0;
      if (live[g]) {
        dt_load_raw<DT, CV>(qkv, base[g], xr[g]);
        if (has_w) dt_load_raw<DT, CV>(hh < HQ ? wq : wk, (int64_t)li * CV, wr[g]);
        dt_load_raw<CT, CV>(cs, (int64_t)t * half + j, cr[g]);
        dt_load_raw<CT, CV>(sn, (int64_t)t * half + j, sr[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float f[CV];
      dt_decode_raw<DT, CV>(xr[g], f);
      if (has_w) {
        float wv[CV];
        dt_decode_raw<DT, CV>(wr[g], wv);
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < CV; ++e) acc += f[e] * f[e];
        for (int off = lpr / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
        const float inv = 1.0f / sqrtf(acc / fd + eps);
#pragma unroll
        for (int e = 0; e < CV; ++e) f[e] = dt_decode<DT>(dt_encode<DT>(f[e] * inv * wv[e]));
      }
      float p[CV];
#pragma unroll
      for (int e = 0; e < CV; ++e) p[e] = __shfl(f[e], partner, 64);
      if (live[g]) {
        float c[CV], s[CV], o[CV];
        dt_decode_raw<CT, CV>(cr[g], c);
        dt_decode_raw<CT, CV>(sr[g], s);
#pragma unroll
        for (int e = 0; e < CV; ++e)
          o[e] = lo ? f[e] * c[e] - p[e] * s[e] : f[e] * c[e] + p[e] * s[e];
        dt_store_vec<DT, CV>(qkv, base[g], o);
      }
    }
  }
}

namespace {
template <int DT, int CT, int CV>
hipError_t launch_qknr_cfg(void *qkv, int64_t row_stride, int S, int HQ, int HK, int D,
                           const void *wq, const void *wk, float eps, const void *cs,
                           const void *sn, QknrVt vtj, hipStream_t st) {
  const int nch = D / CV;
  int lpr = 1;
  while (lpr < nch) lpr <<= 1;
  // row groups per wave pass (RK_QKNR_GROUPS = 1, 2 or 4 overrides). Measured
  // on the Qwen3 q|k|v shape [3633, 4096] fp16: 11.6 / 11.1 / 12.6 µs.
  const int knob = rk_knob("RK_QKNR_GROUPS", 2);
  const int g = knob == 1 || knob == 4 ? knob : 2;
  const int64_t rows = (int64_t)S * (HQ + HK), rows_per_block = 4 * (64 / lpr) * g;
  const int nb = (int)std::min<int64_t>((rows + rows_per_block - 1) / rows_per_block, 16384);
  vtj.nb_norm = nb;
  const unsigned blocks = (unsigned)nb + (vtj.vt ? (unsigned)(vtj.tiles_k * vtj.tiles_d * HK) : 0u);
  if (g == 1)
    hipLaunchKernelGGL((qk_norm_rope_kernel<DT, CT, CV, 1>), dim3(blocks), dim3(256), 0, st, qkv,
                       row_stride, S, HQ, HK, D, lpr, wq, wk, eps, cs, sn, vtj);
  else if (g == 2)
    hipLaunchKernelGGL((qk_norm_rope_kernel<DT, CT, CV, 2>), dim3(blocks), dim3(256), 0, st, qkv,
                       row_stride, S, HQ, HK, D, lpr, wq, wk, eps, cs, sn, vtj);
  else
    hipLaunchKernelGGL((qk_norm_rope_kernel<DT, CT, CV, 4>), dim3(blocks), dim3(256), 0, st, qkv,
                       row_stride, S, HQ, HK, D, lpr, wq, wk, eps, cs, sn, vtj);
  return hipGetLastError();
}

template <int DT, int CT>
hipError_t launch_qknr_t(int cv, void *qkv, int64_t row_stride, int S, int HQ, int HK, int D,
                         const void *wq, const void *wk, float eps, const void *cs,
                         const void *sn, QknrVt vtj, hipStream_t st) {
  switch (cv) {
    case 8:
      if constexpr (DT != RK_DTYPE_F32)
        return launch_qknr_cfg<DT, CT, 8>(qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st);
      break;
    case 4: return launch_qknr_cfg<DT, CT, 4>(qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st);
    case 2: return launch_qknr_cfg<DT, CT, 2>(qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st);
    case 1: return launch_qknr_cfg<DT, CT, 1>(qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st);
  }
  return hipErrorInvalidValue;
}
}  // namespace

int rk_qk_norm_rope_cv(const void *qkv, int64_t row_stride, int D, int dtype, const void *wq,
                       const void *wk, const void *cs, const void *sn, int cs_dtype) {
  const int es = es_of(dtype), ces = es_of(cs_dtype);
  for (int cv = 16 / es; cv >= 1; cv >>= 1) {
    const bool ok = (D / 2) % cv == 0 && row_stride % cv == 0 && D / cv <= 64 &&
                    (uintptr_t)qkv % (cv * es) == 0 && (uintptr_t)wq % (cv * es) == 0 &&
                    (uintptr_t)wk % (cv * es) == 0 &&
                    (((uintptr_t)cs | (uintptr_t)sn) % (cv * ces)) == 0;
    if (ok) return cv;
  }
  return 0;
}

hipError_t rk_launch_qk_norm_rope(void *qkv, int64_t row_stride, int S, int HQ, int HK, int D,
                                  const void *wq, const void *wk, float eps, const void *cs,
                                  const void *sn, int cs_dtype, int dtype, hipStream_t st,
                                  void *vt, int n_kv_pad, int dv_pad) {
  if (S <= 0 || HQ + HK <= 0) return hipSuccess;
  QknrVt vtj{};
  if (vt) {
    // Vᵀ tiles only for fp16 V (the attention kernel's operand type)
    if (dtype != RK_DTYPE_F16 || n_kv_pad % 64 != 0 || D % 8 != 0) return hipErrorInvalidValue;
    vtj.vt = vt;
    vtj.n_kv_pad = n_kv_pad;
    vtj.dv_pad = dv_pad;
    vtj.tiles_k = n_kv_pad / 64;
    vtj.tiles_d = (dv_pad + 63) / 64;
  }
  const int cv = rk_qk_norm_rope_cv(qkv, row_stride, D, dtype, wq, wk, cs, sn, cs_dtype);
  if (cv == 0) return hipErrorInvalidValue;
  const bool cs_f32 = cs_dtype == RK_DTYPE_F32;
  if (cs_dtype != dtype && !cs_f32) return hipErrorInvalidValue;
  switch (dtype) {
    case RK_DTYPE_F32:
      return launch_qknr_t<RK_DTYPE_F32, RK_DTYPE_F32>(cv, qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st);
    case RK_DTYPE_F16:
      return cs_f32 ? launch_qknr_t<RK_DTYPE_F16, RK_DTYPE_F32>(cv, qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st)
                    : launch_qknr_t<RK_DTYPE_F16, RK_DTYPE_F16>(cv, qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st);
    case RK_DTYPE_BF16:
      return cs_f32 ? launch_qknr_t<RK_DTYPE_BF16, RK_DTYPE_F32>(cv, qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st)
                    : launch_qknr_t<RK_DTYPE_BF16, RK_DTYPE_BF16>(cv, qkv, row_stride, S, HQ, HK, D, wq, wk, eps, cs, sn, vtj, st);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// RMSNorm followed by the per-token int8 quantizer, one pass: y = RMSNorm(x)
// rounded to x's type (what the separate op returns), then scale[row] =
// max(amax(y)/127, 1e-12) and q = round-half-away(y·(1/scale)) clamped to
// ±127 (quantize_row_groups with one group per row, host.rs:77-90) — the
// activation side of a per-token W8A8 GEMM after a norm. Rows are held in
// registers (NC chunks of 16 bytes per lane on LPR lanes); the row maximum
// is a butterfly of fmaxf, exact in any order.
// ---------------------------------------------------------------------------
template <int DT, int WT, int LPR, int NC>
__global__ __launch_bounds__(256) void rms_quant_kernel(const void *__restrict__ x,
                                                        const void *__restrict__ w,
                                                        int8_t *__restrict__ q,
                                                        float *__restrict__ qscale, int64_t rows,
                                                        int d, float eps) {
#pragma clang fp contract(off)
  constexpr int CV = 16 / es_of(DT);
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, li = lane % LPR;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t n_waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const int nch = d / CV;
  const float fd = (float)d;
  for (int64_t r0 = wave * RPW; r0 < rows; r0 += n_waves * RPW) {
    const int64_t row = r0 + lane / LPR;
    const bool live = row < rows;
    const int64_t base = row * (int64_t)d;
    float v[NC][CV];
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int ch = li + LPR * i;
#pragma unroll
      for (int e = 0; e < CV; ++e) v[i][e] = 0.f;
      if (live && ch < nch) dt_load_vec<DT, CV>(x, base + (int64_t)ch * CV, v[i]);
    }
#pragma unroll
    for (int i = 0; i < NC; ++i)
#pragma unroll
      for (int e = 0; e < CV; ++e) acc += v[i][e] * v[i][e];
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    const float inv = 1.0f / sqrtf(acc / fd + eps);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int ch = li + LPR * i;
      if (live && ch < nch) {
        float wv[CV];
        if constexpr (WT >= 0) dt_load_vec<WT, CV>(w, (int64_t)ch * CV, wv);
#pragma unroll
        for (int e = 0; e < CV; ++e) {
          const float o = WT >= 0 ? v[i][e] * inv * wv[e] : v[i][e] * inv;
          v[i][e] = dt_decode<DT>(dt_encode<DT>(o));
          amax = fmaxf(amax, fabsf(v[i][e]));
        }
      }
    }
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float s = fmaxf(amax / 127.0f, 1e-12f);
    const float qinv = 1.0f / s;
    if (live && li == 0) qscale[row] = s;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int ch = li + LPR * i;
      if (live && ch < nch) {
        uint32_t words[CV / 4];
#pragma unroll
        for (int k = 0; k < CV / 4; ++k) words[k] = 0;
#pragma unroll
        for (int e = 0; e < CV; ++e) {
          const float c = fminf(fmaxf(roundf(v[i][e] * qinv), -127.0f), 127.0f);
          words[e / 4] |= (uint32_t)(uint8_t)(int8_t)(int)c << (8 * (e % 4));
        }
        int8_t *qp = q + base + (int64_t)ch * CV;
        if constexpr (CV == 8) *(uintx2 *)qp = uintx2{words[0], words[1]};
        else *(uint32_t *)qp = words[0];
      }
    }
  }
}

namespace {
template <int DT, int WT, int LPR, int NC>
hipError_t launch_rq_cfg(const void *x, const void *w, int8_t *q, float *qs, int64_t rows, int d,
                         float eps, hipStream_t st) {
  const int64_t rows_per_block = 4 * (64 / LPR);
  const unsigned blocks =
      (unsigned)std::min<int64_t>((rows + rows_per_block - 1) / rows_per_block, 16384);
  hipLaunchKernelGGL((rms_quant_kernel<DT, WT, LPR, NC>), dim3(blocks), dim3(256), 0, st, x, w, q,
                     qs, rows, d, eps);
  return hipGetLastError();
}
template <int DT, int WT>
hipError_t launch_rq_t(const void *x, const void *w, int8_t *q, float *qs, int64_t rows, int d,
                       float eps, hipStream_t st) {
  const int nch = d / (16 / es_of(DT));
  if (nch <= 8) return launch_rq_cfg<DT, WT, 8, 1>(x, w, q, qs, rows, d, eps, st);
  if (nch <= 16) return launch_rq_cfg<DT, WT, 16, 1>(x, w, q, qs, rows, d, eps, st);
  if (nch <= 32) return launch_rq_cfg<DT, WT, 32, 1>(x, w, q, qs, rows, d, eps, st);
  if (nch <= 64) return launch_rq_cfg<DT, WT, 64, 1>(x, w, q, qs, rows, d, eps, st);
  if (nch <= 128) return launch_rq_cfg<DT, WT, 64, 2>(x, w, q, qs, rows, d, eps, st);
  if (nch <= 256) return launch_rq_cfg<DT, WT, 64, 4>(x, w, q, qs, rows, d, eps, st);
  return launch_rq_cfg<DT, WT, 64, 8>(x, w, q, qs, rows, d, eps, st);
}
}  // namespace

bool rk_rms_quant_fits(const void *x, const void *w, int w_dtype, const int8_t *q, int d, int dtype) {
  const int cv = 16 / es_of(dtype);
  return d % cv == 0 && d / cv <= 512 && (w == nullptr || w_dtype == dtype) &&
         (((uintptr_t)x | (uintptr_t)w) & 15) == 0 && ((uintptr_t)q % cv) == 0;
}

hipError_t rk_launch_rms_quant(const void *x, const void *w, int8_t *q, float *qs, int64_t rows,
                               int d, float eps, int dtype, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  switch (dtype) {
    case RK_DTYPE_F32:
      return w ? launch_rq_t<RK_DTYPE_F32, RK_DTYPE_F32>(x, w, q, qs, rows, d, eps, st)
               : launch_rq_t<RK_DTYPE_F32, -1>(x, w, q, qs, rows, d, eps, st);
    case RK_DTYPE_F16:
      return w ? launch_rq_t<RK_DTYPE_F16, RK_DTYPE_F16>(x, w, q, qs, rows, d, eps, st)
               : launch_rq_t<RK_DTYPE_F16, -1>(x, w, q, qs, rows, d, eps, st);
    case RK_DTYPE_BF16:
      return w ? launch_rq_t<RK_DTYPE_BF16, RK_DTYPE_BF16>(x, w, q, qs, rows, d, eps, st)
               : launch_rq_t<RK_DTYPE_BF16, -1>(x, w, q, qs, rows, d, eps, st);
  }
  return hipErrorInvalidValue;
}
