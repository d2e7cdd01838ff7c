/*
 * oracle.c — CPU restatement of the royalcat/burn-rocket accelerator op surface.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the parity reference or as the
 * timed CPU baseline. The product path (burn-rocket_amd/) never calls it.
 *
 * Each function names the reference file:line it restates. The reference is
 * Rust; its Burn CPU path (burn 0.22 flex, gemm 0.19) is not in this tree, so
 * the GEMM and attention restatements follow what the reference's callers and
 * logs say that path computes (f32 accumulation over fp16-rounded inputs; a
 * TILE_KV=64 online-softmax flash kernel) — their exact accumulation order is
 * not pinned by any reference test.
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off: no FMA
 * contraction, as Rust does not contract a*b+c).
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 ---- */
/* IEEE binary16 conversions with round-to-nearest-even, as the `half` crate
 * (2.7.1) does for f16::from_f32 / to_f32 (ext.rs:2144-2170). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow → inf */
  if (e <= 0) {
    /* subnormal or zero in f16 */
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int shift = 14 - e; /* 1 - e + 13 */
    uint32_t half = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1);
    const uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++; /* may carry into exp: correct */
  return (uint16_t)(sign | half);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

void orc_f32_to_f16_vec(const float *x, uint16_t *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}
void orc_f16_to_f32_vec(const uint16_t *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_to_f32(x[i]);
}

/* ---------------------------------------------------------- fp16 GEMM ---- */
/* c[m][n] = Σ_k f32(a[m][k])·f32(b[n][k]) in f32, k ascending: the Burn CPU
 * matmul on fp16 operands widened to f32 (src/commands/gemm.rs:59-104;
 * matmul_f16's contract, ext.rs:1437-1499). Rows are independent; OpenMP over
 * rows with `threads` threads. */
void orc_gemm_f16(const uint16_t *a, const uint16_t *b, int64_t m, int64_t n, int64_t k,
                  float *c, int threads) {
  float *bf = (float *)malloc(sizeof(float) * (size_t)n * k);
  for (int64_t i = 0; i < n * k; ++i) bf[i] = orc_f16_to_f32(b[i]);
#pragma omp parallel num_threads(threads)
  {
    float *ar = (float *)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
      for (int64_t p = 0; p < k; ++p) ar[p] = orc_f16_to_f32(a[i * k + p]);
      for (int64_t j = 0; j < n; ++j) {
        const float *br = bf + j * k;
        float acc = 0.f;
        for (int64_t p = 0; p < k; ++p) acc += ar[p] * br[p];
        c[i * n + j] = acc;
      }
    }
    free(ar);
  }
  free(bf);
}

/* Same product accumulated in f64 (the board self-test's reference,
 * crates/rocket-npu/src/bin/selftest.rs:45-58). */
void orc_gemm_f16_f64(const uint16_t *a, const uint16_t *b, int64_t m, int64_t n, int64_t k,
                      double *c, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double acc = 0.0;
      for (int64_t p = 0; p < k; ++p)
        acc += (double)orc_f16_to_f32(a[i * k + p]) * (double)orc_f16_to_f32(b[j * k + p]);
      c[i * n + j] = acc;
    }
}

/* ---------------------------------------------------------- quantizers ---- */
/* One row of symmetric group-wise int8 quantization (host.rs:77-90, the same
 * as src/clef/int8.rs:18-31): scale = max(max|x|/127, 1e-12), inv = 1/scale,
 * q = clamp(round_half_away(x·inv), -127, 127). */
void orc_quantize_row_groups(const float *x, int64_t k, int64_t group, int8_t *q, float *s) {
  for (int64_t g = 0; g < k / group; ++g) {
    const float *seg = x + g * group;
    float amax = 0.f;
    for (int64_t i = 0; i < group; ++i) amax = fmaxf(amax, fabsf(seg[i]));
    float scale = amax / 127.0f;
    if (scale < 1e-12f) scale = 1e-12f;
    s[g] = scale;
    const float inv = 1.0f / scale;
    for (int64_t i = 0; i < group; ++i) {
      float v = roundf(seg[i] * inv);
      if (v > 127.f) v = 127.f;
      if (v < -127.f) v = -127.f;
      q[g * group + i] = (int8_t)v;
    }
  }
}

/* Rows of the above (quantize_i8_rows, ext.rs:1017-1029, without the M%4 pad). */
void orc_quantize_rows(const float *x, int64_t m, int64_t k, int64_t group, int8_t *q, float *s,
                       int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t r = 0; r < m; ++r)
    orc_quantize_row_groups(x + r * k, k, group, q + r * k, s + r * (k / group));
}

/* llama.cpp Q8_0 (crates/rocket-npu/src/bin/q8_bench.rs:200-220): per 32-value
 * block d = f16(amax/127), codes quantized against the stored f32(d) with
 * inv = d > 0 ? 1/d : 0, round_half_away, clamp ±127. Writes codes [n][k] and
 * d as f16 bits [n][k/32]. */
void orc_q8_0_quantize(const float *w, int64_t n, int64_t k, int8_t *q, uint16_t *d16) {
  const int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      const float *seg = w + r * k + b * 32;
      float amax = 0.f;
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(seg[i]));
      const uint16_t d = orc_f32_to_f16(amax / 127.0f);
      d16[r * nb + b] = d;
      const float scale = orc_f16_to_f32(d);
      const float inv = scale > 0.f ? 1.0f / scale : 0.f;
      for (int i = 0; i < 32; ++i) {
        float v = roundf(seg[i] * inv);
        if (v > 127.f) v = 127.f;
        if (v < -127.f) v = -127.f;
        q[r * k + b * 32 + i] = (int8_t)v;
      }
    }
}

/* GGUF Q8_0 block layout (src/util/gguf.rs:125-200): 34 bytes per block,
 * little-endian f16 d then 32 int8 codes. */
void orc_q8_0_to_blocks(const int8_t *q, const uint16_t *d16, int64_t n, int64_t k,
                        uint8_t *blocks) {
  const int64_t nb = k / 32;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < nb; ++b) {
      uint8_t *blk = blocks + (r * nb + b) * 34;
      blk[0] = (uint8_t)(d16[r * nb + b] & 0xff);
      blk[1] = (uint8_t)(d16[r * nb + b] >> 8);
      memcpy(blk + 2, q + r * k + b * 32, 32);
    }
}

/* Q8_0 dequantization (gguf.rs dequantize, Q8_0 arm): v = f32(d)·q. */
void orc_q8_0_dequant(const uint8_t *blocks, int64_t nvals, float *out) {
  for (int64_t b = 0; b < nvals / 32; ++b) {
    const uint8_t *blk = blocks + b * 34;
    const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
  }
}

/* QAT activation grid (static_code, ext.rs:1236-1240; matmul_qat
 * ext.rs:1245-1290): rs = in_scale, or per-row max(amax/127, 1e-12) when
 * in_scale == 0; q = clamp(round_ties_even(x·(1/rs)), -128, 127). */
void orc_quantize_static(const float *x, int64_t m, int64_t k, float in_scale, int8_t *q,
                         float *rs) {
  for (int64_t r = 0; r < m; ++r) {
    const float *xr = x + r * k;
    float s = in_scale;
    if (in_scale == 0.f) {
      float amax = 0.f;
      for (int64_t i = 0; i < k; ++i) amax = fmaxf(amax, fabsf(xr[i]));
      s = amax / 127.0f;
      if (s < 1e-12f) s = 1e-12f;
    }
    rs[r] = s;
    const float inv = 1.0f / s;
    for (int64_t i = 0; i < k; ++i) {
      float v = rintf(xr[i] * inv); /* default rounding mode: ties to even */
      if (v > 127.f) v = 127.f;
      if (v < -128.f) v = -128.f;
      q[r * k + i] = (int8_t)v;
    }
  }
}

/* QAT epilogue (matmul_qat, ext.rs:1330-1350): y = acc·(rs[m]·ws[n]); with an
 * output grid, y = static_code(y, 1/out_scale)·out_scale. */
void orc_qat_epilogue(const int64_t *acc, const float *rs, const float *ws, int64_t m, int64_t n,
                      float out_scale, float *y) {
  const float out_inv = out_scale != 0.f ? 1.0f / out_scale : 0.f;
  for (int64_t r = 0; r < m; ++r)
    for (int64_t c = 0; c < n; ++c) {
      float v = (float)acc[r * n + c] * (rs[r] * ws[c]);
      if (out_scale != 0.f) {
        float code = rintf(v * out_inv);
        if (code > 127.f) code = 127.f;
        if (code < -128.f) code = -128.f;
        v = code * out_scale;
      }
      y[r * n + c] = v;
    }
}

/* ------------------------------------------------------- int8 products ---- */
/* Exact integer product in int64 (I8Context::matmul's "integer-exact"
 * contract, crates/rocket-npu/src/matmul/int8.rs:12-13, 606-640;
 * bin/int8_selftest.rs:92-104). */
void orc_matmul_i8_raw(const int8_t *a, const int8_t *w, int64_t m, int64_t n, int64_t k,
                       int64_t *c, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      int64_t acc = 0;
      const int8_t *ar = a + i * k, *wr = w + j * k;
      for (int64_t p = 0; p < k; ++p) acc += (int64_t)ar[p] * (int64_t)wr[p];
      c[i * n + j] = acc;
    }
}

/* Per-32-block int32 partials p[i][j][b] (dot_i8 over one block,
 * src/clef/int8.rs:93-99). */
void orc_i8_block_partials(const int8_t *a, const int8_t *w, int64_t m, int64_t n, int64_t k,
                           int32_t *p, int threads) {
  const int64_t nb = k / 32;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j)
      for (int64_t b = 0; b < nb; ++b) {
        int32_t acc = 0;
        for (int q = 0; q < 32; ++q)
          acc += (int32_t)a[i * k + b * 32 + q] * (int32_t)w[j * k + b * 32 + q];
        p[(i * n + j) * nb + b] = acc;
      }
}

static inline int32_t dot_i8(const int8_t *a, const int8_t *b, int64_t len) {
  int32_t acc = 0;
  for (int64_t i = 0; i < len; ++i) acc += (int32_t)a[i] * (int32_t)b[i];
  return acc;
}

/* Host twin of matmul_gw (emu_matmul_gw, src/clef/int8.rs:101-158; the
 * de-tile formula of layout.rs:504-540): out[m][n] = Σ_g (a_s·w_s[n][g])·P_g,
 * groups ascending, f32 accumulation, the scale product formed first.
 * Weight groups are w_group values wide; the activation scale of group g is
 * a_s[m][(g·w_group)/a_group] (a_group == w_group is the reference's form,
 * a_group == k is per-token quantization). */
void orc_emu_matmul_gw(const int8_t *aq, const float *a_s, int64_t a_group, int64_t m,
                       int64_t k, const int8_t *wq, const float *w_s, int64_t w_group, int64_t n,
                       float *out, int threads) {
  const int64_t ng = k / w_group, nga = k / a_group;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 4)
  for (int64_t r = 0; r < m; ++r) {
    const int8_t *ar = aq + r * k;
    const float *asr = a_s + r * nga;
    for (int64_t j = 0; j < n; ++j) {
      const int8_t *wr = wq + j * k;
      const float *wsr = w_s + j * ng;
      float acc = 0.f;
      for (int64_t g = 0; g < ng; ++g) {
        const int32_t p = dot_i8(ar + g * w_group, wr + g * w_group, w_group);
        const float s = asr[(g * w_group) / a_group] * wsr[g];
        acc += s * (float)p;
      }
      out[r * n + j] = acc;
    }
  }
}

/* ----------------------------------------------------------- attention ---- */
/* Mask predicates on absolute positions (crates/burn-rocket/src/masks.rs:11-114):
 * mode 0 none, 1 causal j <= t, 2 band |t - j| <= w, 3 causal window
 * t - w < j <= t. */
int orc_mask_keep(int mode, int64_t window, int64_t t, int64_t j) {
  switch (mode) {
    case 1: return j <= t;
    case 2: return (t - j <= window) && (j - t <= window);
    case 3: return j <= t && t - j < window;
    default: return 1;
  }
}

/* One pre-softmax score (fa_score, crates/rocket-npu/src/attn/oneshot.rs:193-199):
 * s = qk·scale, soft-capped, plus the additive mask, clamped below at -30000. */
static inline float fa_score(float qk, float scale, float softcap, float mask) {
  float s = qk * scale;
  if (softcap != 0.f) s = softcap * tanhf(s / softcap);
  s = s + mask;
  return s > -30000.0f ? s : -30000.0f;
}

/* f64 attention oracle (flash_attn_ref, attn/oneshot.rs:130-189) on the
 * token-major layout the Burn API uses: q [n_q][H·D], k/v [n_kv][KV·D] as f16
 * bits; head h reads kv head h / (H/KV). The qk dot is f64, narrowed to f32
 * for fa_score; exp, row sum and the AV accumulation are f64. A row whose keys
 * are all masked sees only -30000 scores and averages V over all n_kv keys.
 * out [n_q][H·D] f64. */
void orc_attention_ref(const uint16_t *q, const uint16_t *k, const uint16_t *v, int64_t n_q,
                       int64_t n_kv, int n_head, int n_kv_heads, int head_dim, float scale,
                       float softcap, int mode, int64_t window, int64_t q0, int64_t k0,
                       double *out, int threads) {
  const int gqa = n_head / n_kv_heads, D = head_dim;
  const int64_t qs = (int64_t)n_head * D, ks = (int64_t)n_kv_heads * D;
#pragma omp parallel num_threads(threads)
  {
    double *sc = (double *)malloc(sizeof(double) * (size_t)n_kv);
    double *qf = (double *)malloc(sizeof(double) * (size_t)D);
#pragma omp for collapse(2) schedule(dynamic, 8)
    for (int h = 0; h < n_head; ++h)
      for (int64_t t = 0; t < n_q; ++t) {
        const int hk = h / gqa;
        for (int d = 0; d < D; ++d) qf[d] = orc_f16_to_f32(q[t * qs + h * D + d]);
        double mx = -INFINITY;
        for (int64_t j = 0; j < n_kv; ++j) {
          double qk = 0.0;
          for (int d = 0; d < D; ++d) qk += qf[d] * (double)orc_f16_to_f32(k[j * ks + hk * D + d]);
          const float m = orc_mask_keep(mode, window, q0 + t, k0 + j) ? 0.f : -INFINITY;
          const double s = (double)fa_score((float)qk, scale, softcap, m);
          sc[j] = s;
          if (s > mx) mx = s;
        }
        double sum = 0.0;
        for (int64_t j = 0; j < n_kv; ++j) {
          sc[j] = exp(sc[j] - mx);
          sum += sc[j];
        }
        const double inv = sum > 0.0 ? 1.0 / sum : 0.0;
        for (int d = 0; d < D; ++d) {
          double a = 0.0;
          for (int64_t j = 0; j < n_kv; ++j) a += sc[j] * (double)orc_f16_to_f32(v[j * ks + hk * D + d]);
          out[t * qs + h * D + d] = a * inv;
        }
      }
    free(sc);
    free(qf);
  }
}

/* The Burn CPU attention as the reference runs it on the host: fp16 operands
 * widened to f32, a flash kernel over key tiles of 64 with an f32 online
 * softmax and native GQA (docs/experiments/experiment-log.md:206-211;
 * forward_blocked, src/qwen3_embedding/model.rs:473-563). Masked keys are
 * excluded (additive -inf); a row with no visible key averages V over all
 * n_kv keys, as the f64 oracle does. out [n_q][H·D] f32. */
void orc_attention_flex(const uint16_t *q, const uint16_t *k, const uint16_t *v, int64_t n_q,
                        int64_t n_kv, int n_head, int n_kv_heads, int head_dim, float scale,
                        float softcap, int mode, int64_t window, int64_t q0, int64_t k0,
                        float *out, int threads) {
  const int gqa = n_head / n_kv_heads, D = head_dim;
  const int64_t qs = (int64_t)n_head * D, ks = (int64_t)n_kv_heads * D;
  enum { TILE = 64 };
  float *kf = (float *)malloc(sizeof(float) * (size_t)n_kv * ks);
  float *vf = (float *)malloc(sizeof(float) * (size_t)n_kv * ks);
  for (int64_t i = 0; i < n_kv * ks; ++i) {
    kf[i] = orc_f16_to_f32(k[i]);
    vf[i] = orc_f16_to_f32(v[i]);
  }
#pragma omp parallel num_threads(threads)
  {
    float *qf = (float *)malloc(sizeof(float) * (size_t)D);
    float *acc = (float *)malloc(sizeof(float) * (size_t)D);
    float s[TILE];
#pragma omp for collapse(2) schedule(dynamic, 8)
    for (int h = 0; h < n_head; ++h)
      for (int64_t t = 0; t < n_q; ++t) {
        const int hk = h / gqa;
        for (int d = 0; d < D; ++d) {
          qf[d] = orc_f16_to_f32(q[t * qs + h * D + d]);
          acc[d] = 0.f;
        }
        float m = -INFINITY, l = 0.f;
        int any = 0;
        for (int64_t j0 = 0; j0 < n_kv; j0 += TILE) {
          const int64_t nt = (n_kv - j0) < TILE ? (n_kv - j0) : TILE;
          float mt = -INFINITY;
          for (int64_t jj = 0; jj < nt; ++jj) {
            const int64_t j = j0 + jj;
            if (!orc_mask_keep(mode, window, q0 + t, k0 + j)) {
              s[jj] = -INFINITY;
              continue;
            }
            const float *kr = kf + j * ks + hk * D;
            float dot = 0.f;
            for (int d = 0; d < D; ++d) dot += qf[d] * kr[d];
            float x = dot * scale;
            if (softcap != 0.f) x = softcap * tanhf(x / softcap);
            s[jj] = x;
            if (x > mt) mt = x;
          }
          if (mt == -INFINITY) continue;
          any = 1;
          const float m_new = m > mt ? m : mt;
          const float alpha = expf(m - m_new);
          l *= alpha;
          for (int d = 0; d < D; ++d) acc[d] *= alpha;
          for (int64_t jj = 0; jj < nt; ++jj) {
            if (s[jj] == -INFINITY) continue;
            const float p = expf(s[jj] - m_new);
            l += p;
            const float *vr = vf + (j0 + jj) * ks + hk * D;
            for (int d = 0; d < D; ++d) acc[d] += p * vr[d];
          }
          m = m_new;
        }
        if (!any) { /* no visible key: uniform over all keys */
          for (int d = 0; d < D; ++d) {
            float a = 0.f;
            for (int64_t j = 0; j < n_kv; ++j) a += vf[j * ks + hk * D + d];
            acc[d] = a;
          }
          l = (float)n_kv;
        }
        for (int d = 0; d < D; ++d) out[t * qs + h * D + d] = acc[d] / l;
      }
    free(qf);
    free(acc);
  }
  free(kf);
  free(vf);
}

/* ----------------------------------------------------------------- MoE ---- */
/* Router (route, src/clef/model.rs:462-489): softmax_row over the experts
 * (src/clef/math.rs:138-148: max, exp(v - max), sum, divide), top-k
 * descending with ties to the lower id, optional renormalisation. */
void orc_route(const float *logits, int64_t s, int n_experts, int top_k, int norm_topk,
               uint32_t *ids, float *wts) {
  float *p = (float *)malloc(sizeof(float) * (size_t)n_experts);
  int *used = (int *)malloc(sizeof(int) * (size_t)n_experts);
  for (int64_t t = 0; t < s; ++t) {
    const float *l = logits + t * n_experts;
    float mx = -INFINITY;
    for (int e = 0; e < n_experts; ++e) mx = fmaxf(mx, l[e]);
    float sum = 0.f;
    for (int e = 0; e < n_experts; ++e) {
      p[e] = expf(l[e] - mx);
      sum += p[e];
    }
    for (int e = 0; e < n_experts; ++e) {
      p[e] /= sum;
      used[e] = 0;
    }
    float sel = 0.f;
    for (int j = 0; j < top_k; ++j) {
      int best = -1;
      for (int e = 0; e < n_experts; ++e)
        if (!used[e] && (best < 0 || p[e] > p[best])) best = e; /* strict >: lower id wins ties */
      used[best] = 1;
      ids[t * top_k + j] = (uint32_t)best;
      sel += p[best];
    }
    for (int j = 0; j < top_k; ++j) {
      const float pj = p[ids[t * top_k + j]];
      wts[t * top_k + j] = norm_topk ? pj / sel : pj;
    }
  }
  free(p);
  free(used);
}

static inline float silu(float x) { return x / (1.0f + expf(-x)); } /* model.rs:491-493 */

/* out = silu(g)·u with Clef's silu (src/clef/model.rs:491-493, used by the
 * expert workers, src/clef/engine.rs:1025-1029), in f32 with libm's expf. */
void orc_clef_silu_mul(const float *g, const float *u, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = silu(g[i]) * u[i];
}

/* W8A8 expert FFN over routed tokens, as the reference's host twin of the NPU
 * expert worker computes it (EmuWorker::run, src/clef/engine.rs:990-1043; the
 * NPU worker gw_matmul → quantize_rows(x, k, group), src/clef/engine_npu.rs:
 * 75-110, 149-207). With the Q8_0 group g = 32 of the expert weights:
 *   xq, xs  = x quantized per row per 32-value group (quantize_rows, int8.rs:
 *             18-57), xs [s][H/32];
 *   g, u    = emu_matmul_gw(xq, xs, gate / up codes and scales, group 32)
 *             (int8.rs:101-158: Σ_b (xs[b]·w_s[n][b])·P_b in block order);
 *   act     = silu(g)·u with silu(v) = v / (1 + exp(-v)) (model.rs:491-493);
 *   aq, as  = act quantized per row per 32-value group;
 *   y_e     = emu_matmul_gw(aq, as, down codes and scales, group 32), each
 *             element then multiplied by the router weight (engine.rs:649-650);
 * and each token's expert outputs are summed in ascending expert id (combine,
 * src/clef/engine.rs:317-338). A token's row is quantized the same way in
 * every expert it is routed to, so quantizing x once per token is the same.
 * Weights: gate/up codes [E][I][H] with scales [E][I][H/32], down codes
 * [E][H][I] with scales [E][H][I/32]. y [s][H]: overwritten with the sum, or,
 * with accumulate, holding the residual the expert outputs are added onto
 * (`let mut y = hid; … *a += b`, src/clef/model.rs:606-614). */
void orc_moe_experts(const float *x, int64_t s, int64_t H, int64_t I, int E, int top_k,
                     const uint32_t *ids, const float *wts, const int8_t *gq, const float *gs,
                     const int8_t *uq, const float *us, const int8_t *dq, const float *ds,
                     float *y, int accumulate, int threads) {
  int8_t *xq = (int8_t *)malloc((size_t)s * H);
  float *xs = (float *)malloc(sizeof(float) * (size_t)s * (H / 32));
  orc_quantize_rows(x, s, H, 32, xq, xs, threads);
  float *yslot = (float *)malloc(sizeof(float) * (size_t)s * top_k * H);
#pragma omp parallel num_threads(threads)
  {
    float *g = (float *)malloc(sizeof(float) * (size_t)I);
    float *u = (float *)malloc(sizeof(float) * (size_t)I);
    float *act = (float *)malloc(sizeof(float) * (size_t)I);
    int8_t *aq = (int8_t *)malloc((size_t)I);
    float *as = (float *)malloc(sizeof(float) * (size_t)(I / 32));
#pragma omp for schedule(dynamic, 4)
    for (int64_t slot = 0; slot < s * top_k; ++slot) {
      const int64_t t = slot / top_k;
      const int e = (int)ids[slot];
      const int8_t *xr = xq + t * H;
      const float *xsr = xs + t * (H / 32);
      orc_emu_matmul_gw(xr, xsr, 32, 1, H, gq + (int64_t)e * I * H, gs + (int64_t)e * I * (H / 32), 32, I, g, 1);
      orc_emu_matmul_gw(xr, xsr, 32, 1, H, uq + (int64_t)e * I * H, us + (int64_t)e * I * (H / 32), 32, I, u, 1);
      for (int64_t j = 0; j < I; ++j) act[j] = silu(g[j]) * u[j];
      orc_quantize_row_groups(act, I, 32, aq, as);
      float *yr = yslot + slot * H;
      orc_emu_matmul_gw(aq, as, 32, 1, I, dq + (int64_t)e * H * I, ds + (int64_t)e * H * (I / 32), 32, H, yr, 1);
      for (int64_t c = 0; c < H; ++c) yr[c] *= wts[slot];
    }
    free(g);
    free(u);
    free(act);
    free(aq);
    free(as);
  }
  /* combine: per token, slots in ascending expert id */
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t t = 0; t < s; ++t) {
    int order[256];
    for (int j = 0; j < top_k; ++j) order[j] = j;
    for (int a = 1; a < top_k; ++a) /* insertion sort by expert id */
      for (int b = a; b > 0 && ids[t * top_k + order[b]] < ids[t * top_k + order[b - 1]]; --b) {
        int tmp = order[b];
        order[b] = order[b - 1];
        order[b - 1] = tmp;
      }
    if (!accumulate)
      for (int64_t c = 0; c < H; ++c) y[t * H + c] = 0.f;
    for (int j = 0; j < top_k; ++j) {
      const float *yr = yslot + (t * top_k + order[j]) * H;
      for (int64_t c = 0; c < H; ++c) y[t * H + c] += yr[c];
    }
  }
  free(yslot);
  free(xq);
  free(xs);
}

/* ------------------------------------------------------------ MLP glue --- */
/* sqrt(2/π) as gelu_tanh uses it: the f64 product of FRAC_2_SQRT_PI and
 * FRAC_1_SQRT_2, rounded to f32 (host.rs:9-10, host.rs:16). */
static float sqrt_2_over_pi_f32(void) {
  return (float)(1.12837916709551257390 * 0.70710678118654752440);
}

/* Burn's gelu_approximate, tanh form (host.rs:12-18):
 * (x·(tanh((x + x·x·x·0.044715)·√(2/π)) + 1))·0.5, left to right in f32. */
float orc_gelu_tanh(float x) {
  const float inner = (x + x * x * x * 0.044715f) * sqrt_2_over_pi_f32();
  return (x * (tanhf(inner) + 1.0f)) * 0.5f;
}

/* out = gelu_tanh(gate)·up, elementwise (gelu_mul, host.rs:20-28). */
void orc_gelu_mul(const float *gate, const float *up, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_gelu_tanh(gate[i]) * up[i];
}

/* out = gate·sigmoid(gate)·up with sigmoid(x) = 1/(1 + exp(-x)), evaluated
 * (gate·sigmoid)·up (silu_mul, host.rs:30-39). */
void orc_silu_mul(const float *gate, const float *up, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float g = gate[i];
    const float sigmoid = 1.0f / (1.0f + expf(-g));
    out[i] = g * sigmoid * up[i];
  }
}

/* ------------------------------------------------------ RMSNorm, RoPE ---- */
/* RMSNorm over rows of d values: ms = (Σ x·x, summed left to right) / d,
 * inv = 1/sqrt(ms + eps), out = (x·inv)·w, or x·inv when w is NULL
 * (rms_norm_row, host.rs:40-56; applied per row by rms_norm_impl /
 * rms_norm_noscale_impl ext.rs:1093-1123). */
void orc_rms_norm(const float *x, const float *w, float *out, int64_t rows, int64_t d, float eps) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * d;
    float *o = out + r * d;
    float sum = 0.0f;
    for (int64_t i = 0; i < d; ++i) sum += xr[i] * xr[i];
    const float ms = sum / (float)d;
    const float inv = 1.0f / sqrtf(ms + eps);
    for (int64_t i = 0; i < d; ++i) o[i] = w ? xr[i] * inv * w[i] : xr[i] * inv;
  }
}

/* Rotate-half RoPE of x [b, s, h, d] with cos/sin [s, d/2]; row r of d values
 * uses table row (r / h) mod s (rope_impl ext.rs:1125-1152, rope_row
 * host.rs:58-75). */
void orc_rope(const float *x, const float *cs, const float *sn, float *out, int64_t b, int64_t s,
              int64_t h, int64_t d) {
  const int64_t half = d / 2, rows = b * s * h;
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * d, *c = cs + ((r / h) % s) * half, *sv = sn + ((r / h) % s) * half;
    float *o = out + r * d;
    for (int64_t j = 0; j < half; ++j) {
      const float x1 = xr[j], x2 = xr[half + j];
      o[j] = x1 * c[j] - x2 * sv[j];
      o[half + j] = x2 * c[j] + x1 * sv[j];
    }
  }
}

int orc_max_threads(void) { return omp_get_max_threads(); }
