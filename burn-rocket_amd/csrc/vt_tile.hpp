// The Vᵀ rewrite in front of the attention kernel, as a device function so
// that another launch can run its tiles (the q|k prologue does).
#pragma once

#include "common.hpp"

typedef _Float16 vt_half8 __attribute__((ext_vector_type(8)));

// V [n_kv] × (head g, d) → Vt[g][d][p] for p in [0, n_kv_pad): slot p of each
// 32-key chunk holds key 4·(p/8 % 4) + p%4 + 16·((p%8)/4) of the chunk (the
// order in which the PV operand lanes consume keys). Rows d ≥ D and keys ≥
// n_kv are zero. One tile is 64 keys × 64 d, moved by 256 threads: 16-byte
// loads along d into LDS, 16-byte stores of 8 consecutive slots along the keys.
// The LDS tile holds key row kk as 8 chunks of 8 d, chunk c at position
// c ^ vt_swz(kk): the 8 key rows that one lane group reads for a slot are
// kk0 + {0, 4, 8, 12, 32, 36, 40, 44} (+ a common offset below 4 or 16..19),
// which vt_swz maps to 8 different positions, so the 2-byte reads that
// gather a slot vector hit 8 different bank groups.
__device__ __forceinline__ int vt_swz(int kk) { return ((kk >> 2) & 3) | ((kk >> 3) & 4); }

// Tile (key block kb, d block db, kv head g); tile: 64 × 8 LDS chunks; tid in [0, 256).
__device__ __forceinline__ void vt_tile(const f16 *__restrict__ v, int64_t tok_stride,
                                        int64_t head_stride, int64_t d_stride, int n_kv,
                                        int n_kv_pad, int D, int DVp, f16 *__restrict__ vt, int kb,
                                        int db, int g, vt_half8 (*tile)[8], int tid) {
  const int key0 = kb * 64, d0 = db * 64;
  const f16 *vg = v + (int64_t)g * head_stride;
  if (d_stride == 1) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int idx = r * 256 + tid;  // 64 keys × 8 chunks of 8 d
      const int kk = idx >> 3, ch = idx & 7;
      const int key = key0 + kk, d = d0 + ch * 8;
      vt_half8 x = vt_half8{};
      if (key < n_kv && d < D) x = *(const vt_half8 *)(vg + (int64_t)key * tok_stride + d);
      tile[kk][ch ^ vt_swz(kk)] = x;
    }
  } else {
    f16 *t16 = (f16 *)tile;
    for (int idx = tid; idx < 64 * 64; idx += 256) {
      const int kk = idx / 64, dd = idx % 64;
      const int key = key0 + kk, d = d0 + dd;
      t16[kk * 64 + ((dd >> 3) ^ vt_swz(kk)) * 8 + (dd & 7)] =
          (key < n_kv && d < D) ? vg[(int64_t)key * tok_stride + (int64_t)d * d_stride] : (f16)0.f;
    }
  }
  __syncthreads();
  const f16 *t16 = (const f16 *)tile;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = r * 256 + tid;  // 64 d rows × 8 chunks of 8 slots
    const int dd = idx >> 3, ch = idx & 7;
    const int d = d0 + dd;
    if (d >= DVp) continue;
    vt_half8 y;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int p = ch * 8 + i, pc = p & 31;
      const int kk = (p & ~31) + 4 * ((pc >> 3) & 3) + (pc & 3) + 16 * ((pc & 7) >> 2);
      y[i] = t16[kk * 64 + ((dd >> 3) ^ vt_swz(kk)) * 8 + (dd & 7)];
    }
    *(vt_half8 *)(vt + ((int64_t)g * DVp + d) * n_kv_pad + key0 + ch * 8) = y;
  }
}
