// Host-callable launchers of the gfx950 kernels (defined in the .hip files).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

// Integer tuning knob from the environment (read at every call, like the
// reference's ROCKET_* knobs); `dflt` when unset or not a number.
static inline int rk_knob(const char *name, int dflt) {
  const char *v = getenv(name);
  if (!v || !*v) return dflt;
  char *end = nullptr;
  const long x = strtol(v, &end, 10);
  return (end && *end == 0) ? (int)x : dflt;
}

// fp16 GEMM launch plan: tile configuration, K split and the split's
// workspace (f32 partial tiles, arrival counters that start at zero and are
// left at zero by every launch).
struct F16Plan {
  int cfg = 4, ksplit = 1;
  int64_t part_floats = 0;
  int64_t n_cnt = 0;
};
F16Plan rk_gemm_f16_plan(int M, int N, int K, int num_cus, bool glu);
// fp16 GEMM, C[M,N] = A[M,K]·B[N,K]ᵀ, K % 8 == 0.
hipError_t rk_launch_gemm_f16(const F16Plan &p, const void *A, const void *B, void *C, int M, int N, int K,
                              float *part, unsigned *cnt, hipStream_t st);

// fp16 GEMM with a gate|up glue epilogue: B [N, K] holds gate and up rows
// interleaved per 16 (N = 32·ceil(n_out/16)); C [M, n_out] = glue(gate·a,
// up·a) with both products rounded to fp16 first; glu 1 silu·up, 2 gelu·up;
// C f32 or (out_f16) fp16. p from rk_gemm_f16_plan(.., glu = true).
hipError_t rk_launch_gemm_f16_glu(const F16Plan &p, const void *A, const void *B, void *C, int M, int N, int K,
                                  int n_out, int glu, bool out_f16, float *part, unsigned *cnt, hipStream_t st);
// Element type conversion (RK_DTYPE_* src → dst), round to nearest even.
hipError_t rk_launch_cast(const void *x, int src, void *y, int dst, int64_t n, hipStream_t st);
// f32 rows [n, k] → fp16 (RNE) rows (r/16)·grp_stride + grp_off + r%16 of out.
hipError_t rk_launch_f32_to_f16_rows(const float *x, int64_t n, int64_t k, int grp_stride,
                                     int grp_off, void *out, hipStream_t st);

enum I8Mode { I8_PER_TOKEN = 0, I8_PER_GROUP = 1, I8_RAW = 2, I8_PARTIALS = 3 };

struct I8GemmArgs {
  const int8_t *A;     // [M, K]
  const float *AS;     // activation scales [M, as_stride] (PER_TOKEN: [M, 1])
  int as_stride;       // K / a_group
  int a_gb;            // a_group / 32 (PER_GROUP)
  const int8_t *W;     // [N, K]
  const float *WS;     // weight scale per 32-block [N, ws_stride]
  int ws_stride;       // K/32 rounded up to a multiple of 4
  bool ws_f16 = false; // every weight scale is an fp16 value
  int gb;              // weight group / 32
  void *C;             // f32 / fp16 [M, N], int32 [M, N] (RAW), int32 [M, N, K/32] (PARTIALS)
  int M, N, K;
  int mode;            // I8Mode
  bool out_f16;
  int num_cus;
  // Per-token Q8_0 only: 1 silu·up, 2 gelu·up over gate/up rows interleaved
  // in 16-row groups (N = 32·ceil(n_out/16) rows), output C [M, n_out].
  int glu = 0;
  int n_out = 0;
};
hipError_t rk_launch_gemm_i8(const I8GemmArgs &g, hipStream_t st);

// Element-wise conversions.
hipError_t rk_launch_f32_to_f16(const float *x, void *y, int64_t n, hipStream_t st);
hipError_t rk_launch_f32_to_f16_checked(const float *x, void *y, int64_t n, int *flag, hipStream_t st);
hipError_t rk_launch_f16_to_f32(const void *x, float *y, int64_t n, hipStream_t st);

// MLP glue: op 0 silu_mul, 1 gelu_mul; dtype RK_DTYPE_*.
hipError_t rk_launch_glue(int op, const void *a, const void *b, void *out, int64_t n, int dtype,
                          hipStream_t st);

// RMSNorm over rows of d values: w null (no weight) or of type w_dtype.
hipError_t rk_launch_rms_norm(const void *x, const void *w, int w_dtype, void *out, int64_t rows,
                              int d, float eps, int dtype, hipStream_t st);
// Rotate-half RoPE over rows = B·S·H rows of 2·half values; cos/sin [S, half]
// of type cs_dtype.
hipError_t rk_launch_rope(const void *x, const void *cs, const void *sn, int cs_dtype, void *out,
                          int rows, int S, int H, int half, int dtype, hipStream_t st);

// In-place per-head RMSNorm (weights wq / wk of type dtype, or both null) and
// RoPE over the HQ q heads and HK k heads at the start of each of S token
// rows of a q|k|v buffer. rk_qk_norm_rope_cv: the vector width the launch
// will use, 0 when none fits (then the launch fails).
int rk_qk_norm_rope_cv(const void *qkv, int64_t row_stride, int D, int dtype, const void *wq,
                       const void *wk, const void *cs, const void *sn, int cs_dtype);
// With vt non-null (fp16 only) the same launch also writes V — the HK heads
// after the k heads — as the attention kernel's Vᵀ [HK][dv_pad][n_kv_pad].
struct QknrVt {
  void *vt;        // null: no Vᵀ tiles
  int n_kv_pad, dv_pad;
  int tiles_k, tiles_d;
  int nb_norm;     // blocks of the norm part (set by the launcher)
};
hipError_t rk_launch_qk_norm_rope(void *qkv, int64_t row_stride, int S, int HQ, int HK, int D,
                                  const void *wq, const void *wk, float eps, const void *cs,
                                  const void *sn, int cs_dtype, int dtype, hipStream_t st,
                                  void *vt = nullptr, int n_kv_pad = 0, int dv_pad = 0);

// RMSNorm (w null: scale-free; else of x's type) rounded to x's type, then the
// per-token int8 quantizer, in one pass; rk_rms_quant_fits: whether the
// shape and alignment take this kernel (rows of at most 512 16-byte chunks).
bool rk_rms_quant_fits(const void *x, const void *w, int w_dtype, const int8_t *q, int d, int dtype);
hipError_t rk_launch_rms_quant(const void *x, const void *w, int8_t *q, float *qs, int64_t rows,
                               int d, float eps, int dtype, hipStream_t st);

// Per-row symmetric quantizer (scale = max(amax/127, 1e-12), codes
// round-half-away(x·(1/scale)) clamped to ±127), `group` values per scale.
hipError_t rk_launch_quantize_rows(const float *x, int64_t m, int64_t k, int64_t group,
                                   int8_t *q, float *scale, hipStream_t st);
// Static / dynamic per-row quantizer of the QAT path (ties-to-even, [-128,127]).
hipError_t rk_launch_quantize_static(const float *x, int64_t m, int64_t k, float in_scale,
                                     int8_t *q, float *row_scale, hipStream_t st);
// GGUF Q8_0 quantization of f32 rows into codes + per-block f32 scales, with
// rows remapped as (r/16)·grp_stride + grp_off + r%16 ((16, 0): unchanged).
// frag: write the fragment-major layout of the MoE expert stacks (below)
// instead of row-major codes [n, k] and scales [n, ws_stride].
hipError_t rk_launch_q8_0_quantize(const float *w, int64_t n, int64_t k, int grp_stride,
                                   int grp_off, int8_t *codes, float *scales, int ws_stride,
                                   bool frag, hipStream_t st);

// GGUF Q8_0 blocks [n][k/32] of 34 bytes (f16 d, 32 int8 codes), resident on
// the device (2-byte aligned), split into the layout rk_launch_q8_0_quantize
// writes for the same row remap and `frag` choice; d is widened to f32 exactly.
hipError_t rk_launch_q8_0_unpack(const void *blocks, int64_t n, int64_t k, int grp_stride,
                                 int grp_off, int8_t *codes, float *scales, int ws_stride,
                                 bool frag, hipStream_t st);
// Fragment-major Q8_0 layout of the MoE expert weights: per 32-row block
// (r/32) and 128-value stage (b/4), 4 KB of codes [block b%4][lane][16 bytes]
// with lane 32·h + r%32 holding values 16h..16h+15 of block b of row r, and
// 512 bytes of scales [r%32][b%4]. ws_stride: blocks per row rounded up to a
// multiple of 4 (padding blocks hold zero codes and zero scales).
__host__ __device__ inline int64_t q8_code_offset(int64_t r, int64_t b, int j, int64_t k,
                                                  int ws_stride, int frag) {
  if (!frag) return r * k + b * 32 + j;
  return ((r / 32) * (ws_stride / 4) + b / 4) * 4096 + (b % 4) * 1024 +
         ((j / 16) * 32 + r % 32) * 16 + j % 16;
}
__host__ __device__ inline int64_t q8_scale_offset(int64_t r, int64_t b, int ws_stride, int frag) {
  if (!frag) return r * ws_stride + b;
  return ((r / 32) * (ws_stride / 4) + b / 4) * 128 + (r % 32) * 4 + b % 4;
}
// QAT epilogue: y = acc·(row_scale[m]·w_scale[n]), optionally rounded to the
// out_scale grid.
hipError_t rk_launch_qat_epilogue(const int32_t *acc, const float *row_scale,
                                  const float *w_scale, int64_t m, int64_t n, float out_scale,
                                  float *y, hipStream_t st);

// Attention.
struct AttnArgs {
  const void *q;   // fp16, row (token) stride q_stride, head h at column h·D
  const void *k;   // fp16 [n_kv, k_stride], kv head g at column g·D
  const void *vt;  // fp16 V transposed and key-permuted: [KV][Dv_pad][n_kv_pad]
  void *out;       // fp16, same layout as q (o_stride)
  int64_t q_stride, k_stride, o_stride;  // in elements
  int64_t q_head_stride, k_head_stride, o_head_stride;  // elements between heads
  int64_t q_tok_stride, k_tok_stride, o_tok_stride;     // elements between tokens
  int n_q, n_kv, n_kv_pad;
  int n_head, n_kv_heads, head_dim;
  float scale, softcap;
  int mask_mode;
  int64_t window, q0, k0;
  int num_cus;
  // Key-split workspace (both null: no split). part: per split query tile, two
  // partial softmax states (rk_attn_split_floats values each); cnt: one
  // arrival counter per split query tile, zero between launches.
  float *part;
  unsigned *cnt;
  int n_split;  // query tiles split (the first ones in dispatch order, the longest)
  int mix;      // set by the launcher: interleave the PV and Sᵀ products of a slot
};
// V [n_kv, tok stride] (kv head g at column g·D) → Vt [KV][Dv_pad][n_kv_pad].
hipError_t rk_launch_v_transpose(const void *v, int64_t v_tok_stride, int64_t v_head_stride,
                                 int n_kv, int n_kv_pad, int n_kv_heads, int head_dim,
                                 int dv_pad, void *vt, hipStream_t st);
int rk_attn_dv_pad(int head_dim);
int rk_attn_kv_tile();
hipError_t rk_launch_attention(const AttnArgs &a, hipStream_t st);
// Query tiles whose keys a launch with this shape splits between two
// workgroups when given the workspace (0: no split; the longest tiles come
// first in dispatch order, so they are the ones split), and the floats of one
// half's partial state.
long rk_attn_split_tiles(const AttnArgs &a);
long rk_attn_split_floats(int head_dim);

// MoE helpers.
struct MoeTile {
  int expert;   // expert id
  int row0;     // first bucket row of the tile
  int rows;     // rows in the tile
};
// a_rows: rows of the activation buffer (s tokens for gate|up, bucket rows
// for down); offsets into it are 32-bit, so a_rows·K < 2^31. The activation
// scales are per row per 32-value group: [a_rows, stride] with stride = K/32.
// Tiles hold at most tile_rows (64 or 128) bucket rows: rk_moe_tile_rows() is
// the size a new plan lists (RK_MOE_ROWS), the launches take the plan's.
int rk_moe_tile_rows();
hipError_t rk_launch_moe_gemm_gu(int tile_rows, const int8_t *xq, const float *xs, int xs_stride,
                                 const int32_t *tok, int64_t s, const MoeTile *tiles, int n_tiles, const int8_t *w,
                                 const float *ws, int64_t w_stride_e, int64_t ws_stride_e,
                                 int ws_stride, int N, int K, float *act, hipStream_t st);
// The combine fused into the down launch (src/clef/engine.rs:317-338): y[t]
// (+)= the token's yb rows in ascending expert id, summed by the workgroup
// whose rows complete the token's top_k for its column slice. cnt holds one
// counter per (token, slice of 128 or 256 columns), zero before the launch and
// zero again after it; yb (bucket rows × N f32) must stay below 2^31 bytes.
struct MoeCombine {
  const int32_t *tok = nullptr;   // [rows] token of each bucket row
  const int32_t *slot = nullptr;  // [s, top_k] bucket rows of a token, ascending expert id
  unsigned *cnt = nullptr;        // [s, ceil(N / 128)] arrival counters
  float *y = nullptr;             // [s, N]
  int n_tok = 0;                  // s: rows of y
  int top_k = 0;
  int accumulate = 0;             // 1: y += the sum (onto the residual); 0: y = the sum
  int n_tiles = 0;                // set by the launcher
};
hipError_t rk_launch_moe_gemm_down(int tile_rows, const int8_t *aq, const float *as, int as_stride, int64_t rows,
                                   const MoeTile *tiles, int n_tiles, const int8_t *w, const float *ws,
                                   int64_t w_stride_e, int64_t ws_stride_e, int ws_stride,
                                   int N, int K, const float *row_w, float *yb, const MoeCombine &cmb,
                                   hipStream_t st);

// The static device scratch of rk_attention_dev_noalloc (noalloc.hip):
// rk_noalloc_setup looks up the array's address on `device`, which must be
// current, once; rk_noalloc_scratch returns it (null before setup).
hipError_t rk_noalloc_setup(int device);
void *rk_noalloc_scratch(int device);
